"""The FMHA provider driven the way the reference engine drives it: a host C++
program dlopen()s the library and resolves the qrt_ck_fmha_* symbols
(native_full_prefill.hip.cpp:140-266, NativeQ8192CkProvider), checks the
argument limits, and compares two square-causal launches and one
prefix-extended launch with its own fp64 CPU softmax(QK^T/16)V."""
import os
import subprocess

import pytest

from qwen36_attn import build as B


def _harness():
    if not os.path.exists(B.HARNESS_PATH):
        pytest.skip("provider harness not built (run __graft_entry__.build())")
    return B.HARNESS_PATH


def test_harness_reports_missing_library():
    proc = subprocess.run([_harness(), "/nonexistent/libqwen36_attn.so"],
                          capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "dlopen" in proc.stdout


@pytest.mark.gpu
def test_provider_through_dlopen(gpu):
    proc = subprocess.run([_harness(), B.LIB_PATH], capture_output=True, text=True,
                          timeout=120)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0 and proc.stdout.strip().endswith("PASS")
