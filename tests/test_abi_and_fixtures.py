"""CPU checks: the C-ABI library exports every symbol declared in
include/qwen36_attn.h and rejects bad arguments before touching the GPU; the
committed golden fixtures still match the oracle."""
import ctypes
import os
import re

import pytest
import torch
from safetensors.torch import load_file

from oracle import attention_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen36_attn.h")
FIXTURES = os.path.join(ROOT, "tests", "golden", "fixtures.safetensors")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from qwen36_attn import _lib
    if not os.path.isfile(_lib.library_path()):
        pytest.skip("library not built")
    return ctypes.CDLL(_lib.library_path())


def test_header_lists_expected_entry_points():
    syms = header_symbols()
    assert "qrt_ck_fmha_bf16_launch_ex" in syms and "qwen36_decode_gqa" in syms
    assert len(syms) >= 18


def test_library_exports_every_header_symbol(lib):
    missing = [s for s in header_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_table_matches_header():
    from qwen36_attn import _lib
    assert sorted(_lib.SIGNATURES) == header_symbols()


def test_bad_arguments_rejected_without_launch(lib):
    from qwen36_attn import _lib
    L = _lib.load()
    assert L.qrt_ck_fmha_prepare(0) == 1
    assert L.qrt_ck_fmha_prepare(262145) == 1
    assert L.qrt_ck_fmha_prepare(1) == 0
    assert L.qrt_ck_fmha_release() == 0
    # null pointers / kv < q / oversize: hipErrorInvalidValue, nothing launched
    assert L.qrt_ck_fmha_bf16_launch(None, None, None, None, 16, None) == 1
    assert L.qrt_ck_fmha_bf16_launch_ex(1, 1, 1, 1, 8, 4, None) == 1
    assert L.qrt_ck_fmha_bf16_launch_ex(1, 1, 1, 1, 8, 262145, None) == 1
    # gated FMHA: null gate, short gate stride, misaligned gate / output
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, None, 9216, 16, 8, 8, None, 0, None) == 1
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, 16, 4096, 16, 8, 8, None, 0, None) == 1
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, 18, 9216, 16, 8, 8, None, 0, None) == 1
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, 16, 9216, 24, 8, 8, None, 0, None) == 1
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, 16, 9216, 16, 8, 4, None, 0, None) == 1
    # short prompt without its split workspace
    assert L.qwen36_fmha_prefill_gated(16, 16, 16, 16, 9216, 16, 1024, 1024, None, 0, None) == 1
    assert L.qwen36_decode_gqa(None, None, None, None, None, 0, 1, 1, None, 0, None, None, 0, 0, None) == 1
    # cache_end beyond capacity
    assert L.qwen36_decode_gqa(1, None, None, 1, 1, 0, 9, 8, None, 0, 1, 1, 1 << 20, 0, None) == 1
    # k_new without v_new
    assert L.qwen36_decode_gqa(1, 1, None, 1, 1, 0, 8, 8, None, 0, 1, 1, 1 << 20, 0, None) == 1
    # split_tokens not a multiple of 128
    assert L.qwen36_decode_gqa(1, None, None, 1, 1, 0, 8, 8, None, 0, 1, 1, 1 << 20, 100, None) == 1
    # workspace too small
    assert L.qwen36_decode_gqa(1, None, None, 1, 1, 0, 4096, 4096, None, 0, 1, 1, 16, 0, None) == 1
    assert L.qwen36_decode_gqa_workspace_bytes(0, 0) == 0
    # no-allocation decode: same checks, and more than 256 splits (a workspace
    # beyond its library-owned buffer) rejected before any HIP call
    assert L.qwen36_decode_gqa_noalloc(None, None, None, None, None, 0, 1, 1, None, 0, None, 0, None) == 1
    assert L.qwen36_decode_gqa_noalloc(1, None, None, 1, 1, 0, 257 * 128, 257 * 128, None, 0, 1, 128,
                                       None) == 1
    # vLLM-orientation fused gating update: bad qk_heads, flags, scale
    fgu = L.qwen36_gdn_fused_gating_update
    assert fgu(16, 16, 16, 32, 16, 16, 16, 8, 2048, 16, 4096, 16, 16, 16, 1, 0.088, 1, None) == 1
    assert fgu(16, 16, 16, 32, 16, 16, 16, 16, 2048, 16, 4096, 16, 16, 16, 1, 0.088, 2, None) == 1
    assert fgu(16, 16, 16, 32, 16, 16, 16, 16, 2048, 16, 4096, 16, 16, 16, 1, 0.0, 1, None) == 1
    assert L.qwen36_decode_gqa_workspace_bytes(131072, 0) > 0
    assert L.qwen36_gdn_recurrent(1, 1, 1, 8, 2048, 4096, 1, 1, 1, 1, 1, 1, None) == 1  # qk_heads
    assert L.qwen36_gdn_chunk_prefill(1, 1, 1, 16, 2048, 4096, 1, 1, None, 1, 1, 64, 1, 0, None) == 1
    # chunk prefill: q / k / v base pointers not 16-byte aligned, unknown flags
    big = 1 << 30
    assert L.qwen36_gdn_chunk_prefill(24, 16, 16, 16, 2048, 4096, 16, 16, None, 16, 16, 64, 16,
                                      big, None) == 1
    assert L.qwen36_gdn_chunk_prefill(16, 16, 8, 16, 2048, 4096, 16, 16, None, 16, 16, 64, 16,
                                      big, None) == 1
    cpx = L.qwen36_gdn_chunk_prefill_ex
    assert cpx(16, 16, 16, 16, 2048, 4096, 16, 16, None, 16, 16, 64, 4, 16, big, None) == 1
    assert cpx(16, 24, 16, 16, 2048, 4096, 16, 16, None, 16, 16, 64, 3, 16, big, None) == 1
    # varlen gating update: no cu_seqlens needs one sequence per token; zero
    # sequences or slots; more than 65535 sequences
    fv = L.qwen36_gdn_fused_gating_update_varlen
    base = (16, 16, 16, 32, 16, 16, 16, 16, 2048, 16, 4096, 16, 16, 16)
    assert fv(*base, 4, None, None, 3, 4, 0.088, 1, None) == 1
    assert fv(*base, 4, 16, None, 0, 4, 0.088, 1, None) == 1
    assert fv(*base, 4, 16, None, 2, 0, 0.088, 1, None) == 1
    assert fv(*base, 4, 16, None, 65536, 4, 0.088, 1, None) == 1
    assert L.qwen36_gdn_conv1d(1, 100, 1, 1, 1, 1, 4, None) == 1  # row stride < 8192
    assert L.qwen36_head_norm_rope(1, 8192, 1, 512, 1, 512, 1, 1, 0, 0, 1, 1, 1, None) == 1
    assert L.qwen36_output_gate(1, 0, 1, 100, 1, 1, None) == 1
    assert L.qwen36_rotary_table(None, None, 1, 0, None) == 1
    assert L.qwen36_gdn_gated_norm(1, 1, 100, 1, 1, 1, None) == 1
    assert L.qwen36_gdn_gating(1, 1, 8, 1, 1, 1, 1, 1, 0, None) == 1
    assert L.qwen36_gdn_gating(1, 1, 32, 1, 1, 1, 1, 1, 2, None) == 1
    # fused GDN decode step: aliased / overlapping conv state, bad strides, T = 0
    good = dict(x=16, xs=8192, w=32, ci=4096, co=1 << 20, a=48, b=64, abs_=32, al=80, dt=96,
                z=128, zs=4096, nw=160, si=256, so=256, out=512)
    def step(**kw):
        v = dict(good, **kw)
        return L.qwen36_gdn_decode_step(v["x"], v["xs"], v["w"], v["ci"], v["co"], v["a"], v["b"],
                                        v["abs_"], v["al"], v["dt"], v["z"], v["zs"], v["nw"],
                                        v["si"], v["so"], v["out"], v.get("t", 1), None)
    assert step(co=4096) == 1                 # conv_state_out == conv_state_in
    assert step(co=4096 + 2 * 8192 * 3 - 2) == 1   # overlapping conv buffers
    assert step(xs=100) == 1
    assert step(zs=100) == 1
    assert step(abs_=8) == 1
    assert step(t=0) == 1
    # fused full-attention decode step: nulls, position outside the cache
    assert L.qwen36_decode_step(None, 16, 16, 16, 16, 16, 16, 0, 1, 1, 16, 16, 1 << 20, 0, None) == 1
    assert L.qwen36_decode_step(16, 16, 16, 16, 16, 16, 16, 5, 5, 8, 16, 16, 1 << 20, 0, None) == 1
    assert L.qwen36_decode_step(16, 16, 16, 16, 16, 16, 16, 0, 9, 8, 16, 16, 1 << 20, 0, None) == 1
    # GEMV: K other than 2048/4096, zero rows, misaligned weights
    assert L.qwen36_gemv_bf16(16, 4, 1024, 16, 16, None) == 1
    assert L.qwen36_gemv_bf16(16, 0, 2048, 16, 16, None) == 1
    assert L.qwen36_gemv_bf16(18, 4, 2048, 16, 16, None) == 1
    # MoE decode: expert count out of range / not a multiple of 4, small workspace
    ws = L.qwen36_moe_decode_workspace_bytes()
    assert ws > 0
    assert L.qwen36_moe_decode(16, 16, 16, 16, 16, 16, 16, 4, 16, 16, ws, None) == 1
    assert L.qwen36_moe_decode(16, 16, 16, 16, 16, 16, 16, 257, 16, 16, ws, None) == 1
    assert L.qwen36_moe_decode(16, 16, 16, 16, 16, 16, 16, 30, 16, 16, ws, None) == 1
    assert L.qwen36_moe_decode(16, 16, 16, 16, 16, 16, 16, 32, 16, 16, ws - 1, None) == 1
    # MoE prefill: token count 0 / above 262144, expert count out of range or
    # not a multiple of 4, small workspace, misaligned output
    W = L.qwen36_moe_prefill_workspace_bytes
    assert W(0, 256) == 0 and W(262145, 256) == 0
    assert W(16, 4) == 0 and W(16, 258) == 0 and W(16, 30) == 0
    ws = W(16, 256)
    assert ws > 0 and W(32, 256) > ws
    assert L.qwen36_moe_prefill(16, 16, 16, 16, 16, 16, 16, 256, 0, 16, 16, ws, None) == 1
    assert L.qwen36_moe_prefill(16, 16, 16, 16, 16, 16, 16, 256, 16, 16, 16, ws - 1, None) == 1
    assert L.qwen36_moe_prefill(16, 16, 16, 16, 16, 16, 16, 256, 16, 18, 16, ws, None) == 1
    # prefill GEMM workspace: split planes (a whole number of fp32 [m, n]
    # planes) only for short prompts; 0 for long prompts and invalid k
    G = L.qwen36_prefill_gemm_workspace_bytes
    assert G(8192, 2048, 4096) == 0 and G(1024, 9216, 2048) == 0
    assert G(1024, 2048, 4096) == 2 * 1024 * 2048 * 4
    assert G(256, 2048, 4096) % (256 * 2048 * 4) == 0 and G(256, 2048, 4096) > 0
    assert G(1024, 2048, 4000) == 0 and G(0, 2048, 4096) == 0
    # hipBLASLt form: nulls, m = 0, ldy < n, workspace size without a buffer
    lt = L.qwen36_prefill_gemm_bf16_lt
    assert L.qwen36_prefill_gemm_lt_workspace_bytes() > 0
    assert lt(None, 2048, 16, 16, 2048, 16, 2048, 2048, None, 0, None) == 1
    assert lt(16, 2048, 16, 16, 2048, 0, 2048, 2048, None, 0, None) == 1
    assert lt(16, 2048, 16, 16, 100, 16, 2048, 2048, None, 0, None) == 1
    assert lt(16, 2048, 16, 16, 2048, 16, 2048, 2048, None, 64, None) == 1
    # shapes the launch rejects size no workspace
    assert G(1024, 2048, 16384 + 64) == 0 and G(1024, 65537, 4096) == 0
    assert G(262145, 2048, 4096) == 0
    assert L.qwen36_prefill_gemm_bf16_ws(16, 2048, 16, 16, 2048, 300, 2048, 4096,
                                         16, G(300, 2048, 4096) - 16, None) == 1


def test_scratch_growth_is_geometric_and_bounded():
    """Workspaces that grow with the prompt keep their outgrown buffers (a
    captured graph may hold them), so growth must be geometric: after rising
    requests the dead buffers of a tag stay below its live buffer."""
    from qwen36_attn import _tensors as T
    dev = torch.device("cpu")
    tag = "growth_test"
    for n in range(64, 8193, 64):
        buf = T.scratch(tag, n * 1000, dev)
        assert buf.numel() >= n * 1000
    live = T._SCRATCH[(tag, 0)].numel()
    assert live & (live - 1) == 0            # a power of two
    assert T.retired_bytes(tag) < live
    assert T.scratch(tag, 100, dev).numel() == live   # smaller requests reuse it


def test_prefix_cache_host_bookkeeping_without_device(lib):
    """Pool creation rules and slice validation (no device memory is
    touched before finalize): the reference's 4 / 2 / 1 entry rule
    (native_resident_engine.hip.cpp:553-556), per-token slices must span
    max_tokens rows, 16-byte alignment, lookups on an empty pool miss."""
    import ctypes
    from qwen36_attn import _lib
    L = _lib.load()
    assert not L.qwen36_prefix_cache_create(0, 4096, 0)
    assert not L.qwen36_prefix_cache_create(1024, 4095, 0)
    for cap, n in ((1024, 4), (32768, 4), (32769, 2), (131072, 2), (131073, 1), (262144, 1)):
        p = L.qwen36_prefix_cache_create(cap, 4096, 0)
        assert p and L.qwen36_prefix_cache_entries(p) == n
        assert L.qwen36_prefix_cache_destroy(p) == 0
    p = L.qwen36_prefix_cache_create(100, 4096, 3)
    assert L.qwen36_prefix_cache_entries(p) == 3
    assert L.qwen36_prefix_cache_add_slice(p, 4096, 100 * 1024, 1024) == 0
    assert L.qwen36_prefix_cache_add_slice(p, 4096, 99 * 1024, 1024) == 1    # not max_tokens rows
    assert L.qwen36_prefix_cache_add_slice(p, 4100, 4096, 0) == 1            # misaligned
    assert L.qwen36_prefix_cache_add_slice(p, 4096, 4001, 0) == 1            # size not 16-byte multiple
    toks = (ctypes.c_uint * 3)(1, 2, 3)
    m, i = ctypes.c_uint(9), ctypes.c_uint(9)
    assert L.qwen36_prefix_cache_lookup(p, toks, 3, ctypes.byref(m), ctypes.byref(i)) == 0
    assert (m.value, i.value) == (0, 3)
    assert L.qwen36_prefix_cache_restore(p, 0, None, None) == 1                # not finalized
    assert L.qwen36_prefix_cache_destroy(p) == 0


def test_fixtures_match_oracle():
    from tests.golden.make_fixtures import build
    fresh = build()
    saved = load_file(FIXTURES)
    assert sorted(fresh) == sorted(saved)
    for k, v in saved.items():
        assert torch.equal(fresh[k], v), k


def test_fixture_prefill_is_tail_of_decode_chain():
    f = load_file(FIXTURES)
    # The bf16 prefill output's last row equals a decode of that row over all 9 keys.
    dec = O.decode_attention_grouped_bf16(f["prefill.q"][-1:], f["prefill.k"], f["prefill.v"], 9)
    assert (dec.float() - f["prefill.out_f32"][-1:]).abs().max() <= 2e-2
