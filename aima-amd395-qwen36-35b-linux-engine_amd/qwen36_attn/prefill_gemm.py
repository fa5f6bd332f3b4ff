"""Prefill projections: y = x W^T for T tokens, the reference's
``inp @ weights[...].t()`` (four_layer_mini_engine.py:6566-6573 full
attention, :6386-6395 Gated DeltaNet), which its native prefill runs as
hipBLASLt plans (native_full_prefill.hip.cpp:552-560).

``linear`` runs them through the library's hipBLASLt entry point
(``qwen36_prefill_gemm_bf16_lt``, backend "hipblaslt"), measured faster than
the library's own MFMA kernel at every projection shape of the model from 37
to 8192 tokens on MI355X, or through that MFMA kernel (backend "native",
``qwen36_prefill_gemm_bf16_ws``: for short prompts with a long K it cuts K
into slices whose fp32 partial products go to the shared ``prefill_gemm``
scratch and are summed in slice order -- deterministic, one rounding).
"auto" is hipBLASLt, falling back to the MFMA kernel for a shape hipBLASLt
reports unsupported."""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import ptr, require, scratch, stream_handle


HIP_ERROR_NOT_SUPPORTED = 801


def linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None,
           backend: str = "auto") -> torch.Tensor:
    """x [T, K] bf16 (unit inner stride, row stride a multiple of 8), w [N, K]
    bf16 contiguous -> [T, N] bf16 (fp32 accumulation, one rounding)."""
    if backend not in ("auto", "hipblaslt", "native"):
        raise ValueError(f"unknown backend {backend!r}")
    require(x, "x", torch.bfloat16, contiguous=False)
    require(w, "w", torch.bfloat16)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1] or x.stride(1) != 1:
        raise ValueError("x must be [T, K] with unit inner stride and w [N, K]")
    t, k = x.shape
    n = w.shape[0]
    if out is None:
        out = torch.empty(t, n, dtype=torch.bfloat16, device=x.device)
    require(out, "out", torch.bfloat16, contiguous=False)
    if out.shape != (t, n) or out.stride(1) != 1:
        raise ValueError("out must be [T, N] with unit inner stride")
    if backend != "native":
        lib = _lib.load(("qwen36_prefill_gemm_bf16_lt",))
        nb = lib.qwen36_prefill_gemm_lt_workspace_bytes()
        ws = scratch("prefill_gemm_lt", nb, x.device)
        status = lib.qwen36_prefill_gemm_bf16_lt(ptr(x), x.stride(0), ptr(w), ptr(out),
                                                 out.stride(0), t, n, k, ptr(ws), ws.numel(),
                                                 stream_handle(x.device))
        if status == 0:
            return out
        if status != HIP_ERROR_NOT_SUPPORTED or backend == "hipblaslt":
            raise _lib.KernelError(f"qwen36_prefill_gemm_bf16_lt failed: hip_status={status}")
    lib = _lib.load(("qwen36_prefill_gemm_bf16_ws",))
    nb = lib.qwen36_prefill_gemm_workspace_bytes(t, n, k)
    ws = scratch("prefill_gemm", nb, x.device) if nb else None
    _lib.call("qwen36_prefill_gemm_bf16_ws", ptr(x), x.stride(0), ptr(w), ptr(out), out.stride(0),
              t, n, k, ptr(ws), ws.numel() if ws is not None else 0, stream_handle(x.device))
    return out
