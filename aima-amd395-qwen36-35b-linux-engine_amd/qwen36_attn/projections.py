"""One-token decode projections on the HIP GEMV (``qwen36_gemv_bf16``),
mirroring ``inp @ W.t()`` of four_layer_mini_engine.py:6566-6573 (full
attention: fused q|gate, k, v; o_proj) and :6386-6395 (Gated DeltaNet:
in_proj_qkv, z, b, a; out_proj) for the decode step, the role of the
reference's triton_matvec / bf16_wvsplitk kernels
(native_full_layer.hip.cpp:154-174, native_linear_layer.hip.cpp:151-157)."""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import ptr, require, stream_handle


def gemv(w: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = W x for one token.  w [N, K] bf16 contiguous (K = 2048 or 4096),
    x [K] or [1, K] bf16; returns [1, N] bf16 (fp32 accumulation)."""
    require(w, "w", torch.bfloat16)
    require(x, "x", torch.bfloat16)
    n, k = w.shape
    if x.numel() != k:
        raise ValueError("x must hold K values")
    if out is None:
        out = torch.empty(1, n, dtype=torch.bfloat16, device=w.device)
    _lib.call("qwen36_gemv_bf16", ptr(w), n, k, ptr(x), ptr(out), stream_handle(w.device))
    return out


class FusedProjection:
    """Row-concatenated weights [W_0; W_1; ...] (all [N_i, K]) applied with one
    GEMV; ``__call__(x)`` returns the views [1, N_i] of the one output row, as
    the reference's fused projection kernels return one packed row."""

    def __init__(self, *weights: torch.Tensor) -> None:
        k = weights[0].shape[1]
        if any(w.shape[1] != k for w in weights):
            raise ValueError("fused weights must share K")
        self.w = torch.cat([w.contiguous() for w in weights], dim=0).contiguous()
        self.splits = [w.shape[0] for w in weights]

    def __call__(self, x: torch.Tensor) -> list[torch.Tensor]:
        y = gemv(self.w, x)
        return list(torch.split(y, self.splits, dim=1))

    def split_rows(self, y: torch.Tensor) -> list[torch.Tensor]:
        """Column views [T, N_i] of a [T, sum N_i] product with ``self.w``."""
        return list(torch.split(y, self.splits, dim=1))
