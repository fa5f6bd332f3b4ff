"""Prefill projections: y = x W^T for T tokens (the reference's
``inp @ weights[...].t()``, four_layer_mini_engine.py:6566-6573 and
:6386-6395; native prefill GEMM plans native_full_prefill.hip.cpp:552-560)."""
from __future__ import annotations

import torch


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x [T, K] bf16, w [N, K] bf16 -> [T, N] bf16 (fp32 accumulation)."""
    return x @ w.t()
