"""Host-side mirror of the reference's gated full-attention (GQA) path.

Reference interfaces mirrored here (file:line under the reference tree):
  * ``full_attention(inp, layer_index, weights)`` --
    benchmarks/shape-lab/four_layer_mini_engine.py:6546-6653
  * decode core ``launch_native_grouped_full_attention`` --
    native/src/native_full_attention.hip.cpp:681-765
  * prefill FMHA provider ``qrt_ck_fmha_bf16_launch[_ex]`` --
    benchmarks/shape-lab/native/src/qrt_ck_fmha_q8192_provider.cpp:214-325
  * head RMSNorm + RoPE / sigmoid gate -- native/src/native_pointwise.hip.cpp

All arithmetic runs in ``libqwen36_attn.so`` (HIP, gfx950); this module only
validates shapes, owns scratch buffers and passes pointers and the current
stream.
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import ptr, require, scratch, stream_handle

HQ, HKV, HEAD_DIM = 16, 2, 256
Q_DIM, KV_DIM = HQ * HEAD_DIM, HKV * HEAD_DIM
MAX_TOKENS = 262144


def decode_gqa(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
               position: int, cache_end: int, k_new: torch.Tensor | None = None,
               v_new: torch.Tensor | None = None, gate: torch.Tensor | None = None,
               out: torch.Tensor | None = None, split_tokens: int = 0) -> torch.Tensor:
    """One-token GQA decode over the resident cache (grouped-bmm semantics of
    four_layer_mini_engine.py:6614-6626, computed in fp32 on the GPU).

    q [16,256] (or [1,16,256]) bf16 -- already head-normed and roped.
    k_cache/v_cache [capacity, 2, 256] bf16.  If ``k_new``/``v_new`` ([2,256])
    are given they are first written to row ``position`` (the reference's
    ``write_kv_kernel``).  Attention covers rows [0, cache_end).  If ``gate``
    ([4096] bf16, the per-head gate half of the fused q projection) is given,
    the output is ``attn * sigmoid(gate)`` with the reference's roundings.
    Returns [1, 4096] bf16."""
    dev = q.device
    require(q, "q", torch.bfloat16)
    if q.numel() != Q_DIM:
        raise ValueError("q must hold 16x256 values")
    require(k_cache, "k_cache", torch.bfloat16)
    require(v_cache, "v_cache", torch.bfloat16)
    if k_cache.dim() != 3 or tuple(k_cache.shape[1:]) != (HKV, HEAD_DIM) or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache/v_cache must be [capacity, 2, 256]")
    capacity = k_cache.shape[0]
    if not (0 < cache_end <= capacity):
        raise ValueError("native grouped attention geometry is invalid")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new must be given together")
    if k_new is not None:
        require(k_new, "k_new", torch.bfloat16)
        require(v_new, "v_new", torch.bfloat16)
        if k_new.numel() != KV_DIM or v_new.numel() != KV_DIM:
            raise ValueError("k_new/v_new must hold 2x256 values")
        if not (0 <= position < cache_end):
            raise ValueError("native grouped attention geometry is invalid")
    gate_stride = 0
    if gate is not None:
        require(gate, "gate", torch.bfloat16, contiguous=False)
        if gate.numel() != Q_DIM or gate.stride(-1) != 1:
            raise ValueError("gate must hold 4096 values with unit inner stride")
        gate_stride = HEAD_DIM
    if out is None:
        out = torch.empty(1, Q_DIM, dtype=torch.bfloat16, device=dev)
    require(out, "out", torch.bfloat16)
    lib = _lib.load(("qwen36_decode_gqa",))
    ws_bytes = lib.qwen36_decode_gqa_workspace_bytes(cache_end, split_tokens)
    ws = scratch("decode_gqa", ws_bytes, dev)
    _lib.call("qwen36_decode_gqa", ptr(q), ptr(k_new), ptr(v_new), ptr(k_cache),
              ptr(v_cache), position, cache_end, capacity, ptr(gate), gate_stride,
              ptr(out), ptr(ws), ws.numel(), split_tokens, stream_handle(dev))
    return out


def fmha_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA flash attention through the provider ABI
    ``qrt_ck_fmha_bf16_launch_ex`` (qrt_ck_fmha_q8192_provider.cpp:306-316).

    q [T,16,256] bf16; k, v [S,2,256] bf16 with S >= T (rows [0,S) of the
    cache, the last T of which are the new tokens); top-left mask when S == T,
    bottom-right when S > T.  Returns fp32 [T, 4096]."""
    require(q, "q", torch.bfloat16)
    require(k, "k", torch.bfloat16)
    require(v, "v", torch.bfloat16)
    t = q.shape[0]
    s = k.shape[0]
    if q.dim() != 3 or tuple(q.shape[1:]) != (HQ, HEAD_DIM):
        raise ValueError("q must be [T, 16, 256]")
    if k.dim() != 3 or tuple(k.shape[1:]) != (HKV, HEAD_DIM) or v.shape != k.shape:
        raise ValueError("k/v must be [S, 2, 256]")
    if not (0 < t <= MAX_TOKENS and t <= s <= MAX_TOKENS):
        raise ValueError("FMHA geometry is invalid (need 0 < T <= S <= 262144)")
    if out is None:
        out = torch.empty(t, Q_DIM, dtype=torch.float32, device=q.device)
    require(out, "out", torch.float32, shape=(t, Q_DIM))
    _lib.call("qrt_ck_fmha_bf16_launch_ex", ptr(q), ptr(k), ptr(v), ptr(out), t, s,
              stream_handle(q.device))
    return out


class FmhaProvider:
    """Python mirror of the reference's ctypes FMHA provider wrapper
    (``Q8192CompoundProvider.prepare`` / ``launch_ck_fmha``,
    benchmarks/shape-lab/q8192_compound_provider.py:120-202), backed by this
    library's ``qrt_ck_fmha_*`` exports instead of the CK-Tile build."""

    def __init__(self) -> None:
        self._prepared = False
        self._outputs: dict[tuple, torch.Tensor] = {}

    def prepare(self, tokens: int = 8192) -> None:
        lib = _lib.load(("qrt_ck_fmha_prepare",))
        if lib.qrt_ck_fmha_prepare(tokens) != 0:
            raise RuntimeError("FMHA prepare failed")
        self._prepared = True

    def launch_ck_fmha(self, *, q: torch.Tensor, k: torch.Tensor,
                       value: torch.Tensor) -> torch.Tensor:
        if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
            raise RuntimeError("CK-FMHA q/k/v inputs must be BF16")
        if not self._prepared:
            self.prepare(q.shape[0])
        key = (q.device.index, q.shape[0])
        out = self._outputs.get(key)
        if out is None:
            out = torch.empty(q.shape[0], Q_DIM, dtype=torch.float32, device=q.device)
            self._outputs[key] = out
        try:
            return fmha_prefill(q, k, value, out=out)
        except _lib.KernelError as exc:
            raise RuntimeError(f"CK-FMHA launch failed: {exc}") from exc

    def release(self) -> None:
        _lib.call("qrt_ck_fmha_release")
        self._outputs.clear()
        self._prepared = False
