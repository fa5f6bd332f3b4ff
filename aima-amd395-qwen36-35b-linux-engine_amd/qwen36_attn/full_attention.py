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
        if gate.dim() == 2 and gate.shape == (HQ, HEAD_DIM):
            gate_stride = gate.stride(0)      # e.g. the gate half of [16, 512] q rows
        elif gate.is_contiguous():
            gate_stride = HEAD_DIM
        else:
            raise ValueError("gate must be contiguous [4096] or a [16, 256] view with unit inner stride")
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


def decode_step(q_gate: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                q_norm: torch.Tensor, k_norm: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, position: int, cache_end: int | None = None,
                out: torch.Tensor | None = None, split_tokens: int = 0) -> torch.Tensor:
    """The whole one-token decode of the gated full-attention layer between
    its projections and o_proj (four_layer_mini_engine.py:6546-6653, mode
    "decode") in one fused split launch plus the combine: head norm + RoPE
    of q and the new k, the cache-row write at ``position`` (K normalised, V
    raw), split-K attention over rows [0, cache_end) and the sigmoid output
    gate.  q_gate [1, 8192] (or [8192]) is the fused q projection row; k, v
    [1, 512] raw; returns [1, 4096] bf16.  Same rounding as
    ``head_norm_rope_kv_write`` followed by ``decode_gqa``."""
    dev = q_gate.device
    if cache_end is None:
        cache_end = position + 1
    for name, x, n in (("q_gate", q_gate, 2 * Q_DIM), ("k", k, KV_DIM), ("v", v, KV_DIM)):
        require(x, name, torch.bfloat16)
        if x.numel() != n:
            raise ValueError(f"{name} must hold {n} values")
    require(q_norm, "q_norm", torch.bfloat16, shape=(HEAD_DIM,))
    require(k_norm, "k_norm", torch.bfloat16, shape=(HEAD_DIM,))
    require(k_cache, "k_cache", torch.bfloat16)
    require(v_cache, "v_cache", torch.bfloat16)
    if k_cache.dim() != 3 or tuple(k_cache.shape[1:]) != (HKV, HEAD_DIM) or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache/v_cache must be [capacity, 2, 256]")
    capacity = k_cache.shape[0]
    if not (0 <= position < cache_end <= capacity):
        raise ValueError("native grouped attention geometry is invalid")
    if out is None:
        out = torch.empty(1, Q_DIM, dtype=torch.bfloat16, device=dev)
    require(out, "out", torch.bfloat16)
    lib = _lib.load(("qwen36_decode_step",))
    ws_bytes = lib.qwen36_decode_gqa_workspace_bytes(cache_end, split_tokens)
    ws = scratch("decode_gqa", ws_bytes, dev)
    _lib.call("qwen36_decode_step", ptr(q_gate), ptr(k), ptr(v), ptr(q_norm), ptr(k_norm),
              ptr(k_cache), ptr(v_cache), position, cache_end, capacity, ptr(out), ptr(ws),
              ws.numel(), split_tokens, stream_handle(dev))
    return out


def fmha_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA flash attention, the computation of the provider ABI
    ``qrt_ck_fmha_bf16_launch_ex`` (qrt_ck_fmha_q8192_provider.cpp:306-316),
    through its workspace form ``qwen36_fmha_prefill`` (short prompts split
    their key ranges into a workspace of this package's scratch).

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
    lib = _lib.load(("qwen36_fmha_prefill",))
    nb = lib.qwen36_fmha_prefill_workspace_bytes(t, s)
    ws = scratch("fmha_split", nb, q.device) if nb else None
    _lib.call("qwen36_fmha_prefill", ptr(q), ptr(k), ptr(v), ptr(out), t, s, ptr(ws),
              ws.numel() if ws is not None else 0, stream_handle(q.device))
    return out


def fmha_prefill_gated(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       q_gate: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``fmha_prefill`` with the layer's sigmoid output gate applied in the
    same launches: bf16 ``attn * sigmoid(gate)`` rows, bit-identical (for
    non-NaN gates) to
    ``output_gate(fmha_prefill(q, k, v), q_gate)`` (the reference runs the
    provider FMHA and then full_attention_gate_kernel's f32 form,
    native_full_prefill.hip.cpp:140-266, native_pointwise.hip.cpp:339-359).
    q_gate: [T, 8192] bf16 with unit inner stride (e.g. the column view of
    the fused q|gate|k|v projection).  Returns bf16 [T, 4096]."""
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
    require(q_gate, "q_gate", torch.bfloat16, contiguous=False)
    if q_gate.shape != (t, 2 * Q_DIM) or q_gate.stride(1) != 1:
        raise ValueError("q_gate must be [T, 8192] with unit inner stride")
    if out is None:
        out = torch.empty(t, Q_DIM, dtype=torch.bfloat16, device=q.device)
    require(out, "out", torch.bfloat16, shape=(t, Q_DIM))
    lib = _lib.load(("qwen36_fmha_prefill_gated",))
    nb = lib.qwen36_fmha_prefill_workspace_bytes(t, s)
    ws = scratch("fmha_split", nb, q.device) if nb else None
    _lib.call("qwen36_fmha_prefill_gated", ptr(q), ptr(k), ptr(v), ptr(q_gate), q_gate.stride(0),
              ptr(out), t, s, ptr(ws), ws.numel() if ws is not None else 0,
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
        t, s = q.shape[0], k.shape[0]
        if q.shape != (t, HQ, HEAD_DIM) or k.shape != (s, HKV, HEAD_DIM) or value.shape != k.shape:
            raise RuntimeError("CK-FMHA q must be [T,16,256] and k/value [S,2,256]")
        if not (q.is_contiguous() and k.is_contiguous() and value.is_contiguous()):
            raise RuntimeError("CK-FMHA q/k/v inputs must be contiguous")
        lib = _lib.load(("qrt_ck_fmha_bf16_launch_ex",))
        status = lib.qrt_ck_fmha_bf16_launch_ex(ptr(q), ptr(k), ptr(value), ptr(out), t, s,
                                                stream_handle(q.device))
        if status != 0:
            raise RuntimeError(f"CK-FMHA launch failed: hip_status={status}")
        return out

    def release(self) -> None:
        _lib.call("qrt_ck_fmha_release")
        self._outputs.clear()
        self._prepared = False


def rotary_table(tokens: int, position_start: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables [tokens, 32] for absolute positions
    [position_start, position_start + tokens) (native_pointwise.hip.cpp:224-238)."""
    cos = torch.empty(tokens, 32, dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    _lib.call("qwen36_rotary_table", ptr(cos), ptr(sin), tokens, position_start,
              stream_handle(cos.device))
    return cos, sin


def head_norm_rope_kv_write(q_gate: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            q_norm: torch.Tensor, k_norm: torch.Tensor,
                            k_cache: torch.Tensor, v_cache: torch.Tensor,
                            position_start: int, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Head RMSNorm (w+1) + partial RoPE for the 16 query heads (read from the
    fused [Q|Gate] rows of ``q_gate`` [T, 8192]) and the 2 key heads ([T, 512]);
    K and the raw V are written to cache rows [position_start, +T)
    (four_layer_mini_engine.py:6566-6573 + 5151-5162 + 5980-5986).
    Returns q [T, 16, 256] bf16."""
    t = q_gate.shape[0]
    for name, x, width in (("q_gate", q_gate, 2 * Q_DIM), ("k", k, KV_DIM), ("v", v, KV_DIM)):
        require(x, name, torch.bfloat16, contiguous=False)
        if x.dim() != 2 or x.shape[0] != t or x.shape[1] != width or x.stride(1) != 1:
            raise ValueError(f"{name} must be [T, {width}] with unit inner stride")
    require(q_norm, "q_norm", torch.bfloat16, shape=(HEAD_DIM,))
    require(k_norm, "k_norm", torch.bfloat16, shape=(HEAD_DIM,))
    require(k_cache, "k_cache", torch.bfloat16)
    require(v_cache, "v_cache", torch.bfloat16)
    if position_start + t > k_cache.shape[0]:
        raise ValueError("cache too small for the new rows")
    if q_out is None:
        q_out = torch.empty(t, HQ, HEAD_DIM, dtype=torch.bfloat16, device=q_gate.device)
    _lib.call("qwen36_head_norm_rope", ptr(q_gate), q_gate.stride(0), ptr(k), k.stride(0),
              ptr(v), v.stride(0), ptr(q_norm), ptr(k_norm), t, position_start,
              ptr(q_out), ptr(k_cache), ptr(v_cache), stream_handle(q_gate.device))
    return q_out


def output_gate(attn: torch.Tensor, q_gate: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``attn * sigmoid(gate)`` with the gate half of the fused q-projection
    rows (four_layer_mini_engine.py:6650; native_pointwise.hip.cpp:207-222 and
    :339-359 for fp32 attention).  attn [T, 4096] bf16 or fp32."""
    t = attn.shape[0]
    if attn.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("attn must be bf16 or fp32")
    require(attn, "attn", attn.dtype, shape=(t, Q_DIM))
    require(q_gate, "q_gate", torch.bfloat16, contiguous=False)
    if q_gate.shape != (t, 2 * Q_DIM) or q_gate.stride(1) != 1:
        raise ValueError("q_gate must be [T, 8192] with unit inner stride")
    if out is None:
        out = torch.empty(t, Q_DIM, dtype=torch.bfloat16, device=attn.device)
    _lib.call("qwen36_output_gate", ptr(attn), int(attn.dtype == torch.float32), ptr(q_gate),
              q_gate.stride(0), ptr(out), t, stream_handle(attn.device))
    return out


class FullAttentionLayer:
    """One gated GQA layer with its resident KV cache, mirroring
    ``full_attention(inp, layer_index, weights)``
    (four_layer_mini_engine.py:6546-6653).

    Everything runs in the HIP library: the projections (prefill GEMM over
    the fused q|gate, k, v rows and o_proj; one-token GEMVs in decode),
    head-norm + RoPE + KV write, the attention core (FMHA for prefill,
    split-K decode) and the output gate.
    ``weights``: q_proj [8192,2048], k_proj/v_proj [512,2048],
    o_proj [2048,4096], q_norm/k_norm [256] (all bf16 on the GPU)."""

    def __init__(self, weights: dict, capacity: int, device) -> None:
        self.w = weights
        self.capacity = capacity
        self.k_cache = torch.zeros(capacity, HKV, HEAD_DIM, dtype=torch.bfloat16, device=device)
        self.v_cache = torch.zeros_like(self.k_cache)
        self._qkv = None   # fused decode projection, built on first use

    def forward(self, inp: torch.Tensor, position_start: int, mode: str,
                fused: bool = True) -> torch.Tensor:
        """``mode == "decode"`` runs the native one-token path -- the fused
        q|gate/k/v GEMV, the fused decode step (norm, RoPE, KV write,
        attention and gate in the split + combine launches) and the o_proj
        GEMV -- unless ``fused`` is False (torch projections, separate
        head-norm/RoPE launch, decode core)."""
        t = inp.shape[0]
        if position_start + t > self.capacity:
            raise ValueError("KV cache capacity exceeded")
        w = self.w
        cache_end = position_start + t
        if mode == "decode" and fused:
            # one token: the HIP GEMV for the fused q|gate, k, v projection and
            # o_proj, the fused decode step in between
            if t != 1:
                raise ValueError("decode takes one token")
            if self._qkv is None:
                from .projections import FusedProjection
                self._qkv = FusedProjection(w["q_proj"], w["k_proj"], w["v_proj"])
            q_gate, k, v = self._qkv(inp)
            attn = decode_step(q_gate, k, v, w["q_norm"], w["k_norm"], self.k_cache,
                               self.v_cache, position_start, cache_end)
            from .projections import gemv
            return gemv(w["o_proj"], attn)
        from .prefill_gemm import linear
        if self._qkv is None:
            from .projections import FusedProjection
            self._qkv = FusedProjection(w["q_proj"], w["k_proj"], w["v_proj"])
        # one GEMM over the fused [q|gate; k; v] rows; the three outputs are
        # column views of its [T, 9216] result
        q_gate, k, v = self._qkv.split_rows(linear(inp, self._qkv.w))
        if mode == "decode":
            if t != 1:
                raise ValueError("decode takes one token")
            # norm+rope writes K into the cache row; the decode core then needs no k_new.
            q = head_norm_rope_kv_write(q_gate, k, v, w["q_norm"], w["k_norm"],
                                        self.k_cache, self.v_cache, position_start)
            gate = q_gate.view(HQ, 2 * HEAD_DIM)[:, HEAD_DIM:]
            attn = _decode_with_strided_gate(q, self.k_cache, self.v_cache, cache_end, gate)
        else:
            q = head_norm_rope_kv_write(q_gate, k, v, w["q_norm"], w["k_norm"],
                                        self.k_cache, self.v_cache, position_start)
            attn = fmha_prefill_gated(q, self.k_cache[:cache_end], self.v_cache[:cache_end],
                                      q_gate)
        return linear(attn, w["o_proj"])


def _decode_with_strided_gate(q, k_cache, v_cache, cache_end, gate_view):
    """Decode core with the gate read in place from the fused q projection
    (head stride 512)."""
    dev = q.device
    out = torch.empty(1, Q_DIM, dtype=torch.bfloat16, device=dev)
    lib = _lib.load(("qwen36_decode_gqa",))
    ws_bytes = lib.qwen36_decode_gqa_workspace_bytes(cache_end, 0)
    ws = scratch("decode_gqa", ws_bytes, dev)
    _lib.call("qwen36_decode_gqa", ptr(q), None, None, ptr(k_cache), ptr(v_cache),
              cache_end - 1, cache_end, k_cache.shape[0], gate_view.data_ptr(),
              gate_view.stride(0), ptr(out), ptr(ws), ws.numel(), 0, stream_handle(dev))
    return out
