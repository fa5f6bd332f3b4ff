"""Host-side mirror of the reference's Gated-DeltaNet (linear attention) path.

Reference interfaces mirrored (four_layer_mini_engine.py, "fle"):
  * ``linear_attention(inp, layer_index, weights)`` -- fle:6378-6544
  * ``linear_causal_conv`` -- fle:5293-5403
  * ``torch_chunk_gated_delta_rule(query, key, value, g, beta, initial_state,
    chunk_size=64)`` -- fle:5167-5240
  * ``torch_recurrent_gated_delta_rule(query, key, value, g, beta,
    initial_state)`` -- fle:5242-5276
  * gated RMSNorm -- fle:6531-6541
All arithmetic runs in ``libqwen36_attn.so``.
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import ptr, require, scratch, stream_handle

HK, HV, DK, DV = 16, 32, 128, 128
KEY_DIM, VALUE_DIM = HK * DK, HV * DV
CONV_DIM = 2 * KEY_DIM + VALUE_DIM
CHUNK = 64


def causal_conv1d(mixed_qkv: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor,
                  new_state: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Depthwise causal conv (k=4) + SiLU over [state | x].  mixed_qkv [T, 8192]
    bf16 (unit inner stride), conv_state [8192, 3] bf16, weight [8192, 4] bf16.
    Returns (out [T, 8192] bf16, new_state [8192, 3]); ``new_state`` may be
    ``conv_state`` itself (in-place update)."""
    t = mixed_qkv.shape[0]
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, contiguous=False)
    if mixed_qkv.shape[1] != CONV_DIM or mixed_qkv.stride(1) != 1:
        raise ValueError("mixed_qkv must be [T, 8192] with unit inner stride")
    require(conv_state, "conv_state", torch.bfloat16, shape=(CONV_DIM, 3))
    require(weight, "weight", torch.bfloat16, shape=(CONV_DIM, 4))
    if new_state is None:
        new_state = torch.empty_like(conv_state)
    if out is None:
        out = torch.empty(t, CONV_DIM, dtype=torch.bfloat16, device=mixed_qkv.device)
    _lib.call("qwen36_gdn_conv1d", ptr(mixed_qkv), mixed_qkv.stride(0), ptr(weight),
              ptr(conv_state), ptr(new_state), ptr(out), t, stream_handle(out.device))
    return out, new_state


def gating(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
           dt_bias: torch.Tensor, beta_fp32: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b); fp32 [T, 32]
    (fle:6507-6511).  The layer's torch text evaluates sigmoid on the bf16
    projection output, so beta is rounded to bf16 unless ``beta_fp32`` (the
    vLLM fused gating keeps it in fp32)."""
    t = a.shape[0]
    for name, x in (("a", a), ("b", b)):
        require(x, name, torch.bfloat16, contiguous=False)
        if x.shape != (t, HV) or x.stride(1) != 1:
            raise ValueError(f"{name} must be [T, 32]")
    if a.stride(0) != b.stride(0):
        raise ValueError("a and b must share a row stride")
    a_log = a_log.float().contiguous()
    dt_bias = dt_bias.float().contiguous()
    g = torch.empty(t, HV, dtype=torch.float32, device=a.device)
    beta = torch.empty_like(g)
    _lib.call("qwen36_gdn_gating", ptr(a), ptr(b), a.stride(0), ptr(a_log), ptr(dt_bias),
              ptr(g), ptr(beta), t, 1 if beta_fp32 else 0, stream_handle(a.device))
    return g, beta


def _qkv_views(query, key, value):
    """Accept [T,H,128] or [1,T,H,128] q/k (H = 16 unrepeated or 32 repeated)
    and v [T,32,128] / [1,T,32,128]; return strides for the C ABI."""
    def squeeze(x, name):
        if x.dim() == 4:
            if x.shape[0] != 1:
                raise ValueError(f"{name}: batch must be 1")
            x = x[0]
        if x.dim() != 3:
            raise ValueError(f"{name} must be [T, H, 128]")
        require(x, name, torch.bfloat16, contiguous=False)
        if x.stride(2) != 1 or x.stride(1) != x.shape[2]:
            raise ValueError(f"{name} must have contiguous heads")
        return x
    q, k, v = squeeze(query, "query"), squeeze(key, "key"), squeeze(value, "value")
    t, hq = q.shape[0], q.shape[1]
    if k.shape != q.shape or q.stride(0) != k.stride(0):
        raise ValueError("query and key must share shape and token stride")
    if hq not in (HK, HV) or q.shape[2] != DK:
        raise ValueError("query/key must have 16 or 32 heads of 128")
    if v.shape != (t, HV, DV):
        raise ValueError("value must be [T, 32, 128]")
    return q, k, v, t, hq


def _gb(g, beta, t):
    g = g.reshape(t, HV)
    beta = beta.reshape(t, HV)
    require(g, "g", torch.float32)
    require(beta, "beta", torch.float32)
    return g, beta


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state,
                               final_state: torch.Tensor | None = None):
    """Mirror of ``torch_recurrent_gated_delta_rule`` (fle:5242-5276) with the
    l2norm of q/k done in-kernel.  initial_state [32,128,128] (or [1,...]) fp32
    in [H, dk, dv] orientation.  Returns (out [1,T,32,128] bf16, final_state);
    ``final_state`` may alias ``initial_state``."""
    q, k, v, t, hq = _qkv_views(query, key, value)
    g, beta = _gb(g, beta, t)
    s_in = initial_state.reshape(HV, DK, DV)
    require(s_in, "initial_state", torch.float32)
    if final_state is None:
        final_state = torch.empty_like(s_in)
    out = torch.empty(1, t, HV, DV, dtype=torch.bfloat16, device=q.device)
    _lib.call("qwen36_gdn_recurrent", ptr(q), ptr(k), ptr(v), hq, q.stride(0), v.stride(0),
              ptr(g), ptr(beta), ptr(s_in), ptr(final_state), ptr(out), t,
              stream_handle(q.device))
    return out, final_state.view(1, HV, DK, DV)


def chunk_gated_delta_rule(query, key, value, g, beta, initial_state=None, chunk_size: int = CHUNK,
                           final_state: torch.Tensor | None = None):
    """Mirror of ``torch_chunk_gated_delta_rule`` (fle:5167-5240); chunk 64.
    ``initial_state`` None means zeros.  Returns (out [1,T,32,128] bf16,
    final_state [1,32,128,128] fp32)."""
    if chunk_size != CHUNK:
        raise ValueError("the HIP kernel implements chunk_size=64")
    q, k, v, t, hq = _qkv_views(query, key, value)
    g, beta = _gb(g, beta, t)
    s_in = None
    if initial_state is not None:
        s_in = initial_state.reshape(HV, DK, DV)
        require(s_in, "initial_state", torch.float32)
    if final_state is None:
        final_state = torch.empty(HV, DK, DV, dtype=torch.float32, device=q.device)
    out = torch.empty(1, t, HV, DV, dtype=torch.bfloat16, device=q.device)
    lib = _lib.load(("qwen36_gdn_chunk_prefill",))
    nb = lib.qwen36_gdn_chunk_prefill_workspace_bytes(t)
    ws = scratch("gdn_chunk", nb, q.device)
    _lib.call("qwen36_gdn_chunk_prefill", ptr(q), ptr(k), ptr(v), hq, q.stride(0), v.stride(0),
              ptr(g), ptr(beta), ptr(s_in), ptr(final_state), ptr(out), t, ptr(ws), ws.numel(),
              stream_handle(q.device))
    return out, final_state.view(1, HV, DK, DV)


QK_NORMALIZED, STATE_VK = 1, 2   # qwen36_gdn_chunk_prefill_ex flags


def vllm_chunk_gated_delta_rule(q, k, v, g, beta, scale: float | None = None,
                                initial_state: torch.Tensor | None = None,
                                output_final_state: bool = False,
                                cu_seqlens=None, head_first: bool = False,
                                use_qk_l2norm_in_kernel: bool = False):
    """Mirror of vLLM's ``chunk_gated_delta_rule`` as the reference calls it
    (fle:6474-6483): q, k [1, T, 16, 128] (unrepeated key heads; v-head h
    reads key head h // 2), v [1, T, 32, 128] bf16, g (log decay), beta
    [1, T, 32] fp32, ``initial_state`` [1, 32, 128 (v), 128 (k)] fp32 -- vLLM's
    orientation, the transpose of the torch path's (handoff fle:5482-5502) --
    or None for zeros.  ``use_qk_l2norm_in_kernel=False`` (the reference's
    choice, since fused_post_conv_prep has already normalised q and k) uses
    q and k as given; True normalises them in the kernel.  Returns (o [1, T,
    32, 128] bf16, final_state [1, 32, 128, 128] fp32 in the same [v, k]
    orientation, or None unless ``output_final_state``).  Chunk 64, scale
    1/sqrt(128) (vLLM's default; other scales are rejected), batch 1 without
    varlen packing, as the reference uses it."""
    if cu_seqlens is not None:
        raise NotImplementedError("cu_seqlens (varlen batches) is not provided: the engine "
                                  "runs batch 1")
    if head_first:
        raise ValueError("head_first layout is not supported (vLLM deprecated it)")
    if scale is not None and abs(scale - DK ** -0.5) > 1e-12:
        raise ValueError("the HIP kernel applies scale 1/sqrt(128)")
    qq, kk, vv, t, hq = _qkv_views(q, k, v)
    g, beta = _gb(g, beta, t)
    s_in = None
    if initial_state is not None:
        s_in = initial_state.reshape(HV, DV, DK)
        require(s_in, "initial_state", torch.float32)
    final_state = torch.empty(HV, DV, DK, dtype=torch.float32, device=qq.device)
    out = torch.empty(1, t, HV, DV, dtype=torch.bfloat16, device=qq.device)
    flags = STATE_VK | (0 if use_qk_l2norm_in_kernel else QK_NORMALIZED)
    lib = _lib.load(("qwen36_gdn_chunk_prefill_ex",))
    nb = lib.qwen36_gdn_chunk_prefill_workspace_bytes(t)
    ws = scratch("gdn_chunk", nb, qq.device)
    _lib.call("qwen36_gdn_chunk_prefill_ex", ptr(qq), ptr(kk), ptr(vv), hq, qq.stride(0),
              vv.stride(0), ptr(g), ptr(beta), ptr(s_in), ptr(final_state), ptr(out), t,
              flags, ptr(ws), ws.numel(), stream_handle(qq.device))
    return out, (final_state.view(1, HV, DV, DK) if output_final_state else None)


def gated_rmsnorm(core: torch.Tensor, z: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fle:6531-6541: rmsnorm_128(core) * w -> bf16 -> * SiLU(z) -> bf16.
    core [T,32,128] (or [1,T,32,128]) bf16, z [T,4096]; returns [T, 4096]."""
    core = core.reshape(-1, HV, DV)
    t = core.shape[0]
    require(core, "core", torch.bfloat16)
    require(z, "z", torch.bfloat16, contiguous=False)
    if z.shape != (t, VALUE_DIM) or z.stride(1) != 1:
        raise ValueError("z must be [T, 4096] with unit inner stride")
    require(weight, "weight", torch.bfloat16, shape=(DV,))
    out = torch.empty(t, VALUE_DIM, dtype=torch.bfloat16, device=core.device)
    _lib.call("qwen36_gdn_gated_norm", ptr(core), ptr(z), z.stride(0), ptr(weight), ptr(out), t,
              stream_handle(core.device))
    return out


def gdn_decode_step(mixed_qkv: torch.Tensor, conv_state: torch.Tensor,
                    new_conv_state: torch.Tensor, conv_weight: torch.Tensor,
                    a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
                    dt_bias: torch.Tensor, z: torch.Tensor, norm_weight: torch.Tensor,
                    ssm_state: torch.Tensor, final_state: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """One fused launch for the decode part of ``linear_attention`` between
    the input projections and out_proj (fle:6378-6544, mode "decode"): conv
    + SiLU, gating, l2norm, recurrent delta rule and gated RMSNorm for the
    T rows of ``mixed_qkv``.  ``new_conv_state`` receives the conv state and
    must be a different buffer from ``conv_state``; ``final_state`` (default:
    ``ssm_state`` itself) receives the fp32 recurrent state.  Returns the
    gated output [T, 4096] bf16."""
    t = mixed_qkv.shape[0]
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, contiguous=False)
    if mixed_qkv.shape[1] != CONV_DIM or mixed_qkv.stride(1) != 1:
        raise ValueError("mixed_qkv must be [T, 8192] with unit inner stride")
    require(conv_state, "conv_state", torch.bfloat16, shape=(CONV_DIM, 3))
    require(new_conv_state, "new_conv_state", torch.bfloat16, shape=(CONV_DIM, 3))
    if new_conv_state.data_ptr() == conv_state.data_ptr():
        raise ValueError("new_conv_state must not alias conv_state (double-buffer it)")
    require(conv_weight, "conv_weight", torch.bfloat16, shape=(CONV_DIM, 4))
    for name, x in (("a", a), ("b", b)):
        require(x, name, torch.bfloat16, contiguous=False)
        if x.shape != (t, HV) or x.stride(1) != 1:
            raise ValueError(f"{name} must be [T, 32]")
    if a.stride(0) != b.stride(0):
        raise ValueError("a and b must share a row stride")
    require(z, "z", torch.bfloat16, contiguous=False)
    if z.shape != (t, VALUE_DIM) or z.stride(1) != 1:
        raise ValueError("z must be [T, 4096] with unit inner stride")
    require(norm_weight, "norm_weight", torch.bfloat16, shape=(DV,))
    ssm = ssm_state.reshape(HV, DK, DV)
    require(ssm, "ssm_state", torch.float32)
    if final_state is None:
        final_state = ssm
    require(final_state.reshape(HV, DK, DV), "final_state", torch.float32)
    a_log = a_log.float().contiguous()
    dt_bias = dt_bias.float().contiguous()
    if out is None:
        out = torch.empty(t, VALUE_DIM, dtype=torch.bfloat16, device=mixed_qkv.device)
    _lib.call("qwen36_gdn_decode_step", ptr(mixed_qkv), mixed_qkv.stride(0), ptr(conv_weight),
              ptr(conv_state), ptr(new_conv_state), ptr(a), ptr(b), a.stride(0), ptr(a_log),
              ptr(dt_bias), ptr(z), z.stride(0), ptr(norm_weight), ptr(ssm), ptr(final_state),
              ptr(out), t, stream_handle(out.device))
    return out


class LinearAttentionLayer:
    """One Gated-DeltaNet layer with its carried conv and recurrent states,
    mirroring ``linear_attention(inp, layer_index, weights)``
    (fle:6378-6544, plain-torch branch).  Everything runs in the HIP library:
    the projections (prefill GEMM over the fused qkv|z|b|a rows and out_proj,
    one-token GEMVs in decode), conv, gating, delta rule and gated norm.  ``weights``: in_proj_qkv [8192,2048], in_proj_z [4096,2048],
    in_proj_a/in_proj_b [32,2048], conv1d [8192,4], A_log [32], dt_bias [32],
    norm [128], out_proj [2048,4096]."""

    def __init__(self, weights: dict, device) -> None:
        self.w = weights
        self.conv_state = torch.zeros(CONV_DIM, 3, dtype=torch.bfloat16, device=device)
        self.ssm_state = torch.zeros(HV, DK, DV, dtype=torch.float32, device=device)
        self.conv_spare = None   # second conv-state buffer for the fused decode step
        self._conv_home = self.conv_state
        self._in_proj = None   # fused decode input projection, built on first use

    def normalize_state(self) -> None:
        """Keep the carried conv state in the buffer allocated at construction
        (the fused decode step ping-pongs two buffers), as the reference's
        normalize_linear_decode_state does before a prefix-cache capture
        (native_resident_engine.hip.cpp:272-296): registered state pointers
        stay valid."""
        if self.conv_spare is not None and self.conv_state.data_ptr() != self._conv_home.data_ptr():
            self._conv_home.copy_(self.conv_state)
            self.conv_spare = self.conv_state
            self.conv_state = self._conv_home

    def forward(self, inp: torch.Tensor, mode: str, fused: bool = True) -> torch.Tensor:
        """``mode == "decode"`` runs the native path -- for one token the
        fused in-projection GEMV, the one-launch step (``gdn_decode_step``)
        and the out_proj GEMV; for several tokens torch projections around the
        same step -- unless ``fused`` is False, which runs torch projections
        and the step as four launches (conv, gating, recurrent, gated norm)."""
        w = self.w
        if mode == "decode" and fused and inp.shape[0] == 1:
            # one token: the fused qkv|z|b|a GEMV, the fused step, the out_proj GEMV
            from .projections import FusedProjection, gemv
            if self._in_proj is None:
                self._in_proj = FusedProjection(w["in_proj_qkv"], w["in_proj_z"],
                                                w["in_proj_b"], w["in_proj_a"])
            mixed, z, b, a = self._in_proj(inp)
            if self.conv_spare is None:
                self.conv_spare = torch.empty_like(self.conv_state)
            gated = gdn_decode_step(mixed, self.conv_state, self.conv_spare, w["conv1d"], a, b,
                                    w["A_log"], w["dt_bias"], z, w["norm"], self.ssm_state)
            self.conv_state, self.conv_spare = self.conv_spare, self.conv_state
            return gemv(w["out_proj"], gated)
        from .prefill_gemm import linear
        from .projections import FusedProjection
        if self._in_proj is None:
            self._in_proj = FusedProjection(w["in_proj_qkv"], w["in_proj_z"],
                                            w["in_proj_b"], w["in_proj_a"])
        # one GEMM over the fused [qkv; z; b; a] rows; column views of the
        # [T, 12352] result feed the conv, gating and gated norm in place
        mixed, z, b, a = self._in_proj.split_rows(linear(inp, self._in_proj.w))
        if mode == "decode" and fused:
            if self.conv_spare is None:
                self.conv_spare = torch.empty_like(self.conv_state)
            gated = gdn_decode_step(mixed, self.conv_state, self.conv_spare, w["conv1d"], a, b,
                                    w["A_log"], w["dt_bias"], z, w["norm"], self.ssm_state)
            self.conv_state, self.conv_spare = self.conv_spare, self.conv_state
            return linear(gated, w["out_proj"])
        conv_out, _ = causal_conv1d(mixed, self.conv_state, w["conv1d"], new_state=self.conv_state)
        t = conv_out.shape[0]
        q = conv_out[:, :KEY_DIM].view(t, HK, DK)
        k = conv_out[:, KEY_DIM:2 * KEY_DIM].view(t, HK, DK)
        v = conv_out[:, 2 * KEY_DIM:].view(t, HV, DV)
        g, beta = gating(a, b, w["A_log"], w["dt_bias"])
        if mode == "decode":
            core, _ = recurrent_gated_delta_rule(q, k, v, g, beta, self.ssm_state,
                                                 final_state=self.ssm_state)
        else:
            # in place: each scan lane reads its state elements before it
            # writes them, so the state keeps its buffer (prefix-cache slices)
            core, _ = chunk_gated_delta_rule(q, k, v, g, beta, self.ssm_state,
                                             final_state=self.ssm_state)
        gated = gated_rmsnorm(core, z, w["norm"])
        return linear(gated, w["out_proj"])


def _ab_views(a, b, t):
    a2 = a.reshape(t, HV) if a.dim() == 3 else a
    b2 = b.reshape(t, HV) if b.dim() == 3 else b
    for name, x in (("a", a2), ("b", b2)):
        require(x, name, torch.bfloat16, contiguous=False)
        if x.shape != (t, HV) or x.stride(1) != 1:
            raise ValueError(f"{name} must be [T, 32]")
    if a2.stride(0) != b2.stride(0):
        raise ValueError("a and b must share a row stride")
    return a2, b2


def _int32_vector(x, name, n, device):
    if not isinstance(x, torch.Tensor):
        x = torch.as_tensor(x)
    x = x.reshape(-1)
    if x.numel() != n:
        raise ValueError(f"{name} must hold {n} entries (got {x.numel()})")
    if x.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must be an integer tensor")
    return x.to(device=device, dtype=torch.int32).contiguous()


def fused_sigmoid_gating_delta_rule_update(A_log, a, b, dt_bias, q, k, v, beta: float = 1.0,
                                           threshold: float = 20.0, scale: float | None = None,
                                           initial_state: torch.Tensor | None = None,
                                           inplace_final_state: bool = True,
                                           cu_seqlens=None, ssm_state_indices=None,
                                           num_accepted_tokens=None,
                                           use_qk_l2norm_in_kernel: bool = False):
    """Drop-in for vLLM's ``fused_sigmoid_gating_delta_rule_update`` as the
    reference's decode calls it (four_layer_mini_engine.py:6429-6440): gating
    fused into the recurrent update, state in vLLM's [Hv, dv, dk] orientation
    (``qwen36_gdn_fused_gating_update``).

    q, k [1, T, 16 (or 32), 128] bf16; v [1, T, 32, 128] bf16; a, b [T, 32]
    (or [1, T, 32]) bf16; A_log, dt_bias [32].  One sequence: initial_state
    [1, 32, 128, 128] fp32.  Batched (vLLM's varlen form): ``cu_seqlens``
    [N + 1] token offsets of N sequences, each carrying state slot
    ``ssm_state_indices[n]`` (default n) of the pool ``initial_state``
    [slots, 32, 128, 128]; a slot index outside [0, slots) marks a padding
    sequence, skipped (``qwen36_gdn_fused_gating_update_varlen``).  Returns
    (o [1, T, 32, 128] bf16, final_state): ``initial_state`` itself, updated,
    when ``inplace_final_state``, else an updated copy.  num_accepted_tokens
    (speculative decoding) is not provided; beta/threshold keep vLLM's
    defaults (1.0, 20.0)."""
    if num_accepted_tokens is not None:
        raise NotImplementedError("num_accepted_tokens (speculative decoding) is not provided")
    if beta != 1.0 or threshold != 20.0:
        raise NotImplementedError("softplus beta/threshold other than 1.0/20.0")
    if initial_state is None:
        raise ValueError("initial_state is required")
    qv, kv_, vv, t, hq = _qkv_views(q, k, v)
    if qv.stride(0) % 8:
        raise ValueError("q/k token stride must be a multiple of 8")
    a2, b2 = _ab_views(a, b, t)
    require(initial_state, "initial_state", torch.float32)
    if initial_state.dim() != 4 or tuple(initial_state.shape[1:]) != (HV, DV, DK):
        raise ValueError("initial_state must be [slots, 32, 128, 128]")
    slots = initial_state.shape[0]
    single = cu_seqlens is None and ssm_state_indices is None
    # out of place: a single sequence writes every element of the new state;
    # a batch leaves slots no sequence uses untouched, so it starts from a copy
    final = (initial_state if inplace_final_state else
             torch.empty_like(initial_state) if single else initial_state.clone())
    out = torch.empty(1, t, HV, DV, dtype=torch.bfloat16, device=qv.device)
    a_log = A_log.float().contiguous()
    dtb = dt_bias.float().contiguous()
    if scale is None:
        scale = DK ** -0.5
    flags = 1 if use_qk_l2norm_in_kernel else 0
    if single:
        if slots != 1:
            raise ValueError("a single sequence takes a [1, 32, 128, 128] state")
        _lib.call("qwen36_gdn_fused_gating_update", ptr(a_log), ptr(a2), ptr(b2), a2.stride(0),
                  ptr(dtb), ptr(qv), ptr(kv_), hq, qv.stride(0), ptr(vv), vv.stride(0),
                  ptr(initial_state), ptr(final), ptr(out), t, float(scale), flags,
                  stream_handle(qv.device))
        return out, final
    if cu_seqlens is None:
        cu_seqlens = torch.tensor([0, t], dtype=torch.int32)
    n = (cu_seqlens.numel() if isinstance(cu_seqlens, torch.Tensor) else len(cu_seqlens)) - 1
    cu = _int32_vector(cu_seqlens, "cu_seqlens", n + 1, qv.device)
    idx = None
    if ssm_state_indices is not None:
        idx = _int32_vector(ssm_state_indices, "ssm_state_indices", n, qv.device)
    _lib.call("qwen36_gdn_fused_gating_update_varlen", ptr(a_log), ptr(a2), ptr(b2),
              a2.stride(0), ptr(dtb), ptr(qv), ptr(kv_), hq, qv.stride(0), ptr(vv), vv.stride(0),
              ptr(initial_state), ptr(final), ptr(out), t, ptr(cu), ptr(idx), n, slots,
              float(scale), flags, stream_handle(qv.device))
    return out, final


def fused_recurrent_gated_delta_rule_packed_decode(mixed_qkv, a, b, A_log, dt_bias, scale,
                                                   initial_state, out=None,
                                                   ssm_state_indices=None,
                                                   use_qk_l2norm_in_kernel: bool = True):
    """Mirror of vLLM's packed decode as the reference calls it
    (``vllm_fused_recurrent_gdn_packed_decode``, fle:6396-6417): B decode
    tokens, each its own sequence, read straight from the conv output
    ``mixed_qkv`` [B, 8192] bf16 (q | k | v columns); a, b [B, 32] bf16;
    token n updates slot ``ssm_state_indices[n]`` (default n) of the pool
    ``initial_state`` [slots, 32, 128 (v), 128 (k)] fp32 in place (slots
    outside [0, slots) are padding, skipped).  Returns (out [B, 1, 32, 128]
    bf16, initial_state).  ``out`` may be given (same shape, bf16)."""
    require(mixed_qkv, "mixed_qkv", torch.bfloat16, contiguous=False)
    if mixed_qkv.dim() != 2 or mixed_qkv.shape[1] != CONV_DIM or mixed_qkv.stride(1) != 1:
        raise ValueError("mixed_qkv must be [B, 8192] with unit inner stride")
    n = mixed_qkv.shape[0]
    if mixed_qkv.stride(0) % 8 or mixed_qkv.data_ptr() % 16:
        raise ValueError("mixed_qkv rows must be 16-byte aligned")
    a2, b2 = _ab_views(a, b, n)
    require(initial_state, "initial_state", torch.float32)
    if initial_state.dim() != 4 or tuple(initial_state.shape[1:]) != (HV, DV, DK):
        raise ValueError("initial_state must be [slots, 32, 128, 128]")
    if out is None:
        out = torch.empty(n, 1, HV, DV, dtype=torch.bfloat16, device=mixed_qkv.device)
    require(out, "out", torch.bfloat16)
    if out.numel() != n * HV * DV:
        raise ValueError("out must hold [B, 1, 32, 128]")
    idx = None
    if ssm_state_indices is not None:
        idx = _int32_vector(ssm_state_indices, "ssm_state_indices", n, mixed_qkv.device)
    base = mixed_qkv.data_ptr()
    a_log = A_log.float().contiguous()
    dtb = dt_bias.float().contiguous()
    _lib.call("qwen36_gdn_fused_gating_update_varlen", ptr(a_log), ptr(a2), ptr(b2),
              a2.stride(0), ptr(dtb), base, base + 2 * KEY_DIM, HK, mixed_qkv.stride(0),
              base + 2 * 2 * KEY_DIM, mixed_qkv.stride(0), ptr(initial_state), ptr(initial_state),
              ptr(out), n, None, ptr(idx), n, initial_state.shape[0], float(scale),
              1 if use_qk_l2norm_in_kernel else 0, stream_handle(mixed_qkv.device))
    return out, initial_state
