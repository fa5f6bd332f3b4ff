"""The reference's per-layer attention call signatures, as a drop-in.

In the reference engine the two mixers are closures inside ``run_with_torch``
(four_layer_mini_engine.py:2131) with the signatures

    full_attention(inp, layer_index, weights)      # fle:6546-6653
    linear_attention(inp, layer_index, weights)    # fle:6378-6544

and everything else they need is module state of that closure: the per-layer
KV caches ``full_attention_kv_caches[layer_index]`` (fle:4190), the carried
GDN states ``linear_attention_initial_{conv,ssm}_states[layer_index]`` (read)
and ``linear_attention_{conv,ssm}_states[layer_index]`` (written)
(fle:4268-4310), the position window ``position_start`` / ``position_end`` /
``tokens`` (``set_position_window``, fle:4489-4498) and ``mode``.

``MixerState`` holds exactly that state on the GPU, and ``full_attention`` /
``linear_attention`` below take the reference's arguments and read the
state made current with ``use_state`` (or bound with ``bind``).  Weights use
the reference's tensor names (``layer_tensor_names``, fle:1544-1570): q_proj,
k_proj, v_proj, o_proj, q_norm, k_norm; linear_in_proj_qkv / _z / _a / _b,
linear_conv1d ([8192, 1, 4]) or linear_conv1d_direct_weight ([8192, 4]),
linear_A_log, linear_dt_bias, linear_norm, linear_out_proj.

Every arithmetic step runs in the HIP library: one-token decode is the fused
projection GEMV, the one-launch decode step and the output GEMV; prefill is
the prefill projection GEMM, the head-norm/RoPE/KV-write or conv/gating
launches, the FMHA provider or chunked delta rule, the gate / gated norm and
the output GEMM.
"""
from __future__ import annotations

import contextlib

import torch

from . import full_attention as fa
from . import gated_deltanet as gd
from . import prefill_gemm as pg
from .projections import FusedProjection, gemv

HIDDEN = 2048


class MixerState:
    """Module state read by ``full_attention`` / ``linear_attention``
    (the closure variables of fle:2131 ``run_with_torch``)."""

    def __init__(self, device, mode: str = "prefill") -> None:
        self.device = torch.device(device)
        self.full_attention_kv_caches: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        self.linear_attention_initial_conv_states: dict[int, torch.Tensor] = {}
        self.linear_attention_initial_ssm_states: dict[int, torch.Tensor] = {}
        self.linear_attention_conv_states: dict[int, torch.Tensor] = {}
        self.linear_attention_ssm_states: dict[int, torch.Tensor] = {}
        self.mode = mode
        self.position_start = 0
        self.position_end = 0
        self.tokens = 0
        self._fused: dict[tuple, FusedProjection] = {}

    # -- state set-up (fle:4170-4310) ------------------------------------
    def add_full_attention_layer(self, layer_index: int, capacity: int) -> None:
        """Sequence-major caches [capacity, 2, 256] bf16 (the native layout,
        fle:4122-4126)."""
        k = torch.zeros(capacity, fa.HKV, fa.HEAD_DIM, dtype=torch.bfloat16, device=self.device)
        self.full_attention_kv_caches[layer_index] = (k, torch.zeros_like(k))

    def add_linear_attention_layer(self, layer_index: int,
                                   conv_state: torch.Tensor | None = None,
                                   ssm_state: torch.Tensor | None = None) -> None:
        """Initial conv state [8192, 3] bf16 and recurrent state [32, 128,
        128] fp32 (zeros unless given), plus the output buffers the layer
        writes."""
        conv = torch.zeros(gd.CONV_DIM, 3, dtype=torch.bfloat16, device=self.device)
        ssm = torch.zeros(gd.HV, gd.DK, gd.DV, dtype=torch.float32, device=self.device)
        if conv_state is not None:
            conv.copy_(conv_state)
        if ssm_state is not None:
            ssm.copy_(ssm_state)
        self.linear_attention_initial_conv_states[layer_index] = conv
        self.linear_attention_initial_ssm_states[layer_index] = ssm
        self.linear_attention_conv_states[layer_index] = torch.empty_like(conv)
        self.linear_attention_ssm_states[layer_index] = torch.empty_like(ssm)

    def set_position_window(self, position_start: int, tokens: int, mode: str | None = None) -> None:
        """fle:4489-4498: the call covers absolute positions
        [position_start, position_start + tokens)."""
        if tokens <= 0 or position_start < 0:
            raise ValueError("invalid position window")
        if mode is not None:
            if mode not in ("prefill", "decode"):
                raise ValueError("mode must be 'prefill' or 'decode'")
            self.mode = mode
        self.position_start = int(position_start)
        self.tokens = int(tokens)
        self.position_end = self.position_start + self.tokens

    def carry_linear_states(self) -> None:
        """Make the states the last call wrote the next call's initial states
        (the engine's hand-off between forward calls); the buffers swap, so
        nothing is copied."""
        for i in list(self.linear_attention_conv_states):
            a, b = self.linear_attention_initial_conv_states[i], self.linear_attention_conv_states[i]
            self.linear_attention_initial_conv_states[i], self.linear_attention_conv_states[i] = b, a
            a, b = self.linear_attention_initial_ssm_states[i], self.linear_attention_ssm_states[i]
            self.linear_attention_initial_ssm_states[i], self.linear_attention_ssm_states[i] = b, a

    def fused_projection(self, layer_index: int, kind: str, *weights: torch.Tensor) -> FusedProjection:
        """Row-concatenated projection weights, built once per layer
        (rebuilt if the weight tensors change)."""
        key = (layer_index, kind)
        tag = tuple((w.data_ptr(), tuple(w.shape)) for w in weights)
        fp = self._fused.get(key)
        if fp is None or fp.tag != tag:
            fp = FusedProjection(*weights)
            fp.tag = tag
            self._fused[key] = fp
        return fp


_ACTIVE: list[MixerState] = []


@contextlib.contextmanager
def use_state(state: MixerState):
    """Make ``state`` the module state that ``full_attention`` and
    ``linear_attention`` read."""
    _ACTIVE.append(state)
    try:
        yield state
    finally:
        _ACTIVE.pop()


def _state() -> MixerState:
    if not _ACTIVE:
        raise RuntimeError("no MixerState is active (use qwen36_attn.mixers.use_state)")
    return _ACTIVE[-1]


def _check_inp(st: MixerState, inp: torch.Tensor) -> int:
    if inp.dim() != 2 or inp.shape[1] != HIDDEN or inp.dtype != torch.bfloat16:
        raise ValueError("inp must be [tokens, 2048] bf16")
    if inp.shape[0] != st.tokens:
        raise ValueError(f"inp has {inp.shape[0]} rows, the position window {st.tokens}")
    return inp.shape[0]


def full_attention(inp: torch.Tensor, layer_index: int, weights: dict) -> torch.Tensor:
    """Drop-in for ``full_attention(inp, layer_index, weights)``
    (fle:6546-6653): q|gate, k, v projections; head RMSNorm (w + 1) + RoPE of
    q and k; K (normalised) and raw V written to cache rows
    [position_start, position_end); attention over rows [0, cache_end) with
    cache_end = position_end in decode or when the prefill extends a prefix,
    else tokens (causal, bottom-right when extending); sigmoid output gate;
    o_proj.  Returns [tokens, 2048] bf16."""
    st = _state()
    t = _check_inp(st, inp)
    k_cache, v_cache = st.full_attention_kv_caches[layer_index]
    if st.position_end > k_cache.shape[0]:
        raise ValueError("KV cache capacity exceeded")
    w = weights
    if st.mode == "decode":
        if t != 1:
            raise ValueError("decode takes one token")
        proj = st.fused_projection(layer_index, "qkv", w["q_proj"], w["k_proj"], w["v_proj"])
        q_gate, k, v = proj(inp)
        attn = fa.decode_step(q_gate, k, v, w["q_norm"], w["k_norm"], k_cache, v_cache,
                              st.position_start, st.position_end)
        return gemv(w["o_proj"], attn)
    cache_end = st.position_end if st.position_start > 0 else t
    proj = st.fused_projection(layer_index, "qkv", w["q_proj"], w["k_proj"], w["v_proj"])
    q_gate, k, v = proj.split_rows(pg.linear(inp, proj.w))
    q = fa.head_norm_rope_kv_write(q_gate, k, v, w["q_norm"], w["k_norm"], k_cache, v_cache,
                                   st.position_start)
    attn = fa.fmha_prefill_gated(q, k_cache[:cache_end], v_cache[:cache_end], q_gate)
    return pg.linear(attn, w["o_proj"])


def _conv_weight(weights: dict) -> torch.Tensor:
    w = weights.get("linear_conv1d_direct_weight")
    if w is None:
        w = weights["linear_conv1d"].reshape(gd.CONV_DIM, 4)
    return w.contiguous()


def linear_attention(inp: torch.Tensor, layer_index: int, weights: dict) -> torch.Tensor:
    """Drop-in for ``linear_attention(inp, layer_index, weights)``
    (fle:6378-6544, plain-torch numerics): in_proj qkv / z / a / b; causal
    conv1d + SiLU from ``linear_attention_initial_conv_states[layer_index]``
    (new state -> ``linear_attention_conv_states``); value head j reads key
    head j // 2; beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias);
    recurrent (decode) or chunked (prefill, chunk 64) delta rule from
    ``linear_attention_initial_ssm_states`` (final state ->
    ``linear_attention_ssm_states``); gated RMSNorm (weight without +1) with
    SiLU(z); out_proj.  Returns [tokens, 2048] bf16."""
    st = _state()
    t = _check_inp(st, inp)
    w = weights
    conv_in = st.linear_attention_initial_conv_states[layer_index]
    conv_out = st.linear_attention_conv_states[layer_index]
    ssm_in = st.linear_attention_initial_ssm_states[layer_index]
    ssm_out = st.linear_attention_ssm_states[layer_index]
    cw = _conv_weight(w)
    proj = st.fused_projection(layer_index, "qkvzba", w["linear_in_proj_qkv"],
                               w["linear_in_proj_z"], w["linear_in_proj_b"],
                               w["linear_in_proj_a"])
    # one GEMV (one token) or GEMM over the fused [qkv; z; b; a] rows
    mixed, z, b, a = proj(inp) if t == 1 else proj.split_rows(pg.linear(inp, proj.w))
    if st.mode == "decode":
        gated = gd.gdn_decode_step(mixed, conv_in, conv_out, cw, a, b, w["linear_A_log"],
                                   w["linear_dt_bias"], z, w["linear_norm"], ssm_in,
                                   final_state=ssm_out)
        return gemv(w["linear_out_proj"], gated) if t == 1 else pg.linear(gated, w["linear_out_proj"])
    conv, _ = gd.causal_conv1d(mixed, conv_in, cw, new_state=conv_out)
    q = conv[:, :gd.KEY_DIM].view(t, gd.HK, gd.DK)
    k = conv[:, gd.KEY_DIM:2 * gd.KEY_DIM].view(t, gd.HK, gd.DK)
    v = conv[:, 2 * gd.KEY_DIM:].view(t, gd.HV, gd.DV)
    g, beta = gd.gating(a, b, w["linear_A_log"], w["linear_dt_bias"])
    core, _ = gd.chunk_gated_delta_rule(q, k, v, g, beta, ssm_in, final_state=ssm_out)
    gated = gd.gated_rmsnorm(core, z, w["linear_norm"])
    return pg.linear(gated, w["linear_out_proj"])


def bind(state: MixerState):
    """The two mixers as closures over ``state``, the shape in which the
    reference engine holds them."""
    def _full(inp, layer_index, weights):
        with use_state(state):
            return full_attention(inp, layer_index, weights)

    def _linear(inp, layer_index, weights):
        with use_state(state):
            return linear_attention(inp, layer_index, weights)
    return _full, _linear
