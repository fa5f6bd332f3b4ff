"""CPU restatement (PyTorch, CPU tensors) of the reference's attention mixers.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  Nothing in the product
path imports this module.

Every function restates the arithmetic of one passage of the reference's
frozen Python engine, ``benchmarks/shape-lab/four_layer_mini_engine.py``
(cited below as ``fle:LINE``), where the functions are closures inside
``run_with_torch`` and therefore cannot be imported on their own.  Dtypes and
rounding points follow the reference text: activations are bf16 (``dtype``),
statistics and the delta rule are fp32.

Model geometry (``fle:2835-2873``): hidden 2048; full attention Hq=16, Hkv=2,
D=256, rotary_dim 64, rope_theta 1e7; Gated-DeltaNet Hk=16, Hv=32, dk=dv=128,
conv kernel 4, conv_dim 8192.

Pinning (what checks each function independently of this text) is listed in
``tests/test_oracle.py``; every function here has at least one such check.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

DTYPE = torch.bfloat16
HQ, HKV, HEAD_DIM = 16, 2, 256
Q_DIM, KV_DIM = HQ * HEAD_DIM, HKV * HEAD_DIM
ROTARY_DIM = 64
ROPE_THETA = 1.0e7
GDN_HK, GDN_HV, GDN_DK, GDN_DV = 16, 32, 128, 128
GDN_KEY_DIM = GDN_HK * GDN_DK          # 2048
GDN_VALUE_DIM = GDN_HV * GDN_DV        # 4096
GDN_CONV_DIM = 2 * GDN_KEY_DIM + GDN_VALUE_DIM  # 8192
GDN_CONV_KERNEL = 4
GDN_CONV_STATE = GDN_CONV_KERNEL - 1


# ----------------------------------------------------------------------------
# Full (gated GQA) attention
# ----------------------------------------------------------------------------

def inv_freq(rotary_dim: int = ROTARY_DIM, theta: float = ROPE_THETA) -> torch.Tensor:
    """fle:4470-4471 -- fp32 inverse frequencies 1/theta^(2i/rotary_dim)."""
    seq = torch.arange(0, rotary_dim, 2, dtype=torch.float32)
    return 1.0 / (theta ** (seq / rotary_dim))


def rope_cos_sin(position_start: int, count: int,
                 rotary_dim: int = ROTARY_DIM) -> tuple[torch.Tensor, torch.Tensor]:
    """fle:4489-4498 ``set_position_window`` -- cos/sin [count, 1, rotary_dim/2] fp32
    for absolute positions [position_start, position_start+count)."""
    positions = torch.arange(position_start, position_start + count, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq(rotary_dim))
    return torch.cos(freqs).unsqueeze(1), torch.sin(freqs).unsqueeze(1)


def head_rmsnorm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fle:5151-5153 -- per-head RMSNorm in fp32 with the ``(w + 1)`` convention,
    eps 1e-6, rounded to bf16."""
    var = x.float().pow(2).mean(dim=-1, keepdim=True)
    return (x.float() * torch.rsqrt(var + 1e-6) * (weight.float() + 1.0)).to(DTYPE)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               rotary_dim: int = ROTARY_DIM) -> torch.Tensor:
    """fle:5155-5162 -- rotate-half RoPE on dims [0, rotary_dim) in fp32; the
    remaining dims pass through untouched."""
    rot = x[..., :rotary_dim].float()
    rest = x[..., rotary_dim:]
    half = rotary_dim // 2
    a, b = rot[..., :half], rot[..., half:]
    roped = torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)
    return torch.cat((roped.to(DTYPE), rest), dim=-1)


def write_kv_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor,
                   v: torch.Tensor, position_start: int) -> None:
    """fle:5980-5986 (sequence-major layout [capacity, Hkv, D]) -- rows
    [start, start+T) receive the normalised+roped K and the raw V."""
    t = k.shape[0]
    k_cache[position_start:position_start + t].copy_(k)
    v_cache[position_start:position_start + t].copy_(v)


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      position_start: int, out_dtype: torch.dtype = DTYPE) -> torch.Tensor:
    """fle:6627-6648 -- ``F.scaled_dot_product_attention(..., enable_gqa=True)``
    over the cache rows [0, cache_end), cache_end = position_start + T.

    Mask: ``is_causal`` (top-left) when position_start == 0, otherwise the
    bottom-right mask key_pos <= query_pos (fle:6629-6638).  q [T,16,256],
    caches [>=S, 2, 256] -> [T, 4096].  ``out_dtype=float32`` evaluates the same
    formula on fp32 upcasts of the bf16 inputs, which is what the FMHA provider
    ABI returns (fp32 out, ``qrt_ck_fmha_q8192_provider.cpp:134-210``)."""
    t = q.shape[0]
    s = position_start + t
    kg = k_cache[:s].transpose(0, 1).unsqueeze(0)
    vg = v_cache[:s].transpose(0, 1).unsqueeze(0)
    qq = q.transpose(0, 1).unsqueeze(0)
    if out_dtype == torch.float32:
        qq, kg, vg = qq.float(), kg.float(), vg.float()
    mask = None
    if position_start > 0:
        qpos = torch.arange(position_start, s)
        kpos = torch.arange(s)
        mask = (kpos.unsqueeze(0) <= qpos.unsqueeze(1)).view(1, 1, t, s)
    out = F.scaled_dot_product_attention(qq, kg, vg, attn_mask=mask,
                                         is_causal=mask is None, enable_gqa=True)
    return out.squeeze(0).transpose(0, 1).reshape(t, HQ * q.shape[-1]).to(out_dtype)


def decode_attention_grouped_bf16(q: torch.Tensor, k_cache: torch.Tensor,
                                  v_cache: torch.Tensor, cache_end: int) -> torch.Tensor:
    """fle:6614-6626 (variant ``decode_grouped_bmm_bf16``) -- one query token:
    bf16 grouped bmm scores, x 1/sqrt(D), softmax, probs rounded to bf16, bf16
    bmm with V.  q [1,16,256] -> [1, 4096] bf16."""
    qg = q.view(HKV, HQ // HKV, q.shape[-1])
    kg = k_cache[:cache_end].transpose(0, 1)
    vg = v_cache[:cache_end].transpose(0, 1)
    scores = torch.matmul(qg, kg.transpose(-1, -2)) * (1.0 / math.sqrt(q.shape[-1]))
    probs = torch.softmax(scores, dim=-1).to(DTYPE)
    return torch.matmul(probs, vg).reshape(1, HQ * q.shape[-1])


def decode_attention_f32(q: torch.Tensor, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, cache_end: int) -> torch.Tensor:
    """fle:6614-6626 (fp32 branch, ``scores = matmul(q.float(), k.float())``) --
    the same grouped decode in fp32 throughout; returns fp32 [1, 4096]."""
    qg = q.view(HKV, HQ // HKV, q.shape[-1]).float()
    kg = k_cache[:cache_end].transpose(0, 1).float()
    vg = v_cache[:cache_end].transpose(0, 1).float()
    scores = torch.matmul(qg, kg.transpose(-1, -2)) * (1.0 / math.sqrt(q.shape[-1]))
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, vg).reshape(1, HQ * q.shape[-1])


def output_gate(attn: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """fle:6650 -- attn * sigmoid(gate) with the sigmoid rounded to bf16 first."""
    return attn * torch.sigmoid(gate).to(DTYPE)


def split_q_gate(q_gate: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fle:6560-6562 -- the fused q_proj row holds per head [Q(256) | Gate(256)]."""
    t = q_gate.shape[0]
    qg = q_gate.view(t, HQ, 2 * HEAD_DIM)
    q, gate = qg.chunk(2, dim=-1)
    return q, gate.reshape(t, Q_DIM)


def full_attention(inp: torch.Tensor, weights: dict, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, position_start: int, mode: str) -> torch.Tensor:
    """fle:6546-6653 (plain-torch branches) -- the whole gated GQA layer.

    ``mode`` is "prefill" or "decode".  Decode uses the grouped bf16 bmm
    (fle:6614-6626); prefill uses SDPA with the causal / bottom-right mask.
    The K/V caches are updated in place."""
    t = inp.shape[0]
    q_gate = inp @ weights["q_proj"].t()
    k = (inp @ weights["k_proj"].t()).view(t, HKV, HEAD_DIM)
    v = (inp @ weights["v_proj"].t()).view(t, HKV, HEAD_DIM)
    q, gate = split_q_gate(q_gate)
    cos, sin = rope_cos_sin(position_start, t)
    q = apply_rope(head_rmsnorm(q, weights["q_norm"]), cos, sin)
    k = apply_rope(head_rmsnorm(k, weights["k_norm"]), cos, sin)
    write_kv_cache(k_cache, v_cache, k, v, position_start)
    if mode == "decode":
        attn = decode_attention_grouped_bf16(q, k_cache, v_cache, position_start + t)
    else:
        attn = prefill_attention(q, k_cache, v_cache, position_start)
    attn = output_gate(attn, gate)
    return attn @ weights["o_proj"].t()


# ----------------------------------------------------------------------------
# Gated DeltaNet (linear attention)
# ----------------------------------------------------------------------------

def causal_conv1d(mixed_qkv: torch.Tensor, conv_state: torch.Tensor,
                  weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fle:5368-5386 (direct form with the carried state) and fle:5387-5403
    (``F.conv1d`` with groups=conv_dim; identical when the state is zero).

    mixed_qkv [T, C] bf16, conv_state [C, 3] bf16 (the previous three inputs,
    oldest first), weight [C, 4] (tap 3 multiplies the current token).  The
    convolution accumulates in fp32 (as ``F.conv1d`` does), is rounded to bf16,
    then SiLU is applied and rounded again.  Returns (out [T, C] bf16,
    new_state [C, 3] = last three inputs of [state | x])."""
    t = mixed_qkv.shape[0]
    window = torch.cat((conv_state.float(), mixed_qkv.t().float()), dim=-1)  # [C, 3+T]
    w = weight.float()
    acc = window[:, 0:t] * w[:, 0:1]
    for tap in range(1, GDN_CONV_KERNEL):
        acc = acc + window[:, tap:tap + t] * w[:, tap:tap + 1]
    conv = acc.to(DTYPE)
    out = F.silu(conv.float()).to(DTYPE).t().contiguous()
    new_state = window[:, -GDN_CONV_STATE:].to(conv_state.dtype).contiguous()
    return out, new_state


def l2norm(x: torch.Tensor) -> torch.Tensor:
    """fle:5164-5165 -- x * rsqrt(sum(x^2) + 1e-6) in fp32 (sum, not mean)."""
    return x.float() * torch.rsqrt(x.float().pow(2).sum(dim=-1, keepdim=True) + 1e-6)


def gdn_gating(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
               dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """fle:6507-6511 -- beta = sigmoid(b) evaluated in b's dtype (bf16 for the
    layer's projection output, so beta is rounded to bf16 before the delta
    rule upcasts it); g = -exp(A_log) * softplus(a + dt_bias) in fp32.
    Returns (g, beta), both fp32 [T, Hv]."""
    beta = torch.sigmoid(b).float()
    g = -a_log.float().exp().unsqueeze(0) * F.softplus(a.float() + dt_bias.float().unsqueeze(0))
    return g, beta


def split_gdn_qkv(conv_out: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """fle:6497-6505 -- split [T, 8192] into q,k [T,16,128] and v [T,32,128]
    (no head repeat; see ``repeat_kv_heads``)."""
    t = conv_out.shape[0]
    q, k, v = conv_out.split([GDN_KEY_DIM, GDN_KEY_DIM, GDN_VALUE_DIM], dim=-1)
    return (q.reshape(t, GDN_HK, GDN_DK), k.reshape(t, GDN_HK, GDN_DK),
            v.reshape(t, GDN_HV, GDN_DV))


def repeat_kv_heads(x: torch.Tensor) -> torch.Tensor:
    """fle:6502-6505 -- value head j reads key head j // 2 (repeat_interleave)."""
    return x.repeat_interleave(GDN_HV // GDN_HK, dim=1)


def chunk_gated_delta_rule(query, key, value, g, beta, initial_state, chunk_size: int = 64,
                           qk_l2norm: bool = True):
    """fle:5167-5240 ``torch_chunk_gated_delta_rule``.

    query/key [B,T,H,dk], value [B,T,H,dv] (any float dtype; heads already
    repeated to Hv), g/beta [B,T,H] fp32, initial_state [B,H,dk,dv] fp32.
    Returns (out [B,T,H,dv] bf16, final_state [B,H,dk,dv] fp32).  All
    arithmetic is fp32; the chunk loop is the WY/UT form with the forward
    substitution of fle:5207-5211.  ``qk_l2norm=False`` skips the l2norm of
    q and k (used by the vLLM form below)."""
    if qk_l2norm:
        query = l2norm(query)
        key = l2norm(key)
    query, key, value, beta, g = [x.transpose(1, 2).contiguous().to(torch.float32)
                                  for x in (query, key, value, beta, g)]
    bsz, nh, seq, dk = key.shape
    dv = value.shape[-1]
    pad = (chunk_size - seq % chunk_size) % chunk_size
    query = F.pad(query, (0, 0, 0, pad))
    key = F.pad(key, (0, 0, 0, pad))
    value = F.pad(value, (0, 0, 0, pad))
    beta = F.pad(beta, (0, pad))
    g = F.pad(g, (0, pad))
    total = seq + pad
    query = query * (1.0 / math.sqrt(dk))
    v_beta = value * beta.unsqueeze(-1)
    k_beta = key * beta.unsqueeze(-1)
    query, key, value, k_beta, v_beta = [x.reshape(bsz, nh, -1, chunk_size, x.shape[-1])
                                         for x in (query, key, value, k_beta, v_beta)]
    g = g.reshape(bsz, nh, -1, chunk_size)
    upper_incl = torch.triu(torch.ones(chunk_size, chunk_size, dtype=torch.bool), diagonal=0)
    g = g.cumsum(dim=-1)
    decay = ((g.unsqueeze(-1) - g.unsqueeze(-2)).tril().exp().float()).tril()
    attn = -((k_beta @ key.transpose(-1, -2)) * decay).masked_fill(upper_incl, 0)
    for i in range(1, chunk_size):
        row = attn[..., i, :i].clone()
        sub = attn[..., :i, :i].clone()
        attn[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
    attn = attn + torch.eye(chunk_size, dtype=attn.dtype)
    u = attn @ v_beta
    w = attn @ (k_beta * g.exp().unsqueeze(-1))
    state = initial_state.to(u)
    out = torch.zeros(bsz, nh, total // chunk_size, chunk_size, dv, dtype=u.dtype)
    upper_strict = torch.triu(torch.ones(chunk_size, chunk_size, dtype=torch.bool), diagonal=1)
    for c in range(total // chunk_size):
        q_c, k_c, u_c = query[:, :, c], key[:, :, c], u[:, :, c]
        a_c = (q_c @ k_c.transpose(-1, -2) * decay[:, :, c]).masked_fill_(upper_strict, 0)
        v_new = u_c - w[:, :, c] @ state
        inter = (q_c * g[:, :, c, :, None].exp()) @ state
        out[:, :, c] = inter + a_c @ v_new
        g_last = g[:, :, c, -1]
        state = (state * g_last[..., None, None].exp()
                 + (k_c * (g_last[..., None] - g[:, :, c]).exp()[..., None]).transpose(-1, -2) @ v_new)
    out = out.reshape(bsz, nh, -1, dv)[:, :, :seq]
    return out.transpose(1, 2).contiguous().to(DTYPE), state


def vllm_chunk_gated_delta_rule(q, k, v, g, beta, initial_state,
                                use_qk_l2norm_in_kernel: bool = False):
    """vLLM's ``chunk_gated_delta_rule`` as the reference calls it
    (fle:6474-6483; vLLM 0.19.1rc1.dev300+g29e5d1020, third-party code not
    under the reference tree).  Its published algorithm is the gated delta
    rule of torch_chunk_gated_delta_rule (fle:5167-5240) with three interface
    differences: q, k carry the 16 key heads (v-head j reads key head
    j // 2), the state is stored [Hv, dv, dk] (the transpose; the reference
    hands states over with ``.transpose(-1, -2)``, fle:5482-5502), and q, k are
    l2-normalised in the kernel only when ``use_qk_l2norm_in_kernel`` (the
    reference passes False: fused_post_conv_prep normalised them already).
    q, k [1,T,16,dk], v [1,T,32,dv], g/beta [1,T,32], initial_state
    [1,32,dv,dk] fp32 or None -> (o [1,T,32,dv] bf16, final_state
    [1,32,dv,dk] fp32)."""
    rep = v.shape[2] // q.shape[2]
    qq = q.repeat_interleave(rep, dim=2)
    kk = k.repeat_interleave(rep, dim=2)
    if initial_state is None:
        s0 = torch.zeros(1, v.shape[2], q.shape[-1], v.shape[-1])
    else:
        s0 = initial_state.float().transpose(-1, -2)
    o, s = chunk_gated_delta_rule(qq, kk, v, g, beta, s0, qk_l2norm=use_qk_l2norm_in_kernel)
    return o, s.transpose(-1, -2).contiguous()


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state):
    """fle:5242-5276 ``torch_recurrent_gated_delta_rule`` -- token-by-token
    update of the fp32 state S [B,H,dk,dv]: S *= e^g; kv = S^T k;
    delta = (v - kv) beta; S += k (x) delta; o = S^T q (q pre-scaled by
    1/sqrt(dk)).  Returns (out [B,T,H,dv] bf16, final_state fp32)."""
    query = l2norm(query)
    key = l2norm(key)
    query, key, value, beta, g = [x.transpose(1, 2).contiguous().to(torch.float32)
                                  for x in (query, key, value, beta, g)]
    bsz, nh, seq, dk = key.shape
    dv = value.shape[-1]
    query = query * (1.0 / math.sqrt(dk))
    out = torch.zeros(bsz, nh, seq, dv, dtype=value.dtype)
    state = initial_state.to(value)
    for t in range(seq):
        q_t, k_t, v_t = query[:, :, t], key[:, :, t], value[:, :, t]
        g_t = g[:, :, t].exp().unsqueeze(-1).unsqueeze(-1)
        b_t = beta[:, :, t].unsqueeze(-1)
        state = state * g_t
        kv_mem = (state * k_t.unsqueeze(-1)).sum(dim=-2)
        delta = (v_t - kv_mem) * b_t
        state = state + k_t.unsqueeze(-1) * delta.unsqueeze(-2)
        out[:, :, t] = (state * q_t.unsqueeze(-1)).sum(dim=-2)
    return out.transpose(1, 2).contiguous().to(DTYPE), state


def fused_sigmoid_gating_delta_rule_update(A_log, a, b, dt_bias, q, k, v, initial_state,
                                           use_qk_l2norm_in_kernel: bool = True,
                                           scale: float | None = None,
                                           softplus_threshold: float = 20.0):
    """The decode update the reference calls at fle:6429-6440 (vLLM
    ``fused_sigmoid_gating_delta_rule_update``, vLLM
    0.19.1rc1.dev300+g29e5d1020, module
    ``vllm.model_executor.layers.mamba.gdn_linear_attn``; third-party code not
    under the reference tree).  Its published algorithm, per token and value
    head j (key head j // (Hv / Hk)):
      g = -exp(A_log) * softplus(a + dt_bias)   (fp32, linear above 20)
      beta = sigmoid(b)                          (fp32, not rounded)
      q, k <- x / sqrt(sum(x^2) + 1e-6) if use_qk_l2norm_in_kernel; q *= scale
      H <- H e^g;  v' = (v - H k) beta;  H <- H + v' (x) k;  o = H q
    with the state H stored [Hv, dv, dk] (the transpose of the torch rule's
    [Hv, dk, dv], fle:5433).  q, k [1, T, Hk, dk], v [1, T, Hv, dv], a, b
    [T, Hv], initial_state [1, Hv, dv, dk] fp32 -> (o [1, T, Hv, dv] in q's
    dtype, final_state [1, Hv, dv, dk] fp32)."""
    hv, hk = v.shape[2], q.shape[2]
    dk = q.shape[-1]
    if scale is None:
        scale = dk ** -0.5
    x = a.float().reshape(-1, hv) + dt_bias.float().unsqueeze(0)
    sp = torch.where(x > softplus_threshold, x, torch.log1p(torch.exp(x)))
    g = -A_log.float().exp().unsqueeze(0) * sp
    beta = torch.sigmoid(b.float().reshape(-1, hv))
    qf = q[0].float().repeat_interleave(hv // hk, dim=1)
    kf = k[0].float().repeat_interleave(hv // hk, dim=1)
    if use_qk_l2norm_in_kernel:
        qf = qf * torch.rsqrt(qf.pow(2).sum(-1, keepdim=True) + 1e-6)
        kf = kf * torch.rsqrt(kf.pow(2).sum(-1, keepdim=True) + 1e-6)
    qf = qf * scale
    vf = v[0].float()
    state = initial_state[0].float().clone()          # [Hv, dv, dk]
    out = torch.empty(vf.shape, dtype=torch.float32)
    for t in range(vf.shape[0]):
        state = state * g[t].exp()[:, None, None]
        pred = (state * kf[t][:, None, :]).sum(-1)     # H k   [Hv, dv]
        vn = (vf[t] - pred) * beta[t][:, None]
        state = state + vn[:, :, None] * kf[t][:, None, :]
        out[t] = (state * qf[t][:, None, :]).sum(-1)   # H q
    return out.unsqueeze(0).to(q.dtype), state.unsqueeze(0)


def gated_rmsnorm(core: torch.Tensor, z: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fle:6531-6541 -- per 128-wide v-head: rmsnorm (mean, eps 1e-6) times
    ``weight`` (no +1), rounded to bf16, times SiLU(z), rounded to bf16.
    core [T,32,128], z [T,4096] -> [T,4096]."""
    t = core.shape[0]
    cf = core.reshape(-1, GDN_DV)
    zf = z.reshape(-1, GDN_DV)
    var = cf.float().pow(2).mean(dim=-1, keepdim=True)
    gated = (cf.float() * torch.rsqrt(var + 1e-6) * weight.float()).to(DTYPE)
    gated = (gated.float() * F.silu(zf.float())).to(DTYPE)
    return gated.view(t, GDN_VALUE_DIM)


def linear_attention(inp: torch.Tensor, weights: dict, conv_state: torch.Tensor,
                     ssm_state: torch.Tensor, mode: str, chunk_size: int = 64):
    """fle:6378-6544 (plain-torch branch, fle:6497-6541) -- the whole GDN layer.

    ``conv_state`` [8192,3] bf16 and ``ssm_state`` [32,128,128] fp32 are the
    layer's carried states; returns (out [T,2048], new_conv_state, new_ssm_state).
    Projections follow ``linear_input_projection``: qkv [T,8192], z [T,4096],
    a/b [T,32]."""
    mixed = inp @ weights["in_proj_qkv"].t()
    z = inp @ weights["in_proj_z"].t()
    b = inp @ weights["in_proj_b"].t()
    a = inp @ weights["in_proj_a"].t()
    conv_out, new_conv = causal_conv1d(mixed, conv_state, weights["conv1d"])
    q, k, v = split_gdn_qkv(conv_out)
    q, k = repeat_kv_heads(q), repeat_kv_heads(k)
    g, beta = gdn_gating(a, b, weights["A_log"], weights["dt_bias"])
    fn_args = (q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), g.unsqueeze(0),
               beta.unsqueeze(0), ssm_state.unsqueeze(0))
    if mode == "decode":
        core, final = recurrent_gated_delta_rule(*fn_args)
    else:
        core, final = chunk_gated_delta_rule(*fn_args, chunk_size=chunk_size)
    gated = gated_rmsnorm(core.squeeze(0), z, weights["norm"])
    return gated @ weights["out_proj"].t(), new_conv, final.squeeze(0)


# ---------------------------------------------------------------------------
# MoE block after attention (four_layer_mini_engine.py:8479-8650)
# ---------------------------------------------------------------------------
MOE_TOP_K = 8


def layer_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """fle:5127-5128 -- the layer RMSNorm: fp32 mean of squares, rsqrt,
    weight + 1, rounded to bf16."""
    variance = x.float().pow(2).mean(dim=-1, keepdim=True)
    return (x.float() * torch.rsqrt(variance + eps) * (weight.float() + 1.0)).to(DTYPE)


def moe_block(inp: torch.Tensor, attn_out: torch.Tensor, weights: dict,
              forced_ids: torch.Tensor | None = None, grouped: bool = False) -> torch.Tensor:
    """fle:8479-8490 residual + post-attention norm, fle:7775-7789 router
    (top-8 of the fp32 bf16 logits, softmax over the 8 -> bf16), fle:7791-7803
    routed experts ("expanded" form), fle:8240-8300 shared expert, fle:8636-8640
    sums.  inp, attn_out [T, 2048] bf16; returns [T, 2048] bf16.
    ``forced_ids`` [T, 8] replaces torch.topk's selection (for tied logits).
    ``grouped`` evaluates the routed experts one expert at a time (the rows
    routed to expert e times its weights, as the reference's prefill groups
    them, native_moe_prefill.hip.cpp:325-382) instead of gathering one weight
    matrix per (token, rank): the same per-row products, with memory that does
    not grow with T."""
    after = inp + attn_out
    h2 = layer_rmsnorm(after, weights["post_attention_layernorm"])
    t = h2.shape[0]
    logits = h2 @ weights["router"].t()
    scores, ids = torch.topk(logits.float(), k=MOE_TOP_K, dim=-1)
    if forced_ids is not None:
        ids = forced_ids.long().view(t, MOE_TOP_K)
        scores = logits.float().gather(-1, ids)
    rw = torch.softmax(scores, dim=-1).to(DTYPE)
    flat = ids.reshape(-1)
    if grouped:
        y = torch.empty(flat.numel(), h2.shape[1], dtype=DTYPE)
        for e in flat.unique().tolist():
            rows = (flat == e).nonzero().squeeze(1)
            projected = h2[rows // MOE_TOP_K] @ weights["expert_gate_up"][e].t()
            gate, up = projected.chunk(2, dim=-1)
            act = (F.silu(gate.float()) * up.float()).to(DTYPE)
            y[rows] = act @ weights["expert_down"][e].t()
    else:
        expanded = h2.repeat_interleave(MOE_TOP_K, dim=0)
        gate_up = weights["expert_gate_up"][flat].transpose(1, 2)
        projected = torch.bmm(expanded.unsqueeze(1), gate_up).squeeze(1)
        gate, up = projected.chunk(2, dim=-1)
        act = (F.silu(gate.float()) * up.float()).to(DTYPE)
        down = weights["expert_down"][flat].transpose(1, 2)
        y = torch.bmm(act.unsqueeze(1), down).squeeze(1)
    moe = (y.view(t, MOE_TOP_K, -1) * rw.unsqueeze(-1)).sum(dim=1)
    sg = h2 @ weights["shared_gate"].t()
    sgp = h2 @ weights["shared_gate_proj"].t()
    sup = h2 @ weights["shared_up_proj"].t()
    sact = (F.silu(sgp.float()) * sup.float()).to(DTYPE)
    shared = torch.sigmoid(sg).to(DTYPE) * (sact @ weights["shared_down_proj"].t())
    return after + (moe + shared)
