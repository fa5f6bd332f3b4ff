"""CPU checks that pin the oracle restatement (oracle/attention_oracle.py)
independently of its own text: reference-held constants, closed forms,
brute force in fp64 on tiny shapes, and invariants chosen so that a dropped
term, wrong sign/index or transposed operand fails.

Which check pins which function:
  inv_freq / rope_cos_sin   -> reference KAT table; closed-form rotation
  head_rmsnorm              -> fp64 formula; (w+1) convention (w=-1 -> 0)
  apply_rope                -> fp64 rotation, position 0 identity, norm
  prefill_attention         -> fp64 brute force with explicit mask loops;
                               GQA == MHA on repeated KV; prefix extension
  decode_attention_*        -> last row of prefill; fp64 brute force
  output_gate               -> sigmoid(0) = 1/2 exact; fp64 formula
  causal_conv1d             -> F.conv1d groups=C; state carry
  l2norm / gdn_gating       -> unit norms; fp64 closed form
  chunk/recurrent delta rule-> fp64 brute-force recurrence; chunked ==
                               recurrent; beta=0 pure decay; one step from
                               zero state; state carry across calls
  gated_rmsnorm             -> fp64 formula; weight without +1
  full_attention layer      -> fp64 per-head brute force of the whole layer
                               (prefill, prefix extension, decode), with
                               mutated brute forces that must fail;
                               prefill(T) + decode == prefill(T+1) tail
  split_q_gate / split_gdn_qkv / repeat_kv_heads / write_kv_cache
                            -> arange index identities, sentinel rows
  linear_attention layer    -> fp64 per-head brute force (conv with state,
                               key head j // 2, token-by-token delta rule,
                               gated norm without +1), mutated variants fail
  fused_sigmoid_gating_delta_rule_update (vLLM API)
                            -> fp64 brute-force recurrence with fp32 beta on
                               the transposed [Hv, dv, dk] state
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention_oracle as O
from tests.golden.rope_table import INV_FREQ_KAT

torch.manual_seed(0)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def test_inv_freq_matches_reference_table():
    got = O.inv_freq()
    kat = torch.tensor(INV_FREQ_KAT, dtype=torch.float32)
    assert torch.allclose(got, kat, rtol=3e-7, atol=0)
    exact = torch.tensor([1.0 / math.pow(1e7, 2 * i / 64) for i in range(32)], dtype=torch.float64)
    assert torch.allclose(kat.double(), exact, rtol=1e-7)


def test_rope_cos_sin_and_rotation():
    cos, sin = O.rope_cos_sin(5, 3)
    assert cos.shape == (3, 1, 32)
    pos = torch.tensor([5.0, 6.0, 7.0], dtype=torch.float64)
    ang = pos[:, None] * torch.tensor(INV_FREQ_KAT, dtype=torch.float64)[None]
    assert torch.allclose(cos[:, 0].double(), torch.cos(ang), atol=2e-6)
    assert torch.allclose(sin[:, 0].double(), torch.sin(ang), atol=2e-6)
    x = torch.randn(3, 2, 256, generator=gen(1)).to(torch.bfloat16)
    y = O.apply_rope(x, cos, sin)
    # dims >= 64 untouched; pair (i, i+32) rotated by angle i
    assert torch.equal(y[..., 64:], x[..., 64:])
    xf = x.double()
    a, b = xf[..., :32], xf[..., 32:64]
    c, s = torch.cos(ang)[:, None], torch.sin(ang)[:, None]
    ref = torch.cat((a * c - b * s, b * c + a * s), -1)
    assert (y[..., :64].double() - ref).abs().max() <= 0.02
    # position 0 is the identity
    c0, s0 = O.rope_cos_sin(0, 3)
    y0 = O.apply_rope(x, c0[:1].expand(3, 1, 32), s0[:1].expand(3, 1, 32))
    assert torch.equal(y0, x)


def test_head_rmsnorm_formula_and_plus_one():
    x = torch.randn(4, 3, 256, generator=gen(2)).to(torch.bfloat16)
    w = torch.randn(256, generator=gen(3)).to(torch.bfloat16)
    y = O.head_rmsnorm(x, w)
    xd = x.double()
    ref = xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) * (w.double() + 1)
    assert (y.double() - ref).abs().max() <= 2 ** -8 * ref.abs().max()
    assert torch.count_nonzero(O.head_rmsnorm(x, -torch.ones(256, dtype=torch.bfloat16))) == 0


def brute_attention(q, k, v, position_start):
    """fp64, explicit loops over query rows: softmax(q k^T / sqrt(D)) v with
    key j visible to query i iff j <= i + position_start; head h -> kv h // 8."""
    t, hq, d = q.shape
    out = torch.zeros(t, hq, d, dtype=torch.float64)
    for h in range(hq):
        kv = h // (hq // k.shape[1])
        for i in range(t):
            lim = i + position_start + 1
            s = (k[:lim, kv].double() @ q[i, h].double()) / math.sqrt(d)
            p = torch.softmax(s, 0)
            out[i, h] = p @ v[:lim, kv].double()
    return out.reshape(t, hq * d)


@pytest.mark.parametrize("t,s", [(1, 1), (5, 5), (3, 9), (17, 17), (4, 40)])
def test_prefill_attention_brute_force(t, s):
    g = gen(t * 100 + s)
    q = torch.randn(t, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    ref = brute_attention(q, k, v, s - t)
    got32 = O.prefill_attention(q, k, v, s - t, out_dtype=torch.float32)
    assert (got32.double() - ref).abs().max() <= 1e-5
    got16 = O.prefill_attention(q, k, v, s - t)
    assert (got16.double() - ref).abs().max() <= 2e-2


def test_prefill_gqa_equals_mha_and_prefix_extension():
    g = gen(9)
    s, t = 40, 12
    q = torch.randn(s, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    full = O.prefill_attention(q, k, v, 0, out_dtype=torch.float32)
    tail = O.prefill_attention(q[s - t:], k, v, s - t, out_dtype=torch.float32)
    assert torch.allclose(full[s - t:], tail, atol=1e-6)
    # GQA vs explicit per-head MHA with K/V repeated 8x
    kr = k.repeat_interleave(8, dim=1)
    vr = v.repeat_interleave(8, dim=1)
    mha = F.scaled_dot_product_attention(q.float().transpose(0, 1), kr.float().transpose(0, 1),
                                         vr.float().transpose(0, 1), is_causal=True)
    assert torch.allclose(full, mha.transpose(0, 1).reshape(s, 4096), atol=1e-5)


def test_decode_is_last_row_of_prefill():
    g = gen(10)
    s = 33
    q = torch.randn(s, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    pre = O.prefill_attention(q, k, v, 0, out_dtype=torch.float32)
    dec32 = O.decode_attention_f32(q[-1:], k, v, s)
    assert torch.allclose(pre[-1:], dec32, atol=1e-5)
    dec16 = O.decode_attention_grouped_bf16(q[-1:], k, v, s)
    assert (dec16.float() - dec32).abs().max() <= 2e-2
    # cache_end restricts the keys: same as a shorter cache
    assert torch.allclose(O.decode_attention_f32(q[-1:], k, v, 20),
                          O.decode_attention_f32(q[-1:], k[:20], v[:20], 20))


def test_output_gate_sigmoid_half():
    attn = torch.randn(2, 4096, generator=gen(11)).to(torch.bfloat16)
    assert torch.equal(O.output_gate(attn, torch.zeros(2, 4096, dtype=torch.bfloat16)),
                       attn * 0.5)
    gate = torch.randn(2, 4096, generator=gen(12)).to(torch.bfloat16)
    ref = attn.double() / (1 + torch.exp(-gate.double()))
    assert (O.output_gate(attn, gate).double() - ref).abs().max() <= 2e-2


def test_split_q_gate_layout():
    qg = torch.arange(2 * 8192, dtype=torch.float32).view(2, 8192)
    q, gate = O.split_q_gate(qg)
    assert q[1, 3, 0].item() == 8192 + 3 * 512
    assert gate[1, 3 * 256].item() == 8192 + 3 * 512 + 256


def test_causal_conv1d_textbook_and_carry():
    g = gen(13)
    c = 8192
    x = torch.randn(10, c, generator=g).to(torch.bfloat16)
    w = (torch.randn(c, 4, generator=g) * 0.5).to(torch.bfloat16)
    z = torch.zeros(c, 3, dtype=torch.bfloat16)
    out, st = O.causal_conv1d(x, z, w)
    ref = F.conv1d(x.t().unsqueeze(0).double(), w.double().unsqueeze(1), padding=3, groups=c)[..., :10]
    ref = F.silu(ref).squeeze(0).t()
    # two bf16 roundings (conv, then SiLU): <= 2 * 2^-9 relative
    assert ((out.double() - ref).abs() <= 2 ** -7 * ref.abs() + 1e-3).all()
    assert torch.equal(st, x[-3:].t().contiguous())
    o1, s1 = O.causal_conv1d(x[:4], z, w)
    o2, s2 = O.causal_conv1d(x[4:], s1, w)
    assert torch.equal(torch.cat((o1, o2)), out) and torch.equal(s2, st)
    # T < 3 keeps part of the old state
    o3, s3 = O.causal_conv1d(x[:1], st, w)
    assert torch.equal(s3, torch.cat((st[:, 1:], x[:1].t()), 1))


def test_l2norm_and_gating():
    x = torch.randn(7, 128, generator=gen(14))
    n = O.l2norm(x).norm(dim=-1)
    assert torch.allclose(n, torch.ones(7), atol=1e-5)
    a = torch.randn(5, 32, generator=gen(15)).to(torch.bfloat16)
    b = torch.randn(5, 32, generator=gen(16)).to(torch.bfloat16)
    a_log = torch.randn(32, generator=gen(17))
    dt = torch.randn(32, generator=gen(18))
    g, beta = O.gdn_gating(a, b, a_log, dt)
    ref_g = -torch.exp(a_log.double()) * torch.log1p(torch.exp(a.double() + dt.double()))
    assert torch.allclose(g.double(), ref_g, rtol=1e-5)
    # b is bf16 (a projection output), so sigmoid(b) is evaluated and rounded
    # in bf16 before the delta rule upcasts it (fle:6507): within half a bf16
    # ulp of the exact sigmoid, and exactly representable in bf16
    exact = torch.sigmoid(b.double())
    assert ((beta.double() - exact).abs() <= 2 ** -8 * exact + 1e-12).all()
    assert torch.equal(beta, beta.to(torch.bfloat16).float())
    # fp32 inputs keep an fp32 sigmoid
    _, beta32 = O.gdn_gating(a, b.float(), a_log, dt)
    assert torch.allclose(beta32.double(), exact, rtol=1e-6)


def brute_delta_rule(q, k, v, g, beta, s0, norm=True):
    """fp64 textbook gated delta rule, token by token, per head.
    q,k [T,H,dk] (raw; l2-normalised here unless ``norm`` is False), v
    [T,H,dv], g,beta [T,H], s0 [H,dk,dv]."""
    q = q.double()
    k = k.double()
    if norm:
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q = q / math.sqrt(q.shape[-1])
    s = s0.double().clone()
    outs = []
    for t in range(q.shape[0]):
        s = s * torch.exp(g[t].double())[:, None, None]
        pred = torch.einsum("hkv,hk->hv", s, k[t])
        delta = (v[t].double() - pred) * beta[t].double()[:, None]
        s = s + torch.einsum("hk,hv->hkv", k[t], delta)
        outs.append(torch.einsum("hkv,hk->hv", s, q[t]))
    return torch.stack(outs), s


def _gdn_inputs(t, h, seed, a_max=1.0):
    g = gen(seed)
    q = torch.randn(t, h, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(t, h, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(t, h, 128, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(t, h, generator=g))
    gg = -F.softplus(torch.randn(t, h, generator=g)) * (torch.rand(h, generator=g) * a_max)
    s0 = torch.randn(h, 128, 128, generator=g)
    return q, k, v, gg, beta, s0


@pytest.mark.parametrize("t", [1, 7, 64, 70])
def test_delta_rules_match_brute_force(t):
    q, k, v, gg, beta, s0 = _gdn_inputs(t, 3, seed=t)
    ref_o, ref_s = brute_delta_rule(q, k, v, gg, beta, s0)
    b = lambda x: x.unsqueeze(0)
    ro, rs = O.recurrent_gated_delta_rule(b(q), b(k), b(v), b(gg), b(beta), b(s0))
    co, cs = O.chunk_gated_delta_rule(b(q), b(k), b(v), b(gg), b(beta), b(s0))
    for o, s in ((ro, rs), (co, cs)):
        assert (o[0].double() - ref_o).abs().max() <= 2e-2
        assert ((s[0].double() - ref_s).norm() / ref_s.norm()) <= 1e-5


def test_vllm_chunk_rule_matches_fp64_brute_force():
    """Pins oracle.vllm_chunk_gated_delta_rule (vLLM's chunk API, fle:6474-6483):
    16 key heads read by v-head pairs, the [Hv, dv, dk] state, and q, k used
    as given without the in-kernel l2norm.  The brute force normalises inside,
    given the flag off, the brute force without its normalisation must agree;
    raw inputs must agree with the normalising brute force when the flag is
    on, and differ from it when it is off."""
    t = 70
    g = gen(77)
    q = torch.randn(t, 16, 128, generator=g)
    k = torch.randn(t, 16, 128, generator=g)
    v = torch.randn(t, 32, 128, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(t, 32, generator=g))
    gg = -F.softplus(torch.randn(t, 32, generator=g)) * 0.5
    s0 = torch.randn(32, 128, 128, generator=g)          # [Hv, dk, dv]
    qn = (q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    kn = (k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    rep = lambda x: x.repeat_interleave(2, dim=1)
    ref_o, ref_s = brute_delta_rule(rep(qn), rep(kn), v, gg, beta, s0, norm=False)
    b = lambda x: x.unsqueeze(0)
    o, s = O.vllm_chunk_gated_delta_rule(b(qn), b(kn), b(v), b(gg), b(beta),
                                         b(s0.transpose(-1, -2)), False)
    assert s.shape == (1, 32, 128, 128)
    assert (o[0].double() - ref_o).abs().max() <= 2e-2
    assert ((s[0].transpose(-1, -2).double() - ref_s).norm() / ref_s.norm()) <= 1e-5
    # raw inputs: the flag decides whether they are normalised
    qr, kr = (q * 0.1).to(torch.bfloat16), (k * 0.1).to(torch.bfloat16)
    ref_o2, ref_s2 = brute_delta_rule(rep(qr), rep(kr), v, gg, beta, s0)
    o_on, s_on = O.vllm_chunk_gated_delta_rule(b(qr), b(kr), b(v), b(gg), b(beta),
                                               b(s0.transpose(-1, -2)), True)
    o_off, s_off = O.vllm_chunk_gated_delta_rule(b(qr), b(kr), b(v), b(gg), b(beta),
                                                 b(s0.transpose(-1, -2)), False)
    assert (o_on[0].double() - ref_o2).abs().max() <= 2e-2
    assert ((s_off[0].transpose(-1, -2).double() - ref_s2).norm() / ref_s2.norm()) > 1e-2
    # zero initial state given as None
    oz, sz = O.vllm_chunk_gated_delta_rule(b(qn), b(kn), b(v), b(gg), b(beta), None, False)
    ref_oz, ref_sz = brute_delta_rule(rep(qn), rep(kn), v, gg, beta, torch.zeros(32, 128, 128),
                                      norm=False)
    assert (oz[0].double() - ref_oz).abs().max() <= 2e-2
    assert ((sz[0].transpose(-1, -2).double() - ref_sz).norm() / ref_sz.norm()) <= 1e-5


def test_chunk_size_invariance_and_carry():
    q, k, v, gg, beta, s0 = _gdn_inputs(100, 2, seed=5)
    b = lambda x: x.unsqueeze(0)
    o64, s64 = O.chunk_gated_delta_rule(b(q), b(k), b(v), b(gg), b(beta), b(s0), 64)
    for c in (16, 32):
        oc, sc = O.chunk_gated_delta_rule(b(q), b(k), b(v), b(gg), b(beta), b(s0), c)
        assert (oc.float() - o64.float()).abs().max() <= 2e-2
        assert ((sc - s64).norm() / s64.norm()) <= 1e-5
    o1, s1 = O.chunk_gated_delta_rule(b(q[:37]), b(k[:37]), b(v[:37]), b(gg[:37]), b(beta[:37]), b(s0))
    o2, s2 = O.chunk_gated_delta_rule(b(q[37:]), b(k[37:]), b(v[37:]), b(gg[37:]), b(beta[37:]), s1)
    assert (torch.cat((o1, o2), 1).float() - o64.float()).abs().max() <= 2e-2
    assert ((s2 - s64).norm() / s64.norm()) <= 1e-5


def test_delta_rule_special_cases():
    q, k, v, gg, beta, s0 = _gdn_inputs(6, 2, seed=6)
    b = lambda x: x.unsqueeze(0)
    # beta = 0: the state only decays; o = (q * e^{G}) S0 with G the cumsum
    ro, rs = O.recurrent_gated_delta_rule(b(q), b(k), b(v), b(gg), b(torch.zeros_like(beta)), b(s0))
    decay = torch.exp(gg.sum(0))
    assert torch.allclose(rs[0], s0 * decay[:, None, None], rtol=1e-5, atol=1e-6)
    # one step from the zero state: S = beta k (x) v with k l2-normalised
    zo, zs = O.recurrent_gated_delta_rule(b(q[:1]), b(k[:1]), b(v[:1]), b(gg[:1]), b(beta[:1]),
                                          torch.zeros(1, 2, 128, 128))
    kn = O.l2norm(k[0])
    ref = beta[0][:, None, None] * kn[:, :, None] * v[0].float()[:, None, :]
    assert torch.allclose(zs[0], ref, atol=1e-6)


def test_gated_rmsnorm_formula():
    core = torch.randn(3, 32, 128, generator=gen(19)).to(torch.bfloat16)
    z = torch.randn(3, 4096, generator=gen(20)).to(torch.bfloat16)
    w = torch.randn(128, generator=gen(21)).to(torch.bfloat16)
    got = O.gated_rmsnorm(core, z, w)
    cd = core.double().reshape(-1, 128)
    ref = cd / torch.sqrt(cd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    ref = ref.reshape(3, 4096) * F.silu(z.double())
    assert (got.double() - ref).abs().max() <= 3e-2 * max(1.0, ref.abs().max().item() / 4)


def test_full_attention_prefill_decode_consistency():
    from qwen36_attn import synthetic as syn
    g = syn.gen(22)
    w = syn.full_attention_weights(g)
    x = syn.randn((9, 2048), g, 0.5)
    kc = torch.zeros(9, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    full = O.full_attention(x, w, kc, vc, 0, "prefill")
    kc2 = torch.zeros_like(kc)
    vc2 = torch.zeros_like(kc)
    O.full_attention(x[:8], w, kc2, vc2, 0, "prefill")
    last = O.full_attention(x[8:], w, kc2, vc2, 8, "decode")
    assert (last.float() - full[8:].float()).abs().max() <= 2e-2
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


def test_moe_block_matches_fp64_per_expert_loop():
    """Pins oracle.moe_block (fle:7775-7803, 8240-8300, 8479-8640) with an fp64
    brute force written from the definitions: gate = first 512 rows of an
    expert's gate_up, up = the last 512, SiLU on the gate, routing weights =
    softmax over the 8 largest router logits, shared expert scaled by the
    sigmoid of its gate row, all added to the residual."""
    from qwen36_attn import synthetic as syn
    g = syn.gen(31)
    w = syn.moe_weights(g, n_experts=16)
    inp = syn.randn((2, 2048), g, 0.5)
    attn = syn.randn((2, 2048), g, 0.5)
    got = O.moe_block(inp, attn, w).double()
    got_grouped = O.moe_block(inp, attn, w, grouped=True).double()
    after = (inp.double() + attn.double())
    for t in range(2):
        a = after[t]
        h = a / torch.sqrt((a * a).mean() + 1e-6) * (w["post_attention_layernorm"].double() + 1)
        logits = w["router"].double() @ h
        top = torch.argsort(logits, descending=True)[:8]
        rw = torch.softmax(logits[top], dim=0)
        acc = torch.zeros(2048, dtype=torch.float64)
        for e, r in zip(top.tolist(), rw.tolist()):
            gu = w["expert_gate_up"][e].double() @ h
            act = torch.nn.functional.silu(gu[:512]) * gu[512:]
            acc += r * (w["expert_down"][e].double() @ act)
        sg = torch.sigmoid(w["shared_gate"].double() @ h)
        sact = torch.nn.functional.silu(w["shared_gate_proj"].double() @ h) * (w["shared_up_proj"].double() @ h)
        ref = a + acc + sg * (w["shared_down_proj"].double() @ sact)
        assert (got[t] - ref).abs().max().item() <= 2e-2 * max(1.0, ref.abs().max().item() / 8)
        assert (got_grouped[t] - ref).abs().max().item() <= 2e-2 * max(1.0, ref.abs().max().item() / 8)


def test_moe_block_grouped_equals_expanded():
    """The per-expert evaluation (prefill grouping) and the per-(token, rank)
    expanded form compute the same rows: 6 tokens over 8 experts, so every
    expert serves several rows."""
    from qwen36_attn import synthetic as syn
    g = syn.gen(33)
    w = syn.moe_weights(g, n_experts=8)
    inp = syn.randn((6, 2048), g, 0.5)
    attn = syn.randn((6, 2048), g, 0.5)
    a = O.moe_block(inp, attn, w).float()
    b = O.moe_block(inp, attn, w, grouped=True).float()
    assert (a - b).abs().max().item() <= 1e-2


def test_moe_block_forced_ids_equal_topk():
    from qwen36_attn import synthetic as syn
    g = syn.gen(32)
    w = syn.moe_weights(g, n_experts=12)
    inp = syn.randn((3, 2048), g, 0.5)
    attn = syn.randn((3, 2048), g, 0.5)
    h2 = O.layer_rmsnorm(inp + attn, w["post_attention_layernorm"])
    ids = torch.topk((h2 @ w["router"].t()).float(), 8, dim=-1).indices
    assert torch.equal(O.moe_block(inp, attn, w), O.moe_block(inp, attn, w, forced_ids=ids))


# ---------------------------------------------------------------------------
# Layout identities of the splitting / head-mapping / cache-write helpers
# ---------------------------------------------------------------------------

def test_split_gdn_qkv_and_repeat_layout():
    """fle:6497-6505: columns [0,2048) are q (16 heads x 128), [2048,4096) k,
    [4096,8192) v (32 heads x 128); value head j reads key head j // 2."""
    x = torch.arange(2 * 8192, dtype=torch.float64).view(2, 8192)
    q, k, v = O.split_gdn_qkv(x)
    assert q.shape == (2, 16, 128) and k.shape == (2, 16, 128) and v.shape == (2, 32, 128)
    t, h, d = torch.meshgrid(torch.arange(2), torch.arange(16), torch.arange(128), indexing="ij")
    assert torch.equal(q, (t * 8192 + h * 128 + d).double())
    assert torch.equal(k, (t * 8192 + 2048 + h * 128 + d).double())
    t, j, d = torch.meshgrid(torch.arange(2), torch.arange(32), torch.arange(128), indexing="ij")
    assert torch.equal(v, (t * 8192 + 4096 + j * 128 + d).double())
    r = O.repeat_kv_heads(q)
    assert r.shape == (2, 32, 128)
    for jj in range(32):
        assert torch.equal(r[:, jj], q[:, jj // 2])
    # interleave, not tile: heads 1 and 16 read different key heads
    assert not torch.equal(r[:, 1], q[:, 1]) and torch.equal(r[:, 1], q[:, 0])


def test_write_kv_cache_rows():
    """fle:5980-5986 (sequence-major): rows [start, start+T) take the new K/V,
    every other row keeps its old contents."""
    kc = torch.full((12, 2, 256), -7.0, dtype=torch.bfloat16)
    vc = torch.full((12, 2, 256), -9.0, dtype=torch.bfloat16)
    k = torch.arange(3 * 512, dtype=torch.float32).view(3, 2, 256).to(torch.bfloat16)
    v = (-torch.arange(3 * 512, dtype=torch.float32)).view(3, 2, 256).to(torch.bfloat16)
    O.write_kv_cache(kc, vc, k, v, 5)
    assert torch.equal(kc[5:8], k) and torch.equal(vc[5:8], v)
    assert (kc[:5] == -7).all() and (kc[8:] == -7).all()
    assert (vc[:5] == -9).all() and (vc[8:] == -9).all()


# ---------------------------------------------------------------------------
# Whole-layer brute forces (fp64, explicit per-head / per-token loops)
# ---------------------------------------------------------------------------

def _bf(x):
    """Round an fp64 tensor through bf16 (the reference's activation dtype)."""
    return x.to(torch.bfloat16).double()


def brute_full_attention(inp, w, k_cache, v_cache, start, decode, mutate=None):
    """fp64 gated GQA layer from the definitions (fle:6546-6653), one query
    row at a time.  Per head h the fused q-projection row holds [query(256) |
    gate(256)] at columns 512h..; head h reads KV head h // 8; head norm is
    x / sqrt(mean(x^2) + 1e-6) * (1 + w); RoPE rotates pairs (i, i + 32),
    i < 32, by angle pos * 1e7^(-2i/64) at the absolute position; softmax of
    q.k / 16 over keys 0..pos; output * sigmoid(gate); o_proj.  bf16 rounding
    is applied where the reference holds bf16 tensors.  The K/V rows are
    written into the (fp64) caches.  ``mutate`` names one deliberate wiring
    error (used to show the comparison detects it)."""
    t = inp.shape[0]
    x = inp.double()
    qg = _bf(x @ w["q_proj"].double().t())
    kk = _bf(x @ w["k_proj"].double().t()).view(t, 2, 256)
    vv = _bf(x @ w["v_proj"].double().t()).view(t, 2, 256)
    inv = torch.tensor([1e7 ** (-2.0 * i / 64) for i in range(32)], dtype=torch.float64)

    def norm_rope(vec, weight, pos):
        y = _bf(vec / torch.sqrt(vec.pow(2).mean() + 1e-6) * (1 + weight.double()))
        ang = pos * inv
        c, s = torch.cos(ang), torch.sin(ang)
        out = y.clone()
        if mutate == "rope_interleaved":      # pairs (2i, 2i+1) instead of (i, i+32)
            out[0:64:2] = y[0:64:2] * c - y[1:64:2] * s
            out[1:64:2] = y[1:64:2] * c + y[0:64:2] * s
        else:
            out[:32] = y[:32] * c - y[32:64] * s
            out[32:64] = y[32:64] * c + y[:32] * s
        return _bf(out)

    out = torch.zeros(t, 2048, dtype=torch.float64)
    for i in range(t):
        pos = start + i
        for kv in range(2):
            k_cache[pos, kv] = norm_rope(kk[i, kv], w["k_norm"], pos)
            v_cache[pos, kv] = vv[i, kv]
    for i in range(t):
        pos = start + i
        attn = torch.zeros(4096, dtype=torch.float64)
        for h in range(16):
            base = 512 * h if mutate != "gate_split" else 256 * h
            qpos = i if mutate == "q_pos_relative" else pos   # query rotated at its chunk offset
            qh = norm_rope(qg[i, base:base + 256], w["q_norm"], qpos)
            gate = qg[i, base + 256:base + 512]
            kv = h // 8 if mutate != "kv_head" else h % 2
            keys = k_cache[:pos + 1, kv]
            sc = keys @ qh / 16.0
            p = torch.softmax(sc, 0)
            o = p @ v_cache[:pos + 1, kv]
            attn[256 * h:256 * h + 256] = _bf(o) * _bf(torch.sigmoid(gate))
        out[i] = _bf(attn) @ w["o_proj"].double().t()
    return out


def test_full_attention_matches_fp64_brute_force():
    """Pins oracle.full_attention: prefill from position 0, prefill that
    extends the cached prefix (bottom-right mask), and a decode step, each
    against the fp64 brute force; mutated brute forces (wrong KV head, wrong
    gate split, RoPE pairs interleaved, queries rotated at chunk-relative
    positions) must miss by far more than the tolerance."""
    from qwen36_attn import synthetic as syn
    g = syn.gen(41)
    w = syn.full_attention_weights(g)
    x = syn.randn((11, 2048), g, 0.5)
    cap = 12
    kc = torch.zeros(cap, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    bk = torch.zeros(cap, 2, 256, dtype=torch.float64)
    bv = torch.zeros_like(bk)
    steps = [(0, 6, "prefill"), (6, 4, "prefill"), (10, 1, "decode")]
    for start, t, mode in steps:
        snap = (bk.clone(), bv.clone())
        got = O.full_attention(x[start:start + t], w, kc, vc, start, mode).double()
        ref = brute_full_attention(x[start:start + t], w, bk, bv, start, mode == "decode")
        err = (got - ref).abs().max().item()
        scale = ref.abs().max().item()
        assert err <= 1e-2 * scale, (mode, start, err, scale)
        assert torch.equal(kc[:start + t].double(), bk[:start + t])
        assert torch.equal(vc[:start + t].double(), bv[:start + t])
        # (a RoPE position shifted equally for queries and keys cancels in
        # q.k, so the position mutation rotates only the queries, relative to
        # the chunk start: it shows only when the prefill extends a prefix)
        muts = ["kv_head", "gate_split", "rope_interleaved"] + (["q_pos_relative"] if start else [])
        for m in muts:
            mk, mv = snap[0].clone(), snap[1].clone()
            bad = brute_full_attention(x[start:start + t], w, mk, mv, start, mode == "decode", m)
            assert (got - bad).abs().max().item() >= 10 * max(err, 1e-3 * scale), (m, mode)


def brute_linear_attention(inp, w, conv_state, ssm_state, mutate=None):
    """fp64 Gated-DeltaNet layer from the definitions (fle:6378-6544):
    in_proj qkv / z / a / b; per channel a causal 4-tap conv over the three
    carried inputs then the token, SiLU; value head j uses q, k of key head
    j // 2 (columns 128*(j//2) and 2048 + 128*(j//2)) and v columns
    4096 + 128 j; beta = sigmoid(b) (bf16), g = -exp(A_log) softplus(a +
    dt_bias); q, k l2-normalised, q / sqrt(128); per token S <- S e^g,
    S <- S + k (x) beta (v - S^T k), o = S^T q; gated norm
    o / sqrt(mean(o^2) + 1e-6) * w (no +1) * SiLU(z); out_proj.  Returns
    (out, new_conv_state, new_ssm_state)."""
    t = inp.shape[0]
    x = inp.double()
    mixed = _bf(x @ w["in_proj_qkv"].double().t())
    z = _bf(x @ w["in_proj_z"].double().t())
    a = _bf(x @ w["in_proj_a"].double().t())
    b = _bf(x @ w["in_proj_b"].double().t())
    if mutate == "swap_ab":
        a, b = b, a
    cw = w["conv1d"].double()
    window = torch.cat((conv_state.double(), mixed.t()), 1)     # [8192, 3 + T]
    y = torch.zeros(t, 8192, dtype=torch.float64)
    for i in range(t):
        acc = (window[:, i:i + 4] * cw).sum(1)
        y[i] = _bf(torch.nn.functional.silu(_bf(acc)))
    new_conv = window[:, -3:].clone()
    s = ssm_state.double().clone()
    core = torch.zeros(t, 32, 128, dtype=torch.float64)
    for i in range(t):
        for j in range(32):
            kh = j // 2 if mutate != "tile_heads" else j % 16
            qo, ko = (128 * kh, 2048 + 128 * kh) if mutate != "swap_qk" else (2048 + 128 * kh, 128 * kh)
            q = y[i, qo:qo + 128]
            k = y[i, ko:ko + 128]
            v = y[i, 4096 + 128 * j:4096 + 128 * j + 128]
            q = q / torch.sqrt((q * q).sum() + 1e-6) / math.sqrt(128)
            k = k / torch.sqrt((k * k).sum() + 1e-6)
            beta = _bf(torch.sigmoid(b[i, j]))
            xs = a[i, j] + w["dt_bias"][j].double()
            gg = -torch.exp(w["A_log"][j].double()) * torch.nn.functional.softplus(xs)
            s[j] = s[j] * torch.exp(gg)
            s[j] = s[j] + torch.outer(k, beta * (v - s[j].t() @ k))
            core[i, j] = _bf(s[j].t() @ q)
    gated = torch.zeros(t, 4096, dtype=torch.float64)
    for i in range(t):
        for j in range(32):
            o = core[i, j]
            nv = _bf(o / torch.sqrt(o.pow(2).mean() + 1e-6) * w["norm"].double())
            gated[i, 128 * j:128 * j + 128] = _bf(nv * torch.nn.functional.silu(z[i, 128 * j:128 * j + 128]))
    return gated @ w["out_proj"].double().t(), new_conv, s


def test_linear_attention_matches_fp64_brute_force():
    """Pins oracle.linear_attention: a chunked prefill from the zero state,
    then two decode steps carrying conv and recurrent state, against the fp64
    brute force (outputs within 2% of their scale, states to 1e-3 relative);
    mutated brute forces (heads tiled instead of interleaved, q/k column
    ranges swapped, a/b swapped) must miss by far more."""
    from qwen36_attn import synthetic as syn
    g = syn.gen(42)
    w = syn.linear_attention_weights(g, a_max=1.0)
    w["dt_bias"] = torch.randn(32, generator=g) * 0.5
    x = syn.randn((7, 2048), g, 0.5)
    conv = torch.zeros(8192, 3, dtype=torch.bfloat16)
    ssm = torch.zeros(32, 128, 128)
    bconv = torch.zeros(8192, 3, dtype=torch.float64)
    bssm = torch.zeros(32, 128, 128, dtype=torch.float64)
    for lo, hi, mode in [(0, 5, "prefill"), (5, 6, "decode"), (6, 7, "decode")]:
        snap = (bconv.clone(), bssm.clone())
        got, conv, ssm = O.linear_attention(x[lo:hi], w, conv, ssm, mode)
        ref, bconv, bssm = brute_linear_attention(x[lo:hi], w, bconv, bssm)
        err = (got.double() - ref).abs().max().item()
        scale = ref.abs().max().item()
        assert err <= 2e-2 * scale, (mode, err, scale)
        # the carried conv state is the last three bf16 projection rows: equal
        # up to the last-bit rounding of fp32- vs fp64-accumulated products
        assert ((conv.double() - bconv).abs() <= 2 ** -7 * bconv.abs()).all()
        assert ((ssm.double() - bssm).norm() / bssm.norm()).item() <= 1e-3
        for m in ("tile_heads", "swap_qk", "swap_ab"):
            bad, _, _ = brute_linear_attention(x[lo:hi], w, snap[0], snap[1], m)
            assert (got.double() - bad).abs().max().item() >= 5 * max(err, 1e-3 * scale), (m, mode)


def test_vllm_gating_update_matches_fp64_brute_force():
    """Pins oracle.fused_sigmoid_gating_delta_rule_update (the vLLM decode
    API the reference calls at fle:6429-6440): fp64 brute force with fp32
    beta = sigmoid(b) and the [Hv, dv, dk] state, 3 tokens; and with
    use_qk_l2norm_in_kernel=False the raw q, k enter unnormalised."""
    g = gen(43)
    t = 3
    q = torch.randn(1, t, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, t, 16, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, t, 32, 128, generator=g).to(torch.bfloat16)
    a = torch.randn(t, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(t, 32, generator=g).to(torch.bfloat16)
    a_log = torch.log(torch.rand(32, generator=g) * 4 + 0.1)
    dt = torch.randn(32, generator=g)
    h0 = torch.randn(1, 32, 128, 128, generator=g) * 0.1
    for norm in (True, False):
        o, h = O.fused_sigmoid_gating_delta_rule_update(a_log, a, b, dt, q, k, v, h0, norm)
        hh = h0[0].double().clone()
        for i in range(t):
            for j in range(32):
                qq, kk = q[0, i, j // 2].double(), k[0, i, j // 2].double()
                if norm:
                    qq = qq / torch.sqrt((qq * qq).sum() + 1e-6)
                    kk = kk / torch.sqrt((kk * kk).sum() + 1e-6)
                qq = qq / math.sqrt(128)
                xs = a[i, j].double() + dt[j].double()
                gg = -math.exp(a_log[j].item()) * (xs.item() if xs > 20 else math.log1p(math.exp(xs.item())))
                beta = 1 / (1 + math.exp(-b[i, j].item()))
                hh[j] = hh[j] * math.exp(gg)
                vn = (v[0, i, j].double() - hh[j] @ kk) * beta
                hh[j] = hh[j] + torch.outer(vn, kk)
                ref_o = hh[j] @ qq
                assert (o[0, i, j].double() - ref_o).abs().max() <= 1e-2 * max(1.0, ref_o.abs().max())
        assert ((h[0].double() - hh).norm() / hh.norm()).item() <= 1e-5
