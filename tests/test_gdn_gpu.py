"""GPU parity of the Gated-DeltaNet kernels against the CPU oracle
(four_layer_mini_engine.py:5167-5403, :6497-6541)."""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu

TOL_OUT = 2e-2      # max-abs-err on bf16 outputs (north_star)
TOL_STATE = 1e-3    # relative error on the fp32 state (north_star)


def rel_err(got, ref):
    return ((got.double() - ref.double()).norm() / ref.double().norm().clamp_min(1e-30)).item()


def _to(dev, *xs):
    return [x.to(dev) for x in xs]


@pytest.mark.parametrize("t,a_max,with_state", [
    (1, 16.0, False), (63, 16.0, True), (64, 0.1, False), (65, 0.1, True),
    (200, 1.0, True), (1024, 16.0, False), (1000, 0.05, True)])
def test_chunk_prefill_matches_oracle(gpu, t, a_max, with_state):
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(100 + t)
    q, k, v, gg, beta = syn.gdn_core_inputs(t, g, a_max=a_max)
    s0 = torch.randn(32, 128, 128, generator=g) if with_state else torch.zeros(32, 128, 128)
    print(f"gdn chunk T={t} a_max={a_max} state={with_state}", flush=True)
    qd, kd, vd, gd, bd, sd = _to(gpu, q, k, v, gg, beta, s0)
    out, st = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd if with_state else None)
    torch.cuda.synchronize()
    ref_o, ref_s = O.chunk_gated_delta_rule(
        O.repeat_kv_heads(q).unsqueeze(0), O.repeat_kv_heads(k).unsqueeze(0), v.unsqueeze(0),
        gg.unsqueeze(0), beta.unsqueeze(0), s0.unsqueeze(0))
    assert torch.isfinite(out).all()
    assert (out.cpu().float() - ref_o.float()).abs().max().item() <= TOL_OUT
    assert rel_err(st.cpu(), ref_s) <= TOL_STATE


def test_chunk_prefill_repeated_heads_match_unrepeated(gpu):
    """q/k given as 32 repeated heads (value head j reads head j) give the
    same bits as the 16 key heads (value head j reads head j // 2): each
    value head sees identical inputs, through the other head mapping."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(117)
    t = 130
    q, k, v, gg, beta = syn.gdn_core_inputs(t, g, a_max=4.0)
    s0 = torch.randn(32, 128, 128, generator=g)
    print(f"gdn chunk repeated heads T={t}", flush=True)
    qd, kd, vd, gd, bd, sd = _to(gpu, q, k, v, gg, beta, s0)
    o16, st16 = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd)
    q32 = qd.repeat_interleave(2, dim=-2).contiguous()
    k32 = kd.repeat_interleave(2, dim=-2).contiguous()
    o32, st32 = G.chunk_gated_delta_rule(q32, k32, vd, gd, bd, sd)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32)
    assert torch.equal(st16, st32)


@pytest.mark.parametrize("t,a_max", [(1, 16.0), (5, 0.1), (64, 1.0)])
def test_recurrent_matches_oracle(gpu, t, a_max):
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(200 + t)
    q, k, v, gg, beta = syn.gdn_core_inputs(t, g, a_max=a_max)
    s0 = torch.randn(32, 128, 128, generator=g)
    print(f"gdn recurrent T={t}", flush=True)
    qd, kd, vd, gd, bd, sd = _to(gpu, q, k, v, gg, beta, s0)
    out, st = G.recurrent_gated_delta_rule(qd, kd, vd, gd, bd, sd)
    torch.cuda.synchronize()
    ref_o, ref_s = O.recurrent_gated_delta_rule(
        O.repeat_kv_heads(q).unsqueeze(0), O.repeat_kv_heads(k).unsqueeze(0), v.unsqueeze(0),
        gg.unsqueeze(0), beta.unsqueeze(0), s0.unsqueeze(0))
    assert (out.cpu().float() - ref_o.float()).abs().max().item() <= TOL_OUT
    assert rel_err(st.cpu(), ref_s) <= TOL_STATE


def test_recurrent_in_place_state_and_repeated_heads(gpu):
    """state_out aliasing state_in, and q/k already repeated to 32 heads."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(7)
    q, k, v, gg, beta = syn.gdn_core_inputs(3, g, a_max=1.0)
    q32, k32 = O.repeat_kv_heads(q), O.repeat_kv_heads(k)
    s0 = torch.randn(32, 128, 128, generator=g)
    sd = s0.to(gpu)
    out, st = G.recurrent_gated_delta_rule(q32.to(gpu), k32.to(gpu), v.to(gpu), gg.to(gpu),
                                           beta.to(gpu), sd, final_state=sd)
    torch.cuda.synchronize()
    ref_o, ref_s = O.recurrent_gated_delta_rule(q32.unsqueeze(0), k32.unsqueeze(0),
                                                v.unsqueeze(0), gg.unsqueeze(0),
                                                beta.unsqueeze(0), s0.unsqueeze(0))
    assert rel_err(sd.cpu(), ref_s) <= TOL_STATE
    assert (out.cpu().float() - ref_o.float()).abs().max().item() <= TOL_OUT


def test_chunk_prefill_in_place_state(gpu):
    """state_out aliasing state_in (the layer's prefill path): bit-identical
    to a separate output buffer, with a ragged last chunk."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(8)
    q, k, v, gg, beta = [x.to(gpu) for x in syn.gdn_core_inputs(300, g, a_max=1.0)]
    s0 = torch.randn(32, 128, 128, generator=g).to(gpu)
    sep = torch.empty_like(s0)
    out_a, _ = G.chunk_gated_delta_rule(q, k, v, gg, beta, s0, final_state=sep)
    sd = s0.clone()
    out_b, _ = G.chunk_gated_delta_rule(q, k, v, gg, beta, sd, final_state=sd)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(sep, sd)


def test_config4_prefill_then_decode(gpu):
    """Config 4: chunked prefill of 8192 tokens from zero state, then 64
    recurrent decode steps carrying the fp32 state."""
    from qwen36_attn import gated_deltanet as G
    t, steps = 8192, 64
    g = syn.gen(4)
    q, k, v, gg, beta = syn.gdn_core_inputs(t + steps, g, a_max=16.0)
    print("gdn config4", flush=True)
    qd, kd, vd, gd, bd = _to(gpu, q, k, v, gg, beta)
    out, st = G.chunk_gated_delta_rule(qd[:t], kd[:t], vd[:t], gd[:t], bd[:t], None)
    st_prefill = st.cpu().clone()
    outs = []
    for i in range(t, t + steps):
        o, st = G.recurrent_gated_delta_rule(qd[i:i + 1], kd[i:i + 1], vd[i:i + 1], gd[i:i + 1],
                                             bd[i:i + 1], st, final_state=st)
        outs.append(o)
    torch.cuda.synchronize()
    R = O.repeat_kv_heads
    ref_o, ref_s = O.chunk_gated_delta_rule(R(q[:t]).unsqueeze(0), R(k[:t]).unsqueeze(0),
                                            v[:t].unsqueeze(0), gg[:t].unsqueeze(0),
                                            beta[:t].unsqueeze(0), torch.zeros(1, 32, 128, 128))
    assert (out.cpu().float() - ref_o.float()).abs().max().item() <= TOL_OUT
    assert rel_err(st_prefill, ref_s) <= TOL_STATE
    ref_d, ref_s2 = O.recurrent_gated_delta_rule(R(q[t:]).unsqueeze(0), R(k[t:]).unsqueeze(0),
                                                 v[t:].unsqueeze(0), gg[t:].unsqueeze(0),
                                                 beta[t:].unsqueeze(0), ref_s)
    got_d = torch.cat([o.cpu() for o in outs], dim=1)
    assert (got_d.float() - ref_d.float()).abs().max().item() <= TOL_OUT
    assert rel_err(st.cpu(), ref_s2) <= TOL_STATE


@pytest.mark.parametrize("t", [1, 2, 3, 17, 300, 1000, 4096, 4100])
def test_vector_pointwise_kernels_match_scalar_forms(gpu, t):
    """The 16-byte conv and gated-norm kernels (aligned inputs) give the
    scalar kernels' bits (the same inputs through an odd-strided view, which
    the library routes to the scalar forms); the conv's short-prompt form
    runs up to 4096 tokens, its long form from 4097."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(40 + t)
    x = syn.randn((t, 8192), g)
    w = syn.randn((8192, 4), g, 0.5)
    st = syn.randn((8192, 3), g)
    xd = x.to(gpu)
    wide = torch.zeros(t, 8193, dtype=torch.bfloat16, device=gpu)
    wide[:, 1:] = xd
    print(f"conv / gated norm vector vs scalar T={t}", flush=True)
    out_v, st_v = G.causal_conv1d(xd, st.to(gpu), w.to(gpu))
    out_s, st_s = G.causal_conv1d(wide[:, 1:], st.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out_v, out_s) and torch.equal(st_v, st_s)
    core = syn.randn((t, 32, 128), g).to(gpu)
    z = syn.randn((t, 4096), g).to(gpu)
    zw = torch.zeros(t, 4097, dtype=torch.bfloat16, device=gpu)
    zw[:, 1:] = z
    wn = syn.randn((128,), g, 0.5).to(gpu)
    n_v = G.gated_rmsnorm(core, z, wn)
    n_s = G.gated_rmsnorm(core, zw[:, 1:], wn)
    torch.cuda.synchronize()
    assert torch.equal(n_v, n_s)


def test_vector_conv_silu_every_input_value(gpu):
    """The vector conv's SiLU (hardware exp2 / rcp with the exact form near
    bf16 rounding midpoints) against the scalar kernel's exact form for all
    65536 bf16 conv values: taps (0, 0, 0, 1) make the conv value the input
    itself on every fourth row (the rows between are zero; non-finite inputs
    make NaNs there in both kernels)."""
    from qwen36_attn import gated_deltanet as G
    pats = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(8, 8192)
    x = torch.zeros(32, 8192, dtype=torch.bfloat16)
    x[0::4] = pats.view(torch.bfloat16)
    w = torch.zeros(8192, 4, dtype=torch.bfloat16)
    w[:, 3] = 1.0
    st = torch.zeros(8192, 3, dtype=torch.bfloat16)
    xd = x.to(gpu)
    wide = torch.zeros(32, 8193, dtype=torch.bfloat16, device=gpu)
    wide[:, 1:] = xd
    print("conv SiLU over all bf16 inputs", flush=True)
    out_v, _ = G.causal_conv1d(xd, st.to(gpu), w.to(gpu))
    out_s, _ = G.causal_conv1d(wide[:, 1:], st.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    nan = torch.isnan(out_s)
    assert torch.equal(torch.isnan(out_v), nan)
    assert torch.equal(out_v.view(torch.int16)[~nan], out_s.view(torch.int16)[~nan])
    # NaN conv values only from the 254 NaN inputs and -inf (-inf / inf)
    assert nan[0::4].sum().item() == 255


def test_conv1d_gating_norm(gpu):
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(11)
    for t, with_state in ((1, True), (2, True), (77, False), (300, True)):
        x = syn.randn((t, 8192), g)
        w = syn.randn((8192, 4), g, 0.5)
        st = syn.randn((8192, 3), g) if with_state else torch.zeros(8192, 3, dtype=torch.bfloat16)
        out, ns = G.causal_conv1d(x.to(gpu), st.to(gpu), w.to(gpu))
        ref, ref_s = O.causal_conv1d(x, st, w)
        assert (out.cpu().float() - ref.float()).abs().max().item() <= TOL_OUT
        assert torch.equal(ns.cpu(), ref_s)
        # in-place state
        sd = st.to(gpu)
        out2, _ = G.causal_conv1d(x.to(gpu), sd, w.to(gpu), new_state=sd)
        assert torch.equal(sd.cpu(), ref_s) and torch.equal(out2.cpu(), out.cpu())
    a = syn.randn((50, 32), g)
    b = syn.randn((50, 32), g)
    a_log = torch.log(torch.rand(32, generator=g) * 16).float()
    dt = torch.randn(32, generator=g) * 0.1
    gg, beta = G.gating(a.to(gpu), b.to(gpu), a_log.to(gpu), dt.to(gpu))
    rg, rb = O.gdn_gating(a, b, a_log, dt)
    assert torch.allclose(gg.cpu(), rg, rtol=1e-5, atol=1e-6)
    # beta is sigmoid(b) rounded to bf16 (fle:6507): equal to the oracle's up
    # to one bf16 ulp where the fp32 sigmoids round on either side of a tie
    assert torch.equal(beta.cpu(), beta.cpu().to(torch.bfloat16).float())
    assert ((beta.cpu() - rb).abs() <= 2 ** -8 * rb).all()
    assert (beta.cpu() == rb).float().mean().item() >= 0.99
    # fp32 beta (vLLM fused gating)
    _, beta32 = G.gating(a.to(gpu), b.to(gpu), a_log.to(gpu), dt.to(gpu), beta_fp32=True)
    assert torch.allclose(beta32.cpu(), torch.sigmoid(b.float()), rtol=1e-5, atol=1e-6)
    core = syn.randn((40, 32, 128), g)
    z = syn.randn((40, 4096), g)
    wn = syn.randn((128,), g, 0.5)
    out = G.gated_rmsnorm(core.to(gpu), z.to(gpu), wn.to(gpu))
    ref = O.gated_rmsnorm(core, z, wn)
    assert (out.cpu().float() - ref.float()).abs().max().item() <= TOL_OUT


def test_chunk_prefill_max_tokens_tail(gpu):
    """T = 262144, the largest accepted: every output finite, and the
    full-length prefill's last 64 outputs and final state equal the oracle's
    recurrence over those 64 tokens started from the state the kernels reach
    after the first T - 64 tokens (a prefill of that prefix: the same chunk
    sequence)."""
    from qwen36_attn import gated_deltanet as G
    t, tail = 262144, 64
    g = torch.Generator(device=gpu).manual_seed(9)
    q = torch.randn(t, 16, 128, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(t, 16, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(t, 32, 128, generator=g, device=gpu).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(t, 32, generator=g, device=gpu))
    a = torch.rand(32, generator=g, device=gpu) * 16.0
    gg = (-torch.nn.functional.softplus(torch.randn(t, 32, generator=g, device=gpu)) * a).float()
    print("gdn chunk max tokens", flush=True)
    out, st = G.chunk_gated_delta_rule(q, k, v, gg, beta, None)
    out, st = out.clone(), st.clone()
    _, st_head = G.chunk_gated_delta_rule(q[:-tail], k[:-tail], v[:-tail], gg[:-tail],
                                          beta[:-tail], None)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    R = O.repeat_kv_heads
    ref_o, ref_s = O.recurrent_gated_delta_rule(
        R(q[-tail:].cpu()).unsqueeze(0), R(k[-tail:].cpu()).unsqueeze(0),
        v[-tail:].cpu().unsqueeze(0), gg[-tail:].cpu().unsqueeze(0),
        beta[-tail:].cpu().float().unsqueeze(0), st_head.cpu().reshape(1, 32, 128, 128))
    got = out.reshape(t, -1)[-tail:].cpu().float()
    assert (got - ref_o.float().reshape(tail, -1)).abs().max().item() <= TOL_OUT
    assert rel_err(st.cpu(), ref_s.reshape(st.shape)) <= TOL_STATE
    del q, k, v, beta, gg, out
    torch.cuda.empty_cache()


def test_chunk_prefill_graph_replays_match_eager(gpu):
    """4096 tokens (64 chunks: the prep / scan overlap path with its second
    stream and events) captured in a graph: three replays, with eager work
    and synchronisation between them, each bit-identical to the eager call."""
    from qwen36_attn import gated_deltanet as G
    t = 4096
    g = syn.gen(41)
    q, k, v, gg, beta = syn.gdn_core_inputs(t, g, a_max=1.0)
    s0 = torch.randn(32, 128, 128, generator=g)
    qd, kd, vd, gd, bd, sd = _to(gpu, q, k, v, gg, beta, s0)
    print("gdn chunk graph", flush=True)
    ref_o, ref_s = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd)
    ref_o, ref_s = ref_o.clone(), ref_s.clone()
    out = torch.empty_like(ref_o)
    fin = torch.empty_like(ref_s)

    def run():
        o, s = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd)
        out.copy_(o)
        fin.copy_(s)
    run()   # workspace allocated outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for i in range(3):
        out.zero_()
        fin.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), i
        assert torch.equal(fin, ref_s), i
        G.chunk_gated_delta_rule(qd[:100], kd[:100], vd[:100], gd[:100], bd[:100], None)
        torch.cuda.synchronize()


def test_config4_conv_from_mixed_qkv_then_chunk_prefill(gpu):
    """Config 4 from its first step: the depthwise causal conv + SiLU over
    mixed_qkv [8192, 8192] (zero conv state), its output split into q, k
    [8192, 16, 128] and v [8192, 32, 128] in place, then the chunked prefill
    (chunk 64) from the zero state -- against the oracle's conv, split,
    head repeat and chunked rule (fle:5293-5403, 6497-6505, 5167-5240)."""
    from qwen36_attn import gated_deltanet as G
    t = 8192
    g = syn.gen(44)
    mixed = syn.randn((t, 8192), g)
    w = syn.randn((8192, 4), g, 0.5)
    _, _, _, gg, beta = syn.gdn_core_inputs(t, g, a_max=16.0)
    print("gdn config4 conv + chunk prefill", flush=True)
    zero = torch.zeros(8192, 3, dtype=torch.bfloat16)
    conv_d, st_d = G.causal_conv1d(mixed.to(gpu), zero.to(gpu), w.to(gpu))
    q = conv_d[:, :2048].view(t, 16, 128)
    k = conv_d[:, 2048:4096].view(t, 16, 128)
    v = conv_d[:, 4096:].view(t, 32, 128)
    out, st = G.chunk_gated_delta_rule(q, k, v, gg.to(gpu), beta.to(gpu), None)
    torch.cuda.synchronize()
    ref_conv, ref_cst = O.causal_conv1d(mixed, zero, w)
    assert (conv_d.cpu().float() - ref_conv.float()).abs().max().item() <= TOL_OUT
    assert (conv_d.cpu() == ref_conv).float().mean().item() >= 0.99
    assert torch.equal(st_d.cpu(), ref_cst)
    rq, rk, rv = O.split_gdn_qkv(ref_conv)
    R = O.repeat_kv_heads
    ref_o, ref_s = O.chunk_gated_delta_rule(R(rq).unsqueeze(0), R(rk).unsqueeze(0),
                                            rv.unsqueeze(0), gg.unsqueeze(0), beta.unsqueeze(0),
                                            torch.zeros(1, 32, 128, 128))
    assert (out.cpu().float() - ref_o.float()).abs().max().item() <= TOL_OUT
    assert rel_err(st.cpu(), ref_s) <= TOL_STATE


def test_chunk_prefill_ignores_stale_workspace(gpu):
    """The chunked prefill's result does not depend on what the workspace held
    before the call: a workspace pre-filled with NaN bytes gives the same bits
    as a fresh call (the prep writes every record byte the scan reads)."""
    from qwen36_attn import gated_deltanet as G
    from qwen36_attn import _tensors
    t = 200
    g = syn.gen(321)
    q, k, v, gg, beta = syn.gdn_core_inputs(t, g, a_max=1.0)
    s0 = torch.randn(32, 128, 128, generator=g)
    qd, kd, vd, gd, bd, sd = _to(gpu, q, k, v, gg, beta, s0)
    print("gdn chunk stale workspace T=200", flush=True)
    out1, st1 = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd)
    out1, st1 = out1.clone(), st1.clone()
    _tensors._SCRATCH[("gdn_chunk", gpu.index or 0)].fill_(0xFF)   # every float NaN
    out2, st2 = G.chunk_gated_delta_rule(qd, kd, vd, gd, bd, sd)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2) and torch.equal(st1, st2)
