"""The reference's call signatures, called exactly as the reference calls
them, against the oracle on identical seeded inputs:

  * full_attention(inp, layer_index, weights) / linear_attention(inp,
    layer_index, weights) (four_layer_mini_engine.py:6546, :6378) over a
    MixerState holding the module state they read (caches, carried GDN
    states, position window, mode);
  * vLLM's fused_sigmoid_gating_delta_rule_update(A_log, a, b, dt_bias, q, k,
    v, initial_state, inplace_final_state, use_qk_l2norm_in_kernel)
    (fle:6429-6440) with the [Hv, dv, dk] state, its batched cu_seqlens /
    ssm_state_indices form and the packed decode (fle:6396-6417);
  * vLLM's chunk_gated_delta_rule(q, k, v, g, beta, initial_state,
    output_final_state, use_qk_l2norm_in_kernel) (fle:6474-6483).
"""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _ref_weights_full(g):
    w = syn.full_attention_weights(g)
    return w, dict(w)   # the reference's tensor names are the same (fle:1550-1555)


def _ref_weights_linear(g):
    w = syn.linear_attention_weights(g, a_max=4.0)
    w["dt_bias"] = torch.randn(32, generator=g) * 0.5
    ref_names = {
        "linear_in_proj_qkv": w["in_proj_qkv"], "linear_in_proj_z": w["in_proj_z"],
        "linear_in_proj_a": w["in_proj_a"], "linear_in_proj_b": w["in_proj_b"],
        "linear_conv1d": w["conv1d"].view(8192, 1, 4), "linear_A_log": w["A_log"],
        "linear_dt_bias": w["dt_bias"], "linear_norm": w["norm"],
        "linear_out_proj": w["out_proj"],
    }
    return w, ref_names


def test_full_attention_signature(gpu):
    """Prefill 96 tokens, a prefill of 40 that extends the cached prefix, then
    4 decode steps, all through full_attention(inp, layer_index, weights)."""
    from qwen36_attn import mixers as M
    g = syn.gen(61)
    w_cpu, named = _ref_weights_full(g)
    wd = {k: v.to(gpu) for k, v in named.items()}
    x = syn.randn((140, 2048), g, 0.5)
    layer = 3
    st = M.MixerState(gpu)
    st.add_full_attention_layer(layer, 160)
    kc = torch.zeros(160, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for start, t, mode in [(0, 96, "prefill"), (96, 40, "prefill"), (136, 1, "decode"),
                           (137, 1, "decode"), (138, 1, "decode"), (139, 1, "decode")]:
        print(f"full_attention drop-in {mode} start={start} T={t}", flush=True)
        st.set_position_window(start, t, mode)
        with M.use_state(st):
            got = M.full_attention(x[start:start + t].to(gpu), layer, wd)
        ref = O.full_attention(x[start:start + t], w_cpu, kc, vc, start, mode)
        err = (got.cpu().float() - ref.float()).abs().max().item()
        assert err <= TOL, (mode, start, err)
        kg, vg = st.full_attention_kv_caches[layer]
        end = start + t
        # V rows are the raw v projection: GPU and CPU GEMMs accumulate in a
        # different order, so they agree to the last bf16 bit of the sum
        dv = (vg[:end].cpu().float() - vc[:end].float()).abs()
        assert (dv <= 2 ** -7 * vc[:end].float().abs() + 1e-6).all()
        assert (kg[:end].cpu().float() - kc[:end].float()).abs().max().item() <= TOL


def test_linear_attention_signature(gpu):
    """Prefill 130 tokens from the zero state, then 3 one-token decode steps
    and one 2-token decode, each carrying the conv and recurrent states, all
    through linear_attention(inp, layer_index, weights) (bound as closures,
    the shape in which the engine holds them)."""
    from qwen36_attn import mixers as M
    g = syn.gen(62)
    w_cpu, named = _ref_weights_linear(g)
    wd = {k: v.to(gpu) for k, v in named.items()}
    x = syn.randn((135, 2048), g, 0.5)
    layer = 0
    st = M.MixerState(gpu)
    st.add_linear_attention_layer(layer)
    _, linear = M.bind(st)
    conv = torch.zeros(8192, 3, dtype=torch.bfloat16)
    ssm = torch.zeros(32, 128, 128)
    for lo, hi, mode in [(0, 130, "prefill"), (130, 131, "decode"), (131, 132, "decode"),
                         (132, 133, "decode"), (133, 135, "decode")]:
        print(f"linear_attention drop-in {mode} [{lo}, {hi})", flush=True)
        st.set_position_window(lo, hi - lo, mode)
        got = linear(x[lo:hi].to(gpu), layer, wd)
        ref, conv, ssm = O.linear_attention(x[lo:hi], w_cpu, conv, ssm, mode)
        err = (got.cpu().float() - ref.float()).abs().max().item()
        assert err <= TOL, (mode, lo, err)
        # the conv state is the last three rows of the qkv projection (GPU vs
        # CPU GEMM: equal to the last bf16 bit)
        dc = (st.linear_attention_conv_states[layer].cpu().float() - conv.float()).abs()
        assert (dc <= 2 ** -7 * conv.float().abs() + 1e-6).all()
        fin = st.linear_attention_ssm_states[layer].cpu()
        assert ((fin - ssm).norm() / ssm.norm()).item() <= 1e-3
        st.carry_linear_states()


@pytest.mark.parametrize("t,norm,inplace", [(1, True, True), (1, False, False), (4, True, False)])
def test_fused_sigmoid_gating_delta_rule_update(gpu, t, norm, inplace):
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(63 + t)
    q = syn.randn((1, t, 16, 128), g)
    k = syn.randn((1, t, 16, 128), g)
    v = syn.randn((1, t, 32, 128), g)
    a = syn.randn((t, 32), g)
    b = syn.randn((t, 32), g)
    a_log = torch.log(torch.rand(32, generator=g) * 8 + 0.05).float()
    dt = (torch.randn(32, generator=g) * 0.5).float()
    h0 = torch.randn(1, 32, 128, 128, generator=g) * 0.2
    if not norm:   # unnormalised keys: keep the update contractive
        k = (k.float() * 0.05).to(torch.bfloat16)
        q = (q.float() * 0.05).to(torch.bfloat16)
    print(f"fused gating update T={t} l2norm={norm} inplace={inplace}", flush=True)
    d = lambda x: x.to(gpu)
    state = d(h0).contiguous()
    o, fin = G.fused_sigmoid_gating_delta_rule_update(
        A_log=d(a_log), a=d(a), b=d(b), dt_bias=d(dt), q=d(q), k=d(k), v=d(v),
        initial_state=state, inplace_final_state=inplace, use_qk_l2norm_in_kernel=norm)
    ro, rs = O.fused_sigmoid_gating_delta_rule_update(a_log, a, b, dt, q, k, v, h0, norm)
    assert o.shape == (1, t, 32, 128) and fin.shape == (1, 32, 128, 128)
    assert (o.cpu().float() - ro.float()).abs().max().item() <= TOL
    assert ((fin.cpu() - rs).norm() / rs.norm()).item() <= 1e-3
    if inplace:
        assert fin.data_ptr() == state.data_ptr()
    else:
        assert torch.equal(state.cpu(), h0)
    # the same update through the torch-orientation recurrent rule
    # (state transposed) agrees with the vLLM-orientation one
    if norm:
        x = a.float() + dt
        g_t = -a_log.exp() * torch.nn.functional.softplus(x)
        beta = torch.sigmoid(b.float())
        R = O.repeat_kv_heads
        ro2, rs2 = O.recurrent_gated_delta_rule(R(q[0]).unsqueeze(0), R(k[0]).unsqueeze(0), v,
                                                g_t.unsqueeze(0), beta.unsqueeze(0),
                                                h0.transpose(-1, -2))
        assert (ro2.float() - ro.float()).abs().max().item() <= TOL
        assert ((rs2.transpose(-1, -2) - rs).norm() / rs.norm()).item() <= 1e-5


@pytest.mark.parametrize("t,norm", [(200, False), (64, True)])
def test_vllm_chunk_gated_delta_rule(gpu, t, norm):
    """vLLM's chunk_gated_delta_rule as the reference calls it (fle:6474-6483):
    16-head q/k, the [1, 32, dv, dk] state handed over transposed
    (fle:5482-5502), use_qk_l2norm_in_kernel=False on q/k that
    fused_post_conv_prep already normalised (and True on raw ones)."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(91 + t)
    q = torch.randn(1, t, 16, 128, generator=g)
    k = torch.randn(1, t, 16, 128, generator=g)
    if not norm:
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    v = syn.randn((1, t, 32, 128), g)
    beta = torch.sigmoid(torch.randn(1, t, 32, generator=g))
    gg = -torch.nn.functional.softplus(torch.randn(1, t, 32, generator=g)) * 0.5
    h0 = torch.randn(1, 32, 128, 128, generator=g) * 0.2      # [Hv, dv, dk]
    print(f"vllm chunk rule T={t} l2norm_in_kernel={norm}", flush=True)
    d = lambda x: x.to(gpu)
    o, fin = G.vllm_chunk_gated_delta_rule(q=d(q), k=d(k), v=d(v), g=d(gg), beta=d(beta),
                                           initial_state=d(h0), output_final_state=True,
                                           use_qk_l2norm_in_kernel=norm)
    ro, rs = O.vllm_chunk_gated_delta_rule(q, k, v, gg, beta, h0, norm)
    assert o.shape == (1, t, 32, 128) and fin.shape == (1, 32, 128, 128)
    assert (o.cpu().float() - ro.float()).abs().max().item() <= TOL
    assert ((fin.cpu() - rs).norm() / rs.norm()).item() <= 1e-3
    # zero state as None, no final state requested
    o2, none = G.vllm_chunk_gated_delta_rule(d(q), d(k), d(v), d(gg), d(beta), initial_state=None,
                                             use_qk_l2norm_in_kernel=norm)
    ro2, _ = O.vllm_chunk_gated_delta_rule(q, k, v, gg, beta, None, norm)
    assert none is None
    assert (o2.cpu().float() - ro2.float()).abs().max().item() <= TOL


def _gating_inputs(g, t):
    a = syn.randn((t, 32), g)
    b = syn.randn((t, 32), g)
    a_log = torch.log(torch.rand(32, generator=g) * 8 + 0.05).float()
    dt = (torch.randn(32, generator=g) * 0.5).float()
    return a, b, a_log, dt


def test_fused_gating_update_varlen_state_indices(gpu):
    """vLLM's batched form: cu_seqlens [0, 2, 2, 5, 6] (one empty sequence)
    and ssm_state_indices [3, 0, 1, -1] (the last sequence is padding) over a
    pool of 4 slots; each sequence equals the single-sequence oracle on its
    slot, and untouched slots keep their values."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(404)
    t = 6
    q = syn.randn((1, t, 16, 128), g)
    k = syn.randn((1, t, 16, 128), g)
    v = syn.randn((1, t, 32, 128), g)
    a, b, a_log, dt = _gating_inputs(g, t)
    pool = torch.randn(4, 32, 128, 128, generator=g) * 0.2
    cu = [0, 2, 2, 5, 6]
    idx = [3, 0, 1, -1]
    d = lambda x: x.to(gpu)
    state = d(pool).contiguous()
    print("fused gating update varlen", flush=True)
    o, fin = G.fused_sigmoid_gating_delta_rule_update(
        A_log=d(a_log), a=d(a), b=d(b), dt_bias=d(dt), q=d(q), k=d(k), v=d(v),
        initial_state=state, inplace_final_state=True,
        cu_seqlens=torch.tensor(cu, dtype=torch.int64), ssm_state_indices=torch.tensor(idx),
        use_qk_l2norm_in_kernel=True)
    assert fin.data_ptr() == state.data_ptr()
    fin = fin.cpu()
    o = o.cpu()
    for n in range(4):
        t0, t1, sl = cu[n], cu[n + 1], idx[n]
        if sl < 0 or t1 == t0:
            continue
        ro, rs = O.fused_sigmoid_gating_delta_rule_update(
            a_log, a[t0:t1], b[t0:t1], dt, q[:, t0:t1], k[:, t0:t1], v[:, t0:t1],
            pool[sl:sl + 1], True)
        assert (o[:, t0:t1].float() - ro.float()).abs().max().item() <= TOL
        assert ((fin[sl] - rs[0]).norm() / rs.norm()).item() <= 1e-3
    assert torch.equal(fin[2], pool[2])   # no sequence uses slot 2


def test_packed_decode_from_conv_output(gpu):
    """vLLM's packed decode as the reference calls it (fle:6396-6417): B
    tokens read straight from the [B, 8192] conv output, token n updating
    slot ssm_state_indices[n] in place (-1 = padding)."""
    from qwen36_attn import gated_deltanet as G
    g = syn.gen(405)
    bsz = 3
    mixed = syn.randn((bsz, 8192), g)
    a, b, a_log, dt = _gating_inputs(g, bsz)
    pool = torch.randn(3, 32, 128, 128, generator=g) * 0.2
    idx = [2, 0, -1]
    d = lambda x: x.to(gpu)
    state = d(pool).contiguous()
    print("packed decode", flush=True)
    out, fin = G.fused_recurrent_gated_delta_rule_packed_decode(
        mixed_qkv=d(mixed), a=d(a), b=d(b), A_log=d(a_log), dt_bias=d(dt), scale=128 ** -0.5,
        initial_state=state, ssm_state_indices=d(torch.tensor(idx, dtype=torch.int32)),
        use_qk_l2norm_in_kernel=True)
    assert out.shape == (bsz, 1, 32, 128) and fin.data_ptr() == state.data_ptr()
    out, fin = out.cpu(), fin.cpu()
    for n in range(bsz):
        if idx[n] < 0:
            continue
        qn = mixed[n, :2048].view(1, 1, 16, 128)
        kn = mixed[n, 2048:4096].view(1, 1, 16, 128)
        vn = mixed[n, 4096:].view(1, 1, 32, 128)
        ro, rs = O.fused_sigmoid_gating_delta_rule_update(
            a_log, a[n:n + 1], b[n:n + 1], dt, qn, kn, vn, pool[idx[n]:idx[n] + 1], True)
        assert (out[n].float() - ro[0].float()).abs().max().item() <= TOL
        assert ((fin[idx[n]] - rs[0]).norm() / rs.norm()).item() <= 1e-3
    assert torch.equal(fin[1], pool[1])


def test_chunk_prefill_ex_state_vk_in_place(gpu):
    """qwen36_gdn_chunk_prefill_ex in vLLM's [Hv, dv, dk] state orientation
    with state_out aliasing state_in: bit-identical to separate state
    buffers (ragged last chunk, q/k already normalised)."""
    from qwen36_attn import _lib, gated_deltanet as G
    from qwen36_attn._tensors import ptr, scratch, stream_handle
    g = syn.gen(95)
    t = 200
    q = torch.randn(t, 16, 128, generator=g)
    k = torch.randn(t, 16, 128, generator=g)
    q = (q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).to(gpu)
    k = (k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).to(gpu)
    v = syn.randn((t, 32, 128), g).to(gpu)
    beta = torch.sigmoid(torch.randn(t, 32, generator=g)).to(gpu)
    gg = (-torch.nn.functional.softplus(torch.randn(t, 32, generator=g)) * 0.5).to(gpu)
    h0 = (torch.randn(32, 128, 128, generator=g) * 0.2).to(gpu)      # [Hv, dv, dk]
    lib = _lib.load(("qwen36_gdn_chunk_prefill_ex",))
    ws = scratch("gdn_chunk_test", lib.qwen36_gdn_chunk_prefill_workspace_bytes(t), q.device)
    flags = G.STATE_VK | G.QK_NORMALIZED

    def run(s_in, s_out):
        out = torch.empty(t, 32, 128, dtype=torch.bfloat16, device=gpu)
        _lib.call("qwen36_gdn_chunk_prefill_ex", ptr(q), ptr(k), ptr(v), 16, q.stride(0),
                  v.stride(0), ptr(gg), ptr(beta), ptr(s_in), ptr(s_out), ptr(out), t, flags,
                  ptr(ws), ws.numel(), stream_handle(q.device))
        return out

    print("chunk prefill ex, vk state in place", flush=True)
    sep = torch.empty_like(h0)
    out_a = run(h0, sep)
    sd = h0.clone()
    out_b = run(sd, sd)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(sep, sd)
