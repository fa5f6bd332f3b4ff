"""GPU parity of the fused Gated-DeltaNet decode step (one launch for conv,
gating, l2norm, recurrent delta rule and gated RMSNorm) against the CPU
oracle's composition of the same steps (four_layer_mini_engine.py:6378-6544,
mode "decode") and against the unfused four-launch library path."""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu

TOL_OUT = 2e-2      # max-abs-err on bf16 outputs (north_star)
TOL_STATE = 1e-3    # relative error on the fp32 state (north_star)


def rel_err(got, ref):
    return ((got.double() - ref.double()).norm() / ref.double().norm().clamp_min(1e-30)).item()


def _step_inputs(t, seed, a_max):
    g = syn.gen(seed)
    mixed = syn.randn((t, 8192), g)
    conv_w = syn.randn((8192, 4), g, 0.5)
    conv_state = syn.randn((8192, 3), g)
    a = syn.randn((t, 32), g)
    b = syn.randn((t, 32), g)
    a_log = torch.log((torch.rand(32, generator=g) * a_max).clamp_min(1e-4)).float()
    dt_bias = torch.randn(32, generator=g).float()
    z = syn.randn((t, 4096), g)
    norm_w = syn.randn((128,), g, 0.5)
    ssm = torch.randn(32, 128, 128, generator=g) * 0.2
    return mixed, conv_w, conv_state, a, b, a_log, dt_bias, z, norm_w, ssm


def _oracle_step(mixed, conv_w, conv_state, a, b, a_log, dt_bias, z, norm_w, ssm):
    conv_out, new_conv = O.causal_conv1d(mixed, conv_state, conv_w)
    q, k, v = O.split_gdn_qkv(conv_out)
    q, k = O.repeat_kv_heads(q), O.repeat_kv_heads(k)
    g, beta = O.gdn_gating(a, b, a_log, dt_bias)
    core, final = O.recurrent_gated_delta_rule(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                                               g.unsqueeze(0), beta.unsqueeze(0),
                                               ssm.unsqueeze(0))
    out = O.gated_rmsnorm(core.squeeze(0), z, norm_w)
    return out, new_conv, final.squeeze(0)


@pytest.mark.parametrize("t,a_max", [(1, 16.0), (1, 0.1), (3, 1.0), (8, 16.0)])
def test_decode_step_matches_oracle(gpu, t, a_max):
    from qwen36_attn import gated_deltanet as G
    ins = _step_inputs(t, 300 + t, a_max)
    mixed, conv_w, conv_state, a, b, a_log, dt_bias, z, norm_w, ssm = ins
    print(f"gdn decode step T={t} a_max={a_max}", flush=True)
    d = [x.to(gpu) for x in ins]
    new_conv = torch.empty_like(d[2])
    ssm_d = d[9].clone()
    got = G.gdn_decode_step(d[0], d[2], new_conv, d[1], d[3], d[4], d[5], d[6], d[7], d[8],
                            ssm_d)
    torch.cuda.synchronize()
    ref, ref_conv, ref_ssm = _oracle_step(*ins)
    assert torch.isfinite(got).all()
    assert (got.cpu().float() - ref.float()).abs().max().item() <= TOL_OUT
    assert torch.equal(new_conv.cpu(), ref_conv)          # a copy of inputs: exact
    assert rel_err(ssm_d.cpu(), ref_ssm) <= TOL_STATE


def test_decode_step_equals_unfused_launches(gpu):
    """The fused step and the four-launch path (conv, gating, recurrent,
    gated norm) see identical bf16 intermediates; they differ only in the
    summation order of S^T k and S^T q, so outputs agree to a bf16 rounding
    step and states to fp32 rounding."""
    from qwen36_attn import gated_deltanet as G
    t = 4
    ins = _step_inputs(t, 77, 8.0)
    d = [x.to(gpu) for x in ins]
    mixed, conv_w, conv_state, a, b, a_log, dt_bias, z, norm_w, ssm = d
    print("gdn decode step fused vs unfused", flush=True)
    new_conv = torch.empty_like(conv_state)
    ssm_f = ssm.clone()
    fused = G.gdn_decode_step(mixed, conv_state, new_conv, conv_w, a, b, a_log, dt_bias, z,
                              norm_w, ssm_f)
    conv_out, conv_u = G.causal_conv1d(mixed, conv_state, conv_w)
    q = conv_out[:, :2048].view(t, 16, 128)
    k = conv_out[:, 2048:4096].view(t, 16, 128)
    v = conv_out[:, 4096:].view(t, 32, 128)
    g, beta = G.gating(a, b, a_log, dt_bias)
    ssm_u = ssm.clone()
    core, _ = G.recurrent_gated_delta_rule(q, k, v, g, beta, ssm_u, final_state=ssm_u)
    unfused = G.gated_rmsnorm(core, z, norm_w)
    torch.cuda.synchronize()
    assert torch.equal(new_conv, conv_u)
    diff = (fused.float() - unfused.float()).abs()
    assert diff.max().item() <= 1e-2
    assert (diff > 0).float().mean().item() <= 0.01     # almost all bit-identical
    assert rel_err(ssm_f, ssm_u) <= 1e-5


def test_decode_step_state_carry_over_calls(gpu):
    """T tokens in one launch == T launches of one token each (conv and
    recurrent states carried through the double-buffered conv state)."""
    from qwen36_attn import gated_deltanet as G
    t = 6
    ins = _step_inputs(t, 91, 4.0)
    d = [x.to(gpu) for x in ins]
    mixed, conv_w, conv_state, a, b, a_log, dt_bias, z, norm_w, ssm = d
    print("gdn decode step carry", flush=True)
    conv_once = torch.empty_like(conv_state)
    ssm_once = ssm.clone()
    once = G.gdn_decode_step(mixed, conv_state, conv_once, conv_w, a, b, a_log, dt_bias, z,
                             norm_w, ssm_once)
    cur, spare = conv_state.clone(), torch.empty_like(conv_state)
    ssm_step = ssm.clone()
    rows = []
    for i in range(t):
        rows.append(G.gdn_decode_step(mixed[i:i + 1], cur, spare, conv_w, a[i:i + 1],
                                      b[i:i + 1], a_log, dt_bias, z[i:i + 1], norm_w, ssm_step))
        cur, spare = spare, cur
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(rows), once)
    assert torch.equal(cur, conv_once)
    assert torch.equal(ssm_step, ssm_once)


def test_decode_step_rejects_aliased_conv_state(gpu):
    from qwen36_attn import gated_deltanet as G
    ins = _step_inputs(1, 5, 1.0)
    d = [x.to(gpu) for x in ins]
    with pytest.raises(ValueError):
        G.gdn_decode_step(d[0], d[2], d[2], d[1], d[3], d[4], d[5], d[6], d[7], d[8], d[9])
