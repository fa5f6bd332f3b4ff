"""GPU parity of the pointwise full-attention kernels and of the whole
config-1 layer (prefill 1024 then 16 decode steps) against the oracle."""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu
TOL = 2e-2


def test_rotary_table_known_answer(gpu):
    """Reference-held constant table (native_decode_runner.hip.cpp:26-34)."""
    from qwen36_attn.full_attention import rotary_table
    from tests.golden.rope_table import INV_FREQ_KAT
    cos, sin = rotary_table(3, 1, gpu)
    ang = torch.atan2(sin[0].cpu().double(), cos[0].cpu().double())
    assert torch.allclose(ang.float(), torch.tensor(INV_FREQ_KAT), rtol=2e-7, atol=0)


def test_head_norm_rope_kv_write(gpu):
    from qwen36_attn.full_attention import head_norm_rope_kv_write
    g = syn.gen(5)
    t, start = 37, 1000
    qg = syn.randn((t, 8192), g)
    k = syn.randn((t, 512), g)
    v = syn.randn((t, 512), g)
    qw = syn.randn((256,), g, 0.5)
    kw = syn.randn((256,), g, 0.5)
    kc = torch.zeros(start + t + 3, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    q = head_norm_rope_kv_write(qg.to(gpu), k.to(gpu), v.to(gpu), qw.to(gpu), kw.to(gpu),
                                kcd, vcd, start)
    torch.cuda.synchronize()
    cos, sin = O.rope_cos_sin(start, t)
    rq, _ = O.split_q_gate(qg)
    rq = O.apply_rope(O.head_rmsnorm(rq, qw), cos, sin)
    rk = O.apply_rope(O.head_rmsnorm(k.view(t, 2, 256), kw), cos, sin)
    O.write_kv_cache(kc, vc, rk, v.view(t, 2, 256), start)
    dq = (q.cpu().float() - rq.float()).abs()
    dk = (kcd.cpu().float() - kc.float()).abs()
    assert dq.max().item() <= TOL and dk.max().item() <= TOL
    # bf16 results agree to the last bit for the vast majority of elements
    assert (dq == 0).float().mean().item() > 0.99
    assert torch.equal(vcd.cpu(), vc)


def test_output_gate(gpu):
    from qwen36_attn.full_attention import output_gate
    g = syn.gen(6)
    attn = syn.randn((9, 4096), g)
    qg = syn.randn((9, 8192), g)
    _, gate = O.split_q_gate(qg)
    out = output_gate(attn.to(gpu), qg.to(gpu))
    ref = O.output_gate(attn, gate)
    assert (out.cpu().float() - ref.float()).abs().max().item() <= TOL
    out32 = output_gate(attn.float().to(gpu), qg.to(gpu))
    assert torch.equal(out32.cpu(), out.cpu())


def test_config1_full_layer_prefill_then_decode(gpu):
    """Config 1: x ~ N(0,1)*0.5, weights N(0,0.02); prefill 1024 tokens, then
    16 decode steps, each fed a fresh seeded row (a single layer has no
    greedy token of its own)."""
    from qwen36_attn.full_attention import FullAttentionLayer
    g = syn.gen(1)
    w = syn.full_attention_weights(g)
    t, steps = 1024, 16
    x = syn.randn((t + steps, 2048), g, 0.5)
    layer = FullAttentionLayer({k_: v_.to(gpu) for k_, v_ in w.items()}, t + steps, gpu)
    kc = torch.zeros(t + steps, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    got = layer.forward(x[:t].to(gpu), 0, "prefill").cpu()
    ref = O.full_attention(x[:t], w, kc, vc, 0, "prefill")
    assert (got.float() - ref.float()).abs().max().item() <= TOL
    for i in range(steps):
        pos = t + i
        got = layer.forward(x[pos:pos + 1].to(gpu), pos, "decode").cpu()
        ref = O.full_attention(x[pos:pos + 1], w, kc, vc, pos, "decode")
        assert (got.float() - ref.float()).abs().max().item() <= TOL, i
    assert (layer.k_cache.cpu().float() - kc.float()).abs().max().item() <= TOL


def test_linear_attention_layer_prefill_then_decode(gpu):
    from qwen36_attn.gated_deltanet import LinearAttentionLayer
    g = syn.gen(2)
    w = syn.linear_attention_weights(g, a_max=1.0)
    t, steps = 256, 8
    x = syn.randn((t + steps, 2048), g, 0.5)
    layer = LinearAttentionLayer({k_: v_.to(gpu) for k_, v_ in w.items()}, gpu)
    conv = torch.zeros(8192, 3, dtype=torch.bfloat16)
    ssm = torch.zeros(32, 128, 128)
    got = layer.forward(x[:t].to(gpu), "prefill").cpu()
    ref, conv, ssm = O.linear_attention(x[:t], w, conv, ssm, "prefill")
    assert (got.float() - ref.float()).abs().max().item() <= TOL
    for i in range(steps):
        xi = x[t + i:t + i + 1]
        got = layer.forward(xi.to(gpu), "decode").cpu()
        ref, conv, ssm = O.linear_attention(xi, w, conv, ssm, "decode")
        assert (got.float() - ref.float()).abs().max().item() <= TOL
    rel = ((layer.ssm_state.cpu() - ssm).norm() / ssm.norm()).item()
    assert rel <= 1e-3
