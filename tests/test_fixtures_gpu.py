"""GPU kernels against the committed golden fixtures (tests/golden)."""
import os

import pytest
import torch
from safetensors.torch import load_file

pytestmark = pytest.mark.gpu
FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.safetensors")


@pytest.fixture(scope="module")
def fx():
    return load_file(FIX)


def test_fixture_prefill_and_decode(gpu, fx):
    from qwen36_attn import full_attention as fa
    d = lambda n: fx[n].to(gpu)
    out = fa.fmha_prefill(d("prefill.q"), d("prefill.k"), d("prefill.v")).cpu()
    assert (out - fx["prefill.out_f32"]).abs().max().item() <= 5e-3
    dec = fa.decode_gqa(d("decode.q"), d("decode.k"), d("decode.v"), 32, 33).cpu()
    assert (dec.float() - fx["decode.out_bf16"].float()).abs().max().item() <= 2e-2


def test_fixture_norm_rope_and_conv(gpu, fx):
    from qwen36_attn import full_attention as fa
    from qwen36_attn import gated_deltanet as G
    d = lambda n: fx[n].to(gpu)
    kc = torch.zeros(10, 2, 256, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    q = fa.head_norm_rope_kv_write(d("norm_rope.q_gate"), d("norm_rope.k"), d("norm_rope.k"),
                                   d("norm_rope.q_w"), d("norm_rope.k_w"), kc, vc, 7)
    assert (q.cpu().float() - fx["norm_rope.q_out"].float()).abs().max().item() <= 2e-2
    assert (kc[7:10].cpu().float() - fx["norm_rope.k_out"].float()).abs().max().item() <= 2e-2
    out, ns = G.causal_conv1d(d("conv.x"), d("conv.state"), d("conv.w"))
    assert (out.cpu().float() - fx["conv.out"].float()).abs().max().item() <= 2e-2
    assert torch.equal(ns.cpu(), fx["conv.new_state"])


def test_fixture_delta_rule(gpu, fx):
    from qwen36_attn import gated_deltanet as G
    d = lambda n: fx[n].to(gpu)
    args = (d("gdn.q"), d("gdn.k"), d("gdn.v"), d("gdn.g"), d("gdn.beta"))
    co, cs = G.chunk_gated_delta_rule(*args, None)
    ro, rs = G.recurrent_gated_delta_rule(*args, torch.zeros(32, 128, 128, device=gpu))
    for o, s, ko, ks in ((co, cs, "gdn.chunk_out", "gdn.chunk_state_h0_h31"),
                         (ro, rs, "gdn.recurrent_out", "gdn.recurrent_state_h0_h31")):
        assert (o[0].cpu().float() - fx[ko].float()).abs().max().item() <= 2e-2
        ref = fx[ks]
        got = s[0, [0, 31]].cpu()
        assert ((got - ref).norm() / ref.norm()).item() <= 1e-3
