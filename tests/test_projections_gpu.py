"""GPU parity of the one-token projection GEMV (qwen36_gemv_bf16) against an
fp32 reference of ``inp @ W.t()`` (four_layer_mini_engine.py:6566-6573,
:6386-6395), and of the native decode layer paths against the torch-projection
paths."""
import pytest
import torch

from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(1, 2048), (3, 2048), (32, 2048), (512, 2048), (9216, 2048),
                                 (12352, 2048), (2048, 4096), (7, 4096), (70001, 2048)])
def test_gemv_matches_fp32(gpu, n, k):
    from qwen36_attn.projections import gemv
    g = syn.gen(n + k)
    w = syn.randn((n, k), g, 0.05)
    x = syn.randn((1, k), g)
    print(f"gemv N={n} K={k}", flush=True)
    got = gemv(w.to(gpu), x.to(gpu)).cpu().float()
    ref = x.float() @ w.float().t()
    # fp32 accumulation, one bf16 rounding of the result
    assert ((got - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-4).all()


def test_gemv_rejects_bad_shapes(gpu):
    from qwen36_attn import _lib
    L = _lib.load()
    x = torch.zeros(1024, dtype=torch.bfloat16, device=gpu)
    assert L.qwen36_gemv_bf16(x.data_ptr(), 4, 1024, x.data_ptr(), x.data_ptr(), None) == 1
    assert L.qwen36_gemv_bf16(x.data_ptr(), 0, 2048, x.data_ptr(), x.data_ptr(), None) == 1


def test_native_decode_paths_match_torch_projection_paths(gpu):
    """Layer decode with the GEMV projections vs the same layer with torch
    projections (fused=False): both within the north_star bar of each other."""
    from qwen36_attn.full_attention import FullAttentionLayer
    from qwen36_attn.gated_deltanet import LinearAttentionLayer
    g = syn.gen(12)
    wf = {k_: v_.to(gpu) for k_, v_ in syn.full_attention_weights(g).items()}
    wl = {k_: v_.to(gpu) for k_, v_ in syn.linear_attention_weights(g, a_max=1.0).items()}
    x = syn.randn((40, 2048), g, 0.5).to(gpu)
    fa, fb = FullAttentionLayer(wf, 64, gpu), FullAttentionLayer(wf, 64, gpu)
    la, lb = LinearAttentionLayer(wl, gpu), LinearAttentionLayer(wl, gpu)
    print("native decode vs torch projections", flush=True)
    fa.forward(x[:32], 0, "prefill"); fb.forward(x[:32], 0, "prefill")
    la.forward(x[:32], "prefill"); lb.forward(x[:32], "prefill")
    for i in range(32, 40):
        a1 = fa.forward(x[i:i + 1], i, "decode")
        b1 = fb.forward(x[i:i + 1], i, "decode", fused=False)
        a2 = la.forward(x[i:i + 1], "decode")
        b2 = lb.forward(x[i:i + 1], "decode", fused=False)
        assert (a1.float() - b1.float()).abs().max().item() <= 2e-2
        assert (a2.float() - b2.float()).abs().max().item() <= 2e-2
