"""GPU parity of the one-token MoE block (qwen36_moe_decode) against the CPU
oracle (four_layer_mini_engine.py:8479-8650)."""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu

TOL = 2e-2


@pytest.mark.parametrize("n_experts,seed", [(8, 1), (32, 2), (256, 3)])
def test_moe_decode_matches_oracle(gpu, n_experts, seed):
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(500 + seed)
    w = syn.moe_weights(g, n_experts=n_experts)
    inp = syn.randn((1, 2048), g, 0.5)
    attn = syn.randn((1, 2048), g, 0.5)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print(f"moe decode E={n_experts}", flush=True)
    out, ids, rw, logits = block.decode(inp.to(gpu), attn.to(gpu), debug=True)
    torch.cuda.synchronize()
    out, ids, rw, logits = out.cpu(), ids.cpu().long(), rw.cpu(), logits.cpu().float()
    # router logits: fp32-accumulated GEMV vs the CPU bf16 matmul
    h2 = O.layer_rmsnorm(inp + attn, w["post_attention_layernorm"])
    ref_logits = (h2 @ w["router"].t()).float().view(-1)
    assert (logits - ref_logits).abs().max().item() <= 1e-2 * max(1.0, ref_logits.abs().max().item())
    # a valid top-8 of the kernel's own logits (ties to the lower index), in order
    sel = logits[ids]
    rest = torch.ones(n_experts, dtype=torch.bool)
    rest[ids] = False
    assert len(set(ids.tolist())) == 8
    assert (sel[:-1] >= sel[1:]).all()
    if rest.any():
        assert sel.min().item() >= logits[rest].max().item()
    assert torch.equal(rw, torch.softmax(sel, dim=0).to(torch.bfloat16).float())
    # the block's output, with the oracle routed to the same experts
    ref = O.moe_block(inp, attn, w, forced_ids=ids.view(1, 8))
    assert torch.isfinite(out.float()).all()
    assert (out.float() - ref.float()).abs().max().item() <= TOL
