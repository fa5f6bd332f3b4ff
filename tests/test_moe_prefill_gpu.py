"""GPU parity of the T-token MoE block (qwen36_moe_prefill, the reference's
native MoE prefill native_moe_prefill.hip.cpp) against the CPU oracle
(four_layer_mini_engine.py:8479-8650, grouped per expert)."""
import pytest
import torch

from oracle import attention_oracle as O
from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _check_routing(ids, rw, logits, n_experts):
    """Each row's ids are a valid top-8 of the kernel's own logits, in
    descending order with ties to the lower index, and rw is the bf16 softmax
    of the selected logits."""
    t = ids.shape[0]
    ids = ids.long()
    sel = logits.gather(1, ids)
    assert ((ids >= 0) & (ids < n_experts)).all()
    assert all(len(set(r.tolist())) == 8 for r in ids)
    assert (sel[:, :-1] >= sel[:, 1:]).all()
    if n_experts > 8:
        rest = torch.ones(t, n_experts, dtype=torch.bool)
        rest.scatter_(1, ids, False)
        rest_max = logits.masked_fill(~rest, -float("inf")).max(dim=1).values
        assert (sel.min(dim=1).values >= rest_max).all()
    assert torch.equal(rw, torch.softmax(sel, dim=1).to(torch.bfloat16).float())


@pytest.mark.parametrize("n_experts,tokens,seed", [
    (8, 1, 1),       # one token: 9 tiles of one row each
    (8, 300, 2),     # 300 rows per expert: five 64-row tiles per group
    (32, 37, 3),     # ragged groups
    (256, 513, 4),   # model geometry, ~16 rows per expert
    (32, 1500, 5),   # router in two K slices (1024 < T <= 8192)
])
def test_moe_prefill_matches_oracle(gpu, n_experts, tokens, seed):
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(600 + seed)
    w = syn.moe_weights(g, n_experts=n_experts)
    inp = syn.randn((tokens, 2048), g, 0.5)
    attn = syn.randn((tokens, 2048), g, 0.5)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print(f"moe prefill E={n_experts} T={tokens}", flush=True)
    out, ids, rw, logits, sg = block.prefill(inp.to(gpu), attn.to(gpu), debug=True)
    torch.cuda.synchronize()
    out, ids, rw = out.cpu(), ids.cpu(), rw.cpu()
    logits, sg = logits.cpu().float(), sg.cpu().float()
    h2 = O.layer_rmsnorm(inp + attn, w["post_attention_layernorm"])
    ref_logits = (h2 @ w["router"].t()).float()
    assert (logits - ref_logits).abs().max().item() <= 1e-2 * max(1.0, ref_logits.abs().max().item())
    ref_sg = (h2 @ w["shared_gate"].t()).float().view(-1)
    assert (sg - ref_sg).abs().max().item() <= 1e-2 * max(1.0, ref_sg.abs().max().item())
    _check_routing(ids, rw, logits, n_experts)
    ref = O.moe_block(inp, attn, w, forced_ids=ids, grouped=True)
    assert torch.isfinite(out.float()).all()
    assert (out.float() - ref.float()).abs().max().item() <= TOL


def test_moe_prefill_rows_match_decode(gpu):
    """Each prefill row equals the one-token decode of that row (same
    formulas; the GEMM and GEMV accumulate in different orders, so the bar is
    the output tolerance) and routes to the same experts."""
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(610)
    w = syn.moe_weights(g, n_experts=64)
    inp = syn.randn((5, 2048), g, 0.5).to(gpu)
    attn = syn.randn((5, 2048), g, 0.5).to(gpu)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print("moe prefill vs decode", flush=True)
    out, ids, _, logits, _ = block.prefill(inp, attn, debug=True)
    same = 0
    for t in range(5):
        d, dids, _, dlogits = block.decode(inp[t:t + 1], attn[t:t + 1], debug=True)
        torch.cuda.synchronize()
        assert (dlogits.float() - logits[t].float()).abs().max().item() <= 1e-2
        # a 1-ulp logit difference may swap a near-tied 8th expert
        if set(dids.cpu().tolist()) == set(ids[t].cpu().tolist()):
            same += 1
            assert (d.float() - out[t:t + 1].float()).abs().max().item() <= TOL
    assert same >= 4


@pytest.mark.parametrize("t", [
    2048,   # the last length aligned by one workgroup (16384 ids)
    2049,   # the first aligned by histogram / scan / scatter launches
    8192,   # bench size
])
def test_moe_prefill_sampled_rows(gpu, t):
    """E = 256 at lengths either side of the alignment forms and at the bench
    size: every output finite, the router logits of 48 sampled rows against
    h2 @ router^T, their routing against their own logits, and their outputs
    against the oracle (the block is row-independent, so a subset of rows is
    an exact check of those rows)."""
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(620)
    w = syn.moe_weights(g, n_experts=256)
    inp = syn.randn((t, 2048), g, 0.5)
    attn = syn.randn((t, 2048), g, 0.5)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print(f"moe prefill T={t}", flush=True)
    out, ids, rw, logits, sg = block.prefill(inp.to(gpu), attn.to(gpu), debug=True)
    torch.cuda.synchronize()
    out, ids, rw, logits = out.cpu(), ids.cpu(), rw.cpu(), logits.cpu().float()
    sg = sg.cpu().float()
    assert torch.isfinite(out.float()).all()
    rows = torch.randperm(t, generator=syn.gen(621))[:48]
    # the router's K-sliced partials, summed by the top-8 kernel
    h2 = O.layer_rmsnorm(inp[rows] + attn[rows], w["post_attention_layernorm"])
    ref_logits = (h2 @ w["router"].t()).float()
    assert (logits[rows] - ref_logits).abs().max().item() <= 1e-2 * max(1.0, ref_logits.abs().max().item())
    ref_sg = (h2 @ w["shared_gate"].t()).float().view(-1)
    assert (sg[rows] - ref_sg).abs().max().item() <= 1e-2 * max(1.0, ref_sg.abs().max().item())
    _check_routing(ids[rows], rw[rows], logits[rows], 256)
    ref = O.moe_block(inp[rows], attn[rows], w, forced_ids=ids[rows], grouped=True)
    assert (out[rows].float() - ref.float()).abs().max().item() <= TOL



def test_moe_prefill_max_tokens_sampled_rows(gpu):
    """T = 262144, the largest accepted (alignment chunks capped, so each
    histogram workgroup covers 8192 ids): inputs drawn on the device, every
    output finite, sampled rows against the oracle."""
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(630)
    w = syn.moe_weights(g, n_experts=256)
    t = 262144
    gd = torch.Generator(device=gpu).manual_seed(631)
    inp = (torch.randn(t, 2048, generator=gd, device=gpu) * 0.5).to(torch.bfloat16)
    attn = (torch.randn(t, 2048, generator=gd, device=gpu) * 0.5).to(torch.bfloat16)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print("moe prefill T=262144", flush=True)
    out, ids, rw, logits, _ = block.prefill(inp, attn, debug=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    rows = torch.tensor([0, 1, 4095, 4096, 131071, 200000, t - 2, t - 1])
    ids_r, rw_r, lg_r = ids[rows].cpu(), rw[rows].cpu(), logits[rows].cpu().float()
    _check_routing(ids_r, rw_r, lg_r, 256)
    ref = O.moe_block(inp[rows].cpu(), attn[rows].cpu(), w, forced_ids=ids_r, grouped=True)
    assert (out[rows].cpu().float() - ref.float()).abs().max().item() <= TOL
    del inp, attn, out, block
    torch.cuda.empty_cache()


def test_moe_prefill_and_decode_ignore_stale_workspace(gpu):
    """The MoE block's results do not depend on what its shared workspaces
    (routing ids, histograms, aligned row lists, activations, partial rows)
    held before the call: 0xFF-filled scratch gives the same bits."""
    from qwen36_attn.moe import MoEBlock
    from qwen36_attn import _tensors
    g = syn.gen(620)
    w = syn.moe_weights(g, n_experts=32)
    inp = syn.randn((37, 2048), g, 0.5).to(gpu)
    attn = syn.randn((37, 2048), g, 0.5).to(gpu)
    block = MoEBlock({k: v.to(gpu) for k, v in w.items()})
    print("moe stale workspace T=37 E=32", flush=True)
    a = block.prefill(inp, attn).clone()
    d = block.decode(inp[:1], attn[:1]).clone()
    torch.cuda.synchronize()
    dev = gpu.index or 0
    _tensors._SCRATCH[("moe_prefill", dev)].fill_(0xFF)
    _tensors._SCRATCH[("moe_decode", dev)].fill_(0xFF)
    b = block.prefill(inp, attn)
    e = block.decode(inp[:1], attn[:1])
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(d, e)
