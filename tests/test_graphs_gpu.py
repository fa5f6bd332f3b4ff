"""HIP graph capture of the library's entry points: every replay must
reproduce the eager result bit for bit, with unrelated eager work (and a
larger call that grows the shared scratch buffer) between the replays.

Each case captures its calls after one eager warm-up of the same sizes (the
package's scratch buffers may not grow inside a capture), replays three times
and compares each replay against the eager output.  Inputs that the calls
update in place are restored from a copy before every replay, so each replay
starts from the same state as the eager call."""
import pytest
import torch

from qwen36_attn import synthetic as syn

pytestmark = pytest.mark.gpu


def _capture(fn):
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()   # warm-up: scratch and library state sized outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def _replay_and_check(graph, reset, outputs, refs, between):
    for i in range(3):
        reset()
        for o in outputs:
            o.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for j, (o, r) in enumerate(zip(outputs, refs)):
            assert torch.equal(o, r), f"replay {i}, output {j}"
        between(i)
        torch.cuda.synchronize()


def test_graph_decode_gqa_and_fused_step(gpu):
    """Split-K decode with the new-row write and gate, and the fused decode
    step (norm + RoPE + KV write + attention + gate), captured together."""
    from qwen36_attn import full_attention as fa
    g = syn.gen(900)
    cap, end = 6000, 5000
    k = syn.randn((cap, 2, 256), g).to(gpu)
    v = syn.randn((cap, 2, 256), g).to(gpu)
    q = syn.randn((16, 256), g).to(gpu)
    kn = syn.randn((2, 256), g).to(gpu)
    vn = syn.randn((2, 256), g).to(gpu)
    gate = syn.randn((4096,), g).to(gpu)
    q_gate = syn.randn((1, 8192), g).to(gpu)
    kr = syn.randn((1, 512), g).to(gpu)
    vr = syn.randn((1, 512), g).to(gpu)
    qw = syn.randn((256,), g, 0.1).to(gpu)
    kw = syn.randn((256,), g, 0.1).to(gpu)
    k0, v0 = k.clone(), v.clone()
    out1 = torch.empty(1, 4096, dtype=torch.bfloat16, device=gpu)
    out2 = torch.empty_like(out1)
    print("graph: decode_gqa + decode_step, 5000 rows", flush=True)

    def run():
        fa.decode_gqa(q, k, v, end - 1, end, k_new=kn, v_new=vn, gate=gate, out=out1)
        fa.decode_step(q_gate, kr, vr, qw, kw, k, v, end, end + 1, out=out2)

    def reset():
        k.copy_(k0)
        v.copy_(v0)

    reset()
    run()
    torch.cuda.synchronize()
    refs = [out1.clone(), out2.clone(), k.clone(), v.clone()]
    graph = _capture(run)
    big_k = torch.zeros(140000, 2, 256, dtype=torch.bfloat16, device=gpu)

    def between(i):
        # other eager work on the same scratch tag, then a larger call that
        # grows the decode scratch (the graph keeps the old buffer)
        fa.decode_gqa(q, k0, v0, 99, 100)
        fa.decode_gqa(q, big_k, big_k, 0, 140000 - i, split_tokens=128 * 8)
    _replay_and_check(graph, reset, [out1, out2], refs[:2], between)
    assert torch.equal(k, refs[2]) and torch.equal(v, refs[3])


def test_graph_fmha_split_and_unsplit(gpu):
    """A short prompt (split key ranges + combine through the scratch) and a
    long one (one workgroup per query tile)."""
    from qwen36_attn import full_attention as fa
    g = syn.gen(901)
    qs = syn.randn((300, 16, 256), g).to(gpu)
    ks = syn.randn((800, 2, 256), g).to(gpu)
    vs = syn.randn((800, 2, 256), g).to(gpu)
    ql = syn.randn((4096, 16, 256), g).to(gpu)
    kl = syn.randn((4096, 2, 256), g).to(gpu)
    vl = syn.randn((4096, 2, 256), g).to(gpu)
    os_ = torch.empty(300, 4096, dtype=torch.float32, device=gpu)
    ol = torch.empty(4096, 4096, dtype=torch.float32, device=gpu)
    print("graph: fmha 300 over 800 (split), 4096 causal", flush=True)

    def run():
        fa.fmha_prefill(qs, ks, vs, out=os_)
        fa.fmha_prefill(ql, kl, vl, out=ol)

    run()
    torch.cuda.synchronize()
    refs = [os_.clone(), ol.clone()]
    graph = _capture(run)

    def between(i):
        fa.fmha_prefill(qs[:100], ks[:500], vs[:500])
    _replay_and_check(graph, lambda: None, [os_, ol], refs, between)


def test_graph_gdn_decode_step_and_moe_decode(gpu):
    """The fused GDN decode step (conv state and fp32 state written to
    separate buffers) and the three-launch MoE decode block."""
    from qwen36_attn import gated_deltanet as G
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(902)
    mixed = syn.randn((1, 8192), g).to(gpu)
    conv_w = syn.randn((8192, 4), g, 0.5).to(gpu)
    conv_state = syn.randn((8192, 3), g).to(gpu)
    a = syn.randn((1, 32), g).to(gpu)
    b = syn.randn((1, 32), g).to(gpu)
    a_log = torch.log(torch.rand(32, generator=g).clamp_min(1e-4) * 8).float().to(gpu)
    dt_bias = torch.randn(32, generator=g).float().to(gpu)
    z = syn.randn((1, 4096), g).to(gpu)
    norm_w = syn.randn((128,), g, 0.5).to(gpu)
    ssm = (torch.randn(32, 128, 128, generator=g) * 0.2).to(gpu)
    new_conv = torch.empty_like(conv_state)
    fin = torch.empty_like(ssm)
    gout = torch.empty(1, 4096, dtype=torch.bfloat16, device=gpu)
    w = {k_: v_.to(gpu) for k_, v_ in syn.moe_weights(g, n_experts=64).items()}
    block = MoEBlock(w)
    inp = syn.randn((1, 2048), g, 0.5).to(gpu)
    attn = syn.randn((1, 2048), g, 0.5).to(gpu)
    mout = torch.empty(1, 2048, dtype=torch.bfloat16, device=gpu)
    print("graph: gdn decode step + moe decode (64 experts)", flush=True)

    def run():
        G.gdn_decode_step(mixed, conv_state, new_conv, conv_w, a, b, a_log, dt_bias, z, norm_w,
                          ssm, final_state=fin, out=gout)
        block.decode(inp, attn, out=mout)

    run()
    torch.cuda.synchronize()
    refs = [gout.clone(), new_conv.clone(), fin.clone(), mout.clone()]
    graph = _capture(run)

    def between(i):
        block.decode(attn, inp)
        G.gdn_decode_step(mixed, conv_state, torch.empty_like(conv_state), conv_w, a, b, a_log,
                          dt_bias, z, norm_w, ssm, final_state=torch.empty_like(ssm))
    _replay_and_check(graph, lambda: None, [gout, new_conv, fin, mout], refs, between)


def test_graph_moe_prefill_with_side_stream(gpu):
    """The MoE block over T tokens: its shared-expert GEMMs run on the
    library's side stream between a fork and a join event recorded on the
    caller's stream, so the capture takes them into the graph as a branch."""
    from qwen36_attn.moe import MoEBlock
    g = syn.gen(904)
    w = {k_: v_.to(gpu) for k_, v_ in syn.moe_weights(g, n_experts=64).items()}
    block = MoEBlock(w)
    inp = syn.randn((300, 2048), g, 0.5).to(gpu)
    attn = syn.randn((300, 2048), g, 0.5).to(gpu)
    out = torch.empty(300, 2048, dtype=torch.bfloat16, device=gpu)
    print("graph: moe prefill T=300 (64 experts, side stream)", flush=True)

    def run():
        block.prefill(inp, attn, out=out)

    run()
    torch.cuda.synchronize()
    refs = [out.clone()]
    graph = _capture(run)

    def between(i):
        block.prefill(attn[:100], inp[:100])
    _replay_and_check(graph, lambda: None, [out], refs, between)


def test_scratch_refuses_to_grow_during_capture(gpu):
    """A call whose workspace would outgrow the shared scratch inside a
    capture raises instead of allocating graph-private memory."""
    from qwen36_attn import full_attention as fa
    from qwen36_attn import _tensors
    g = syn.gen(903)
    q = syn.randn((16, 256), g).to(gpu)
    k = syn.randn((4096, 2, 256), g).to(gpu)
    fa.decode_gqa(q, k, k, 0, 256)
    torch.cuda.synchronize()
    have = _tensors._SCRATCH[("decode_gqa", gpu.index or 0)].numel()
    need = 2 * have
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match="during graph capture"):
            with torch.cuda.graph(graph):
                _tensors.scratch("decode_gqa", need, gpu)
    torch.cuda.synchronize()
