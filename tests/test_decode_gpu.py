"""GPU parity of the split-K GQA decode against the CPU oracle
(four_layer_mini_engine.py:6614-6626 grouped decode)."""
import pytest
import torch

from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2   # max-abs-err bar on bf16 outputs (north_star)
# vs the fp32 restatement: the kernel computes in fp32 except that the
# probabilities enter the PV MFMA as bf16 (relative error <= 2^-9 each, so at
# most 2^-9 * max|v| on the output) and the output is rounded to bf16
# (2^-8 relative).
REL_BF16 = 2.0 ** -8
P_ROUND = 2.0 ** -9


def _inputs(capacity, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(capacity, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(capacity, 2, 256, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("cache_end", [1, 7, 31, 128, 1000, 4096, 32768])
def test_decode_matches_oracle(gpu, cache_end):
    from qwen36_attn.full_attention import decode_gqa
    q, k, v = _inputs(cache_end + 5, seed=cache_end)
    print(f"decode cache_end={cache_end}", flush=True)
    out = decode_gqa(q.to(gpu), k.to(gpu), v.to(gpu), cache_end - 1, cache_end)
    torch.cuda.synchronize()
    got = out.cpu().float()
    ref16 = O.decode_attention_grouped_bf16(q.view(1, 16, 256), k, v, cache_end).float()
    ref32 = O.decode_attention_f32(q.view(1, 16, 256), k, v, cache_end)
    assert torch.isfinite(got).all()
    assert (got - ref16).abs().max().item() <= TOL_BF16
    vmax = v[:cache_end].float().abs().max().item()
    assert ((got - ref32).abs() <= REL_BF16 * ref32.abs() + P_ROUND * vmax + 1e-4).all()


def test_decode_writes_kv_row_and_gate(gpu):
    from qwen36_attn.full_attention import decode_gqa
    S = 3000
    q, k, v = _inputs(S + 10, seed=5)
    g = torch.Generator().manual_seed(9)
    k_new = torch.randn(2, 256, generator=g).to(torch.bfloat16)
    v_new = torch.randn(2, 256, generator=g).to(torch.bfloat16)
    gate = torch.randn(4096, generator=g).to(torch.bfloat16)
    kd, vd = k.to(gpu), v.to(gpu)
    out = decode_gqa(q.to(gpu), kd, vd, S - 1, S, k_new=k_new.to(gpu), v_new=v_new.to(gpu),
                     gate=gate.to(gpu))
    torch.cuda.synchronize()
    kr, vr = k.clone(), v.clone()
    O.write_kv_cache(kr, vr, k_new.view(1, 2, 256), v_new.view(1, 2, 256), S - 1)
    assert torch.equal(kd.cpu(), kr) and torch.equal(vd.cpu(), vr)
    ref = O.output_gate(O.decode_attention_grouped_bf16(q.view(1, 16, 256), kr, vr, S),
                        gate.view(1, 4096)).float()
    assert (out.cpu().float() - ref).abs().max().item() <= TOL_BF16


@pytest.mark.parametrize("split_tokens", [128, 256, 1024, 8192])
def test_decode_split_invariance(gpu, split_tokens):
    """The split-K combine is independent of the split count."""
    from qwen36_attn.full_attention import decode_gqa
    S = 8192 + 77
    q, k, v = _inputs(S, seed=11)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    base = decode_gqa(qd, kd, vd, 0, S).float()
    alt = decode_gqa(qd, kd, vd, 0, S, split_tokens=split_tokens).float()
    torch.cuda.synchronize()
    assert (base - alt).abs().max().item() <= 2e-3


@pytest.mark.parametrize("cache_end", [131072, 262143])
def test_decode_full_size_matches_oracle(gpu, cache_end):
    """The benchmarked KV lengths (config 5), with the new row appended at the
    last position, against the oracle's grouped bf16 decode."""
    from qwen36_attn.full_attention import decode_gqa
    q, k, v = _inputs(cache_end, seed=cache_end % 1000)
    g = torch.Generator().manual_seed(7)
    k_new = torch.randn(2, 256, generator=g).to(torch.bfloat16)
    v_new = torch.randn(2, 256, generator=g).to(torch.bfloat16)
    print(f"decode full size cache_end={cache_end}", flush=True)
    kd, vd = k.to(gpu), v.to(gpu)
    out = decode_gqa(q.to(gpu), kd, vd, cache_end - 1, cache_end,
                     k_new=k_new.to(gpu), v_new=v_new.to(gpu))
    torch.cuda.synchronize()
    O.write_kv_cache(k, v, k_new.view(1, 2, 256), v_new.view(1, 2, 256), cache_end - 1)
    assert torch.equal(kd[cache_end - 1].cpu(), k[cache_end - 1])
    ref = O.decode_attention_grouped_bf16(q.view(1, 16, 256), k, v, cache_end).float()
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= TOL_BF16


def test_decode_rejects_bad_geometry(gpu):
    from qwen36_attn.full_attention import decode_gqa
    q, k, v = _inputs(64, seed=1)
    with pytest.raises(ValueError):
        decode_gqa(q.to(gpu), k.to(gpu), v.to(gpu), 0, 65)


@pytest.mark.parametrize("cache_end,position,split_tokens", [
    (1, 0, 0), (33, 32, 0), (1000, 999, 0), (4097, 4096, 0), (4096, 1234, 0),
    (20000, 19999, 256), (131072, 131071, 0)])
def test_decode_step_equals_norm_rope_then_decode(gpu, cache_end, position, split_tokens):
    """The fused decode step (head norm + RoPE + KV-row write + attention +
    gate in the split/combine launches) rounds exactly like the two-launch
    path qwen36_head_norm_rope -> qwen36_decode_gqa: outputs and cache rows
    are bit-identical."""
    from qwen36_attn.full_attention import (decode_step, decode_gqa,
                                            head_norm_rope_kv_write)
    g = torch.Generator().manual_seed(cache_end + position)
    cap = cache_end + 5
    kc = torch.randn(cap, 2, 256, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(cap, 2, 256, generator=g).to(torch.bfloat16).to(gpu)
    q_gate = (torch.randn(1, 8192, generator=g) * 2).to(torch.bfloat16).to(gpu)
    k = (torch.randn(1, 512, generator=g) * 2).to(torch.bfloat16).to(gpu)
    v = torch.randn(1, 512, generator=g).to(torch.bfloat16).to(gpu)
    qn = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    kn = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    print(f"decode step S={cache_end} pos={position}", flush=True)
    kc2, vc2 = kc.clone(), vc.clone()
    fused = decode_step(q_gate, k, v, qn, kn, kc, vc, position, cache_end,
                        split_tokens=split_tokens)
    q = head_norm_rope_kv_write(q_gate, k, v, qn, kn, kc2, vc2, position)
    gate = q_gate.view(16, 512)[:, 256:]
    ref = decode_gqa(q, kc2, vc2, position, cache_end, gate=gate, split_tokens=split_tokens)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert torch.equal(fused, ref)


def test_decode_ignores_stale_workspace(gpu):
    """A decode's result does not depend on what the shared split-partial
    workspace held before the call: NaN-filled scratch gives the same bits."""
    from qwen36_attn.full_attention import decode_gqa
    from qwen36_attn import _tensors
    q, k, v = _inputs(5000, seed=77)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    print("decode stale workspace cache_end=4999", flush=True)
    a = decode_gqa(qd, kd, vd, 4998, 4999).clone()
    _tensors._SCRATCH[("decode_gqa", gpu.index or 0)].fill_(0xFF)   # every float NaN
    b = decode_gqa(qd, kd, vd, 4998, 4999)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
