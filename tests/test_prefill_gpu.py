"""GPU parity of the causal GQA FMHA prefill (provider ABI) against the CPU
oracle (four_layer_mini_engine.py:6627-6648 SDPA, fp32 evaluation)."""
import pytest
import torch

from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-2        # max-abs-err bar (north_star)
TOL_TIGHT = 5e-3  # fp32 output vs fp32 oracle: only P's bf16 rounding differs


def _inputs(t, s, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(t, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(s, 2, 256, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("t,s", [(1, 1), (7, 7), (64, 64), (128, 128), (300, 300),
                                 (1, 513), (100, 4196), (129, 257), (1000, 1000),
                                 (512, 2048)])
def test_prefill_matches_oracle(gpu, t, s):
    from qwen36_attn.full_attention import fmha_prefill
    q, k, v = _inputs(t, s, seed=t * 7 + s)
    print(f"prefill T={t} S={s}", flush=True)
    got = fmha_prefill(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    ref = O.prefill_attention(q, k, v, position_start=s - t, out_dtype=torch.float32)
    err = (got - ref).abs().max().item()
    assert torch.isfinite(got).all()
    assert err <= TOL_TIGHT, err


def test_prefill_config3_sampled_rows(gpu):
    """Config 3: 8192 new tokens over a 4096-token cached prefix (S=12288).
    Rows are independent, so a spread of rows (first, last, tile edges) is
    checked exactly against the oracle restricted to those rows."""
    from qwen36_attn.full_attention import fmha_prefill
    t, s = 8192, 12288
    q, k, v = _inputs(t, s, seed=3)
    print("prefill config3", flush=True)
    got = fmha_prefill(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    rows = torch.tensor([0, 1, 63, 64, 127, 128, 129, 2047, 4095, 4096, 6000, 8190, 8191])
    off = s - t
    for r in rows.tolist():
        lim = r + off + 1
        ref = O.prefill_attention(q[r:r + 1], k[:lim], v[:lim], position_start=lim - 1,
                                  out_dtype=torch.float32)
        assert (got[r:r + 1] - ref).abs().max().item() <= TOL_TIGHT, r
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("t", [256, 1536, 2304, 2560, 2561])
def test_short_prompt_split_plans_sampled_rows(gpu, t):
    """Short square prompts through the split plans the chunk-count table
    picks (T = 256: 2 chunks, 1536: 3, 2304 and 2560: 3 over 9 and 10 query
    tiles) and the first unsplit length (2561: 11 tiles, a one-row last
    tile), plain and gated: rows at chunk and tile edges against the
    oracle."""
    from qwen36_attn.full_attention import fmha_prefill, fmha_prefill_gated, output_gate
    q, k, v = _inputs(t, t, seed=70 + t)
    g = torch.Generator().manual_seed(71 + t)
    gate = torch.randn(t, 8192, generator=g).to(torch.bfloat16)
    print(f"short-prompt split plan T={t}", flush=True)
    qd, kd, vd, gd = q.to(gpu), k.to(gpu), v.to(gpu), gate.to(gpu)
    got = fmha_prefill(qd, kd, vd).cpu()
    gated = fmha_prefill_gated(qd, kd, vd, gd).cpu()
    rows = sorted({0, 1, 127, 128, 255, t // 3, t // 2 - 1, t // 2, 2 * t // 3, t - 257, t - 256,
                   t - 2, t - 1} - {-1})
    for r in rows:
        ref = O.prefill_attention(q[r:r + 1], k[:r + 1], v[:r + 1], position_start=r,
                                  out_dtype=torch.float32)
        assert (got[r:r + 1] - ref).abs().max().item() <= TOL_TIGHT, r
        gref = O.output_gate(ref.to(torch.bfloat16), O.split_q_gate(gate[r:r + 1])[1])
        assert (gated[r:r + 1].float() - gref.float()).abs().max().item() <= TOL, r
    assert torch.isfinite(got).all()
    assert torch.equal(gated, output_gate(got.to(gpu), gd).cpu())


def test_prefill_8k_causal_sampled_rows(gpu):
    """The benchmarked 8192-token causal prefill: rows spread over the whole
    range (tile and workgroup edges) against the oracle for those rows."""
    from qwen36_attn.full_attention import fmha_prefill
    t = 8192
    q, k, v = _inputs(t, t, seed=8)
    print("prefill 8k causal", flush=True)
    got = fmha_prefill(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    for r in [0, 1, 31, 32, 127, 128, 255, 256, 1000, 4095, 4096, 8063, 8064, 8191]:
        ref = O.prefill_attention(q[r:r + 1], k[:r + 1], v[:r + 1], position_start=r,
                                  out_dtype=torch.float32)
        assert (got[r:r + 1] - ref).abs().max().item() <= TOL_TIGHT, r
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("s,t,tol", [
    # short: both launches split the key range, in different chunks, so P is
    # rounded to bf16 against different per-chunk reference maxima
    (1500, 700, TOL_TIGHT),
    # long, tile-aligned: both launches run the same unsplit 256-row tiles
    (8192, 4096, 1e-6)])
def test_prefix_extension_equals_tail_of_full_prefill(gpu, s, t, tol):
    """Bottom-right prefill over S equals the last T rows of a full causal
    prefill over S (prefix-cache continuation)."""
    from qwen36_attn.full_attention import fmha_prefill
    q, k, v = _inputs(s, s, seed=21)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    print(f"prefill prefix extension S={s} T={t}", flush=True)
    full = fmha_prefill(qd, kd, vd)
    tail = fmha_prefill(qd[s - t:].contiguous(), kd, vd)
    torch.cuda.synchronize()
    assert (full[s - t:] - tail).abs().max().item() <= tol


def test_provider_mirror_and_errors(gpu):
    from qwen36_attn import _lib
    from qwen36_attn.full_attention import FmhaProvider
    lib = _lib.load()
    assert lib.qrt_ck_fmha_prepare(0) == 1
    assert lib.qrt_ck_fmha_prepare(262145) == 1
    assert lib.qrt_ck_fmha_prepare(8192) == 0
    # kv_tokens < query_tokens is rejected without a launch.
    assert lib.qrt_ck_fmha_bf16_launch_ex(None, None, None, None, 4, 2, None) == 1
    prov = FmhaProvider()
    q, k, v = _inputs(256, 256, seed=2)
    out = prov.launch_ck_fmha(q=q.to(gpu), k=k.to(gpu), value=v.to(gpu))
    ref = O.prefill_attention(q, k, v, 0, out_dtype=torch.float32)
    assert (out.cpu() - ref).abs().max().item() <= TOL_TIGHT
    prov.release()


@pytest.mark.parametrize("t,s", [(256, 256), (300, 1500)])
def test_prefill_rising_scores_rescale(gpu, t, s):
    """Key norms grow along the sequence, so every row's running max keeps
    rising tile after tile and the kernel's rescale branch (O and l moved to
    a new reference max) runs repeatedly."""
    from qwen36_attn.full_attention import fmha_prefill
    q, k, v = _inputs(t, s, seed=11 + t)
    growth = torch.linspace(0.05, 6.0, s).view(s, 1, 1)
    k = (k.float() * growth).to(torch.bfloat16)
    print(f"prefill rising T={t} S={s}", flush=True)
    got = fmha_prefill(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    ref = O.prefill_attention(q, k, v, position_start=s - t, out_dtype=torch.float32)
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= TOL


def test_prefill_overflowing_jump_rescale(gpu):
    """Tiny keys in the first tile, then keys ~10^4 times larger: the first
    probabilities computed against the first tile's max overflow to inf, and
    the rescale branch must recompute them against the new max."""
    from qwen36_attn.full_attention import fmha_prefill
    t = s = 200
    q, k, v = _inputs(t, s, seed=5)
    scale = torch.full((s, 1, 1), 60.0)
    scale[:32] = 0.005
    k = (k.float() * scale).to(torch.bfloat16)
    print("prefill overflow jump", flush=True)
    got = fmha_prefill(q.to(gpu), k.to(gpu), v.to(gpu)).cpu()
    ref = O.prefill_attention(q, k, v, position_start=0, out_dtype=torch.float32)
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("t,s", [(262144, 262144), (131072, 262144)])
def test_prefill_max_tokens_sampled_rows(gpu, t, s):
    """The largest sizes the provider accepts (262144 tokens; square and
    bottom-right): inputs drawn on the device, every output finite, and rows
    spread over the range (first, tile edges, last) against the oracle
    restricted to those rows."""
    from qwen36_attn.full_attention import fmha_prefill
    g = torch.Generator(device=gpu).manual_seed(262 + t)
    q = torch.randn(t, 16, 256, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(s, 2, 256, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(s, 2, 256, generator=g, device=gpu).to(torch.bfloat16)
    print(f"prefill max T={t} S={s}", flush=True)
    got = fmha_prefill(q, k, v)
    assert torch.isfinite(got).all().item()
    kc, vc = k.cpu(), v.cpu()
    off = s - t
    for r in [0, 255, 256, t // 2 + 37, t - 257, t - 1]:
        lim = r + off + 1
        ref = O.prefill_attention(q[r:r + 1].cpu(), kc[:lim], vc[:lim], position_start=lim - 1,
                                  out_dtype=torch.float32)
        assert (got[r:r + 1].cpu() - ref).abs().max().item() <= TOL_TIGHT, r
    del q, k, v, got
    torch.cuda.empty_cache()


def test_short_prefills_on_two_streams(gpu):
    """Two short prompts (split-K launches) enqueued on two streams at once,
    through the provider ABI (the provider scratch belongs to the first
    stream that splits; the other stream's launch runs unsplit) and through
    qwen36_fmha_prefill with one workspace per stream: every output equals
    the oracle."""
    from qwen36_attn import _lib
    lib = _lib.load()
    assert lib.qrt_ck_fmha_prepare(1024) == 0
    cases = [_inputs(300, 300, seed=91), _inputs(500, 1400, seed=92)]
    refs = [O.prefill_attention(q, k, v, k.shape[0] - q.shape[0], out_dtype=torch.float32)
            for q, k, v in cases]
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    dev = [tuple(x.to(gpu) for x in c) for c in cases]
    for form in ("provider", "workspace"):
        print(f"two-stream short prefill ({form})", flush=True)
        outs, keep = [], []
        torch.cuda.synchronize()
        for rep in range(3):
            for (q, k, v), s in zip(dev, streams):
                out = torch.full((q.shape[0], 4096), float("nan"), device=gpu)
                with torch.cuda.stream(s):
                    # the NaN fill ran on the default stream: order it first
                    s.wait_stream(torch.cuda.default_stream(gpu))
                    h = s.cuda_stream
                    if form == "provider":
                        rc = lib.qrt_ck_fmha_bf16_launch_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                            out.data_ptr(), q.shape[0], k.shape[0], h)
                    else:
                        nb = lib.qwen36_fmha_prefill_workspace_bytes(q.shape[0], k.shape[0])
                        assert nb > 0
                        ws = torch.empty(nb, dtype=torch.uint8, device=gpu)
                        keep.append(ws)
                        rc = lib.qwen36_fmha_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                     out.data_ptr(), q.shape[0], k.shape[0],
                                                     ws.data_ptr(), nb, h)
                    assert rc == 0
                outs.append(out)
        torch.cuda.synchronize()
        for i, out in enumerate(outs):
            assert (out.cpu() - refs[i % 2]).abs().max().item() <= TOL_TIGHT, (form, i)
    # the workspace form rejects a missing or short workspace for a split geometry
    q, k, v = dev[0]
    out = torch.empty(q.shape[0], 4096, device=gpu)
    nb = lib.qwen36_fmha_prefill_workspace_bytes(q.shape[0], k.shape[0])
    assert lib.qwen36_fmha_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                   q.shape[0], k.shape[0], None, 0, None) == 1
    assert lib.qwen36_fmha_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                   q.shape[0], k.shape[0], 1, nb - 1, None) == 1
    assert lib.qwen36_fmha_prefill_workspace_bytes(8192, 8192) == 0


def test_config3_norm_rope_kv_write_and_gated_output(gpu):
    """Config 3 end to end: raw Q|gate [8192, 16 x 512], K/V new [8192, 2,
    256] and a 4096-row cached prefix.  Head norm + RoPE at absolute positions
    4096..12287 write K (normalised) and V (raw) into cache rows 4096..12287;
    the FMHA runs bottom-right causal over the 12288 rows; the sigmoid gate is
    applied.  Written rows vs the oracle's head_rmsnorm / apply_rope /
    write_kv_cache (V bit-exact, K to the bf16 bar with >= 99% bit-equal),
    the gated output on sampled rows vs the oracle's SDPA + output_gate
    (fle:5151-5162, 5980-5986, 6627-6650)."""
    from qwen36_attn.full_attention import (fmha_prefill, fmha_prefill_gated,
                                            head_norm_rope_kv_write, output_gate)
    from qwen36_attn import synthetic as syn
    t, pre = 8192, 4096
    s = pre + t
    g = syn.gen(33)
    qg = syn.randn((t, 8192), g)
    kn = syn.randn((t, 512), g)
    vn = syn.randn((t, 512), g)
    qw = syn.randn((256,), g, 0.1)
    kw = syn.randn((256,), g, 0.1)
    kc = torch.zeros(s, 2, 256, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[:pre] = syn.randn((pre, 2, 256), g)
    vc[:pre] = syn.randn((pre, 2, 256), g)
    print("config3 norm+rope+kv write + fmha + gate", flush=True)
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    qgd = qg.to(gpu)
    q = head_norm_rope_kv_write(qgd, kn.to(gpu), vn.to(gpu), qw.to(gpu), kw.to(gpu), kcd, vcd, pre)
    attn32 = fmha_prefill(q, kcd, vcd)
    gated_d = output_gate(attn32, qgd)
    # the fused form (gate in the FMHA epilogue) is the same bits
    assert torch.equal(fmha_prefill_gated(q, kcd, vcd, qgd), gated_d)
    gated = gated_d.cpu()
    kcg, vcg, qh = kcd.cpu(), vcd.cpu(), q.cpu()
    # oracle: the same three steps on the CPU
    cos, sin = O.rope_cos_sin(pre, t)
    q_ref, gate_ref = O.split_q_gate(qg)
    q_ref = O.apply_rope(O.head_rmsnorm(q_ref, qw), cos, sin)
    k_ref = O.apply_rope(O.head_rmsnorm(kn.view(t, 2, 256), kw), cos, sin)
    O.write_kv_cache(kc, vc, k_ref, vn.view(t, 2, 256), pre)
    assert torch.equal(vcg, vc)                      # raw V rows, and the prefix untouched
    assert torch.equal(kcg[:pre], kc[:pre])
    dk = (kcg[pre:].float() - kc[pre:].float()).abs()
    assert dk.max().item() <= TOL and (dk == 0).float().mean().item() >= 0.99
    dq = (qh.float() - q_ref.float()).abs()
    assert dq.max().item() <= TOL and (dq == 0).float().mean().item() >= 0.99
    # sampled rows of the gated output (rows are independent); the oracle
    # attends with its own K rows and the kernel's Q rows
    rows = [0, 1, 255, 256, 4095, 4096, 8191]
    for r in rows:
        lim = pre + r + 1
        a = O.prefill_attention(qh[r:r + 1], kc[:lim], vc[:lim], lim - 1, out_dtype=torch.float32)
        ref = O.output_gate(a.to(torch.bfloat16), gate_ref[r:r + 1])
        assert (gated[r:r + 1].float() - ref.float()).abs().max().item() <= TOL, r


@pytest.mark.parametrize("t,s", [(1, 1), (300, 300), (1024, 1024), (100, 4196), (4096, 4096),
                                 (2048, 6144), (4000, 4000), (3900, 5000)])
def test_gated_prefill_equals_fmha_then_gate(gpu, t, s):
    """The gate applied in the FMHA epilogue (unsplit) or in the split-K
    combine equals the two-launch path -- fp32 FMHA rows, then the gate
    kernel -- bit for bit, with the gate read through the [T, 9216] fused
    projection rows' column view."""
    from qwen36_attn.full_attention import fmha_prefill, fmha_prefill_gated, output_gate
    q, k, v = _inputs(t, s, seed=t + 3 * s)
    g = torch.Generator().manual_seed(t)
    fused = (torch.randn(t, 9216, generator=g) * 2).to(torch.bfloat16).to(gpu)
    q_gate = fused[:, :8192]
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    print(f"gated prefill T={t} S={s}", flush=True)
    two = output_gate(fmha_prefill(qd, kd, vd), q_gate)
    one = fmha_prefill_gated(qd, kd, vd, q_gate)
    torch.cuda.synchronize()
    assert torch.equal(one, two)
    assert one.shape == (t, 4096) and one.dtype == torch.bfloat16


@pytest.mark.parametrize("t", [16, 4096])
def test_gated_prefill_every_gate_value(gpu, t):
    """Every one of the 65536 bf16 gate bit patterns (infinities,
    subnormals, zeros of both signs included) through the fused gate --
    the split combine (T = 16) and the FMHA epilogue (T = 4096) -- gives the
    gate kernel's bits exactly (compared as bit patterns); a NaN gate gives
    a NaN in both (its sign and payload are not part of the contract)."""
    from qwen36_attn.full_attention import fmha_prefill, fmha_prefill_gated, output_gate
    q, k, v = _inputs(t, t, seed=77 + t)
    pats = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(16, 4096)
    gate = pats.repeat((t + 15) // 16, 1)[:t].view(torch.bfloat16)
    qg = torch.zeros(t, 8192, dtype=torch.bfloat16)
    qg.view(t, 16, 512)[:, :, 256:] = gate.view(t, 16, 256)
    qd, kd, vd, qgd = q.to(gpu), k.to(gpu), v.to(gpu), qg.to(gpu)
    print(f"gated prefill, all gate values, T={t}", flush=True)
    two = output_gate(fmha_prefill(qd, kd, vd), qgd)
    one = fmha_prefill_gated(qd, kd, vd, qgd)
    torch.cuda.synchronize()
    nan = torch.isnan(two)
    assert torch.equal(torch.isnan(one), nan)
    assert torch.equal(one.view(torch.int16)[~nan], two.view(torch.int16)[~nan])
    assert nan.sum().item() == 254 * t * 4096 // 65536   # the NaN patterns only


@pytest.mark.parametrize("t,pos", [(3072, 0), (3077, 4093), (4100, 123457)])
def test_head_norm_rope_rows_kernel_matches_per_head_form(gpu, t, pos):
    """The one-wave-per-token head norm + RoPE kernel (8-byte aligned rows,
    from 3072 tokens) gives the per-(token, head) kernel's bits (the same
    rows through an odd-strided view, which the library routes to that
    form): q, the normalised K rows and the raw V rows in the caches."""
    from qwen36_attn.full_attention import head_norm_rope_kv_write
    from qwen36_attn import synthetic as syn
    g = syn.gen(60 + t)
    qg = syn.randn((t, 8192), g).to(gpu)
    kr = syn.randn((t, 512), g).to(gpu)
    vr = syn.randn((t, 512), g).to(gpu)
    qw = syn.randn((256,), g, 0.1).to(gpu)
    kw = syn.randn((256,), g, 0.1).to(gpu)
    wide = torch.zeros(t, 8193, dtype=torch.bfloat16, device=gpu)
    wide[:, 1:] = qg
    cap = pos + t
    caches = [torch.zeros(cap, 2, 256, dtype=torch.bfloat16, device=gpu) for _ in range(4)]
    print(f"head norm rope rows vs per-head T={t} pos={pos}", flush=True)
    q1 = head_norm_rope_kv_write(qg, kr, vr, qw, kw, caches[0], caches[1], pos)
    q2 = head_norm_rope_kv_write(wide[:, 1:], kr, vr, qw, kw, caches[2], caches[3], pos)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])


def test_split_prefill_ignores_stale_workspace(gpu):
    """A short prompt (split key ranges + combine through the shared scratch)
    does not depend on what the scratch held before the call: NaN-filled
    scratch gives the same bits."""
    from qwen36_attn.full_attention import fmha_prefill
    from qwen36_attn import _tensors
    q, k, v = _inputs(700, 1500, seed=55)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    print("prefill stale workspace T=700 S=1500", flush=True)
    a = fmha_prefill(qd, kd, vd).clone()
    _tensors._SCRATCH[("fmha_split", gpu.index or 0)].fill_(0xFF)   # every float NaN
    b = fmha_prefill(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_q8192_f32_packed_launch(gpu):
    """The legacy fp32-packed provider launch (qrt_ck_fmha_q8192_f32_launch,
    qrt_ck_fmha_q8192_provider.cpp:228-271): rows [q | unused | k | v] of
    9216 fp32 values, rounded to bf16 and attended causally over 8192
    tokens -- equal, bit for bit, to the bf16 launch on the same rounded
    tensors; a second call after release re-allocates the staging."""
    from qwen36_attn import _lib
    from qwen36_attn.full_attention import fmha_prefill
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(8192)
    packed = torch.randn(8192, 9216, generator=g, device=gpu)
    q = packed[:, :4096].to(torch.bfloat16).view(8192, 16, 256).contiguous()
    k = packed[:, 8192:8704].to(torch.bfloat16).view(8192, 2, 256).contiguous()
    v = packed[:, 8704:].to(torch.bfloat16).view(8192, 2, 256).contiguous()
    print("q8192 f32 packed launch", flush=True)
    ref = fmha_prefill(q, k, v)
    h = torch.cuda.current_stream(gpu).cuda_stream
    for _ in range(2):
        out = torch.full((8192, 4096), float("nan"), device=gpu)
        assert lib.qrt_ck_fmha_q8192_prepare() == 0
        assert lib.qrt_ck_fmha_q8192_f32_launch(packed.data_ptr(), out.data_ptr(), h) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert lib.qrt_ck_fmha_q8192_release() == 0
    assert lib.qrt_ck_fmha_q8192_f32_launch(None, out.data_ptr(), h) == 1
