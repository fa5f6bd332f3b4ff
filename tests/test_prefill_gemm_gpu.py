"""GPU parity of the prefill projection GEMM -- the MFMA kernel
(qwen36_prefill_gemm_bf16[_ws]) and the hipBLASLt entry point
(qwen36_prefill_gemm_bf16_lt) -- against an fp32 GEMM of the same bf16 operands: y = bf16(x W^T) rounds once,
so every output is within half a bf16 ulp of the fp32 result plus the
fp32 summation-order difference."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _check(y, ref):
    err = (y.float() - ref).abs()
    bound = 2 ** -8 * ref.abs() + 1e-4 * ref.abs().max()
    assert (err <= bound).all(), (err - bound).max().item()


@pytest.mark.parametrize("m,n,k", [(1, 32, 2048), (37, 9216, 2048), (300, 2048, 4096),
                                   (1024, 12352, 2048), (777, 512, 2048), (129, 300, 128),
                                   (8192, 2048, 4096)])
@pytest.mark.parametrize("backend", ["native", "hipblaslt"])
def test_prefill_gemm_matches_fp32(gpu, m, n, k, backend):
    from qwen36_attn.prefill_gemm import linear
    g = torch.Generator(device=gpu).manual_seed(m * 31 + n)
    x = (torch.randn(m, k, generator=g, device=gpu) * 0.5).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    print(f"prefill gemm {m}x{n}x{k} {backend}", flush=True)
    y = linear(x, w, backend=backend)
    ref = x.float() @ w.float().t()
    _check(y, ref)


@pytest.mark.parametrize("backend", ["native", "hipblaslt"])
def test_prefill_gemm_strided_operands(gpu, backend):
    """x a column slice of a wider row (ldx > K), y written into a column
    slice of a wider output (ldy > N); the rest of the output untouched."""
    from qwen36_attn.prefill_gemm import linear
    g = torch.Generator(device=gpu).manual_seed(5)
    xb = torch.randn(513, 4096 + 64, generator=g, device=gpu).to(torch.bfloat16)
    x = xb[:, 64:]
    w = (torch.randn(2048, 4096, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    yb = torch.full((513, 3000), 7.0, dtype=torch.bfloat16, device=gpu)
    y = linear(x, w, out=yb[:, 500:2548], backend=backend)
    _check(y, x.float() @ w.float().t())
    assert (yb[:, :500] == 7).all() and (yb[:, 2548:] == 7).all()


@pytest.mark.parametrize("m", [300, 600])
def test_prefill_gemm_lt_split_width_strided_output(gpu, m):
    """An output width past a multiple of 4096 (4160 = 4096 + 64), which the
    hipBLASLt entry runs as one product up to 512 rows and as two from 513,
    written into a column slice of a wider output: every part lands in its
    columns, the rest untouched."""
    from qwen36_attn.prefill_gemm import linear
    g = torch.Generator(device=gpu).manual_seed(6)
    x = torch.randn(m, 256, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(4160, 256, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    yb = torch.full((m, 4400), 7.0, dtype=torch.bfloat16, device=gpu)
    y = linear(x, w, out=yb[:, 120:4280], backend="hipblaslt")
    _check(y, x.float() @ w.float().t())
    assert (yb[:, :120] == 7).all() and (yb[:, 4280:] == 7).all()


def test_prefill_gemm_rejects_bad_shapes(gpu):
    from qwen36_attn import _lib
    lib = _lib.load()
    x = torch.zeros(4, 2048, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(8, 2048, dtype=torch.bfloat16, device=gpu)
    y = torch.zeros(4, 8, dtype=torch.bfloat16, device=gpu)
    call = lambda *a: lib.qwen36_prefill_gemm_bf16(*a, None)
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 8, 4, 8, 2000) == 1   # k % 64
    assert call(x.data_ptr(), 2000, w.data_ptr(), y.data_ptr(), 8, 4, 8, 2048) == 1   # ldx < k
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 4, 4, 8, 2048) == 1   # ldy < n
    assert call(x.data_ptr() + 2, 2048, w.data_ptr(), y.data_ptr(), 8, 4, 8, 2048) == 1
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 8, 0, 8, 2048) == 1


@pytest.mark.parametrize("m,n,k", [(1024, 2048, 4096), (300, 2048, 4096), (256, 2048, 4096),
                                   (37, 9216, 2048), (1, 32, 2048), (1024, 1024, 2048)])
def test_prefill_gemm_split_k_matches_whole_k(gpu, m, n, k):
    """Shapes whose workspace form cuts K into slices: the sliced result is
    within the fp32 bound of the fp32 GEMM, deterministic across calls (the
    slices are summed in order), and the workspace is fully rewritten (a
    workspace full of NaN from an earlier use changes nothing)."""
    from qwen36_attn import _lib
    lib = _lib.load()
    nb = lib.qwen36_prefill_gemm_workspace_bytes(m, n, k)
    assert nb >= 2 * m * n * 4 and nb % (m * n * 4) == 0
    g = torch.Generator(device=gpu).manual_seed(m + 7 * n)
    x = (torch.randn(m, k, generator=g, device=gpu) * 0.5).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    ws = torch.full((nb // 4,), float("nan"), device=gpu)
    h = torch.cuda.current_stream(gpu).cuda_stream
    print(f"split-K gemm {m}x{n}x{k}, workspace {nb} B", flush=True)
    ys = []
    for _ in range(2):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        assert lib.qwen36_prefill_gemm_bf16_ws(x.data_ptr(), k, w.data_ptr(), y.data_ptr(), n,
                                               m, n, k, ws.data_ptr(), nb, h) == 0
        ys.append(y)
    y0 = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    assert lib.qwen36_prefill_gemm_bf16(x.data_ptr(), k, w.data_ptr(), y0.data_ptr(), n,
                                        m, n, k, h) == 0
    torch.cuda.synchronize()
    ref = x.float() @ w.float().t()
    _check(ys[0], ref)
    _check(y0, ref)
    assert torch.equal(ys[0], ys[1])
    # one rounding of nearly the same fp32 sum: at most one bf16 ulp apart
    d = (ys[0].float() - y0.float()).abs()
    assert (d <= 2 ** -7 * y0.float().abs() + 1e-6).all()


def test_prefill_gemm_ws_rejects_small_workspace(gpu):
    from qwen36_attn import _lib
    lib = _lib.load()
    m, n, k = 300, 2048, 4096
    nb = lib.qwen36_prefill_gemm_workspace_bytes(m, n, k)
    assert nb > 0
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=gpu)
    y = torch.zeros(m, n, dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(nb, dtype=torch.uint8, device=gpu)
    call = lambda p, b: lib.qwen36_prefill_gemm_bf16_ws(x.data_ptr(), k, w.data_ptr(),
                                                        y.data_ptr(), n, m, n, k, p, b, None)
    assert call(ws.data_ptr(), nb - 16) == 1
    assert call(None, 0) == 1
    assert call(ws.data_ptr() + 4, nb - 16) == 1
    # a shape that runs unsplit needs no workspace
    assert lib.qwen36_prefill_gemm_workspace_bytes(8192, 2048, 4096) == 0
    x2 = torch.zeros(8192, 4096, dtype=torch.bfloat16, device=gpu)
    y2 = torch.zeros(8192, 2048, dtype=torch.bfloat16, device=gpu)
    assert lib.qwen36_prefill_gemm_bf16_ws(x2.data_ptr(), k, w.data_ptr(), y2.data_ptr(), n,
                                           8192, n, k, None, 0, None) == 0
    torch.cuda.synchronize()


def test_prefill_gemm_lt_rejects_bad_arguments(gpu):
    from qwen36_attn import _lib
    lib = _lib.load()
    nb = lib.qwen36_prefill_gemm_lt_workspace_bytes()
    ws = torch.zeros(nb, dtype=torch.uint8, device=gpu)
    x = torch.zeros(4, 2048, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(8, 2048, dtype=torch.bfloat16, device=gpu)
    y = torch.zeros(4, 8, dtype=torch.bfloat16, device=gpu)
    call = lambda *a: lib.qwen36_prefill_gemm_bf16_lt(*a, ws.data_ptr(), nb, None)
    assert call(x.data_ptr(), 2000, w.data_ptr(), y.data_ptr(), 8, 4, 8, 2048) == 1   # ldx < k
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 4, 4, 8, 2048) == 1   # ldy < n
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 8, 0, 8, 2048) == 1   # m = 0
    assert call(x.data_ptr(), 2048, w.data_ptr(), y.data_ptr(), 8, 4, 8, 2048) == 0
    torch.cuda.synchronize()
