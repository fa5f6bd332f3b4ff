"""GPU parity of the prefill projection GEMM (qwen36_prefill_gemm_bf16)
against an fp32 GEMM of the same bf16 operands: y = bf16(x W^T) rounds once,
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
def test_prefill_gemm_matches_fp32(gpu, m, n, k):
    from qwen36_attn.prefill_gemm import linear
    g = torch.Generator(device=gpu).manual_seed(m * 31 + n)
    x = (torch.randn(m, k, generator=g, device=gpu) * 0.5).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    print(f"prefill gemm {m}x{n}x{k}", flush=True)
    y = linear(x, w)
    ref = x.float() @ w.float().t()
    _check(y, ref)


def test_prefill_gemm_strided_operands(gpu):
    """x a column slice of a wider row (ldx > K), y written into a column
    slice of a wider output (ldy > N); the rest of the output untouched."""
    from qwen36_attn.prefill_gemm import linear
    g = torch.Generator(device=gpu).manual_seed(5)
    xb = torch.randn(513, 4096 + 64, generator=g, device=gpu).to(torch.bfloat16)
    x = xb[:, 64:]
    w = (torch.randn(2048, 4096, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    yb = torch.full((513, 3000), 7.0, dtype=torch.bfloat16, device=gpu)
    y = linear(x, w, out=yb[:, 500:2548])
    _check(y, x.float() @ w.float().t())
    assert (yb[:, :500] == 7).all() and (yb[:, 2548:] == 7).all()


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
