"""GPU parity of the decode-batch linear layer (mvme_linear_rows) and
HipLinear, the hip counterpart of the reference's CudaLinear
(mini_engine/kernels/linear.py:14-30; tests/test_prefill_linear_chat.py:33-40).
Tolerance: fp32 accumulation rounded once to the output type -- within two
output ulps of the fp32 product, and at least 99 % of the elements equal to
the fp32 product rounded to the type."""

import pytest
import torch

from mini_engine_hip.kernels.linear import HipLinear, linear_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ulp(x, dtype):
    bits = 10 if dtype == torch.float16 else 7
    return torch.clamp(x.abs(), min=2.0 ** -14) * 2.0 ** -bits


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,k,n,bias", [
    (1, 2048, 2048, False), (7, 64, 48, True), (16, 256, 16, False), (32, 2048, 2048, False),
    (33, 512, 1024, True), (64, 1024, 512, False), (0, 64, 16, False),
])
def test_linear_rows_matches_fp32_product(dtype, rows, k, n, bias):
    gen = torch.Generator().manual_seed(rows * 7 + k + n)
    x = torch.randn(rows, k, generator=gen).to(dtype)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(dtype)
    b = torch.randn(n, generator=gen).to(dtype) if bias else None
    actual = linear_rows(x.to(DEV), w.to(DEV), b.to(DEV) if bias else None).cpu()
    exact = x.float() @ w.float().t() + (b.float() if bias else 0.0)
    assert actual.shape == (rows, n)
    if rows == 0:
        return
    assert ((actual.float() - exact).abs() <= 2 * ulp(exact, dtype) + 1e-6).all()
    assert (actual == exact.to(dtype)).float().mean().item() >= 0.99


def test_linear_rows_strided_input_rows():
    """x as a row slice of a wider buffer (row stride > in_features)."""
    gen = torch.Generator().manual_seed(3)
    buf = torch.randn(5, 96, generator=gen).to(torch.bfloat16)
    x = buf[:, 16:80]
    w = (torch.randn(32, 64, generator=gen) * 0.125).to(torch.bfloat16)
    dev = buf.to(DEV)[:, 16:80]
    actual = linear_rows(dev, w.to(DEV)).cpu()
    exact = x.float() @ w.float().t()
    assert ((actual.float() - exact).abs() <= 2 * ulp(exact, torch.bfloat16) + 1e-6).all()


def test_hip_linear_matches_torch_linear():
    """The reference's test_cuda_linear_matches_torch_linear for HipLinear, and the
    decode shape that takes the HIP kernel."""
    torch.manual_seed(73)
    ref = torch.nn.Linear(7, 5, bias=True, device=DEV, dtype=torch.bfloat16).eval()
    actual = HipLinear(7, 5, bias=True, device=DEV, dtype=torch.bfloat16).eval()
    actual.load_state_dict(ref.state_dict())
    x = torch.randn(2, 3, 7, device=DEV, dtype=torch.bfloat16)
    torch.testing.assert_close(actual(x), ref(x), atol=0.004, rtol=0.01)
    ref = torch.nn.Linear(2048, 2048, bias=False, device=DEV, dtype=torch.bfloat16).eval()
    actual = HipLinear(2048, 2048, bias=False, device=DEV, dtype=torch.bfloat16).eval()
    actual.load_state_dict(ref.state_dict())
    x = torch.randn(32, 2048, device=DEV, dtype=torch.bfloat16)
    torch.testing.assert_close(actual(x), ref(x), atol=0.004, rtol=0.01)
    # 65 rows are a GEMM for the library: same answer.
    x = torch.randn(65, 2048, device=DEV, dtype=torch.bfloat16)
    torch.testing.assert_close(actual(x), ref(x), atol=0.004, rtol=0.01)


def test_linear_rows_rejects_unsupported_shapes():
    x = torch.randn(65, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(16, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="at most 64 rows"):
        linear_rows(x, w)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        linear_rows(torch.randn(4, 40, device=DEV, dtype=torch.bfloat16),
                    torch.randn(16, 40, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="multiple of 16"):
        linear_rows(torch.randn(4, 64, device=DEV, dtype=torch.bfloat16),
                    torch.randn(24, 64, device=DEV, dtype=torch.bfloat16))
    # A caller-supplied output must match the product exactly.
    x = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(16, 64, device=DEV, dtype=torch.bfloat16)
    for bad in (torch.empty(4, 8, device=DEV, dtype=torch.bfloat16),
                torch.empty(4, 16, device=DEV, dtype=torch.float16),
                torch.empty(16, 4, device=DEV, dtype=torch.bfloat16).t(),
                torch.empty(4, 16, dtype=torch.bfloat16)):
        with pytest.raises(ValueError, match="out must be"):
            linear_rows(x, w, out=bad)
    with pytest.raises(ValueError, match="share a device"):
        linear_rows(x, w, torch.zeros(16, dtype=torch.bfloat16))
