"""GPU parity of the fused add + RMSNorm kernel and the matmul entry point
(scope row f4: the reference's kernels/fused_rmsnorm_residual.py and
kernels/tiled_matmul.py, with its tests kernels/tests/test_fused_rmsnorm_residual.py
and kernels/tests/test_tiled_matmul.py as the model).

RMSNorm against oracle.model.add_rmsnorm_reference at the reference test's
shapes and tolerances (fp32 1e-5, bf16/fp16 2e-2), plus widths that take the
16-byte register path at its largest (16384), the scalar path (20000, odd
widths, strided rows) and the no-residual form; h must equal x + residual
exactly.
"""
import pytest
import torch

from lightserve_amd.kernels.fused_rmsnorm_residual import fused_add_rmsnorm, rmsnorm
from lightserve_amd.kernels.tiled_matmul import matmul
from oracle.model import add_rmsnorm_reference

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (1, 17), (37, 300), (8, 4096), (4, 4097), (2, 8192), (3, 16384), (2, 20000), (64, 1000)]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


@pytest.mark.parametrize("M,N", SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matches_reference(M, N, dtype):
    print(f"case rmsnorm M={M} N={N} {dtype}", flush=True)
    torch.manual_seed(0)
    x = torch.randn(M, N, device="cuda", dtype=dtype)
    residual = torch.randn(M, N, device="cuda", dtype=dtype)
    weight = torch.randn(N, device="cuda", dtype=dtype)
    out, h = fused_add_rmsnorm(x, residual, weight, 1e-6)
    ref_out, ref_h = add_rmsnorm_reference(x, residual, weight, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(h, ref_h)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out, ref_out, atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", DTYPES)
def test_without_residual_and_strided_rows(dtype):
    """rmsnorm(x) with rows of a wider buffer (row stride > cols)."""
    print(f"case rmsnorm strided {dtype}", flush=True)
    torch.manual_seed(1)
    big = torch.randn(16, 4200, device="cuda", dtype=dtype)
    x = big[:, 8:4104]                       # 4096 columns, row stride 4200, 16-byte aligned start
    w = torch.randn(4096, device="cuda", dtype=dtype)
    out = rmsnorm(x, w, 1e-5)
    ref, _ = add_rmsnorm_reference(x, None, w, 1e-5)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out, ref, atol=tol, rtol=tol)
    x2 = big[:, 3:4099]                      # misaligned start: scalar path
    torch.testing.assert_close(rmsnorm(x2, w, 1e-5), add_rmsnorm_reference(x2, None, w, 1e-5)[0], atol=tol, rtol=tol)


def test_output_is_unit_rms_before_weight():
    print("case rmsnorm unit rms", flush=True)
    torch.manual_seed(0)
    x = torch.randn(16, 512, device="cuda")
    r = torch.randn(16, 512, device="cuda")
    out, _ = fused_add_rmsnorm(x, r, torch.ones(512, device="cuda"), eps=1e-6)
    torch.testing.assert_close(out.pow(2).mean(-1).sqrt(), torch.ones(16, device="cuda"), atol=1e-3, rtol=1e-3)


def test_zero_row_stays_finite_via_eps():
    print("case rmsnorm zero rows", flush=True)
    x = torch.zeros(4, 128, device="cuda")
    out, h = fused_add_rmsnorm(x, torch.zeros_like(x), torch.randn(128, device="cuda"), eps=1e-6)
    assert torch.isfinite(out).all() and (h == 0).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (128, 4096, 14336), (37, 100, 29)])
def test_matmul(M, K, N, dtype):
    print(f"case matmul {M}x{K}x{N} {dtype}", flush=True)
    torch.manual_seed(0)
    a = torch.randn(M, K, device="cuda", dtype=dtype)
    b = torch.randn(K, N, device="cuda", dtype=dtype)
    c = matmul(a, b)
    ref = (a.double() @ b.double())
    tol = 1e-3 * K ** 0.5 if dtype == torch.float32 else 2e-2 * K ** 0.5
    torch.testing.assert_close(c.double(), ref, atol=tol, rtol=1e-2)
