"""Fused residual add + RMSNorm on MI355X (the reference's kernel 2).

    fused_add_rmsnorm(x, residual, weight, eps=1e-6) -> (out, h)

h = x + residual (the new residual, in the input dtype) and
out = h / sqrt(mean(h^2, -1) + eps) * weight with fp32 statistics, as the
reference computes them (kernels/fused_rmsnorm_residual.py:30-70, same
signature, argument checks and AssertionErrors in the same order,
:73-103). One HIP launch (lsfa_rmsnorm), one workgroup per row.
rmsnorm(x, weight, eps) is the same kernel without the residual (the first
norm of a decoder, whose input is the embedding itself).
"""
import torch

from .. import _lib


def _launch(x, residual, weight, eps, out, residual_out):
    M, N = x.shape
    args = _lib.RmsNormArgs(
        x=x.data_ptr(), residual=residual.data_ptr() if residual is not None else None,
        weight=weight.data_ptr(), out=out.data_ptr(),
        residual_out=residual_out.data_ptr() if residual_out is not None else None,
        x_stride=x.stride(0), residual_stride=residual.stride(0) if residual is not None else 0,
        out_stride=out.stride(0), residual_out_stride=residual_out.stride(0) if residual_out is not None else 0,
        dtype=_lib.TORCH_TO_LSFA[x.dtype], rows=M, cols=N, eps=float(eps),
    )
    with torch.cuda.device(x.device):
        _lib.rmsnorm(args, _lib.current_stream(x.device))


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    """h = x + residual; returns (rmsnorm(h) * weight, h)."""
    assert x.shape == residual.shape and x.ndim == 2, (
        f"x {tuple(x.shape)} and residual {tuple(residual.shape)} must both be 2D and equal-shaped"
    )
    assert weight.ndim == 1 and weight.shape[0] == x.shape[1], (
        f"weight shape {tuple(weight.shape)} must match x's last dim {x.shape[1]}"
    )
    assert x.is_cuda and residual.is_cuda and weight.is_cuda, "the gfx950 kernels need GPU tensors"
    assert x.dtype == residual.dtype == weight.dtype, (
        f"dtype mismatch: x={x.dtype} residual={residual.dtype} weight={weight.dtype}"
    )
    assert x.stride(1) == 1 and residual.stride(1) == 1, (
        "x and residual must be contiguous along the last dim (row-major, no transposed views)"
    )
    assert x.dtype in _lib.TORCH_TO_LSFA, f"unsupported dtype {x.dtype}"
    out = torch.empty_like(x)
    residual_out = torch.empty_like(x)
    if x.numel():
        _launch(x, residual, weight.contiguous(), eps, out, residual_out)
    return out, residual_out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    """x / sqrt(mean(x^2, -1) + eps) * weight for x [M, N] (fp32 statistics)."""
    assert x.ndim == 2 and weight.ndim == 1 and weight.shape[0] == x.shape[1], "x [M, N] and weight [N] expected"
    assert x.is_cuda and weight.is_cuda, "the gfx950 kernels need GPU tensors"
    assert x.dtype == weight.dtype and x.dtype in _lib.TORCH_TO_LSFA, "x and weight must share a supported dtype"
    assert x.stride(1) == 1, "x must be contiguous along the last dim"
    out = torch.empty_like(x)
    if x.numel():
        _launch(x, None, weight.contiguous(), eps, out, None)
    return out
