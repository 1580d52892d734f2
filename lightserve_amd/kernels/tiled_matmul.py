"""C = A @ B for the model's linear layers (the reference's kernel 3).

The reference writes its own tiled Triton GEMM (kernels/tiled_matmul.py) and
measures it against cuBLAS. On MI355X the plain library GEMM is hipBLASLt,
reached through torch.matmul; this module keeps the reference's entry point,
argument checks and AssertionErrors (kernels/tiled_matmul.py:135-140) so the
model code and the reference's tests call it unchanged. fp32 operands use
IEEE fp32 (torch's default, allow_tf32 off), as the reference's
input_precision="ieee" does.
"""
import torch


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A @ B. a: [M, K], b: [K, N], same dtype, both on the GPU."""
    assert a.ndim == 2 and b.ndim == 2, f"expected 2D matrices, got {a.ndim}D and {b.ndim}D"
    assert a.shape[1] == b.shape[0], f"inner dims must match: a is {tuple(a.shape)}, b is {tuple(b.shape)}"
    assert a.is_cuda and b.is_cuda, "the gfx950 path needs GPU tensors"
    assert a.dtype == b.dtype, f"dtype mismatch: a={a.dtype} b={b.dtype}"
    return torch.matmul(a, b)
