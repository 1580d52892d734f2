"""C = A @ B for the model's linear layers (the reference's kernel 3).

The reference writes its own tiled Triton GEMM (kernels/tiled_matmul.py) and
measures it against cuBLAS. On MI355X the plain library GEMM is hipBLASLt,
reached through torch.matmul; this module keeps the reference's entry point,
argument checks and AssertionErrors (kernels/tiled_matmul.py:135-140) so the
model code and the reference's tests call it unchanged. fp32 operands use
IEEE fp32 (torch's default, allow_tf32 off), as the reference's
input_precision="ieee" does.

Decode-time calls carry one row per sequence in the batch. There a GEMM is a
single pass over B's bytes, so bf16/fp16 products with M <= 2 go to the
library's skinny kernel (lsfa_gemv: one launch, a K-split pass over B at HBM
rate whose last workgroup per column block sums the fp32 partials and rounds
once), which hipBLASLt's general tiles reach at a fraction of the bandwidth.
From 3 to 32 rows, plain products whose widths are multiples of 128 run on
a second kernel that computes them on MFMA (W tiles through LDS, transposed
reads); measured on MI355X over the LLaMA-3-8B decode projections it beats
hipBLASLt up to 8 rows on the narrow products (q/k/v, o, down) but not on the
wide ones (gate/up, LM head), so matmul routes 3-8 rows to it only for
products of at most 8192 columns. The fused norm and SwiGLU inputs are
routed at up to 2 rows only: the MFMA kernel takes a gate too, but every
workgroup then evaluates the activation over its whole K-range for all 32
padded rows before its first product, which measured slower (batch-8 decode
step 1.043 ms) than torch's SiLU and multiply ahead of the plain product
(0.885 ms).

Projections that share their input (a decoder's q/k/v, gate/up) go through
matmul_shared_input, which runs them as one lsfa_gemv_group launch over their
concatenated columns when they qualify for the skinny kernel.
add_rmsnorm_matmul_shared_input also folds the residual add + RMSNorm that
precedes such projections into that launch (the norm computed exactly as
fused_add_rmsnorm computes it).

lsfa_gemv's workspace carries arrival counters (its first
LSFA_GEMV_COUNTER_BYTES) that must start at zero and that every call leaves
at zero, so this module keeps one workspace per (device, stream), zeroes its
counter bytes once when it is created, and reuses it for every call on that
stream (stream order keeps the calls apart). Workspaces start at 16 MB, so
they rarely grow. The cache is bounded: a workspace that grows is freed
unless a graph capture used it (a captured HIP graph that recorded it keeps
using it, so such workspaces stay until release_workspaces()), and at most
MAX_CACHED_STREAMS streams keep one, the least recently used uncaptured entry
going first. (A workspace first created inside a graph capture records its
counter fill into the graph, which then clears the 256 KB on every replay.)
"""
import collections

import torch

from .. import _lib

SKINNY_MAX_ROWS = 32  # what lsfa_gemv takes (more than 8 rows: MFMA kernel only)
AUTO_MAX_ROWS = 2    # rows that every product (and the fused norm / SwiGLU inputs) routes to it
# From 3 to 8 rows, plain products whose matrices are multiples of 128 columns
# wide and total at most this many columns run on the library's MFMA kernel
# (faster than hipBLASLt there: the q/k/v, o and down projections of a
# decoder); wider ones (gate/up, the LM head) stay on hipBLASLt.
MFMA_AUTO_ROWS = 8
MFMA_AUTO_MAX_COLS = 8192

MAX_CACHED_STREAMS = 8


class _Entry:
    __slots__ = ("buf", "captured", "kept")

    def __init__(self):
        self.buf = None       # the workspace in use
        self.captured = False  # a graph capture used buf
        self.kept = []         # smaller workspaces a captured graph may still use


# (device index, stream handle) -> _Entry, least recently used first
_workspaces = collections.OrderedDict()


def _workspace(device, stream, nbytes):
    key = (device.index, stream)
    entry = _workspaces.pop(key, None) or _Entry()
    if entry.buf is None or entry.buf.numel() < nbytes:
        if entry.buf is not None and entry.captured:
            entry.kept.append(entry.buf)
        entry.buf = torch.empty(max(nbytes, 16 << 20), dtype=torch.uint8, device=device)
        entry.buf[:_lib.GEMV_COUNTER_BYTES].zero_()
        entry.captured = False
    if torch.cuda.is_current_stream_capturing():
        entry.captured = True
    _workspaces[key] = entry
    while len(_workspaces) > MAX_CACHED_STREAMS:
        victim = next((k for k, e in _workspaces.items() if not e.captured and not e.kept), None)
        if victim is None:
            break
        del _workspaces[victim]
    return entry.buf


def release_workspaces():
    """Frees every cached skinny-GEMM workspace. Call it once no captured HIP
    graph that ran a skinny product is alive (those graphs keep using the
    workspaces they recorded)."""
    _workspaces.clear()


def _skinny_ok(a: torch.Tensor, b: torch.Tensor, max_rows: int = SKINNY_MAX_ROWS) -> bool:
    ok = (a.shape[0] <= max_rows and a.dtype in (torch.bfloat16, torch.float16)
          and a.stride(1) == 1 and b.stride(1) == 1 and b.shape[1] % 8 == 0
          and b.stride(0) % 8 == 0 and b.stride(0) >= b.shape[1] and b.data_ptr() % 16 == 0)
    if ok and a.shape[0] > 8:  # the MFMA kernel's conditions
        ok = (b.shape[1] % 128 == 0 and a.shape[1] % 8 == 0 and a.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0)
    return ok


def skinny_matmul(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
    """C = A @ B for a [M <= 32, K], b [K, N] (bf16/fp16, N % 8 == 0, rows of
    b 16-byte aligned) through lsfa_gemv; fp32 accumulation, one rounding."""
    assert _skinny_ok(a, b), ("skinny_matmul needs M <= 8 (or up to 32 with N % 128 == 0 and 16-byte aligned a "
                              "rows), bf16/fp16, unit column strides, N % 8 == 0")
    assert a.shape[1] == b.shape[0] and a.dtype == b.dtype and a.is_cuda and b.is_cuda, (
        "a [M, K] and b [K, N] must share K, dtype and device")
    M, K = a.shape
    N = b.shape[1]
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    assert out.shape == (M, N) and out.dtype == a.dtype and out.is_cuda and out.stride(1) == 1, (
        "out must be [M, N] in a's dtype with unit column stride")
    if M == 0 or N == 0:
        return out
    if K == 0:
        return out.zero_()
    args = _lib.GemvArgs(x=a.data_ptr(), w=b.data_ptr(), y=out.data_ptr(), workspace=None, workspace_bytes=0,
                         x_stride=a.stride(0), w_stride=b.stride(0), y_stride=out.stride(0),
                         dtype=_lib.TORCH_TO_LSFA[a.dtype], m=M, k=K, n=N)
    nbytes = _lib.gemv_workspace_size(args)
    with torch.cuda.device(a.device):
        stream = _lib.current_stream(a.device)
        if nbytes:
            ws = _workspace(a.device, stream, nbytes)
            args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
        _lib.gemv(args, stream)
    return out


def skinny_matmul_group(a: torch.Tensor, bs, outs=None, gate: torch.Tensor = None):
    """[a @ b for b in bs] for up to four b sharing a (each as for
    skinny_matmul) in one lsfa_gemv_group launch. With gate (a's shape and
    dtype), the products read F.silu(gate) * a instead of a, rounded as torch
    rounds it."""
    assert 1 <= len(bs) <= _lib.GEMV_MAX_GROUP, f"1..{_lib.GEMV_MAX_GROUP} matrices per group"
    assert gate is None or (gate.shape == a.shape and gate.dtype == a.dtype and gate.stride(1) == 1), (
        "gate must match a's shape and dtype, with unit column stride")
    assert all(_skinny_ok(a, b) and b.shape[0] == a.shape[1] and b.dtype == a.dtype for b in bs), (
        "every matrix must qualify for skinny_matmul with the shared input")
    M, K = a.shape
    assert a.is_cuda and all(b.is_cuda for b in bs), "GPU tensors expected"
    if outs is None:
        outs = [torch.empty(M, b.shape[1], dtype=a.dtype, device=a.device) for b in bs]
    assert len(outs) == len(bs) and all(
        o.shape == (M, b.shape[1]) and o.dtype == a.dtype and o.is_cuda and o.stride(1) == 1 for o, b in zip(outs, bs)), (
        "outs must be [M, N_i] in a's dtype with unit column stride")
    if M == 0 or sum(b.shape[1] for b in bs) == 0:
        return outs
    if K == 0:
        return [o.zero_() for o in outs]
    args = _lib.GemvGroupArgs(x=a.data_ptr(), x_stride=a.stride(0), dtype=_lib.TORCH_TO_LSFA[a.dtype], m=M, k=K,
                              count=len(bs))
    if gate is not None:
        args.x_gate, args.x_gate_stride = gate.data_ptr(), gate.stride(0)
    for i, (b, o) in enumerate(zip(bs, outs)):
        args.w[i], args.y[i] = b.data_ptr(), o.data_ptr()
        args.w_stride[i], args.y_stride[i], args.n[i] = b.stride(0), o.stride(0), b.shape[1]
    nbytes = _lib.gemv_group_workspace_size(args)
    with torch.cuda.device(a.device):
        stream = _lib.current_stream(a.device)
        if nbytes:
            ws = _workspace(a.device, stream, nbytes)
            args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
        _lib.gemv_group(args, stream)
    return outs


def _auto_skinny(a: torch.Tensor, bs) -> bool:
    """Whether matmul / matmul_shared_input route these products to the
    skinny kernels (see AUTO_MAX_ROWS and MFMA_AUTO_*)."""
    if not (len(bs) <= _lib.GEMV_MAX_GROUP and a.ndim == 2 and a.is_cuda and all(
            b.ndim == 2 and b.is_cuda and b.dtype == a.dtype and b.shape[0] == a.shape[1] for b in bs)):
        return False
    if a.shape[0] <= AUTO_MAX_ROWS:
        return all(_skinny_ok(a, b, AUTO_MAX_ROWS) for b in bs)
    return (a.shape[0] <= MFMA_AUTO_ROWS and sum(b.shape[1] for b in bs) <= MFMA_AUTO_MAX_COLS
            and all(_skinny_ok(a, b) and b.shape[1] % 128 == 0 for b in bs)
            and a.shape[1] % 8 == 0 and a.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0)


def matmul_shared_input(a: torch.Tensor, bs):
    """[matmul(a, b) for b in bs]: one grouped skinny launch when the
    products qualify for the skinny kernels, else one matmul each."""
    if _auto_skinny(a, bs):
        return skinny_matmul_group(a, bs)
    return [matmul(a, b) for b in bs]


def swiglu_matmul(gate: torch.Tensor, up: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """matmul(F.silu(gate) * up, b), the activation folded into the skinny
    kernel's load of its input when the product qualifies for it."""
    if (gate.ndim == 2 and gate.shape == up.shape and gate.dtype == up.dtype == b.dtype and gate.is_cuda
            and b.ndim == 2 and b.shape[0] == up.shape[1] and gate.stride(1) == 1 and _skinny_ok(up, b, AUTO_MAX_ROWS)):
        return skinny_matmul_group(up, [b], gate=gate)[0]
    return matmul(torch.nn.functional.silu(gate) * up, b)


def _rows_addressable(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def add_rmsnorm_matmul_shared_input(x, residual, weight, eps, bs, write_residual=True):
    """(outs, h) for h = x + residual (x alone when residual is None) and
    outs = [matmul(rmsnorm(h) * weight, b) for b in bs], the norm as
    fused_add_rmsnorm computes it. Products of at most AUTO_MAX_ROWS rows run
    as one skinny launch that also forms the norm (and writes h, when
    write_residual and residual is given); others run fused_add_rmsnorm (or
    rmsnorm) then matmul_shared_input. h is residual's replacement, as from
    fused_add_rmsnorm, or x itself when residual is None."""
    from .fused_rmsnorm_residual import fused_add_rmsnorm, rmsnorm
    assert x.ndim == 2 and weight.ndim == 1 and weight.shape[0] == x.shape[1], "x [M, K] and weight [K] expected"
    M, K = x.shape
    fused = (len(bs) <= _lib.GEMV_MAX_GROUP and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
             and K % 8 == 0 and _rows_addressable(x) and weight.is_contiguous() and weight.data_ptr() % 16 == 0
             and weight.dtype == x.dtype and (residual is None or (residual.shape == x.shape and residual.dtype == x.dtype
                                                                   and _rows_addressable(residual)))
             and all(b.ndim == 2 and b.is_cuda and b.dtype == x.dtype and b.shape[0] == K
                     and _skinny_ok(x, b, AUTO_MAX_ROWS) for b in bs))
    if not fused:
        normed, h = (fused_add_rmsnorm(x, residual, weight, eps) if residual is not None
                     else (rmsnorm(x, weight, eps), x))
        return matmul_shared_input(normed, bs), h
    h = torch.empty_like(x) if (residual is not None and write_residual) else None
    outs = [torch.empty(M, b.shape[1], dtype=x.dtype, device=x.device) for b in bs]
    if M == 0:
        return outs, (h if residual is not None else x)
    args = _lib.GemvGroupArgs(x=x.data_ptr(), x_stride=x.stride(0), dtype=_lib.TORCH_TO_LSFA[x.dtype], m=M, k=K,
                              count=len(bs), norm_weight=weight.data_ptr(), eps=float(eps))
    if residual is not None:
        args.residual, args.residual_stride = residual.data_ptr(), residual.stride(0)
    if h is not None:
        args.residual_out, args.residual_out_stride = h.data_ptr(), h.stride(0)
    for i, (b, o) in enumerate(zip(bs, outs)):
        args.w[i], args.y[i] = b.data_ptr(), o.data_ptr()
        args.w_stride[i], args.y_stride[i], args.n[i] = b.stride(0), o.stride(0), b.shape[1]
    nbytes = _lib.gemv_group_workspace_size(args)
    with torch.cuda.device(x.device):
        stream = _lib.current_stream(x.device)
        if nbytes:
            ws = _workspace(x.device, stream, nbytes)
            args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
        _lib.gemv_group(args, stream)
    return outs, (h if residual is not None else x)


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A @ B. a: [M, K], b: [K, N], same dtype, both on the GPU."""
    assert a.ndim == 2 and b.ndim == 2, f"expected 2D matrices, got {a.ndim}D and {b.ndim}D"
    assert a.shape[1] == b.shape[0], f"inner dims must match: a is {tuple(a.shape)}, b is {tuple(b.shape)}"
    assert a.is_cuda and b.is_cuda, "the gfx950 path needs GPU tensors"
    assert a.dtype == b.dtype, f"dtype mismatch: a={a.dtype} b={b.dtype}"
    if _auto_skinny(a, [b]):
        return skinny_matmul(a, b)
    return torch.matmul(a, b)
