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
from lightserve_amd import _lib
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


def _assert_one_rounding(c, a, b):
    """c must be the fp32 product rounded once to c's dtype: within one ulp of
    the dtype (2^-7 relative for bf16, 2^-10 for fp16) of the fp64 product,
    plus the fp32 accumulation error of a K-term sum."""
    ref = a.double() @ b.double()
    K = a.shape[1]
    rel = 2.0 ** -7 if c.dtype == torch.bfloat16 else 2.0 ** -10
    bound = ref.abs() * rel + 4 * K * 2.0 ** -24 * (a.double().abs() @ b.double().abs()) + 1e-30
    err = (c.double() - ref).abs()
    assert (err <= bound).all(), f"max excess {(err - bound).max().item():.3e}"


SKINNY_KN = [(4096, 4096), (4096, 1024), (14336, 4096), (4096, 14336), (100, 8), (1, 8), (4097, 4104),
             (20000, 264), (2048, 128256)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,N", SKINNY_KN)
def test_skinny_matmul_all_row_counts(K, N, dtype):
    """lsfa_gemv for 1..8 rows (capacities 1/2/4/8, and 3, 5-7 through the
    next one up) against the fp64 product, one rounding from fp32."""
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul
    print(f"case gemv K={K} N={N} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(K + N)
    b = (torch.randn(K, N, device="cuda", generator=g) / K ** 0.5).to(dtype)
    for M in range(1, 9):
        a = torch.randn(M, K, device="cuda", generator=g).to(dtype)
        c = skinny_matmul(a, b)
        torch.cuda.synchronize()
        _assert_one_rounding(c, a, b)


def test_skinny_matmul_strided_and_dispatch():
    """Row strides on x, w and y; matmul routes M <= 2 to the skinny kernel
    (bit-identical) and larger M to hipBLASLt; results are deterministic."""
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul
    print("case gemv strided / dispatch", flush=True)
    torch.manual_seed(3)
    xb = torch.randn(6, 3000, device="cuda", dtype=torch.bfloat16)
    wb = (torch.randn(2500, 1104, device="cuda") / 50).to(torch.bfloat16)
    x, w = xb[:, 5:2505], wb[:, 8:1032]        # x misaligned start, w rows 16-byte aligned
    yb = torch.zeros(6, 1200, device="cuda", dtype=torch.bfloat16)
    y = skinny_matmul(x, w, out=yb[:, 16:1040])
    torch.cuda.synchronize()
    _assert_one_rounding(y, x, w)
    assert (yb[:, :16] == 0).all() and (yb[:, 1040:] == 0).all()
    assert torch.equal(skinny_matmul(x, w), y)
    assert torch.equal(matmul(x[:2], w), skinny_matmul(x[:2], w))
    big = torch.randn(3, 2500, device="cuda", dtype=torch.bfloat16)
    torch.testing.assert_close(matmul(big, w).float(), (big.float() @ w.float()), atol=5e-2, rtol=2e-2)
    assert skinny_matmul(x[:, :0], w[:0]).abs().sum() == 0  # K = 0: zeros


def test_skinny_matmul_in_graph_replays():
    """Captured in a HIP graph, every replay matches the eager result (the
    workspace comes from the graph's pool; no memsets are recorded)."""
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul
    print("case gemv graph", flush=True)
    torch.manual_seed(4)
    x = torch.randn(4, 4096, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(4096, 4096, device="cuda") / 64).to(torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        skinny_matmul(x, w)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = skinny_matmul(x, w)
    for i in range(4):
        x.copy_(torch.randn(4, 4096, device="cuda", dtype=torch.bfloat16))
        eager = skinny_matmul(x, w)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"


def test_skinny_workspace_cache_is_bounded():
    """The skinny GEMM's per-stream workspace cache keeps at most
    MAX_CACHED_STREAMS entries (the least recently used entry no graph capture
    used goes first), results stay exact on every stream, a workspace used
    under graph capture is kept, and release_workspaces() empties the cache."""
    from lightserve_amd.kernels import tiled_matmul as tm
    print("case skinny workspace cache", flush=True)
    tm.release_workspaces()
    torch.manual_seed(9)
    a = torch.randn(1, 8192, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(8192, 1024, device="cuda", dtype=torch.bfloat16)
    args = _lib.GemvArgs(x=16, w=16, y=16, workspace=None, workspace_bytes=0, x_stride=8192, w_stride=1024,
                         y_stride=1024, dtype=_lib.DTYPE_BF16, m=1, k=8192, n=1024)
    assert _lib.gemv_workspace_size(args) > 0  # split K: the call needs a workspace
    ref = tm.skinny_matmul(a, b)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(tm.MAX_CACHED_STREAMS + 4)]
    for s in streams:
        with torch.cuda.stream(s):
            out = tm.skinny_matmul(a, b)
        s.synchronize()
        assert torch.equal(out, ref)
        assert len(tm._workspaces) <= tm.MAX_CACHED_STREAMS
    # a capture on a fresh stream marks its workspace as used by a graph
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        out = tm.skinny_matmul(a, b)  # creates the workspace (and zeroes its counters) outside the capture
        cap.synchronize()
        with torch.cuda.graph(g, stream=cap):
            out = tm.skinny_matmul(a, b)
    key = (torch.cuda.current_device(), cap.cuda_stream)
    assert tm._workspaces[key].captured
    for s in streams:
        with torch.cuda.stream(s):
            tm.skinny_matmul(a, b)
        s.synchronize()
    assert key in tm._workspaces  # captured: never evicted
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    del g
    tm.release_workspaces()
    assert not tm._workspaces


def test_skinny_matmul_counters_return_to_zero():
    """The last workgroup of each column block clears its arrival counter:
    after calls of several shapes the stream's workspace counters read zero,
    and repeated calls give bit-identical results."""
    from lightserve_amd.kernels import tiled_matmul
    print("case gemv counters", flush=True)
    torch.manual_seed(5)
    for M, K, N in [(3, 4096, 4096), (1, 14336, 4096), (8, 4096, 14336), (2, 4096, 128256)]:
        x = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        w = (torch.randn(K, N, device="cuda") / K ** 0.5).to(torch.bfloat16)
        first = tiled_matmul.skinny_matmul(x, w)
        again = tiled_matmul.skinny_matmul(x, w)
        torch.cuda.synchronize()
        assert torch.equal(first, again), (M, K, N)
        ws = tiled_matmul._workspaces[(0, torch.cuda.current_stream().cuda_stream)].buf
        # the whole counter region: the VALU kernel keeps 16 counters per 256
        # columns, the MFMA kernel (3 and 8 rows here) 16 per 128
        assert (ws[:_lib.GEMV_COUNTER_BYTES] == 0).all(), (M, K, N)


@pytest.mark.parametrize("M", [1, 3, 8])
def test_skinny_matmul_group(M):
    """One grouped launch over matrices of widths that do not divide into
    256-column blocks (blocks straddle matrices), with strided outputs; the
    decoder's q/k/v and gate/up groups through matmul_shared_input."""
    from lightserve_amd.kernels.tiled_matmul import matmul_shared_input, skinny_matmul_group
    print(f"case gemv group M={M}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M)
    K = 3000
    a = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    bs = [(torch.randn(K, n, device="cuda", generator=g) / K ** 0.5).to(torch.bfloat16) for n in (264, 8, 1000, 128)]
    big = torch.zeros(M, 2000, device="cuda", dtype=torch.bfloat16)
    outs = [torch.empty(M, 264, device="cuda", dtype=torch.bfloat16), big[:, 8:16],
            big[:, 16:1016], torch.empty(M, 128, device="cuda", dtype=torch.bfloat16)]
    res = skinny_matmul_group(a, bs, outs)
    torch.cuda.synchronize()
    for c, b in zip(res, bs):
        _assert_one_rounding(c, a, b)
    assert (big[:, :8] == 0).all() and (big[:, 1016:] == 0).all()
    H, F = 4096, 14336
    h = torch.randn(M, H, device="cuda", generator=g).to(torch.bfloat16)
    for shapes in ([(H, H), (H, 1024), (H, 1024)], [(H, F), (H, F)]):
        ws = [(torch.randn(*s, device="cuda", generator=g) / H ** 0.5).to(torch.bfloat16) for s in shapes]
        for c, w in zip(matmul_shared_input(h, ws), ws):
            _assert_one_rounding(c, h, w)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
def test_swiglu_matmul(M):
    """The SwiGLU input folded into the skinny kernels' loads equals
    matmul(F.silu(gate) * up, w) computed by torch ops then the same kernel
    (same rounding of the activation and the product), bit for bit, on the
    VALU kernel (at most 2 rows) and the MFMA kernel (from 3 rows);
    swiglu_matmul routes 1-2 rows to the fused launch and larger row counts
    to torch's SiLU and multiply ahead of the plain product, the same kernel
    on the same x, so every route agrees bit for bit."""
    import torch.nn.functional as F
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul, skinny_matmul_group, swiglu_matmul
    print(f"case gemv swiglu M={M}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(10 + M)
    F_, H = 14336, 4096
    gate = (torch.randn(M, F_, device="cuda", generator=g) * 3).to(torch.bfloat16)
    up = torch.randn(M, F_, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(F_, H, device="cuda", generator=g) / F_ ** 0.5).to(torch.bfloat16)
    fused = skinny_matmul_group(up, [w], gate=gate)[0]
    x = F.silu(gate) * up
    ref = skinny_matmul(x, w)  # the same kernel on the same staged x
    torch.cuda.synchronize()
    assert torch.equal(fused, ref)
    _assert_one_rounding(fused, x, w)
    routed = swiglu_matmul(gate, up, w)
    assert torch.equal(routed, fused)


@pytest.mark.parametrize("M", [1, 2, 5])
@pytest.mark.parametrize("with_residual", [True, False])
def test_rmsnorm_folded_into_skinny_matmul(M, with_residual):
    """add_rmsnorm_matmul_shared_input: at M <= 2 one launch forms the norm
    in the vector RMSNorm kernel's order and equals fused_add_rmsnorm (or
    rmsnorm) followed by the same grouped skinny GEMM bit for bit, h
    included; at M = 5 it falls back to those two calls."""
    from lightserve_amd.kernels.tiled_matmul import add_rmsnorm_matmul_shared_input, skinny_matmul_group
    print(f"case gemv rmsnorm M={M} residual={with_residual}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(20 + M)
    H = 4096
    x = torch.randn(M, H, device="cuda", generator=g).to(torch.bfloat16)
    r = torch.randn(M, H, device="cuda", generator=g).to(torch.bfloat16) if with_residual else None
    w_norm = (torch.rand(H, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    ws = [(torch.randn(H, n, device="cuda", generator=g) / H ** 0.5).to(torch.bfloat16) for n in (4096, 1024, 1024)]
    outs, h = add_rmsnorm_matmul_shared_input(x, r, w_norm, 1e-5, ws)
    if r is not None:
        normed, h_ref = fused_add_rmsnorm(x, r, w_norm, 1e-5)
    else:
        normed, h_ref = rmsnorm(x, w_norm, 1e-5), x
    refs = skinny_matmul_group(normed, ws)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    for c, ref, w in zip(outs, refs, ws):
        if M <= 2:
            assert torch.equal(c, ref)
        _assert_one_rounding(c, normed, w)
    # without writing h the products are the same
    outs2, _ = add_rmsnorm_matmul_shared_input(x, r, w_norm, 1e-5, ws, write_residual=False)
    for c, c2 in zip(outs, outs2):
        assert torch.equal(c, c2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [3, 8, 16, 32])
def test_skinny_matmul_mfma_rows(M, dtype):
    """3..32 rows with widths that are multiples of 128 run on the MFMA kernel
    (W tiles through LDS, transposed reads): within one rounding of the fp64
    product on the decode shapes, K-ranges that end inside a tile (K = 1000,
    2056), a single split (K = 192), grouped matrices, and repeat calls that
    agree bit for bit."""
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul, skinny_matmul_group
    print(f"case gemv mfma M={M} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(40 + M)
    for K, N in [(4096, 4096), (14336, 4096), (4096, 14336), (1000, 256), (2056, 384), (192, 128)]:
        a = torch.randn(M, K, device="cuda", generator=g).to(dtype)
        b = (torch.randn(K, N, device="cuda", generator=g) / K ** 0.5).to(dtype)
        c = skinny_matmul(a, b)
        c2 = skinny_matmul(a, b)
        torch.cuda.synchronize()
        _assert_one_rounding(c, a, b)
        assert torch.equal(c, c2), (K, N)
    a = torch.randn(M, 4096, device="cuda", generator=g).to(dtype)
    ws = [(torch.randn(4096, n, device="cuda", generator=g) / 64).to(dtype) for n in (4096, 1024, 1024)]
    for c, w in zip(skinny_matmul_group(a, ws), ws):
        _assert_one_rounding(c, a, w)


@pytest.mark.parametrize("M", [3, 8, 16, 32])
def test_gemv_abi_empty_k(M):
    """k = 0 through the C ABI at row counts the MFMA kernel takes (widths
    multiples of 128): y must come back zero, and no x row may be read (x here
    is a one-row, 16-byte allocation)."""
    print(f"case gemv abi k=0 M={M}", flush=True)
    N = 256
    x = torch.zeros(8, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(1, N, device="cuda", dtype=torch.bfloat16)
    y = torch.full((M, N), float("nan"), device="cuda", dtype=torch.bfloat16)
    args = _lib.GemvArgs(x=x.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), workspace=None, workspace_bytes=0,
                         x_stride=8, w_stride=N, y_stride=N, dtype=_lib.DTYPE_BF16, m=M, k=0, n=N)
    assert _lib.gemv_check(args)[0] == 0
    nbytes = _lib.gemv_workspace_size(args)
    ws = torch.zeros(max(nbytes, 16), device="cuda", dtype=torch.uint8)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.gemv(args, _lib.current_stream(x.device))
    torch.cuda.synchronize()
    assert (y == 0).all()
