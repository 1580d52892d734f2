"""CPU-only checks of the drop-in boundary: the reference's validation tests
(kernels/tests/test_flash_attention.py:80-122,
kernels/tests/test_flash_attention_backward.py:127-139) against the new entry
points, and the C ABI library loading, exporting every declared symbol, and
rejecting bad arguments on the host (no GPU call is made here)."""
import ctypes
import os
import re

import pytest
import torch

from lightserve_amd import _lib
from lightserve_amd.kernels.flash_attention import flash_attention_forward
from lightserve_amd.kernels.flash_attention_backward import flash_attention
from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "lightserve_fa.h")

ENTRY_POINTS = [flash_attention_forward, flash_attention]


@pytest.mark.parametrize("fn", ENTRY_POINTS)
def test_rejects_shape_mismatch(fn):
    q = torch.randn(1, 2, 16, 32)
    k = torch.randn(1, 2, 16, 32)
    v = torch.randn(1, 2, 8, 32)
    with pytest.raises(AssertionError):
        fn(q, k, v)


@pytest.mark.parametrize("fn", ENTRY_POINTS)
def test_rejects_dtype_mismatch(fn):
    q = torch.randn(1, 2, 16, 32, dtype=torch.float32)
    k = torch.randn(1, 2, 16, 32, dtype=torch.float16)
    v = torch.randn(1, 2, 16, 32, dtype=torch.float32)
    with pytest.raises(AssertionError):
        fn(q, k, v)


@pytest.mark.parametrize("fn", ENTRY_POINTS)
def test_rejects_wrong_ndim(fn):
    q = torch.randn(2, 16, 32)
    with pytest.raises(AssertionError):
        fn(q, q, q)


@pytest.mark.parametrize("fn", ENTRY_POINTS)
def test_rejects_cpu_tensor(fn):
    q = torch.randn(1, 2, 16, 32)
    with pytest.raises(AssertionError):
        fn(q, q.clone(), q.clone())


@pytest.mark.parametrize("fn", ENTRY_POINTS)
def test_rejects_head_dim_mismatch(fn):
    q = torch.randn(1, 2, 16, 32)
    v = torch.randn(1, 2, 16, 64)
    with pytest.raises(AssertionError):
        fn(q, q, v)


def test_varlen_validation():
    q = torch.randn(8, 4, 16)
    k = torch.randn(10, 2, 16)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(AssertionError):  # CPU tensors
        flash_attention_varlen_forward(q, k, k, cu, torch.tensor([0, 10], dtype=torch.int32), 8, 10)
    with pytest.raises(AssertionError):  # heads not a multiple
        flash_attention_varlen_forward(q, torch.randn(10, 3, 16), torch.randn(10, 3, 16), cu, cu, 8, 10)
    with pytest.raises(AssertionError):  # 4-D input
        flash_attention_varlen_forward(q[None], k, k, cu, cu, 8, 10)


def test_varlen_backward_validation_cpu():
    """The varlen backward and the differentiable varlen entry point validate
    before touching the library: host tensors, 4-D inputs and groupless head
    counts raise AssertionError in a GPU-less process."""
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen, flash_attention_varlen_backward
    q = torch.randn(8, 4, 16, dtype=torch.bfloat16)
    k = torch.randn(10, 2, 16, dtype=torch.bfloat16)
    lse = torch.zeros(4, 8)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    cu_k = torch.tensor([0, 10], dtype=torch.int32)
    with pytest.raises(AssertionError):  # host tensors
        flash_attention_varlen_backward(q, q, k, k, q, lse, cu, cu_k, 8, 10)
    with pytest.raises(AssertionError):  # 4-D input
        flash_attention_varlen_backward(q[None], q[None], k, k, q[None], lse, cu, cu_k, 8, 10)
    k3 = torch.randn(10, 3, 16, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):  # 4 query heads over 3 kv heads
        flash_attention_varlen_backward(q, q, k3, k3, q, lse, cu, cu_k, 8, 10)
    with pytest.raises(AssertionError):
        flash_attention_varlen(q.requires_grad_(), k, k, cu, cu_k, 8, 10)


def test_import_loads_no_native_code():
    """Importing the package must not need the library or a GPU (the
    reference's CI runs validation tests on CPU-only runners)."""
    import subprocess
    import sys
    code = ("import lightserve_amd.kernels, lightserve_amd._lib as L, sys; "
            "sys.exit(0 if L._lib is None else 1)")
    assert subprocess.run([sys.executable, "-c", code], cwd=os.path.dirname(HEADER) + "/..").returncode == 0


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(lsfa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol(built_library):
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    lib = ctypes.CDLL(built_library)
    for name in declared:
        assert hasattr(lib, name), name
    assert _lib.load().lsfa_abi_version() == _lib.ABI_VERSION


def test_library_exports_nothing_else(built_library):
    """The dynamic symbol table holds exactly the declared C ABI: no host
    helper, kernel stub or C++ symbol leaks out of the drop-in library (the
    compiler's __hip_cuid_* markers aside)."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("no nm")
    out = subprocess.run([nm, "-D", "--defined-only", built_library], capture_output=True, text=True,
                         check=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.strip()}
    names = {n for n in names if not n.startswith("__hip_cuid_")}
    assert names == set(_lib.EXPORTED_SYMBOLS), sorted(names ^ set(_lib.EXPORTED_SYMBOLS))


def test_struct_layout_matches_header(built_library):
    """ctypes mirrors must have the C struct sizes (checked with the
    host compiler against the header)."""
    import shutil
    import subprocess
    import tempfile
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    src = ('#include <stdio.h>\n#include <stddef.h>\n#include "lightserve_fa.h"\n'
           'int main(void){printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(lsfa_fwd_args),'
           ' sizeof(lsfa_bwd_args), offsetof(lsfa_fwd_args, sm_scale), offsetof(lsfa_bwd_args, sm_scale),'
           ' sizeof(lsfa_decode_args), offsetof(lsfa_decode_args, block_table_stride),'
           ' offsetof(lsfa_decode_args, sm_scale), sizeof(lsfa_rope_args), offsetof(lsfa_rope_args, table_stride),'
           ' offsetof(lsfa_rope_args, max_pos)); printf("%zu %zu %zu\\n", sizeof(lsfa_rmsnorm_args),'
           ' offsetof(lsfa_rmsnorm_args, dtype), offsetof(lsfa_rmsnorm_args, eps));'
           ' printf("%zu %zu %zu %zu\\n", sizeof(lsfa_prefill_paged_args),'
           ' offsetof(lsfa_prefill_paged_args, block_table_stride), offsetof(lsfa_prefill_paged_args, causal),'
           ' offsetof(lsfa_prefill_paged_args, sm_scale)); printf("%zu %zu %zu\\n", sizeof(lsfa_gemv_args),'
           ' offsetof(lsfa_gemv_args, dtype), offsetof(lsfa_gemv_args, n));'
           ' printf("%zu %zu %zu %zu\\n", sizeof(lsfa_gemv_group_args), offsetof(lsfa_gemv_group_args, y_stride),'
           ' offsetof(lsfa_gemv_group_args, n), offsetof(lsfa_gemv_group_args, count)); return 0;}\n')
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write(src)
        subprocess.run([cc, "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        sizes = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert sizes == [ctypes.sizeof(_lib.FwdArgs), ctypes.sizeof(_lib.BwdArgs),
                     _lib.FwdArgs.sm_scale.offset, _lib.BwdArgs.sm_scale.offset, ctypes.sizeof(_lib.DecodeArgs),
                     _lib.DecodeArgs.block_table_stride.offset, _lib.DecodeArgs.sm_scale.offset,
                     ctypes.sizeof(_lib.RopeArgs), _lib.RopeArgs.table_stride.offset, _lib.RopeArgs.max_pos.offset,
                     ctypes.sizeof(_lib.RmsNormArgs), _lib.RmsNormArgs.dtype.offset, _lib.RmsNormArgs.eps.offset,
                     ctypes.sizeof(_lib.PrefillPagedArgs), _lib.PrefillPagedArgs.block_table_stride.offset,
                     _lib.PrefillPagedArgs.causal.offset, _lib.PrefillPagedArgs.sm_scale.offset,
                     ctypes.sizeof(_lib.GemvArgs), _lib.GemvArgs.dtype.offset, _lib.GemvArgs.n.offset,
                     ctypes.sizeof(_lib.GemvGroupArgs), _lib.GemvGroupArgs.y_stride.offset,
                     _lib.GemvGroupArgs.n.offset, _lib.GemvGroupArgs.count.offset]


def _fwd_args(**kw):
    st = _lib._i64x4(8 * 4 * 64, 8 * 64, 64, 1)
    base = dict(q=16, k=32, v=48, o=64, lse=None, q_stride=st, k_stride=st, v_stride=st, o_stride=st,
                lse_stride=_lib._i64x3(32, 8, 1), cu_seqlens_q=None, cu_seqlens_k=None,
                dtype=_lib.DTYPE_BF16, batch=1, heads_q=4, heads_kv=4, seqlen_q=8, seqlen_k=8,
                head_dim=64, causal=1, sm_scale=0.125, reserved=0)
    base.update(kw)
    return _lib.FwdArgs(**base)


def test_abi_host_validation(built_library):
    """Host-only validation paths; fake (never dereferenced) pointers."""
    assert _lib.fwd_check(_fwd_args())[0] == 0
    rc, msg = _lib.fwd_check(_fwd_args(dtype=7))
    assert rc == -1 and "dtype" in msg
    rc, msg = _lib.fwd_check(_fwd_args(head_dim=256))
    assert rc == -2 and "head_dim" in msg
    rc, msg = _lib.fwd_check(_fwd_args(heads_q=6, heads_kv=4))
    assert rc == -1 and "multiple" in msg
    rc, msg = _lib.fwd_check(_fwd_args(q=None))
    assert rc == -1 and "non-NULL" in msg
    rc, msg = _lib.fwd_check(_fwd_args(q=18))
    assert rc == -2 and "aligned" in msg
    rc, msg = _lib.fwd_check(_fwd_args(q_stride=_lib._i64x4(2048, 512, 64, 2)))
    assert rc == -2 and "stride" in msg
    rc, msg = _lib.fwd_check(_fwd_args(cu_seqlens_q=16))
    assert rc == -1 and "cu_seqlens" in msg
    rc, msg = _lib.fwd_check(_fwd_args(sm_scale=float("nan")))
    assert rc == -1 and "sm_scale" in msg
    # fp32 accepts any stride and head dim up to 128
    assert _lib.fwd_check(_fwd_args(dtype=_lib.DTYPE_FP32, head_dim=12, q=18,
                                    q_stride=_lib._i64x4(7, 5, 3, 2)))[0] == 0
    # the launching entry point validates first and never reaches the GPU on bad input
    with pytest.raises(RuntimeError, match="LSFA_ERR_INVALID"):
        _lib.fwd(_fwd_args(batch=-1), 0)
    # empty problems are a successful no-op
    _lib.fwd(_fwd_args(seqlen_q=0, q=None, k=None, v=None, o=None), 0)


def test_abi_backward_validation(built_library):
    st = _lib._i64x4(2048, 512, 64, 1)
    args = _lib.BwdArgs(q=16, k=32, v=48, o=64, dout=80, lse=96, dq=112, dk=128, dv=144, workspace=4096,
                        workspace_bytes=1 << 20,
                        q_stride=st, k_stride=st, v_stride=st, o_stride=st, do_stride=st, dq_stride=st,
                        dk_stride=st, dv_stride=st, lse_stride=_lib._i64x3(32, 8, 1),
                        cu_seqlens_q=None, cu_seqlens_k=None, dtype=_lib.DTYPE_BF16, batch=1,
                        heads_q=4, heads_kv=4, seqlen_q=8, seqlen_k=8, head_dim=64, causal=1,
                        sm_scale=0.125, flags=0)
    assert _lib.bwd_check(args)[0] == 0
    # GQA (heads_kv dividing heads_q) on the bf16/fp16 default path; not with
    # the stored-dS path or in fp32; heads_kv must divide heads_q
    args.heads_kv = 2
    assert _lib.bwd_check(args)[0] == 0
    args.flags = _lib.BWD_STORED_DS
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "GQA" in msg
    args.flags, args.dtype = 0, _lib.DTYPE_FP32
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "GQA" in msg and "fp32" in msg
    args.dtype, args.heads_kv = _lib.DTYPE_BF16, 3
    rc, msg = _lib.bwd_check(args)
    assert rc == -1 and "multiple" in msg
    args.heads_kv = 4
    args.workspace = None
    rc, msg = _lib.bwd_check(args)
    assert rc == -1
    args.workspace = 4096
    # varlen (cu_seqlens) on the bf16/fp16 default path only; both or neither
    args.cu_seqlens_q = 16
    args.cu_seqlens_k = 32
    assert _lib.bwd_check(args)[0] == 0
    args.flags = _lib.BWD_STORED_DS
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "varlen" in msg
    args.flags, args.dtype = 0, _lib.DTYPE_FP32
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "varlen" in msg
    args.dtype, args.cu_seqlens_k = _lib.DTYPE_BF16, None
    rc, msg = _lib.bwd_check(args)
    assert rc == -1 and "cu_seqlens" in msg
    args.cu_seqlens_q = args.cu_seqlens_k = None
    # flags: at most one phase (LSFA_BWD_ONLY_DQ / ONLY_DKDV), with or without
    # LSFA_BWD_STORED_DS; the fp32 path takes no phase (STORED_DS is ignored)
    args.workspace_bytes = 1 << 40
    for f in (_lib.BWD_ONLY_DQ, _lib.BWD_ONLY_DKDV, _lib.BWD_STORED_DS):
        for r in (0, _lib.BWD_STORED_DS):
            args.flags = f | r
            assert _lib.bwd_check(args)[0] == 0, args.flags
    for f in (3, 8, 3 | _lib.BWD_STORED_DS, -1):
        args.flags = f
        rc, msg = _lib.bwd_check(args)
        assert rc == -1 and "flags" in msg, f
    args.flags, args.dtype = _lib.BWD_ONLY_DQ, _lib.DTYPE_FP32
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "fp32" in msg
    args.flags = _lib.BWD_STORED_DS
    assert _lib.bwd_check(args)[0] == 0
    args.flags, args.dtype, args.workspace_bytes = 0, _lib.DTYPE_BF16, 0


def test_abi_backward_noalloc_limit(built_library):
    """lsfa_bwd_noalloc rejects, before touching any GPU, a problem whose
    workspace exceeds the library's scratch array (LSFA_BWD_SCRATCH_BYTES), and
    validates its arguments as lsfa_bwd does."""
    st = _lib._i64x4(2048, 512, 64, 1)
    args = _lib.BwdArgs(q=16, k=32, v=48, o=64, dout=80, lse=96, dq=112, dk=128, dv=144, workspace=None,
                        workspace_bytes=0,
                        q_stride=st, k_stride=st, v_stride=st, o_stride=st, do_stride=st, dq_stride=st,
                        dk_stride=st, dv_stride=st, lse_stride=_lib._i64x3(32, 8, 1),
                        cu_seqlens_q=None, cu_seqlens_k=None, dtype=_lib.DTYPE_BF16, batch=4,
                        heads_q=32, heads_kv=32, seqlen_q=16385, seqlen_k=16385, head_dim=64, causal=1,
                        sm_scale=0.125, flags=0)
    assert _lib.bwd_workspace_size(args) > _lib.BWD_SCRATCH_BYTES
    rc = _lib.load().lsfa_bwd_noalloc(ctypes.byref(args), None)
    assert rc == -2 and "scratch" in _lib.load().lsfa_last_error().decode()
    args.heads_kv, args.dtype = 16, _lib.DTYPE_FP32  # the fp32 backward has no GQA: rejected like lsfa_bwd
    args.seqlen_q = args.seqlen_k = 128
    rc = _lib.load().lsfa_bwd_noalloc(ctypes.byref(args), None)
    assert rc == -2 and "GQA" in _lib.load().lsfa_last_error().decode()


def test_abi_backward_workspace(built_library):
    """Workspace size. Default path (and fp32, and LSFA_BWD_STORED_DS at
    head_dim <= 64): (L*log2e, delta) fp32 pairs for every (b, h, query) with
    queries padded to 128, 256-byte aligned. Stored-dS path
    (LSFA_BWD_STORED_DS, bf16/fp16, head_dim above 64): those pairs, then dS
    of a chunk of heads (seqlen_k rounded up to 32 by seqlen_q rounded up to
    256 elements per head, as many heads as fit in 4 GiB, at least one). Too
    small or misaligned workspaces are rejected before any launch; stored-dS
    problems that run in several chunks take no LSFA_BWD_ONLY_* flag."""
    st = _lib._i64x4(2048, 512, 64, 1)
    args = _lib.BwdArgs(q=16, k=32, v=48, o=64, dout=80, lse=96, dq=112, dk=128, dv=144, workspace=4096,
                        workspace_bytes=0,
                        q_stride=st, k_stride=st, v_stride=st, o_stride=st, do_stride=st, dq_stride=st,
                        dk_stride=st, dv_stride=st, lse_stride=_lib._i64x3(32, 8, 1),
                        cu_seqlens_q=None, cu_seqlens_k=None, dtype=_lib.DTYPE_BF16, batch=1,
                        heads_q=4, heads_kv=4, seqlen_q=8, seqlen_k=8, head_dim=64, causal=1,
                        sm_scale=0.125, flags=0)
    rows = 1 * 4 * 128
    expected = rows * 8
    assert _lib.bwd_workspace_size(args) == expected
    args.seqlen_q = 128
    assert _lib.bwd_workspace_size(args) == expected
    args.seqlen_q = 129  # two query tiles
    assert _lib.bwd_workspace_size(args) == 2 * expected
    args.seqlen_q = 8
    args.workspace_bytes = expected - 1
    rc, msg = _lib.bwd_check(args)
    assert rc == -1 and "workspace_bytes" in msg
    args.workspace_bytes = expected
    assert _lib.bwd_check(args)[0] == 0
    args.workspace = 4096 + 128
    rc, msg = _lib.bwd_check(args)
    assert rc == -1 and "aligned" in msg
    args.workspace = 4096
    # fp32 needs only the (L, delta) pairs, whatever the flags
    args.dtype = _lib.DTYPE_FP32
    assert _lib.bwd_workspace_size(args) == rows * 8
    args.flags = _lib.BWD_STORED_DS
    assert _lib.bwd_workspace_size(args) == rows * 8

    # head_dim 64: the stored-dS flag does not apply
    args.dtype = _lib.DTYPE_BF16
    assert _lib.bwd_workspace_size(args) == rows * 8
    # stored-dS path
    args.head_dim = 128
    args.flags = 0
    assert _lib.bwd_workspace_size(args) == rows * 8
    args.flags = _lib.BWD_STORED_DS
    for nq, nk in ((8, 8), (256, 8), (257, 100), (1000, 3)):
        args.seqlen_q, args.seqlen_k = nq, nk
        ld = 4 * ((nq + 127) // 128 * 128) * 8
        ds = 4 * ((nk + 31) // 32 * 32) * ((nq + 255) // 256 * 256) * 2
        want = ld + (ds + 255) // 256 * 256
        assert _lib.bwd_workspace_size(args) == want, (nq, nk)
        args.workspace_bytes = want - 1
        assert _lib.bwd_check(args)[0] == -1
        args.workspace_bytes = want
        assert _lib.bwd_check(args)[0] == 0
    args.seqlen_k = 0  # no keys: no dS
    assert _lib.bwd_workspace_size(args) == 4 * 1024 * 8
    # several chunks: 4 x 32 heads of 16416 x 16640 elements (546 MB) run 7 heads at a time
    args.batch, args.heads_q, args.heads_kv, args.seqlen_q, args.seqlen_k = 4, 32, 32, 16385, 16385
    head = 16416 * 16640 * 2
    ld = 128 * 16512 * 8
    assert _lib.bwd_workspace_size(args) == ld + (7 * head + 255) // 256 * 256
    args.workspace_bytes = 1 << 40
    assert _lib.bwd_check(args)[0] == 0
    args.flags = _lib.BWD_ONLY_DQ | _lib.BWD_STORED_DS
    rc, msg = _lib.bwd_check(args)
    assert rc == -2 and "chunk" in msg
    args.flags = _lib.BWD_ONLY_DQ
    assert _lib.bwd_check(args)[0] == 0


def _rope_args(**kw):
    st = _lib._i64x4(4 * 16 * 64, 64, 4 * 64, 1)  # [B, N, H, D] storage viewed as (b, h, n, d)
    base = dict(q=4096, k=8192, cos=12288, sin=16384, positions=None, cu_seqlens=None, q_stride=st,
                k_stride=st, table_stride=64, dtype=_lib.DTYPE_BF16, batch=2, seqlen=16, heads_q=4,
                heads_kv=4, head_dim=64, max_pos=128, reserved=0)
    base.update(kw)
    return _lib.RopeArgs(**base)


def test_abi_rope_validation(built_library):
    """Host-only validation of lsfa_rope (fake, never dereferenced pointers)."""
    assert _lib.rope_check(_rope_args())[0] == 0
    rc, msg = _lib.rope_check(_rope_args(dtype=9))
    assert rc == -1 and "dtype" in msg
    rc, msg = _lib.rope_check(_rope_args(head_dim=24))  # half of 24 is not a multiple of 8
    assert rc == -2 and "head_dim" in msg
    assert _lib.rope_check(_rope_args(dtype=_lib.DTYPE_FP32, head_dim=24, table_stride=24))[0] == 0
    rc, msg = _lib.rope_check(_rope_args(k=None))
    assert rc == -1 and "k is NULL" in msg
    assert _lib.rope_check(_rope_args(k=None, heads_kv=0))[0] == 0  # q only
    rc, msg = _lib.rope_check(_rope_args(cos=None))
    assert rc == -1 and "cos" in msg
    rc, msg = _lib.rope_check(_rope_args(table_stride=32))
    assert rc == -2 and "table_stride" in msg
    rc, msg = _lib.rope_check(_rope_args(q=4100))
    assert rc == -2 and "aligned" in msg
    rc, msg = _lib.rope_check(_rope_args(q_stride=_lib._i64x4(4096, 64, 256, 2)))
    assert rc == -2 and "stride" in msg
    rc, msg = _lib.rope_check(_rope_args(max_pos=0))
    assert rc == -1 and "max_pos" in msg
    # K/V cache append: v, both caches and slots together, aligned strides
    cache = dict(v=1 << 20, k_cache=1 << 21, v_cache=1 << 22, slots=1 << 23, v_stride=_lib._i64x4(4096, 64, 256, 1),
                 num_slots=64)
    a = _rope_args(**cache)
    a.cache_stride[0], a.cache_stride[1] = 4 * 64, 64
    assert _lib.rope_check(a)[0] == 0
    a = _rope_args(**{**cache, "slots": None})
    a.cache_stride[0], a.cache_stride[1] = 4 * 64, 64
    rc, msg = _lib.rope_check(a)
    assert rc == -1 and "slots" in msg
    a = _rope_args(**cache)
    a.cache_stride[0], a.cache_stride[1] = 64, 64  # a slot must hold every head
    rc, msg = _lib.rope_check(a)
    assert rc == -2 and "caches" in msg
    # empty problems are a successful no-op; bad input never reaches the GPU
    _lib.rope(_rope_args(seqlen=0, q=None, k=None), 0)
    with pytest.raises(RuntimeError, match="LSFA_ERR_INVALID"):
        _lib.rope(_rope_args(batch=-1), 0)


def _decode_args(**kw):
    base = dict(q=4096, k_cache=8192, v_cache=12288, o=16384, lse=None, block_tables=20480, seq_lens=24576,
                workspace=None, workspace_bytes=0, q_stride=_lib._i64x3(1024, 128, 1),
                k_stride=_lib._i64x4(16 * 2 * 128, 256, 128, 1), v_stride=_lib._i64x4(16 * 2 * 128, 256, 128, 1),
                o_stride=_lib._i64x3(1024, 128, 1), lse_stride=_lib._i64x2(8, 1), block_table_stride=8,
                dtype=_lib.DTYPE_BF16, batch=2, heads_q=8, heads_kv=2, head_dim=128, block_size=16, num_blocks=16,
                max_blocks_per_seq=8, max_seq_len=128, sm_scale=0.088)
    base.update(kw)
    return _lib.DecodeArgs(**base)


def test_abi_decode_validation(built_library):
    """Host-only validation of lsfa_decode (fake, never dereferenced pointers):
    group sizes up to 32 with blocks of 16 or more (the MFMA kernel), only
    1/2/4/8 with smaller blocks (the lane-group kernel)."""
    assert _lib.decode_check(_decode_args())[0] == 0
    assert _lib.decode_check(_decode_args(heads_q=6))[0] == 0  # group of 3, 16-token blocks
    assert _lib.decode_check(_decode_args(heads_q=64))[0] == 0  # group of 32
    assert _lib.decode_check(_decode_args(block_size=4, k_stride=_lib._i64x4(4 * 256, 256, 128, 1),
                                          v_stride=_lib._i64x4(4 * 256, 256, 128, 1)))[0] == 0
    rc, msg = _lib.decode_check(_decode_args(heads_q=66))  # group of 33
    assert rc == -2 and "heads_q / heads_kv" in msg
    rc, msg = _lib.decode_check(_decode_args(heads_q=6, block_size=8))  # group of 3, small blocks
    assert rc == -2 and "heads_q / heads_kv" in msg
    rc, msg = _lib.decode_check(_decode_args(block_size=24))
    assert rc == -2 and "power of two" in msg
    rc, msg = _lib.decode_check(_decode_args(dtype=_lib.DTYPE_FP32))
    assert rc == -2
    rc, msg = _lib.decode_check(_decode_args(heads_q=7))
    assert rc == -1 and "multiple" in msg
    rc, msg = _lib.decode_check(_decode_args(seq_lens=None))
    assert rc == -1 and "non-NULL" in msg


def _prefill_args(**kw):
    base = dict(q=4096, k_cache=8192, v_cache=12288, o=16384, lse=None, cu_seqlens_q=20480, seq_lens_k=24576,
                block_tables=28672, q_stride=_lib._i64x2(1024, 128), k_stride=_lib._i64x3(16 * 2 * 128, 256, 128),
                v_stride=_lib._i64x3(16 * 2 * 128, 256, 128), o_stride=_lib._i64x2(1024, 128),
                lse_stride=_lib._i64x2(64, 1), block_table_stride=8, dtype=_lib.DTYPE_BF16, batch=2, heads_q=8,
                heads_kv=2, head_dim=128, block_size=16, num_blocks=16, max_blocks_per_seq=8, max_seqlen_q=32,
                causal=1, sm_scale=0.088, reserved=0)
    base.update(kw)
    return _lib.PrefillPagedArgs(**base)


def test_abi_prefill_paged_validation(built_library):
    """Host-only validation of lsfa_prefill_paged (fake, never dereferenced pointers)."""
    assert _lib.prefill_paged_check(_prefill_args())[0] == 0
    assert _lib.prefill_paged_check(_prefill_args(heads_q=6))[0] == 0  # group of 3 is fine here
    assert _lib.prefill_paged_check(_prefill_args(batch=0, q=None))[0] == 0  # empty: nothing checked further
    rc, msg = _lib.prefill_paged_check(_prefill_args(block_size=8))
    assert rc == -2 and "block_size" in msg
    rc, msg = _lib.prefill_paged_check(_prefill_args(block_size=48))
    assert rc == -2
    rc, msg = _lib.prefill_paged_check(_prefill_args(dtype=_lib.DTYPE_FP32))
    assert rc == -2
    rc, msg = _lib.prefill_paged_check(_prefill_args(heads_q=5))
    assert rc == -1 and "multiple" in msg
    rc, msg = _lib.prefill_paged_check(_prefill_args(head_dim=100))
    assert rc == -2
    rc, msg = _lib.prefill_paged_check(_prefill_args(block_tables=None))
    assert rc == -1
    rc, msg = _lib.prefill_paged_check(_prefill_args(block_table_stride=4))
    assert rc == -1 and "block_table_stride" in msg
    rc, msg = _lib.prefill_paged_check(_prefill_args(q=4100))
    assert rc == -2 and "aligned" in msg
    rc, msg = _lib.prefill_paged_check(_prefill_args(sm_scale=float("inf")))
    assert rc == -1
    _lib.prefill_paged(_prefill_args(batch=0), 0)  # empty: no-op, no GPU touched
    with pytest.raises(RuntimeError, match="block_size"):
        _lib.prefill_paged(_prefill_args(block_size=4), 0)


def _norm_args(**kw):
    base = dict(x=4096, residual=8192, weight=12288, out=16384, residual_out=20480, x_stride=4096,
                residual_stride=4096, out_stride=4096, residual_out_stride=4096, dtype=_lib.DTYPE_BF16,
                rows=8, cols=4096, eps=1e-6)
    base.update(kw)
    return _lib.RmsNormArgs(**base)


def test_abi_rmsnorm_validation(built_library):
    """Host-only validation of lsfa_rmsnorm (fake, never dereferenced pointers)."""
    assert _lib.rmsnorm_check(_norm_args())[0] == 0
    assert _lib.rmsnorm_check(_norm_args(residual=None, residual_out=None))[0] == 0  # plain RMSNorm
    assert _lib.rmsnorm_check(_norm_args(cols=17, x=4098))[0] == 0  # odd widths/alignment: scalar path
    rc, msg = _lib.rmsnorm_check(_norm_args(dtype=5))
    assert rc == -1 and "dtype" in msg
    rc, msg = _lib.rmsnorm_check(_norm_args(x=None))
    assert rc == -1 and "non-NULL" in msg
    rc, msg = _lib.rmsnorm_check(_norm_args(out_stride=100))
    assert rc == -1 and "stride" in msg
    rc, msg = _lib.rmsnorm_check(_norm_args(eps=float("nan")))
    assert rc == -1 and "eps" in msg
    _lib.rmsnorm(_norm_args(rows=0, x=None, out=None), 0)  # empty: no-op
    with pytest.raises(RuntimeError, match="LSFA_ERR_INVALID"):
        _lib.rmsnorm(_norm_args(rows=-1), 0)


def _gemv_args(**kw):
    base = dict(x=4096, w=8192, y=12288, workspace=1 << 20, workspace_bytes=1 << 30, x_stride=4096,
                w_stride=4096, y_stride=4096, dtype=_lib.DTYPE_BF16, m=4, k=4096, n=4096)
    base.update(kw)
    return _lib.GemvArgs(**base)


def test_abi_gemv_validation(built_library):
    """Host-only validation and workspace sizing of lsfa_gemv (fake pointers)."""
    assert _lib.gemv_check(_gemv_args())[0] == 0
    for m in range(1, 9):
        assert _lib.gemv_check(_gemv_args(m=m))[0] == 0
    for m in (9, 16, 32):  # the MFMA kernel: widths multiples of 128, no fused norm
        assert _lib.gemv_check(_gemv_args(m=m))[0] == 0
    rc, msg = _lib.gemv_check(_gemv_args(m=33))
    assert rc == -2 and "8 rows" in msg
    rc, msg = _lib.gemv_check(_gemv_args(m=9, n=4104, w_stride=4104))  # not a multiple of 128
    assert rc == -2 and "8 rows" in msg
    # MFMA workspace: K-ranges of 256 rows -> 16 splits at K = 4096
    assert _lib.gemv_workspace_size(_gemv_args(m=16)) == 262144 + 16 * 16 * 4096 * 4
    rc, msg = _lib.gemv_check(_gemv_args(n=4092, w_stride=4096))
    assert rc == -2 and "n % 8" in msg
    rc, msg = _lib.gemv_check(_gemv_args(w=8194))
    assert rc == -2 and "aligned" in msg
    rc, msg = _lib.gemv_check(_gemv_args(w_stride=4100))
    assert rc == -2
    rc, msg = _lib.gemv_check(_gemv_args(dtype=_lib.DTYPE_FP32))
    assert rc == -2 and "bf16" in msg
    rc, msg = _lib.gemv_check(_gemv_args(x_stride=100))
    assert rc == -1 and "x_stride" in msg
    rc, msg = _lib.gemv_check(_gemv_args(workspace=1 << 20 | 64))
    assert rc == -1 and "aligned" in msg
    need = _lib.gemv_workspace_size(_gemv_args())
    assert need % 256 == 0 and need >= 4 * 4096 * 4  # at least one fp32 partial row block per row
    rc, msg = _lib.gemv_check(_gemv_args(workspace_bytes=need - 256))
    assert rc == -1 and "workspace_bytes" in msg
    assert _lib.gemv_check(_gemv_args(workspace_bytes=need))[0] == 0
    # the split keeps K-ranges within 64..2048 rows and about 1024 workgroups;
    # layout: a fixed 256 KB of counters, then [splits][m][n] fp32
    for k, n in [(4096, 4096), (14336, 4096), (4096, 128256), (100000, 1024)]:
        col_blocks = (n + 255) // 256
        splits = (_lib.gemv_workspace_size(_gemv_args(m=1, k=k, n=n)) - 262144) // 4 // n
        assert 2 <= splits <= max(-(-1024 // col_blocks), (k + 2047) // 2048), (k, n, splits)
    assert _lib.gemv_workspace_size(_gemv_args(m=1, k=64, n=64)) == 0  # one split: no workspace
    assert _lib.gemv_check(_gemv_args(m=1, k=64, n=64, workspace=None, workspace_bytes=0))[0] == 0
    rc, msg = _lib.gemv_check(_gemv_args(n=1048576 + 8, w_stride=1048576 + 8))
    assert rc == -2 and "columns" in msg
    _lib.gemv(_gemv_args(m=0, x=None, y=None), 0)  # empty: no-op, no GPU touched
    with pytest.raises(RuntimeError, match="8 rows"):
        _lib.gemv(_gemv_args(m=33), 0)


def _group_args(ns, **kw):
    a = _lib.GemvGroupArgs(x=4096, workspace=1 << 20, workspace_bytes=1 << 30, x_stride=4096,
                           dtype=_lib.DTYPE_BF16, m=2, k=4096, count=len(ns))
    for i, n in enumerate(ns):
        a.w[i], a.y[i] = (1 << 24) * (i + 1), (1 << 28) + (1 << 20) * i
        a.w_stride[i], a.y_stride[i], a.n[i] = n, n, n
    for key, value in kw.items():
        setattr(a, key, value)
    return a


def test_gemv_constants_match_header():
    import re
    text = open(HEADER).read()
    assert int(re.search(r"#define LSFA_GEMV_COUNTER_BYTES (\d+)", text).group(1)) == _lib.GEMV_COUNTER_BYTES
    assert int(re.search(r"#define LSFA_GEMV_MAX_GROUP (\d+)", text).group(1)) == _lib.GEMV_MAX_GROUP


def test_abi_gemv_group_validation(built_library):
    """The grouped skinny GEMM: validation per matrix, workspace sized for
    the concatenated columns (the same as one matrix of that width)."""
    ns = [4096, 1024, 1024]
    assert _lib.gemv_group_check(_group_args(ns))[0] == 0
    assert _lib.gemv_group_workspace_size(_group_args(ns)) == _lib.gemv_workspace_size(
        _gemv_args(m=2, k=4096, n=sum(ns)))
    rc, msg = _lib.gemv_group_check(_group_args(ns, x_gate=8192, x_gate_stride=100))
    assert rc == -1 and "x_gate_stride" in msg
    assert _lib.gemv_group_check(_group_args(ns, x_gate=8192, x_gate_stride=4096))[0] == 0
    rc, msg = _lib.gemv_group_check(_group_args(ns, count=5))
    assert rc == -1 and "count" in msg
    rc, msg = _lib.gemv_group_check(_group_args(ns, count=0))
    assert rc == -1 and "count" in msg
    bad = _group_args(ns)
    bad.n[1] = 1020
    assert _lib.gemv_group_check(bad)[0] == -2
    bad = _group_args(ns)
    bad.w[2] = (1 << 24) + 8
    rc, msg = _lib.gemv_group_check(bad)
    assert rc == -2 and "aligned" in msg
    bad = _group_args(ns)
    bad.y[1] = None
    rc, msg = _lib.gemv_group_check(bad)
    assert rc == -1 and "non-NULL" in msg
    bad = _group_args(ns)
    bad.y_stride[2] = 100
    rc, msg = _lib.gemv_group_check(bad)
    assert rc == -1 and "y_stride" in msg
    # RMSNorm folded in: excludes x_gate; h must not overlap x or residual
    norm = dict(norm_weight=1 << 23, residual=1 << 22, residual_stride=4096, residual_out=1 << 21,
                residual_out_stride=4096, eps=1e-5)
    assert _lib.gemv_group_check(_group_args(ns, **norm))[0] == 0
    rc, msg = _lib.gemv_group_check(_group_args(ns, **{**norm, "x_gate": 8192, "x_gate_stride": 4096}))
    assert rc == -1 and "exclude" in msg
    rc, msg = _lib.gemv_group_check(_group_args(ns, **{**norm, "residual_out": 4096 + 64}))
    assert rc == -1 and "overlaps x" in msg
    rc, msg = _lib.gemv_group_check(_group_args(ns, **{**norm, "residual_out": 1 << 22}))
    assert rc == -1 and "overlaps residual" in msg
    rc, msg = _lib.gemv_group_check(_group_args(ns, **{**norm, "eps": float("nan")}))
    assert rc == -1 and "eps" in msg
    rc, msg = _lib.gemv_group_check(_group_args(ns, **{**norm, "k": 4092}))
    assert rc != 0
    _lib.gemv_group(_group_args(ns, m=0, x=None), 0)  # empty: no-op


def test_abi_greedy_validation(built_library):
    base = dict(logits=4096, tokens=8192, seq_lens=None, logits_stride=128256, dtype=_lib.DTYPE_BF16, rows=4,
                cols=128256)
    assert _lib.greedy_check(_lib.GreedyArgs(**base))[0] == 0
    for kw, code, word in [(dict(cols=0), -1, "empty"), (dict(logits_stride=100), -1, "logits_stride"),
                           (dict(dtype=9), -1, "dtype"), (dict(tokens=None), -1, "non-NULL"),
                           (dict(rows=70000), -2, "rows")]:
        rc, msg = _lib.greedy_check(_lib.GreedyArgs(**{**base, **kw}))
        assert rc == code and word in msg, (kw, rc, msg)
    _lib.greedy(_lib.GreedyArgs(**{**base, "rows": 0, "logits": None}), 0)  # empty: no-op


def test_skinny_matmul_argument_checks_cpu():
    """Shape checks of the skinny GEMM's Python entry points run before any
    library call (CPU tensors reach the assertions first)."""
    from lightserve_amd.kernels.tiled_matmul import add_rmsnorm_matmul_shared_input, skinny_matmul, skinny_matmul_group
    a = torch.randn(2, 16).to(torch.bfloat16)
    b = torch.randn(16, 8).to(torch.bfloat16)
    with pytest.raises(AssertionError):
        skinny_matmul(a, b)  # CPU tensors
    with pytest.raises(AssertionError):
        skinny_matmul_group(a, [b])
    with pytest.raises(AssertionError):
        add_rmsnorm_matmul_shared_input(a, None, torch.randn(15).to(torch.bfloat16), 1e-6, [b])


def test_rmsnorm_and_matmul_validation_cpu():
    """The reference's argument checks, in its order, raise AssertionError on
    CPU tensors before any library call (kernels/tests/test_fused_rmsnorm_residual.py,
    kernels/tests/test_tiled_matmul.py)."""
    from lightserve_amd.kernels.fused_rmsnorm_residual import fused_add_rmsnorm
    from lightserve_amd.kernels.tiled_matmul import matmul
    x = torch.randn(4, 8)
    with pytest.raises(AssertionError):
        fused_add_rmsnorm(x, torch.randn(4, 9), torch.randn(8))
    with pytest.raises(AssertionError):
        fused_add_rmsnorm(x, x, torch.randn(9))
    with pytest.raises(AssertionError):  # CPU tensors
        fused_add_rmsnorm(x, x, torch.randn(8))
    with pytest.raises(AssertionError):
        matmul(torch.randn(2, 3), torch.randn(4, 5))
    with pytest.raises(AssertionError):  # CPU tensors
        matmul(torch.randn(2, 3), torch.randn(3, 5))


def _integration_stub():
    """The reference-side ctypes stub of INTEGRATION.md section 2, as text."""
    import os
    import re
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")
    blocks = re.findall(r"```python\n(.*?)```", open(path).read(), flags=re.S)
    stub = [b for b in blocks if b.startswith("# kernels/_lsfa.py")]
    assert len(stub) == 1, "INTEGRATION.md must hold one ctypes stub starting '# kernels/_lsfa.py'"
    return stub[0]


def test_integration_stub_binds_this_library(built_library):
    """The documented stub runs against the built library: its ABI assertion
    holds, its FwdArgs has the header's layout (field by field against the
    package's mirror), and an argument block it builds passes lsfa_fwd_check
    (host-only validation, no GPU), while a bad head dim is refused."""
    code = _integration_stub().replace("/path/to/lightserve_amd/liblsfa_gfx950.so", built_library)
    ns = {}
    exec(compile(code, "INTEGRATION.md stub", "exec"), ns)  # runs its `assert lsfa_abi_version() == ...`
    Stub = ns["FwdArgs"]
    assert ctypes.sizeof(Stub) == ctypes.sizeof(_lib.FwdArgs)
    for (name, _), (mname, _) in zip(Stub._fields_, _lib.FwdArgs._fields_):
        assert name == mname and getattr(Stub, name).offset == getattr(_lib.FwdArgs, mname).offset, name
    lib = ns["_lib"]
    lib.lsfa_fwd_check.argtypes = [ctypes.POINTER(Stub)]
    lib.lsfa_fwd_check.restype = ctypes.c_int
    B, H, N, D = 2, 4, 64, 128
    st = (H * N * D, N * D, D, 1)
    ptr = 1 << 20  # aligned placeholder: the check never dereferences it
    a = Stub(q=ptr, k=ptr, v=ptr, o=ptr, lse=None, q_stride=ns["_i64x4"](*st), k_stride=ns["_i64x4"](*st),
             v_stride=ns["_i64x4"](*st), o_stride=ns["_i64x4"](*st), lse_stride=ns["_i64x3"](0, 0, 0),
             cu_seqlens_q=None, cu_seqlens_k=None, dtype=ns["_DT"][torch.bfloat16], batch=B, heads_q=H,
             heads_kv=H, seqlen_q=N, seqlen_k=N, head_dim=D, causal=1, sm_scale=D ** -0.5, reserved=0)
    assert lib.lsfa_fwd_check(ctypes.byref(a)) == 0, lib.lsfa_last_error()
    a.head_dim = 12
    assert lib.lsfa_fwd_check(ctypes.byref(a)) != 0
