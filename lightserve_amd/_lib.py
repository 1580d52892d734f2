"""ctypes binding of liblsfa_gfx950.so (declared in include/lightserve_fa.h).

The library is loaded lazily, once, under a lock: importing the package needs
neither the library nor a GPU, so argument validation (AssertionError, as in
the reference) runs in CPU-only processes. Calls that reach the library on a
machine where it is missing raise RuntimeError; there is no fallback path.
"""
import ctypes
import os
import threading

import torch

_LIB_NAME = "liblsfa_gfx950.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)
ABI_VERSION = 9
BWD_SCRATCH_BYTES = 16777216  # LSFA_BWD_SCRATCH_BYTES: lsfa_bwd_noalloc's workspace limit
BWD_ONLY_DQ, BWD_ONLY_DKDV = 1, 2  # lsfa_bwd_args.flags: run one backward phase (timing)
BWD_STORED_DS = 4  # lsfa_bwd_args.flags: dk/dv kernel stores dS, dq is a GEMM over it (head_dim > 64)

DTYPE_FP32, DTYPE_FP16, DTYPE_BF16 = 0, 1, 2
TORCH_TO_LSFA = {torch.float32: DTYPE_FP32, torch.float16: DTYPE_FP16, torch.bfloat16: DTYPE_BF16}

STATUS = {0: "LSFA_OK", -1: "LSFA_ERR_INVALID", -2: "LSFA_ERR_UNSUPPORTED", -3: "LSFA_ERR_LAUNCH"}

EXPORTED_SYMBOLS = ("lsfa_abi_version", "lsfa_last_error", "lsfa_fwd_check", "lsfa_fwd",
                    "lsfa_bwd_check", "lsfa_bwd_workspace_size", "lsfa_bwd", "lsfa_bwd_noalloc",
                    "lsfa_decode_check", "lsfa_decode_workspace_size", "lsfa_decode",
                    "lsfa_rope_check", "lsfa_rope", "lsfa_rmsnorm_check", "lsfa_rmsnorm",
                    "lsfa_prefill_paged_check", "lsfa_prefill_paged",
                    "lsfa_gemv_check", "lsfa_gemv_workspace_size", "lsfa_gemv",
                    "lsfa_gemv_group_check", "lsfa_gemv_group_workspace_size", "lsfa_gemv_group",
                    "lsfa_greedy_check", "lsfa_greedy")

_i64x4 = ctypes.c_int64 * 4
_i64x3 = ctypes.c_int64 * 3


class FwdArgs(ctypes.Structure):
    """Mirror of lsfa_fwd_args."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("q_stride", _i64x4), ("k_stride", _i64x4), ("v_stride", _i64x4), ("o_stride", _i64x4),
        ("lse_stride", _i64x3),
        ("cu_seqlens_q", ctypes.c_void_p), ("cu_seqlens_k", ctypes.c_void_p),
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32), ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("causal", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class BwdArgs(ctypes.Structure):
    """Mirror of lsfa_bwd_args."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("dout", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64),
        ("q_stride", _i64x4), ("k_stride", _i64x4), ("v_stride", _i64x4), ("o_stride", _i64x4),
        ("do_stride", _i64x4), ("dq_stride", _i64x4), ("dk_stride", _i64x4), ("dv_stride", _i64x4),
        ("lse_stride", _i64x3),
        ("cu_seqlens_q", ctypes.c_void_p), ("cu_seqlens_k", ctypes.c_void_p),
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32), ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("causal", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("flags", ctypes.c_int32),
    ]


_i64x2 = ctypes.c_int64 * 2


class DecodeArgs(ctypes.Structure):
    """Mirror of lsfa_decode_args."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p), ("seq_lens", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64),
        ("q_stride", _i64x3), ("k_stride", _i64x4), ("v_stride", _i64x4), ("o_stride", _i64x3),
        ("lse_stride", _i64x2), ("block_table_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32), ("max_blocks_per_seq", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32), ("sm_scale", ctypes.c_float),
    ]


class PrefillPagedArgs(ctypes.Structure):
    """Mirror of lsfa_prefill_paged_args."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("cu_seqlens_q", ctypes.c_void_p), ("seq_lens_k", ctypes.c_void_p), ("block_tables", ctypes.c_void_p),
        ("q_stride", _i64x2), ("k_stride", _i64x3), ("v_stride", _i64x3), ("o_stride", _i64x2),
        ("lse_stride", _i64x2), ("block_table_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32), ("max_blocks_per_seq", ctypes.c_int32),
        ("max_seqlen_q", ctypes.c_int32), ("causal", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class GemvArgs(ctypes.Structure):
    """Mirror of lsfa_gemv_args."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("y", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64),
        ("x_stride", ctypes.c_int64), ("w_stride", ctypes.c_int64), ("y_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("m", ctypes.c_int32), ("k", ctypes.c_int32), ("n", ctypes.c_int32),
    ]


GEMV_MAX_GROUP = 4
GEMV_COUNTER_BYTES = 262144  # LSFA_GEMV_COUNTER_BYTES


class GemvGroupArgs(ctypes.Structure):
    """Mirror of lsfa_gemv_group_args."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64),
        ("x_stride", ctypes.c_int64), ("x_gate", ctypes.c_void_p), ("x_gate_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p * GEMV_MAX_GROUP), ("y", ctypes.c_void_p * GEMV_MAX_GROUP),
        ("w_stride", ctypes.c_int64 * GEMV_MAX_GROUP), ("y_stride", ctypes.c_int64 * GEMV_MAX_GROUP),
        ("n", ctypes.c_int32 * GEMV_MAX_GROUP),
        ("dtype", ctypes.c_int32), ("m", ctypes.c_int32), ("k", ctypes.c_int32), ("count", ctypes.c_int32),
        ("norm_weight", ctypes.c_void_p), ("residual", ctypes.c_void_p), ("residual_out", ctypes.c_void_p),
        ("residual_stride", ctypes.c_int64), ("residual_out_stride", ctypes.c_int64), ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class GreedyArgs(ctypes.Structure):
    """Mirror of lsfa_greedy_args."""
    _fields_ = [
        ("logits", ctypes.c_void_p), ("tokens", ctypes.c_void_p), ("seq_lens", ctypes.c_void_p),
        ("logits_stride", ctypes.c_int64), ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32),
        ("cols", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None


class RopeArgs(ctypes.Structure):
    """Mirror of lsfa_rope_args."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("positions", ctypes.c_void_p), ("cu_seqlens", ctypes.c_void_p),
        ("q_stride", _i64x4), ("k_stride", _i64x4), ("table_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("batch", ctypes.c_int32), ("seqlen", ctypes.c_int32),
        ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("max_pos", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("v", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("slots", ctypes.c_void_p), ("v_stride", _i64x4), ("cache_stride", ctypes.c_int64 * 2),
        ("num_slots", ctypes.c_int64), ("block_tables", ctypes.c_void_p), ("block_table_stride", ctypes.c_int64),
        ("block_size", ctypes.c_int32), ("max_blocks_per_seq", ctypes.c_int32),
    ]


class RmsNormArgs(ctypes.Structure):
    """Mirror of lsfa_rmsnorm_args."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("residual", ctypes.c_void_p), ("weight", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("residual_out", ctypes.c_void_p),
        ("x_stride", ctypes.c_int64), ("residual_stride", ctypes.c_int64), ("out_stride", ctypes.c_int64),
        ("residual_out_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32), ("eps", ctypes.c_float),
    ]


def library_path():
    return _LIB_PATH


def load():
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"{_LIB_NAME} is not built ({_LIB_PATH} missing); run "
                "`python -m lightserve_amd.csrc.build` (or __graft_entry__.build()) first")
        lib = ctypes.CDLL(_LIB_PATH)
        lib.lsfa_abi_version.restype = ctypes.c_int
        lib.lsfa_abi_version.argtypes = []
        lib.lsfa_last_error.restype = ctypes.c_char_p
        lib.lsfa_last_error.argtypes = []
        for name, struct in (("lsfa_fwd_check", FwdArgs), ("lsfa_bwd_check", BwdArgs),
                             ("lsfa_decode_check", DecodeArgs), ("lsfa_rope_check", RopeArgs),
                             ("lsfa_rmsnorm_check", RmsNormArgs), ("lsfa_prefill_paged_check", PrefillPagedArgs),
                             ("lsfa_gemv_check", GemvArgs), ("lsfa_gemv_group_check", GemvGroupArgs),
                             ("lsfa_greedy_check", GreedyArgs)):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(struct)]
        for name, struct in (("lsfa_fwd", FwdArgs), ("lsfa_bwd", BwdArgs), ("lsfa_bwd_noalloc", BwdArgs),
                             ("lsfa_decode", DecodeArgs),
                             ("lsfa_rope", RopeArgs), ("lsfa_rmsnorm", RmsNormArgs),
                             ("lsfa_prefill_paged", PrefillPagedArgs), ("lsfa_gemv", GemvArgs),
                             ("lsfa_gemv_group", GemvGroupArgs), ("lsfa_greedy", GreedyArgs)):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(struct), ctypes.c_void_p]
        lib.lsfa_bwd_workspace_size.restype = ctypes.c_int
        lib.lsfa_bwd_workspace_size.argtypes = [ctypes.POINTER(BwdArgs), ctypes.POINTER(ctypes.c_uint64)]
        lib.lsfa_gemv_group_workspace_size.restype = ctypes.c_int
        lib.lsfa_gemv_group_workspace_size.argtypes = [ctypes.POINTER(GemvGroupArgs), ctypes.POINTER(ctypes.c_uint64)]
        lib.lsfa_gemv_workspace_size.restype = ctypes.c_int
        lib.lsfa_gemv_workspace_size.argtypes = [ctypes.POINTER(GemvArgs), ctypes.POINTER(ctypes.c_uint64)]
        lib.lsfa_decode_workspace_size.restype = ctypes.c_int
        lib.lsfa_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_uint64)]
        version = lib.lsfa_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{_LIB_NAME} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return _lib


def _raise_on(rc, what):
    if rc != 0:
        msg = load().lsfa_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {STATUS.get(rc, rc)}: {msg}")


def fwd_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    lib = load()
    rc = lib.lsfa_fwd_check(ctypes.byref(args))
    return rc, lib.lsfa_last_error().decode(errors="replace")


def bwd_check(args):
    lib = load()
    rc = lib.lsfa_bwd_check(ctypes.byref(args))
    return rc, lib.lsfa_last_error().decode(errors="replace")


def bwd_workspace_size(args):
    """Bytes of device workspace lsfa_bwd needs for these arguments (host only)."""
    n = ctypes.c_uint64(0)
    _raise_on(load().lsfa_bwd_workspace_size(ctypes.byref(args), ctypes.byref(n)), "lsfa_bwd_workspace_size")
    return n.value


def decode_check(args):
    lib = load()
    rc = lib.lsfa_decode_check(ctypes.byref(args))
    return rc, lib.lsfa_last_error().decode(errors="replace")


def decode_workspace_size(args):
    """Bytes of device workspace lsfa_decode needs (host only; 0 when unsplit)."""
    n = ctypes.c_uint64(0)
    _raise_on(load().lsfa_decode_workspace_size(ctypes.byref(args), ctypes.byref(n)), "lsfa_decode_workspace_size")
    return n.value


def decode(args, stream):
    _raise_on(load().lsfa_decode(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_decode")


def prefill_paged_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_prefill_paged_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def prefill_paged(args, stream):
    _raise_on(load().lsfa_prefill_paged(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_prefill_paged")


def gemv_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_gemv_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def gemv_workspace_size(args):
    """Bytes of device workspace lsfa_gemv needs (host only)."""
    n = ctypes.c_uint64(0)
    _raise_on(load().lsfa_gemv_workspace_size(ctypes.byref(args), ctypes.byref(n)), "lsfa_gemv_workspace_size")
    return n.value


def gemv(args, stream):
    _raise_on(load().lsfa_gemv(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_gemv")


def gemv_group_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_gemv_group_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def gemv_group_workspace_size(args):
    n = ctypes.c_uint64(0)
    _raise_on(load().lsfa_gemv_group_workspace_size(ctypes.byref(args), ctypes.byref(n)),
              "lsfa_gemv_group_workspace_size")
    return n.value


def gemv_group(args, stream):
    _raise_on(load().lsfa_gemv_group(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_gemv_group")


def greedy_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_greedy_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def greedy(args, stream):
    _raise_on(load().lsfa_greedy(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_greedy")


def rope_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_rope_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def rope(args, stream):
    _raise_on(load().lsfa_rope(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_rope")


def rmsnorm_check(args):
    """Host-only validation (no GPU access); returns (status, message)."""
    rc = load().lsfa_rmsnorm_check(ctypes.byref(args))
    return rc, load().lsfa_last_error().decode(errors="replace")


def rmsnorm(args, stream):
    _raise_on(load().lsfa_rmsnorm(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_rmsnorm")


def fwd(args, stream):
    _raise_on(load().lsfa_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_fwd")


def bwd(args, stream):
    _raise_on(load().lsfa_bwd(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_bwd")


def bwd_noalloc(args, stream):
    """lsfa_bwd_noalloc: the backward with the library's own scratch array as
    workspace (args.workspace is ignored)."""
    _raise_on(load().lsfa_bwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream)), "lsfa_bwd_noalloc")


def strides4(t):
    """Element strides of a [b, h, n, d] tensor."""
    return _i64x4(*t.stride())


def strides_thd(t):
    """Element strides of a packed [tokens, heads, d] tensor in ABI order (b, h, n, d)."""
    st = t.stride()
    return _i64x4(0, st[1], st[0], st[2])


def fast_layout_ok(t):
    """Whether the bf16/fp16 kernels can address t in place: unit head-dim
    stride, head_dim and every other stride a multiple of 8 elements, 16-byte
    aligned base (the requirements lsfa_fwd_check/lsfa_bwd_check enforce)."""
    if t.stride(-1) != 1 or t.shape[-1] % 8 != 0 or t.data_ptr() % 16 != 0:
        return False
    return all(s % 8 == 0 for s in t.stride()[:-1])


def current_stream(device):
    return torch.cuda.current_stream(device).cuda_stream
