"""Packed variable-length forward with grouped-query attention (chunked prefill).

Not present in the reference, which requires q.shape == k.shape == v.shape
(model/minimal_llama.py:8-12) and documents chunked prefill over a cached
prefix as missing (engine/README.md:142-147). The head grouping follows the
reference's own GQA convention, query head h reads kv head h // (Hq // Hkv)
(repeat_interleave in benchmarks/profiling/roofline/measure_roofline.py:94-98).

Layout: q [total_q, Hq, D], k/v [total_k, Hkv, D], int32 prefix offsets
cu_seqlens_q/cu_seqlens_k of length batch+1 on the GPU. Causal masking is
bottom-right aligned: query i of a sequence with Nq queries and Nk keys sees
keys j <= i + Nk - Nq, i.e. a chunk of new tokens attends to the whole cached
prefix plus itself causally.
"""
import math

import torch

from .. import _lib
from .flash_attention import SUPPORTED_DTYPES, as_kernel_layout, lse_args


def _check_varlen_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k):
    """Argument checks shared by the varlen forward and backward, made before
    the library is touched (AssertionError, as the reference's entry points,
    kernels/flash_attention.py:192-199)."""
    assert q.ndim == 3 and k.ndim == 3 and v.ndim == 3, "expected packed [tokens, heads, D] tensors"
    assert k.shape == v.shape, f"k/v shapes must match, got {tuple(k.shape)}/{tuple(v.shape)}"
    assert q.shape[2] == k.shape[2], "q and k/v head dims must match"
    assert k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0, "query heads must be a multiple of kv heads"
    assert q.is_cuda and k.is_cuda and v.is_cuda, "the gfx950 kernels need GPU tensors"
    assert q.dtype == k.dtype == v.dtype, f"dtype mismatch: q={q.dtype} k={k.dtype} v={v.dtype}"
    assert q.dtype in SUPPORTED_DTYPES, f"unsupported dtype {q.dtype}"
    assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32, "cu_seqlens must be int32"
    assert cu_seqlens_q.is_cuda and cu_seqlens_k.is_cuda, "cu_seqlens must be GPU tensors"
    assert cu_seqlens_q.ndim == 1 and cu_seqlens_q.shape == cu_seqlens_k.shape and cu_seqlens_q.numel() >= 2, (
        "cu_seqlens_q/k must be 1-D of equal length batch+1")


def flash_attention_varlen_forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                   causal=True, sm_scale=None):
    """Returns (o [total_q, Hq, D] in q's dtype, lse fp32 [Hq, total_q]).

    max_seqlen_q / max_seqlen_k must bound every sequence's length (the grid
    and the workspace are sized by them, as in the usual varlen attention
    APIs; checking them would cost a device-to-host copy per call)."""
    _check_varlen_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k)
    Tq, Hq, D = q.shape
    Hkv = k.shape[1]
    batch = cu_seqlens_q.numel() - 1
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    o = torch.empty_like(q)
    lse = torch.empty((Hq, Tq), device=q.device, dtype=torch.float32)
    if Tq == 0:
        return o, lse
    dp = D if q.dtype == torch.float32 else (D + 7) // 8 * 8
    qk, kk, vk = (as_kernel_layout(t, dp) for t in (q, k, v))
    direct = q.dtype == torch.float32 or (dp == D and _lib.fast_layout_ok(o))
    ok = o if direct else torch.empty(Tq, Hq, dp, device=q.device, dtype=q.dtype)
    cu_q = cu_seqlens_q.contiguous()
    cu_k = cu_seqlens_k.contiguous()
    lse_ptr, _ = lse_args(lse)
    args = _lib.FwdArgs(
        q=qk.data_ptr(), k=kk.data_ptr(), v=vk.data_ptr(), o=ok.data_ptr(), lse=lse_ptr,
        q_stride=_lib.strides_thd(qk), k_stride=_lib.strides_thd(kk), v_stride=_lib.strides_thd(vk),
        o_stride=_lib.strides_thd(ok), lse_stride=_lib._i64x3(0, lse.stride(0), lse.stride(1)),
        cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_k=cu_k.data_ptr(),
        dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=batch, heads_q=Hq, heads_kv=Hkv,
        seqlen_q=int(max_seqlen_q), seqlen_k=int(max_seqlen_k),
        head_dim=dp, causal=int(bool(causal)), sm_scale=scale, reserved=0,
    )
    with torch.cuda.device(q.device):
        _lib.fwd(args, _lib.current_stream(q.device))
    if ok is not o:
        o.copy_(ok[..., :D])
    return o, lse


def flash_attention_varlen_backward(do, q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                    causal=True, sm_scale=None):
    """Gradients of the packed varlen (and GQA) forward: returns (dq, dk, dv)
    in the inputs' dtype and layout, dk/dv per KV head summed over its group.
    lse is the forward's [Hq, total_q] fp32 output. bf16/fp16 (the fp32
    kernels have no varlen backward); head dims that are not a multiple of 8
    are zero-padded as in the forward."""
    _check_varlen_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k)
    assert q.dtype in (torch.bfloat16, torch.float16), "the varlen backward runs on bf16/fp16"
    assert do.shape == q.shape == o.shape, "do and o must have q's shape"
    assert do.dtype == q.dtype and o.dtype == q.dtype, "do and o must have q's dtype"
    assert do.is_cuda and o.is_cuda and lse.is_cuda, "the gfx950 kernels need GPU tensors"
    assert lse.dtype == torch.float32 and lse.shape == (q.shape[1], q.shape[0]), "lse must be fp32 [Hq, total_q]"
    Tq, Hq, D = q.shape
    Tk, Hkv = k.shape[0], k.shape[1]
    batch = cu_seqlens_q.numel() - 1
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    if Tq == 0 or Tk == 0:  # no query sees a key: every gradient is zero
        return dq.zero_(), dk.zero_(), dv.zero_()
    dp = (D + 7) // 8 * 8
    qk, kk, vk, ok_, dok = (as_kernel_layout(t, dp) for t in (q, k, v, o, do))
    outs = [t if dp == D and _lib.fast_layout_ok(t) else torch.empty(*t.shape[:2], dp, device=t.device, dtype=t.dtype)
            for t in (dq, dk, dv)]
    dqk, dkk, dvk = outs
    lse = lse.contiguous()
    cu_q = cu_seqlens_q.contiguous()
    cu_k = cu_seqlens_k.contiguous()
    th = _lib.strides_thd
    args = _lib.BwdArgs(
        q=qk.data_ptr(), k=kk.data_ptr(), v=vk.data_ptr(), o=ok_.data_ptr(), dout=dok.data_ptr(),
        lse=lse.data_ptr(), dq=dqk.data_ptr(), dk=dkk.data_ptr(), dv=dvk.data_ptr(), workspace=None,
        workspace_bytes=0, q_stride=th(qk), k_stride=th(kk), v_stride=th(vk), o_stride=th(ok_), do_stride=th(dok),
        dq_stride=th(dqk), dk_stride=th(dkk), dv_stride=th(dvk),
        lse_stride=_lib._i64x3(0, lse.stride(0), lse.stride(1)),
        cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_k=cu_k.data_ptr(), dtype=_lib.TORCH_TO_LSFA[q.dtype],
        batch=batch, heads_q=Hq, heads_kv=Hkv, seqlen_q=int(max_seqlen_q), seqlen_k=int(max_seqlen_k),
        head_dim=dp, causal=int(bool(causal)), sm_scale=scale, flags=0)
    n = _lib.bwd_workspace_size(args)
    ws = torch.empty(max(n, 1), device=q.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = ws.data_ptr(), n
    with torch.cuda.device(q.device):
        _lib.bwd(args, _lib.current_stream(q.device))
    for t, tk in zip((dq, dk, dv), outs):
        if tk is not t:
            t.copy_(tk[..., :D])
    return dq, dk, dv


class _VarlenFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_q, max_k, causal, sm_scale):
        o, lse = flash_attention_varlen_forward(q, k, v, cu_q, cu_k, max_q, max_k, causal, sm_scale)
        ctx.save_for_backward(q, k, v, o, lse, cu_q, cu_k)
        ctx.cfg = (max_q, max_k, causal, sm_scale)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, cu_q, cu_k = ctx.saved_tensors
        dq, dk, dv = flash_attention_varlen_backward(do, q, k, v, o, lse, cu_q, cu_k, *ctx.cfg)
        return dq, dk, dv, None, None, None, None, None, None


def flash_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal=True, sm_scale=None):
    """Differentiable packed varlen / GQA attention: o [total_q, Hq, D]. The
    backward runs on bf16/fp16: fp32 inputs that require grad are refused here,
    before the forward runs, not at .backward()."""
    _check_varlen_inputs(q, k, v, cu_seqlens_q, cu_seqlens_k)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        assert q.dtype in (torch.bfloat16, torch.float16), (
            "the varlen backward runs on bf16/fp16; fp32 inputs cannot require grad here")
    return _VarlenFunction.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal, sm_scale)
