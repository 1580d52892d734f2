"""FlashAttention forward on MI355X (gfx950 HIP kernels behind a C ABI).

Drop-in for the reference's `kernels/flash_attention.py`
(`flash_attention_forward`, kernels/flash_attention.py:182-222): same
signature, same [B, H, N, D] layout with arbitrary strides, same validation
(AssertionError, in the same order, :192-199), same default scale 1/sqrt(D)
(:203), output allocated with `torch.empty_like(q)` so it keeps q's strides
(:202). Keyword-only extras: `sm_scale` and `return_lse` (the logsumexp
L = m + ln(l) in natural-log, scaled-score units, fp32 [B, H, N]).

The launch goes on the caller's current stream with no host synchronisation
and no tuning at call time, so the call can be captured in a HIP graph
(the reference captures its model forward in model/cuda_graph_decode.py:137-139).
"""
import math

import torch
import torch.nn.functional as F

from .. import _lib

SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def check_inputs(q, k, v):
    """The reference's argument checks (kernels/flash_attention.py:192-199)."""
    assert q.ndim == 4 and k.ndim == 4 and v.ndim == 4, (
        f"expected q/k/v as [B, H, N, D], got {q.ndim}D/{k.ndim}D/{v.ndim}D"
    )
    assert q.shape == k.shape == v.shape, (
        f"q/k/v shapes must match, got {tuple(q.shape)}/{tuple(k.shape)}/{tuple(v.shape)}"
    )
    assert q.is_cuda and k.is_cuda and v.is_cuda, "the gfx950 kernels need GPU tensors"
    assert q.dtype == k.dtype == v.dtype, f"dtype mismatch: q={q.dtype} k={k.dtype} v={v.dtype}"
    assert q.dtype in SUPPORTED_DTYPES, f"unsupported dtype {q.dtype} (float32, float16 or bfloat16)"


def default_scale(head_dim, sm_scale):
    return 1.0 / math.sqrt(head_dim) if sm_scale is None else float(sm_scale)


def padded_head_dim(t):
    """Head dim the bf16/fp16 kernels will see for t (next multiple of 8)."""
    d = t.shape[-1]
    return d if t.dtype == torch.float32 else (d + 7) // 8 * 8


def as_kernel_layout(t, dp):
    """Returns t itself when the kernels can address it in place, else a packed
    copy whose head dim is zero-padded to dp (zero columns add nothing to any
    dot product and produce output columns that are discarded)."""
    if t.dtype == torch.float32:
        return t
    if t.shape[-1] == dp and _lib.fast_layout_ok(t):
        return t
    t = t.contiguous()
    if t.shape[-1] != dp:
        t = F.pad(t, (0, dp - t.shape[-1]))
    return t


def lse_args(lse):
    """(pointer, strides) of an optional fp32 lse tensor for the ABI structs."""
    if lse is None:
        return None, _lib._i64x3(0, 0, 0)
    return lse.data_ptr(), _lib._i64x3(*lse.stride())


def forward_into(q, k, v, causal, scale, want_lse):
    """Runs the forward kernel; returns (o, lse or None). o is empty_like(q)."""
    B, H, N, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32) if want_lse else None
    if o.numel() == 0:
        if lse is not None:
            lse.fill_(-math.inf)
        return o, lse
    dp = padded_head_dim(q)
    qk, kk, vk = (as_kernel_layout(t, dp) for t in (q, k, v))
    direct = q.dtype == torch.float32 or (dp == D and _lib.fast_layout_ok(o))
    ok = o if direct else torch.empty(B, H, N, dp, device=q.device, dtype=q.dtype)
    lse_ptr, lse_stride = lse_args(lse)
    args = _lib.FwdArgs(
        q=qk.data_ptr(), k=kk.data_ptr(), v=vk.data_ptr(), o=ok.data_ptr(), lse=lse_ptr,
        q_stride=_lib.strides4(qk), k_stride=_lib.strides4(kk), v_stride=_lib.strides4(vk),
        o_stride=_lib.strides4(ok), lse_stride=lse_stride,
        cu_seqlens_q=None, cu_seqlens_k=None,
        dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, heads_q=H, heads_kv=H, seqlen_q=N, seqlen_k=N,
        head_dim=dp, causal=int(bool(causal)), sm_scale=scale, reserved=0,
    )
    with torch.cuda.device(q.device):
        _lib.fwd(args, _lib.current_stream(q.device))
    if ok is not o:
        o.copy_(ok[..., :D])
    return o, lse


def flash_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False, *,
                            sm_scale=None, return_lse: bool = False):
    """O = softmax(Q @ K^T * sm_scale) @ V (sm_scale defaults to 1/sqrt(D)).

    q, k, v: [B, H, N, D], same shape, same dtype (float32, float16 or
    bfloat16), on the GPU. Returns O (q's dtype and strides), or (O, lse) when
    return_lse is set.
    """
    check_inputs(q, k, v)
    scale = default_scale(q.shape[-1], sm_scale)
    o, lse = forward_into(q, k, v, causal, scale, return_lse)
    return (o, lse) if return_lse else o
