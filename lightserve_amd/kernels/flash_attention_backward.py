"""FlashAttention forward-with-logsumexp, backward and autograd on MI355X.

Drop-in for the reference's `kernels/flash_attention_backward.py`:
  - `_flash_attention_forward_lse(q, k, v, causal)` -> (o, L) with
    L = m + ln(l) fp32 [B, H, N] (kernels/flash_attention_backward.py:172-199);
  - `_flash_attention_backward(do, q, k, v, o, L, causal)` -> (dq, dk, dv)
    (:333-382);
  - `_FlashAttentionFunction` (:385-397) saving (q, k, v, o, L);
  - `flash_attention(q, k, v, causal=False)` (:400-420), with the same
    assertions as the forward-only entry point.
Keyword-only extra on every entry point: `sm_scale` (default 1/sqrt(D)).

The backward recomputes P from L. The dQ kernel's prologue writes
delta = rowsum(dO * O) (with L*log2(e) and transposed copies of q and dO) into
a workspace allocated here for the dK/dV kernel, and dq/dk/dv come back in the input dtype from two deterministic
kernels (no fp32 dq buffer, no atomics).
"""
import torch

from .. import _lib
from .flash_attention import (as_kernel_layout, check_inputs, default_scale, forward_into,
                              padded_head_dim)


def _flash_attention_forward_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                                 sm_scale=None):
    """Forward that also returns L (fp32 [B, H, N]), the state the backward needs."""
    scale = default_scale(q.shape[-1], sm_scale)
    return forward_into(q, k, v, causal, scale, True)


def _backward_args(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                   L: torch.Tensor, causal: bool, sm_scale=None, flags=0):
    """The lsfa_bwd arguments for these tensors, and what they point into:
    (args, keep) with keep = (dq, dk, dv, the kernel-layout outputs, the
    inputs' kernel-layout views or copies, workspace). None for an empty
    problem. flags: lsfa_bwd_args.flags (the workspace is sized for them)."""
    B, H, N, D = q.shape
    scale = default_scale(D, sm_scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    if q.numel() == 0:
        return None, (dq, dk, dv)
    dp = padded_head_dim(q)
    qk, kk, vk, ok_, dok = (as_kernel_layout(t, dp) for t in (q, k, v, o, do))
    outs = []
    for t in (dq, dk, dv):
        direct = t.dtype == torch.float32 or (dp == D and _lib.fast_layout_ok(t))
        outs.append(t if direct else torch.empty(B, H, N, dp, device=q.device, dtype=q.dtype))
    dqk, dkk, dvk = outs
    L = L.contiguous()
    assert L.shape == (B, H, N) and L.dtype == torch.float32, "L must be fp32 [B, H, N]"
    args = _lib.BwdArgs(
        q=qk.data_ptr(), k=kk.data_ptr(), v=vk.data_ptr(), o=ok_.data_ptr(), dout=dok.data_ptr(),
        lse=L.data_ptr(), dq=dqk.data_ptr(), dk=dkk.data_ptr(), dv=dvk.data_ptr(), workspace=None,
        workspace_bytes=0,
        q_stride=_lib.strides4(qk), k_stride=_lib.strides4(kk), v_stride=_lib.strides4(vk),
        o_stride=_lib.strides4(ok_), do_stride=_lib.strides4(dok), dq_stride=_lib.strides4(dqk),
        dk_stride=_lib.strides4(dkk), dv_stride=_lib.strides4(dvk), lse_stride=_lib._i64x3(*L.stride()),
        cu_seqlens_q=None, cu_seqlens_k=None,
        dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, heads_q=H, heads_kv=H, seqlen_q=N, seqlen_k=N,
        head_dim=dp, causal=int(bool(causal)), sm_scale=scale, flags=flags,
    )
    nbytes = _lib.bwd_workspace_size(args)
    # The caching allocator hands out 512-byte aligned blocks (the ABI asks for 256).
    workspace = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = workspace.data_ptr(), nbytes
    return args, (dq, dk, dv, (dqk, dkk, dvk), (qk, kk, vk, ok_, dok, L), workspace)


def _flash_attention_backward(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              o: torch.Tensor, L: torch.Tensor, causal: bool, sm_scale=None):
    """Returns (dq, dk, dv) in the input dtype (dq like q, dk like k, dv like v)."""
    args, keep = _backward_args(do, q, k, v, o, L, causal, sm_scale)
    dq, dk, dv = keep[:3]
    if args is None:
        return dq, dk, dv
    with torch.cuda.device(q.device):
        _lib.bwd(args, _lib.current_stream(q.device))
    D = q.shape[-1]
    for t, tk in zip((dq, dk, dv), keep[3]):
        if tk is not t:
            t.copy_(tk[..., :D])
    return dq, dk, dv


class _FlashAttentionFunction(torch.autograd.Function):
    """The reference's autograd Function (kernels/flash_attention_backward.py:385-397):
    `_FlashAttentionFunction.apply(q, k, v, causal)` as there, with sm_scale
    an optional fifth argument (default 1/sqrt(D))."""

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale=None):
        o, L = _flash_attention_forward_lse(q, k, v, causal, sm_scale)
        ctx.save_for_backward(q, k, v, o, L)
        ctx.causal = causal
        ctx.sm_scale = sm_scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, L = ctx.saved_tensors
        dq, dk, dv = _flash_attention_backward(do, q, k, v, o, L, ctx.causal, ctx.sm_scale)
        return dq, dk, dv, None, None


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False, *,
                    sm_scale=None) -> torch.Tensor:
    """Autograd-enabled FlashAttention (forward with L, recomputation backward).

    q, k, v: [B, H, N, D], same shape, same dtype, on the GPU.
    """
    check_inputs(q, k, v)
    return _FlashAttentionFunction.apply(q, k, v, causal, sm_scale)
