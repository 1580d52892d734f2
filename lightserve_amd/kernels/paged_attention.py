"""Paged-KV decode attention on MI355X: one new query token per sequence
against a KV cache addressed through block tables.

The reference has no such kernel. Its engine keeps the block tables
(engine/block_manager.py:56-60: entry i of a request's table holds tokens
[i*block_size, (i+1)*block_size)) and documents decode attention as the
missing piece (engine/README.md, "No decode-shaped attention kernel": Nq = 1
against a paged Nkv; engine/request.py is_prefill). A cache block holds
block_size x n_kv_heads x head_dim elements per layer for K and for V
(engine/config.py:5-7), so the caches here are
[num_blocks, block_size, heads_kv, head_dim].

    paged_attention_decode(q, k_cache, v_cache, block_tables, seq_lens, *,
                           max_seq_len=None, sm_scale=None, return_lse=False)

q is [batch, heads_q, head_dim]; block_tables int32 [batch, max_blocks];
seq_lens int32 [batch] counts each sequence's cached tokens (the new token's
K/V already written). Query head h reads KV head h // (heads_q // heads_kv).
Returns o like q (and lse fp32 [batch, heads_q], natural log, when asked).
max_seq_len bounds seq_lens and sets how sequences are split across
workgroups; when it is None it is read from seq_lens (a device sync, so pass
it under graph capture).

    paged_prefill(q, k_cache, v_cache, block_tables, cu_seqlens_q, seq_lens_k, *,
                  max_seqlen_q=None, causal=True, sm_scale=None, return_lse=False)

Chunked prefill against the same cache: the engine's scheduled-tokens > 1
path, which its scheduler documents as missing (engine/request.py:86-93,
engine/scheduler.py:34-44). q is packed [total_q, heads_q, head_dim] with
sequence b owning rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 (a chunk of
new tokens); seq_lens_k int32 [batch] counts the sequence's cached keys
with the chunk's own K/V already written. Causal masking is bottom-right
aligned: chunk query i of n sits at position seq_lens_k[b] - n + i. Returns
o like q (and lse fp32 [heads_q, total_q] when asked); block_size must be a
power of two of at least 16. One launch of the forward kernel with its K/V
tiles gathered through the block tables.
"""
import math

import torch

from .. import _lib


def _check(q, k_cache, v_cache, block_tables, seq_lens):
    assert q.dim() == 3, "q must be [batch, heads_q, head_dim]"
    assert k_cache.dim() == 4 and v_cache.shape == k_cache.shape, \
        "k_cache and v_cache must both be [num_blocks, block_size, heads_kv, head_dim]"
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                    ("seq_lens", seq_lens)):
        assert t.is_cuda, f"{name} must be a GPU tensor"
    assert q.dtype == k_cache.dtype == v_cache.dtype, "q, k_cache and v_cache must share a dtype"
    assert q.dtype in (torch.float16, torch.bfloat16), "paged decode supports bf16 and fp16"
    assert block_tables.dtype == torch.int32 and seq_lens.dtype == torch.int32, \
        "block_tables and seq_lens must be int32"
    assert block_tables.dim() == 2 and block_tables.shape[0] == q.shape[0], "block_tables must be [batch, max_blocks]"
    assert seq_lens.shape == (q.shape[0],), "seq_lens must be [batch]"
    assert q.shape[2] == k_cache.shape[3], "head_dim of q and of the caches differ"
    assert q.shape[1] % k_cache.shape[2] == 0, "heads_q must be a multiple of heads_kv"


def paged_attention_decode(q, k_cache, v_cache, block_tables, seq_lens, *, max_seq_len=None, sm_scale=None,
                           return_lse=False):
    _check(q, k_cache, v_cache, block_tables, seq_lens)
    B, Hq, D = q.shape
    num_blocks, block_size, Hkv, _ = k_cache.shape
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if B > 0 else 0
    q_ = q if (q.stride(-1) == 1 and all(s % 8 == 0 for s in q.stride()[:2]) and q.data_ptr() % 16 == 0) \
        else q.contiguous()
    bt = block_tables if block_tables.stride(1) == 1 else block_tables.contiguous()
    sl = seq_lens.contiguous()
    o = torch.empty(B, Hq, D, device=q.device, dtype=q.dtype)
    lse = torch.empty(B, Hq, device=q.device, dtype=torch.float32) if return_lse else None
    args = _lib.DecodeArgs(
        q=q_.data_ptr(), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(), o=o.data_ptr(),
        lse=lse.data_ptr() if lse is not None else None, block_tables=bt.data_ptr(), seq_lens=sl.data_ptr(),
        workspace=None, workspace_bytes=0,
        q_stride=_lib._i64x3(*q_.stride()), k_stride=_lib._i64x4(*k_cache.stride()),
        v_stride=_lib._i64x4(*v_cache.stride()), o_stride=_lib._i64x3(*o.stride()),
        lse_stride=_lib._i64x2(*(lse.stride() if lse is not None else (0, 0))),
        block_table_stride=bt.stride(0), dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, heads_q=Hq,
        heads_kv=Hkv, head_dim=D, block_size=block_size, num_blocks=num_blocks,
        max_blocks_per_seq=bt.shape[1], max_seq_len=int(max_seq_len), sm_scale=scale,
    )
    nbytes = _lib.decode_workspace_size(args)
    ws = None
    if nbytes > 0:
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)  # 512-byte aligned blocks
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(q.device):
        _lib.decode(args, _lib.current_stream(q.device))
    return (o, lse) if return_lse else o


def paged_prefill(q, k_cache, v_cache, block_tables, cu_seqlens_q, seq_lens_k, *, max_seqlen_q=None, causal=True,
                  sm_scale=None, return_lse=False):
    assert q.dim() == 3, "q must be packed [total_q, heads_q, head_dim]"
    assert k_cache.dim() == 4 and v_cache.shape == k_cache.shape, \
        "k_cache and v_cache must be [num_blocks, block_size, heads_kv, head_dim] of one shape"
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                    ("cu_seqlens_q", cu_seqlens_q), ("seq_lens_k", seq_lens_k)):
        assert t.is_cuda, f"{name} must be a GPU tensor"
    assert q.dtype == k_cache.dtype == v_cache.dtype, "q, k_cache and v_cache must share a dtype"
    assert q.dtype in (torch.float16, torch.bfloat16), "paged prefill supports bf16 and fp16"
    assert block_tables.dtype == torch.int32 and cu_seqlens_q.dtype == torch.int32 and \
        seq_lens_k.dtype == torch.int32, "block_tables, cu_seqlens_q and seq_lens_k must be int32"
    assert block_tables.dim() == 2, "block_tables must be [batch, max_blocks]"
    B = block_tables.shape[0]
    assert cu_seqlens_q.shape == (B + 1,) and seq_lens_k.shape == (B,), \
        "cu_seqlens_q must be [batch + 1] and seq_lens_k [batch]"
    assert q.shape[2] == k_cache.shape[3], "head_dim of q and of the caches differ"
    assert q.shape[1] % k_cache.shape[2] == 0, "heads_q must be a multiple of heads_kv"
    T, Hq, D = q.shape
    num_blocks, block_size, Hkv, _ = k_cache.shape
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    if max_seqlen_q is None:
        max_seqlen_q = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) if B > 0 else 0
    q_ = q if (q.stride(-1) == 1 and all(s % 8 == 0 for s in q.stride()[:2]) and q.data_ptr() % 16 == 0) \
        else q.contiguous()
    assert k_cache.stride(3) == 1 and v_cache.stride(3) == 1, "the caches' head-dim stride must be 1"
    bt = block_tables if block_tables.stride(1) == 1 else block_tables.contiguous()
    cu, sl = cu_seqlens_q.contiguous(), seq_lens_k.contiguous()  # kept alive until the launch
    o = torch.empty(T, Hq, D, device=q.device, dtype=q.dtype)
    lse = torch.empty(Hq, T, device=q.device, dtype=torch.float32) if return_lse else None
    args = _lib.PrefillPagedArgs(
        q=q_.data_ptr(), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(), o=o.data_ptr(),
        lse=lse.data_ptr() if lse is not None else None, cu_seqlens_q=cu.data_ptr(),
        seq_lens_k=sl.data_ptr(), block_tables=bt.data_ptr(),
        q_stride=_lib._i64x2(*q_.stride()[:2]), k_stride=_lib._i64x3(*k_cache.stride()[:3]),
        v_stride=_lib._i64x3(*v_cache.stride()[:3]), o_stride=_lib._i64x2(*o.stride()[:2]),
        lse_stride=_lib._i64x2(*(lse.stride() if lse is not None else (0, 0))),
        block_table_stride=bt.stride(0), dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, heads_q=Hq,
        heads_kv=Hkv, head_dim=D, block_size=block_size, num_blocks=num_blocks, max_blocks_per_seq=bt.shape[1],
        max_seqlen_q=int(max_seqlen_q), causal=int(bool(causal)), sm_scale=scale, reserved=0,
    )
    if T > 0:
        with torch.cuda.device(q.device):
            _lib.prefill_paged(args, _lib.current_stream(q.device))
    return (o, lse) if return_lse else o
