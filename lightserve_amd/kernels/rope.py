"""Rotary position embedding on MI355X: q and k rotated in one HIP launch.

The reference applies RoPE with plain tensor ops (model/minimal_llama.py:163-173):

    apply_rope(q, k, cos, sin, n) -> (q * cos + rotate_half(q) * sin,
                                      k * cos + rotate_half(k) * sin)

for q, k [B, n_heads, N, head_dim] and cos/sin [max_seq_len, head_dim] tables
(precompute_rope, model/minimal_llama.py:144-156) sliced to rows 0..n-1. Here
the same rotation runs in one kernel (lsfa_rope) that reads each element of
q and k once, computes in fp32 and writes the result rounded once:

    apply_rope(q, k, cos, sin, n)                   # the reference's signature; new tensors
    apply_rope_(q, k, cos, sin, positions=None)     # in place (what the model calls)

`positions` (int32 [B], optional) gives the position of each sequence's first
token, so the same call rotates a decode step's single token (positions =
tokens already cached) or a prefill chunk. k may be None (q only) and may
have fewer heads than q (GQA). The kernels address q and k in place when the
head dim is contiguous and the other strides are multiples of 16 bytes; the
[B, H, N, D] transposed views of a [B, N, H*D] projection output qualify.
"""
import torch

from .. import _lib


def _check(q, k, cos, sin):
    assert q.dim() == 4, "q must be [batch, heads, seqlen, head_dim]"
    assert q.is_cuda, "q must be a GPU tensor"
    if k is not None:
        assert k.dim() == 4 and k.is_cuda, "k must be a 4-D GPU tensor"
        assert k.dtype == q.dtype, "q and k must share a dtype"
        assert k.shape[0] == q.shape[0] and k.shape[2:] == q.shape[2:], "q and k differ in batch, seqlen or head_dim"
    assert cos.dim() == 2 and sin.shape == cos.shape, "cos and sin must both be [max_pos, head_dim]"
    assert cos.shape[1] == q.shape[3], "table width differs from head_dim"
    assert cos.dtype == sin.dtype == q.dtype, "cos/sin must have q's dtype (as precompute_rope returns them)"
    assert cos.is_cuda and sin.is_cuda, "cos and sin must be GPU tensors"
    assert q.dtype in _lib.TORCH_TO_LSFA, f"unsupported dtype {q.dtype}"


def _addressable(t):
    elem = t.element_size()
    return t.stride(-1) == 1 and all((s * elem) % 16 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0


def apply_rope_(q, k, cos, sin, positions=None, *, v=None, k_cache=None, v_cache=None, slots=None,
                block_tables=None):
    """Rotates q and k (None: q only) in place and returns them. With
    k_cache/v_cache ([num_blocks, block_size, heads_kv, head_dim]), v (k's
    shape) and slots (int64 [batch * seqlen], token b*seqlen+n -> cache slot
    block * block_size + offset; negative: not stored) or block_tables (int32
    [batch, max_blocks]: the slot of token n of sequence b follows from its
    position positions[b] + n), the rotated k rows and v's rows are also
    written into the caches by the same launch."""
    _check(q, k, cos, sin)
    if k_cache is not None:
        assert k is not None and v is not None and v_cache is not None, (
            "a cache append needs k, v, k_cache, v_cache and slots or block_tables")
        assert v.shape == k.shape and v.dtype == k.dtype and _addressable(v), "v must match k and be addressable"
        assert k_cache.shape == v_cache.shape and k_cache.dim() == 4 and k_cache.dtype == k.dtype, (
            "k_cache and v_cache must be [num_blocks, block_size, heads_kv, head_dim] in k's dtype")
        assert k_cache.shape[2:] == (k.shape[1], k.shape[3]), "cache heads / head_dim differ from k"
        assert k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous"
        assert (slots is None) != (block_tables is None), "give either slots or block_tables"
        if slots is not None:
            assert slots.dtype == torch.int64 and slots.is_cuda and slots.numel() == k.shape[0] * k.shape[2], (
                "slots must be an int64 GPU tensor with one entry per token")
        else:
            assert block_tables.dtype == torch.int32 and block_tables.is_cuda and block_tables.dim() == 2 and \
                block_tables.shape[0] == k.shape[0] and block_tables.stride(1) == 1, (
                    "block_tables must be an int32 GPU tensor [batch, max_blocks] with unit column stride")
    assert _addressable(q) and (k is None or _addressable(k)), \
        "apply_rope_ needs unit head-dim stride and 16-byte aligned strides (use apply_rope for other layouts)"
    B, Hq, N, D = q.shape
    if positions is not None:
        assert positions.dtype == torch.int32 and positions.shape == (B,) and positions.is_cuda, \
            "positions must be an int32 GPU tensor of shape [batch]"
        positions = positions.contiguous()
    c, s = cos.contiguous(), sin.contiguous()  # no copies for precompute_rope's tables
    args = _lib.RopeArgs(
        q=q.data_ptr(), k=k.data_ptr() if k is not None else None, cos=c.data_ptr(), sin=s.data_ptr(),
        positions=positions.data_ptr() if positions is not None else None, cu_seqlens=None,
        q_stride=_lib.strides4(q), k_stride=_lib.strides4(k) if k is not None else _lib._i64x4(0, 0, 0, 0),
        table_stride=c.stride(0), dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, seqlen=N, heads_q=Hq,
        heads_kv=k.shape[1] if k is not None else 0, head_dim=D, max_pos=c.shape[0], reserved=0,
    )
    if k_cache is not None:
        sl = slots.contiguous() if slots is not None else None
        args.v, args.k_cache, args.v_cache = v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
        if sl is not None:
            args.slots = sl.data_ptr()
        else:
            args.block_tables, args.block_table_stride = block_tables.data_ptr(), block_tables.stride(0)
            args.block_size, args.max_blocks_per_seq = k_cache.shape[1], block_tables.shape[1]
        args.v_stride = _lib.strides4(v)
        args.cache_stride[0], args.cache_stride[1] = k_cache.stride(1), k_cache.stride(2)
        args.num_slots = k_cache.shape[0] * k_cache.shape[1]
    with torch.cuda.device(q.device):
        _lib.rope(args, _lib.current_stream(q.device))
    return q, k


def apply_rope(q, k, cos, sin, n):
    """Drop-in for the reference's apply_rope: returns rotated copies of q and
    k ([B, H, n, D]) using table rows 0..n-1; the inputs are unchanged."""
    _check(q, k, cos, sin)
    assert q.shape[2] == n and k.shape[2] == n, "n must equal the sequence length of q and k"
    assert n <= cos.shape[0], "n exceeds the table's rows"
    q_rot = torch.empty_like(q, memory_format=torch.contiguous_format).copy_(q)
    k_rot = torch.empty_like(k, memory_format=torch.contiguous_format).copy_(k)
    return apply_rope_(q_rot, k_rot, cos, sin)
