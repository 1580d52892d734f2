"""Attention oracle (CPU, float64 by default) -- test infrastructure only.

Conventions (the reference's): scores S = (q . k) * sm_scale, computed after
the dot product (kernels/flash_attention.py:148); lse L = m + ln(l) in
natural-log, scaled-score units (kernels/flash_attention_backward.py:162);
sm_scale defaults to 1/sqrt(D) (kernels/flash_attention.py:203). Causal masks
are bottom-right aligned: query i of Nq sees key j iff j <= i + (Nk - Nq); for
Nq == Nk this is `offs_m >= offs_n` (kernels/flash_attention.py:152).
Rows that see no key get o = 0 and lse = -inf.
"""
import math

import torch


def _scale(d, sm_scale):
    return 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)


def causal_mask(nq, nk, device=None):
    """Boolean [nq, nk] mask of visible (query, key) pairs, bottom-right aligned."""
    i = torch.arange(nq, device=device).unsqueeze(1)
    j = torch.arange(nk, device=device).unsqueeze(0)
    return j <= i + (nk - nq)


def attention_reference(q, k, v, causal=False, sm_scale=None, *, dtype=torch.float64):
    """Closed form o = softmax(q k^T * s) v and lse, in `dtype`.

    q: [..., Nq, D], k/v: [..., Nk, D] (leading dims broadcast). This is the
    reference's test oracle F.scaled_dot_product_attention
    (kernels/tests/test_flash_attention.py:47) written out, plus the logsumexp
    the training forward stores (kernels/flash_attention_backward.py:157-169).
    """
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    nq, nk, d = q.shape[-2], k.shape[-2], q.shape[-1]
    s = torch.matmul(q, k.transpose(-1, -2)) * _scale(d, sm_scale)
    if causal:
        s = s.masked_fill(~causal_mask(nq, nk, s.device), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse.unsqueeze(-1))
    p = torch.nan_to_num(p, nan=0.0)  # rows that see no key: -inf - -inf
    return torch.matmul(p, v), lse


def attention_grads(q, k, v, do, causal=False, sm_scale=None, *, dtype=torch.float64):
    """(dq, dk, dv) of attention_reference by autograd in `dtype`, the
    reference's gradient oracle (SDPA autograd,
    kernels/tests/test_flash_attention_backward.py:78-91)."""
    qd, kd, vd = (t.detach().to(dtype).requires_grad_() for t in (q, k, v))
    o, _ = attention_reference(qd, kd, vd, causal, sm_scale, dtype=dtype)
    o.backward(do.to(dtype))
    return qd.grad, kd.grad, vd.grad


def bwd_delta(o, do, *, dtype=torch.float64):
    """delta_i = rowsum(dO_i * O_i) (kernels/flash_attention_backward.py:228)."""
    return (o.to(dtype) * do.to(dtype)).sum(-1)


def flash_forward_tiled(q, k, v, causal=False, sm_scale=None, *, block_n=64, p_dtype=None):
    """Restatement of the reference's online-softmax tile loop
    (kernels/flash_attention.py:135-179) in fp32 on the CPU: per key tile,
    s = dot * scale (:148), mask to -inf (:150-153), m_new = max(m, rowmax(s)),
    p = exp(s - m_new), alpha = exp(m - m_new), l = alpha*l + sum(p)
    (:157-162), acc = acc*alpha + p.to(p_dtype) @ v (:168), o = acc / l (:175),
    L = m + ln(l) (kernels/flash_attention_backward.py:162).

    All query rows are processed together (the reference splits them into
    BLOCK_M tiles; rows are independent, so the result is the same). p_dtype
    is the dtype p is rounded to before the PV product (v's dtype in the
    reference); None keeps fp32.
    """
    qf, kf, vf = q.float(), k.float(), v.float()
    nq, nk, d = q.shape[-2], k.shape[-2], q.shape[-1]
    scale = _scale(d, sm_scale)
    lead, dev = q.shape[:-2], q.device
    m = torch.full((*lead, nq), float("-inf"), device=dev)
    l = torch.zeros((*lead, nq), device=dev)
    acc = torch.zeros((*lead, nq, vf.shape[-1]), device=dev)
    rows = torch.arange(nq, device=dev).unsqueeze(1)
    for start in range(0, nk, block_n):
        kt, vt = kf[..., start:start + block_n, :], vf[..., start:start + block_n, :]
        s = torch.matmul(qf, kt.transpose(-1, -2)) * scale
        cols = torch.arange(start, start + kt.shape[-2], device=dev).unsqueeze(0)
        if causal:
            s = s.masked_fill(cols > rows + (nk - nq), float("-inf"))
        m_new = torch.maximum(m, s.amax(-1))
        m_use = torch.where(m_new == float("-inf"), torch.zeros_like(m_new), m_new)
        p = torch.exp(s - m_use.unsqueeze(-1))
        alpha = torch.exp(m - m_use)
        l = alpha * l + p.sum(-1)
        pr = p if p_dtype is None else p.to(p_dtype).float()
        acc = acc * alpha.unsqueeze(-1) + torch.matmul(pr, vt)
        m = m_new
    safe_l = torch.where(l > 0, l, torch.ones_like(l))
    o = torch.where(l.unsqueeze(-1) > 0, acc / safe_l.unsqueeze(-1), torch.zeros_like(acc))
    lse = torch.where(l > 0, m + torch.log(safe_l), torch.full_like(l, float("-inf")))
    return o, lse


def flash_backward_tiled(q, k, v, o, lse, do, causal=False, sm_scale=None, *, block_n=64, op_dtype=None):
    """Restatement of the reference's recomputation backward
    (kernels/flash_attention_backward.py:211-330) in fp32 on the CPU, key tile
    by key tile: delta = rowsum(dO*O) (:228); P = exp(S - L), masked to 0
    (:314); dV += P^T(op_dtype) dO (:316); dP = dO V^T (:318);
    dS = (P * (dP - delta)).to(op_dtype) (:319); dK += dS^T Q * scale (:321);
    dQ += dS K * scale (:323-325). op_dtype None keeps fp32 throughout.
    """
    qf, kf, vf, of, dof = (t.float() for t in (q, k, v, o, do))
    nq, nk, d = q.shape[-2], k.shape[-2], q.shape[-1]
    scale = _scale(d, sm_scale)
    rnd = (lambda t: t) if op_dtype is None else (lambda t: t.to(op_dtype).float())
    delta = (dof * of).sum(-1)
    lse = lse.float()
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    rows = torch.arange(nq, device=q.device).unsqueeze(1)
    for start in range(0, nk, block_n):
        end = min(start + block_n, nk)
        kt, vt = kf[..., start:end, :], vf[..., start:end, :]
        s = torch.matmul(qf, kt.transpose(-1, -2)) * scale
        p = torch.exp(s - lse.unsqueeze(-1))
        if causal:
            cols = torch.arange(start, end, device=q.device).unsqueeze(0)
            p = p.masked_fill(cols > rows + (nk - nq), 0.0)
        dv[..., start:end, :] = torch.matmul(rnd(p).transpose(-1, -2), dof)
        dp = torch.matmul(dof, vt.transpose(-1, -2))
        ds = rnd(p * (dp - delta.unsqueeze(-1)))
        dk[..., start:end, :] = torch.matmul(ds.transpose(-1, -2), qf) * scale
        dq += torch.matmul(ds, kt) * scale
    return dq, dk, dv


def varlen_reference(q, k, v, cu_seqlens_q, cu_seqlens_k, causal=True, sm_scale=None, *, dtype=torch.float64):
    """Packed varlen GQA attention: q [Tq, Hq, D], k/v [Tk, Hkv, D]; query head
    h uses kv head h // (Hq // Hkv), the reference's repeat_interleave
    convention (benchmarks/profiling/roofline/measure_roofline.py:94-98).
    Returns (o [Tq, Hq, D], lse [Hq, Tq]) in `dtype`."""
    hq, hkv = q.shape[1], k.shape[1]
    group = hq // hkv
    scale = _scale(q.shape[-1], sm_scale)
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    o = torch.zeros(q.shape, dtype=dtype)
    lse = torch.zeros((hq, q.shape[0]), dtype=dtype)
    for b in range(len(cq) - 1):
        qb = q[cq[b]:cq[b + 1]].transpose(0, 1)
        kb = k[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, dim=0)
        vb = v[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, dim=0)
        ob, lb = attention_reference(qb, kb, vb, causal, scale, dtype=dtype)
        o[cq[b]:cq[b + 1]] = ob.transpose(0, 1).cpu()
        lse[:, cq[b]:cq[b + 1]] = lb.cpu()
    return o, lse


def naive_attention(q, k, v, causal=False, sm_scale=None, group=1):
    """Pure-Python loops over nested lists (tiny inputs only); an implementation
    independent of torch used to pin attention_reference.

    q: [H][Nq][D], k/v: [H // group][Nk][D]. Returns (o [H][Nq][D], lse [H][Nq]).
    """
    heads, nq, d = len(q), len(q[0]), len(q[0][0])
    nk = len(k[0])
    scale = 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)
    o_all, lse_all = [], []
    for h in range(heads):
        kh, vh = k[h // group], v[h // group]
        o_h, lse_h = [], []
        for i in range(nq):
            vis = [j for j in range(nk) if (not causal) or j <= i + (nk - nq)]
            if not vis:
                o_h.append([0.0] * len(vh[0]) if nk else [0.0] * d)
                lse_h.append(float("-inf"))
                continue
            sc = [sum(q[h][i][t] * kh[j][t] for t in range(d)) * scale for j in vis]
            mx = max(sc)
            ex = [math.exp(s - mx) for s in sc]
            tot = sum(ex)
            o_h.append([sum(ex[a] * vh[j][c] for a, j in enumerate(vis)) / tot for c in range(len(vh[0]))])
            lse_h.append(mx + math.log(tot))
        o_all.append(o_h)
        lse_all.append(lse_h)
    return o_all, lse_all


def paged_decode_reference(q, k_cache, v_cache, block_tables, seq_lens, sm_scale=None, *, dtype=torch.float64):
    """Decode attention over a paged KV cache: for each sequence b, gather its
    seq_lens[b] tokens through block_tables[b] (entry i holds tokens
    [i*block_size, (i+1)*block_size), engine/block_manager.py:56-60), expand
    the KV heads to the query heads (h -> h // group) and apply
    attention_reference without a mask (the new token sees every cached
    token). q [B, Hq, D]; caches [num_blocks, block_size, Hkv, D].
    Returns (o [B, Hq, D], lse [B, Hq]); a sequence of length 0 gives o = 0,
    lse = -inf."""
    B, Hq, D = q.shape
    bs, Hkv = k_cache.shape[1], k_cache.shape[2]
    group = Hq // Hkv
    outs, lses = [], []
    for b in range(B):
        n = int(seq_lens[b])
        nblk = (n + bs - 1) // bs
        ids = block_tables[b, :nblk].long().cpu()
        k = k_cache.cpu()[ids].reshape(nblk * bs, Hkv, D)[:n].transpose(0, 1).repeat_interleave(group, 0)
        v = v_cache.cpu()[ids].reshape(nblk * bs, Hkv, D)[:n].transpose(0, 1).repeat_interleave(group, 0)
        if n == 0:
            outs.append(torch.zeros(Hq, D, dtype=dtype))
            lses.append(torch.full((Hq,), float("-inf"), dtype=dtype))
            continue
        o, lse = attention_reference(q[b].cpu().unsqueeze(1), k, v, False, sm_scale, dtype=dtype)
        outs.append(o[:, 0])
        lses.append(lse[:, 0])
    return torch.stack(outs), torch.stack(lses)


def gather_paged(cache, block_table_row, n):
    """The first n token rows [n, Hkv, D] of one sequence in a paged cache
    [num_blocks, block_size, Hkv, D]: entry i of its block-table row holds
    tokens [i*block_size, (i+1)*block_size) (engine/block_manager.py:56-60)."""
    bs = cache.shape[1]
    nblk = (n + bs - 1) // bs
    ids = block_table_row[:nblk].long().cpu()
    return cache.cpu()[ids].reshape(nblk * bs, *cache.shape[2:])[:n]


def paged_prefill_reference(q, k_cache, v_cache, block_tables, cu_seqlens_q, seq_lens_k, causal=True,
                            sm_scale=None, *, dtype=torch.float64):
    """Chunked prefill over a paged KV cache: sequence b's chunk
    q[cu_seqlens_q[b]:cu_seqlens_q[b+1]] attends to its seq_lens_k[b] cached
    keys (gathered with gather_paged), bottom-right causal, KV heads expanded
    h -> h // group. q [Tq, Hq, D]; returns (o [Tq, Hq, D], lse [Hq, Tq]) in
    `dtype`; a query that sees no key gives o = 0, lse = -inf."""
    Tq, Hq, D = q.shape
    group = Hq // k_cache.shape[2]
    cq = [int(x) for x in cu_seqlens_q]
    o = torch.zeros((Tq, Hq, D), dtype=dtype)
    lse = torch.full((Hq, Tq), float("-inf"), dtype=dtype)
    for b in range(len(cq) - 1):
        nq, nk = cq[b + 1] - cq[b], int(seq_lens_k[b])
        if nq == 0 or nk == 0:
            continue
        kb = gather_paged(k_cache, block_tables[b], nk).transpose(0, 1).repeat_interleave(group, 0)
        vb = gather_paged(v_cache, block_tables[b], nk).transpose(0, 1).repeat_interleave(group, 0)
        ob, lb = attention_reference(q[cq[b]:cq[b + 1]].cpu().transpose(0, 1), kb, vb, causal, sm_scale, dtype=dtype)
        o[cq[b]:cq[b + 1]] = ob.transpose(0, 1)
        lse[:, cq[b]:cq[b + 1]] = lb
    return o, lse