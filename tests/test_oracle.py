"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Checks, per oracle function:
  attention_reference  vs pure-Python loop fixtures (tests/golden), closed-form
                       invariants, torch SDPA (float64);
  attention_grads      float64 gradcheck;
  flash_forward_tiled  (restated reference tile loop) vs attention_reference;
  flash_backward_tiled (restated reference backward) vs attention_grads;
  bwd_delta            vs the identity delta_i = sum_j P_ij dP_ij;
  varlen_reference     vs pure-Python loops with GQA;
  paged_decode_reference vs pure-Python loops on a cache the test scatters
                       itself, and invariance under a block permutation;
  paged_prefill_reference vs pure-Python loops (ragged chunks, GQA, empty
                       chunks and sequences), a block permutation, and the
                       chunking invariant: prefilling a sequence chunk by
                       chunk gives the rows of one causal pass over all of it;
and planted mistakes in copies of the oracle must fail these checks.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import (attention_grads, attention_reference, bwd_delta, causal_mask,
                              flash_backward_tiled, flash_forward_tiled, naive_attention,
                              gather_paged, paged_decode_reference, paged_prefill_reference, varlen_reference)
from lightserve_amd.workloads import CONFIGS, make_config_inputs, make_varlen_inputs, varlen_fwd_flops

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)  # allow_pickle stays False


def _tiny_names(golden):
    return sorted({k.split("/")[0] for k in golden.files if not k.startswith("cfg1")})


def test_golden_tiny_cases(golden):
    names = _tiny_names(golden)
    assert len(names) == 8
    for name in names:
        H, Hkv, nq, nk, d, causal, scale = golden[f"{name}/meta"].tolist()
        scale = None if scale < 0 else scale
        q, k, v = (torch.from_numpy(golden[f"{name}/{t}"]) for t in "qkv")
        group = int(H) // int(Hkv)
        k_rep = k.repeat_interleave(group, dim=0)
        v_rep = v.repeat_interleave(group, dim=0)
        o, lse = attention_reference(q, k_rep, v_rep, bool(causal), scale)
        np.testing.assert_allclose(o.numpy(), golden[f"{name}/o"], atol=1e-12, rtol=1e-12, err_msg=name)
        np.testing.assert_allclose(lse.numpy(), golden[f"{name}/lse"], atol=1e-12, rtol=1e-12, err_msg=name)


def test_golden_config1(golden):
    """Config 1 (the CPU plumbing case): inputs regenerate bit-identically from
    the seed, and the float64 oracle matches the pure-Python loop outputs."""
    import hashlib
    inp = make_config_inputs(1)
    for i, n in enumerate("qkv"):
        assert hashlib.sha256(inp[n].contiguous().numpy().tobytes()).hexdigest() == golden["cfg1/sha256"][i]
    o, lse = attention_reference(inp["q"], inp["k"], inp["v"], causal=True)
    np.testing.assert_allclose(lse[0].numpy(), golden["cfg1/lse"], atol=1e-10)
    np.testing.assert_allclose(o[0, :, ::8, :].numpy(), golden["cfg1/o_rows"], atol=1e-10)
    np.testing.assert_allclose([o.sum().item(), (o * o).sum().item()], golden["cfg1/o_sum"], rtol=1e-10)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(7, 7), (5, 11)])
def test_invariant_zero_query(causal, nq, nk):
    """q = 0: every visible key scores 0, so o is the mean of the visible v rows
    and lse = ln(#visible keys)."""
    g = torch.Generator().manual_seed(5)
    q = torch.zeros(2, nq, 16, dtype=torch.float64)
    k = torch.randn(2, nk, 16, generator=g, dtype=torch.float64)
    v = torch.randn(2, nk, 16, generator=g, dtype=torch.float64)
    o, lse = attention_reference(q, k, v, causal)
    for i in range(nq):
        n_vis = min(nk, i + 1 + nk - nq) if causal else nk
        torch.testing.assert_close(o[:, i], v[:, :n_vis].mean(1), atol=1e-12, rtol=0)
        torch.testing.assert_close(lse[:, i], torch.full((2,), math.log(n_vis), dtype=torch.float64))


def test_invariant_causal_first_row():
    """Causal, Nq == Nk: row 0 sees only key 0, so o_0 = v_0 and L_0 = s*q_0.k_0."""
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(3, 9, 8, generator=g, dtype=torch.float64) for _ in range(3))
    o, lse = attention_reference(q, k, v, causal=True, sm_scale=0.3)
    torch.testing.assert_close(o[:, 0], v[:, 0], atol=1e-14, rtol=0)
    torch.testing.assert_close(lse[:, 0], 0.3 * (q[:, 0] * k[:, 0]).sum(-1), atol=1e-14, rtol=0)


@pytest.mark.parametrize("shape", [(1, 1, 17, 32), (2, 2, 64, 64), (1, 4, 130, 64), (1, 2, 100, 96)])
@pytest.mark.parametrize("causal", [False, True])
def test_matches_sdpa_float64(shape, causal):
    """Library routine: torch SDPA (the reference's own oracle) in float64."""
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(*shape, generator=g, dtype=torch.float64) for _ in range(3))
    o, _ = attention_reference(q, k, v, causal)
    torch.testing.assert_close(o, F.scaled_dot_product_attention(q, k, v, is_causal=causal), atol=1e-12, rtol=1e-12)


def test_lse_is_logsumexp_of_masked_scores():
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(2, 6, 10, 8, generator=g, dtype=torch.float64) for _ in range(3))
    _, lse = attention_reference(q, k, v, True, 0.5)
    s = (q @ k.transpose(-1, -2)) * 0.5
    expect = torch.stack([torch.logsumexp(s[..., i, : i + 1], -1) for i in range(10)], -1)
    torch.testing.assert_close(lse, expect, atol=1e-13, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_grads_gradcheck(causal):
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 2, 6, 4, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda a, b, c: attention_reference(a, b, c, causal)[0], (q, k, v))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(130, 130), (70, 150)])
def test_tiled_forward_restatement(causal, nq, nk):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 3, nq, 64, generator=g)
    k = torch.randn(2, 3, nk, 64, generator=g)
    v = torch.randn(2, 3, nk, 64, generator=g)
    o_ref, l_ref = attention_reference(q, k, v, causal)
    o, l = flash_forward_tiled(q, k, v, causal, block_n=32)
    torch.testing.assert_close(o.double(), o_ref, atol=2e-6, rtol=0)
    torch.testing.assert_close(l.double(), l_ref, atol=2e-6, rtol=0)
    # p rounded to bf16 before PV (the reference's p.to(v.dtype)) stays inside the max-abs 2e-2 / mean-abs 2e-3 gate
    ob, _ = flash_forward_tiled(q, k, v, causal, block_n=32, p_dtype=torch.bfloat16)
    err = (ob.double() - o_ref).abs()
    assert err.max() < 2e-2 and err.mean() < 2e-3


@pytest.mark.parametrize("causal", [False, True])
def test_tiled_backward_restatement(causal):
    g = torch.Generator().manual_seed(10)
    q, k, v, do = (torch.randn(2, 2, 100, 32, generator=g) for _ in range(4))
    o, lse = attention_reference(q, k, v, causal)
    dq_r, dk_r, dv_r = attention_grads(q, k, v, do, causal)
    dq, dk, dv = flash_backward_tiled(q, k, v, o.float(), lse.float(), do, causal, block_n=32)
    for got, ref in ((dq, dq_r), (dk, dk_r), (dv, dv_r)):
        torch.testing.assert_close(got.double(), ref, atol=2e-5, rtol=0)


def test_varlen_matches_loops():
    g = torch.Generator().manual_seed(11)
    cu_q = torch.tensor([0, 3, 5, 9], dtype=torch.int32)
    cu_k = torch.tensor([0, 7, 9, 18], dtype=torch.int32)
    q = torch.randn(9, 4, 8, generator=g, dtype=torch.float64)
    k = torch.randn(18, 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(18, 2, 8, generator=g, dtype=torch.float64)
    o, lse = varlen_reference(q, k, v, cu_q, cu_k, causal=True)
    for b in range(3):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        on, ln = naive_attention(q[qs:qe].transpose(0, 1).tolist(), k[ks:ke].transpose(0, 1).tolist(),
                                 v[ks:ke].transpose(0, 1).tolist(), True, None, group=2)
        np.testing.assert_allclose(o[qs:qe].transpose(0, 1).numpy(), np.array(on), atol=1e-12)
        np.testing.assert_allclose(lse[:, qs:qe].numpy(), np.array(ln), atol=1e-12)


def _scatter_cache(seqs_k, seqs_v, block_size, num_blocks, perm):
    """Writes each sequence's K/V [n, Hkv, D] into a cache through a block
    table that hands out the physical blocks in the order `perm`."""
    hkv, d = seqs_k[0].shape[1:]
    kc = torch.zeros(num_blocks, block_size, hkv, d, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    max_blocks = max((k.shape[0] + block_size - 1) // block_size for k in seqs_k)
    table = torch.full((len(seqs_k), max(max_blocks, 1)), -1, dtype=torch.int32)
    nxt = 0
    for b, (k, v) in enumerate(zip(seqs_k, seqs_v)):
        for t in range(k.shape[0]):
            if t % block_size == 0:
                table[b, t // block_size] = perm[nxt]
                nxt += 1
            kc[table[b, t // block_size], t % block_size] = k[t]
            vc[table[b, t // block_size], t % block_size] = v[t]
    return kc, vc, table


def test_paged_decode_matches_loops():
    g = torch.Generator().manual_seed(13)
    lens, hq, hkv, d, bs = [5, 0, 9, 4], 4, 2, 8, 4
    seqs_k = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens]
    seqs_v = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens]
    q = torch.randn(len(lens), hq, d, generator=g, dtype=torch.float64)
    num_blocks = 8
    perm = torch.randperm(num_blocks, generator=g).tolist()
    kc, vc, table = _scatter_cache(seqs_k, seqs_v, bs, num_blocks, perm)
    o, lse = paged_decode_reference(q, kc, vc, table, torch.tensor(lens, dtype=torch.int32), 0.3)
    for b, n in enumerate(lens):
        on, ln = naive_attention(q[b].unsqueeze(1).tolist(), seqs_k[b].transpose(0, 1).tolist(),
                                 seqs_v[b].transpose(0, 1).tolist(), False, 0.3, group=hq // hkv)
        if n == 0:
            assert torch.equal(o[b], torch.zeros(hq, d)) and torch.isinf(lse[b]).all()
            continue
        np.testing.assert_allclose(o[b].numpy(), np.array(on)[:, 0], atol=1e-12)
        np.testing.assert_allclose(lse[b].numpy(), np.array(ln)[:, 0], atol=1e-12)


def test_paged_decode_block_permutation():
    g = torch.Generator().manual_seed(17)
    lens, hkv, d, bs = [7, 12, 1], 2, 8, 4
    seqs_k = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens]
    seqs_v = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens]
    q = torch.randn(3, 8, d, generator=g, dtype=torch.float64)
    sl = torch.tensor(lens, dtype=torch.int32)
    a = paged_decode_reference(q, *_scatter_cache(seqs_k, seqs_v, bs, 8, list(range(8))), sl)
    b = paged_decode_reference(q, *_scatter_cache(seqs_k, seqs_v, bs, 8, [7, 3, 5, 0, 6, 1, 2, 4]), sl)
    torch.testing.assert_close(a[0], b[0], atol=1e-14, rtol=0)
    torch.testing.assert_close(a[1], b[1], atol=1e-14, rtol=0)


def test_causal_mask_bottom_right():
    m = causal_mask(2, 4)
    assert m.tolist() == [[True, True, True, False], [True, True, True, True]]
    assert torch.equal(causal_mask(5, 5), torch.ones(5, 5, dtype=torch.bool).tril())


def test_config_recipes():
    a = make_config_inputs(3, shape_override=(1, 2, 64, 32))
    b = make_config_inputs(3, shape_override=(1, 2, 64, 32))
    assert all(torch.equal(a[n], b[n]) for n in ("q", "k", "v", "do"))
    assert a["q"].dtype == torch.bfloat16 and a["q"].float().abs().max() < 4
    c = make_config_inputs(4, shape_override=(1, 2, 400, 16))
    idx = c["scaled_rows"]
    assert idx.numel() == 4
    # the scaled rows carry ~8x the norm of the others
    norms = c["k"].float().norm(dim=-1)[0, 0]
    mask = torch.zeros(400, dtype=torch.bool)
    mask[idx] = True
    assert norms[mask].mean() > 5 * norms[~mask].mean()
    vl = make_varlen_inputs(batch=3, chunk=16, prefix=(10, 20), heads=(4, 2), D=8)
    assert vl["q"].shape == (48, 4, 8) and vl["cu_seqlens_k"][-1] == vl["k"].shape[0]
    assert all(10 <= int(p) <= 20 for p in vl["prefix"])
    assert CONFIGS[5]["Hq"] % CONFIGS[5]["Hkv"] == 0
    # exact varlen FLOPs: brute force pair count
    cu_q, cu_k = vl["cu_seqlens_q"], vl["cu_seqlens_k"]
    pairs = sum(int(causal_mask(int(cu_q[b + 1] - cu_q[b]), int(cu_k[b + 1] - cu_k[b])).sum()) for b in range(3))
    assert varlen_fwd_flops(cu_q, cu_k, 4, 8) == 4 * 8 * 4 * pairs


# --- planted mistakes: each broken copy of the oracle must fail a check above ---

def _broken_scale_twice(q, k, v, causal=False, sm_scale=None):
    d = q.shape[-1]
    s = (1.0 / math.sqrt(d)) if sm_scale is None else sm_scale
    return attention_reference(q, k, v, causal, s * s)


def _broken_transposed_v(q, k, v, causal=False, sm_scale=None):
    o, lse = attention_reference(q, k, v.transpose(-1, -2).contiguous().transpose(-1, -2).flip(-2), causal, sm_scale)
    return o, lse


def _broken_top_left_mask(q, k, v, causal=False, sm_scale=None):
    q64, k64, v64 = q.double(), k.double(), v.double()
    s = (q64 @ k64.transpose(-1, -2)) / math.sqrt(q.shape[-1]) if sm_scale is None else (q64 @ k64.transpose(-1, -2)) * sm_scale
    if causal:
        nq, nk = s.shape[-2:]
        s = s.masked_fill(torch.ones(nq, nk, dtype=torch.bool).triu(1), float("-inf"))
    lse = torch.logsumexp(s, -1)
    return torch.exp(s - lse.unsqueeze(-1)) @ v64, lse


@pytest.mark.parametrize("causal", [False, True])
def test_delta_identity(causal):
    """delta_i = rowsum(dO_i * O_i) equals sum_j P_ij dP_ij with dP = dO V^T,
    because O = P V; the right-hand side never forms O."""
    g = torch.Generator().manual_seed(11)
    q, k, v, do = (torch.randn(2, 3, 19, 16, generator=g, dtype=torch.float64) for _ in range(4))
    o, _ = attention_reference(q, k, v, causal)
    s = (q @ k.transpose(-1, -2)) / math.sqrt(16)
    if causal:
        s = s.masked_fill(~causal_mask(19, 19), float("-inf"))
    p = torch.softmax(s, -1)
    dp = do @ v.transpose(-1, -2)
    torch.testing.assert_close(bwd_delta(o, do), (p * dp).sum(-1), atol=1e-12, rtol=1e-12)
    # a mistake that drops the dO factor is caught
    assert not torch.allclose(o.sum(-1), (p * dp).sum(-1))


@pytest.mark.parametrize("broken", [_broken_scale_twice, _broken_transposed_v, _broken_top_left_mask])
def test_planted_mistakes_are_caught(golden, broken):
    caught = 0
    for name in _tiny_names(golden):
        H, Hkv, nq, nk, d, causal, scale = golden[f"{name}/meta"].tolist()
        q, k, v = (torch.from_numpy(golden[f"{name}/{t}"]) for t in "qkv")
        group = int(H) // int(Hkv)
        o, _ = broken(q, k.repeat_interleave(group, 0), v.repeat_interleave(group, 0), bool(causal),
                      None if scale < 0 else scale)
        if not np.allclose(o.numpy(), golden[f"{name}/o"], atol=1e-9):
            caught += 1
    assert caught > 0, f"{broken.__name__} passed every golden case"


def _prefill_case(seed, lens_k, lens_q, hq, hkv, d, bs, num_blocks, perm):
    g = torch.Generator().manual_seed(seed)
    seqs_k = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens_k]
    seqs_v = [torch.randn(n, hkv, d, generator=g, dtype=torch.float64) for n in lens_k]
    q = torch.randn(sum(lens_q), hq, d, generator=g, dtype=torch.float64)
    cu = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    kc, vc, table = _scatter_cache(seqs_k, seqs_v, bs, num_blocks, perm)
    return q, cu, seqs_k, seqs_v, kc, vc, table


@pytest.mark.parametrize("causal", [True, False])
def test_paged_prefill_matches_loops(causal):
    lens_k, lens_q, hq, hkv, d, bs = [9, 5, 0, 12, 3], [4, 5, 0, 1, 0], 4, 2, 4, 4
    q, cu, seqs_k, seqs_v, kc, vc, table = _prefill_case(21, lens_k, lens_q, hq, hkv, d, bs, 12,
                                                         [5, 0, 11, 2, 7, 9, 1, 3, 10, 4, 6, 8])
    sl = torch.tensor(lens_k, dtype=torch.int32)
    o, lse = paged_prefill_reference(q, kc, vc, table, cu, sl, causal, 0.4)
    for b in range(len(lens_k)):
        rows = slice(int(cu[b]), int(cu[b + 1]))
        if lens_q[b] == 0:
            continue
        if lens_k[b] == 0:
            assert torch.equal(o[rows], torch.zeros_like(o[rows])) and torch.isinf(lse[:, rows]).all()
            continue
        on, ln = naive_attention(q[rows].transpose(0, 1).tolist(), seqs_k[b].transpose(0, 1).tolist(),
                                 seqs_v[b].transpose(0, 1).tolist(), causal, 0.4, group=hq // hkv)
        np.testing.assert_allclose(o[rows].transpose(0, 1).numpy(), np.array(on), atol=1e-12)
        np.testing.assert_allclose(lse[:, rows].numpy(), np.array(ln), atol=1e-12)


def test_paged_prefill_block_permutation():
    args = ([10, 7], [3, 7], 2, 1, 8, 4, 6)
    a = _prefill_case(22, *args, list(range(6)))
    b = _prefill_case(22, *args, [4, 2, 5, 0, 3, 1])
    sl = torch.tensor(args[0], dtype=torch.int32)
    ra = paged_prefill_reference(a[0], a[4], a[5], a[6], a[1], sl)
    rb = paged_prefill_reference(b[0], b[4], b[5], b[6], b[1], sl)
    torch.testing.assert_close(ra[0], rb[0], atol=1e-14, rtol=0)
    torch.testing.assert_close(ra[1], rb[1], atol=1e-14, rtol=0)


def _chunked_prefill(oracle_fn, q_full, kc, vc, table, chunks):
    """Runs a sequence's prefill chunk by chunk: chunk c attends to the keys
    cached so far (its own included). Returns the concatenated outputs."""
    outs, start = [], 0
    for c in chunks:
        cu = torch.tensor([0, c], dtype=torch.int32)
        o, _ = oracle_fn(q_full[start:start + c], kc, vc, table, cu, torch.tensor([start + c], dtype=torch.int32))
        outs.append(o)
        start += c
    return torch.cat(outs)


def test_paged_prefill_chunking_invariant():
    n, hq, hkv, d, bs = 13, 4, 2, 8, 4
    g = torch.Generator().manual_seed(23)
    q = torch.randn(n, hq, d, generator=g, dtype=torch.float64)
    k = torch.randn(n, hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(n, hkv, d, generator=g, dtype=torch.float64)
    kc, vc, table = _scatter_cache([k], [v], bs, 4, [2, 0, 3, 1])
    whole, _ = varlen_reference(q, k, v, torch.tensor([0, n]), torch.tensor([0, n]), causal=True)
    for chunks in ([13], [5, 8], [4, 4, 4, 1], [1] * 13):
        torch.testing.assert_close(_chunked_prefill(paged_prefill_reference, q, kc, vc, table, chunks), whole,
                                   atol=1e-12, rtol=0)

    # planted mistake: top-left causal alignment (query i of a chunk sees keys
    # 0..i, as SDPA's is_causal does for Nq != Nk) breaks the invariant
    def top_left(qc, kc_, vc_, table_, cu, sl):
        nq, nk = qc.shape[0], int(sl[0])
        kk = gather_paged(kc_, table_[0], nk).transpose(0, 1)
        vv = gather_paged(vc_, table_[0], nk).transpose(0, 1)
        kk, vv = kk.repeat_interleave(hq // hkv, 0), vv.repeat_interleave(hq // hkv, 0)
        s = torch.matmul(qc.transpose(0, 1), kk.transpose(-1, -2)) / math.sqrt(d)
        mask = torch.arange(nk).view(1, -1) <= torch.arange(nq).view(-1, 1)
        p = torch.softmax(s.masked_fill(~mask, float("-inf")), -1)
        return torch.matmul(p, vv).transpose(0, 1), None
    bad = _chunked_prefill(top_left, q, kc, vc, table, [5, 8])
    assert (bad - whole).abs().max() > 1e-3
