"""GPU parity of the packed varlen GQA forward (config 5: chunked prefill over
a cached prefix) against oracle.attention.varlen_reference."""
import math

import pytest
import torch

from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
from oracle.attention import attention_reference, varlen_reference
from lightserve_amd.workloads import make_varlen_inputs
from tests.gates import assert_gate, assert_lse

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("causal", [True, False])
def test_varlen_small(gpu, dtype, causal):
    inp = make_varlen_inputs(device=gpu, batch=3, chunk=70, prefix=(100, 300), heads=(8, 2), D=128)
    q, k, v = (inp[n].to(dtype) for n in ("q", "k", "v"))
    o, lse = flash_attention_varlen_forward(q, k, v, inp["cu_seqlens_q"], inp["cu_seqlens_k"],
                                            inp["max_seqlen_q"], inp["max_seqlen_k"], causal=causal)
    o_ref, lse_ref = varlen_reference(q.cpu(), k.cpu(), v.cpu(), inp["cu_seqlens_q"].cpu(),
                                      inp["cu_seqlens_k"].cpu(), causal=causal)
    if dtype == torch.float32:
        torch.testing.assert_close(o.cpu().double(), o_ref, atol=1e-3, rtol=1e-3)
    else:
        assert_gate(o.cpu(), o_ref, f"varlen {dtype} causal={causal}")
    assert_lse(lse.cpu(), lse_ref, "varlen")


def test_varlen_ragged_and_empty_sequences(gpu):
    """Sequences of length 0, 1 and not a multiple of the tile, including a
    chunk longer than its key range (rows that see no key: o=0, lse=-inf)."""
    torch.manual_seed(3)
    lens_q = [5, 0, 1, 130, 64]
    lens_k = [17, 3, 1, 200, 40]
    cu_q = torch.tensor([0] + list(torch.tensor(lens_q).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lens_k).cumsum(0)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), 4, 64, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(int(cu_k[-1]), 1, 64, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(int(cu_k[-1]), 1, 64, device=gpu, dtype=torch.bfloat16)
    o, lse = flash_attention_varlen_forward(q, k, v, cu_q.to(gpu), cu_k.to(gpu), max(lens_q), max(lens_k))
    o_ref, lse_ref = varlen_reference(q.cpu(), k.cpu(), v.cpu(), cu_q, cu_k, causal=True)
    assert_gate(o.cpu(), o_ref, "ragged varlen")
    assert_lse(lse.cpu(), lse_ref, "ragged varlen")


def test_varlen_config5_full_size(gpu):
    """Config 5 at full size (B=8, 32 q heads over 8 kv heads, 512-token
    chunks after 1024-8192-token prefixes); oracle in fp32 on the GPU."""
    inp = make_varlen_inputs(device=gpu)
    q, k, v = inp["q"], inp["k"], inp["v"]
    cu_q, cu_k = inp["cu_seqlens_q"], inp["cu_seqlens_k"]
    o, lse = flash_attention_varlen_forward(q, k, v, cu_q, cu_k, inp["max_seqlen_q"], inp["max_seqlen_k"])
    cq, ck = cu_q.tolist(), cu_k.tolist()
    group = q.shape[1] // k.shape[1]
    for b in range(len(cq) - 1):
        qb = q[cq[b]:cq[b + 1]].transpose(0, 1)
        kb = k[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, 0)
        vb = v[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(group, 0)
        ob, lb = attention_reference(qb, kb, vb, True, dtype=torch.float32)
        assert_gate(o[cq[b]:cq[b + 1]].transpose(0, 1), ob, f"config 5 seq {b}")
        assert_lse(lse[:, cq[b]:cq[b + 1]], lb, f"config 5 seq {b}")


def _varlen_poisoned(q, k, v, cu_q, cu_k, max_q, max_k, causal):
    """The varlen forward through the C ABI into NaN-filled o and lse, so a
    (sequence, head, query tile) that no workgroup takes shows as NaN."""
    from lightserve_amd import _lib
    from lightserve_amd.kernels.flash_attention import lse_args
    Tq, Hq, D = q.shape
    o = torch.full_like(q, float("nan"))
    lse = torch.full((Hq, Tq), float("nan"), device=q.device, dtype=torch.float32)
    lse_ptr, _ = lse_args(lse)
    args = _lib.FwdArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), lse=lse_ptr,
        q_stride=_lib.strides_thd(q), k_stride=_lib.strides_thd(k), v_stride=_lib.strides_thd(v),
        o_stride=_lib.strides_thd(o), lse_stride=_lib._i64x3(0, lse.stride(0), lse.stride(1)),
        cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_k=cu_k.data_ptr(),
        dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=cu_q.numel() - 1, heads_q=Hq, heads_kv=k.shape[1],
        seqlen_q=max_q, seqlen_k=max_k, head_dim=D, causal=int(causal), sm_scale=1.0 / math.sqrt(D), reserved=0)
    with torch.cuda.device(q.device):
        _lib.fwd(args, _lib.current_stream(q.device))
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("B,Hq,Hkv,causal,long_q,dtype", [(64, 8, 2, True, False, torch.bfloat16),
                                                           (65, 8, 2, True, False, torch.bfloat16),
                                                           (40, 6, 3, False, False, torch.bfloat16),
                                                           (23, 16, 4, True, False, torch.bfloat16),
                                                           (1, 24, 8, True, False, torch.bfloat16),
                                                           (64, 8, 2, True, True, torch.bfloat16),
                                                           (65, 8, 2, True, True, torch.bfloat16),
                                                           (23, 16, 4, True, True, torch.bfloat16),
                                                           (40, 6, 3, False, True, torch.bfloat16),
                                                           (23, 16, 4, True, True, torch.float16),
                                                           (40, 6, 3, False, True, torch.float16)])
def test_varlen_every_item_once(gpu, B, Hq, Hkv, causal, long_q, dtype):
    """Batches of up to 64 sequences take their (sequence, query tile) items
    longest-first, found per workgroup from cu_seqlens; longer batches keep
    the head-major order. Lengths mix empty chunks, chunks longer than their
    keys, and tile-edge sizes; query heads are or are not a multiple of the
    8 XCDs. With runs of 512 queries or more (long_q) batches of up to 64
    sequences take 256-row tiles (8-wave workgroups), so the lengths also
    straddle 256-row edges. Every output row must be written once and match
    the oracle."""
    print(f"case varlen order B={B} Hq={Hq} Hkv={Hkv} causal={causal} long_q={long_q} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + Hq + (7 if long_q else 0))
    choices_q = [0, 1, 64, 127, 128, 129, 200, 256, 300]
    if long_q:
        choices_q = [0, 1, 129, 255, 256, 257, 511, 512, 700]
    lens_q = [choices_q[int(i)] for i in torch.randint(0, len(choices_q), (B,), generator=g)]
    lens_k = [max(0, lq + int(d)) for lq, d in zip(lens_q, torch.randint(-150, 500, (B,), generator=g))]
    if B == 1:
        lens_q, lens_k = [300], [1100]
    if long_q:
        lens_q[0] = 700  # at least one run of 512 or more
    cu_q = torch.tensor([0] + torch.tensor(lens_q).cumsum(0).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + torch.tensor(lens_k).cumsum(0).tolist(), dtype=torch.int32)
    D = 64
    q = torch.randn(int(cu_q[-1]), Hq, D, generator=g).to(dtype)
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dtype)
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dtype)
    o, lse = _varlen_poisoned(q.to(gpu), k.to(gpu), v.to(gpu), cu_q.to(gpu), cu_k.to(gpu),
                              max(lens_q), max(lens_k), causal)
    assert not torch.isnan(o).any(), "output rows left unwritten"
    assert not torch.isnan(lse).any(), "lse rows left unwritten"
    o_ref, lse_ref = varlen_reference(q, k, v, cu_q, cu_k, causal=causal)
    assert_gate(o.cpu(), o_ref, f"varlen order B={B}")
    assert_lse(lse.cpu(), lse_ref, f"varlen order B={B}")


def test_varlen_random_batches(gpu):
    """Seeded random batches through both launch shapes (4-wave and, with runs
    of 512 queries or more, 8-wave workgroups) and both orders (up to 64
    sequences longest-first, more head-major): batch sizes 1-70, ragged and
    empty chunks, chunks longer than their keys, GQA groups 1-8, head dims
    64/96/128, bf16/fp16, causal or not. Every row must be written once
    (NaN-poisoned outputs) and match the oracle."""
    rng = torch.Generator().manual_seed(2024)
    ri = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=rng))
    for case in range(24):
        # modes bound the fp64 oracle's work: few long runs (8-wave), many
        # short sequences (past the 64-sequence limit), or in between
        mode = case % 3
        B = ri(1, 6) if mode == 0 else (ri(40, 70) if mode == 1 else ri(1, 20))
        qmax, kextra = (900, 700) if mode == 0 else ((100, 150) if mode == 1 else (300, 400))
        Hkv = [1, 2, 4][ri(0, 2)]
        G = [1, 2, 3, 4, 8][ri(0, 4)]
        D = [64, 96, 128][ri(0, 2)]
        dtype = [torch.bfloat16, torch.float16][ri(0, 1)]
        causal = bool(ri(0, 1))
        lens_q = torch.randint(0, qmax + 1, (B,), generator=rng).tolist()
        if mode == 0:
            lens_q[0] = max(lens_q[0], 512)
        lens_k = [max(0, lq + int(d)) for lq, d in zip(lens_q, torch.randint(-qmax // 8, kextra, (B,), generator=rng))]
        print(f"case varlen random {case}: B={B} Hq={Hkv * G} Hkv={Hkv} D={D} {dtype} causal={causal} "
              f"max_q={max(lens_q)}", flush=True)
        cu_q = torch.tensor([0] + torch.tensor(lens_q).cumsum(0).tolist(), dtype=torch.int32)
        cu_k = torch.tensor([0] + torch.tensor(lens_k).cumsum(0).tolist(), dtype=torch.int32)
        if int(cu_q[-1]) == 0:
            continue
        q = torch.randn(int(cu_q[-1]), Hkv * G, D, generator=rng).to(dtype)
        k = torch.randn(max(int(cu_k[-1]), 1), Hkv, D, generator=rng).to(dtype)
        v = torch.randn(max(int(cu_k[-1]), 1), Hkv, D, generator=rng).to(dtype)
        o, lse = _varlen_poisoned(q.to(gpu), k.to(gpu), v.to(gpu), cu_q.to(gpu), cu_k.to(gpu),
                                  max(lens_q), max(max(lens_k), 1), causal)
        assert not torch.isnan(o).any(), f"case {case}: output rows left unwritten"
        assert not torch.isnan(lse).any(), f"case {case}: lse rows left unwritten"
        o_ref, lse_ref = varlen_reference(q, k, v, cu_q, cu_k, causal=causal)
        assert_gate(o.cpu(), o_ref, f"varlen random {case}")
        assert_lse(lse.cpu(), lse_ref, f"varlen random {case}")


def _varlen_grad_reference(q, k, v, do, lens_q, lens_k, causal, scale):
    """Per sequence: the oracle's forward and float64 gradients on K/V
    repeated over each group (query head h reads KV head h // G), dK/dV
    summed over the group; plus the reference algorithm's gradients."""
    from oracle.attention import attention_grads, attention_reference, flash_backward_tiled
    Hq, Hkv, D = q.shape[1], k.shape[1], q.shape[2]
    G = Hq // Hkv
    outs = {n: [] for n in ("o", "dq", "dk", "dv", "aq", "ak", "av")}
    cq = ck = 0
    for nq, nk in zip(lens_q, lens_k):
        qb, dob = (t[cq:cq + nq].transpose(0, 1)[None] for t in (q, do))
        kb, vb = (t[ck:ck + nk].transpose(0, 1)[None].repeat_interleave(G, dim=1) for t in (k, v))
        o_r, l_r = attention_reference(qb, kb, vb, causal, scale)
        ex = attention_grads(qb, kb, vb, dob, causal, scale)
        al = flash_backward_tiled(qb, kb, vb, o_r.nan_to_num().to(q.dtype), l_r, dob, causal, scale, op_dtype=q.dtype)
        grp = lambda t: t.reshape(1, Hkv, G, nk, D).sum(2)[0].transpose(0, 1)  # noqa: E731
        outs["o"].append(o_r.nan_to_num()[0].transpose(0, 1))
        outs["dq"].append(ex[0].nan_to_num()[0].transpose(0, 1))
        outs["aq"].append(al[0].nan_to_num()[0].transpose(0, 1))
        outs["dk"].append(grp(ex[1].nan_to_num()))
        outs["ak"].append(grp(al[1].nan_to_num()))
        outs["dv"].append(grp(ex[2].nan_to_num()))
        outs["av"].append(grp(al[2].nan_to_num()))
        cq += nq
        ck += nk
    return {n: torch.cat(v, dim=0) for n, v in outs.items()}


@pytest.mark.parametrize("lens_q,lens_k,Hq,Hkv,D,causal,dtype", [
    ([300, 0, 77, 513], [300, 40, 200, 513], 8, 2, 128, True, torch.bfloat16),
    ([128, 1000, 64], [1100, 1000, 0], 4, 4, 64, True, torch.float16),
    ([17, 250, 129], [400, 250, 33], 6, 3, 96, False, torch.bfloat16),
    ([1, 700, 2], [1, 900, 5], 32, 8, 128, True, torch.float16),
    ([4160, 96], [4160, 300], 4, 1, 128, True, torch.bfloat16),
    ([90, 33], [120, 33], 4, 2, 12, True, torch.bfloat16),
    ([65, 200], [65, 150], 2, 1, 40, False, torch.float16)])
def test_varlen_backward(gpu, lens_q, lens_k, Hq, Hkv, D, causal, dtype):
    """Packed varlen (and GQA) forward + backward through the autograd
    wrapper against the oracle per sequence (bottom-right causal, empty
    sequences, Nq != Nk, rows that see no key, head dims the wrapper pads to a
    multiple of 8 in both directions)."""
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen
    from tests.gates import assert_grad_parity
    print(f"case varlen bwd lens_q={lens_q} lens_k={lens_k} {Hq}/{Hkv} D={D} causal={causal} {dtype}", flush=True)
    g = torch.Generator().manual_seed(sum(lens_q) + Hq)
    Tq, Tk = sum(lens_q), sum(lens_k)
    q, do = (torch.randn(Tq, Hq, D, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(Tk, Hkv, D, generator=g).to(dtype) for _ in range(2))
    cu = lambda ls: torch.tensor([0] + list(torch.tensor(ls).cumsum(0)), dtype=torch.int32, device=gpu)  # noqa: E731
    scale = D ** -0.5
    qg, kg, vg = (t.to(gpu).requires_grad_() for t in (q, k, v))
    o = flash_attention_varlen(qg, kg, vg, cu(lens_q), cu(lens_k), max(lens_q), max(lens_k), causal, scale)
    o.backward(do.to(gpu))
    torch.cuda.synchronize()
    ref = _varlen_grad_reference(q, k, v, do, lens_q, lens_k, causal, scale)
    assert_gate(o.detach().cpu(), ref["o"], "varlen o")
    for name, got, ex, al in (("dq", qg.grad, ref["dq"], ref["aq"]), ("dk", kg.grad, ref["dk"], ref["ak"]),
                              ("dv", vg.grad, ref["dv"], ref["av"])):
        assert got.shape == ex.shape, name
        assert_grad_parity(got.cpu(), ex, al, f"varlen {name}")


def test_varlen_backward_no_queries(gpu):
    """A batch with no query rows: every gradient is zero (no launch)."""
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_backward
    q = torch.empty(0, 4, 64, device=gpu, dtype=torch.bfloat16)
    k, v = (torch.randn(50, 2, 64, device=gpu).bfloat16() for _ in range(2))
    lse = torch.empty(4, 0, device=gpu, dtype=torch.float32)
    cu_q = torch.zeros(3, dtype=torch.int32, device=gpu)
    cu_k = torch.tensor([0, 20, 50], dtype=torch.int32, device=gpu)
    dq, dk, dv = flash_attention_varlen_backward(q, q, k, v, q, lse, cu_q, cu_k, 0, 30, True)
    assert dq.shape == q.shape and torch.count_nonzero(dk) == 0 and torch.count_nonzero(dv) == 0


def test_varlen_backward_validation(gpu):
    """The varlen backward makes the forward's checks before any launch:
    int64 or host cu_seqlens, unequal cu_seqlens lengths, head counts that
    do not group, a wrong lse shape; fp32 inputs that require grad are refused
    by the differentiable entry point before its forward runs."""
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen, flash_attention_varlen_backward
    q = torch.randn(40, 4, 64, device=gpu).bfloat16()
    k = torch.randn(50, 2, 64, device=gpu).bfloat16()
    lse = torch.zeros(4, 40, device=gpu)
    cu_q = torch.tensor([0, 20, 40], dtype=torch.int32, device=gpu)
    cu_k = torch.tensor([0, 20, 50], dtype=torch.int32, device=gpu)
    bad = [
        dict(cu_seqlens_q=cu_q.long()),
        dict(cu_seqlens_k=cu_k.cpu()),
        dict(cu_seqlens_k=cu_k[:2]),
        dict(k=torch.randn(50, 3, 64, device=gpu).bfloat16(), v=torch.randn(50, 3, 64, device=gpu).bfloat16()),
        dict(lse=torch.zeros(40, 4, device=gpu)),
        dict(do=q.cpu()),
    ]
    for over in bad:
        a = dict(do=q, q=q, k=k, v=k, o=q, lse=lse, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=20,
                 max_seqlen_k=30)
        a.update(over)
        with pytest.raises(AssertionError):
            flash_attention_varlen_backward(**a)
    qf = torch.randn(40, 4, 64, device=gpu, requires_grad=True)
    kf = torch.randn(50, 2, 64, device=gpu)
    with pytest.raises(AssertionError):
        flash_attention_varlen(qf, kf, kf, cu_q, cu_k, 20, 30)
    with torch.no_grad():  # no gradient wanted: the fp32 forward runs
        o = flash_attention_varlen(qf, kf, kf, cu_q, cu_k, 20, 30)
    assert o.shape == qf.shape
