"""GPU parity of chunked prefill over a paged KV cache (lsfa_prefill_paged).

The reference has no such kernel: its engine documents prefill with more than
one scheduled token as the missing path (engine/request.py:86-93,
engine/scheduler.py:34-44). Parity is against
oracle.attention.paged_prefill_reference (gather through the block table, then
the closed-form attention with the bottom-right causal mask) under the
correctness gate (max-abs 2e-2, mean-abs 2e-3, LSE 1e-3), and, where the cache holds the same K/V as a packed layout,
against the packed varlen forward bit for bit (the paged loads fill the same
LDS tiles). Cases: GQA groups 1/3/4/8, head dims 64/96/128, block sizes
16/32/64, ragged and empty chunks and sequences, single-token chunks, shuffled
physical blocks, the device-side clamp of seq_lens_k, chunk-by-chunk prefill
against one causal pass, and the config-5 shape (B=8, Hq=32, Hkv=8, D=128, 512-token chunks).
"""
import pytest
import torch

from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
from lightserve_amd.kernels.paged_attention import paged_prefill
from oracle.attention import paged_prefill_reference
from tests.gates import assert_gate, assert_lse

pytestmark = pytest.mark.gpu


def _make_case(lens_k, lens_q, hq, hkv, d, bs, dtype, seed, extra_blocks=3):
    """Random cache with every sequence's blocks scattered over a shuffled
    pool, and packed query chunks (chunk b has lens_q[b] <= lens_k[b] rows)."""
    g = torch.Generator().manual_seed(seed)
    nblk = [(n + bs - 1) // bs for n in lens_k]
    num_blocks = sum(nblk) + extra_blocks
    perm = torch.randperm(num_blocks, generator=g)
    table = torch.zeros(len(lens_k), max(max(nblk), 1), dtype=torch.int32)
    at = 0
    for b, k in enumerate(nblk):
        table[b, :k] = perm[at:at + k].to(torch.int32)
        at += k
    kc = (torch.randn(num_blocks, bs, hkv, d, generator=g) * 0.5).to(dtype)
    vc = torch.randn(num_blocks, bs, hkv, d, generator=g).to(dtype)
    q = (torch.randn(sum(lens_q), hq, d, generator=g) * 0.5).to(dtype)
    cu = torch.tensor([0] + [sum(lens_q[:i + 1]) for i in range(len(lens_q))], dtype=torch.int32)
    return q, kc, vc, table, cu, torch.tensor(lens_k, dtype=torch.int32)


def _run(q, kc, vc, table, cu, sl, causal=True, **kw):
    o, lse = paged_prefill(q.cuda(), kc.cuda(), vc.cuda(), table.cuda(), cu.cuda(), sl.cuda(), causal=causal,
                           return_lse=True, **kw)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu()


def _check(case, label, causal=True, lens_ref=None, **kw):
    q, kc, vc, table, cu, sl = case
    o, lse = _run(q, kc, vc, table, cu, sl, causal, **kw)
    o_ref, lse_ref = paged_prefill_reference(q, kc, vc, table, cu, sl if lens_ref is None else lens_ref, causal,
                                             kw.get("sm_scale"))
    assert_gate(o, o_ref, f"{label} o")
    seen = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse), seen), label
    if seen.any():
        assert_lse(lse[seen], lse_ref[seen], f"{label} lse")


LENS_K = [300, 17, 1000, 64, 0, 129, 500, 16]
LENS_Q = [128, 17, 1, 0, 0, 64, 300, 16]
# Runs of 512 queries or more: batches of up to 64 sequences then take 8-wave
# workgroups (256-row tiles, 8-row pieces of a cache block per wave).
LENS_K_LONG = [900, 17, 1000, 64, 0, 600, 1200, 16]
LENS_Q_LONG = [600, 17, 1, 0, 0, 513, 700, 16]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (12, 4), (16, 4), (32, 4)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged(gpu, hq, hkv, dtype, causal):
    print(f"case prefill ragged hq={hq} hkv={hkv} {dtype} causal={causal}", flush=True)
    _check(_make_case(LENS_K, LENS_Q, hq, hkv, 128, 16, dtype, seed=hq + hkv), f"hq={hq} hkv={hkv}", causal)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (12, 4), (32, 4)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged_long_chunks(gpu, hq, hkv, causal):
    print(f"case prefill ragged long hq={hq} hkv={hkv} causal={causal}", flush=True)
    _check(_make_case(LENS_K_LONG, LENS_Q_LONG, hq, hkv, 128, 16, torch.bfloat16, seed=40 + hq + hkv),
           f"long hq={hq} hkv={hkv}", causal)


@pytest.mark.parametrize("bs", [16, 32, 64])
@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("long_q", [False, True])
def test_prefill_block_sizes_and_head_dims(gpu, bs, d, long_q):
    print(f"case prefill bs={bs} d={d} long_q={long_q}", flush=True)
    lens_k, lens_q = ([900, 77, 31, 1100], [600, 40, 31, 513]) if long_q else ([200, 77, 31, 513], [200, 40, 31, 100])
    _check(_make_case(lens_k, lens_q, 8, 2, d, bs, torch.bfloat16, seed=bs + d + (1 if long_q else 0)),
           f"bs={bs} d={d} long_q={long_q}", sm_scale=0.1)


@pytest.mark.parametrize("long_q", [False, True])
def test_prefill_matches_packed_varlen_bitwise(gpu, long_q):
    """With the cache holding the packed K/V in order, the paged and packed
    forwards fill identical LDS tiles: outputs and lse agree bit for bit
    (with runs of 512 queries or more both take 8-wave workgroups)."""
    print(f"case prefill vs packed varlen long_q={long_q}", flush=True)
    lens_k, lens_q, hq, hkv, d, bs = [700, 64, 257, 1], [300, 64, 1, 1], 16, 4, 128, 16
    if long_q:
        lens_k, lens_q = [1500, 64, 700, 1], [700, 64, 513, 1]
    q, kc, vc, table, cu, sl = _make_case(lens_k, lens_q, hq, hkv, d, bs, torch.bfloat16, seed=5)
    k_packed = torch.cat([kc[table[b, :(n + bs - 1) // bs].long()].reshape(-1, hkv, d)[:n]
                          for b, n in enumerate(lens_k)])
    v_packed = torch.cat([vc[table[b, :(n + bs - 1) // bs].long()].reshape(-1, hkv, d)[:n]
                          for b, n in enumerate(lens_k)])
    cu_k = torch.tensor([0] + [sum(lens_k[:i + 1]) for i in range(len(lens_k))], dtype=torch.int32)
    o, lse = _run(q, kc, vc, table, cu, sl)
    o2, lse2 = flash_attention_varlen_forward(q.cuda(), k_packed.cuda(), v_packed.cuda(), cu.cuda(), cu_k.cuda(),
                                              max(lens_q), max(lens_k), causal=True)
    assert torch.equal(o, o2.cpu())
    assert torch.equal(lse, lse2.cpu())


def test_prefill_chunk_by_chunk_equals_one_pass(gpu):
    """Prefilling a sequence in chunks (each against the keys cached so far)
    gives the rows of one causal pass over the whole sequence."""
    print("case prefill chunked vs one pass", flush=True)
    n, hq, hkv, d, bs = 1000, 8, 2, 128, 16
    q, kc, vc, table, _, _ = _make_case([n], [n], hq, hkv, d, bs, torch.bfloat16, seed=6)
    whole, _ = _run(q, kc, vc, table, torch.tensor([0, n], dtype=torch.int32), torch.tensor([n], dtype=torch.int32))
    parts, start = [], 0
    for c in (256, 1, 300, 64, 379):
        o, _ = _run(q[start:start + c], kc, vc, table, torch.tensor([0, c], dtype=torch.int32),
                    torch.tensor([start + c], dtype=torch.int32))
        parts.append(o)
        start += c
    assert_gate(torch.cat(parts), whole, "chunked vs whole", max_abs=4e-3, mean_abs=2e-4)


def test_prefill_seq_lens_clamped_on_device(gpu):
    """seq_lens_k beyond the block table's capacity is clamped by the kernel."""
    print("case prefill clamp", flush=True)
    case = _make_case([64, 40], [16, 40], 4, 2, 64, 16, torch.bfloat16, seed=9)
    q, kc, vc, table, cu, _ = case
    claimed = torch.tensor([90, 40], dtype=torch.int32)  # 90 > 4 blocks of 16
    _check((q, kc, vc, table, cu, claimed), "clamp", lens_ref=torch.tensor([64, 40]))


def test_prefill_config5_shape(gpu):
    """Config 5 (B=8, Hq=32, Hkv=8, D=128, 512-token chunks after
    prefixes of 1024..8192 tokens) with K/V in a shuffled 16-token-block cache:
    bit-identical to the packed varlen forward, and one sequence's first and
    last heads against the oracle."""
    print("case prefill config5 shape", flush=True)
    g = torch.Generator().manual_seed(4)
    prefix = torch.randint(1024, 8193, (8,), generator=g).tolist()
    lens_k = [p + 512 for p in prefix]
    case = _make_case(lens_k, [512] * 8, 32, 8, 128, 16, torch.bfloat16, seed=11)
    q, kc, vc, table, cu, sl = case
    o, lse = _run(q, kc, vc, table, cu, sl, max_seqlen_q=512)
    bs = 16
    kp = torch.cat([kc[table[b, :(n + bs - 1) // bs].long()].reshape(-1, 8, 128)[:n] for b, n in enumerate(lens_k)])
    vp = torch.cat([vc[table[b, :(n + bs - 1) // bs].long()].reshape(-1, 8, 128)[:n] for b, n in enumerate(lens_k)])
    cu_k = torch.tensor([0] + [sum(lens_k[:i + 1]) for i in range(8)], dtype=torch.int32)
    o2, lse2 = flash_attention_varlen_forward(q.cuda(), kp.cuda(), vp.cuda(), cu.cuda(), cu_k.cuda(), 512,
                                              max(lens_k), causal=True)
    assert torch.equal(o, o2.cpu()) and torch.equal(lse, lse2.cpu())
    b = 3
    rows = slice(512 * b, 512 * (b + 1))
    heads = [0, 31]
    one = (q[rows][:, heads].contiguous(), kc, vc, table[b:b + 1], torch.tensor([0, 512], dtype=torch.int32),
           sl[b:b + 1])
    o_ref, lse_ref = paged_prefill_reference(one[0], kc[:, :, [0, 7]].contiguous(), vc[:, :, [0, 7]].contiguous(),
                                             one[3], one[4], one[5])
    assert_gate(o[rows][:, heads], o_ref, "config5 o (sequence 3, heads 0 and 31)")
    assert_lse(lse[heads][:, rows], lse_ref, "config5 lse")


def test_prefill_rejects_bad_arguments(gpu):
    q, kc, vc, table, cu, sl = _make_case([40], [8], 4, 2, 64, 8, torch.bfloat16, seed=1)
    with pytest.raises(RuntimeError, match="block_size"):
        _run(q, kc, vc, table, cu, sl)
    q, kc, vc, table, cu, sl = _make_case([40], [8], 4, 2, 64, 16, torch.bfloat16, seed=1)
    o = paged_prefill(q[:0].cuda(), kc.cuda(), vc.cuda(), table.cuda(), torch.zeros(2, dtype=torch.int32).cuda(),
                      sl.cuda(), max_seqlen_q=0)
    assert o.shape == (0, 4, 64)
