"""GPU parity of the paged-KV decode kernel against the oracle.

The reference has no decode kernel (its engine documents it as missing,
engine/README.md "No decode-shaped attention kernel"), so parity is against
oracle.attention.paged_decode_reference (gather through the block table,
then the closed-form attention), under the correctness gate (max-abs 2e-2,
mean-abs 2e-3, lse 1e-3). Two kernels are covered: the MFMA kernel (block
sizes that are multiples of 16, any group size up to 32) and the lane-group
kernel (smaller blocks, groups 1/2/4/8). Cases: GQA group sizes 1-32, head
dims 32-128, block sizes 1/16/32/64, ragged and empty sequences, lengths at
block and tile boundaries, shuffled physical blocks, split and unsplit
launches, the device-side clamp of seq_lens to max_seq_len, and 20 seeded
random batches over all of these.
"""
import pytest
import torch

from lightserve_amd.kernels.paged_attention import paged_attention_decode
from oracle.attention import paged_decode_reference
from tests.gates import assert_gate, assert_lse

pytestmark = pytest.mark.gpu


def _make_case(lens, hq, hkv, d, bs, dtype, device, seed, extra_blocks=3):
    """Random cache with every sequence's blocks scattered over a shuffled pool."""
    g = torch.Generator().manual_seed(seed)
    nblk = [(n + bs - 1) // bs for n in lens]
    num_blocks = sum(nblk) + extra_blocks
    perm = torch.randperm(num_blocks, generator=g)
    max_blocks = max(max(nblk), 1)
    table = torch.zeros(len(lens), max_blocks, dtype=torch.int32)
    at = 0
    for b, k in enumerate(nblk):
        table[b, :k] = perm[at:at + k].to(torch.int32)
        at += k
    kc = (torch.randn(num_blocks, bs, hkv, d, generator=g) * 0.5).to(dtype)
    vc = torch.randn(num_blocks, bs, hkv, d, generator=g).to(dtype)
    q = (torch.randn(len(lens), hq, d, generator=g) * 0.5).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32)
    return q, kc, vc, table, sl


def _check(q, kc, vc, table, sl, label, max_seq_len=None, sm_scale=None, lens_ref=None):
    dev = "cuda"
    o, lse = paged_attention_decode(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), sl.to(dev),
                                    max_seq_len=max_seq_len, sm_scale=sm_scale, return_lse=True)
    torch.cuda.synchronize()
    o_ref, lse_ref = paged_decode_reference(q, kc, vc, table, sl if lens_ref is None else lens_ref, sm_scale)
    assert_gate(o.cpu(), o_ref, f"{label} o")
    seen = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse.cpu()), seen), label
    if seen.any():
        assert_lse(lse.cpu()[seen], lse_ref[seen], f"{label} lse")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (32, 8), (16, 2)])
@pytest.mark.parametrize("d", [128, 64])
def test_decode_small(gpu, hq, hkv, d, dtype):
    lens = [1, 15, 16, 17, 0, 100, 333]
    print(f"case decode small hq={hq} hkv={hkv} d={d} {dtype}", flush=True)
    _check(*_make_case(lens, hq, hkv, d, 16, dtype, gpu, seed=hq + d), f"hq={hq} hkv={hkv} d={d}")


@pytest.mark.parametrize("bs", [1, 32, 64])
@pytest.mark.parametrize("d", [32, 96])
def test_decode_block_sizes_and_padded_dims(gpu, bs, d):
    print(f"case decode bs={bs} d={d}", flush=True)
    _check(*_make_case([3, 64, 200, 31], 8, 2, d, bs, torch.bfloat16, gpu, seed=bs * d), f"bs={bs} d={d}",
           sm_scale=0.2)


@pytest.mark.parametrize("lens", [[5000], [4096, 1, 3000], [12000, 700]])
def test_decode_long_split(gpu, lens):
    """Few (sequence, kv head) pairs and long sequences: the launch splits the
    sequences and merges the partial outputs with their logsumexps."""
    print(f"case decode split lens={lens}", flush=True)
    _check(*_make_case(lens, 8, 1, 128, 16, torch.bfloat16, gpu, seed=len(lens)), f"split {lens}")


def test_decode_more_splits_than_one_combine_batch(gpu):
    """Block size 1 caps a split at 448 tokens (511 table slots in LDS), so
    240000 tokens make 536 splits: more than the 512 logsumexps the combine
    kernel stages at a time, which exercises its running-max merge across
    batches."""
    print("case decode 240000 tokens, block size 1 (536 splits)", flush=True)
    _check(*_make_case([240000], 2, 1, 64, 1, torch.bfloat16, gpu, seed=11), "536 splits")


def test_decode_many_sequences_unsplit(gpu):
    """Enough (sequence, kv head) pairs to fill the GPU: no split."""
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1, 300, (160,), generator=g).tolist()
    print("case decode 160 sequences", flush=True)
    _check(*_make_case(lens, 32, 8, 128, 16, torch.bfloat16, gpu, seed=7), "160 seqs")


def test_decode_seq_lens_clamped_on_device(gpu):
    """seq_lens above max_seq_len are clamped by the kernel (no reads past the
    declared extent): the result equals attention over max_seq_len tokens."""
    q, kc, vc, table, sl = _make_case([40, 64, 64], 4, 2, 64, 16, torch.bfloat16, gpu, seed=9)
    sl_claimed = torch.tensor([40, 64, 90], dtype=torch.int32)  # 90 > 64 = 4 blocks of 16
    print("case decode clamp", flush=True)
    _check(q, kc, vc, table, sl_claimed, "clamp", max_seq_len=64, lens_ref=torch.tensor([40, 64, 64]))


@pytest.mark.parametrize("hq,hkv,bs", [(12, 4, 16), (32, 2, 16), (32, 1, 64), (24, 8, 32)])
def test_decode_mfma_group_sizes(gpu, hq, hkv, bs):
    """Group sizes only the MFMA kernel takes (3, 16, 32), and 64-token blocks."""
    lens = [1, 31, 32, 33, 0, 640, 2000, 129]
    print(f"case decode groups hq={hq} hkv={hkv} bs={bs}", flush=True)
    _check(*_make_case(lens, hq, hkv, 128, bs, torch.bfloat16, gpu, seed=hq + bs), f"hq={hq} hkv={hkv} bs={bs}")


def test_decode_rejects_bad_arguments(gpu):
    q, kc, vc, table, sl = _make_case([4], 6, 2, 64, 8, torch.bfloat16, gpu, seed=1)
    with pytest.raises(RuntimeError, match="heads_q / heads_kv"):  # group of 3 with 8-token blocks
        paged_attention_decode(q.cuda(), kc.cuda(), vc.cuda(), table.cuda(), sl.cuda())
    q, kc, vc, table, sl = _make_case([4], 64, 1, 64, 16, torch.bfloat16, gpu, seed=1)
    with pytest.raises(RuntimeError, match="heads_q / heads_kv"):  # group of 64
        paged_attention_decode(q.cuda(), kc.cuda(), vc.cuda(), table.cuda(), sl.cuda())
    q, kc, vc, table, sl = _make_case([4], 4, 2, 64, 12, torch.bfloat16, gpu, seed=1)
    with pytest.raises(RuntimeError, match="power of two"):
        paged_attention_decode(q.cuda(), kc.cuda(), vc.cuda(), table.cuda(), sl.cuda())


def _random_decode_case(seed):
    import random
    r = random.Random(seed)
    hkv = r.choice([1, 2, 4, 8])
    group = r.choice([1, 2, 4, 8, 3, 6, 12])
    bs = r.choice([16, 32, 64]) if group not in (1, 2, 4, 8) else r.choice([1, 8, 16, 32, 64])
    d = r.choice([32, 64, 96, 128])
    dtype = r.choice([torch.bfloat16, torch.float16])
    nseq = r.randint(1, 40)
    lens = [r.choice([0, r.randint(1, 64), r.randint(1, 2000), r.randint(2000, 9000)]) for _ in range(nseq)]
    return lens, hkv * group, hkv, d, bs, dtype


@pytest.mark.parametrize("seed", range(20))
def test_decode_random_batches(gpu, seed):
    """Seeded random batches: ragged and empty sequences, group sizes for both
    kernels, head dims 32-128, block sizes 1-64, bf16/fp16."""
    lens, hq, hkv, d, bs, dtype = _random_decode_case(seed)
    label = f"random decode seed={seed} B={len(lens)} hq={hq} hkv={hkv} d={d} bs={bs} {dtype}"
    print(f"case {label} lens={lens}", flush=True)
    q, kc, vc, table, sl = _make_case(lens, hq, hkv, d, bs, dtype, "cuda", 500 + seed)
    _check(q, kc, vc, table, sl, label)
