"""GPU parity of the forward kernels against the oracle (oracle/attention.py).

Mirrors the reference's forward tests (kernels/tests/test_flash_attention.py:
shapes :24-31, dtypes and tolerances :40-61, non-contiguous input :65-77)
with the oracle in place of SDPA, adds fp16, logsumexp, the correctness gate (max-abs 2e-2, mean-abs 2e-3, LSE 1e-3) at
the full config sizes, head dims that need padding, graph capture and a
side stream.
"""
import math
import os

import numpy as np
import pytest
import torch

from lightserve_amd.kernels.flash_attention import flash_attention_forward
from oracle.attention import attention_reference
from lightserve_amd.workloads import make_config_inputs
from tests.gates import assert_gate, assert_lse

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 1, 8), (1, 1, 17, 32), (2, 2, 64, 64), (1, 4, 130, 64), (2, 8, 256, 128), (1, 2, 100, 96)]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _oracle_cpu(q, k, v, causal, sm_scale=None):
    return attention_reference(q.cpu(), k.cpu(), v.cpu(), causal, sm_scale)


def _oracle_gpu_chunked(q, k, v, causal, heads_per_chunk=8):
    """fp32 oracle on the GPU, a few heads at a time (large configs)."""
    B, H = q.shape[:2]
    o = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    for b in range(B):
        for h0 in range(0, H, heads_per_chunk):
            sl = (b, slice(h0, h0 + heads_per_chunk))
            ob, lb = attention_reference(q[sl], k[sl], v[sl], causal, dtype=torch.float32)
            o[sl], lse[sl] = ob, lb
    return o, lse


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,H,N,D", SHAPES)
def test_matches_oracle_reference_shapes(gpu, B, H, N, D, dtype, causal):
    print(f"case fwd {B}x{H}x{N}x{D} {dtype} causal={causal}", flush=True)
    torch.manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, device=gpu, dtype=dtype) for _ in range(3))
    o, lse = flash_attention_forward(q, k, v, causal=causal, return_lse=True)
    o_ref, lse_ref = _oracle_cpu(q, k, v, causal)
    if dtype == torch.float32:
        torch.testing.assert_close(o.cpu().double(), o_ref, atol=1e-3, rtol=1e-3)
    else:
        torch.testing.assert_close(o.cpu().double(), o_ref, atol=2e-2, rtol=2e-2)
        assert_gate(o.cpu(), o_ref, f"o {dtype}")
    assert_lse(lse.cpu(), lse_ref, "lse")
    o_only = flash_attention_forward(q, k, v, causal=causal)
    assert torch.equal(o_only, o), "return_lse must not change the output"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_offset_raised_by_later_tiles(gpu, D, dtype, causal):
    """The forward's exponent offset starts at the first key tile's row max
    and is raised only when a tile's exponentials come near the operand
    dtype's range (2^64 for bf16, 2^15 for fp16). Here a few keys far into the
    sequence score ~55 natural-log units above everything in the first tile
    (q has a common component, the spike keys are constant vectors along
    it), which must take the raise-and-recompute path on that tile; the
    spike keys then carry nearly all of the weight of the rows that see
    them."""
    print(f"case fwd offset raise D={D} {dtype} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(11)
    B, H, N = 1, 2, 600
    q = torch.randn(B, H, N, D, generator=g) * 0.3 + 1.0
    k = torch.randn(B, H, N, D, generator=g) * 0.5
    v = torch.randn(B, H, N, D, generator=g)
    spikes = [301, 302, 450, 451, 452]
    k[:, :, spikes, :] = 55.0 / math.sqrt(D)
    q, k, v = (t.to(dtype).to(gpu) for t in (q, k, v))
    o, lse = flash_attention_forward(q, k, v, causal=causal, return_lse=True)
    o_ref, lse_ref = _oracle_cpu(q, k, v, causal)
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    assert_gate(o.cpu(), o_ref, f"o {dtype}")
    assert_lse(lse.cpu(), lse_ref, "lse")
    assert lse_ref.max() > 40  # the spikes dominate the rows that see them


@pytest.mark.parametrize("B,H,N,causal", [(1, 13, 1024, True), (3, 5, 2048, True), (1, 13, 1500, False)])
def test_grouped_tile_order_covers_every_tile(gpu, B, H, N, causal):
    """Workgroups take (head, query tile) in groups of heads sized to a few MB
    of K/V (here 4-16 heads: 13 and 15 heads leave a partial last group, and
    13 * 8 = 104 or 13 * 12 = 156 tiles are or are not a multiple of the 8
    XCDs): every query row of every head must be computed exactly once, so
    each (b, h) slice matches the oracle, forward and backward (gradients
    under the gradient gate: max-abs 2e-2 and mean-abs 2e-3, or within 1.5x
    of the restated reference algorithm's own error)."""
    from lightserve_amd.kernels.flash_attention_backward import _flash_attention_backward, _flash_attention_forward_lse
    from oracle.attention import flash_backward_tiled
    from tests.gates import assert_grad_parity
    print(f"case grouped order {B}x{H}x{N} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(12)
    qc, kc, vc, doc = (torch.randn(B, H, N, 128, generator=g).to(torch.bfloat16) for _ in range(4))
    q, k, v, do = (t.to(gpu) for t in (qc, kc, vc, doc))
    o, lse = _flash_attention_forward_lse(q, k, v, causal)
    dq, dk, dv = _flash_attention_backward(do, q, k, v, o, lse, causal)
    torch.cuda.synchronize()
    # the reference's algorithm (bf16 rounding points), on the host, from the
    # closed-form forward
    o_cf, l_cf = attention_reference(qc, kc, vc, causal, dtype=torch.float32)
    ref_alg = flash_backward_tiled(qc, kc, vc, o_cf.to(torch.bfloat16), l_cf, doc, causal, op_dtype=torch.bfloat16)
    from tests.test_fa_backward_gpu import _grads_gpu_fp32
    for b in range(B):
        for h in range(H):
            sl = (slice(b, b + 1), slice(h, h + 1))
            o_ref, l_ref = attention_reference(q[sl].float(), k[sl].float(), v[sl].float(), causal, dtype=torch.float32)
            assert_gate(o[sl].float(), o_ref, f"o (b={b},h={h})")
            assert_lse(lse[sl], l_ref, f"lse (b={b},h={h})")
            exact = _grads_gpu_fp32(q[sl], k[sl], v[sl], do[sl], causal)
            for name, got, want, ra in zip(("dq", "dk", "dv"), (dq[sl], dk[sl], dv[sl]), exact, ref_alg):
                assert_grad_parity(got.float().cpu(), want.float().cpu(), ra[sl], f"grouped {name} (b={b},h={h})")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_matches_oracle_non_contiguous(gpu, dtype):
    """The reference's transposed-heads view (kernels/tests/test_flash_attention.py:65-77)."""
    torch.manual_seed(0)
    q = torch.randn(1, 64, 4, 32, device=gpu, dtype=dtype).transpose(1, 2)
    k = torch.randn(1, 4, 64, 32, device=gpu, dtype=dtype)
    v = torch.randn(1, 4, 64, 32, device=gpu, dtype=dtype)
    o = flash_attention_forward(q, k, v)
    assert o.stride() == q.stride(), "o must keep q's strides (empty_like)"
    o_ref, _ = _oracle_cpu(q, k, v, False)
    tol = 1e-3 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(o.cpu().double(), o_ref, atol=tol, rtol=tol)


def test_model_layout_bf16(gpu):
    """q/k/v as the model passes them: [B, H, N, D] views over [B, N, H, D]
    memory (model/minimal_llama.py:216-221), read in place."""
    torch.manual_seed(1)
    B, N, H, D = 2, 300, 8, 128
    q, k, v = (torch.randn(B, N, H, D, device=gpu, dtype=torch.bfloat16).transpose(1, 2) for _ in range(3))
    o, lse = flash_attention_forward(q, k, v, causal=True, return_lse=True)
    o_ref, lse_ref = _oracle_cpu(q, k, v, True)
    assert_gate(o.cpu(), o_ref, "model layout o")
    assert_lse(lse.cpu(), lse_ref, "model layout")


@pytest.mark.parametrize("D", [12, 40, 72])
def test_padded_head_dim_bf16(gpu, D):
    """Head dims that are not multiples of 8 go through a zero-padded copy."""
    torch.manual_seed(2)
    q, k, v = (torch.randn(2, 3, 77, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    o, lse = flash_attention_forward(q, k, v, causal=True, return_lse=True)
    o_ref, lse_ref = _oracle_cpu(q, k, v, True)
    assert_gate(o.cpu(), o_ref, f"D={D} o")
    assert_lse(lse.cpu(), lse_ref, f"D={D}")


def test_sm_scale_argument(gpu):
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, 2, 200, 64, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    o, lse = flash_attention_forward(q, k, v, causal=False, sm_scale=0.3, return_lse=True)
    o_ref, lse_ref = _oracle_cpu(q, k, v, False, 0.3)
    assert_gate(o.cpu(), o_ref, "sm_scale o")
    assert_lse(lse.cpu(), lse_ref, "sm_scale")


def test_config1_against_golden(gpu):
    """Config 1 (fp32 causal 1x4x256x64, seed 0) against the pure-Python loop
    fixture of tests/golden."""
    golden = np.load(os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz"))
    inp = make_config_inputs(1, device=gpu)
    o, lse = flash_attention_forward(inp["q"], inp["k"], inp["v"], causal=True, return_lse=True)
    np.testing.assert_allclose(o[0, :, ::8, :].cpu().double().numpy(), golden["cfg1/o_rows"], atol=1e-4)
    np.testing.assert_allclose(lse[0].cpu().double().numpy(), golden["cfg1/lse"], atol=1e-4)


@pytest.mark.parametrize("cfg", [2, 3, 4])
def test_config_forward_full_size(gpu, cfg):
    """The max-abs / mean-abs / LSE gate at the full config size, every (batch, head)
    (oracle in fp32 on the GPU, one head at a time at config 4's 16384 keys)."""
    print(f"case config {cfg} forward full size", flush=True)
    inp = make_config_inputs(cfg, device=gpu)
    q, k, v, causal = inp["q"], inp["k"], inp["v"], inp["causal"]
    o, lse = flash_attention_forward(q, k, v, causal=causal, return_lse=True)
    o_ref, lse_ref = _oracle_gpu_chunked(q, k, v, causal, **({"heads_per_chunk": 1} if cfg == 4 else {}))
    assert_gate(o, o_ref, f"config {cfg} o")
    assert_lse(lse, lse_ref, f"config {cfg}")


def test_zero_query_property_full_size(gpu):
    """Size-independent closed form at config 3's shape: with q = 0 every
    visible key scores 0, so o_i is the mean of v_0..v_i and L_i = ln(i+1)."""
    inp = make_config_inputs(3, device=gpu)
    v = inp["v"][:, :4]
    q = torch.zeros_like(v)
    o, lse = flash_attention_forward(q, inp["k"][:, :4], v, causal=True, return_lse=True)
    n = v.shape[2]
    idx = torch.arange(1, n + 1, device=gpu, dtype=torch.float64)
    mean = v.double().cumsum(2) / idx.view(1, 1, n, 1)
    assert_gate(o, mean, "q=0 prefix mean")
    torch.testing.assert_close(lse.double(), torch.log(idx).expand_as(lse), atol=1e-4, rtol=0)


def test_edge_sizes(gpu):
    torch.manual_seed(4)
    for (B, H, N, D) in [(1, 1, 1, 128), (3, 1, 129, 64), (1, 2, 255, 32), (1, 1, 513, 128)]:
        q, k, v = (torch.randn(B, H, N, D, device=gpu, dtype=torch.bfloat16) for _ in range(3))
        for causal in (False, True):
            o, lse = flash_attention_forward(q, k, v, causal=causal, return_lse=True)
            o_ref, lse_ref = _oracle_cpu(q, k, v, causal)
            assert_gate(o.cpu(), o_ref, f"edge {B}x{H}x{N}x{D} causal={causal}")
            assert_lse(lse.cpu(), lse_ref, "edge")
    empty = torch.empty(1, 2, 0, 64, device=gpu, dtype=torch.bfloat16)
    assert flash_attention_forward(empty, empty, empty).shape == empty.shape


def test_graph_capture_and_side_stream(gpu):
    """The call captures into a HIP graph (no host sync, no allocation by the
    library); every replay matches the eager result, with eager work and
    synchronisation between replays."""
    torch.manual_seed(5)
    q, k, v = (torch.randn(2, 4, 333, 128, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    eager = flash_attention_forward(q, k, v, causal=True)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        o_side = flash_attention_forward(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o_side, eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        flash_attention_forward(q, k, v, causal=True)  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=side):
            out = flash_attention_forward(q, k, v, causal=True)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        _ = (q.float() * 2).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("B,H,N,D,causal,dtype", [(1, 5, 4100, 128, True, torch.bfloat16),
                                                   (1, 3, 4352, 64, False, torch.bfloat16),
                                                   (2, 2, 4097, 64, True, torch.bfloat16),
                                                   (1, 3, 4160, 128, True, torch.float16)])
def test_wide_workgroups(gpu, B, H, N, D, causal, dtype):
    """Dense launches of at least 4096 queries (head dim >= 64) run 8-wave,
    256-row workgroups: sequence ends that are not a multiple of 256 (or of
    the 64-key tile), every (b, h) slice against the oracle."""
    print(f"case wide forward {B}x{H}x{N}x{D} causal={causal} {dtype}", flush=True)
    g = torch.Generator().manual_seed(N + D)
    q, k, v = (torch.randn(B, H, N, D, generator=g).to(dtype).to(gpu) for _ in range(3))
    o, lse = flash_attention_forward(q, k, v, causal=causal, return_lse=True)
    o_ref, lse_ref = _oracle_gpu_chunked(q.float(), k.float(), v.float(), causal, heads_per_chunk=1)
    assert_gate(o.float(), o_ref, f"wide {N} o")
    assert_lse(lse, lse_ref, f"wide {N}")


def _abi_fwd(q, k, v, causal, scale):
    """Forward with L through the C ABI (Nq != Nk allowed), into NaN-filled
    outputs so that a row the kernel never writes shows."""
    from lightserve_amd import _lib
    B, H, Nq, D = q.shape
    o = torch.full_like(q, float("nan"))
    L = torch.full((B, H, Nq), float("nan"), device=q.device, dtype=torch.float32)
    fa = _lib.FwdArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), lse=L.data_ptr(),
                      q_stride=_lib.strides4(q), k_stride=_lib.strides4(k), v_stride=_lib.strides4(v),
                      o_stride=_lib.strides4(o), lse_stride=_lib._i64x3(*L.stride()),
                      cu_seqlens_q=None, cu_seqlens_k=None, dtype=_lib.TORCH_TO_LSFA[q.dtype], batch=B, heads_q=H,
                      heads_kv=k.shape[1], seqlen_q=Nq, seqlen_k=k.shape[2], head_dim=D, causal=int(causal),
                      sm_scale=scale, reserved=0)
    _lib.fwd(fa, _lib.current_stream(q.device))
    return o, L


@pytest.mark.parametrize("B,H,Nq,Nk,D,causal,dtype,layout", [
    (4, 16, 4096, 4096, 128, True, torch.bfloat16, "bhnd"),   # 1024 items, 4 per workgroup
    (4, 32, 2048, 2048, 128, True, torch.float16, "bhnd"),    # 2048 queries (config-2 shape)
    (4, 64, 4200, 4200, 128, False, torch.bfloat16, "bhnd"),  # 4352 items, ragged last query tile
    (4, 16, 4096, 4096, 64, False, torch.float16, "bhnd"),    # head dim 64
    (4, 32, 2048, 2048, 96, False, torch.bfloat16, "bhnd"),   # padded head dim
    (4, 16, 4096, 4096, 128, True, torch.bfloat16, "bnhd"),   # rows strided by H * D
    (3, 24, 4096, 4096, 64, False, torch.float16, "bhnd"),    # 1152 items: 4 or 5 per workgroup
    (4, 16, 4200, 4200, 128, True, torch.bfloat16, "bhnd"),   # fixed split unbalanced: per-item kernel
    (4, 16, 4096, 4608, 128, True, torch.bfloat16, "bhnd"),   # Nk > Nq (unbalanced): per-item kernel
    (2, 16, 4200, 4200, 128, True, torch.bfloat16, "bhnd"),   # 544 items: too few, per-item kernel
])
def test_persistent_forward(gpu, B, H, Nq, Nk, D, causal, dtype, layout):
    """Dense launches from 4096 queries (2048 at head dim 128) with at least
    four (b, h, 256-row tile) items per CU (1024 on MI355X) whose fixed split
    is balanced run one workgroup per CU that streams its items (the K/V
    tiles of consecutive items through one double buffer, the next item's Q
    rows and first score tile during the current item's last step, O and L
    stored one step late): every row of every (b, h) written once and within
    the gate. The last three shapes take the per-item kernel instead."""
    print(f"case persistent forward {B}x{H} Nq={Nq} Nk={Nk} D={D} causal={causal} {dtype} {layout}", flush=True)
    g = torch.Generator().manual_seed(Nq + Nk + D)
    if layout == "bnhd":
        q = torch.randn(B, Nq, H, D, generator=g).to(dtype).to(gpu).transpose(1, 2)
        k, v = (torch.randn(B, Nk, H, D, generator=g).to(dtype).to(gpu).transpose(1, 2) for _ in range(2))
    else:
        q = torch.randn(B, H, Nq, D, generator=g).to(dtype).to(gpu)
        k, v = (torch.randn(B, H, Nk, D, generator=g).to(dtype).to(gpu) for _ in range(2))
    o, lse = _abi_fwd(q, k, v, causal, 1.0 / math.sqrt(D))
    assert not torch.isnan(o).any() and not torch.isnan(lse).any(), "a row was left unwritten"
    o_ref, lse_ref = _oracle_gpu_chunked(q.float(), k.float(), v.float(), causal, heads_per_chunk=4)
    assert_gate(o.float(), o_ref, f"persistent {Nq}x{Nk} o")
    assert_lse(lse, lse_ref, f"persistent {Nq}x{Nk}")


@pytest.mark.parametrize("B,H,Nq,Nk,D,causal,dtype,scale", [
    (12, 8, 4096, 4096, 64, True, torch.bfloat16, -0.125),           # negative sm_scale
    (5, 32, 2304, 3081, 128, False, torch.float16, 128 ** -0.5),     # Nk > Nq, ragged key tail
    (6, 16, 3072, 3136, 128, True, torch.float16, 128 ** -0.5),      # causal with Nk > Nq
    (6, 16, 3072, 3072, 128, False, torch.float16, -(128 ** -0.5)),  # negative sm_scale, head dim 128
    (3, 32, 4160, 3860, 128, True, torch.bfloat16, 0.0442),          # causal Nk < Nq: rows that see no key
    (16, 8, 4352, 4416, 96, True, torch.bfloat16, 96 ** -0.5),       # padded head dim
    (3, 32, 4160, 8320, 128, False, torch.bfloat16, 128 ** -0.5),    # Nk = 2 Nq
    (6, 16, 8192, 16384, 64, True, torch.float16, -0.125),           # long keys, negative sm_scale
])
def test_dense_forward_random_shapes(gpu, B, H, Nq, Nk, D, causal, dtype, scale):
    """Seeded shapes around the persistent kernel's dispatch limits (item
    counts per CU, balanced or not, Nq != Nk both ways, ragged tails, padded
    head dims, any sm_scale): whichever kernel the host picks, every row is
    written once and O / L pass the gate against the oracle."""
    print(f"case dense forward {B}x{H} Nq={Nq} Nk={Nk} D={D} causal={causal} {dtype} scale={scale:.4f}", flush=True)
    g = torch.Generator().manual_seed(Nq * 7 + Nk + D)
    q = torch.randn(B, H, Nq, D, generator=g).to(dtype).to(gpu)
    k, v = (torch.randn(B, H, Nk, D, generator=g).to(dtype).to(gpu) for _ in range(2))
    o, lse = _abi_fwd(q, k, v, causal, scale)
    assert not torch.isnan(o).any() and not torch.isnan(lse).any(), "a row was left unwritten"
    o_ref = torch.empty(o.shape, device=gpu, dtype=torch.float32)
    lse_ref = torch.empty(lse.shape, device=gpu, dtype=torch.float32)
    for b in range(B):
        for h0 in range(0, H, 4):
            sl = (b, slice(h0, h0 + 4))
            o_ref[sl], lse_ref[sl] = attention_reference(q[sl], k[sl], v[sl], causal, scale, dtype=torch.float32)
    assert_gate(o.float(), o_ref, f"dense {Nq}x{Nk} o")
    assert_lse(lse, lse_ref, f"dense {Nq}x{Nk}")
