"""GPU parity of the backward kernels against the oracle's gradients.

Mirrors the reference's backward tests
(kernels/tests/test_flash_attention_backward.py: gradcheck :44-65, gradients
vs autograd :68-104, forward-with-LSE vs forward-only :107-124) with the
oracle's autograd (float64 on the CPU, or fp32 on the GPU for full-size
configs) in place of SDPA, and adds the max-abs 2e-2 / mean-abs 2e-3 gate at config sizes,
determinism and odd strides of dO.
"""
import pytest
import torch

from lightserve_amd.kernels.flash_attention import flash_attention_forward
from lightserve_amd.kernels.flash_attention_backward import (_backward_args, _flash_attention_backward,
                                                             _flash_attention_forward_lse, _FlashAttentionFunction,
                                                             flash_attention)
from oracle.attention import attention_grads, attention_reference, flash_backward_tiled
from lightserve_amd.workloads import make_config_inputs
from tests.gates import assert_gate, assert_grad_parity, assert_lse

pytestmark = pytest.mark.gpu

GRADCHECK_SHAPES = [(1, 1, 4, 8), (1, 2, 9, 16)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,N,D", GRADCHECK_SHAPES)
def test_gradcheck(gpu, B, H, N, D, causal):
    torch.manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, device=gpu, dtype=torch.float32, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda a, b, c: flash_attention(a, b, c, causal=causal), (q, k, v),
                                    eps=1e-3, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("causal", [False, True])
def test_reference_apply_signature(gpu, causal):
    """The reference calls `_FlashAttentionFunction.apply(q, k, v, causal)`
    (kernels/flash_attention_backward.py:385-397, :420): four arguments, no
    scale. Gradcheck through that exact call, and the same output as the
    entry point."""
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, 2, 9, 16, device=gpu, dtype=torch.float32, requires_grad=True) for _ in range(3))
    out = _FlashAttentionFunction.apply(q, k, v, causal)
    torch.testing.assert_close(out, flash_attention(q, k, v, causal=causal), atol=0, rtol=0)
    assert torch.autograd.gradcheck(lambda a, b, c: _FlashAttentionFunction.apply(a, b, c, causal), (q, k, v),
                                    eps=1e-3, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,N,D", [(1, 1, 17, 32), (2, 2, 64, 64), (1, 4, 130, 64), (2, 8, 256, 128)])
def test_matches_oracle_autograd(gpu, B, H, N, D, dtype, causal):
    print(f"case bwd {B}x{H}x{N}x{D} {dtype} causal={causal}", flush=True)
    torch.manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, device=gpu, dtype=dtype, requires_grad=True) for _ in range(3))
    do = torch.randn(B, H, N, D, device=gpu, dtype=dtype)
    out = flash_attention(q, k, v, causal=causal)
    out.backward(do)
    dq_r, dk_r, dv_r = attention_grads(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), do.cpu(), causal)
    tol = 1e-3 if dtype == torch.float32 else 3e-2
    for name, got, ref in (("dq", q.grad, dq_r), ("dk", k.grad, dk_r), ("dv", v.grad, dv_r)):
        assert got.dtype == dtype
        torch.testing.assert_close(got.cpu().double(), ref, atol=tol, rtol=tol, msg=lambda m: f"{name}: {m}")
        if dtype != torch.float32:
            assert_gate(got.cpu(), ref, f"{name} {dtype}")


def test_forward_matches_forward_only_kernel(gpu):
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 4, 130, 64, device=gpu, dtype=torch.float32) for _ in range(3))
    torch.testing.assert_close(flash_attention(q, k, v, causal=True),
                               flash_attention_forward(q, k, v, causal=True), atol=1e-3, rtol=1e-3)


def test_backward_deterministic_and_strided_do(gpu):
    """No atomics: two backward passes are bitwise equal; a non-contiguous dO
    gives the same gradients as its contiguous copy."""
    torch.manual_seed(1)
    q, k, v = (torch.randn(2, 4, 300, 128, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    o, L = _flash_attention_forward_lse(q, k, v, True)
    do_t = torch.randn(2, 300, 4, 128, device=gpu, dtype=torch.bfloat16).transpose(1, 2)
    g1 = _flash_attention_backward(do_t, q, k, v, o, L, True)
    g2 = _flash_attention_backward(do_t.contiguous(), q, k, v, o, L, True)
    g3 = _flash_attention_backward(do_t, q, k, v, o, L, True)
    for a, b, c in zip(g1, g2, g3):
        assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("D", [12, 96])
def test_backward_padded_head_dim(gpu, D):
    torch.manual_seed(2)
    q, k, v = (torch.randn(1, 2, 90, D, device=gpu, dtype=torch.bfloat16, requires_grad=True) for _ in range(3))
    do = torch.randn(1, 2, 90, D, device=gpu, dtype=torch.bfloat16)
    flash_attention(q, k, v, causal=True).backward(do)
    refs = attention_grads(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), do.cpu(), True)
    for name, got, ref in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), refs):
        assert_gate(got.cpu(), ref, f"D={D} {name}")


def _grads_gpu_fp32(q, k, v, do, causal):
    return attention_grads(q, k, v, do, causal, dtype=torch.float32)


def _backward_with_flags(do, q, k, v, o, L, causal, flags):
    """_flash_attention_backward with lsfa_bwd_args.flags set (equal head dims
    that need no padding: the outputs are written in place)."""
    from lightserve_amd import _lib
    args, keep = _backward_args(do, q, k, v, o, L, causal, flags=flags)
    assert all(a is b for a, b in zip(keep[:3], keep[3])), "needs an unpadded, kernel-ready layout"
    _lib.bwd(args, _lib.current_stream(q.device))
    return keep[:3]


@pytest.mark.parametrize("cfg,stored", [(3, False), (4, False), (3, True)])
def test_config_backward_full_size(gpu, cfg, stored):
    """The max-abs / mean-abs gate on dQ/dK/dV at the full config size, on every
    (batch, head) slice, with the oracle's fp32 autograd on the GPU (a gradient
    that misses the gate must be within 1.5x of the reference algorithm's own
    error, tests/gates.py). stored: the opt-in stored-dS path
    (LSFA_BWD_STORED_DS), checked against the oracle the same way."""
    from lightserve_amd import _lib
    print(f"case config {cfg} backward full size stored_ds={stored}", flush=True)
    inp = make_config_inputs(cfg, device=gpu)
    q, k, v, do, causal = inp["q"], inp["k"], inp["v"], inp["do"], inp["causal"]
    o, L = _flash_attention_forward_lse(q, k, v, causal)
    if stored:
        dq, dk, dv = _backward_with_flags(do, q, k, v, o, L, causal, _lib.BWD_STORED_DS)
    else:
        dq, dk, dv = _flash_attention_backward(do, q, k, v, o, L, causal)
    slices = [(b, h) for b in range(q.shape[0]) for h in range(q.shape[1])]
    for b, h in slices:
        sl = (slice(b, b + 1), slice(h, h + 1))
        exact = _grads_gpu_fp32(q[sl], k[sl], v[sl], do[sl], causal)
        o_ref, lse_ref = attention_reference(q[sl], k[sl], v[sl], causal, dtype=torch.float32)
        assert_gate(o[sl], o_ref, f"config {cfg} (b={b},h={h}) o")
        # the reference's own algorithm: stored o in the input dtype, fp32 L,
        # P and dS rounded to the input dtype before their products
        ref_alg = flash_backward_tiled(q[sl], k[sl], v[sl], o_ref.to(q.dtype), lse_ref, do[sl], causal,
                                       block_n=256, op_dtype=q.dtype)
        for name, got, ex, ra in zip(("dq", "dk", "dv"), (dq[sl], dk[sl], dv[sl]), exact, ref_alg):
            assert_grad_parity(got, ex, ra, f"config {cfg} (b={b},h={h}) {name}")


def _abi_fwd_bwd(q, k, v, do, causal, scale, phases=(0,), poison=False):
    """Forward with L, then backward (lsfa_bwd once per entry of phases, with
    that entry as flags), through the C ABI directly (the Python mirror keeps
    the reference's square-only contract). poison: the workspace starts as
    NaN bytes."""
    from lightserve_amd import _lib
    B, H, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    L = torch.empty(B, H, Nq, device=q.device, dtype=torch.float32)
    dt = _lib.TORCH_TO_LSFA[q.dtype]
    fa = _lib.FwdArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), lse=L.data_ptr(),
                      q_stride=_lib.strides4(q), k_stride=_lib.strides4(k), v_stride=_lib.strides4(v),
                      o_stride=_lib.strides4(o), lse_stride=_lib._i64x3(*L.stride()),
                      cu_seqlens_q=None, cu_seqlens_k=None, dtype=dt, batch=B, heads_q=H, heads_kv=Hkv,
                      seqlen_q=Nq, seqlen_k=Nk, head_dim=D, causal=int(causal), sm_scale=scale, reserved=0)
    stream = _lib.current_stream(q.device)
    _lib.fwd(fa, stream)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ba = _lib.BwdArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), dout=do.data_ptr(),
                      lse=L.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(), workspace=None,
                      workspace_bytes=0, q_stride=_lib.strides4(q), k_stride=_lib.strides4(k),
                      v_stride=_lib.strides4(v), o_stride=_lib.strides4(o), do_stride=_lib.strides4(do),
                      dq_stride=_lib.strides4(dq), dk_stride=_lib.strides4(dk), dv_stride=_lib.strides4(dv),
                      lse_stride=_lib._i64x3(*L.stride()), cu_seqlens_q=None, cu_seqlens_k=None, dtype=dt,
                      batch=B, heads_q=H, heads_kv=Hkv, seqlen_q=Nq, seqlen_k=Nk, head_dim=D,
                      causal=int(causal), sm_scale=scale, flags=phases[0])
    n = _lib.bwd_workspace_size(ba)
    ws = torch.empty(max(n, 1), device=q.device, dtype=torch.uint8)
    if poison:
        ws.fill_(0xFF)
    ba.workspace, ba.workspace_bytes = ws.data_ptr(), n
    for f in phases:
        ba.flags = f
        _lib.bwd(ba, stream)
    return o, L, dq, dk, dv


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Nq,Nk", [(70, 200), (200, 70), (1, 129), (129, 1), (300, 555), (555, 300)])
def test_abi_backward_non_square(gpu, Nq, Nk, causal, dtype, D):
    """Nq != Nk through the C ABI: causal masking is bottom-right aligned
    (query i sees keys <= i + Nk - Nq); rows that see no key get zero
    gradients and L = -inf."""
    print(f"case abi bwd Nq={Nq} Nk={Nk} causal={causal} {dtype} D={D}", flush=True)
    g = torch.Generator().manual_seed(5)
    B, H = 2, 3
    q, do = (torch.randn(B, H, Nq, D, generator=g).to(dtype).to(gpu) for _ in range(2))
    k, v = (torch.randn(B, H, Nk, D, generator=g).to(dtype).to(gpu) for _ in range(2))
    scale = D ** -0.5
    o, L, dq, dk, dv = _abi_fwd_bwd(q, k, v, do, causal, scale)
    torch.cuda.synchronize()
    qc, kc, vc, doc = (t.cpu() for t in (q, k, v, do))
    o_ref, l_ref = attention_reference(qc, kc, vc, causal, scale)
    refs = attention_grads(qc, kc, vc, doc, causal, scale)
    seen = torch.isfinite(l_ref)
    assert torch.equal(torch.isfinite(L.cpu()), seen)
    tol = 1e-4 if dtype == torch.float32 else 3e-2
    torch.testing.assert_close(L.cpu()[seen].double(), l_ref[seen], atol=1e-3 if dtype != torch.float32 else 1e-5,
                               rtol=0)
    torch.testing.assert_close(o.cpu().double().nan_to_num(), o_ref.nan_to_num(), atol=tol, rtol=tol)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
        torch.testing.assert_close(got.cpu().double(), ref.nan_to_num(), atol=tol, rtol=tol,
                                   msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_abi_backward_phases(gpu, causal, stored):
    """The backward's phases one at a time on one workspace (the timing mode
    the benchmark uses) give the full call's gradients bit for bit: default
    path LSFA_BWD_ONLY_DQ (which writes the per-row values) then
    LSFA_BWD_ONLY_DKDV; stored-dS path LSFA_BWD_ONLY_DKDV (which stores dS)
    then LSFA_BWD_ONLY_DQ. The workspace starts as NaN bytes in both runs, so
    a phase that reads what it did not write fails."""
    from lightserve_amd import _lib
    print(f"case abi bwd phases causal={causal} stored={stored}", flush=True)
    g = torch.Generator().manual_seed(6)
    q, k, v, do = (torch.randn(2, 3, 300, 128, generator=g).to(torch.bfloat16).to(gpu) for _ in range(4))
    r = _lib.BWD_STORED_DS if stored else 0
    order = (_lib.BWD_ONLY_DKDV, _lib.BWD_ONLY_DQ) if stored else (_lib.BWD_ONLY_DQ, _lib.BWD_ONLY_DKDV)
    full = _abi_fwd_bwd(q, k, v, do, causal, 128 ** -0.5, phases=(r,), poison=True)
    split = _abi_fwd_bwd(q, k, v, do, causal, 128 ** -0.5, phases=tuple(f | r for f in order), poison=True)
    torch.cuda.synchronize()
    for a, b in zip(full, split):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H,Nq,Nk,causal", [(2, 3, 300, 300, True), (1, 2, 700, 333, True), (1, 2, 333, 700, True),
                                               (2, 2, 513, 513, False), (1, 9, 16384, 16384, False)])
def test_stored_ds_matches_default(gpu, B, H, Nq, Nk, causal):
    """The stored-dS path (LSFA_BWD_STORED_DS, head dim 128) against the
    default path on the same inputs: dV comes from the same kernel arithmetic
    and is equal bit for bit; dK (delta summed in another order) and dQ (a
    GEMM over the stored dS instead of recomputed S and dP) agree to bf16
    rounding. Non-square causal shapes leave dS blocks left of a key block's
    first query tile unwritten (NaN here), which the dQ GEMM must mask. 9
    heads of 16384 x 16384 need 4.5 GiB of dS, more than one 4 GiB chunk, so
    that case runs the dK/dV kernel and the dQ GEMM in two chunks of heads."""
    from lightserve_amd import _lib
    print(f"case stored-dS vs default {B}x{H} Nq={Nq} Nk={Nk} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(7)
    q, do = (torch.randn(B, H, Nq, 128, generator=g).to(torch.bfloat16).to(gpu) for _ in range(2))
    k, v = (torch.randn(B, H, Nk, 128, generator=g).to(torch.bfloat16).to(gpu) for _ in range(2))
    _, _, dq0, dk0, dv0 = _abi_fwd_bwd(q, k, v, do, causal, 128 ** -0.5, phases=(_lib.BWD_STORED_DS,), poison=True)
    _, _, dq1, dk1, dv1 = _abi_fwd_bwd(q, k, v, do, causal, 128 ** -0.5, poison=True)
    torch.cuda.synchronize()
    assert torch.equal(dv0, dv1)
    for name, a, b in (("dq", dq0, dq1), ("dk", dk0, dk1)):
        assert torch.isfinite(a).all(), name
        err = (a.float() - b.float()).abs()
        scale = b.float().abs().max().item()
        assert err.max().item() <= 1e-2 * scale and err.mean().item() <= 1e-3 * scale, (name, err.max().item(), scale)

def _random_case(seed):
    import random
    r = random.Random(seed)
    B, H = r.randint(1, 3), r.randint(1, 4)
    Nq = r.choice([r.randint(1, 80), r.randint(60, 700), r.randint(500, 1200)])
    Nk = Nq if r.random() < 0.5 else r.randint(1, 1200)
    D = r.choice([16, 32, 64, 80, 96, 128])
    dtype = r.choice([torch.bfloat16, torch.float16])
    return B, H, Nq, Nk, D, dtype, r.random() < 0.5


def _check_fwd_bwd(gpu, B, H, Nq, Nk, D, dtype, causal, seed, what, flags=0, scale=None):
    """Forward with L and backward through the C ABI (workspace poisoned with
    NaN bytes; lsfa_bwd_args.flags = flags; sm_scale = scale, 1/sqrt(D) when
    None) against the oracle: L and o under the forward gate (rows that see
    no key: L = -inf, o = 0), dQ/dK/dV against the float64 autograd under the
    gradient gate."""
    g = torch.Generator().manual_seed(1000 + seed)
    q, do = (torch.randn(B, H, Nq, D, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, H, Nk, D, generator=g).to(dtype) for _ in range(2))
    scale = D ** -0.5 if scale is None else scale
    o, L, dq, dk, dv = _abi_fwd_bwd(*(t.to(gpu) for t in (q, k, v, do)), causal, scale, phases=(flags,),
                                    poison=True)
    torch.cuda.synchronize()
    o_ref, l_ref = attention_reference(q, k, v, causal, scale)
    assert_lse(L.cpu(), l_ref, f"{what} L")
    seen = torch.isfinite(l_ref)
    assert torch.equal(o.cpu()[~seen], torch.zeros_like(o.cpu()[~seen])), "rows that see no key must give o = 0"
    assert_gate(o.cpu().double()[seen], o_ref[seen], f"{what} o")
    exact = attention_grads(q, k, v, do, causal, scale)
    ref_alg = flash_backward_tiled(q, k, v, o_ref.nan_to_num().to(dtype), l_ref, do, causal, scale,
                                   op_dtype=dtype)
    for name, got, ex, ra in zip(("dq", "dk", "dv"), (dq, dk, dv), exact, ref_alg):
        assert_grad_parity(got.cpu(), ex.nan_to_num(), ra.nan_to_num(), f"{what} {name}")


@pytest.mark.parametrize("B,H,Nq,Nk,causal,dtype", [
    (2, 3, 300, 300, True, torch.bfloat16), (1, 2, 700, 333, True, torch.bfloat16),
    (1, 2, 333, 700, True, torch.float16), (2, 2, 513, 513, False, torch.bfloat16),
    (1, 3, 1, 129, True, torch.bfloat16), (1, 2, 1100, 77, False, torch.float16)])
def test_stored_ds_oracle(gpu, B, H, Nq, Nk, causal, dtype):
    """The stored-dS path (LSFA_BWD_STORED_DS, head dim 128: dS written by the
    dK/dV kernel, dQ a GEMM over it) against the float64 oracle under the
    gradient gate, on the non-square causal shapes whose unwritten dS blocks
    the dQ GEMM must mask, with the workspace poisoned."""
    from lightserve_amd import _lib
    print(f"case stored-dS oracle {B}x{H} Nq={Nq} Nk={Nk} causal={causal} {dtype}", flush=True)
    _check_fwd_bwd(gpu, B, H, Nq, Nk, 128, dtype, causal, Nq * 7 + Nk, f"stored-dS {Nq}x{Nk}",
                   flags=_lib.BWD_STORED_DS)


@pytest.mark.parametrize("seed", range(24))
def test_random_fwd_bwd(gpu, seed):
    """Seeded random shapes (ragged lengths on both sides, Nq != Nk, head dims
    that need padding, bf16/fp16, causal or not) through the C ABI."""
    B, H, Nq, Nk, D, dtype, causal = _random_case(seed)
    print(f"case random bwd seed={seed} {B}x{H} Nq={Nq} Nk={Nk} D={D} {dtype} causal={causal}", flush=True)
    _check_fwd_bwd(gpu, B, H, Nq, Nk, D, dtype, causal, seed, f"seed {seed}")


@pytest.mark.parametrize("B,H,Nq,Nk,D,causal,dtype,scale", [
    (2, 3, 700, 700, 128, True, torch.bfloat16, -(128 ** -0.5)),  # negative sm_scale
    (1, 2, 500, 900, 64, True, torch.float16, -0.05),              # negative, causal Nk > Nq
    (1, 2, 900, 400, 96, True, torch.bfloat16, 0.25),              # larger than 1/sqrt(D), rows that see no key
    (2, 2, 640, 640, 128, False, torch.float16, 0.02),             # small scale
])
def test_fwd_bwd_sm_scale(gpu, B, H, Nq, Nk, D, causal, dtype, scale):
    """sm_scale other than 1/sqrt(D), negative included (the forward negates q
    on load to keep its exponent scale positive; the backward's P, dK and dQ
    carry the sign), through the C ABI against the oracle."""
    print(f"case sm_scale bwd {B}x{H} Nq={Nq} Nk={Nk} D={D} {dtype} causal={causal} scale={scale}", flush=True)
    _check_fwd_bwd(gpu, B, H, Nq, Nk, D, dtype, causal, Nq + Nk + D, f"scale {scale}", scale=scale)


@pytest.mark.parametrize("Nq,Nk,causal,dtype", [(4160, 4160, True, torch.bfloat16), (4100, 700, True, torch.float16),
                                                (4097, 5000, False, torch.bfloat16), (4352, 4352, False, torch.float16)])
def test_long_query_fwd_bwd(gpu, Nq, Nk, causal, dtype):
    """Sequences past 4096 queries at head dim 128 (where the forward runs
    8-wave workgroups): ragged ends, rows that see no key, Nq != Nk."""
    print(f"case long-q dq Nq={Nq} Nk={Nk} causal={causal} {dtype}", flush=True)
    _check_fwd_bwd(gpu, 1, 2, Nq, Nk, 128, dtype, causal, Nq + Nk, f"long-q {Nq}x{Nk}")


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal,dtype", [
    (2, 8, 2, 300, 300, 128, True, torch.bfloat16), (1, 32, 8, 1024, 1024, 128, True, torch.bfloat16),
    (2, 6, 3, 200, 333, 64, False, torch.float16), (1, 4, 1, 513, 257, 64, True, torch.bfloat16),
    (1, 8, 4, 129, 700, 96, True, torch.float16), (3, 4, 2, 77, 77, 32, False, torch.bfloat16),
    (1, 8, 2, 4160, 4160, 128, True, torch.bfloat16)])
def test_abi_backward_gqa(gpu, B, Hq, Hkv, Nq, Nk, D, causal, dtype):
    """GQA backward through the C ABI (query head h reads KV head h / G,
    G = Hq / Hkv): dQ per query head, dK/dV per KV head summed over its G
    query heads. Checked against the oracle on K/V repeated G times (as the
    reference's own GQA convention, repeat_interleave over the head axis),
    with dK/dV summed over each group."""
    print(f"case gqa bwd {B}x{Hq}/{Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal} {dtype}", flush=True)
    G = Hq // Hkv
    g = torch.Generator().manual_seed(Nq + 7 * Hq)
    q, do = (torch.randn(B, Hq, Nq, D, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, Hkv, Nk, D, generator=g).to(dtype) for _ in range(2))
    scale = D ** -0.5
    o, L, dq, dk, dv = _abi_fwd_bwd(*(t.to(gpu) for t in (q, k, v, do)), causal, scale, poison=True)
    torch.cuda.synchronize()
    ke, ve = k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1)
    o_ref, l_ref = attention_reference(q, ke, ve, causal, scale)
    what = f"gqa {Hq}/{Hkv} {Nq}x{Nk}"
    assert_lse(L.cpu(), l_ref, f"{what} L")
    seen = torch.isfinite(l_ref)
    assert_gate(o.cpu().double()[seen], o_ref[seen], f"{what} o")
    grp = lambda t: t.reshape(B, Hkv, G, Nk, D).sum(2)  # noqa: E731
    dq_e, dk_e, dv_e = attention_grads(q, ke, ve, do, causal, scale)
    dq_a, dk_a, dv_a = flash_backward_tiled(q, ke, ve, o_ref.nan_to_num().to(dtype), l_ref, do, causal, scale,
                                            op_dtype=dtype)
    for name, got, ex, ra in (("dq", dq, dq_e, dq_a), ("dk", dk, grp(dk_e), grp(dk_a)), ("dv", dv, grp(dv_e), grp(dv_a))):
        assert got.shape == ex.shape, name
        assert_grad_parity(got.cpu(), ex.nan_to_num(), ra.nan_to_num(), f"{what} {name}")
