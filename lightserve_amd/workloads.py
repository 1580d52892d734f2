"""Seeded synthetic inputs and FLOP counts of the five benchmark workloads.

Recipe (fixed here; the workload definitions name only shapes, scales and
seeds): a CPU torch.Generator seeded with the config's seed draws fp32 randn
tensors in the order q, k, v, (dO), then config-specific extras; the scale
factor is applied in fp32, then the tensors are cast to the config dtype. Oracles use
the cast values upcast to fp32/fp64. bench.py and the GPU tests both build
their inputs from here, so they see identical data. Nothing on the kernel
path imports this module.
"""
import torch

CONFIGS = {
    1: dict(name="cpu_plumbing_fp32_causal", B=1, H=4, N=256, D=64, dtype=torch.float32,
            causal=True, seed=0, mul=1.0, backward=False),
    2: dict(name="llama3_8b_prefill_fp16_causal", B=4, H=32, N=2048, D=128, dtype=torch.float16,
            causal=True, seed=1, mul=0.5, backward=False),
    3: dict(name="training_fwd_bwd_bf16_causal", B=4, H=32, N=4096, D=128, dtype=torch.bfloat16,
            causal=True, seed=2, mul=0.5, backward=True),
    4: dict(name="long_context_bf16_noncausal", B=1, H=16, N=16384, D=64, dtype=torch.bfloat16,
            causal=False, seed=3, mul=1.0, backward=True),
    5: dict(name="chunked_prefill_varlen_gqa_bf16", B=8, Hq=32, Hkv=8, D=128, chunk=512,
            prefix=(1024, 8192), dtype=torch.bfloat16, causal=True, seed=4, mul=0.5, backward=False),
}


def make_config_inputs(cfg_id, device="cpu", shape_override=None):
    """Returns a dict with q, k, v (and do for backward configs) for configs
    1-4, laid out [B, H, N, D]. shape_override=(B, H, N, D) keeps the recipe
    (seed, order, scale, perturbation) at a smaller shape for tests."""
    cfg = CONFIGS[cfg_id]
    assert cfg_id in (1, 2, 3, 4), "config 5 is varlen: use make_varlen_inputs"
    B, H, N, D = shape_override or (cfg["B"], cfg["H"], cfg["N"], cfg["D"])
    g = torch.Generator().manual_seed(cfg["seed"])
    q = torch.randn(B, H, N, D, generator=g) * cfg["mul"]
    k = torch.randn(B, H, N, D, generator=g) * cfg["mul"]
    v = torch.randn(B, H, N, D, generator=g) * cfg["mul"]
    out = {}
    if cfg["backward"]:
        out["do"] = torch.randn(B, H, N, D, generator=g)
    if cfg_id == 4:
        idx = torch.randperm(N, generator=g)[: max(1, N // 100)]
        k[:, :, idx, :] *= 8.0
        out["scaled_rows"] = idx
    dt = cfg["dtype"]
    out.update(q=q.to(dt).to(device), k=k.to(dt).to(device), v=v.to(dt).to(device))
    if "do" in out:
        out["do"] = out["do"].to(dt).to(device)
    out["causal"] = cfg["causal"]
    return out


def make_varlen_inputs(cfg_id=5, device="cpu", batch=None, chunk=None, prefix=None, heads=None, D=None):
    """Config 5: packed THD inputs. Draw order: prefix lengths P_b (uniform in
    [lo, hi]), then q [B*chunk, Hq, D], k and v [sum(P_b + chunk), Hkv, D].
    Keyword overrides shrink the problem for tests with the same recipe."""
    cfg = CONFIGS[cfg_id]
    B = batch or cfg["B"]
    C = chunk or cfg["chunk"]
    lo, hi = prefix or cfg["prefix"]
    Hq, Hkv = heads or (cfg["Hq"], cfg["Hkv"])
    D = D or cfg["D"]
    g = torch.Generator().manual_seed(cfg["seed"])
    P = torch.randint(lo, hi + 1, (B,), generator=g)
    lens_k = P + C
    cu_q = torch.arange(0, (B + 1) * C, C, dtype=torch.int32)
    cu_k = torch.zeros(B + 1, dtype=torch.int32)
    cu_k[1:] = torch.cumsum(lens_k, 0).to(torch.int32)
    Tq, Tk = int(cu_q[-1]), int(cu_k[-1])
    q = torch.randn(Tq, Hq, D, generator=g) * cfg["mul"]
    k = torch.randn(Tk, Hkv, D, generator=g) * cfg["mul"]
    v = torch.randn(Tk, Hkv, D, generator=g) * cfg["mul"]
    dt = cfg["dtype"]
    return dict(q=q.to(dt).to(device), k=k.to(dt).to(device), v=v.to(dt).to(device),
                cu_seqlens_q=cu_q.to(device), cu_seqlens_k=cu_k.to(device),
                max_seqlen_q=C, max_seqlen_k=int(lens_k.max()), prefix=P, causal=True)


def fwd_flops(B, H, N, D, causal):
    """The reference's count (kernels/benchmark_flash_attention.py:55-64)."""
    f = 4 * B * H * N * N * D
    return f // 2 if causal else f


def bwd_flops(B, H, N, D, causal):
    """kernels/benchmark_flash_attention_backward.py:65-68: 2.5x the forward."""
    return fwd_flops(B, H, N, D, causal) * 5 // 2


def varlen_fwd_flops(cu_q, cu_k, Hq, D):
    """Exact count for bottom-right causal varlen: 4*D*Hq*sum_b sum_i (P_b + i + 1)."""
    total = 0
    for b in range(len(cu_q) - 1):
        nq = int(cu_q[b + 1] - cu_q[b])
        nk = int(cu_k[b + 1] - cu_k[b])
        p = nk - nq
        total += nq * p + nq * (nq + 1) // 2
    return 4 * D * Hq * total
