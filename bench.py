"""Benchmark of the gfx950 FlashAttention hot path (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config 3] [--no-cpu-baseline]

A step is one pass of the training hot path over one batch of synthetic
input: forward with logsumexp, then backward (dQ, dK, dV), on the benchmark
config 3 (causal bf16, B=4, H=32, N=4096, D=128, q/k/v ~ N(0,1)*0.5, dO ~
N(0,1), seed 2) by default; --config 2/4/5 time the other configurations
(forward only for 2 and 5). Inputs are resident in HBM before the timed
region. FLOPs follow the reference's convention
(kernels/benchmark_flash_attention.py:55-64,
kernels/benchmark_flash_attention_backward.py:65-68): F_fwd = 4*B*H*N^2*D,
halved when causal; F_bwd = 2.5*F_fwd; a fwd+bwd step counts 3.5*F_fwd.

Timing: W untimed warm-up steps, continued (untimed) until at least 200 ms
of GPU work has gone into the warm-up (the reference's do_bench also warms up
by time; an MI355X coming out of idle runs short kernels up to ~20% slower
until tens of ms of sustained load have passed); then K steps back to back, bracketed by
torch.cuda.synchronize() on both sides, with one pair of HIP events on the
launch stream around them (ms_per_step = their interval / K). For training
steps a second pass with an event between the forward and the backward of
each step gives the forward's share; forward-only steps take the forward
time from the timed region itself. Correctness is re-checked against the
oracle on every (batch, head) slice before timing, as the reference does
(kernels/benchmark_flash_attention.py:104-106): o and lse, and dq/dk/dv when
the step has a backward, all gated.

The CPU baseline is the reference's test oracle (F.scaled_dot_product_attention
in fp32 with autograd, kernels/tests/test_flash_attention_backward.py:86)
on a bounded sample of heads of the same workload, run on this host's cores
and scaled linearly to the full job.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16/fp16 MFMA: 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0
METRIC = "attention TFLOP/s fwd & fwd+bwd, % of MI355X bf16 MFMA peak, 1 GPU"
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic.txt")


WARM_MS = 200.0


def warm_up(fn, n, stream=None, min_ms=WARM_MS, cap=200000):
    """Runs fn() n times, then more, untimed, until at least min_ms of GPU time
    has gone into the warm-up. Returns the number of calls made."""
    import torch

    done, runs, batch = 0.0, 0, max(1, n)
    while True:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(batch):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        done += e0.elapsed_time(e1)
        runs += batch
        if done >= min_ms or runs >= cap:
            return runs
        per = max(done / runs, 1e-3)
        batch = min(cap - runs, max(1, int(math.ceil((min_ms - done) / per))))


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3, 4, 5])
    ap.add_argument("--workload", default="attention",
                    choices=["attention", "decode", "prefill", "rope", "rmsnorm", "gemv", "sweep"],
                    help="attention: a benchmark config 2-5 (default 3); decode: a paged-KV decode step; "
                         "prefill: config 5's chunks over a paged KV cache; "
                         "rope: in-place RoPE of config 3's q and k projections; "
                         "rmsnorm: fused residual add + RMSNorm, [2048, 8192] bf16; "
                         "sweep: B=1 H=32 D=128 bf16 over N 512-8192 beside torch's SDPA")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="config 3: skip the compact runs of configs 2, 4 and 5 added to its line")
    ap.add_argument("--skip-parity", action="store_true",
                    help="skip the oracle re-check before timing (profiler runs only, whose per-kernel counters "
                         "should cover the timed kernels; the JSON line then says parity was not checked)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="rmsnorm: skip the sweep over the reference's other shapes (profiler runs, whose "
                         "per-kernel averages must cover the headline shape only)")
    ap.add_argument("--cpu-heads", type=int, default=128,
                    help="(batch, head) slices in the CPU-baseline sample (bounded by memory; ~10 s of CPU work)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="before the warm-up, run 3 plain device copies of MIB MiB each (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counters to bytes)")
    return ap.parse_args()


def measured_traffic(kernel, workload):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (profiles/hbm_traffic.txt: `kernel workload bytes_per_launch`), or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        parts = line.split()
        if len(parts) >= 3 and not line.startswith("#") and parts[0] == kernel and parts[1] == workload:
            return float(parts[2])
    return None


def fwd_kernel_name(B, H, Nq, Nk, D, causal, dtype):
    """The forward kernel the library launches for a dense call (the host
    dispatch of lightserve_amd/csrc/fa_fwd.hip, launch_fwd and
    persist_balanced): the persistent 8-wave kernel from 4096 queries (2048
    at head dims above 64) when every CU gets at least four (b, h, 256-row
    tile) items (at most 64) that split evenly over the 8 XCDs, every item
    has two key tiles and, when causal, the fixed split's largest workgroup
    holds at most 2% more key tiles than the mean; else the
    one-workgroup-per-item kernel."""
    import torch
    dp = 32 if D <= 32 else (64 if D <= 64 else 128)
    if dtype == torch.float32 or dp < 64 or Nq < (2048 if dp >= 128 else 4096):
        return "fa_fwd_kernel"
    nqt = -(-Nq // 256)
    BH = B * H
    total = nqt * BH
    grid = torch.cuda.get_device_properties(0).multi_processor_count // 8 * 8
    PU, T8 = grid // 8, total // 8
    if not (grid >= 8 and total >= 4 * grid and total % 8 == 0 and -(-T8 // PU) <= 64
            and Nk > 64 and (not causal or Nk >= Nq)):
        return "fa_fwd_kernel"
    if not causal:
        return "fa_fwd_persist_kernel"
    hg = max(1, min(16, (8 << 20) // (Nk * dp * 4)))
    off, tot, worst = Nk - Nq, 0, 0
    for x in range(8):
        for u in range(PU):
            w, i = 0, 0
            while True:
                j = i * PU + ((PU - 1 - u) if i & 1 else u)
                if j >= T8:
                    break
                W = x * T8 + j
                g0 = (W // (hg * nqt)) * hg
                level = (W - g0 * nqt) // min(hg, BH - g0)
                q0 = ((nqt - 1 - level) if causal else level) * 256
                w += ((min(q0 + 256 + off, Nk) if causal else Nk) + 63) // 64
                i += 1
            tot += w
            worst = max(worst, w)
    return "fa_fwd_persist_kernel" if worst * 8 * PU * 50 <= tot * 51 else "fa_fwd_kernel"


def check_parity(cfg, inp, outs, slices=None):
    """Oracle check of every (batch, head) slice (fp32 oracle on the GPU), or
    of the given (batch, head) slices.

    o and lse against the closed form; dq/dk/dv against fp32 autograd. The
    gate is max-abs <= 2e-2 and mean-abs <= 2e-3 (lse max-abs <= 1e-3); a
    gradient that misses it passes only if it is within 1.5x of the error of
    the reference's own algorithm (the restated tiled backward with its bf16
    rounding points of P and dS), the rule the parity tests apply."""
    import torch
    from oracle.attention import attention_grads, attention_reference, flash_backward_tiled
    q, k, v, causal = inp["q"], inp["k"], inp["v"], inp["causal"]
    B, H = q.shape[:2]
    stats = {}  # name -> [max, sum of per-slice means, slices]

    def add(key, got, ref):
        err = (got.double() - ref.double()).abs()
        st = stats.setdefault(key, [0.0, 0.0, 0])
        st[0] = max(st[0], err.max().item())
        st[1] += err.mean().item()
        st[2] += 1

    if slices is None:
        slices = [(b, h) for b in range(B) for h in range(H)]
    for b, h in slices:
        sl = (slice(b, b + 1), slice(h, h + 1))
        o_ref, lse_ref = attention_reference(q[sl], k[sl], v[sl], causal, dtype=torch.float32)
        add("o", outs["o"][sl], o_ref)
        add("lse", outs["lse"][sl], lse_ref)
        if "dq" in outs:
            exact = attention_grads(q[sl], k[sl], v[sl], inp["do"][sl], causal, dtype=torch.float32)
            alg = flash_backward_tiled(q[sl], k[sl], v[sl], o_ref.to(q.dtype), lse_ref, inp["do"][sl], causal,
                                       block_n=256, op_dtype=q.dtype)
            for name, ex, ra in zip(("dq", "dk", "dv"), exact, alg):
                add(name, outs[name][sl], ex)
                add(name + "_ref_alg", ra.to(q.dtype), ex)
    res = {n: {"max_abs": float(f"{m:.3e}"), "mean_abs": float(f"{t / c:.3e}")} for n, (m, t, c) in stats.items()}
    ok = res["o"]["max_abs"] <= 2e-2 and res["o"]["mean_abs"] <= 2e-3 and res["lse"]["max_abs"] <= 1e-3
    for name in ("dq", "dk", "dv"):
        if name not in res:
            continue
        r, a = res[name], res.pop(name + "_ref_alg")
        gate = r["max_abs"] <= 2e-2 and r["mean_abs"] <= 2e-3
        rel = r["max_abs"] <= 1.5 * a["max_abs"] and r["mean_abs"] <= 1.5 * a["mean_abs"]
        r["rule"] = "gate" if gate else ("1.5x reference algorithm" if rel else "failed")
        r["reference_algorithm"] = a
        ok = ok and (gate or rel)
    res["slices_checked"] = len(slices)
    return ok, res


def cpu_baseline(cfg, inp, n_heads, flops_full, step_kind):
    """Times F.scaled_dot_product_attention (fp32, CPU) on n_heads heads of the
    workload (1 warm-up, median of 5) and scales to the full job."""
    import torch
    import torch.nn.functional as F
    B, H, N = inp["q"].shape[:3]
    # at most ~8 GB of fp32 score matrices (autograd keeps a few of them)
    n_heads = max(1, min(n_heads, B * H, int(8e9 // (N * N * 4))))

    def sample(t):  # the first n_heads (batch, head) slices, as [1, n_heads, N, D]
        return t.reshape(1, B * H, *t.shape[2:])[:, :n_heads].float().cpu()

    q, k, v = (sample(inp[n]) for n in ("q", "k", "v"))
    do = sample(inp["do"]) if "do" in inp else None
    causal = inp["causal"]

    def run():
        if step_kind == "fwd+bwd":
            qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
            F.scaled_dot_product_attention(qq, kk, vv, is_causal=causal).backward(do)
        else:
            F.scaled_dot_product_attention(q, k, v, is_causal=causal)

    run()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    total_heads = inp["q"].shape[0] * inp["q"].shape[1]
    full_s = t * total_heads / n_heads
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(flops_full / full_s / 1e12, 4), "unit": "TFLOP/s",
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"F.scaled_dot_product_attention fp32 {step_kind} on {n_heads} of {total_heads} (b,h) heads "
                   f"(1 warm-up, median of 5: {t:.2f} s), scaled linearly; os.cpu_count()={os.cpu_count()}; "
                   f"{cpu_model}"),
    }


# (batch, head) slices the compact runs of configs 2 and 4 check against the oracle
OTHER_CONFIG_SLICES = {2: [(0, 0), (1, 9), (2, 18), (3, 31)], 4: [(0, 0), (0, 5), (0, 10), (0, 15)]}


def other_configs(steps, warmup):
    """Configs 2, 4 and 5 timed back to back after the headline config, each
    the way --config N times it (W warm-up steps continued until 200 ms of GPU
    work, then `steps` steps between one event pair; config 4's forward share
    from a second pass with an event between forward and backward), with
    parity on a fixed sample: four (batch, head) slices of configs 2 and 4
    (o, lse; dq/dk/dv at config 4) and two whole sequences of config 5 (o and
    lse of every query head). Compact: no CPU baseline, no per-kernel split."""
    import torch
    from lightserve_amd.kernels.flash_attention_backward import (_flash_attention_backward,
                                                                 _flash_attention_forward_lse)
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
    from lightserve_amd.workloads import CONFIGS, bwd_flops, fwd_flops, make_config_inputs, make_varlen_inputs, \
        varlen_fwd_flops
    from oracle.attention import attention_reference
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    out = {}
    for c in (2, 4, 5):
        cfg = CONFIGS[c]
        t_cfg = time.perf_counter()
        if c == 5:
            inp = make_varlen_inputs(device=dev)
            q, k, v = inp["q"], inp["k"], inp["v"]
            cu_q, cu_k = inp["cu_seqlens_q"], inp["cu_seqlens_k"]
            f_fwd = varlen_fwd_flops(cu_q.cpu(), cu_k.cpu(), cfg["Hq"], cfg["D"])
            f_step, bwd = f_fwd, None

            def fwd():
                return flash_attention_varlen_forward(q, k, v, cu_q, cu_k, inp["max_seqlen_q"], inp["max_seqlen_k"])
        else:
            inp = make_config_inputs(c, device=dev)
            q, k, v, causal = inp["q"], inp["k"], inp["v"], inp["causal"]
            f_fwd = fwd_flops(*q.shape, causal)
            f_step = f_fwd + (bwd_flops(*q.shape, causal) if cfg["backward"] else 0)

            def fwd():
                return _flash_attention_forward_lse(q, k, v, causal)
            bwd = (lambda o, lse: _flash_attention_backward(inp["do"], q, k, v, o, lse, causal)) \
                if cfg["backward"] else None
        o, lse = fwd()
        outs = {"o": o, "lse": lse}
        if bwd is not None:
            outs["dq"], outs["dk"], outs["dv"] = bwd(o, lse)
        torch.cuda.synchronize()
        if c == 5:
            cq, ck = cu_q.tolist(), cu_k.tolist()
            G = cfg["Hq"] // cfg["Hkv"]
            worst = {"o": [0.0, 0.0], "lse": [0.0, 0.0]}
            for b in (0, len(cq) - 2):
                qb = q[cq[b]:cq[b + 1]].transpose(0, 1)[None]
                kb = k[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(G, 0)[None]
                vb = v[ck[b]:ck[b + 1]].transpose(0, 1).repeat_interleave(G, 0)[None]
                o_ref, l_ref = attention_reference(qb, kb, vb, True, dtype=torch.float32)
                for name, got, ref in (("o", o[cq[b]:cq[b + 1]].transpose(0, 1)[None], o_ref),
                                       ("lse", lse[:, cq[b]:cq[b + 1]][None], l_ref)):
                    err = (got.double() - ref.double()).abs()
                    worst[name] = [max(worst[name][0], err.max().item()), max(worst[name][1], err.mean().item())]
            parity = {n: {"max_abs": float(f"{w[0]:.3e}"), "mean_abs": float(f"{w[1]:.3e}")} for n, w in worst.items()}
            parity["sequences_checked"] = 2
            ok = worst["o"][0] <= 2e-2 and worst["o"][1] <= 2e-3 and worst["lse"][0] <= 1e-3
        else:
            ok, parity = check_parity(cfg, inp, outs, OTHER_CONFIG_SLICES[c])
        del outs

        def step():
            o, lse = fwd()
            if bwd is not None:
                bwd(o, lse)

        warm_up(step, warmup, stream)
        h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        h0.record(stream)
        for _ in range(steps):
            step()
        h1.record(stream)
        torch.cuda.synchronize()
        ms = h0.elapsed_time(h1) / steps
        tf = f_step / (ms * 1e-3) / 1e12
        r = {"workload": cfg["name"], "step": "fwd+bwd" if bwd is not None else "fwd",
             "ms_per_step": round(ms, 5), "tflops": round(tf, 2), "pct_of_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2)}
        if bwd is not None:
            ev = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
            torch.cuda.synchronize()
            for e0, e1, e2 in ev:
                e0.record(stream)
                o, lse = fwd()
                e1.record(stream)
                bwd(o, lse)
                e2.record(stream)
            torch.cuda.synchronize()
            fms = sum(a.elapsed_time(b) for a, b, _ in ev) / steps
            bms = sum(b.elapsed_time(c) for _, b, c in ev) / steps
            r["fwd"] = {"ms": round(fms, 5), "pct_of_peak": round(100 * f_fwd / (fms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)}
            fb = f_step - f_fwd
            r["bwd"] = {"ms": round(bms, 5), "pct_of_peak": round(100 * fb / (bms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)}
        r["parity"] = {"ok": bool(ok), **parity}
        r["wall_s"] = round(time.perf_counter() - t_cfg, 2)
        out[f"config{c}"] = r
        del inp, q, k, v, o, lse
        torch.cuda.empty_cache()
    return out


def calibration_copy(dev, mib):
    """A plain device copy of known size (reads and writes exactly mib MiB),
    the reference kernel for scaling FETCH_SIZE / WRITE_SIZE counters."""
    if mib <= 0:
        return
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


DECODE = dict(batch=32, heads_q=32, heads_kv=8, head_dim=128, block_size=16, min_len=1024, max_len=8192, seed=4)


def bench_decode(args):
    """One paged-KV decode step (Llama-3-8B shapes, a batch of 32 sequences
    with context lengths uniform in [1024, 8192], seed 4, blocks scattered
    over a shuffled cache pool). HBM-bound: the metric is K/V bytes streamed
    per second."""
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.paged_attention import paged_attention_decode
    from oracle.attention import paged_decode_reference

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    c = DECODE
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(c["seed"])
    B, Hq, Hkv, D, bs = c["batch"], c["heads_q"], c["heads_kv"], c["head_dim"], c["block_size"]
    lens = torch.randint(c["min_len"], c["max_len"] + 1, (B,), generator=g)
    nblk = (lens + bs - 1) // bs
    num_blocks = int(nblk.sum())
    perm = torch.randperm(num_blocks, generator=g).to(torch.int32)
    table = torch.zeros(B, int(nblk.max()), dtype=torch.int32)
    at = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[at:at + int(nblk[b])]
        at += int(nblk[b])
    q = (torch.randn(B, Hq, D, generator=g) * 0.5).to(torch.bfloat16)
    kc = (torch.randn(num_blocks, bs, Hkv, D, generator=g) * 0.5).to(torch.bfloat16)
    vc = torch.randn(num_blocks, bs, Hkv, D, generator=g).to(torch.bfloat16)
    qd, kd, vd, td = q.to(dev), kc.to(dev), vc.to(dev), table.to(dev)
    sl = lens.to(torch.int32).to(dev)
    max_len = int(lens.max())

    def step():
        return paged_attention_decode(qd, kd, vd, td, sl, max_seq_len=max_len, return_lse=True)

    o, lse = step()
    torch.cuda.synchronize()
    worst = {"o": [0.0, 0.0], "lse": [0.0, 0.0]}
    for b in (0, B - 1):  # oracle check of two sequences
        o_ref, lse_ref = paged_decode_reference(q[b:b + 1], kc, vc, table[b:b + 1], lens[b:b + 1].to(torch.int32))
        for name, got, ref in (("o", o[b:b + 1].cpu(), o_ref), ("lse", lse[b:b + 1].cpu(), lse_ref)):
            err = (got.double() - ref.double()).abs()
            worst[name] = [max(worst[name][0], err.max().item()), max(worst[name][1], err.mean().item())]
    parity = {n: {"max_abs": float(f"{v[0]:.3e}"), "mean_abs": float(f"{v[1]:.3e}")} for n, v in worst.items()}
    parity_ok = worst["o"][0] <= 2e-2 and worst["o"][1] <= 2e-3 and worst["lse"][0] <= 1e-3

    calibration_copy(dev, args.calibrate_copy)
    warm_runs = warm_up(step, args.warmup)
    # A decode step lasts ~0.1 ms, so the steps are enqueued back to back
    # between one event pair (as a serving loop issues them): per-step event
    # pairs would count the host's Python time before each launch.
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    steps = max(args.steps, 200)  # 20 steps of ~0.1 ms are too short to time
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    tokens = int(lens.sum())
    kv_bytes = tokens * Hkv * D * 2 * 2          # K and V rows, bf16
    other_bytes = B * Hq * D * 2 * 2 + B * Hq * 4 + table.numel() * 4 + B * 4  # q, o, lse, tables, lens
    alg_bytes = kv_bytes + other_bytes
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "paged-KV decode attention: algorithmic HBM GB/s (K/V streamed), 1 GPU",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_calls": warm_runs,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": f"synthetic, seeded (seed {c['seed']}), cache resident in HBM",
        "config": {"workload": (f"decode: B={B} Hq={Hq} Hkv={Hkv} D={D} block_size={bs} "
                                f"context uniform in [{c['min_len']}, {c['max_len']}] ({tokens} cached tokens)"),
                   "bytes_per_step": alg_bytes},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": parity_ok, **parity},
        "roofline": {"kernel": "fa_decode_split_kernel (+ fa_decode_combine_kernel)", "bound": "hbm",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic("fa_decode_split_kernel", "decode"),
                     "bytes_per_launch": alg_bytes, "avg_launch_ms": round(ms, 5)},
    }
    if not args.no_cpu_baseline:
        # the oracle's gather + closed form in fp32 on the host cores, on a sample of sequences
        n_cpu = 8
        t_start = time.perf_counter()
        reps = 0
        while True:
            paged_decode_reference(q[:n_cpu], kc, vc, table[:n_cpu], lens[:n_cpu].to(torch.int32), dtype=torch.float32)
            reps += 1
            if time.perf_counter() - t_start > 5.0:
                break
        t = (time.perf_counter() - t_start) / reps
        sample_bytes = int(lens[:n_cpu].sum()) * Hkv * D * 2 * 2
        result["cpu_baseline"] = {
            "value": round(sample_bytes / t / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"oracle paged_decode_reference (gather + closed form, fp32) on {n_cpu} of {B} sequences, "
                       f"{reps} repetitions in {time.perf_counter() - t_start:.1f} s"),
        }
    print(json.dumps(result), flush=True)


def bench_rope(args):
    """In-place RoPE of the q and k projections of config 3's shape with
    LLaMA-3's 8 KV heads (q [4, 4096, 32, 128], k [4, 4096, 8, 128] bf16,
    rotated through [B, H, N, D] views), the model's per-layer call. HBM-bound:
    each element of q and k is read and written once."""
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.rope import apply_rope_
    from lightserve_amd.model.minimal_llama import llama3_8b_shape, precompute_rope
    from oracle.model import apply_rope  # parity check only

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda", 0)
    B, N, Hq, Hkv, D = 4, 4096, 32, 8, 128
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, N, Hq, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, N, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    cos, sin = precompute_rope(llama3_8b_shape(max_seq_len=N), dev)  # LLaMA-3 tables, bf16
    qv, kv = q.transpose(1, 2), k.transpose(1, 2)
    # parity on one (batch, head) slice of each, against the oracle in float64
    q0, k0 = qv[:1, :1].double().cpu(), kv[:1, :1].double().cpu()
    apply_rope_(qv, kv, cos, sin)
    torch.cuda.synchronize()
    qr, kr = apply_rope(q0, k0, cos.double().cpu(), sin.double().cpu(), N)
    err = max((qv[:1, :1].double().cpu() - qr).abs().max().item(), (kv[:1, :1].double().cpu() - kr).abs().max().item())
    calibration_copy(dev, args.calibrate_copy)
    warm_runs = warm_up(lambda: apply_rope_(qv, kv, cos, sin), args.warmup)
    stream = torch.cuda.current_stream(dev)
    steps = max(args.steps, 200)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        apply_rope_(qv, kv, cos, sin)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    alg_bytes = 2 * (q.numel() + k.numel()) * 2 + 2 * N * D * 2  # q, k read and written; cos/sin rows read
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "RoPE of q and k in place: algorithmic HBM GB/s, 1 GPU", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_calls": warm_runs, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic, seeded (seed 2), resident in HBM",
        "config": {"workload": f"rope: q [{B},{N},{Hq},{D}] and k [{B},{N},{Hkv},{D}] bf16 as [B,H,N,D] views",
                   "bytes_per_step": alg_bytes},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": err <= 2 ** -8 * 8, "max_abs_vs_float64": float(f"{err:.3e}")},
        "roofline": {"kernel": "fa_rope_kernel", "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("fa_rope_kernel", "rope"), "bytes_per_launch": alg_bytes,
                     "avg_launch_ms": round(ms, 5)},
    }))


def bench_prefill(args):
    """Chunked prefill over a paged KV cache (lsfa_prefill_paged): benchmark
    config 5's workload (B=8, Hq=32, Hkv=8, D=128, a 512-token chunk after a
    prefix of 1024..8192 tokens per sequence, bf16, seed 4) with each
    sequence's K/V in a cache of 16-token blocks handed out in a shuffled
    order, as the engine's block manager does. Same FLOPs as config 5; the
    packed varlen forward on the same K/V is timed in the same process. The
    timed loops call the C ABI with prebuilt arguments."""
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
    from lightserve_amd.kernels.paged_attention import paged_prefill
    from lightserve_amd.workloads import CONFIGS, make_varlen_inputs, varlen_fwd_flops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda", 0)
    cfg = CONFIGS[5]
    inp = make_varlen_inputs(device=dev)
    q, k, v = inp["q"], inp["k"], inp["v"]
    cu_q, cu_k = inp["cu_seqlens_q"], inp["cu_seqlens_k"]
    B, Hq, Hkv, D, bs = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"], 16
    lens_k = (cu_k[1:] - cu_k[:-1]).cpu()
    nblk = (lens_k + bs - 1) // bs
    num_blocks = int(nblk.sum())
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(5))
    max_blocks = int(nblk.max())
    table = torch.zeros(B, max_blocks, dtype=torch.int32)
    slot_of_token = []
    at = 0
    for b in range(B):
        n = int(nblk[b])
        table[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
        t = torch.arange(int(lens_k[b]))
        slot_of_token.append(table[b, t // bs].long() * bs + t % bs)
    slots = torch.cat(slot_of_token).to(dev)
    kc = torch.zeros(num_blocks * bs, Hkv, D, dtype=q.dtype, device=dev)
    vc = torch.zeros_like(kc)
    kc.index_copy_(0, slots, k)
    vc.index_copy_(0, slots, v)
    kc, vc = kc.view(num_blocks, bs, Hkv, D), vc.view(num_blocks, bs, Hkv, D)
    table, seq_lens_k = table.to(dev), lens_k.to(torch.int32).to(dev)
    f_fwd = varlen_fwd_flops(cu_q.cpu(), cu_k.cpu(), Hq, D)

    o, lse = paged_prefill(q, kc, vc, table, cu_q, seq_lens_k, max_seqlen_q=cfg["chunk"], return_lse=True)
    o_ref, lse_ref = flash_attention_varlen_forward(q, k, v, cu_q, cu_k, cfg["chunk"], inp["max_seqlen_k"])
    torch.cuda.synchronize()
    bit_identical = bool(torch.equal(o, o_ref) and torch.equal(lse, lse_ref))
    # the oracle on one sequence's first query head (parity of the packed path is covered by the tests)
    from oracle.attention import paged_prefill_reference
    b0 = 0
    rows = slice(int(cu_q[b0]), int(cu_q[b0 + 1]))
    o1, l1 = paged_prefill_reference(q[rows][:, :1].float().cpu(), kc[:, :, :1].float().cpu(),
                                     vc[:, :, :1].float().cpu(), table[b0:b0 + 1].cpu(),
                                     torch.tensor([0, rows.stop - rows.start], dtype=torch.int32),
                                     seq_lens_k[b0:b0 + 1].cpu(), True, dtype=torch.float32)
    err = (o[rows][:, :1].float().cpu() - o1).abs()
    lerr = (lse[:1, rows].cpu() - l1).abs().max().item()
    parity_ok = bit_identical and err.max().item() <= 2e-2 and err.mean().item() <= 2e-3 and lerr <= 1e-3

    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    pa = _lib.PrefillPagedArgs(
        q=q.data_ptr(), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(), o=o.data_ptr(), lse=lse.data_ptr(),
        cu_seqlens_q=cu_q.data_ptr(), seq_lens_k=seq_lens_k.data_ptr(), block_tables=table.data_ptr(),
        q_stride=_lib._i64x2(*q.stride()[:2]), k_stride=_lib._i64x3(*kc.stride()[:3]),
        v_stride=_lib._i64x3(*vc.stride()[:3]), o_stride=_lib._i64x2(*o.stride()[:2]),
        lse_stride=_lib._i64x2(*lse.stride()), block_table_stride=table.stride(0), dtype=_lib.DTYPE_BF16,
        batch=B, heads_q=Hq, heads_kv=Hkv, head_dim=D, block_size=bs, num_blocks=num_blocks,
        max_blocks_per_seq=max_blocks, max_seqlen_q=cfg["chunk"], causal=1, sm_scale=1 / D ** 0.5, reserved=0)
    fa = _lib.FwdArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), o=o_ref.data_ptr(), lse=lse_ref.data_ptr(),
        q_stride=_lib.strides_thd(q), k_stride=_lib.strides_thd(k), v_stride=_lib.strides_thd(v),
        o_stride=_lib.strides_thd(o_ref), lse_stride=_lib._i64x3(0, lse_ref.stride(0), lse_ref.stride(1)),
        cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_k=cu_k.data_ptr(), dtype=_lib.DTYPE_BF16, batch=B, heads_q=Hq,
        heads_kv=Hkv, seqlen_q=cfg["chunk"], seqlen_k=inp["max_seqlen_k"], head_dim=D, causal=1,
        sm_scale=1 / D ** 0.5, reserved=0)
    calibration_copy(dev, args.calibrate_copy)

    def timed(fn, n):
        warm_up(fn, args.warmup, stream)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record(stream)
        for _ in range(n):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n

    steps = max(args.steps, 50)
    t0 = time.perf_counter()
    ms = timed(lambda: _lib.prefill_paged(pa, sptr), steps)
    wall = time.perf_counter() - t0
    ms_packed = timed(lambda: _lib.fwd(fa, sptr), steps)
    tf = f_fwd / (ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        # the oracle (gather + closed form, fp32, the host's cores) on one sequence's 4 query heads of one
        # KV group, scaled by FLOPs to the whole job
        b1, hs = B - 1, 4
        rows1 = slice(int(cu_q[b1]), int(cu_q[b1 + 1]))
        qs = q[rows1][:, :hs].float().cpu()
        ks, vs = kc[:, :, :1].float().cpu(), vc[:, :, :1].float().cpu()
        tb, cu1, sl1 = table[b1:b1 + 1].cpu(), torch.tensor([0, 512], dtype=torch.int32), seq_lens_k[b1:b1 + 1].cpu()
        paged_prefill_reference(qs, ks, vs, tb, cu1, sl1, True, dtype=torch.float32)
        ts = []
        for _ in range(3):
            c0 = time.perf_counter()
            paged_prefill_reference(qs, ks, vs, tb, cu1, sl1, True, dtype=torch.float32)
            ts.append(time.perf_counter() - c0)
        tc = sorted(ts)[1]
        nk1 = int(seq_lens_k[b1])
        f_sample = 4 * D * hs * (512 * (nk1 - 512) + 512 * 513 // 2)
        cpu = {"value": round(f_sample / tc / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": (f"oracle paged_prefill_reference (block-table gather + closed form, fp32) "
                                          f"on sequence {b1}'s 4 query heads of KV head 0 ({nk1} keys), median of "
                                          f"3: {tc:.2f} s, scaled by FLOPs")}
    print(json.dumps({
        "metric": "chunked prefill over a paged KV cache: attention TFLOP/s, % of MI355X bf16 MFMA peak, 1 GPU",
        "value": round(tf, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic, config 5 recipe (seed 4), cache blocks shuffled (seed 5), resident in HBM",
        "config": {"workload": (f"prefill: config-5 chunks (B={B} Hq={Hq} Hkv={Hkv} D={D} chunk 512, prefixes "
                                f"{int(lens_k.min()) - 512}..{int(lens_k.max()) - 512}) over a {num_blocks}-block "
                                f"cache of {bs}-token blocks"), "flops_per_step": f_fwd},
        "pct_of_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2),
        "packed_varlen_same_kv": {"ms": round(ms_packed, 5),
                                  "tflops": round(f_fwd / (ms_packed * 1e-3) / 1e12, 2)},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": bool(parity_ok), "bit_identical_to_packed_varlen": bit_identical,
                   "max_abs_vs_oracle_seq0_head0": float(f"{err.max().item():.3e}"),
                   "lse_max_abs": float(f"{lerr:.3e}")},
        "roofline": {"kernel": "fa_fwd_kernel<bf16,128,causal,varlen,LSE,paged>", "bound": "mfma",
                     "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic("fa_fwd_kernel", "prefill"),
                     "flops_per_launch": f_fwd, "avg_launch_ms": round(ms, 5)},
        "cpu_baseline": cpu,
    }), flush=True)


RMSNORM_SHAPES = [(1, 4096), (8, 4096), (128, 4096), (2048, 4096), (1, 8192), (128, 8192), (2048, 8192)]


def bench_rmsnorm(args):
    """Fused residual add + RMSNorm (lsfa_rmsnorm) at the reference benchmark's
    largest shape, x and residual [2048, 8192] bf16
    (kernels/benchmark_fused_rmsnorm_residual.py:30). HBM-bound: x and residual
    read, h and out written, 4 * M * N elements (the weight row stays in
    cache). The timed loop calls the C ABI with prebuilt arguments, so the
    host issues launches faster than the kernel retires them; the reference's
    other shapes are reported under "sweep" through the Python entry point
    (the reference's timing method: events around back-to-back calls)."""
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.fused_rmsnorm_residual import fused_add_rmsnorm
    from oracle.model import add_rmsnorm_reference  # parity check and CPU baseline only

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda", 0)
    M, N, eps = 2048, 8192, 1e-6
    g = torch.Generator().manual_seed(3)
    x_h = torch.randn(M, N, generator=g).to(torch.bfloat16)
    r_h = torch.randn(M, N, generator=g).to(torch.bfloat16)
    w_h = torch.randn(N, generator=g).to(torch.bfloat16)
    x, r, w = x_h.to(dev), r_h.to(dev), w_h.to(dev)
    out, h = fused_add_rmsnorm(x, r, w, eps)
    torch.cuda.synchronize()
    ref_out, ref_h = add_rmsnorm_reference(x_h[:64], r_h[:64], w_h, eps)
    err = (out[:64].cpu().float() - ref_out.float()).abs().max().item()
    parity_ok = torch.equal(h[:64].cpu(), ref_h) and err <= 2e-2
    args_c = _lib.RmsNormArgs(x=x.data_ptr(), residual=r.data_ptr(), weight=w.data_ptr(), out=out.data_ptr(),
                              residual_out=h.data_ptr(), x_stride=N, residual_stride=N, out_stride=N,
                              residual_out_stride=N, dtype=_lib.TORCH_TO_LSFA[torch.bfloat16], rows=M, cols=N,
                              eps=eps)
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    calibration_copy(dev, args.calibrate_copy)
    warm_runs = warm_up(lambda: _lib.rmsnorm(args_c, sptr), args.warmup, stream)
    steps = max(args.steps, 200)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        _lib.rmsnorm(args_c, sptr)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    alg_bytes = 4 * M * N * 2 + N * 2
    gbs = alg_bytes / (ms * 1e-3) / 1e9

    def per_call_ms(fn, iters=100):
        for _ in range(10):
            fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record(stream)
        for _ in range(iters):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters

    sweep = []
    for (m, n) in ([] if args.no_sweep else RMSNORM_SHAPES):
        for dt in (torch.float32, torch.bfloat16):
            xs = torch.randn(m, n, device=dev, dtype=dt)
            rs = torch.randn(m, n, device=dev, dtype=dt)
            ws = torch.randn(n, device=dev, dtype=dt)
            t_fused = per_call_ms(lambda: fused_add_rmsnorm(xs, rs, ws, eps))
            t_naive = per_call_ms(lambda: add_rmsnorm_reference(xs, rs, ws, eps))  # torch ops on the GPU
            b = 4 * m * n * xs.element_size()
            sweep.append({"shape": f"{m}x{n}", "dtype": str(dt)[6:], "fused_ms": round(t_fused, 5),
                          "torch_unfused_ms": round(t_naive, 5), "fused_gbs": round(b / (t_fused * 1e-3) / 1e9, 1)})
            del xs, rs, ws

    cpu = None
    if not args.no_cpu_baseline:
        add_rmsnorm_reference(x_h[:256], r_h[:256], w_h, eps)
        t = []
        for _ in range(5):
            c0 = time.perf_counter()
            add_rmsnorm_reference(x_h, r_h, w_h, eps)
            t.append(time.perf_counter() - c0)
        tc = sorted(t)[2]
        cpu = {"value": round(alg_bytes / tc / 1e9, 2), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": (f"oracle add_rmsnorm_reference (torch CPU ops) on the full {M}x{N} bf16 "
                                          f"workload, median of 5: {tc * 1e3:.1f} ms")}
    print(json.dumps({
        "metric": "fused add + RMSNorm: algorithmic HBM GB/s, 1 GPU", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_calls": warm_runs, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic, seeded (seed 3), resident in HBM",
        "config": {"workload": f"rmsnorm: fused_add_rmsnorm x, residual [{M},{N}] bf16, eps {eps}",
                   "bytes_per_step": alg_bytes},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": bool(parity_ok), "max_abs_vs_oracle_first_64_rows": float(f"{err:.3e}")},
        "roofline": {"kernel": "fa_add_rmsnorm_vec_kernel", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("fa_add_rmsnorm_vec_kernel", "rmsnorm"),
                     "bytes_per_launch": alg_bytes, "avg_launch_ms": round(ms, 5)},
        "cpu_baseline": cpu,
        "sweep": sweep,
    }), flush=True)


GEMV_SWEEP = [  # LLaMA-3-8B decode-step projections (hidden 4096, 32 q / 8 kv heads of 128, MLP 14336)
    ("qkv", 4096, (4096, 1024, 1024)), ("o", 4096, (4096,)), ("gate_up", 4096, (14336, 14336)),
    ("down", 14336, (4096,)), ("lm_head", 4096, (128256,))]


def bench_gemv(args):
    """Skinny GEMM of a decode step (lsfa_gemv): the LLaMA-3-8B output
    projection y[1, 128256] = x[1, 4096] @ W[4096, 128256] bf16, the largest
    per-step weight pass. HBM-bound: W (1.05 GB) is read once, x and y are
    noise (algorithmic bytes = K*N*2 + M*K*2 + M*N*2). The timed loop calls the
    C ABI with prebuilt arguments. The sweep times every projection shape of
    the step at batch 1 and 8 (grouped where the decoder groups them) next to
    torch.matmul (hipBLASLt); the skinny kernel is called directly, whatever
    row count tiled_matmul.matmul would route to it."""
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.tiled_matmul import skinny_matmul, skinny_matmul_group

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda", 0)
    M, K, N = 1, 4096, 128256
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(K, N, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    y = skinny_matmul(x, w)
    ref = (x.double() @ w.double())
    torch.cuda.synchronize()
    err = (y.double() - ref).abs()
    parity_ok = bool((err <= ref.abs() * 2.0 ** -7 + 1e-3).all())
    args_c = _lib.GemvArgs(x=x.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), workspace=None, workspace_bytes=0,
                           x_stride=K, w_stride=N, y_stride=N, dtype=_lib.TORCH_TO_LSFA[torch.bfloat16], m=M, k=K,
                           n=N)
    nbytes = _lib.gemv_workspace_size(args_c)
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
    args_c.workspace, args_c.workspace_bytes = ws.data_ptr(), ws.numel()
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    calibration_copy(dev, args.calibrate_copy)
    warm_runs = warm_up(lambda: _lib.gemv(args_c, sptr), args.warmup, stream)
    steps = max(args.steps, 100)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        _lib.gemv(args_c, sptr)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    alg_bytes = K * N * 2 + M * K * 2 + M * N * 2
    gbs = alg_bytes / (ms * 1e-3) / 1e9

    def per_call_ms(fn, iters=50):
        for _ in range(5):
            fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record(stream)
        for _ in range(iters):
            fn()
        e.record(stream)
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters

    sweep = []
    for rows in ([] if args.no_sweep else (1, 2, 3, 4, 8, 16, 32)):
        for name, k, ns in GEMV_SWEEP:
            a = torch.randn(rows, k, device=dev, generator=g).to(torch.bfloat16)
            ws_ = [(torch.randn(k, n, device=dev, generator=g) / k ** 0.5).to(torch.bfloat16) for n in ns]
            t_lib = per_call_ms(lambda: skinny_matmul_group(a, ws_))
            t_blas = per_call_ms(lambda: [torch.matmul(a, b) for b in ws_])
            b = sum(k * n * 2 for n in ns)
            sweep.append({"proj": name, "m": rows, "k": k, "n": list(ns), "lsfa_ms": round(t_lib, 5),
                          "hipblaslt_ms": round(t_blas, 5), "lsfa_gbs": round(b / (t_lib * 1e-3) / 1e9, 1),
                          "hipblaslt_gbs": round(b / (t_blas * 1e-3) / 1e9, 1)})
            del a, ws_

    cpu = None
    if not args.no_cpu_baseline:
        xc, wc = x.float().cpu(), w[:, :16384].float().cpu()  # the checker's product on 16384 of the columns
        xc @ wc
        t = []
        for _ in range(5):
            c0 = time.perf_counter()
            xc @ wc
            t.append(time.perf_counter() - c0)
        tc = sorted(t)[2]
        cpu = {"value": round(K * 16384 * 2 / tc / 1e9, 2), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": (f"torch CPU fp32 x @ W over 16384 of the {N} columns (the same product the "
                                          f"parity check forms in fp64 on the GPU), median of 5: {tc * 1e3:.2f} ms; "
                                          "GB/s counts the bf16 weight bytes")}
    print(json.dumps({
        "metric": "decode skinny GEMM (lm_head): algorithmic HBM GB/s, 1 GPU", "value": round(gbs, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup, "warmup_calls": warm_runs, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic, seeded (seed 5), resident in HBM",
        "config": {"workload": f"gemv: x [{M},{K}] @ W [{K},{N}] bf16 (LLaMA-3-8B lm_head at batch 1)",
                   "bytes_per_step": alg_bytes},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": parity_ok, "max_abs_vs_fp64": float(f"{err.max().item():.3e}")},
        "roofline": {"kernel": "fa_gemv_kernel", "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("fa_gemv_kernel", "gemv"),
                     "bytes_per_launch": alg_bytes, "avg_launch_ms": round(ms, 5)},
        "cpu_baseline": cpu,
        "sweep": sweep,
    }), flush=True)


def bench_sweep(args):
    """Attention sweep beside the vendor kernel on the same GPU, as the
    reference's kernels/benchmark_flash_attention.py:36-110 does: B=1, H=32,
    D=128, bf16, N = 512 ... 8192, causal and not. "vendor" is torch's own
    scaled_dot_product_attention forced onto its flash backend (the
    memory-efficient backend if flash cannot run; the line names which).
    Forward: the inference entry point (flash_attention_forward, no
    logsumexp) against SDPA; backward alone: .backward(retain_graph=True)
    on a graph built once (the reference's backward benchmark,
    kernels/benchmark_flash_attention_backward.py:89-107), flash_attention
    against SDPA; forward+backward: the training pair (forward with L,
    lsfa_bwd) against SDPA under autograd. Outputs and
    gradients are compared with the vendor's before each shape is timed.
    Timing: 10 warm-up calls, then the median of 5 blocks of 30 calls
    (HIP events)."""
    import statistics
    import torch
    import torch.nn.functional as F
    from lightserve_amd.kernels.flash_attention import flash_attention_forward
    from lightserve_amd.kernels.flash_attention_backward import (_flash_attention_backward,
                                                                 _flash_attention_forward_lse, flash_attention)
    from lightserve_amd.workloads import bwd_flops, fwd_flops
    dev = torch.device("cuda", 0)
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
    except ImportError:  # pragma: no cover - torch without the context manager
        SDPBackend = sdpa_kernel = None

    def vendor(q, k, v, causal, backend):
        with sdpa_kernel(backend):
            return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

    def timed(fn, warmup=10, iters=30, repeats=5):
        warm_up(fn, warmup, min_ms=50.0)
        blocks = []
        for _ in range(repeats):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize()
            blocks.append(e0.elapsed_time(e1) / iters)
        return statistics.median(blocks)

    B, H, D = 1, 32, 128
    rows = []
    backend_used = None
    t_start = time.time()
    for n in (512, 1024, 2048, 4096, 8192):
        for causal in (False, True):
            g = torch.Generator(device="cpu").manual_seed(n + int(causal))
            q, k, v, do = (torch.randn(B, H, n, D, generator=g).to(dev, torch.bfloat16) for _ in range(4))
            row = {"shape": f"{B}x{H}x{n}x{D}", "causal": causal}
            ours = flash_attention_forward(q, k, v, causal=causal)
            ref = None
            for be in ((SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION) if SDPBackend else ()):
                try:
                    ref = vendor(q, k, v, causal, be)
                    backend_used = backend_used or str(be).split(".")[-1]
                    vbe = be
                    break
                except RuntimeError:
                    continue
            if ref is not None:
                err = (ours.float() - ref.float()).abs().max().item()
                row["fwd_max_abs_vs_vendor"] = round(err, 5)
                row["fwd_ok"] = err <= 2e-2
            f_fwd = fwd_flops(B, H, n, D, causal)
            ms = timed(lambda: flash_attention_forward(q, k, v, causal=causal))
            row["fwd_ms"] = round(ms, 5)
            row["fwd_tflops"] = round(f_fwd / (ms * 1e-3) / 1e12, 2)
            if ref is not None:
                vms = timed(lambda: vendor(q, k, v, causal, vbe))
                row["vendor_fwd_ms"] = round(vms, 5)
                row["vendor_fwd_tflops"] = round(f_fwd / (vms * 1e-3) / 1e12, 2)
                row["fwd_pct_of_vendor"] = round(100 * vms / ms, 1)
            row["fwd_pct_of_peak"] = round(100 * row["fwd_tflops"] / PEAK_BF16_TFLOPS, 2)

            # forward + backward
            f_step = f_fwd + bwd_flops(B, H, n, D, causal)

            def ours_step():
                o, lse = _flash_attention_forward_lse(q, k, v, causal)
                return _flash_attention_backward(do, q, k, v, o, lse, causal)
            dq, dk, dv = ours_step()
            if ref is not None:
                qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))

                def vendor_step():
                    qg.grad = kg.grad = vg.grad = None
                    vendor(qg, kg, vg, causal, vbe).backward(do)
                vendor_step()
                gerr = max((a.float() - b.grad.float()).abs().max().item() for a, b in ((dq, qg), (dk, kg), (dv, vg)))
                row["grad_max_abs_vs_vendor"] = round(gerr, 5)
                row["grad_ok"] = gerr <= 5e-2
            # backward alone, as the reference's backward benchmark times it
            # (kernels/benchmark_flash_attention_backward.py:89-107): the graph
            # is built once by one forward, then only .backward(retain_graph=True)
            # is timed
            f_bwd = bwd_flops(B, H, n, D, causal)

            def backward_step(fn):
                qb, kb, vb = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
                out = fn(qb, kb, vb)

                def run():
                    qb.grad = kb.grad = vb.grad = None
                    out.backward(do, retain_graph=True)
                return run
            ms = timed(backward_step(lambda a, b, c: flash_attention(a, b, c, causal=causal)))
            row["bwd_ms"] = round(ms, 5)
            row["bwd_tflops"] = round(f_bwd / (ms * 1e-3) / 1e12, 2)
            if ref is not None:
                vms = timed(backward_step(lambda a, b, c: vendor(a, b, c, causal, vbe)))
                row["vendor_bwd_ms"] = round(vms, 5)
                row["vendor_bwd_tflops"] = round(f_bwd / (vms * 1e-3) / 1e12, 2)
                row["bwd_pct_of_vendor"] = round(100 * vms / ms, 1)
            row["bwd_pct_of_peak"] = round(100 * row["bwd_tflops"] / PEAK_BF16_TFLOPS, 2)
            ms = timed(ours_step)
            row["fwd_bwd_ms"] = round(ms, 5)
            row["fwd_bwd_tflops"] = round(f_step / (ms * 1e-3) / 1e12, 2)
            if ref is not None:
                vms = timed(vendor_step)
                row["vendor_fwd_bwd_ms"] = round(vms, 5)
                row["vendor_fwd_bwd_tflops"] = round(f_step / (vms * 1e-3) / 1e12, 2)
                row["fwd_bwd_pct_of_vendor"] = round(100 * vms / ms, 1)
            row["fwd_bwd_pct_of_peak"] = round(100 * row["fwd_bwd_tflops"] / PEAK_BF16_TFLOPS, 2)
            rows.append(row)
            print(f"sweep {row['shape']} causal={causal}: fwd {row['fwd_tflops']} TF/s "
                  f"({row.get('fwd_pct_of_vendor', '-')}% of vendor), bwd {row['bwd_tflops']} TF/s "
                  f"({row.get('bwd_pct_of_vendor', '-')}% of vendor), fwd+bwd {row['fwd_bwd_tflops']} TF/s "
                  f"({row.get('fwd_bwd_pct_of_vendor', '-')}% of vendor)", file=sys.stderr, flush=True)
            del q, k, v, do, ours, ref
    gm = math.exp(sum(math.log(r["fwd_tflops"]) for r in rows) / len(rows))
    ok = all(r.get("fwd_ok", True) and r.get("grad_ok", True) for r in rows)
    result = {
        "metric": "attention sweep B=1 H=32 D=128 bf16, N 512-8192: geometric-mean forward TFLOP/s",
        "value": round(gm, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": 150, "warmup": 10,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic, seeded per shape, inputs resident in HBM",
        "config": {"workload": "sweep over the reference's kernels/benchmark_flash_attention.py shapes"},
        "vendor": {"kernel": "torch.nn.functional.scaled_dot_product_attention", "backend": backend_used,
                   "torch": torch.__version__},
        "parity": {"ok": ok, "against": "vendor outputs and gradients (fwd max-abs <= 2e-2, grads <= 5e-2)"},
        "wall_s": round(time.time() - t_start, 1),
        "sweep": rows,
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "decode":
        bench_decode(args)
        return
    if args.workload == "rope":
        bench_rope(args)
        return
    if args.workload == "rmsnorm":
        bench_rmsnorm(args)
        return
    if args.workload == "prefill":
        bench_prefill(args)
        return
    if args.workload == "sweep":
        bench_sweep(args)
        return
    if args.workload == "gemv":
        bench_gemv(args)
        return
    import torch
    from lightserve_amd import _lib
    from lightserve_amd.kernels.flash_attention_backward import (_flash_attention_backward,
                                                                 _flash_attention_forward_lse)
    from lightserve_amd.kernels.flash_attention_varlen import flash_attention_varlen_forward
    from lightserve_amd.workloads import CONFIGS, bwd_flops, fwd_flops, make_config_inputs, make_varlen_inputs, varlen_fwd_flops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    stream = torch.cuda.current_stream(dev)

    if args.config == 5:
        inp = make_varlen_inputs(device=dev)
        q, k, v = inp["q"], inp["k"], inp["v"]
        f_fwd = varlen_fwd_flops(inp["cu_seqlens_q"].cpu(), inp["cu_seqlens_k"].cpu(), cfg["Hq"], cfg["D"])
        f_step = f_fwd
        step_kind = "fwd"

        def fwd():
            return flash_attention_varlen_forward(q, k, v, inp["cu_seqlens_q"], inp["cu_seqlens_k"],
                                                  inp["max_seqlen_q"], inp["max_seqlen_k"])
        bwd = None
        workload = (f"config5: varlen GQA chunked prefill bf16 B=8 Hq=32 Hkv=8 D=128 chunk=512 "
                    f"prefix={inp['prefix'].tolist()}")
    else:
        inp = make_config_inputs(args.config, device=dev)
        q, k, v, causal = inp["q"], inp["k"], inp["v"], inp["causal"]
        B, H, N, D = q.shape
        f_fwd = fwd_flops(B, H, N, D, causal)
        step_kind = "fwd+bwd" if cfg["backward"] else "fwd"
        f_step = f_fwd + (bwd_flops(B, H, N, D, causal) if cfg["backward"] else 0)

        def fwd():
            return _flash_attention_forward_lse(q, k, v, causal)

        if cfg["backward"]:
            do = inp["do"]

            def bwd(o, lse):
                return _flash_attention_backward(do, q, k, v, o, lse, causal)
        else:
            bwd = None
        workload = (f"config{args.config}: {'causal' if causal else 'non-causal'} {str(q.dtype)[6:]} {step_kind} "
                    f"B={B} H={H} N={N} D={D}")

    # correctness re-check before timing
    o, lse = fwd()
    outs = {"o": o, "lse": lse}
    if bwd is not None:
        outs["dq"], outs["dk"], outs["dv"] = bwd(o, lse)
    torch.cuda.synchronize()
    if args.config == 5:
        from oracle.attention import attention_reference
        cq, ck = inp["cu_seqlens_q"].tolist(), inp["cu_seqlens_k"].tolist()
        qb = q[cq[0]:cq[1]].transpose(0, 1)
        kb = k[ck[0]:ck[1]].transpose(0, 1).repeat_interleave(4, 0)
        vb = v[ck[0]:ck[1]].transpose(0, 1).repeat_interleave(4, 0)
        o_ref, _ = attention_reference(qb, kb, vb, True, dtype=torch.float32)
        err = (o[cq[0]:cq[1]].transpose(0, 1).double() - o_ref.double()).abs()
        parity = {"o": {"max_abs": float(f"{err.max().item():.3e}"), "mean_abs": float(f"{err.mean().item():.3e}")}}
        parity_ok = parity["o"]["max_abs"] <= 2e-2 and parity["o"]["mean_abs"] <= 2e-3
    elif args.skip_parity:
        parity_ok, parity = None, {"skipped": "--skip-parity (profiler run)"}
    else:
        parity_ok, parity = check_parity(cfg, inp, outs)
    del outs

    def step():
        o, lse = fwd()
        if bwd is not None:
            bwd(o, lse)

    calibration_copy(dev, args.calibrate_copy)

    warm_runs = warm_up(step, args.warmup, stream)

    # Timed region: exactly --steps steps back to back, one event pair around
    # them (per-step events would count the host's time to enqueue a step
    # whenever the GPU drains the queue, which short forward-only steps do).
    h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    h0.record(stream)
    for _ in range(args.steps):
        step()
    h1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = h0.elapsed_time(h1) / args.steps
    value = f_step / (ms_per_step * 1e-3) / 1e12
    if bwd is None:
        fwd_avg, bwd_ms = ms_per_step, None
    else:
        # forward / backward split of a training step: a second pass with an
        # event between the two halves of every step
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
               torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        torch.cuda.synchronize()
        for i in range(args.steps):
            e0, e1, e2 = ev[i]
            e0.record(stream)
            o, lse = fwd()
            e1.record(stream)
            bwd(o, lse)
            e2.record(stream)
        torch.cuda.synchronize()
        fwd_ms = [a.elapsed_time(b) for a, b, _ in ev]
        bwd_ms = [b.elapsed_time(c) for _, b, c in ev]
        fwd_avg = sum(fwd_ms) / len(fwd_ms)
    fwd_tflops = f_fwd / (fwd_avg * 1e-3) / 1e12

    wl_key = f"config{args.config}"
    # Per-kernel launch times on the launch stream (HIP events around
    # back-to-back launches): the forward from the timed steps; the backward's
    # two kernels one at a time through lsfa_bwd's phase flags (the dK/dV
    # phase reuses the workspace the dQ phase just wrote). The opt-in
    # stored-dS backward (LSFA_BWD_STORED_DS: dK/dV kernel storing dS, then a
    # dQ GEMM over it) is timed the same way, whole and per phase, and
    # reported beside the default; its dQ GEMM moves dS once, so it is priced
    # against HBM bandwidth (algorithmic bytes: the visible dS entries, 2
    # bytes each, plus K and dQ).
    fwd_name = fwd_kernel_name(*q.shape[:3], k.shape[2], q.shape[3], inp["causal"], q.dtype)
    kernels = [{"kernel": fwd_name, "bound": "mfma", "flops_per_launch": f_fwd,
                "mfma_flops_per_launch": f_fwd, "avg_launch_ms": fwd_avg}]
    stored_ds = None
    if bwd is not None:
        from lightserve_amd.kernels.flash_attention_backward import _backward_args
        from lightserve_amd import _lib as lib
        o_t, lse_t = fwd()
        raw = stream.cuda_stream
        unit = f_fwd / 2  # one B*H*N^2*D GEMM (halved when causal)
        Bq, Hq, Nq, Dq = q.shape
        pairs = Nq * (Nq + 1) // 2 if inp["causal"] else Nq * Nq
        dq_bytes = Bq * Hq * (2 * pairs + 2 * 2 * Nq * Dq)

        def time_flags(ba, flags):
            ba.flags = flags
            for _ in range(2):
                lib.bwd(ba, raw)
            k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            k0.record(stream)
            for _ in range(args.steps):
                lib.bwd(ba, raw)
            k1.record(stream)
            torch.cuda.synchronize()
            return k0.elapsed_time(k1) / args.steps

        ba, keep = _backward_args(inp["do"], q, k, v, o_t, lse_t, inp["causal"])
        for flag, name, alg_units, mfma_units in ((lib.BWD_ONLY_DQ, "fa_bwd_dq_kernel", 1, 3),
                                                  (lib.BWD_ONLY_DKDV, "fa_bwd_dkdv_kernel", 4, 4)):
            kernels.append({"kernel": name, "bound": "mfma", "flops_per_launch": alg_units * unit,
                            "mfma_flops_per_launch": mfma_units * unit, "avg_launch_ms": time_flags(ba, flag)})
        del keep
        if Dq > 64 and q.dtype != torch.float32:
            ba, keep = _backward_args(inp["do"], q, k, v, o_t, lse_t, inp["causal"], flags=lib.BWD_STORED_DS)
            sd = lib.BWD_STORED_DS
            stored_ds = {"flag": "LSFA_BWD_STORED_DS", "workspace_bytes": int(ba.workspace_bytes),
                         "ms": round(time_flags(ba, sd), 5),
                         "dkdv_phase_ms": round(time_flags(ba, sd | lib.BWD_ONLY_DKDV), 5),
                         "dq_gemm_ms": round(time_flags(ba, sd | lib.BWD_ONLY_DQ), 5),
                         "dq_gemm_bytes": dq_bytes}
            stored_ds["dq_gemm_gbs"] = round(dq_bytes / (stored_ds["dq_gemm_ms"] * 1e-3) / 1e9, 1)
            stored_ds["dq_gemm_hbm_frac"] = round(stored_ds["dq_gemm_gbs"] / HBM_PEAK_GBS, 4)
            stored_ds["dq_gemm_traffic"] = measured_traffic("fa_bwd_dq_ds_kernel", wl_key)
            del keep
    for kd in kernels:
        kd["achieved"] = round(kd["flops_per_launch"] / (kd["avg_launch_ms"] * 1e-3) / 1e12, 2)
        kd["frac"] = round(kd["achieved"] / PEAK_BF16_TFLOPS, 4)
        kd["mfma_frac"] = round(kd["mfma_flops_per_launch"] / (kd["avg_launch_ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
        kd["traffic"] = measured_traffic(kd["kernel"], wl_key)
        kd["avg_launch_ms"] = round(kd["avg_launch_ms"], 5)
    dom = max(kernels, key=lambda kd: kd["avg_launch_ms"])
    roofline = {"kernel": dom["kernel"], "bound": "mfma", "achieved": dom["achieved"], "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": dom["frac"], "traffic": dom["traffic"],
                "flops_per_launch": dom["flops_per_launch"], "avg_launch_ms": dom["avg_launch_ms"],
                "kernels": kernels}
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "warmup_calls": warm_runs, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if q.dtype == torch.bfloat16 else ("fp16" if q.dtype == torch.float16 else "fp32"),
        "data": f"synthetic, seeded (seed {cfg['seed']}), inputs resident in HBM",
        "config": {"workload": workload, "step": step_kind, "flops_per_step": f_step},
        "pct_of_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "fwd": {"tflops": round(fwd_tflops, 2), "ms": round(fwd_avg, 5),
                "pct_of_peak": round(100 * fwd_tflops / PEAK_BF16_TFLOPS, 2)},
        "wall_s_timed": round(wall, 4),
        "parity": {"ok": parity_ok, **parity},
        "roofline": roofline,
    }
    if bwd is not None:
        # The reference's forward benchmark times the inference entry point
        # (kernels/benchmark_flash_attention.py: flash_attention_forward, no
        # logsumexp); timed here the same way, back to back over --steps calls.
        from lightserve_amd.kernels.flash_attention import flash_attention_forward
        for _ in range(2):
            flash_attention_forward(q, k, v, causal=inp["causal"])
        fi0, fi1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        fi0.record(stream)
        for _ in range(args.steps):
            flash_attention_forward(q, k, v, causal=inp["causal"])
        fi1.record(stream)
        torch.cuda.synchronize()
        fi_ms = fi0.elapsed_time(fi1) / args.steps
        result["fwd_inference"] = {"tflops": round(f_fwd / (fi_ms * 1e-3) / 1e12, 2), "ms": round(fi_ms, 5),
                                   "pct_of_peak": round(100 * f_fwd / (fi_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                                   "entry": "flash_attention_forward (no logsumexp), back to back"}
        bwd_avg = sum(bwd_ms) / len(bwd_ms)
        fb = bwd_flops(*q.shape, inp["causal"])
        result["bwd"] = {"tflops": round(fb / (bwd_avg * 1e-3) / 1e12, 2), "ms": round(bwd_avg, 5),
                         "pct_of_peak": round(100 * fb / (bwd_avg * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                         "kernels": "fa_bwd_dq_kernel + fa_bwd_dkdv_kernel"}
        if stored_ds is not None:
            stored_ds["tflops"] = round(fb / (stored_ds["ms"] * 1e-3) / 1e12, 2)
            result["bwd"]["stored_ds"] = stored_ds
        result["fwd_bwd"] = {"tflops": round(value, 2), "ms": round(ms_per_step, 5),
                             "pct_of_peak": round(100 * value / PEAK_BF16_TFLOPS, 2)}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, inp, args.cpu_heads, f_step, step_kind) if args.config != 5 else None
    if args.config == 3 and not args.no_other_configs:
        del inp, q, k, v
        torch.cuda.empty_cache()
        result["other_configs"] = other_configs(args.steps, args.warmup)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
