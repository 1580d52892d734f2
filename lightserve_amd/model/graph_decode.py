"""Decode steps of the LLaMA-shaped model captured in HIP graphs, timed
against the same steps run eagerly (the reference's model/cuda_graph_decode.py).

Two decode loops:

  full     The reference's design (model/cuda_graph_decode.py:10-30): a fixed
           [B, max_seq_len] token buffer, every step reruns the whole causal
           forward over it and reads the logits of row cur_len - 1. Same
           defaults and timing method, so the numbers compare with the
           reference's cuda_graph_decode_results.json.
  kvcache  What the reference could not express (its kernel needs Nq == Nkv):
           one new token per sequence per step. The token's K/V rows are
           rotated at their position (lsfa_rope with per-sequence positions)
           and written into a paged cache ([num_blocks, block_size, Hkv, D],
           the engine's layout, engine/config.py:5-7), and attention is
           paged_attention_decode over the block tables. Static shapes, no
           host synchronisation: one graph replay per step.

    python -m lightserve_amd.model.graph_decode [--mode full|kvcache|both] [--n-layers 4] ...

Per-step latencies are HIP-event timed around each step with a synchronize
after it, as the reference does (model/cuda_graph_decode.py:86-103), so idle
gaps from the host issuing launches are included: that is what graphs remove.
"""
import argparse
import json
import statistics

import torch
import torch.nn.functional as F

from ..kernels.paged_attention import paged_attention_decode, paged_prefill
from ..kernels.rope import apply_rope_
from ..kernels.fused_rmsnorm_residual import fused_add_rmsnorm
from ..kernels.greedy import greedy_next_token
from ..kernels.tiled_matmul import add_rmsnorm_matmul_shared_input, matmul, swiglu_matmul
from .minimal_llama import add_norm, init_weights, llama3_8b_shape, llama_forward, precompute_rope

SEED_TOKEN_ID = 1


def make_seeded_buffer(batch_size, max_seq_len, device):
    ids = torch.zeros(batch_size, max_seq_len, dtype=torch.long, device=device)
    ids[:, 0] = SEED_TOKEN_ID
    return ids


def count_launches(step_fn):
    """Kernels one call of step_fn issues (torch.profiler; None if unavailable)."""
    step_fn()
    torch.cuda.synchronize()
    try:
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
            step_fn()
            torch.cuda.synchronize()
        return sum(1 for e in prof.events() if e.device_type == torch.profiler.DeviceType.CUDA)
    except Exception as e:  # noqa: BLE001 -- a secondary number
        print(f"  (kernel-launch count unavailable: {e})")
        return None


def time_steps(step_fn, num_steps, warmup_steps):
    for _ in range(warmup_steps):
        step_fn()
    torch.cuda.synchronize()
    out = []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(num_steps):
        start.record()
        step_fn()
        end.record()
        torch.cuda.synchronize()
        out.append(start.elapsed_time(end))
    return out


def capture(fn, warmup=3):
    """Side-stream warm-up, then capture fn() in a graph; returns (graph, outputs)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


# --------------------------------------------------------------------- full
class FullRecomputeDecoder:
    """The reference's static-shape loop: the whole buffer, every step."""

    def __init__(self, weights, config, batch_size, device="cuda"):
        self.w, self.cfg = weights, config
        self.ids = make_seeded_buffer(batch_size, config.max_seq_len, device)
        self.tables = precompute_rope(config, device)
        self.cur_len = 1

    def forward(self):
        return llama_forward(self.w, self.cfg, self.ids, causal=True, rope_tables=self.tables)

    def advance(self, logits):
        nxt = logits[:, self.cur_len - 1, :].argmax(dim=-1)
        self.ids[:, self.cur_len] = nxt
        self.cur_len += 1
        return nxt


# ------------------------------------------------------------------ kvcache
class KVCacheDecoder:
    """One token per sequence per step against a paged KV cache.

    State on the device: tokens [B] (the step's input), seq_lens [B] (tokens
    cached so far), k/v caches per layer and the block tables. step() issues
    only device work of static shape, so it can be captured and replayed;
    prefill() caches a prompt chunk by chunk before the decode steps."""

    def __init__(self, weights, config, batch_size, block_size=16, device="cuda", shuffle_blocks=True, seed=0):
        self.w, self.cfg, self.B = weights, config, batch_size
        nkv, hd = config.kv_heads, config.head_dim
        self.bs = block_size
        self.max_blocks = (config.max_seq_len + block_size - 1) // block_size
        n_blocks = batch_size * self.max_blocks
        order = torch.randperm(n_blocks, generator=torch.Generator().manual_seed(seed)) if shuffle_blocks \
            else torch.arange(n_blocks)
        self.block_tables = order.to(torch.int32).view(batch_size, self.max_blocks).to(device)
        shape = (n_blocks, block_size, nkv, hd)
        self.k_cache = [torch.zeros(shape, dtype=config.dtype, device=device) for _ in weights.layers]
        self.v_cache = [torch.zeros(shape, dtype=config.dtype, device=device) for _ in weights.layers]
        self.seq_lens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self.tokens = torch.full((batch_size,), SEED_TOKEN_ID, dtype=torch.long, device=device)
        self.cos, self.sin = precompute_rope(config, device)

    def step(self):
        """Logits [B, vocab] of the current tokens; appends their K/V."""
        cfg, B = self.cfg, self.B
        nh, nkv, hd = cfg.n_heads, cfg.kv_heads, cfg.head_dim
        pos = self.seq_lens
        lens = pos + 1
        residual = F.embedding(self.tokens, self.w.embed_tokens)  # [B, H]
        pending = None
        for i, layer in enumerate(self.w.layers):
            # residual add + RMSNorm folded into the q/k/v launch (the first layer's input is the embedding)
            x_in, r_in = (residual, None) if pending is None else (pending, residual)
            (q, k, v), residual = add_rmsnorm_matmul_shared_input(
                x_in, r_in, layer.input_layernorm_weight, cfg.rms_eps, (layer.q_proj, layer.k_proj, layer.v_proj))
            # RoPE at each sequence's position; the same launch stores the rotated k and v rows at the slot
            # its block table gives for that position
            apply_rope_(q.view(B, nh, 1, hd), k.view(B, nkv, 1, hd), self.cos, self.sin, positions=pos,
                        v=v.view(B, nkv, 1, hd), k_cache=self.k_cache[i], v_cache=self.v_cache[i],
                        block_tables=self.block_tables)
            o = paged_attention_decode(q.view(B, nh, hd), self.k_cache[i], self.v_cache[i], self.block_tables,
                                       lens, max_seq_len=cfg.max_seq_len)
            (gate, up), residual = add_rmsnorm_matmul_shared_input(
                matmul(o.view(B, nh * hd), layer.o_proj), residual, layer.post_attention_layernorm_weight,
                cfg.rms_eps, (layer.gate_proj, layer.up_proj))
            pending = swiglu_matmul(gate, up, layer.down_proj)
        (logits,), _ = add_rmsnorm_matmul_shared_input(pending, residual, self.w.norm_weight, cfg.rms_eps,
                                                       (self.w.lm_head,), write_residual=False)
        return logits

    def prefill(self, prompt, chunk_size):
        """Caches a prompt [B, P] chunk by chunk (the engine's chunked prefill:
        each chunk's K/V rows are rotated at their positions and written into
        the paged cache, then the chunk's queries attend to everything cached
        so far through paged_prefill). Returns the logits [B, vocab] of the
        last prompt token and makes their argmax the next decode token."""
        cfg, B = self.cfg, self.B
        nh, nkv, hd, H = cfg.n_heads, cfg.kv_heads, cfg.head_dim, cfg.hidden_size
        assert prompt.shape[0] == B and prompt.shape[1] > 0, "prompt must be [batch, P] with P > 0"
        P = prompt.shape[1]
        logits = None
        for s in range(0, P, chunk_size):
            c = min(chunk_size, P - s)
            pos = self.seq_lens  # [B] first position of the chunk
            t = torch.arange(c, device=pos.device, dtype=torch.int32)
            abs_pos = (pos.view(B, 1) + t.view(1, c)).long()  # [B, c]
            slot = (self.block_tables.gather(1, abs_pos // self.bs).long() * self.bs + abs_pos % self.bs).view(-1)
            cu = torch.arange(0, (B + 1) * c, c, device=pos.device, dtype=torch.int32)
            lens = pos + c
            residual = F.embedding(prompt[:, s:s + c].reshape(-1), self.w.embed_tokens)  # [B*c, H]
            pending = None
            for i, layer in enumerate(self.w.layers):
                h, residual = add_norm(pending, residual, layer.input_layernorm_weight, cfg.rms_eps)
                q = matmul(h, layer.q_proj)
                k = matmul(h, layer.k_proj)
                v = matmul(h, layer.v_proj)
                apply_rope_(q.view(B, c, nh, hd).transpose(1, 2), k.view(B, c, nkv, hd).transpose(1, 2),
                            self.cos, self.sin, positions=pos, v=v.view(B, c, nkv, hd).transpose(1, 2),
                            k_cache=self.k_cache[i], v_cache=self.v_cache[i], slots=slot)
                o = paged_prefill(q.view(B * c, nh, hd), self.k_cache[i], self.v_cache[i], self.block_tables, cu, lens,
                                  max_seqlen_q=c)
                h2, residual = fused_add_rmsnorm(matmul(o.view(B * c, nh * hd), layer.o_proj), residual,
                                                 layer.post_attention_layernorm_weight, cfg.rms_eps)
                mlp = F.silu(matmul(h2, layer.gate_proj)) * matmul(h2, layer.up_proj)
                pending = matmul(mlp, layer.down_proj)
            last = slice(c - 1, B * c, c)  # each sequence's last token of the chunk
            final, _ = add_norm(pending[last].contiguous() if pending is not None else None,
                                residual[last].contiguous(), self.w.norm_weight, cfg.rms_eps)
            logits = matmul(final, self.w.lm_head)
            self.seq_lens.add_(c)
        greedy_next_token(logits, out=self.tokens)
        return logits

    def advance(self, logits):
        """Greedy next token; one more cached token per sequence (one launch)."""
        greedy_next_token(logits, out=self.tokens, seq_lens=self.seq_lens)
        return self.tokens


def summarize(lat):
    s = sorted(lat)
    return {"median_ms": statistics.median(s), "mean_ms": statistics.mean(s), "p95_ms": s[int(0.95 * (len(s) - 1))],
            "min_ms": s[0], "max_ms": s[-1]}


def make_decoder(mode, weights, config, args):
    if mode == "full":
        return FullRecomputeDecoder(weights, config, args.batch_size)
    return KVCacheDecoder(weights, config, args.batch_size, block_size=args.block_size)


def step_fn(dec):
    return dec.forward() if isinstance(dec, FullRecomputeDecoder) else dec.step()


def run_mode(mode, weights, config, args):
    """Kernels per step, then eager and graph-replay step latencies, each on a
    fresh decoder starting from the seed token."""
    res = {"launches": count_launches(lambda: step_fn(make_decoder(mode, weights, config, args)))}
    dec = make_decoder(mode, weights, config, args)
    res["eager"] = summarize(time_steps(lambda: dec.advance(step_fn(dec)), args.num_steps, args.warmup_steps))
    dec = make_decoder(mode, weights, config, args)
    graph, out = capture(lambda: step_fn(dec))
    dec = reset(dec, config, args)

    def replay():
        graph.replay()
        dec.advance(out)
    res["graph"] = summarize(time_steps(replay, args.num_steps, args.warmup_steps))
    res["speedup_median"] = res["eager"]["median_ms"] / res["graph"]["median_ms"]
    return res


def reset(dec, config, args):
    """Back to the seed token after capture's warm-up calls (state tensors are
    reused in place: the graph holds their addresses)."""
    if isinstance(dec, FullRecomputeDecoder):
        dec.ids.copy_(make_seeded_buffer(args.batch_size, config.max_seq_len, dec.ids.device))
        dec.cur_len = 1
    else:
        dec.seq_lens.zero_()
        dec.tokens.fill_(SEED_TOKEN_ID)
    return dec


def prefill_main(args):
    """Times KVCacheDecoder.prefill of a P-token prompt per sequence (chunks
    of --chunk tokens; HIP events around each whole prefill, median of
    --num-steps runs after --warmup-steps, each from an empty cache)."""
    P, C = args.prefill, args.chunk
    config = llama3_8b_shape(n_layers=args.n_layers, max_seq_len=max(args.max_seq_len, P + 1), gqa=args.gqa)
    weights = init_weights(config, device="cuda", seed=args.seed)
    prompt = torch.randint(0, config.vocab_size, (args.batch_size, P), generator=torch.Generator().manual_seed(1))
    prompt = prompt.cuda()
    dec = KVCacheDecoder(weights, config, args.batch_size, block_size=args.block_size)
    lat = []
    for i in range(args.warmup_steps + args.num_steps):
        dec.seq_lens.zero_()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dec.prefill(prompt, C)
        e1.record()
        torch.cuda.synchronize()
        if i >= args.warmup_steps:
            lat.append(e0.elapsed_time(e1))
    med = statistics.median(lat)
    tokens = args.batch_size * P
    res = {"prefill_tokens": P, "chunk": C, "batch_size": args.batch_size, "n_layers": config.n_layers,
           "n_kv_heads": config.kv_heads, "median_ms": med, "tokens_per_s": tokens / (med * 1e-3)}
    print(json.dumps(res), flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(res, f, indent=2)
    return res


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--mode", choices=["full", "kvcache", "both"], default="both")
    ap.add_argument("--n-layers", type=int, default=4)
    ap.add_argument("--max-seq-len", type=int, default=128)
    ap.add_argument("--batch-size", type=int, default=1)
    ap.add_argument("--num-steps", type=int, default=50)
    ap.add_argument("--warmup-steps", type=int, default=5)
    ap.add_argument("--block-size", type=int, default=16)
    ap.add_argument("--gqa", action="store_true", help="LLaMA-3-8B's real 8 KV heads (kvcache mode and full)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--out", default=None, help="write the results JSON here")
    ap.add_argument("--prefill", type=int, default=0, metavar="P",
                    help="instead of decode steps: time the chunked prefill of a P-token prompt per sequence "
                         "(max_seq_len is raised to fit it)")
    ap.add_argument("--chunk", type=int, default=512, help="prefill chunk size")
    args = ap.parse_args(argv)
    assert torch.cuda.is_available(), "needs a GPU"
    if args.prefill:
        return prefill_main(args)
    config = llama3_8b_shape(n_layers=args.n_layers, max_seq_len=args.max_seq_len, gqa=args.gqa)
    needed = args.warmup_steps + args.num_steps + 3
    assert needed < config.max_seq_len, f"--max-seq-len {config.max_seq_len} too small for {needed} decode steps"
    print(f"Config: n_layers={config.n_layers} hidden={config.hidden_size} n_heads={config.n_heads} "
          f"n_kv_heads={config.kv_heads} head_dim={config.head_dim} intermediate={config.intermediate_size} "
          f"vocab={config.vocab_size} max_seq_len={config.max_seq_len} batch_size={args.batch_size} "
          f"dtype={config.dtype}", flush=True)
    weights = init_weights(config, device="cuda", seed=args.seed)
    modes = ["full", "kvcache"] if args.mode == "both" else [args.mode]
    results = {"config": {"n_layers": config.n_layers, "hidden_size": config.hidden_size,
                          "n_heads": config.n_heads, "n_kv_heads": config.kv_heads, "head_dim": config.head_dim,
                          "intermediate_size": config.intermediate_size, "vocab_size": config.vocab_size,
                          "max_seq_len": config.max_seq_len, "batch_size": args.batch_size,
                          "dtype": str(config.dtype), "block_size": args.block_size}}
    print(f"\n{'mode':<18} {'launches':>8} {'median (ms)':>12} {'mean (ms)':>10} {'p95 (ms)':>9}")
    for m in modes:
        r = run_mode(m, weights, config, args)
        results[m] = r
        for kind in ("eager", "graph"):
            st = r[kind]
            print(f"{m + ' ' + kind:<18} {str(r['launches']):>8} {st['median_ms']:>12.3f} {st['mean_ms']:>10.3f} "
                  f"{st['p95_ms']:>9.3f}", flush=True)
        print(f"{m}: graph speedup (median) {r['speedup_median']:.2f}x", flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(results, f, indent=2)
    print(json.dumps({m: {k: results[m][k] for k in ("launches", "speedup_median")} | {
        "eager_median_ms": results[m]["eager"]["median_ms"], "graph_median_ms": results[m]["graph"]["median_ms"]}
        for m in modes}))
    return results


if __name__ == "__main__":
    main()
