"""GPU parity of the RoPE kernel and of the LLaMA-shaped forward built on this
library (the model row of the hot-path scope: the reference's
model/minimal_llama.py and model/cuda_graph_decode.py).

RoPE: lsfa_rope against oracle.model.apply_rope evaluated in float64 on the
same (rounded) inputs and tables; the kernel rounds once, so its error is at
most half an ulp of the dtype plus fp32 arithmetic. Model: llama_forward
against oracle.model.reference_llama_forward with the same weights, at the
reference test's tolerances (model/tests/test_minimal_llama.py: 5e-3 fp32,
8e-2 bf16), the oracle run on the CPU in the model dtype (bf16 attention on
the GPU's math path is avoided in references). The LLaMA-3-8B one-layer shape
(MHA and the real GQA) is checked against the oracle in fp32 on the GPU.
Graph capture: replays with new token ids in between match eager calls.
"""
from dataclasses import replace

import pytest
import torch

from lightserve_amd.kernels.rope import apply_rope, apply_rope_
from lightserve_amd.model.minimal_llama import (TOY_CONFIG, init_weights, llama3_8b_shape, llama_forward,
                                                precompute_rope)
from oracle import model as om

pytestmark = pytest.mark.gpu

ULP_HALF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -23}


def _rope_case(B, Hq, Hkv, N, D, dtype, seed, packed):
    g = torch.Generator().manual_seed(seed)
    if packed:  # [B, N, H*D] storage viewed as [B, H, N, D], as the model's projections
        q = torch.randn(B, N, Hq, D, generator=g).to(dtype).cuda().transpose(1, 2)
        k = torch.randn(B, N, Hkv, D, generator=g).to(dtype).cuda().transpose(1, 2)
    else:
        q = torch.randn(B, Hq, N, D, generator=g).to(dtype).cuda()
        k = torch.randn(B, Hkv, N, D, generator=g).to(dtype).cuda()
    return q, k


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,Hq,Hkv,N,D,packed", [(2, 4, 2, 37, 64, True), (1, 32, 8, 5, 128, True),
                                                 (3, 2, 2, 17, 32, False), (1, 8, 1, 300, 128, False)])
@pytest.mark.parametrize("with_positions", [False, True])
def test_rope_kernel_matches_oracle(B, Hq, Hkv, N, D, packed, dtype, with_positions):
    print(f"case rope B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} packed={packed} {dtype} pos={with_positions}", flush=True)
    q, k = _rope_case(B, Hq, Hkv, N, D, dtype, seed=N + D, packed=packed)
    cos, sin = om.precompute_rope(D, 512, 500000.0, dtype, "cuda")
    pos = torch.tensor([7 * b + 3 for b in range(B)], dtype=torch.int32, device="cuda") if with_positions else None
    q_ref, k_ref = om.apply_rope(q.double().cpu(), k.double().cpu(), cos.double().cpu(), sin.double().cpu(), N,
                                 positions=None if pos is None else pos.cpu())
    apply_rope_(q, k, cos, sin, positions=pos)
    torch.cuda.synchronize()
    u = ULP_HALF[dtype]
    torch.testing.assert_close(q.double().cpu(), q_ref, atol=1e-5, rtol=1.01 * u)
    torch.testing.assert_close(k.double().cpu(), k_ref, atol=1e-5, rtol=1.01 * u)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,Hq,Hkv,N,D", [(3, 8, 2, 1, 128), (2, 4, 4, 37, 64)])
def test_rope_appends_kv_to_cache(B, Hq, Hkv, N, D, dtype):
    """The K/V cache append of apply_rope_ equals rotating then copying rows
    with index_copy_ (bit for bit), skips negative slots, and leaves every
    other slot of the caches untouched."""
    print(f"case rope cache B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * N + D)
    q = torch.randn(B, N, Hq, D, generator=g).to(dtype).cuda().transpose(1, 2)
    k = torch.randn(B, N, Hkv, D, generator=g).to(dtype).cuda().transpose(1, 2)
    v = torch.randn(B, N, Hkv, D, generator=g).to(dtype).cuda().transpose(1, 2)
    cos, sin = om.precompute_rope(D, 512, 500000.0, dtype, "cuda")
    pos = torch.tensor([11 * b + 2 for b in range(B)], dtype=torch.int32, device="cuda")
    nblocks, bs = 64, 16
    slots = torch.randperm(nblocks * bs, generator=g)[:B * N].cuda()
    slots[1] = -1  # a padding token: not stored
    kc = torch.full((nblocks, bs, Hkv, D), 7.0, dtype=dtype, device="cuda")
    vc = torch.full_like(kc, 7.0)
    q2, k2 = q.clone(), k.clone()
    apply_rope_(q, k, cos, sin, positions=pos, v=v, k_cache=kc, v_cache=vc, slots=slots)
    apply_rope_(q2, k2, cos, sin, positions=pos)  # the same rotation without the append
    kr = torch.full_like(kc, 7.0)
    vr = torch.full_like(vc, 7.0)
    keep = slots >= 0
    rows_k = k2.transpose(1, 2).reshape(B * N, Hkv, D)[keep]
    rows_v = v.transpose(1, 2).reshape(B * N, Hkv, D)[keep]
    kr.view(-1, Hkv, D).index_copy_(0, slots[keep], rows_k)
    vr.view(-1, Hkv, D).index_copy_(0, slots[keep], rows_v)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(k, k2)
    assert torch.equal(kc, kr) and torch.equal(vc, vr)
    # the same slots named by a block table and the positions instead
    nb_seq = (11 * (B - 1) + 2 + N + bs - 1) // bs + 1
    table = torch.randperm(nblocks, generator=g)[:B * nb_seq].view(B, nb_seq).to(torch.int32)
    table[0, 0] = -1  # a block id outside the cache: that token is not stored
    tp = torch.tensor([[11 * b + 2 + n for n in range(N)] for b in range(B)])
    tslots = (table.long().gather(1, tp // bs) * bs + tp % bs).view(-1)
    tslots[tslots < 0] = -1
    kc2 = torch.full_like(kc, 7.0)
    vc2 = torch.full_like(vc, 7.0)
    q3, k3 = q2.clone(), k.clone()  # rotate the unrotated inputs again
    q3.copy_(torch.randn(B, N, Hq, D, generator=g).to(dtype).cuda().transpose(1, 2))
    k3 = torch.randn(B, N, Hkv, D, generator=g).to(dtype).cuda().transpose(1, 2)
    q4, k4 = q3.clone(), k3.clone()
    kc3, vc3 = torch.full_like(kc, 7.0), torch.full_like(vc, 7.0)
    apply_rope_(q3, k3, cos, sin, positions=pos, v=v, k_cache=kc2, v_cache=vc2, block_tables=table.cuda())
    apply_rope_(q4, k4, cos, sin, positions=pos, v=v, k_cache=kc3, v_cache=vc3, slots=tslots.cuda())
    torch.cuda.synchronize()
    assert torch.equal(q3, q4) and torch.equal(k3, k4)
    assert torch.equal(kc2, kc3) and torch.equal(vc2, vc3)


def test_rope_q_only_and_positions_clamped():
    """k = None rotates q alone; positions past the table clamp to its last row."""
    print("case rope q-only, clamp", flush=True)
    q, _ = _rope_case(2, 4, 1, 3, 64, torch.bfloat16, seed=5, packed=False)
    cos, sin = om.precompute_rope(64, 16, 10000.0, torch.bfloat16, "cuda")
    pos = torch.tensor([0, 40], dtype=torch.int32, device="cuda")  # sequence 1 runs past row 15
    q0 = q.clone()
    apply_rope_(q, None, cos, sin, positions=pos)
    torch.cuda.synchronize()
    ref0, _ = om.apply_rope(q0[:1].double().cpu(), q0[:1].double().cpu(), cos.double().cpu(), sin.double().cpu(), 3)
    c15 = cos.double().cpu()[15].view(1, 1, 1, -1)
    s15 = sin.double().cpu()[15].view(1, 1, 1, -1)
    ref1 = q0[1:].double().cpu() * c15 + om.rotate_half(q0[1:].double().cpu()) * s15
    torch.testing.assert_close(q[:1].double().cpu(), ref0, atol=1e-5, rtol=2 ** -8)
    torch.testing.assert_close(q[1:].double().cpu(), ref1, atol=1e-5, rtol=2 ** -8)


def test_apply_rope_dropin_keeps_inputs():
    """apply_rope (the reference's signature) returns new tensors and leaves
    its inputs alone; the values equal the in-place call's."""
    print("case rope drop-in", flush=True)
    q, k = _rope_case(1, 4, 4, 9, 64, torch.bfloat16, seed=2, packed=True)
    cos, sin = precompute_rope(replace(TOY_CONFIG, max_seq_len=16), "cuda")
    q0, k0 = q.clone(), k.clone()
    qr, kr = apply_rope(q, k, cos, sin, 9)
    assert torch.equal(q, q0) and torch.equal(k, k0)
    apply_rope_(q, k, cos, sin)
    assert torch.equal(qr, q) and torch.equal(kr, k)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N", [(1, 8), (2, 37), (1, 64)])
@pytest.mark.parametrize("n_kv_heads", [None, 2])
def test_model_matches_reference(B, N, dtype, causal, n_kv_heads):
    print(f"case model B={B} N={N} {dtype} causal={causal} kv={n_kv_heads}", flush=True)
    torch.manual_seed(0)
    config = replace(TOY_CONFIG, dtype=dtype, n_kv_heads=n_kv_heads)
    weights = init_weights(config, device="cuda", seed=0)
    input_ids = torch.randint(0, config.vocab_size, (B, N), device="cuda")
    logits = llama_forward(weights, config, input_ids, causal=causal)
    torch.cuda.synchronize()
    cpu_w = _to(weights, "cpu", dtype)
    ref = om.reference_llama_forward(cpu_w, config, input_ids.cpu(), causal=causal)
    assert logits.shape == (B, N, config.vocab_size)
    tol = 5e-3 if dtype == torch.float32 else 8e-2
    torch.testing.assert_close(logits.cpu(), ref, atol=tol, rtol=tol)


@pytest.mark.parametrize("gqa", [False, True])
def test_model_llama3_8b_layer(gqa):
    """One LLaMA-3-8B layer (hidden 4096, 32 heads of 128, MLP 14336, vocab
    128256) in bf16 at N = 128, against the oracle in fp32 on the GPU."""
    print(f"case model llama3-8b layer gqa={gqa}", flush=True)
    config = llama3_8b_shape(n_layers=1, max_seq_len=128, gqa=gqa)
    weights = init_weights(config, device="cuda", seed=1)
    input_ids = torch.randint(0, config.vocab_size, (1, 128), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    logits = llama_forward(weights, config, input_ids, causal=True)
    ref = om.reference_llama_forward(_to(weights, "cuda", torch.float32), replace(config, dtype=torch.float32),
                                     input_ids, causal=True)
    torch.cuda.synchronize()
    err = (logits.float() - ref).abs()
    print(f"[gate] llama3-8b layer gqa={gqa}: max-abs {err.max().item():.3e}, mean-abs {err.mean().item():.3e}, "
          f"|ref| max {ref.abs().max().item():.3e}", flush=True)
    torch.testing.assert_close(logits.float(), ref, atol=8e-2, rtol=8e-2)


def test_model_graph_capture_replays():
    """The forward captured in a HIP graph: three replays, each after new token
    ids were written and other eager work ran, match eager forwards."""
    print("case model graph replay", flush=True)
    config = replace(TOY_CONFIG, n_kv_heads=2)
    weights = init_weights(config, device="cuda", seed=0)
    ids = torch.randint(0, config.vocab_size, (2, 32), device="cuda")
    tables = precompute_rope(config, "cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            llama_forward(weights, config, ids, rope_tables=tables)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_logits = llama_forward(weights, config, ids, rope_tables=tables)
    for r in range(3):
        ids.copy_(torch.randint(0, config.vocab_size, ids.shape, device="cuda", generator=torch.Generator("cuda").manual_seed(r)))
        _ = torch.randn(1000, 1000, device="cuda").sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = llama_forward(weights, config, ids, rope_tables=tables)
        torch.cuda.synchronize()
        assert torch.equal(static_logits, eager), f"replay {r} differs from eager"


@pytest.mark.parametrize("n_kv_heads,block_size", [(2, 4), (None, 16)])
def test_kvcache_decode_matches_full_forward(n_kv_heads, block_size):
    """Incremental decode (RoPE at per-sequence positions, K/V appended to a
    shuffled paged cache, paged_attention_decode) gives, at every step, the
    logits the full causal forward gives for the last token of the same
    sequence."""
    from lightserve_amd.model.graph_decode import KVCacheDecoder
    print(f"case kv-cache decode kv={n_kv_heads} bs={block_size}", flush=True)
    config = replace(TOY_CONFIG, n_kv_heads=n_kv_heads)
    weights = init_weights(config, device="cuda", seed=0)
    dec = KVCacheDecoder(weights, config, batch_size=2, block_size=block_size)
    dec.tokens.copy_(torch.tensor([1, 5], device="cuda"))
    ids = dec.tokens.view(2, 1).clone()
    for t in range(8):
        logits = dec.step()
        full = llama_forward(weights, config, ids)[:, -1]
        torch.testing.assert_close(logits.float(), full.float(), atol=8e-2, rtol=8e-2, msg=f"step {t}")
        dec.advance(logits)
        ids = torch.cat([ids, dec.tokens.view(2, 1)], dim=1)


@pytest.mark.parametrize("n_kv_heads,chunk", [(2, 7), (None, 16), (1, 1)])
def test_chunked_prefill_then_decode_matches_full_forward(n_kv_heads, chunk):
    """A prompt cached chunk by chunk through paged_prefill (RoPE at each
    chunk's positions, K/V written into a shuffled paged cache of 16-token
    blocks) gives the full forward's logits for the prompt's last token, and
    the decode steps after it continue to match the full forward."""
    from lightserve_amd.model.graph_decode import KVCacheDecoder
    print(f"case chunked prefill kv={n_kv_heads} chunk={chunk}", flush=True)
    config = replace(TOY_CONFIG, n_kv_heads=n_kv_heads)
    weights = init_weights(config, device="cuda", seed=0)
    dec = KVCacheDecoder(weights, config, batch_size=2, block_size=16)
    prompt = torch.randint(0, config.vocab_size, (2, 20), generator=torch.Generator().manual_seed(3)).cuda()
    logits = dec.prefill(prompt, chunk)
    full = llama_forward(weights, config, prompt)[:, -1]
    torch.testing.assert_close(logits.float(), full.float(), atol=8e-2, rtol=8e-2, msg="prefill")
    assert torch.equal(dec.seq_lens.cpu(), torch.tensor([20, 20], dtype=torch.int32))
    ids = torch.cat([prompt, dec.tokens.view(2, 1)], dim=1)
    for t in range(4):
        logits = dec.step()
        full = llama_forward(weights, config, ids)[:, -1]
        torch.testing.assert_close(logits.float(), full.float(), atol=8e-2, rtol=8e-2, msg=f"decode step {t}")
        dec.advance(logits)
        ids = torch.cat([ids, dec.tokens.view(2, 1)], dim=1)


def test_kvcache_decode_graph_replay_matches_eager():
    """The decode step captured once and replayed (tokens and lengths advanced
    on the device between replays) equals an eager decoder step by step."""
    from lightserve_amd.model.graph_decode import KVCacheDecoder, capture
    print("case kv-cache decode graph replay", flush=True)
    config = replace(TOY_CONFIG, n_kv_heads=2)
    weights = init_weights(config, device="cuda", seed=0)
    eager, graphed = (KVCacheDecoder(weights, config, batch_size=3, block_size=4) for _ in range(2))
    graph, out = capture(graphed.step)
    graphed.seq_lens.zero_()
    graphed.tokens.fill_(1)
    for t in range(6):
        ref = eager.step()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"step {t}"
        eager.advance(ref)
        graphed.advance(out)


def _to(weights, device, dtype):
    """Copy of a LlamaWeights on another device/dtype."""
    from lightserve_amd.model.minimal_llama import LayerWeights, LlamaWeights
    cv = lambda t: t.to(device=device, dtype=dtype)  # noqa: E731
    layers = [LayerWeights(**{f: cv(getattr(L, f)) for f in L.__dataclass_fields__}) for L in weights.layers]
    return LlamaWeights(embed_tokens=cv(weights.embed_tokens), layers=layers, norm_weight=cv(weights.norm_weight),
                        lm_head=cv(weights.lm_head))
