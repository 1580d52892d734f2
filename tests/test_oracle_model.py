"""Pins of oracle/model.py (the reference's model forward restated in torch).

apply_rope is checked against RoPE's definition as a rotation: each pair
(x[d], x[d + D/2]) at position p turned by the angle p * theta^(-d/(D/2)),
built element by element in float64. reference_llama_forward is checked
against a pure-Python float64 loop over a tiny one-layer model (embedding,
RMSNorm, projections, RoPE, causal / full softmax attention, GQA head
sharing, SiLU-gated MLP, final norm and LM head). Planted mistakes (the
rotation's sign, a dropped RMSNorm epsilon, the GQA head mapping) fail them.
"""
import math

import pytest
import torch

from lightserve_amd.model.minimal_llama import LlamaConfig, init_weights
from oracle import model as om


def _rope_by_definition(x, positions, theta):
    """x [H, N, D] float64; position of token n is positions[n]."""
    H, N, D = x.shape
    half = D // 2
    out = x.clone()
    for h in range(H):
        for n in range(N):
            for d in range(half):
                ang = positions[n] * theta ** (-d / half)
                a, b = x[h, n, d].item(), x[h, n, d + half].item()
                out[h, n, d] = a * math.cos(ang) - b * math.sin(ang)
                out[h, n, d + half] = b * math.cos(ang) + a * math.sin(ang)
    return out


@pytest.mark.parametrize("offset", [None, 5])
def test_apply_rope_is_a_rotation(offset):
    g = torch.Generator().manual_seed(0)
    D, N, theta = 8, 4, 10000.0
    q = torch.randn(1, 2, N, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, N, D, generator=g, dtype=torch.float64)
    cos, sin = om.precompute_rope(D, 16, theta, torch.float64, "cpu")
    pos = None if offset is None else torch.tensor([offset], dtype=torch.int32)
    qr, kr = om.apply_rope(q, k, cos, sin, N, positions=pos)
    positions = [(offset or 0) + n for n in range(N)]
    torch.testing.assert_close(qr[0], _rope_by_definition(q[0], positions, theta), atol=1e-5, rtol=0)
    torch.testing.assert_close(kr[0], _rope_by_definition(k[0], positions, theta), atol=1e-5, rtol=0)
    # norms are preserved (a rotation), and a planted sign flip is caught
    torch.testing.assert_close(qr.norm(dim=-1), q.norm(dim=-1))
    bad = q * cos[:N].view(1, 1, N, -1) - om.rotate_half(q) * sin[:N].view(1, 1, N, -1)
    assert (bad[0] - _rope_by_definition(q[0], positions, theta)).abs().max() > 1e-2


def _tiny_config(n_kv_heads):
    """Plain MHA: 2 heads of 4 dims; GQA: 4 query heads of 2 dims on n_kv_heads."""
    nh, hd = (2, 4) if n_kv_heads is None else (4, 2)
    return LlamaConfig(vocab_size=11, hidden_size=8, intermediate_size=6, n_layers=1, n_heads=nh, head_dim=hd,
                       max_seq_len=8, rope_theta=100.0, rms_eps=1e-5, dtype=torch.float64, n_kv_heads=n_kv_heads)


def _forward_loops(w, cfg, ids, causal, eps=None, round_robin=False):
    """Pure-Python float64 forward of a one-layer model, batch of 1. Query head
    h reads KV head h // (n_heads / n_kv_heads) (round_robin: h % n_kv_heads,
    a planted mistake)."""
    eps = cfg.rms_eps if eps is None else eps
    N, H, hd, nh = len(ids), cfg.hidden_size, cfg.head_dim, cfg.n_heads
    nkv = cfg.kv_heads
    grp = nh // nkv

    def mat(rows, m):  # rows [N][in] @ m [in][out]
        return [[sum(r[i] * m[i][j] for i in range(len(r))) for j in range(len(m[0]))] for r in rows]

    def norm(rows, wt):
        out = []
        for r in rows:
            s = math.sqrt(sum(x * x for x in r) / len(r) + eps)
            out.append([r[i] / s * wt[i] for i in range(len(r))])
        return out

    T = lambda t: t.tolist()  # noqa: E731
    L = w.layers[0]
    x = [T(w.embed_tokens[i]) for i in ids]
    h = norm(x, T(L.input_layernorm_weight))
    q, k, v = mat(h, T(L.q_proj)), mat(h, T(L.k_proj)), mat(h, T(L.v_proj))
    half = hd // 2

    def rope(vec, pos):
        out = list(vec)
        for d in range(half):
            ang = pos * cfg.rope_theta ** (-d / half)
            a, b = vec[d], vec[d + half]
            out[d] = a * math.cos(ang) - b * math.sin(ang)
            out[d + half] = b * math.cos(ang) + a * math.sin(ang)
        return out

    attn = [[0.0] * (nh * hd) for _ in range(N)]
    for head in range(nh):
        kvh = head % nkv if round_robin else head // grp
        for i in range(N):
            qi = rope(q[i][head * hd:(head + 1) * hd], i)
            js = range(i + 1) if causal else range(N)
            sc = [sum(a * b for a, b in zip(qi, rope(k[j][kvh * hd:(kvh + 1) * hd], j))) / math.sqrt(hd) for j in js]
            m = max(sc)
            e = [math.exp(s - m) for s in sc]
            z = sum(e)
            for d in range(hd):
                attn[i][head * hd + d] = sum(e[t] / z * v[j][kvh * hd + d] for t, j in enumerate(js))
    o = mat(attn, T(L.o_proj))
    res = [[x[i][c] + o[i][c] for c in range(H)] for i in range(N)]
    h2 = norm(res, T(L.post_attention_layernorm_weight))
    gate, up = mat(h2, T(L.gate_proj)), mat(h2, T(L.up_proj))
    mlp = [[g / (1 + math.exp(-g)) * u for g, u in zip(gr, ur)] for gr, ur in zip(gate, up)]
    d = mat(mlp, T(L.down_proj))
    res = [[res[i][c] + d[i][c] for c in range(H)] for i in range(N)]
    return torch.tensor(mat(norm(res, T(w.norm_weight)), T(w.lm_head)), dtype=torch.float64)


@pytest.mark.parametrize("n_kv_heads", [None, 2])
@pytest.mark.parametrize("causal", [True, False])
def test_reference_forward_matches_loops(n_kv_heads, causal):
    cfg = _tiny_config(n_kv_heads)
    w = init_weights(cfg, device="cpu", seed=3)
    # weights of order 1 so that every sublayer moves the logits visibly
    for t in [w.embed_tokens, w.lm_head] + [getattr(w.layers[0], f) for f in
                                            ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")]:
        t.mul_(50.0)
    ids = [3, 7, 1, 10, 0]
    got = om.reference_llama_forward(w, cfg, torch.tensor([ids]), causal=causal)[0]
    want = _forward_loops(w, cfg, ids, causal)
    # The tables follow the reference's float32 angle computation
    # (model/minimal_llama.py:151-153), so they match float64 angles to ~1e-6.
    torch.testing.assert_close(got, want, atol=2e-5, rtol=1e-4)
    # planted mistakes: RMSNorm without its epsilon; GQA heads mapped round-robin
    assert (_forward_loops(w, cfg, ids, causal, eps=1e-1) - want).abs().max() > 1e-2
    if n_kv_heads is not None:
        assert (_forward_loops(w, cfg, ids, causal, round_robin=True) - want).abs().max() > 1e-2


@pytest.mark.parametrize("with_residual", [True, False])
def test_add_rmsnorm_reference_matches_loops(with_residual):
    """h = x + r; out_j = h_j / sqrt(sum_i h_i^2 / N + eps) * w_j, by hand."""
    g = torch.Generator().manual_seed(1)
    x, r = torch.randn(3, 5, generator=g, dtype=torch.float64), torch.randn(3, 5, generator=g, dtype=torch.float64)
    w = torch.randn(5, generator=g, dtype=torch.float64)
    eps = 1e-6
    out, h = om.add_rmsnorm_reference(x, r if with_residual else None, w, eps)
    for i in range(3):
        hv = [x[i, j].item() + (r[i, j].item() if with_residual else 0.0) for j in range(5)]
        s = math.sqrt(sum(v * v for v in hv) / 5 + eps)
        for j in range(5):
            assert abs(h[i, j].item() - hv[j]) < 1e-12
            # statistics in fp32, as the reference computes them (.float())
            assert abs(out[i, j].item() - hv[j] / s * w[j].item()) < 1e-6 * max(1.0, abs(out[i, j].item()))
    # planted mistake: eps added outside the square root (visible with a large eps)
    big, _ = om.add_rmsnorm_reference(x, r if with_residual else None, w, 0.5)
    bad = h / (h.pow(2).mean(-1, keepdim=True).sqrt() + 0.5) * w
    assert (bad - big).abs().max() > 1e-2
    # unit RMS before the weight
    ones, _ = om.add_rmsnorm_reference(x, r, torch.ones(5, dtype=torch.float64), 0.0)
    torch.testing.assert_close(ones.pow(2).mean(-1), torch.ones(3, dtype=torch.float64))
