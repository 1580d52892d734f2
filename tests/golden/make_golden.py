"""Writes the golden fixtures used by tests/test_oracle.py.

    python tests/golden/make_golden.py

The reference ships no golden vectors (its checks are runtime comparisons
with SDPA), so these fixtures come from an implementation that shares no code
with the torch oracle: the pure-Python loops of oracle.attention.naive_attention
(math.exp, float64 sums). Inputs are stored alongside (small cases) or pinned
by a SHA-256 of their bytes (config 1, regenerated from its seed).
"""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.attention import naive_attention  # noqa: E402
from lightserve_amd.workloads import make_config_inputs  # noqa: E402


def tensor_sha256(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def tiny_cases():
    """(name, H, Hkv, Nq, Nk, D, causal, scale) edge cases: single row, odd
    lengths, non-power-of-two head dim, Nq != Nk (bottom-right causal), GQA."""
    return [
        ("n1_d8", 1, 1, 1, 1, 8, False, None),
        ("n1_d8_causal", 1, 1, 1, 1, 8, True, None),
        ("n17_d32", 1, 1, 17, 17, 32, False, None),
        ("n17_d32_causal", 1, 1, 17, 17, 32, True, None),
        ("h2_n9_d16_causal", 2, 2, 9, 9, 16, True, None),
        ("n10_d12_causal_scale", 1, 1, 10, 10, 12, True, 0.37),
        ("nq5_nk12_causal", 2, 2, 5, 12, 16, True, None),
        ("gqa_h4_kv2_nq6_nk9_causal", 4, 2, 6, 9, 8, True, None),
    ]


def main():
    out = {}
    g = torch.Generator().manual_seed(1234)
    for name, H, Hkv, nq, nk, d, causal, scale in tiny_cases():
        q = torch.randn(H, nq, d, generator=g, dtype=torch.float64)
        k = torch.randn(Hkv, nk, d, generator=g, dtype=torch.float64)
        v = torch.randn(Hkv, nk, d, generator=g, dtype=torch.float64)
        o, lse = naive_attention(q.tolist(), k.tolist(), v.tolist(), causal, scale, group=H // Hkv)
        out[f"{name}/q"] = q.numpy()
        out[f"{name}/k"] = k.numpy()
        out[f"{name}/v"] = v.numpy()
        out[f"{name}/o"] = np.array(o)
        out[f"{name}/lse"] = np.array(lse)
        out[f"{name}/meta"] = np.array([H, Hkv, nq, nk, d, int(causal), -1.0 if scale is None else scale])

    # Config 1 (fp32, causal, 1x4x256x64, seed 0): outputs of every 8th row.
    inp = make_config_inputs(1)
    q, k, v = inp["q"][0].double(), inp["k"][0].double(), inp["v"][0].double()
    o, lse = naive_attention(q.tolist(), k.tolist(), v.tolist(), True, None)
    o = np.array(o)
    out["cfg1/o_rows"] = o[:, ::8, :]
    out["cfg1/lse"] = np.array(lse)
    out["cfg1/o_sum"] = np.array([o.sum(), (o * o).sum()])
    out["cfg1/sha256"] = np.array([tensor_sha256(inp[n]) for n in ("q", "k", "v")])
    path = os.path.join(HERE, "attention_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
