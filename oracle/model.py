"""Plain-PyTorch restatement of the reference's minimal LLaMA forward -- TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py for who may import it).

Follows model/minimal_llama.py (the reference):
  precompute_rope         :144-156  cos/sin tables [max_seq_len, head_dim], cast to the model dtype
  rotate_half, apply_rope :159-173  x * cos + rotate_half(x) * sin on [B, H, N, D]
  add_rmsnorm_reference   kernels/fused_rmsnorm_residual.py:40-70 (fused add + RMSNorm)
  reference_llama_forward :254-293  F.linear / SDPA / hand-written RMSNorm, the ground truth
                                    its llama_forward is tested against
                                    (model/tests/test_minimal_llama.py)
One extension the reference lacks: n_kv_heads < n_heads (grouped-query
attention), expanded with repeat_interleave over the head axis, the
reference's own GQA convention (benchmarks/profiling/roofline/measure_roofline.py:94-98).

Pinned in tests/test_oracle_model.py: apply_rope against the rotation-matrix form
of RoPE built element by element (each pair (d, d + D/2) rotated by the
angle pos * theta^(-2d/D)), which also fixes the table construction;
reference_llama_forward's attention against attention_reference, and the
whole forward against a pure-Python loop on a tiny one-layer model;
add_rmsnorm_reference against per-element Python sums (a planted eps outside
the square root fails).
"""
import torch
import torch.nn.functional as F


def precompute_rope(head_dim, max_seq_len, theta, dtype, device):
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))
    positions = torch.arange(max_seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    cos = torch.cat([freqs.cos(), freqs.cos()], dim=-1).to(dtype)
    sin = torch.cat([freqs.sin(), freqs.sin()], dim=-1).to(dtype)
    return cos, sin


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def apply_rope(q, k, cos, sin, n, positions=None):
    """q, k [B, H, n, D]; rows 0..n-1 of the tables (or rows positions[b] + i).
    Evaluated in the tables' dtype, as the reference does."""
    if positions is None:
        c = cos[:n].view(1, 1, n, -1)
        s = sin[:n].view(1, 1, n, -1)
    else:
        idx = positions.long().view(-1, 1) + torch.arange(n, device=cos.device).view(1, -1)
        c = cos[idx].unsqueeze(1)
        s = sin[idx].unsqueeze(1)
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s


def add_rmsnorm_reference(x, residual, weight, eps):
    """The reference's fused add + RMSNorm semantics
    (kernels/fused_rmsnorm_residual.py:40-70, its test's reference
    kernels/tests/test_fused_rmsnorm_residual.py:24-29): h = x + residual in
    the input dtype, fp32 statistics, output rounded once. residual None: h = x."""
    h = x if residual is None else x + residual
    var = h.float().pow(2).mean(-1, keepdim=True)
    return (h.float() * torch.rsqrt(var + eps) * weight.float()).to(x.dtype), h


def rmsnorm(h, weight, eps):
    h32 = h.float()
    var = h32.pow(2).mean(-1, keepdim=True)
    return (h32 * torch.rsqrt(var + eps)).to(h.dtype) * weight


def reference_llama_forward(weights, config, input_ids, causal=True):
    """The reference's reference_llama_forward (model/minimal_llama.py:254-293)
    with GQA support; `weights`/`config` are lightserve_amd.model's dataclasses
    (same fields as the reference's)."""
    B, N = input_ids.shape
    hd, nh = config.head_dim, config.n_heads
    nkv = config.n_kv_heads or nh
    cos, sin = precompute_rope(hd, config.max_seq_len, config.rope_theta, config.dtype, input_ids.device)
    x = F.embedding(input_ids, weights.embed_tokens)
    residual = x
    for layer in weights.layers:
        normed = rmsnorm(residual, layer.input_layernorm_weight, config.rms_eps)
        q = F.linear(normed, layer.q_proj.t()).view(B, N, nh, hd).transpose(1, 2)
        k = F.linear(normed, layer.k_proj.t()).view(B, N, nkv, hd).transpose(1, 2)
        v = F.linear(normed, layer.v_proj.t()).view(B, N, nkv, hd).transpose(1, 2)
        q, k = apply_rope(q, k, cos, sin, N)
        if nkv != nh:
            k = k.repeat_interleave(nh // nkv, dim=1)
            v = v.repeat_interleave(nh // nkv, dim=1)
        attn = F.scaled_dot_product_attention(q, k.contiguous(), v.contiguous(), is_causal=causal)
        attn = attn.transpose(1, 2).reshape(B, N, nh * hd)
        residual = residual + F.linear(attn, layer.o_proj.t())
        normed2 = rmsnorm(residual, layer.post_attention_layernorm_weight, config.rms_eps)
        mlp = F.silu(F.linear(normed2, layer.gate_proj.t())) * F.linear(normed2, layer.up_proj.t())
        residual = residual + F.linear(mlp, layer.down_proj.t())
    return F.linear(rmsnorm(residual, weights.norm_weight, config.rms_eps), weights.lm_head.t())
