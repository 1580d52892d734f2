"""Minimal LLaMA-shaped forward on MI355X around this library's attention.

Mirror of the reference's model/minimal_llama.py (same dataclasses, weight
layout, initialisation and entry points), so its tests and
model/cuda_graph_decode.py run against this module unchanged. What differs:

  - Attention is lightserve_amd's (flash_attention_forward for plain MHA, as
    the reference calls it at model/minimal_llama.py:221; the varlen entry
    point for grouped-query attention, which the reference's kernel cannot
    express, model/minimal_llama.py:8-12). n_kv_heads selects GQA; None keeps
    the reference's MHA shape.
  - RoPE is one HIP launch that rotates q and k in place (lsfa_rope)
    instead of the reference's elementwise tensor ops (:163-173).
  - Every residual add + RMSNorm is one lsfa_rmsnorm launch
    (kernels.fused_rmsnorm_residual.fused_add_rmsnorm), as the reference uses
    its fused kernel (:197-238): a sublayer's output is folded into the
    residual by the next norm. The first norm has no pending output and is
    the same kernel without the add (the reference adds a zero tensor).
  - Linear layers go through kernels.tiled_matmul.matmul on the reference's
    [in, out] weights, as the reference's do through its tiled GEMM: hipBLASLt
    for prefill-sized products, the library's skinny kernel (lsfa_gemv) for
    products of at most 8 rows (decode steps).
The forward needs no host synchronisation, so it can be captured in a HIP
graph (model/graph_decode.py).
"""
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

from ..kernels.flash_attention import flash_attention_forward
from ..kernels.fused_rmsnorm_residual import fused_add_rmsnorm
from ..kernels.fused_rmsnorm_residual import rmsnorm as rmsnorm_kernel
from ..kernels.flash_attention_varlen import flash_attention_varlen_forward
from ..kernels.rope import apply_rope_
from ..kernels.tiled_matmul import matmul


@dataclass
class LlamaConfig:
    """model/minimal_llama.py:49-67, plus n_kv_heads (None: plain MHA)."""
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    n_layers: int
    n_heads: int
    head_dim: int
    max_seq_len: int
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    dtype: torch.dtype = torch.bfloat16
    n_kv_heads: Optional[int] = None

    def __post_init__(self):
        assert self.hidden_size == self.n_heads * self.head_dim, (
            f"hidden_size ({self.hidden_size}) must equal n_heads*head_dim "
            f"({self.n_heads}*{self.head_dim}={self.n_heads * self.head_dim})"
        )
        if self.n_kv_heads is not None:
            assert 0 < self.n_kv_heads <= self.n_heads and self.n_heads % self.n_kv_heads == 0, \
                f"n_heads ({self.n_heads}) must be a multiple of n_kv_heads ({self.n_kv_heads})"

    @property
    def kv_heads(self):
        return self.n_kv_heads or self.n_heads


TOY_CONFIG = LlamaConfig(
    vocab_size=256, hidden_size=256, intermediate_size=688,
    n_layers=2, n_heads=4, head_dim=64, max_seq_len=64,
)


def llama3_8b_shape(n_layers: int = 4, max_seq_len: int = 128, gqa: bool = False) -> LlamaConfig:
    """LLaMA-3-8B's per-layer shape (model/minimal_llama.py:76-85); gqa=True
    uses its real 8 KV heads."""
    return LlamaConfig(
        vocab_size=128256, hidden_size=4096, intermediate_size=14336,
        n_layers=n_layers, n_heads=32, head_dim=128, max_seq_len=max_seq_len,
        n_kv_heads=8 if gqa else None,
    )


@dataclass
class LayerWeights:
    input_layernorm_weight: torch.Tensor
    q_proj: torch.Tensor
    k_proj: torch.Tensor
    v_proj: torch.Tensor
    o_proj: torch.Tensor
    post_attention_layernorm_weight: torch.Tensor
    gate_proj: torch.Tensor
    up_proj: torch.Tensor
    down_proj: torch.Tensor


@dataclass
class LlamaWeights:
    embed_tokens: torch.Tensor
    layers: list = field(default_factory=list)
    norm_weight: torch.Tensor = None
    lm_head: torch.Tensor = None


def init_weights(config: LlamaConfig, device: str = "cuda", seed: int = 0) -> LlamaWeights:
    """Random weights with the reference's draw order and scale
    (model/minimal_llama.py:107-141: N(0, 0.02) in fp32, cast), so a given
    seed gives the reference's weights for the MHA shape."""
    g = torch.Generator(device=device).manual_seed(seed)

    def randn(*shape):
        return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * 0.02).to(config.dtype)

    def ones(*shape):
        return torch.ones(*shape, device=device, dtype=config.dtype)

    H, I, V = config.hidden_size, config.intermediate_size, config.vocab_size
    q_dim = config.n_heads * config.head_dim
    kv_dim = config.kv_heads * config.head_dim
    layers = []
    for _ in range(config.n_layers):
        layers.append(LayerWeights(
            input_layernorm_weight=ones(H),
            q_proj=randn(H, q_dim), k_proj=randn(H, kv_dim), v_proj=randn(H, kv_dim), o_proj=randn(q_dim, H),
            post_attention_layernorm_weight=ones(H),
            gate_proj=randn(H, I), up_proj=randn(H, I), down_proj=randn(I, H),
        ))
    return LlamaWeights(embed_tokens=randn(V, H), layers=layers, norm_weight=ones(H), lm_head=randn(H, V))


def precompute_rope(config: LlamaConfig, device):
    """cos/sin tables [max_seq_len, head_dim] in the model dtype
    (model/minimal_llama.py:144-156)."""
    half = config.head_dim // 2
    inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))
    positions = torch.arange(config.max_seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    cos = torch.cat([freqs.cos(), freqs.cos()], dim=-1).to(config.dtype)
    sin = torch.cat([freqs.sin(), freqs.sin()], dim=-1).to(config.dtype)
    return cos, sin


def add_norm(x, residual, weight, eps):
    """(rmsnorm(x + residual) * weight, x + residual) in one launch; x None
    (nothing pending) normalises the residual alone."""
    if x is None:
        return rmsnorm_kernel(residual, weight, eps), residual
    return fused_add_rmsnorm(x, residual, weight, eps)


def attention_block(layer, config, normed_2d, B, N, cos, sin, causal, positions=None):
    """q/k/v projections, in-place RoPE, attention; returns [B*N, n_heads*head_dim]."""
    nh, nkv, hd = config.n_heads, config.kv_heads, config.head_dim
    q = matmul(normed_2d, layer.q_proj)   # [B*N, nh*hd]
    k = matmul(normed_2d, layer.k_proj)   # [B*N, nkv*hd]
    v = matmul(normed_2d, layer.v_proj)
    q4 = q.view(B, N, nh, hd).transpose(1, 2)   # [B, nh, N, hd] views, no copies
    k4 = k.view(B, N, nkv, hd).transpose(1, 2)
    apply_rope_(q4, k4, cos, sin, positions)
    if nkv == nh:
        o = flash_attention_forward(q4, k4, v.view(B, N, nh, hd).transpose(1, 2), causal=causal)
        return o.transpose(1, 2).reshape(B * N, nh * hd)
    cu = torch.arange(0, (B + 1) * N, N, device=q.device, dtype=torch.int32)
    o, _ = flash_attention_varlen_forward(q.view(B * N, nh, hd), k.view(B * N, nkv, hd), v.view(B * N, nkv, hd),
                                          cu, cu, N, N, causal=causal)
    return o.reshape(B * N, nh * hd)


def llama_forward(weights: LlamaWeights, config: LlamaConfig, input_ids: torch.Tensor, causal: bool = True,
                  rope_tables=None) -> torch.Tensor:
    """input_ids [B, N] -> logits [B, N, vocab_size] (model/minimal_llama.py:181-251).
    rope_tables: precomputed (cos, sin), to keep them out of a captured graph."""
    B, N = input_ids.shape
    H = config.hidden_size
    cos, sin = rope_tables if rope_tables is not None else precompute_rope(config, input_ids.device)
    residual = F.embedding(input_ids, weights.embed_tokens).reshape(B * N, H)
    pending = None  # the last sublayer's output, added to the residual by the next norm
    for layer in weights.layers:
        normed, residual = add_norm(pending, residual, layer.input_layernorm_weight, config.rms_eps)
        attn = attention_block(layer, config, normed, B, N, cos, sin, causal)
        normed2, residual = fused_add_rmsnorm(matmul(attn, layer.o_proj), residual,
                                              layer.post_attention_layernorm_weight, config.rms_eps)
        mlp = F.silu(matmul(normed2, layer.gate_proj)) * matmul(normed2, layer.up_proj)
        pending = matmul(mlp, layer.down_proj)
    final, _ = add_norm(pending, residual, weights.norm_weight, config.rms_eps)
    return matmul(final, weights.lm_head).reshape(B, N, config.vocab_size)
