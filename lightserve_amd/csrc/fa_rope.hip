// Rotary position embedding applied in place to q and k, one pass, one launch.
//
// The reference applies RoPE with plain tensor ops on [B, H, N, D] views of
// the projection outputs (model/minimal_llama.py:163-173): x * cos +
// rotate_half(x) * sin, rotate_half(x) = cat(-x2, x1) for the two halves
// x1 = x[..., :D/2], x2 = x[..., D/2:], with cos/sin rows taken at the
// token's position. That is eight or so elementwise kernels per layer, each
// reading and writing q or k. Here one kernel reads each 16-byte group of
// the first half together with its partner group in the second half, forms
//   y1 = x1 * cos[:D/2] - x2 * sin[:D/2]
//   y2 = x2 * cos[D/2:] + x1 * sin[D/2:]
// in fp32 and writes both back rounded once to the input dtype.
//
// Thread layout: one thread per (token, head, group of VEC elements of the
// first half), VEC = 16 bytes / element size. q's heads come first, then
// k's, so a token's q and k rows are rotated by neighbouring threads.
// Positions: token n of sequence b sits at pos0[b] + n (pos0 = 0 when no
// start positions are given), clamped to the table's rows.
// With a K/V cache, each rotated k group is also stored at the token's cache
// slot, and a third run of threads (after q's and k's heads) copies v's
// groups (both halves) into the v cache: the append of a decode step or a
// prefill chunk needs no launch of its own.
#include "fa_common.hpp"

namespace lsfa {

template <typename T>
struct RopeVec;
template <>
struct RopeVec<__bf16> {
  using V = bf16x8;
  static constexpr int N = 8;
};
template <>
struct RopeVec<_Float16> {
  using V = f16x8;
  static constexpr int N = 8;
};
template <>
struct RopeVec<float> {
  typedef float V __attribute__((ext_vector_type(4)));
  static constexpr int N = 4;
};

template <typename T>
__global__ __launch_bounds__(256) void fa_rope_kernel(const RopeParams p) {
  using V = typename RopeVec<T>::V;
  constexpr int VEC = RopeVec<T>::N;
  const int b = blockIdx.y;
  const int half = p.D / 2;
  const int groups = half / VEC;
  const bool cache = p.k_cache != nullptr;
  const int heads = p.Hq + p.Hkv + (cache ? p.Hkv : 0);
  const int64_t per_tok = (int64_t)heads * groups;
  int n_tok = p.N;
  int64_t tok0 = 0;
  if (p.cu_seqlens != nullptr) {
    tok0 = p.cu_seqlens[b];
    n_tok = min(p.cu_seqlens[b + 1] - (int)tok0, p.N);
  }
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n_tok * per_tok) return;
  const int n = (int)(idx / per_tok);
  const int rem = (int)(idx - (int64_t)n * per_tok);
  const int hd = rem / groups;
  const int g = rem - hd * groups;

  int64_t slot = -1;
  if (cache) {
    if (p.block_tables != nullptr) {
      const int tp = (p.pos0 != nullptr ? p.pos0[b] : 0) + n;
      const int bi = tp >= 0 ? tp / p.block_size : -1;
      if (bi >= 0 && bi < p.max_blocks) {
        const int64_t blk = p.block_tables[(int64_t)b * p.sbt + bi];
        if (blk >= 0) slot = blk * p.block_size + (tp - bi * p.block_size);
      }
    } else {
      slot = p.slots[p.cu_seqlens != nullptr ? tok0 + n : (int64_t)b * p.N + n];
    }
    if (slot >= p.num_slots) slot = -1;
  }
  if (hd >= p.Hq + p.Hkv) {  // v head: copy into the cache
    if (slot < 0) return;
    const int h = hd - p.Hq - p.Hkv;
    const int64_t vrow = p.cu_seqlens != nullptr ? (tok0 + n) * p.sv[2] : (int64_t)b * p.sv[0] + (int64_t)n * p.sv[2];
    const T* vx = (const T*)p.v + vrow + (int64_t)h * p.sv[1];
    T* dst = (T*)p.v_cache + slot * p.cs_slot + (int64_t)h * p.cs_head;
    const int d1 = g * VEC, d2 = d1 + half;
    *(V*)(dst + d1) = *(const V*)(vx + d1);
    *(V*)(dst + d2) = *(const V*)(vx + d2);
    return;
  }
  const bool is_q = hd < p.Hq;
  const int h = is_q ? hd : hd - p.Hq;
  const int64_t* st = is_q ? p.sq : p.sk;
  T* base = (T*)(is_q ? p.q : p.k);
  const int64_t row = p.cu_seqlens != nullptr ? (tok0 + n) * st[2] : (int64_t)b * st[0] + (int64_t)n * st[2];
  T* x = base + row + (int64_t)h * st[1];

  int pos = (p.pos0 != nullptr ? p.pos0[b] : 0) + n;
  pos = min(max(pos, 0), p.max_pos - 1);
  const T* cs = (const T*)p.cos + (int64_t)pos * p.table_stride;
  const T* sn = (const T*)p.sin + (int64_t)pos * p.table_stride;

  const int d1 = g * VEC, d2 = d1 + half;
  const V x1 = *(const V*)(x + d1), x2 = *(const V*)(x + d2);
  const V c1 = *(const V*)(cs + d1), c2 = *(const V*)(cs + d2);
  const V s1 = *(const V*)(sn + d1), s2 = *(const V*)(sn + d2);
  V y1, y2;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float a = (float)x1[e], c = (float)x2[e];
    y1[e] = (T)(a * (float)c1[e] - c * (float)s1[e]);
    y2[e] = (T)(c * (float)c2[e] + a * (float)s2[e]);
  }
  *(V*)(x + d1) = y1;
  *(V*)(x + d2) = y2;
  if (!is_q && slot >= 0) {
    T* dst = (T*)p.k_cache + slot * p.cs_slot + (int64_t)h * p.cs_head;
    *(V*)(dst + d1) = y1;
    *(V*)(dst + d2) = y2;
  }
}

// Host entry used by the C ABI layer (arguments already validated).
hipError_t rope_inplace(const RopeParams& p, int dtype, hipStream_t s) {
  const int vec = dtype == 0 ? 4 : 8;
  const int64_t threads = (int64_t)p.N * (p.Hq + p.Hkv + (p.k_cache != nullptr ? p.Hkv : 0)) * (p.D / 2 / vec);
  if (threads == 0 || p.B == 0) return hipSuccess;
  const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)p.B);
  if (dtype == 0)
    hipLaunchKernelGGL(fa_rope_kernel<float>, grid, dim3(256), 0, s, p);
  else if (dtype == 1)
    hipLaunchKernelGGL(fa_rope_kernel<_Float16>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(fa_rope_kernel<__bf16>, grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace lsfa
