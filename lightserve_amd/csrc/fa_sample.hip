// Greedy next token for a decode step: tokens[r] = argmax(logits[r, :]) and,
// optionally, seq_lens[r] += 1, in one launch (the reference takes the argmax
// of the step's logits with torch, model/cuda_graph_decode.py:114 and :145,
// and advances the sequence length separately).
//
// One 1024-thread workgroup per row. Each thread scans columns tid*8 + j*8192
// with 16-byte loads (8 elements) when the row is 16-byte aligned and its
// width a multiple of 8, else one element at a time; the running best is
// merged with wave shuffles and one LDS exchange between the 16 waves.
// Comparison as torch's argmax: NaN beats every number, and equal values
// (or two NaNs) go to the lower index. The scan compares order-preserving
// integer keys (branch-free): a float's bits with the sign bit flipped for
// positives and all bits flipped for negatives, every NaN mapped to the
// largest key and -0 to +0, so equal values have equal keys; a thread visits
// its columns in increasing order and keeps the first of equal keys.
#include "fa_common.hpp"

namespace lsfa {

struct GreedyParams {
  const void* logits;
  int64_t stride;
  int64_t* tokens;
  int32_t* seq_lens;  // optional
  int rows, cols;
  bool vec;
};

constexpr int kGreedyThreads = 1024;

__device__ __forceinline__ uint32_t greedy_key(float f) {
  uint32_t u = __float_as_uint(f);
  u = u == 0x80000000u ? 0u : u;
  const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return f != f ? 0xffffffffu : key;
}
__device__ __forceinline__ bool greedy_better(uint32_t a, int ia, uint32_t b, int ib) {
  return a > b || (a == b && ia < ib);
}

template <typename T>
__global__ __launch_bounds__(kGreedyThreads) void fa_greedy_kernel(const GreedyParams p) {
  __shared__ uint32_t best_v[kGreedyThreads / 64];
  __shared__ int best_i[kGreedyThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const T* x = (const T*)p.logits + (int64_t)row * p.stride;
  uint32_t bv = 0;  // below every key (the smallest, that of -inf, is 0x007fffff)
  int bi = 0x7fffffff;
  bool scanned = false;
  if constexpr (sizeof(T) == 2) {
    if (p.vec) {
      // Eight 16-byte loads in flight per thread before the comparisons (one
      // workgroup streams the row, so latency, not bandwidth, sets its time).
      using V = typename VecT<T>::x8;
      constexpr int kStride = kGreedyThreads * 8;
      for (int c0 = tid * 8; c0 < p.cols; c0 += 8 * kStride) {
        V v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int c = c0 + u * kStride;
          if (c < p.cols) v[u] = __builtin_nontemporal_load((const V*)(x + c));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int c = c0 + u * kStride;
          if (c < p.cols) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t key = greedy_key((float)v[u][e]);
              const bool take = key > bv;  // columns rise: the first of equal keys stays
              bv = take ? key : bv;
              bi = take ? c + e : bi;
            }
          }
        }
      }
      scanned = true;
    }
  }
  if (!scanned) {
    for (int c = tid; c < p.cols; c += kGreedyThreads) {
      const uint32_t key = greedy_key((float)x[c]);
      const bool take = key > bv;
      bv = take ? key : bv;
      bi = take ? c : bi;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (greedy_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { best_v[tid >> 6] = bv; best_i[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kGreedyThreads / 64; ++w)
      if (greedy_better(best_v[w], best_i[w], bv, bi)) { bv = best_v[w]; bi = best_i[w]; }
    // A row of -inf only (or an empty row) still names a column: the first.
    p.tokens[row] = bi == 0x7fffffff ? 0 : bi;
    if (p.seq_lens) p.seq_lens[row] += 1;
  }
}

// Host entry used by the C ABI layer (arguments validated there).
hipError_t greedy(const void* logits, int64_t stride, int dtype, int rows, int cols, int64_t* tokens,
                  int32_t* seq_lens, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  GreedyParams p;
  p.logits = logits; p.stride = stride; p.tokens = tokens; p.seq_lens = seq_lens; p.rows = rows; p.cols = cols;
  p.vec = dtype != 0 && cols % 8 == 0 && stride % 8 == 0 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
  if (dtype == 0)
    hipLaunchKernelGGL(fa_greedy_kernel<float>, dim3(rows), dim3(kGreedyThreads), 0, s, p);
  else if (dtype == 1)
    hipLaunchKernelGGL(fa_greedy_kernel<_Float16>, dim3(rows), dim3(kGreedyThreads), 0, s, p);
  else
    hipLaunchKernelGGL(fa_greedy_kernel<__bf16>, dim3(rows), dim3(kGreedyThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace lsfa
