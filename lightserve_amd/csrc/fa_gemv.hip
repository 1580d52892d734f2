// Skinny GEMM (M <= 8 rows) for decode-time projections: y[M, N] = x[M, K] @ W[K, N]
// with W in the [in, out] row-major layout the model stores
// (model/minimal_llama.py's weights), bf16/fp16 in, fp32 accumulate. Up to
// four matrices that share x (a decoder's q/k/v or gate/up projections) run
// as one launch over their concatenated columns. The input may be given as
// the operands of a residual add + RMSNorm (the norm then needs no launch of
// its own) or of SwiGLU.
//
// At M <= 8 the product is a pass over W (about M FLOP per weight byte), so it
// is HBM-bound: the kernel is built to stream W once at full rate, in one
// launch.
//   Grid (ceil(N / 256), splits). A workgroup owns 256 columns and one K-range
//   of kc rows; thread (cg, kg) = (tid % 32, tid / 32) reads 16 bytes
//   (8 columns) of rows kg, kg + 8, ... of the range, eight rows in flight, so
//   each wave-load covers two 512-byte row segments, and keeps M x 8 fp32
//   sums. The products run on v_dot2_f32_{bf16,f16}: a thread's rows k and
//   k + 8 (k % 16 < 8) are paired column by column with one v_perm_b32 per two
//   columns, and x's K-range sits in LDS as the matching pairs
//   (x[k], x[k + 8]), so two rows cost 8 permutes and 8 * M dot2 instead of
//   16 conversions and 16 * M fp32 FMAs. The 8 K-groups are summed through
//   LDS.
//   With one split the workgroup rounds its sums into y. Otherwise it stores
//   them as an fp32 partial block [split][M][256 columns] and counts its
//   arrival in two levels: split s adds one to sub-counter s % 8 of its column
//   block, and the last arrival of each sub-group adds one to the block's main
//   counter. Atomics on one address serialise at about 175 ns each on MI355X,
//   so one counter for 64 splits costs 11 us; two levels cost at most 8 + 8.
//   The workgroup that arrives last at the main counter sums the splits'
//   partials, rounds once into y, and every counter is put back to zero by the
//   workgroup that completed it, so all are zero again when the launch ends.
//   Deterministic: the order of the sum does not depend on which workgroup
//   arrives last. No memsets: graph-capturable.
//   Hand-over without cache maintenance: the partials are written and read
//   with device-scope atomic stores and loads (coherent across the XCDs' L2s
//   without a writeback or an invalidate) and every store has completed
//   (s_waitcnt vmcnt(0)) before the workgroup's barrier and its counter add.
//   That is the compiler's own release sequence for device scope minus the L2
//   writeback (buffer_wbl2), which only non-atomic stores need; a release
//   fence would write the L2 back once per workgroup, about 10x the time of
//   the whole pass.
#include "fa_common.hpp"

namespace lsfa {

constexpr int kGemvCols = 256;  // columns per workgroup (32 groups of 8)
constexpr int kGemvKG = 8;      // K-groups per workgroup
constexpr int kGemvCounterSlots = 16;  // per column block: 8 sub-counters, the main counter, padding
typedef uint64_t u64x2x2[4];    // 8 fp32 partials as four 8-byte words

// Matrix of virtual column n (uniform selects, no indexing of the kernel
// arguments by a lane value).
__device__ __forceinline__ int gemv_group(const GemvParams& p, int n) {
  return (n >= p.col_off[1]) + (n >= p.col_off[2]) + (n >= p.col_off[3]);
}
template <typename V>
__device__ __forceinline__ V gemv_pick(int g, V a0, V a1, V a2, V a3) {
  return g == 0 ? a0 : (g == 1 ? a1 : (g == 2 ? a2 : a3));
}
template <typename T>
__device__ __forceinline__ T* gemv_out(const GemvParams& p, int n, int m) {
  const int g = gemv_group(p, n);
  T* y = (T*)gemv_pick(g, p.y[0], p.y[1], p.y[2], p.y[3]);
  const int64_t sy = gemv_pick(g, p.sy[0], p.sy[1], p.sy[2], p.sy[3]);
  const int col_off = gemv_pick(g, p.col_off[0], p.col_off[1], p.col_off[2], p.col_off[3]);
  return y + (int64_t)m * sy + (n - col_off);
}

// acc + w.x * x.x + w.y * x.y for two packed bf16/fp16 pairs.
__device__ __forceinline__ float gemv_dot2(uint32_t w, uint32_t x, float acc, __bf16*) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x), acc, false);
}
__device__ __forceinline__ float gemv_dot2(uint32_t w, uint32_t x, float acc, _Float16*) {
  typedef __fp16 half2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w), __builtin_bit_cast(half2_t, x), acc, false);
}
template <typename T>
__device__ __forceinline__ uint32_t gemv_pack(T a, T b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
// Pair slots of a K-range of kc rows: pair (k, k + 8) with k % 16 < 8 sits at
// (k / 16) * 8 + k % 8.
__host__ __device__ constexpr int gemv_pair_slots(int kc) { return (kc + 15) / 16 * 8; }

// M is the compile-time row capacity (1, 2, 4 or 8); p.M <= M rows are real.
// Rows past p.M have x = 0 in LDS and their sums are not stored.
template <typename T, int M>
__global__ __launch_bounds__(256) void fa_gemv_kernel(const GemvParams p) {
  extern __shared__ float gemv_smem[];  // x chunk [M][kc], then the K-group sums
  __shared__ int last_arrival;
  const int tid = threadIdx.x;
  const int cg = tid & 31, kg = tid >> 5;
  const int n0 = blockIdx.x * kGemvCols + cg * 8;
  const int split = blockIdx.y;
  const int k_begin = split * p.kc;
  const int k_len = max(0, min(p.K, k_begin + p.kc) - k_begin);
  // This thread's rows of W: kg, kg + 8, ... of the K-range, in batches of
  // eight (one 16-byte load each, all issued before the first use). The
  // first batch is in flight before x is staged, so the two latencies
  // overlap.
  const bool has_cols = n0 < p.N;
  const int rows_t = (has_cols && kg < k_len) ? (k_len - kg + kGemvKG - 1) / kGemvKG : 0;
  const int full = rows_t >> 3, rem = rows_t & 7;
  const T* wp = nullptr;
  int64_t step = 0;
  if (has_cols) {
    const int g = gemv_group(p, n0);
    const int64_t sw = gemv_pick(g, p.sw[0], p.sw[1], p.sw[2], p.sw[3]);
    wp = (const T*)gemv_pick(g, p.w[0], p.w[1], p.w[2], p.w[3]) + (int64_t)(k_begin + kg) * sw +
         (n0 - gemv_pick(g, p.col_off[0], p.col_off[1], p.col_off[2], p.col_off[3]));
    step = (int64_t)kGemvKG * sw;
  }
  u32x4 cur[8];
  if (full > 0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = __builtin_nontemporal_load((const u32x4*)(wp + u * step));
    wp += 8 * step;
  }

  // RMSNorm input: every workgroup forms the whole row's sum of squares of
  // h = x + residual in the order of the vector RMSNorm kernel (256 threads,
  // thread t adds columns (c * 256 + t) * 8 + e, then wave shuffles and the 4
  // waves in order), so the scaled rows equal fused_add_rmsnorm's bit for bit
  // where that kernel takes its vector path.
  __shared__ float norm_red[8][4];
  float rrms[M];
  if (p.nw != nullptr) {
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      ss[m] = 0.f;
      if (m < p.M) {
        const T* xr = (const T*)p.x + (int64_t)m * p.sx;
        const T* rr = p.nr != nullptr ? (const T*)p.nr + (int64_t)m * p.snr : nullptr;
        T* hr = (p.nh != nullptr && blockIdx.x == 0 && blockIdx.y == 0) ? (T*)p.nh + (int64_t)m * p.snh : nullptr;
        for (int col = tid * 8; col < p.K; col += 256 * 8) {
          typename VecT<T>::x8 v = *(const typename VecT<T>::x8*)(xr + col);
          if (rr != nullptr) {
            const typename VecT<T>::x8 rv = *(const typename VecT<T>::x8*)(rr + col);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (T)((float)v[e] + (float)rv[e]);
          }
          if (hr != nullptr) *(typename VecT<T>::x8*)(hr + col) = v;
#pragma unroll
          for (int e = 0; e < 8; ++e) ss[m] = fmaf((float)v[e], (float)v[e], ss[m]);
        }
      }
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) ss[m] += __shfl_xor(ss[m], sh);
      if ((tid & 63) == 0) norm_red[m][tid >> 6] = ss[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) t += norm_red[m][w];
      rrms[m] = 1.f / sqrtf(t / (float)p.K + p.eps);
    }
  }

  // x's K-range as (x[k], x[k + 8]) pairs in the input dtype; rows past the
  // range and rows past p.M are zero.
  uint32_t* xs = (uint32_t*)gemv_smem;
  const int pslots = gemv_pair_slots(p.kc);
  auto x_at = [&](int m, int k) -> T {
    if (k >= k_len) return (T)0.f;
    if (p.nw != nullptr) {
      const int kk = k_begin + k;
      T h = ((const T*)p.x)[(int64_t)m * p.sx + kk];
      if (p.nr != nullptr) h = (T)((float)h + (float)((const T*)p.nr)[(int64_t)m * p.snr + kk]);
      float r = 0.f;
#pragma unroll
      for (int i = 0; i < M; ++i) r = i == m ? rrms[i] : r;  // no dynamic register indexing
      return (T)((float)h * r * (float)((const T*)p.nw)[kk]);
    }
    if (p.xg == nullptr) return ((const T*)p.x)[(int64_t)m * p.sx + k_begin + k];
    // SwiGLU input: silu(gate) rounded to T, times x rounded to T (the two
    // roundings of F.silu(gate) * up on bf16/fp16 tensors).
    const float g = (float)((const T*)p.xg)[(int64_t)m * p.sxg + k_begin + k];
    const float act = (float)(T)(g / (1.0f + expf(-g)));
    return (T)(act * (float)((const T*)p.x)[(int64_t)m * p.sx + k_begin + k]);
  };
  const int npairs = gemv_pair_slots(k_len);
  for (int idx = tid; idx < M * npairs; idx += 256) {
    const int m = idx / npairs, q = idx - m * npairs;
    const int k0 = (q >> 3) * 16 + (q & 7);
    xs[m * pslots + q] = m < p.M ? gemv_pack<T>(x_at(m, k0), x_at(m, k0 + 8)) : 0u;
  }
  __syncthreads();

  float acc[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;

  // Rows k (raw0) and k + 8 (raw1) of this thread's 8 columns, k % 16 < 8.
  auto dot_rows = [&](const u32x4 raw0, const u32x4 raw1, int k) {
    const int q = (k >> 4) * 8 + (k & 7);
    uint32_t xv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) xv[m] = xs[m * pslots + q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = __builtin_amdgcn_perm(raw1[e], raw0[e], 0x05040100u);  // column 2e of both rows
      const uint32_t hi = __builtin_amdgcn_perm(raw1[e], raw0[e], 0x07060302u);  // column 2e + 1
#pragma unroll
      for (int m = 0; m < M; ++m) {
        acc[m][2 * e] = gemv_dot2(lo, xv[m], acc[m][2 * e], (T*)nullptr);
        acc[m][2 * e + 1] = gemv_dot2(hi, xv[m], acc[m][2 * e + 1], (T*)nullptr);
      }
    }
  };
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  int k = kg;
  for (int b = 0; b < full; ++b) {
    if (b > 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = __builtin_nontemporal_load((const u32x4*)(wp + u * step));
      wp += 8 * step;
      __builtin_amdgcn_sched_barrier(0);  // all eight loads issue before the first use
    }
#pragma unroll
    for (int u = 0; u < 8; u += 2) dot_rows(cur[u], cur[u + 1], k + u * kGemvKG);
    k += 8 * kGemvKG;
  }
  if (rem >= 4) {
    u32x4 r4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) r4[u] = __builtin_nontemporal_load((const u32x4*)(wp + u * step));
    __builtin_amdgcn_sched_barrier(0);
    wp += 4 * step;
    dot_rows(r4[0], r4[1], k);
    dot_rows(r4[2], r4[3], k + 2 * kGemvKG);
    k += 4 * kGemvKG;
  }
  if ((rem & 3) >= 2) {
    const u32x4 r0 = __builtin_nontemporal_load((const u32x4*)wp);
    const u32x4 r1 = __builtin_nontemporal_load((const u32x4*)(wp + step));
    wp += 2 * step;
    dot_rows(r0, r1, k);
    k += 2 * kGemvKG;
  }
  if (rem & 1) dot_rows(__builtin_nontemporal_load((const u32x4*)wp), zero4, k);  // row k + 8 is past the range

  // Sum the K-groups: red[kg][m][column] over the x chunk.
  __syncthreads();  // every thread is done with xs
  float* red = gemv_smem;
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(kg * M + m) * kGemvCols + cg * 8 + e] = acc[m][e];
  __syncthreads();
  const int n = blockIdx.x * kGemvCols + tid;
  const bool col_ok = n < p.N;
  float sum[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    sum[m] = 0.f;
#pragma unroll
    for (int g = 0; g < kGemvKG; ++g) sum[m] += red[(g * M + m) * kGemvCols + tid];
  }

  if (p.splits == 1) {
    if (col_ok) {
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (m < p.M) *gemv_out<T>(p, n, m) = (T)sum[m];
    }
    return;
  }

  if (col_ok) {
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (m < p.M)
        __hip_atomic_store(p.partial + ((int64_t)split * p.M + m) * p.N + n, sum[m], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  // Handoff to the workgroup that arrives last, built on gfx950's device
  // coherence rather than on release/acquire fences: the partials are
  // agent-scope atomic stores (write-through to the device-coherent level,
  // sc1), every wave waits for their completion (vmcnt(0)) before the
  // barrier and thread 0's agent-scope counter RMWs, and the last workgroup
  // reads them with agent-scope atomic loads (sc1: never a stale line of its
  // own XCD's L2) issued only after its RMW has returned. Release/acquire
  // fences at agent scope would be the HIP memory model's way; they lower to
  // a whole-L2 write-back (buffer_wbl2 sc1) per arrival and an invalidate
  // (buffer_inv sc1) per acquire, and measured 1.4-1.9x slower on the
  // LM-head product (6.7 -> 3.6-4.8 TB/s), more on the narrow decode
  // projections whose ~1000 workgroups each would pay a write-back.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partials have reached device scope
  __syncthreads();
  if (tid == 0) {
    int* ctr = p.counters + blockIdx.x * kGemvCounterSlots;
    const int group = split & 7;
    const int group_size = (p.splits - group + 7) >> 3;
    const int groups = min(p.splits, 8);
    bool last = false;
    if (__hip_atomic_fetch_add(ctr + group, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == group_size - 1) {
      __hip_atomic_store(ctr + group, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = __hip_atomic_fetch_add(ctr + 8, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1;
      if (last) __hip_atomic_store(ctr + 8, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    last_arrival = last;
  }
  __syncthreads();
  if (!last_arrival) return;
  // The last workgroup sums the splits with the same (cg, kg) split of the
  // work as the pass: thread (cg, kg) adds 8 columns of splits kg, kg + 8, ...
  // (independent 8-byte loads, many in flight), then the K-groups are added
  // through LDS in a fixed order.
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;
  if (n0 < p.N) {
    const int64_t sstride = (int64_t)p.M * p.N;
    constexpr int SB = M >= 8 ? 1 : 8 / M;  // splits per batch: 32 loads in flight
    for (int s0 = kg; s0 < p.splits; s0 += SB * kGemvKG) {
      u64x2x2 v[SB][M];
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        const int s2 = s0 + b * kGemvKG;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          uint64_t* src = (uint64_t*)(p.partial + s2 * sstride + (int64_t)m * p.N + n0);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[b][m][q] = (s2 < p.splits && m < p.M)
                             ? __hip_atomic_load(src + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < SB; ++b)
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[m][2 * q] += __uint_as_float((uint32_t)v[b][m][q]);
            acc[m][2 * q + 1] += __uint_as_float((uint32_t)(v[b][m][q] >> 32));
          }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(kg * M + m) * kGemvCols + cg * 8 + e] = acc[m][e];
  __syncthreads();
  if (col_ok) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m < p.M) {
        float t = 0.f;
#pragma unroll
        for (int g = 0; g < kGemvKG; ++g) t += red[(g * M + m) * kGemvCols + tid];
        *gemv_out<T>(p, n, m) = (T)t;
      }
    }
  }
}

template <typename T, int M>
static hipError_t launch_gemv_m(const GemvParams& p, hipStream_t s) {
  const size_t xs_bytes = (size_t)M * gemv_pair_slots(p.kc) * 4;
  const size_t red_bytes = (size_t)kGemvKG * M * kGemvCols * 4;
  const size_t lds = xs_bytes > red_bytes ? xs_bytes : red_bytes;
  const dim3 grid((unsigned)((p.N + kGemvCols - 1) / kGemvCols), (unsigned)p.splits);
  hipLaunchKernelGGL((fa_gemv_kernel<T, M>), grid, dim3(256), lds, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_gemv(const GemvParams& p, hipStream_t s) {
  switch (p.M) {
    case 1: return launch_gemv_m<T, 1>(p, s);
    case 2: return launch_gemv_m<T, 2>(p, s);
    case 3:
    case 4: return launch_gemv_m<T, 4>(p, s);
    default: return launch_gemv_m<T, 8>(p, s);
  }
}

// Row capacity of the kernel that serves m rows (3 and 5..7 run the next one up).
int gemv_capacity(int m) { return m <= 2 ? m : (m <= 4 ? 4 : 8); }

// Host entry used by the C ABI layer (arguments validated, the split chosen
// so that kc * capacity * 4 bytes of x fit in 32 KB of LDS).
hipError_t gemv(const GemvParams& p, bool is_bf16, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  return is_bf16 ? launch_gemv<__bf16>(p, s) : launch_gemv<_Float16>(p, s);
}

}  // namespace lsfa
