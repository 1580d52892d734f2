// Skinny GEMM on MFMA for 3..32 rows: y[M, N] = x[M, K] @ W[K, N] (W in the
// model's [in, out] row-major layout, bf16/fp16, fp32 accumulate, one rounding),
// for the decode steps of a batch, where the VALU kernel (fa_gemv.hip) spends
// more time on its products than on the weight bytes.
//
// The product is computed transposed, y^T = W^T x^T, on v_mfma_f32_32x32x16:
// the A operand W^T [32 columns x 16 rows of K] comes from LDS through the
// transposing read (ds_read_b64_tr_b16) of W tiles stored row-major, exactly as
// the attention kernels read V^T; the B operand x^T [16 x 32 rows of x] (rows
// past M are zero) stays in registers for the whole K-range.
//   Grid (N / 128 column blocks, splits): a 4-wave workgroup owns 128 columns
//   (one 32-column block per wave) and a K-range of at most 256 rows, i.e. four
//   64 x 128 tiles (16 KB each) that go global -> LDS by direct loads
//   (buffer_load ... lds) into four separate buffers, all issued up front: the
//   workgroup keeps 64 KB in flight and no buffer is reused, so the loop needs
//   no barrier beyond one per tile for the other waves' parts. Tiles past the
//   K-range are issued with empty descriptors (they load zeros and cost no HBM
//   traffic), which keeps each wave's count of outstanding loads fixed.
//   With one split a wave rounds its 32 x M sums into y; otherwise the partial
//   sums, two-level arrival counters and last-workgroup reduction work as in
//   fa_gemv.hip (device-scope atomic stores and loads, no cache maintenance),
//   with the partials stored column-major, [split][column][row], so that the
//   32 lanes of each accumulator register (32 rows of one column) store
//   consecutive words and the last workgroup reads them back contiguously.
#include "fa_common.hpp"

namespace lsfa {

constexpr int kMfmaCols = 128;     // columns per workgroup (LDS tile width)
constexpr int kMfmaTileRows = 64;  // rows per LDS tile
constexpr int kMfmaTiles = 4;      // tiles per workgroup: K-range <= 256 rows
constexpr int kMfmaTileElems = kMfmaTileRows * kMfmaCols;
constexpr int kMfmaCounterSlots = 16;

template <typename T>
__global__ __launch_bounds__(256) void fa_gemv_mfma_kernel(const GemvParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int DP = kMfmaCols;
  extern __shared__ __attribute__((aligned(16))) char mfma_raw[];  // kMfmaTiles tiles
  T* mfma_smem = (T*)mfma_raw;
  __shared__ int last_arrival;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int split = blockIdx.y;
  const int k_begin = split * p.kc;
  const int k_len = max(0, min(p.K, k_begin + p.kc) - k_begin);

  // Matrix of this column block (every matrix's width is a multiple of 128).
  const int n_blk = blockIdx.x * kMfmaCols;  // virtual column
  const int g = (n_blk >= p.col_off[1]) + (n_blk >= p.col_off[2]) + (n_blk >= p.col_off[3]);
  const int col_off = g == 0 ? p.col_off[0] : (g == 1 ? p.col_off[1] : (g == 2 ? p.col_off[2] : p.col_off[3]));
  const T* w = (const T*)(g == 0 ? p.w[0] : (g == 1 ? p.w[1] : (g == 2 ? p.w[2] : p.w[3])));
  T* y = (T*)(g == 0 ? p.y[0] : (g == 1 ? p.y[1] : (g == 2 ? p.y[2] : p.y[3])));
  const int64_t sw = g == 0 ? p.sw[0] : (g == 1 ? p.sw[1] : (g == 2 ? p.sw[2] : p.sw[3]));
  const int64_t sy = g == 0 ? p.sy[0] : (g == 1 ? p.sy[1] : (g == 2 ? p.sy[2] : p.sy[3]));
  const int n_local = n_blk - col_off;

  // x^T as the B operand for every 16-row step of the K-range. The
  // transposed read below gives the A operand its 16 rows in the order
  // 4hh + (0..3), 8 + 4hh + (0..3) (slot s <-> row 8(s/4) + 4hh + s%4), so B
  // takes the same order: lane holds x[l32][16 step + 4hh .. + 3] and
  // x[l32][16 step + 8 + 4hh .. + 3]. Rows past M and columns past the range
  // are zero (the loads are clamped in bounds, then masked).
  // With a gate the operand is bf16(bf16(silu(gate)) * x), the two roundings
  // of F.silu(gate) * up.
  X8 xop[kMfmaTiles * 4];
  {
    const int m = min(l32, p.M - 1);
    const T* xr = (const T*)p.x + (int64_t)m * p.sx + k_begin;
    const T* gr = p.xg != nullptr ? (const T*)p.xg + (int64_t)m * p.sxg + k_begin : nullptr;
    auto load4 = [&](int k) -> u32x2 {
      u32x2 v = *(const u32x2*)(xr + k);
      if (gr != nullptr) {
        const X4 up = __builtin_bit_cast(X4, v);
        const X4 gt = __builtin_bit_cast(X4, *(const u32x2*)(gr + k));
        X4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gv = (float)gt[e];
          const float act = (float)(T)(gv / (1.0f + expf(-gv)));
          o[e] = (T)(act * (float)up[e]);
        }
        v = __builtin_bit_cast(u32x2, o);
      }
      return v;
    };
#pragma unroll
    for (int st = 0; st < kMfmaTiles * 4; ++st) {
      const int k0 = 16 * st + 4 * hh, k1 = k0 + 8;
      // An empty K-range (k = 0, or a split past the end) loads nothing: the
      // clamped index would fall before the row (uniform branch).
      u32x2 lo = u32x2{0u, 0u}, hi = u32x2{0u, 0u};
      if (k_len > 0) {
        lo = load4(min(k0, k_len - 4));
        hi = load4(min(k1, k_len - 4));
      }
      if (l32 >= p.M || k0 >= k_len) lo = u32x2{0u, 0u};
      if (l32 >= p.M || k1 >= k_len) hi = u32x2{0u, 0u};
      const u32x4 raw = {lo[0], lo[1], hi[0], hi[1]};
      xop[st] = __builtin_bit_cast(X8, raw);
    }
  }

  // Direct tile loads: wave w moves rows 16w .. 16w + 15 of each tile (four
  // 1 KB chunks); lane t of chunk c lands at tile byte (4w + c) * 1024 + 16t
  // = (row, swizzled 16-byte segment). Descriptors are clipped to the rows of
  // the K-range, so rows past it read as zero.
  int vo[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int byte = (wave * 4 + c) * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    vo[c] = (int)(row * sw * 2) + seg * 16;
  }
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    const int rows = min(k_len - t * kMfmaTileRows, kMfmaTileRows);
    const T* base = w + (int64_t)(k_begin + t * kMfmaTileRows) * sw + n_local;
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(rows > 0 ? base : w, rows > 0 ? (int)(rows * sw * 2) : 0);
    LDS_AS char* dst = (LDS_AS char*)(mfma_smem + t * kMfmaTileElems);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(dst + (wave * 4 + c) * 1024), 16, vo[c], 0, 0, 0);
  }

  // Transposed-read offsets of this wave's 32 columns (as the attention
  // kernels' V^T reads).
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int voff0 = swz_off<DP>(tr_row, 32 * wave + tr_col) * 2;
  const int voff1 = swz_off<DP>(tr_row + 8, 32 * wave + tr_col) * 2;

  f32x16 acc = f32x16{};
  const int ntiles = (k_len + kMfmaTileRows - 1) / kMfmaTileRows;
#pragma unroll
  for (int t = 0; t < kMfmaTiles; ++t) {
    // Each wave issued 4 loads per tile; tile t has landed once at most
    // 4 * (tiles after t) of them are outstanding.
    if (t == 0) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    if (t == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    if (t == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    if (t == 3) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // the other waves' rows of tile t have landed too
    if (t < ntiles) {
      const LDS_AS char* tile = (const LDS_AS char*)(mfma_smem + t * kMfmaTileElems);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const LDS_AS char* b = tile + ks * 16 * DP * 2;
        const X8 a = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(b + voff0)), lds_read_tr((const LDS_AS T*)(b + voff1)));
        acc = mfma32(a, xop[4 * t + ks], acc);
      }
    }
  }

  // acc: lane l, register i holds y^T[column 32w + 8(i/4) + 4hh + i%4][row l32].
  const int m = l32;
  if (p.splits == 1) {
    if (m < p.M) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int n = 32 * wave + 8 * (i >> 2) + 4 * hh + (i & 3);
        y[(int64_t)m * sy + n_local + n] = (T)acc[i];
      }
    }
    return;
  }
  if (m < p.M) {
    float* dst = p.partial + ((int64_t)split * p.N + n_blk) * p.M + m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int n = 32 * wave + 8 * (i >> 2) + 4 * hh + (i & 3);
      __hip_atomic_store(dst + (int64_t)n * p.M, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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
    int* ctr = p.counters + blockIdx.x * kMfmaCounterSlots;
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
  // The last workgroup: the block's 128 x M partials are contiguous per
  // split; thread tid sums elements tid, tid + 256, ... (element e is column
  // e / M, row e % M) over the splits in split order.
  const int64_t sstride = (int64_t)p.N * p.M;
  const float* base = p.partial + (int64_t)n_blk * p.M;
  for (int e = tid; e < kMfmaCols * p.M; e += 256) {
    float s = 0.f;
#pragma unroll 8
    for (int s2 = 0; s2 < p.splits; ++s2)
      s += __hip_atomic_load(base + s2 * sstride + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int c = e / p.M, mr = e - c * p.M;
    y[(int64_t)mr * sy + n_local + c] = (T)s;
  }
}

// Host entry used by the C ABI layer: arguments validated, every matrix's
// width a multiple of 128, kc a multiple of 64 of at most 256, 3 <= M <= 32.
hipError_t gemv_mfma(const GemvParams& p, bool is_bf16, hipStream_t s) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  const dim3 grid((unsigned)(p.N / kMfmaCols), (unsigned)p.splits);
  const size_t lds = (size_t)kMfmaTiles * kMfmaTileElems * 2;
  if (is_bf16)
    hipLaunchKernelGGL(fa_gemv_mfma_kernel<__bf16>, grid, dim3(256), lds, s, p);
  else
    hipLaunchKernelGGL(fa_gemv_mfma_kernel<_Float16>, grid, dim3(256), lds, s, p);
  return hipGetLastError();
}

}  // namespace lsfa
