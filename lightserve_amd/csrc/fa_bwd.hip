// FlashAttention backward for gfx950 (bf16/fp16 operands, fp32 accumulate).
//
// Math (kernels/flash_attention_backward.py:290-330): with the saved
// L = m + ln(l), P = exp(S*scale - L) is recomputed exactly; then
//   delta_i = rowsum(dO_i * O_i)                       (:211-229)
//   dV += P^T dO      (P rounded to the input dtype, :316)
//   dP  = dO V^T
//   dS  = P * (dP - delta)  (rounded to the input dtype, :319)
//   dK += dS^T Q * scale,   dQ += dS K * scale.
//
// Unlike the reference (one key-stationary kernel with fp32 atomic adds into
// a dq workspace, :323-325, followed by a cast, :382), the work is split into
//   fa_bwd_dq_kernel   : query-stationary; computes delta for its rows, then
//                        dQ = scale * dS K over all visible key tiles, stored
//                        straight in the input dtype;
//   fa_bwd_dkdv_kernel : key-stationary; dK, dV over all visible query tiles.
// Both recompute S and dP. There are no atomics and no fp32 dq buffer, so the
// result is deterministic; the dq kernel must run first (it writes delta).
#include "fa_common.hpp"

namespace lsfa {

constexpr float kLog2eB = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// dQ (and delta). Workgroup = 4 waves x 32 query rows, at most 256 registers
// per wave so two workgroups share a CU. K/V tiles of 64 keys go global ->
// LDS with buffer_load ... lds (double-buffered, zero past the sequence end).
// Per key tile and wave:
//   S^T  = K Q^T          A = K rows (LDS),  B = Q^T  (registers)
//   dP^T = V dO^T         A = V rows (LDS),  B = dO^T (registers)
//   dS^T = P^T (dP^T - delta)  -> rounded into B operands
//   dQ^T += K^T dS^T      A = K^T via transpose reads of the same LDS tile
// ---------------------------------------------------------------------------
template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fa_bwd_dq_kernel(const BwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int NW = 4, BM = NW * 32, BN = 64;
  constexpr int TILE = BN * DP;
  constexpr int LDI = TILE * 2 / 1024 / NW;
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int KB = BN / 32;
  static_assert(LDI >= 1, "tile too small for the workgroup");

  __shared__ __attribute__((aligned(1024))) T smem_raw[4 * TILE];  // K0 K1 V0 V1
  LDS_AS char* sm = (LDS_AS char*)smem_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31, hh = lane >> 5;
  int bh, qt;
  map_tile(p.num_tiles, gridDim.x, bh, qt, CAUSAL);
  const int b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D;
  const int q0 = qt * BM;
  const int off = nk - nq;

  const T* Q = (const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const T* K = (const T*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const T* V = (const T*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const T* Og = (const T*)p.o + (int64_t)b * p.sob + (int64_t)h * p.soh;
  const T* dO = (const T*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  T* dQ = (T*)p.dq + (int64_t)b * p.sdqb + (int64_t)h * p.sdqh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  float* Dg = p.delta + (int64_t)b * p.slb + (int64_t)h * p.slh;

  const int qw_lo = q0 + wave * 32;
  const int qrow = qw_lo + l32;
  const bool qvalid = qrow < nq;

  X8 qreg[KSTEPS], doreg[KSTEPS];
  float dpart = 0.f;
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    u32x4 rq = {0, 0, 0, 0}, rd = {0, 0, 0, 0}, ro = {0, 0, 0, 0};
    if (qvalid && col < D) {
      rq = ldg16(Q + (int64_t)qrow * p.sqn + col);
      rd = ldg16(dO + (int64_t)qrow * p.sdon + col);
      ro = ldg16(Og + (int64_t)qrow * p.son + col);
    }
    qreg[kk] = __builtin_bit_cast(X8, rq);
    doreg[kk] = __builtin_bit_cast(X8, rd);
    const X8 ov = __builtin_bit_cast(X8, ro);
#pragma unroll
    for (int s = 0; s < 8; ++s) dpart += (float)doreg[kk][s] * (float)ov[s];
  }
  const float delta = half_sum(dpart);
  float lrow = qvalid ? Lg[(int64_t)qrow * p.sln] : INFINITY;
  if (lrow == -INFINITY) lrow = INFINITY;  // row saw no key: P == 0
  const float l2 = lrow * kLog2eB;
  if (qvalid && hh == 0) Dg[(int64_t)qrow * p.sln] = delta;

  int kv_end = nk;
  if (CAUSAL) kv_end = min(nk, q0 + BM + off);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  // Direct tile loads: lane t of chunk c fills LDS bytes [16t, 16t+16) of
  // that chunk, i.e. stored segment (byte % 2DP)/16 of a tile row, which holds
  // logical segment stored ^ seg_swz(row). The buffer descriptor is rebuilt
  // per tile (scalar work) and clipped to the rows that exist, so the
  // per-lane byte offsets are loop-invariant and rows past nk read as zero.
  int kvo[LDI], vvo[LDI];
#pragma unroll
  for (int c = 0; c < LDI; ++c) {
    const int byte = (wave * LDI + c) * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    kvo[c] = (int)(row * p.skn * 2) + seg * 16;
    vvo[c] = (int)(row * p.svn * 2) + seg * 16;
  }
  auto tile_load = [&](const T* base, int64_t sn, const int* vo, int j, int buf) {
    const int rows = min(nk - j * BN, BN);
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(base + (int64_t)j * BN * sn, (int)(rows * sn * 2));
    LDS_AS char* dst = sm + buf * TILE * 2;
#pragma unroll
    for (int c = 0; c < LDI; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(dst + (wave * LDI + c) * 1024), 16, vo[c], 0, 0, 0);
  };

  int koff[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) koff[kk] = swz_off<DP>(l32, 16 * kk + 8 * hh) * 2;
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int troff[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    troff[dt][0] = swz_off<DP>(tr_row, 32 * dt + tr_col) * 2;
    troff[dt][1] = swz_off<DP>(tr_row + 8, 32 * dt + tr_col) * 2;
  }

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  const float sl2 = p.scale_log2;

  if (ntiles > 0) {
    tile_load(K, p.skn, kvo, 0, 0);
    tile_load(V, p.svn, vvo, 0, 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    if (j + 1 < ntiles) {
      tile_load(K, p.skn, kvo, j + 1, (j + 1) & 1);
      tile_load(V, p.svn, vvo, j + 1, 2 + ((j + 1) & 1));
    }
    const int kbase = j * BN;
    const bool active = !CAUSAL || (kbase <= qw_lo + 31 + off);
    if (active) {
      const LDS_AS char* Ks = sm + (j & 1) * TILE * 2;
      const LDS_AS char* Vs = sm + (2 + (j & 1)) * TILE * 2;
      f32x16 s[KB], dp[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s[kb] = f32x16{};
        dp[kb] = f32x16{};
      }
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int o = kb * 32 * DP * 2 + koff[kk];
          s[kb] = mfma32(*(const LDS_AS X8*)(Ks + o), qreg[kk], s[kb]);
          dp[kb] = mfma32(*(const LDS_AS X8*)(Vs + o), doreg[kk], dp[kb]);
        }
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = fast_exp2(fmaf(s[kb][i], sl2, -l2));
          s[kb][i] = pv * (dp[kb][i] - delta);
        }
      if (CAUSAL && kbase + BN - 1 > qw_lo + off) {  // tile crosses the diagonal
        const int lim = qrow + off - kbase - 4 * hh;  // masked if 32kb + 8(i/4) + i%4 > lim
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kb][i] = (32 * kb + 8 * (i >> 2) + (i & 3) > lim) ? 0.f : s[kb][i];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int ks = 0; ks < 2 * KB; ++ks) {
          const LDS_AS char* base = Ks + ks * 16 * DP * 2;
          const X8 a = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(base + troff[dt][0])),
                                    lds_read_tr((const LDS_AS T*)(base + troff[dt][1])));
          acc[dt] = mfma32(a, pack8<T>(s[ks >> 1], 8 * (ks & 1)), acc[dt]);
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  if (qvalid) {
    T* row = dQ + (int64_t)qrow * p.sdqn;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
        if (d < D) {
          X4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)(acc[dt][4 * g + e] * sc);
          *(X4*)(row + d) = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dK, dV. Workgroup = 8 waves (two per SIMD, at most 256 registers each)
// over 128 keys. K and V of those keys stay in LDS for the whole kernel.
// Query tiles of 64 rows are staged in LDS twice: row-major (A operand of
// S = Q K^T and dP = dO V^T) and transposed with the row order permuted so
// that each MFMA operand of dV^T += dO^T P and dK^T += Q^T dS is a single
// ds_read_b128 (no transpose reads in the loop). Wave w owns keys
// 32*(w%4)..+31 and query rows 32*(w/4)..+31 of every tile:
//   S  = Q K^T            A = Q rows (LDS),   B = K rows (LDS)
//   dP = dO V^T           A = dO rows (LDS),  B = V rows (LDS)
//   P  = exp2(S*scale*log2e - L*log2e), dS = P (dP - delta)
//   dV^T += dO^T P        A = dO^T (LDS),     B = P  (registers)
//   dK^T += Q^T dS        A = Q^T (LDS),      B = dS (registers)
// The two query halves' partial dK/dV are summed through LDS at the end.
// Query rows beyond the sequence get L = +inf, so their P is exactly 0.
// ---------------------------------------------------------------------------

// Position of tile-local query q (0..63) in a transposed tile row: bits 2
// and 3 swap, so that the 8 queries one lane half feeds to a 32x32x16 MFMA
// (16*kk + 8*(s/4) + 4*h + s%4, s = 0..7) sit in 16 contiguous bytes.
__device__ __forceinline__ int tpos(int q) { return (q & ~12) | ((q & 4) << 1) | ((q & 8) >> 1); }
// Byte offset of (row d, position pos) in a transposed [DP][64] tile; the
// 16-byte column is XOR-swizzled with (d/2)%8 so 16 consecutive rows read
// at one column hit distinct banks.
__device__ __forceinline__ int toff(int d, int pos) { return d * 128 + ((((pos >> 3) ^ ((d >> 1) & 7))) << 4) + (pos & 7) * 2; }

template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fa_bwd_dkdv_kernel(const BwdParams p) {
  using X8 = typename VecT<T>::x8;
  constexpr int NW = 8, BNK = 128, BMQ = 64;
  constexpr int SEGS = DP / 8;
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int KV_BYTES = BNK * DP * 2;               // one of K or V
  constexpr int QT_BYTES = BMQ * DP * 2;               // one Q-side tile (any layout)
  constexpr int UNITS = (BMQ / 4) * SEGS;              // 4-row x 8-column units per tensor
  constexpr int LDI = KV_BYTES / 1024 / NW;            // direct 1 KB loads per wave for K or V
  static_assert(LDI >= 1 && UNITS <= 256, "tile shape");
  // LDS: K | V | Qr | dOr | Qt | dOt | L | delta
  constexpr int OFF_K = 0, OFF_V = KV_BYTES, OFF_QR = 2 * KV_BYTES, OFF_OR = OFF_QR + QT_BYTES;
  constexpr int OFF_QT = OFF_OR + QT_BYTES, OFF_OT = OFF_QT + QT_BYTES, OFF_L = OFF_OT + QT_BYTES;
  constexpr int LDS_BYTES = OFF_L + 2 * BMQ * 4;
  __shared__ __attribute__((aligned(1024))) char smem_raw[LDS_BYTES];
  LDS_AS char* sm = (LDS_AS char*)smem_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int kbw = wave & 3, qh = wave >> 2;  // key block and query half of this wave
  int bh, kt;
  map_tile(p.num_tiles, gridDim.x, bh, kt, false);
  const int b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D;
  const int k0 = kt * BNK;
  const int off = nk - nq;

  const T* Q = (const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const T* K = (const T*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh + (int64_t)k0 * p.skn;
  const T* V = (const T*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh + (int64_t)k0 * p.svn;
  const T* dO = (const T*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  T* dK = (T*)p.dk + (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
  T* dV = (T*)p.dv + (int64_t)b * p.sdvb + (int64_t)h * p.sdvh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float* Dg = p.delta + (int64_t)b * p.slb + (int64_t)h * p.slh;

  // K and V of the 128 keys: direct loads, zero past the sequence end.
  {
    const int kn = max(0, min(BNK, nk - k0));
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void*)K, (short)0, (int)((int64_t)kn * p.skn * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)V, (short)0, (int)((int64_t)kn * p.svn * 2), 0x00020000);
#pragma unroll
    for (int c = 0; c < LDI; ++c) {
      const int byte = (wave * LDI + c) * 1024 + lane * 16;
      const int row = byte / (DP * 2);
      const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (LDS_AS void*)(sm + OFF_K + (wave * LDI + c) * 1024), 16,
                                               (int)(((int64_t)row * p.skn + seg * 8) * 2), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (LDS_AS void*)(sm + OFF_V + (wave * LDI + c) * 1024), 16,
                                               (int)(((int64_t)row * p.svn + seg * 8) * 2), 0, 0, 0);
    }
  }

  // Query range that can see this key tile.
  int q_lo = 0;
  if (CAUSAL) q_lo = max(0, k0 - off);
  q_lo = (q_lo / BMQ) * BMQ;
  const int ntiles = (nq > q_lo) ? (nq - q_lo + BMQ - 1) / BMQ : 0;

  // Staging: thread t < 2*UNITS loads one 4-row x 8-column unit of Q (t <
  // UNITS) or dO; threads 0..15 also load 4 values of L, threads 16..31 of
  // delta.
  const bool is_do = tid >= UNITS;
  const int u = is_do ? tid - UNITS : tid;
  const bool stager = tid < 2 * UNITS;
  const int g4 = u % (BMQ / 4), dseg = u / (BMQ / 4);
  const T* src = is_do ? dO : Q;
  const int64_t sstride = is_do ? p.sdon : p.sqn;
  u32x4 st[4];
  f32x4 lst = {0.f, 0.f, 0.f, 0.f};
  const int lrow = tid;  // 0..15: L, 16..31: delta
  auto gload = [&](int t) {
    const int qs = q_lo + t * BMQ;
    if (stager) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = qs + 4 * g4 + r;
        st[r] = (q < nq && dseg * 8 < D) ? ldg16(src + (int64_t)q * sstride + dseg * 8) : u32x4{0, 0, 0, 0};
      }
    }
    if (lrow < 32) {
      const int base = qs + 4 * (lrow & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = base + e;
        if (lrow < 16) {
          float lv = q < nq ? Lg[(int64_t)q * p.sln] : INFINITY;
          if (lv == -INFINITY) lv = INFINITY;  // row saw no key: P == 0
          lst[e] = lv * 1.4426950408889634f;
        } else {
          lst[e] = q < nq ? Dg[(int64_t)q * p.sln] : 0.f;
        }
      }
    }
  };
  auto sstore = [&]() {
    if (stager) {
      const int qr = is_do ? OFF_OR : OFF_QR;
      const int qt = is_do ? OFF_OT : OFF_QT;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *(LDS_AS u32x4*)(sm + qr + swz_off<DP>(4 * g4 + r, dseg * 8) * 2) = st[r];
      // Transposed: row d = 8*dseg + i holds the 4 queries' values of column i.
      const int pos = tpos(4 * g4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int w = i >> 1, sh = (i & 1) * 16;
        const uint32_t lo = ((st[0][w] >> sh) & 0xffffu) | (((st[1][w] >> sh) & 0xffffu) << 16);
        const uint32_t hi = ((st[2][w] >> sh) & 0xffffu) | (((st[3][w] >> sh) & 0xffffu) << 16);
        *(LDS_AS u32x2*)(sm + qt + toff(dseg * 8 + i, pos)) = u32x2{lo, hi};
      }
    }
    if (lrow < 32) {
      *(LDS_AS f32x4*)(sm + OFF_L + lrow * 16) = lst;
    }
  };

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  const float sl2 = p.scale_log2;
  const int krow = k0 + 32 * kbw + l32;  // key owned by this lane (C-layout column)
  int aoff[KSTEPS];                      // Q/dO rows (A) and K/V rows (B): same swizzle
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) aoff[kk] = swz_off<DP>(l32, 16 * kk + 8 * hh) * 2;
  int toffs[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int kk2 = 0; kk2 < 2; ++kk2) toffs[dt][kk2] = toff(32 * dt + l32, 32 * qh + 16 * kk2 + 8 * hh);

  if (ntiles > 0) gload(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();  // previous tile fully consumed (and K/V resident on t = 0)
    sstore();
    if (t == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 1 < ntiles) gload(t + 1);
    const int qs = q_lo + t * BMQ;
    const int qw = qs + 32 * qh;          // first query row of this wave
    const int kw = k0 + 32 * kbw;         // first key of this wave
    // Tiles where every key of the wave lies after every query row are not
    // skipped: the causal mask zeroes their P and dS (they only occur among
    // the first tiles of the sweep), which keeps the loop body branch-free
    // apart from the mask itself.
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const X8 aq = *(const LDS_AS X8*)(sm + OFF_QR + 32 * qh * DP * 2 + aoff[kk]);
      const X8 ao = *(const LDS_AS X8*)(sm + OFF_OR + 32 * qh * DP * 2 + aoff[kk]);
      const X8 bk = *(const LDS_AS X8*)(sm + OFF_K + 32 * kbw * DP * 2 + aoff[kk]);
      const X8 bv = *(const LDS_AS X8*)(sm + OFF_V + 32 * kbw * DP * 2 + aoff[kk]);
      s = mfma32(aq, bk, s);
      dp = mfma32(ao, bv, dp);
    }
    // Register 4g+e holds query qw + 8g + 4hh + e of this lane's key.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int qi = 32 * qh + 8 * g + 4 * hh;
      const f32x4 lv = *(const LDS_AS f32x4*)(sm + OFF_L + qi * 4);
      const f32x4 dl = *(const LDS_AS f32x4*)(sm + OFF_L + BMQ * 4 + qi * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pv = fast_exp2(fmaf(s[4 * g + e], sl2, -lv[e]));
        s[4 * g + e] = pv;
        dp[4 * g + e] = pv * (dp[4 * g + e] - dl[e]);
      }
    }
    if (CAUSAL && qw + off < kw + 31) {  // tile crosses the diagonal: drop keys after the query
      const int lim = krow - off - qw - 4 * hh;  // masked if 8(i/4) + i%4 < lim
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool m = 8 * (i >> 2) + (i & 3) < lim;
        s[i] = m ? 0.f : s[i];
        dp[i] = m ? 0.f : dp[i];
      }
    }
    const X8 pb0 = pack8<T>(s, 0), pb1 = pack8<T>(s, 8);
    const X8 db0 = pack8<T>(dp, 0), db1 = pack8<T>(dp, 8);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const X8 ao0 = *(const LDS_AS X8*)(sm + OFF_OT + toffs[dt][0]);
      const X8 ao1 = *(const LDS_AS X8*)(sm + OFF_OT + toffs[dt][1]);
      const X8 aq0 = *(const LDS_AS X8*)(sm + OFF_QT + toffs[dt][0]);
      const X8 aq1 = *(const LDS_AS X8*)(sm + OFF_QT + toffs[dt][1]);
      dv[dt] = mfma32(ao0, pb0, dv[dt]);
      dk[dt] = mfma32(aq0, db0, dk[dt]);
      dv[dt] = mfma32(ao1, pb1, dv[dt]);
      dk[dt] = mfma32(aq1, db1, dk[dt]);
    }
  }

  // Sum the two query halves: waves 4..7 park their partials in LDS (over
  // K/V, whose direct loads must have landed even if no tile ran).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  LDS_AS f32x4* park = (LDS_AS f32x4*)sm;  // (4 waves) x (2*DT*4) x 64 lanes x 16 B <= 128 KB
  if (qh == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        park[((kbw * 2 * DT + dt) * 4 + g) * 64 + lane] = f32x4{dk[dt][4 * g], dk[dt][4 * g + 1], dk[dt][4 * g + 2], dk[dt][4 * g + 3]};
        park[(((kbw * 2 + 1) * DT + dt) * 4 + g) * 64 + lane] = f32x4{dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3]};
      }
  }
  __syncthreads();
  if (qh == 0 && krow < nk) {
    T* rk = dK + (int64_t)krow * p.sdkn;
    T* rv = dV + (int64_t)krow * p.sdvn;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 ok = park[((kbw * 2 * DT + dt) * 4 + g) * 64 + lane];
        const f32x4 ov = park[(((kbw * 2 + 1) * DT + dt) * 4 + g) * 64 + lane];
        const int d = 32 * dt + 8 * g + 4 * hh;
        if (d < D) {
          typename VecT<T>::x4 a, c;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[e] = (T)((dk[dt][4 * g + e] + ok[e]) * sc);
            c[e] = (T)(dv[dt][4 * g + e] + ov[e]);
          }
          *(typename VecT<T>::x4*)(rk + d) = a;
          *(typename VecT<T>::x4*)(rv + d) = c;
        }
      }
    }
  }
}

template <typename T, int DP, bool CAUSAL>
static hipError_t launch_bwd(BwdParams p, hipStream_t s) {
  // An empty axis means an empty grid: that kernel has nothing to write.
  p.num_tiles = (p.Nq + 127) / 128;
  if (p.num_tiles > 0) {
    hipLaunchKernelGGL((fa_bwd_dq_kernel<T, DP, CAUSAL>), dim3(p.num_tiles * p.B * p.H), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  p.num_tiles = (p.Nk + 127) / 128;
  if (p.num_tiles > 0) {
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<T, DP, CAUSAL>), dim3(p.num_tiles * p.B * p.H), dim3(512), 0, s, p);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <typename T>
static hipError_t dispatch_bwd_t(const BwdParams& p, int dp, bool causal, hipStream_t s) {
  switch (dp) {
    case 32: return causal ? launch_bwd<T, 32, true>(p, s) : launch_bwd<T, 32, false>(p, s);
    case 64: return causal ? launch_bwd<T, 64, true>(p, s) : launch_bwd<T, 64, false>(p, s);
    default: return causal ? launch_bwd<T, 128, true>(p, s) : launch_bwd<T, 128, false>(p, s);
  }
}

hipError_t bwd_mfma(const BwdParams& p, bool is_bf16, int dp, bool causal, hipStream_t s) {
  if (is_bf16) return dispatch_bwd_t<__bf16>(p, dp, causal, s);
  return dispatch_bwd_t<_Float16>(p, dp, causal, s);
}

}  // namespace lsfa
