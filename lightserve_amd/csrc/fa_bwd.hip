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
//   fa_bwd_dq_kernel   : query-stationary. Its prologue does the reference's
//                        preprocess (:341-350): delta and L*log2(e) per query
//                        row into the workspace. Then dQ = scale * dS K over
//                        all visible key tiles, stored straight in the input
//                        dtype;
//   fa_bwd_dkdv_kernel : key-stationary; dK, dV over all visible query tiles
//                        (runs after the dq kernel, which feeds it).
// Both kernels recompute S and dP. There are no atomics and no fp32 dq
// buffer, so results are deterministic.
#include "fa_common.hpp"

namespace lsfa {

constexpr float kLog2eB = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// dQ. Workgroup = 4 waves x 32 query rows, at most 256 registers
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

  const int qw_lo = q0 + wave * 32;
  const int qrow = qw_lo + l32;
  const bool qvalid = qrow < nq;

  // Lane byte offset of chunk lc of a row-major tile (rows of 2*DP bytes):
  // lane t fills LDS bytes [16t, 16t+16) of the chunk, i.e. stored segment
  // (byte % 2DP)/16 of a row, which holds logical segment stored ^
  // seg_swz(row). Logical columns at or past D get an offset past any
  // descriptor's end, so they read as zero.
  auto row_voff = [&](int lc, int64_t sn) -> int {
    const int byte = lc * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    return seg * 8 < D ? (int)(row * sn * 2) + seg * 16 : (int)0x80000000;
  };
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int troff[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    troff[dt][0] = swz_off<DP>(tr_row, 32 * dt + tr_col) * 2;
    troff[dt][1] = swz_off<DP>(tr_row + 8, 32 * dt + tr_col) * 2;
  }

  // Prologue (the backward's per-query-row pass): the tile's Q and dO rows
  // go to LDS (rows past nq and columns past D as zero), then
  //   - Q^T and dO^T B operands of this kernel come from LDS;
  //   - delta = rowsum(dO * O) and L*log2e are written to the workspace for
  //     the dK/dV kernel.
  constexpr int TB = BM * DP * 2;  // bytes of one 128-row tile
  static_assert(2 * TB <= 4 * TILE * 2, "Q/dO tiles must fit in the K/V buffers");
  {
    constexpr int CPW = 2 * TB / 1024 / NW;  // chunks per wave (waves 0..1: Q, 2..3: dO)
    const bool w_do = wave >= NW / 2;
    const int64_t sn = w_do ? p.sdon : p.sqn;
    const int rows = min(nq - q0, BM);
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc((w_do ? dO : Q) + (int64_t)q0 * sn, (int)(rows * sn * 2));
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = wave * CPW + i;
      const int vo = row_voff(c % (TB / 1024), sn);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(sm + c * 1024), 16, vo, 0, 0, 0);
    }
  }
  u32x4 oraw[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    oraw[kk] = u32x4{0, 0, 0, 0};
    if (qvalid && col < D) oraw[kk] = ldg16(Og + (int64_t)qrow * p.son + col);
  }
  float lraw = -INFINITY;
  if (qvalid) lraw = p.lse[(int64_t)b * p.slb + (int64_t)h * p.slh + (int64_t)qrow * p.sln];
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  X8 qreg[KSTEPS], doreg[KSTEPS];
  float dpart = 0.f;
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int o = swz_off<DP>(32 * wave + l32, 16 * kk + 8 * hh) * 2;
    qreg[kk] = *(const LDS_AS X8*)(sm + o);
    doreg[kk] = *(const LDS_AS X8*)(sm + TB + o);
    const X8 ov = __builtin_bit_cast(X8, oraw[kk]);
#pragma unroll
    for (int s = 0; s < 8; ++s) dpart += (float)doreg[kk][s] * (float)ov[s];
  }
  const float delta = half_sum(dpart);
  const float l2 = lraw == -INFINITY ? INFINITY : lraw * kLog2eB;  // no visible key / padding: P == 0
  if (hh == 0) {
    float2 v;
    v.x = l2;
    v.y = delta;
    *(float2*)(p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh + 2 * (int64_t)qrow) = v;
  }
  __syncthreads();  // the K/V tiles below reuse the Q/dO buffers

  int kv_end = nk;
  if (CAUSAL) kv_end = min(nk, q0 + BM + off);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  // Direct tile loads of K and V (see row_voff). The buffer descriptor is
  // rebuilt per tile (scalar work) and clipped to the rows that exist, so
  // the per-lane byte offsets are loop-invariant and rows past nk read as zero.
  int kvo[LDI], vvo[LDI];
#pragma unroll
  for (int c = 0; c < LDI; ++c) {
    kvo[c] = row_voff(wave * LDI + c, p.skn);
    vvo[c] = row_voff(wave * LDI + c, p.svn);
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
// over 128 keys; K and V of those keys stay in LDS for the whole kernel.
// Every operand reaches LDS with buffer_load ... lds (no register staging):
// per 64-query tile, the row-major Q/dO tile with L*log2e and delta, in two
// stages. Wave w owns keys 32*(w%4)..+31 and query rows 32*(w/4)..+31 of
// every tile:
//   S  = Q K^T            A = Q rows (LDS),   B = K rows (LDS)
//   dP = dO V^T           A = dO rows (LDS),  B = V rows (LDS)
//   P  = exp2(S*scale*log2e - L*log2e), dS = P (dP - delta)
//   dV^T += dO^T P        A = dO^T (transpose reads of the dO rows), B = P
//   dK^T += Q^T dS        A = Q^T (transpose reads of the Q rows),   B = dS
// The two waves of a SIMD (same keys, the two query halves) run half a tile
// apart (see the loop), so one's softmax VALU work overlaps the other's
// dV/dK MFMAs.
// The two query halves' partial dK/dV are summed through LDS at the end.
// Query rows beyond the sequence have L = +inf in the workspace (written by
// the dq kernel's prologue), so their P is exactly 0; head-dim columns at or
// past D load as zero.
// ---------------------------------------------------------------------------
template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fa_bwd_dkdv_kernel(const BwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int NW = 8, BNK = 128, BMQ = 64;
  constexpr int KSTEPS = DP / 16, DT = DP / 32;
  constexpr int KV_B = BNK * DP * 2;  // bytes of K (or V)
  constexpr int R_B = BMQ * DP * 2;   // bytes of a row-major Q (or dO) tile
  // Two row stages, each Q | dO | (L*log2e, delta) pairs, 1 KB aligned.
  constexpr int RS_B = 2 * R_B + 1024;
  constexpr int OFF_K = 0, OFF_V = KV_B, OFF_R = 2 * KV_B;
  constexpr int LDS_B = OFF_R + 2 * RS_B;
  constexpr int NG = 2 * DT * 4;  // f32x4 groups of dK^T and dV^T per lane
  static_assert((NW / 2) * NG * 64 * 16 <= LDS_B, "epilogue does not fit in LDS");
  constexpr int CKV = 2 * KV_B / 1024 / NW;  // 1 KB chunks per wave: K|V
  constexpr int CR = 2 * R_B / 1024 / NW;    //                        Q|dO rows
  static_assert(CKV >= 1 && CR >= 1, "tile too small for the workgroup");

  __shared__ __attribute__((aligned(1024))) char sm_raw[LDS_B];
  LDS_AS char* sm = (LDS_AS char*)sm_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31, hh = lane >> 5;
  const int kb = wave & 3, qh = wave >> 2;
  const bool w_hi = wave >= NW / 2;  // waves 4..7 load V and dO; 0..3 load K and Q
  int bh, kt;
  map_tile(p.num_tiles, gridDim.x, bh, kt, false);  // low key tiles see the most queries
  const int b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D;
  const int k0 = kt * BNK;
  const int off = nk - nq;

  const T* K = (const T*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh + (int64_t)k0 * p.skn;
  const T* V = (const T*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh + (int64_t)k0 * p.svn;
  const T* Q = (const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const T* dO = (const T*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  const float* LD = p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh;

  // Lane byte offset of row-major chunk lc (tile rows of 2*DP bytes): lane t
  // fills stored segment (byte % 2DP)/16, which holds logical segment
  // stored ^ seg_swz(row). Logical columns at or past D get an offset past
  // any descriptor's end, so they read as zero.
  auto row_voff = [&](int lc, int64_t sn) -> int {
    const int byte = lc * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    return seg * 8 < D ? (int)(row * sn * 2) + seg * 16 : (int)0x80000000;
  };

  // K and V of the 128 keys (rows past nk read as zero).
  {
    const int rows = max(0, min(BNK, nk - k0));
    const int64_t sn = w_hi ? p.svn : p.skn;
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(w_hi ? V : K, (int)(rows * sn * 2));
#pragma unroll
    for (int i = 0; i < CKV; ++i) {
      const int c = wave * CKV + i;  // chunk of the K|V region
      const int vo = row_voff(c % (KV_B / 1024), sn);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(sm + OFF_K + c * 1024), 16, vo, 0, 0, 0);
    }
  }

  int rvo[CR];
#pragma unroll
  for (int i = 0; i < CR; ++i) rvo[i] = row_voff((wave % (NW / 2)) * CR + i, w_hi ? p.sdon : p.sqn);

  // (Offset arrays go in as pointers and lambda results are hoisted into
  // locals: an array-reference lambda parameter, or a lambda call inside a
  // builtin's argument list, makes clang's host pass silently drop the
  // kernel's launch stub.)
  auto load_rows = [&](int t, int stage, const int* vo) {
    const int q0 = t * BMQ;
    const int rows = min(nq - q0, BMQ);
    const int64_t sn = w_hi ? p.sdon : p.sqn;
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc((w_hi ? dO : Q) + (int64_t)q0 * sn, (int)(rows * sn * 2));
    LDS_AS char* base = sm + OFF_R + stage * RS_B;
#pragma unroll
    for (int i = 0; i < CR; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(base + (wave * CR + i) * 1024), 16, vo[i], 0, 0, 0);
    if (wave == 0 && lane < BMQ * 8 / 16) {
      const __amdgpu_buffer_rsrc_t lrs = tile_rsrc(LD + 2 * (int64_t)q0, BMQ * 8);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(lrs, (LDS_AS void*)(base + 2 * R_B), 16, lane * 16, 0, 0, 0);
    }
  };

  // LDS read offsets. Row-major tiles: the swizzle depends on row & 15, so
  // the wave's 32-row blocks are plain byte offsets; Q^T and dO^T come from
  // the same row-major tiles through transpose reads (16-query steps).
  int roff[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) roff[kk] = swz_off<DP>(l32, 16 * kk + 8 * hh) * 2;
  const int qrow_b = 32 * qh * DP * 2, krow_b = 32 * kb * DP * 2;
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int troff[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    troff[dt][0] = swz_off<DP>(tr_row, 32 * dt + tr_col) * 2;
    troff[dt][1] = swz_off<DP>(tr_row + 8, 32 * dt + tr_col) * 2;
  }

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  const float sl2 = p.scale_log2;
  const int n_qt = (nq + BMQ - 1) / BMQ;  // every tile starts below nq
  int t_begin = 0;
  if (CAUSAL) t_begin = max(0, k0 - off) / BMQ;  // first tile holding a query that sees key k0
  const int kcol = k0 + 32 * kb + l32;            // this lane's key
  const int n_t = max(0, n_qt - t_begin);

  // The two query halves run half a tile apart, so that on every SIMD one
  // wave computes S, dP and the softmax (MFMA then VALU) while its partner
  // (same keys, other query half) accumulates dV and dK (MFMA only). Step
  // 2i of a wave is phase 1 of its i-th tile, step 2i+1 phase 2; the qh = 1
  // waves are one step behind, so tile i's rows are read in segments 2i ..
  // 2i+2 and tile i+2 (same row stage) loads during segment 2i+3.
  X8 P0{}, P1{}, G0{}, G1{};  // phase 1 -> phase 2 of the same tile
  auto phase1 = [&](int t, const LDS_AS char* st) {
    const int q0 = t * BMQ;
    f32x16 s = f32x16{}, dp = f32x16{};
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      s = mfma32(*(const LDS_AS X8*)(st + qrow_b + roff[kk]), *(const LDS_AS X8*)(sm + OFF_K + krow_b + roff[kk]), s);
      dp = mfma32(*(const LDS_AS X8*)(st + R_B + qrow_b + roff[kk]),
                  *(const LDS_AS X8*)(sm + OFF_V + krow_b + roff[kk]), dp);
    }
    __builtin_amdgcn_s_setprio(0);
    // Register i holds query q0 + 32*qh + 8*(i/4) + 4*hh + i%4 of key kcol;
    // (L*log2e, delta) of those four consecutive queries are two 16-byte reads.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const LDS_AS f32x4* ldp = (const LDS_AS f32x4*)(st + 2 * R_B + (32 * qh + 8 * j + 4 * hh) * 8);
      const f32x4 a = ldp[0], c = ldp[1];
      const float l2v[4] = {a[0], a[2], c[0], c[2]};
      const float dlv[4] = {a[1], a[3], c[1], c[3]};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * j + e;
        const float pv = fast_exp2(fmaf(s[i], sl2, -l2v[e]));
        s[i] = pv;
        dp[i] = pv * (dp[i] - dlv[e]);
      }
    }
    if (CAUSAL && k0 + 32 * kb + 31 > q0 + 32 * qh + off) {  // block crosses the diagonal
      const int lim = kcol - (q0 + 32 * qh + 4 * hh + off);  // masked if 8*(i/4) + i%4 < lim
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool m = 8 * (i >> 2) + (i & 3) < lim;
        s[i] = m ? 0.f : s[i];
        dp[i] = m ? 0.f : dp[i];
      }
    }
    P0 = pack8<T>(s, 0);
    P1 = pack8<T>(s, 8);
    G0 = pack8<T>(dp, 0);
    G1 = pack8<T>(dp, 8);
  };
  auto phase2 = [&](const LDS_AS char* st) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const LDS_AS char* qb = st + (32 * qh + 16 * ks) * DP * 2;
        const X8 ado = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(qb + R_B + troff[dt][0])),
                                    lds_read_tr((const LDS_AS T*)(qb + R_B + troff[dt][1])));
        const X8 aq = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(qb + troff[dt][0])),
                                   lds_read_tr((const LDS_AS T*)(qb + troff[dt][1])));
        dv[dt] = mfma32(ado, ks == 0 ? P0 : P1, dv[dt]);
        dk[dt] = mfma32(aq, ks == 0 ? G0 : G1, dk[dt]);
      }
    }
  };

  if (n_t > 0) load_rows(t_begin, 0, rvo);
  if (n_t > 1) load_rows(t_begin + 1, 1, rvo);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // One loop per query half (wave-uniform branch outside the loops), so each
  // phase's registers are live only in its own segment; both loops pass the
  // same 2*n_t + 1 barriers. Segment 2i+1 (i >= 1) loads tile i+1 into the
  // stage tile i-1 used.
  auto seg_end = [&]() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  if (qh == 0) {
    for (int i = 0; i < n_t; ++i) {
      const LDS_AS char* st = sm + OFF_R + (i & 1) * RS_B;
      phase1(t_begin + i, st);  // segment 2i
      seg_end();
      if (i >= 1 && i + 1 < n_t) load_rows(t_begin + i + 1, (i + 1) & 1, rvo);  // segment 2i+1
      phase2(st);
      seg_end();
    }
    seg_end();  // segment 2*n_t: the other half's last phase 2
  } else {
    seg_end();  // segment 0: the other half's first phase 1
    for (int i = 0; i < n_t; ++i) {
      const LDS_AS char* st = sm + OFF_R + (i & 1) * RS_B;
      if (i >= 1 && i + 1 < n_t) load_rows(t_begin + i + 1, (i + 1) & 1, rvo);  // segment 2i+1
      phase1(t_begin + i, st);
      seg_end();
      phase2(st);  // segment 2i+2
      seg_end();
    }
  }

  // Sum the two query halves through LDS (f32x4 groups, lane-contiguous).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  LDS_AS f32x4* park = (LDS_AS f32x4*)sm + kb * NG * 64 + lane;
  if (qh == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        park[(dt * 4 + g) * 64] = f32x4{dk[dt][4 * g], dk[dt][4 * g + 1], dk[dt][4 * g + 2], dk[dt][4 * g + 3]};
        park[(DT * 4 + dt * 4 + g) * 64] = f32x4{dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3]};
      }
  }
  __syncthreads();
  if (qh == 0 && kcol < nk) {
    T* rk = (T*)p.dk + (int64_t)b * p.sdkb + (int64_t)h * p.sdkh + (int64_t)kcol * p.sdkn;
    T* rv = (T*)p.dv + (int64_t)b * p.sdvb + (int64_t)h * p.sdvh + (int64_t)kcol * p.sdvn;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
        if (d < D) {
          const f32x4 ok = park[(dt * 4 + g) * 64];
          const f32x4 ov = park[(DT * 4 + dt * 4 + g) * 64];
          X4 ck, cv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ck[e] = (T)((dk[dt][4 * g + e] + ok[e]) * sc);
            cv[e] = (T)(dv[dt][4 * g + e] + ov[e]);
          }
          *(X4*)(rk + d) = ck;
          *(X4*)(rv + d) = cv;
        }
      }
  }
}

// phases: bit 0 the dq kernel, bit 1 the dk/dv kernel.
template <typename T, int DP, bool CAUSAL>
static hipError_t launch_bwd(BwdParams p, int phases, hipStream_t s) {
  // An empty axis means an empty grid: that kernel has nothing to write
  // (with no queries dK = dV = 0 still needs the dK/dV kernel, which then
  // runs no query tile).
  hipError_t e = hipSuccess;
  p.num_tiles = (p.Nq + 127) / 128;
  if ((phases & 1) && p.num_tiles > 0) {
    hipLaunchKernelGGL((fa_bwd_dq_kernel<T, DP, CAUSAL>), dim3(p.num_tiles * p.B * p.H), dim3(256), 0, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  p.num_tiles = (p.Nk + 127) / 128;
  if ((phases & 2) && p.num_tiles > 0) {
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<T, DP, CAUSAL>), dim3(p.num_tiles * p.B * p.H), dim3(512), 0, s, p);
    e = hipGetLastError();
  }
  return e;
}

template <typename T>
static hipError_t dispatch_bwd_t(const BwdParams& p, int dp, bool causal, int ph, hipStream_t s) {
  switch (dp) {
    case 32: return causal ? launch_bwd<T, 32, true>(p, ph, s) : launch_bwd<T, 32, false>(p, ph, s);
    case 64: return causal ? launch_bwd<T, 64, true>(p, ph, s) : launch_bwd<T, 64, false>(p, ph, s);
    default: return causal ? launch_bwd<T, 128, true>(p, ph, s) : launch_bwd<T, 128, false>(p, ph, s);
  }
}

hipError_t bwd_mfma(const BwdParams& p, bool is_bf16, int dp, bool causal, int phases, hipStream_t s) {
  if (is_bf16) return dispatch_bwd_t<__bf16>(p, dp, causal, phases, s);
  return dispatch_bwd_t<_Float16>(p, dp, causal, phases, s);
}

}  // namespace lsfa
