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
// dQ (and delta). Workgroup = 4 waves x 32 query rows; K/V tiles of 64 keys
// double-buffered in LDS. Per key tile and wave:
//   S^T  = K Q^T          A = K rows (LDS),  B = Q^T  (registers)
//   dP^T = V dO^T         A = V rows (LDS),  B = dO^T (registers)
//   dS^T = P^T (dP^T - delta)  -> rounded into B operands
//   dQ^T += K^T dS^T      A = K^T via transpose reads of the same LDS tile
// ---------------------------------------------------------------------------
template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fa_bwd_dq_kernel(const BwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int BM = 128, BN = 64, SEGS = DP / 8;
  constexpr int TILE = BN * DP;
  constexpr int CH = BN * SEGS / 256;
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int KB = BN / 32;

  __shared__ __attribute__((aligned(16))) T smem_raw[4 * TILE];
  LDS_AS T* smem = (LDS_AS T*)smem_raw;

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

  u32x4 kst[CH], vst[CH];
  auto gload = [&](int j) {
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / SEGS, col = (c % SEGS) * 8;
      const int key = j * BN + row;
      const bool ok = key < nk && col < D;
      kst[r] = ok ? ldg16(K + (int64_t)key * p.skn + col) : u32x4{0, 0, 0, 0};
      vst[r] = ok ? ldg16(V + (int64_t)key * p.svn + col) : u32x4{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int stage) {
    LDS_AS T* Ks = smem + stage * 2 * TILE;
    LDS_AS T* Vs = Ks + TILE;
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / SEGS, col = (c % SEGS) * 8;
      const int o = swz_off<DP>(row, col);
      *(LDS_AS u32x4*)(Ks + o) = kst[r];
      *(LDS_AS u32x4*)(Vs + o) = vst[r];
    }
  };

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  const float sl2 = p.scale_log2;
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    if (j + 1 < ntiles) gload(j + 1);
    const int kbase = j * BN;
    const bool active = !CAUSAL || (kbase <= qw_lo + 31 + off);
    if (active) {
      const LDS_AS T* Ks = smem + (j & 1) * 2 * TILE;
      const LDS_AS T* Vs = Ks + TILE;
      f32x16 s[KB], dp[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s[kb] = f32x16{};
        dp[kb] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          const int o = swz_off<DP>(kb * 32 + l32, 16 * kk + 8 * hh);
          s[kb] = mfma32(lds_read8<T>(Ks + o), qreg[kk], s[kb]);
          dp[kb] = mfma32(lds_read8<T>(Vs + o), doreg[kk], dp[kb]);
        }
      }
      const bool need_mask = CAUSAL && (kbase + BN - 1 > qw_lo + off);
      X8 dsb[2 * KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float pv = fast_exp2(s[kb][i] * sl2 - l2);
          if (need_mask) {
            const int key = kbase + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
            if (key > qrow + off) pv = 0.f;
          }
          s[kb][i] = pv * (dp[kb][i] - delta);
        }
        dsb[2 * kb] = pack8<T>(s[kb], 0);
        dsb[2 * kb + 1] = pack8<T>(s[kb], 8);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int ks = 0; ks < 2 * KB; ++ks) {
          const int row = ks * 16 + tr_row;
          const int col = 32 * dt + tr_col;
          X4 a0 = lds_read_tr(Ks + swz_off<DP>(row, col));
          X4 a1 = lds_read_tr(Ks + swz_off<DP>(row + 8, col));
          acc[dt] = mfma32(cat4<X8, X4>(a0, a1), dsb[ks], acc[dt]);
        }
      }
    }
    if (j + 1 < ntiles) sstore((j + 1) & 1);
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
// dK, dV. Workgroup = 4 waves x 32 keys; query tiles of 64 rows (Q, dO, and
// the per-row L and delta) double-buffered in LDS. Per query tile and wave,
// for each 32-row half qb:
//   S  = Q K^T            A = Q rows (LDS),  B = K^T (registers)
//   dP = dO V^T           A = dO rows (LDS), B = V^T (registers)
//   P  = exp2(S*scale*log2e - L*log2e), dS = P (dP - delta)
//   dV^T += dO^T P        A = dO^T via transpose reads, B = P (registers)
//   dK^T += Q^T dS        A = Q^T via transpose reads,  B = dS (registers)
// Query rows beyond the sequence get L = +inf, so their P is exactly 0.
// ---------------------------------------------------------------------------
template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_kernel(const BwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int BNK = 128, BMQ = 64, SEGS = DP / 8;
  constexpr int TILE = BMQ * DP;
  constexpr int CH = BMQ * SEGS / 256;
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int STAGE = 2 * TILE * (int)sizeof(T) + 2 * BMQ * 4;  // bytes

  __shared__ __attribute__((aligned(16))) char smem_raw[2 * STAGE];
  LDS_AS char* smem = (LDS_AS char*)smem_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31, hh = lane >> 5;
  int bh, kt;
  map_tile(p.num_tiles, gridDim.x, bh, kt, false);
  const int b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D;
  const int k0 = kt * BNK;
  const int off = nk - nq;

  const T* Q = (const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const T* K = (const T*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const T* V = (const T*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const T* dO = (const T*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  T* dK = (T*)p.dk + (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
  T* dV = (T*)p.dv + (int64_t)b * p.sdvb + (int64_t)h * p.sdvh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float* Dg = p.delta + (int64_t)b * p.slb + (int64_t)h * p.slh;

  const int kw_lo = k0 + wave * 32;
  const int krow = kw_lo + l32;
  const bool kvalid = krow < nk;

  X8 kreg[KSTEPS], vreg[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    u32x4 rk = {0, 0, 0, 0}, rv = {0, 0, 0, 0};
    if (kvalid && col < D) {
      rk = ldg16(K + (int64_t)krow * p.skn + col);
      rv = ldg16(V + (int64_t)krow * p.svn + col);
    }
    kreg[kk] = __builtin_bit_cast(X8, rk);
    vreg[kk] = __builtin_bit_cast(X8, rv);
  }

  // Query range that can see this key tile.
  int q_lo = 0;
  if (CAUSAL) q_lo = max(0, k0 - off);
  q_lo = (q_lo / BMQ) * BMQ;
  const int ntiles = (nq > q_lo) ? (nq - q_lo + BMQ - 1) / BMQ : 0;

  u32x4 qst[CH], dost[CH];
  float lst = 0.f;
  auto gload = [&](int t) {
    const int qs = q_lo + t * BMQ;
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / SEGS, col = (c % SEGS) * 8;
      const int q = qs + row;
      const bool ok = q < nq && col < D;
      qst[r] = ok ? ldg16(Q + (int64_t)q * p.sqn + col) : u32x4{0, 0, 0, 0};
      dost[r] = ok ? ldg16(dO + (int64_t)q * p.sdon + col) : u32x4{0, 0, 0, 0};
    }
    if (tid < 2 * BMQ) {
      const int q = qs + (tid & (BMQ - 1));
      if (tid < BMQ) {
        float lv = q < nq ? Lg[(int64_t)q * p.sln] : INFINITY;
        if (lv == -INFINITY) lv = INFINITY;
        lst = lv * kLog2eB;
      } else {
        lst = q < nq ? Dg[(int64_t)q * p.sln] : 0.f;
      }
    }
  };
  auto sstore = [&](int stage) {
    LDS_AS char* base = smem + stage * STAGE;
    LDS_AS T* Qs = (LDS_AS T*)base;
    LDS_AS T* dOs = Qs + TILE;
    LDS_AS float* Ls = (LDS_AS float*)(dOs + TILE);
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      const int c = tid + 256 * r;
      const int row = c / SEGS, col = (c % SEGS) * 8;
      const int o = swz_off<DP>(row, col);
      *(LDS_AS u32x4*)(Qs + o) = qst[r];
      *(LDS_AS u32x4*)(dOs + o) = dost[r];
    }
    if (tid < 2 * BMQ) Ls[tid] = lst;
  };

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  const float sl2 = p.scale_log2;
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) gload(t + 1);
    const int qs = q_lo + t * BMQ;
    // Causal: every key of this wave is beyond every query of the tile.
    const bool active = !CAUSAL || (qs + BMQ - 1 + off >= kw_lo);
    if (active) {
      LDS_AS char* base = smem + (t & 1) * STAGE;
      const LDS_AS T* Qs = (const LDS_AS T*)base;
      const LDS_AS T* dOs = Qs + TILE;
      const LDS_AS float* Ls = (const LDS_AS float*)(dOs + TILE);
      const LDS_AS float* Ds = Ls + BMQ;
      const bool need_mask = CAUSAL && (qs + off < kw_lo + 31);
#pragma unroll
      for (int qb = 0; qb < BMQ / 32; ++qb) {
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          const int o = swz_off<DP>(qb * 32 + l32, 16 * kk + 8 * hh);
          s = mfma32(lds_read8<T>(Qs + o), kreg[kk], s);
          dp = mfma32(lds_read8<T>(dOs + o), vreg[kk], dp);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int qi = qb * 32 + 8 * g + 4 * hh;  // tile-local row of register 4g
          const f32x4 lv = *(const LDS_AS f32x4*)(Ls + qi);
          const f32x4 dl = *(const LDS_AS f32x4*)(Ds + qi);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float pv = fast_exp2(s[4 * g + e] * sl2 - lv[e]);
            if (need_mask && krow > qs + qi + e + off) pv = 0.f;
            s[4 * g + e] = pv;
            dp[4 * g + e] = pv * (dp[4 * g + e] - dl[e]);
          }
        }
        const X8 pb0 = pack8<T>(s, 0), pb1 = pack8<T>(s, 8);
        const X8 db0 = pack8<T>(dp, 0), db1 = pack8<T>(dp, 8);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int col = 32 * dt + tr_col;
#pragma unroll
          for (int kk2 = 0; kk2 < 2; ++kk2) {
            const int row = qb * 32 + kk2 * 16 + tr_row;
            const int o0 = swz_off<DP>(row, col), o1 = swz_off<DP>(row + 8, col);
            const X8 doT = cat4<X8, X4>(lds_read_tr(dOs + o0), lds_read_tr(dOs + o1));
            const X8 qT = cat4<X8, X4>(lds_read_tr(Qs + o0), lds_read_tr(Qs + o1));
            dv[dt] = mfma32(doT, kk2 ? pb1 : pb0, dv[dt]);
            dk[dt] = mfma32(qT, kk2 ? db1 : db0, dk[dt]);
          }
        }
      }
    }
    if (t + 1 < ntiles) sstore((t + 1) & 1);
    __syncthreads();
  }

  if (kvalid) {
    T* krow_k = dK + (int64_t)krow * p.sdkn;
    T* krow_v = dV + (int64_t)krow * p.sdvn;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
        if (d < D) {
          X4 a, c;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[e] = (T)(dk[dt][4 * g + e] * sc);
            c[e] = (T)dv[dt][4 * g + e];
          }
          *(X4*)(krow_k + d) = a;
          *(X4*)(krow_v + d) = c;
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
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<T, DP, CAUSAL>), dim3(p.num_tiles * p.B * p.H), dim3(256), 0, s, p);
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
