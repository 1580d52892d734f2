// FlashAttention forward for gfx950: bf16/fp16 operands on
// v_mfma_f32_32x32x16, fp32 online softmax in base 2.
//
// Algorithm (same per-tile order as kernels/flash_attention.py:121-179 and
// kernels/flash_attention_backward.py:129-169): for each key tile, scores are
// computed and scaled, masked to -inf (key beyond the sequence, or causal),
// the running row max is raised, p = exp(s - m) and alpha = exp(m_old - m),
// l = alpha*l + sum(p), acc = alpha*acc + p(cast to the input dtype) @ V; at
// the end o = acc / l and lse = m + ln(l).
//
// Work decomposition
//   workgroup = 4 waves = 128 query rows of one (batch, head); wave w owns
//   rows 32w..32w+31, one row per lane pair (l, l+32).
//   K/V tiles of 64 keys are staged in LDS, double-buffered, 16-byte segments
//   XOR-swizzled per row.
//   S^T = K Q^T on MFMA (A = K rows from LDS, B = Q held in registers), so
//   every lane owns one query row: the row max/sum need one permlane32 swap.
//   The fp32 S^T accumulator is rounded in registers into the B operand of
//   O^T += V^T P^T; V^T comes from LDS through ds_read_b64_tr_b16.
#include "fa_common.hpp"

namespace lsfa {

constexpr float kLn2 = 0.6931471805599453f;

template <typename T, int DP, bool CAUSAL, bool VARLEN>
__global__ __launch_bounds__(256, 2) void fa_fwd_kernel(const FwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int BM = 128, BN = 64, SEGS = DP / 8;
  constexpr int TILE = BN * DP;
  constexpr int CH = BN * SEGS / 256;  // 16-byte chunks per thread per tensor
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int KB = BN / 32;
  static_assert(CH >= 1, "tile too small for the workgroup");

  __shared__ __attribute__((aligned(16))) T smem_raw[4 * TILE];
  LDS_AS T* smem = (LDS_AS T*)smem_raw;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hh = lane >> 5;
  int bh, qt;
  map_tile(p.num_q_tiles, gridDim.x, bh, qt, CAUSAL);
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  int nq = p.Nq, nk = p.Nk;
  int64_t rq0 = 0, rk0 = 0;
  if (VARLEN) {
    rq0 = p.cu_q[b];
    nq = p.cu_q[b + 1] - (int)rq0;
    rk0 = p.cu_k[b];
    nk = p.cu_k[b + 1] - (int)rk0;
  }
  const int q0 = qt * BM;
  if (q0 >= nq) return;  // uniform across the workgroup, before any barrier
  const int off = nk - nq;  // bottom-right causal alignment

  const T* Q = (const T*)p.q + (VARLEN ? 0 : (int64_t)b * p.sqb) + (int64_t)h * p.sqh + rq0 * p.sqn;
  const T* K = (const T*)p.k + (VARLEN ? 0 : (int64_t)b * p.skb) + (int64_t)hk * p.skh + rk0 * p.skn;
  const T* V = (const T*)p.v + (VARLEN ? 0 : (int64_t)b * p.svb) + (int64_t)hk * p.svh + rk0 * p.svn;
  T* O = (T*)p.o + (VARLEN ? 0 : (int64_t)b * p.sob) + (int64_t)h * p.soh + rq0 * p.son;

  int kv_end = nk;
  if (CAUSAL) kv_end = min(nk, q0 + BM + off);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const int D = p.D;
  const int qw_lo = q0 + wave * 32;
  const int qrow = qw_lo + l32;

  // Q as the B operand of S^T = K Q^T: lane holds row qrow, columns 16kk+8hh..+7.
  X8 qreg[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    u32x4 raw = {0, 0, 0, 0};
    if (qrow < nq && col < D) raw = ldg16(Q + (int64_t)qrow * p.sqn + col);
    qreg[kk] = __builtin_bit_cast(X8, raw);
  }

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
  float m = -INFINITY, l = 0.f;
  const float sl2 = p.scale_log2;

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  // Per-lane constant parts of the LDS addresses.
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  for (int j = 0; j < ntiles; ++j) {
    if (j + 1 < ntiles) gload(j + 1);
    const int kbase = j * BN;
    const bool active = !CAUSAL || (kbase <= qw_lo + 31 + off);
    if (active) {
      const LDS_AS T* Ks = smem + (j & 1) * 2 * TILE;
      const LDS_AS T* Vs = Ks + TILE;
      f32x16 s[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        s[kb] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          X8 a = lds_read8<T>(Ks + swz_off<DP>(kb * 32 + l32, 16 * kk + 8 * hh));
          s[kb] = mfma32(a, qreg[kk], s[kb]);
        }
      }
      const bool need_mask = (kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > qw_lo + off);
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float t = s[kb][i] * sl2;
          if (need_mask) {
            const int key = kbase + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
            if (key >= nk || (CAUSAL && key > qrow + off)) t = -INFINITY;
          }
          s[kb][i] = t;
          mx = fmaxf(mx, t);
        }
      }
      mx = half_max(mx);
      const float m_new = fmaxf(m, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = fast_exp2(s[kb][i] - m_use);
          s[kb][i] = e;
          rs += e;
        }
      }
      l = l * alpha + rs;
      m = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      X8 pb[2 * KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        pb[2 * kb] = pack8<T>(s[kb], 0);
        pb[2 * kb + 1] = pack8<T>(s[kb], 8);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int ks = 0; ks < 2 * KB; ++ks) {
          const int row = ks * 16 + tr_row;
          const int col = 32 * dt + tr_col;
          X4 a0 = lds_read_tr(Vs + swz_off<DP>(row, col));
          X4 a1 = lds_read_tr(Vs + swz_off<DP>(row + 8, col));
          acc[dt] = mfma32(cat4<X8, X4>(a0, a1), pb[ks], acc[dt]);
        }
      }
    }
    if (j + 1 < ntiles) sstore((j + 1) & 1);
    __syncthreads();
  }

  const float lt = half_sum(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (qrow < nq) {
    T* orow = O + (int64_t)qrow * p.son;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * hh;
        if (d < D) {
          X4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)(acc[dt][4 * g + e] * inv);
          *(X4*)(orow + d) = v;
        }
      }
    }
    if (p.lse != nullptr && hh == 0) {
      float* L = p.lse + (VARLEN ? 0 : (int64_t)b * p.slb) + (int64_t)h * p.slh + (rq0 + qrow) * p.sln;
      *L = lt > 0.f ? (m + __log2f(lt)) * kLn2 : -INFINITY;
    }
  }
}

template <typename T, int DP, bool CAUSAL, bool VARLEN>
static hipError_t launch_fwd(const FwdParams& p, hipStream_t s) {
  const int total = p.num_q_tiles * p.B * p.Hq;
  hipLaunchKernelGGL((fa_fwd_kernel<T, DP, CAUSAL, VARLEN>), dim3(total), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int DP>
static hipError_t dispatch_fwd_dp(const FwdParams& p, bool causal, bool varlen, hipStream_t s) {
  if (varlen) return causal ? launch_fwd<T, DP, true, true>(p, s) : launch_fwd<T, DP, false, true>(p, s);
  return causal ? launch_fwd<T, DP, true, false>(p, s) : launch_fwd<T, DP, false, false>(p, s);
}

template <typename T>
static hipError_t dispatch_fwd_t(const FwdParams& p, int dp, bool causal, bool varlen, hipStream_t s) {
  switch (dp) {
    case 32: return dispatch_fwd_dp<T, 32>(p, causal, varlen, s);
    case 64: return dispatch_fwd_dp<T, 64>(p, causal, varlen, s);
    default: return dispatch_fwd_dp<T, 128>(p, causal, varlen, s);
  }
}

// Host entry used by the C ABI layer. is_bf16 selects bf16 vs fp16 operands;
// dp is the padded head dim (32, 64 or 128). Query tile height is 128 rows.
hipError_t fwd_mfma(FwdParams p, bool is_bf16, int dp, bool causal, bool varlen, hipStream_t s) {
  p.num_q_tiles = (p.Nq + 127) / 128;
  if (is_bf16) return dispatch_fwd_t<__bf16>(p, dp, causal, varlen, s);
  return dispatch_fwd_t<_Float16>(p, dp, causal, varlen, s);
}

}  // namespace lsfa
