// Exact fp32 FlashAttention (forward and backward) on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32: fp32 operands, fp32 accumulate).
//
// This is the path for float32 inputs: the reference checks its fp32 results
// against SDPA at 1e-3 and runs gradcheck in fp32
// (kernels/tests/test_flash_attention.py:49-53,
// kernels/tests/test_flash_attention_backward.py:44-65), so nothing here is
// rounded to a narrower type. Arbitrary element strides and any head_dim
// <= 128 (zero-padded to DP = 32, 64 or 128) are accepted.
//
// Math is the same as the bf16/fp16 kernels (kernels/flash_attention.py:
// 135-179, kernels/flash_attention_backward.py:290-330), with a row max per
// 32-key block (standard online softmax) and exponentials in base 2.
//
// Operand layouts of v_mfma_f32_32x32x2_f32 (checked on the device): lane l
// supplies A[l % 32][l / 32] and B[l / 32][l % 32]; register i of lane l
// holds C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]. With hh = l / 32:
//   - a product over the head dim takes step kk (0 .. DP/2 - 1) as the dims
//     kk (hh = 0) and kk + DP/2 (hh = 1); the row operand (K, Q or dO rows)
//     is read from LDS, four steps per ds_read_b128, and the column operand
//     (Q, dO, K or V of the lane's own row) is held in registers;
//   - a product over a 32-row block of the score tile takes step j (0..15)
//     as rows 8 (j / 4) + 4 hh + j % 4, which is exactly register j of the
//     score tile: the B operand is the score register itself, and the A
//     operand is one row per half-wave of a V, K, dO or Q tile (32
//     consecutive floats per half-wave, one ds_read_b32).
// Tiles are staged through LDS with padded rows: row stride DP + 4 floats
// for tiles read four steps at a time by 16 rows (every 16-byte read of a
// quarter-wave hits distinct banks), DP + 8 for tiles read one row per
// half-wave (the two rows of a read, 4 apart, land 32 banks apart).
#include "fa_common.hpp"

namespace lsfa {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2f = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Stage rows [r0, r0 + R) of a strided fp32 matrix (rows x D valid) into LDS
// rows of stride LD (zero outside the matrix or past D).
template <int R, int DP, int LD>
__device__ __forceinline__ void stage_rows(float* dst, const float* src, int64_t srow, int64_t scol, int r0, int rows,
                                           int D, int tid, int nthreads) {
  for (int idx = tid; idx < R * DP; idx += nthreads) {
    const int r = idx / DP, c = idx - r * DP, g = r0 + r;
    dst[r * LD + c] = (g < rows && c < D) ? src[(int64_t)g * srow + (int64_t)c * scol] : 0.f;
  }
}

// Column operand of a head-dim product: this lane's row, dims kk + hh * DP/2.
template <int DP>
__device__ __forceinline__ void load_row_operand(float (&reg)[DP / 2], const float* src, int64_t srow, int64_t scol,
                                                 int row, int rows, int D, int hh) {
#pragma unroll
  for (int kk = 0; kk < DP / 2; ++kk) {
    const int d = kk + hh * (DP / 2);
    reg[kk] = (row < rows && d < D) ? src[(int64_t)row * srow + (int64_t)d * scol] : 0.f;
  }
}

// C = (rows of A tile) x reg^T over the head dim: 32 tile rows (LDS, stride
// LD, first row base) against this lane's register row.
template <int DP, int LD>
__device__ __forceinline__ f32x16 dim_product(const float* base, const float (&reg)[DP / 2], int l32, int hh) {
  f32x16 c = f32x16{};
  const float* row = base + l32 * LD + hh * (DP / 2);
#pragma unroll
  for (int k4 = 0; k4 < DP / 8; ++k4) {
    const f32x4 a = *(const f32x4*)(row + 4 * k4);
#pragma unroll
    for (int e = 0; e < 4; ++e) c = mfma_f32(a[e], reg[4 * k4 + e], c);
  }
  return c;
}

// acc[dt] += (tile rows)^T x scores over a 32-row block: tile rows r_j (LDS,
// stride LD) times register j of the score tile s.
template <int DT, int LD>
__device__ __forceinline__ void block_product(f32x16 (&acc)[DT], const float* tile, const f32x16& s, int l32, int hh) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float* row = tile + (8 * (j >> 2) + 4 * hh + (j & 3)) * LD + l32;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = mfma_f32(row[32 * dt], s[j], acc[dt]);
  }
}

__device__ __forceinline__ float hmax(float x) { return half_max(x); }
__device__ __forceinline__ float hsum(float x) { return half_sum(x); }

// Forward: workgroup = 4 waves x 32 queries; keys in blocks of 32. S^T = K Q^T
// (lane = query, registers = keys), O^T += V^T P^T.
template <int DP, bool VARLEN>
__global__ __launch_bounds__(256) void fa_fwd_f32_kernel(const FwdParams p, int causal, float scale) {
  constexpr int BM = 128, BN = 32, DT = DP / 32, LDK = DP + 4, LDV = DP + 8;
  __shared__ __attribute__((aligned(16))) float Ks[BN * LDK];
  __shared__ __attribute__((aligned(16))) float Vs[BN * LDV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int bh = blockIdx.y, b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  int nq = p.Nq, nk = p.Nk;
  int64_t rq0 = 0, rk0 = 0;
  if (VARLEN) {
    rq0 = p.cu_q[b];
    nq = p.cu_q[b + 1] - (int)rq0;
    rk0 = p.cu_k[b];
    nk = p.cu_k[b + 1] - (int)rk0;
  }
  const int q0 = blockIdx.x * BM;
  if (q0 >= nq) return;  // uniform, before any barrier
  const int off = nk - nq, D = p.D;
  const float* Q = (const float*)p.q + (VARLEN ? 0 : (int64_t)b * p.sqb) + (int64_t)h * p.sqh + rq0 * p.sqn;
  const float* K = (const float*)p.k + (VARLEN ? 0 : (int64_t)b * p.skb) + (int64_t)hk * p.skh + rk0 * p.skn;
  const float* V = (const float*)p.v + (VARLEN ? 0 : (int64_t)b * p.svb) + (int64_t)hk * p.svh + rk0 * p.svn;
  float* O = (float*)p.o + (VARLEN ? 0 : (int64_t)b * p.sob) + (int64_t)h * p.soh + rq0 * p.son;
  const int qw = q0 + 32 * wave, qrow = qw + l32;
  const float sl2 = scale * kLog2e;

  float qreg[DP / 2];
  load_row_operand<DP>(qreg, Q, p.sqn, p.sqd, qrow, nq, D, hh);
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;  // log2 units

  int kv_end = nk;
  if (causal) kv_end = min(nk, q0 + BM + off);
  for (int kt = 0; kt < kv_end; kt += BN) {
    __syncthreads();
    stage_rows<BN, DP, LDK>(Ks, K, p.skn, p.skd, kt, nk, D, tid, 256);
    stage_rows<BN, DP, LDV>(Vs, V, p.svn, p.svd, kt, nk, D, tid, 256);
    __syncthreads();
    if (causal && kt > qw + 31 + off) continue;  // wave-uniform: no key of the block is visible
    f32x16 s = dim_product<DP, LDK>(Ks, qreg, l32, hh);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kt + 8 * (i >> 2) + 4 * hh + (i & 3);
      float x = s[i] * sl2;
      if (key >= nk || (causal && key > qrow + off)) x = -INFINITY;
      s[i] = x;
      mx = fmaxf(mx, x);
    }
    const float m_new = fmaxf(m, hmax(mx));
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m - m_use);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = exp2f(s[i] - m_use);
      sum += s[i];
    }
    l = l * alpha + hsum(sum);
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
    block_product<DT, LDV>(acc, Vs, s, l32, hh);
  }
  if (qrow < nq) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 32 * dt + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (d < D) O[(int64_t)qrow * p.son + (int64_t)d * p.sod] = acc[dt][i] * inv;
      }
    if (p.lse != nullptr && hh == 0) {
      float* L = p.lse + (VARLEN ? 0 : (int64_t)b * p.slb) + (int64_t)h * p.slh + (rq0 + qrow) * p.sln;
      *L = l > 0.f ? (m + __log2f(l)) * kLn2f : -INFINITY;
    }
  }
}

// Query-stationary dQ (and delta = rowsum(dO * O), stored beside L for the
// dK/dV kernel): S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - delta),
// dQ^T += K^T dS^T.
template <int DP>
__global__ __launch_bounds__(256) void fa_bwd_dq_f32_kernel(const BwdParams p, int causal) {
  constexpr int BM = 128, BN = 32, DT = DP / 32, LDK = DP + 4, LDV = DP + 4;
  __shared__ __attribute__((aligned(16))) float Ks[BN * LDK];
  __shared__ __attribute__((aligned(16))) float Vs[BN * LDV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D, off = nk - nq;
  const int q0 = blockIdx.x * BM;
  const float* Q = (const float*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const float* K = (const float*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const float* V = (const float*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const float* Og = (const float*)p.o + (int64_t)b * p.sob + (int64_t)h * p.soh;
  const float* dO = (const float*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  float* dQ = (float*)p.dq + (int64_t)b * p.sdqb + (int64_t)h * p.sdqh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  float* Dg = p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh + 1;  // delta of query q at Dg[2q]
  const int qw = q0 + 32 * wave, qrow = qw + l32;
  const bool valid = qrow < nq;

  float qreg[DP / 2], doreg[DP / 2];
  load_row_operand<DP>(qreg, Q, p.sqn, p.sqd, qrow, nq, D, hh);
  load_row_operand<DP>(doreg, dO, p.sdon, p.sdod, qrow, nq, D, hh);
  float dpart = 0.f;
#pragma unroll
  for (int kk = 0; kk < DP / 2; ++kk) {
    const int d = kk + hh * (DP / 2);
    if (valid && d < D) dpart += doreg[kk] * Og[(int64_t)qrow * p.son + (int64_t)d * p.sod];
  }
  const float delta = hsum(dpart);
  float L2 = valid ? Lg[(int64_t)qrow * p.sln] : INFINITY;
  if (L2 == -INFINITY) L2 = INFINITY;  // a row that sees no key: P = 0
  L2 *= kLog2e;
  if (valid && hh == 0) Dg[2 * (int64_t)qrow] = delta;
  const float sl2 = p.scale * kLog2e;

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  int kv_end = nk;
  if (q0 < nq && causal) kv_end = min(nk, q0 + BM + off);
  if (q0 >= nq) kv_end = 0;
  for (int kt = 0; kt < kv_end; kt += BN) {
    __syncthreads();
    stage_rows<BN, DP, LDK>(Ks, K, p.skn, p.skd, kt, nk, D, tid, 256);
    stage_rows<BN, DP, LDV>(Vs, V, p.svn, p.svd, kt, nk, D, tid, 256);
    __syncthreads();
    if (causal && kt > qw + 31 + off) continue;
    f32x16 s = dim_product<DP, LDK>(Ks, qreg, l32, hh);
    const f32x16 dp = dim_product<DP, LDV>(Vs, doreg, l32, hh);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kt + 8 * (i >> 2) + 4 * hh + (i & 3);
      float pr = exp2f(s[i] * sl2 - L2);
      if (key >= nk || (causal && key > qrow + off)) pr = 0.f;
      s[i] = pr * (dp[i] - delta);
    }
    block_product<DT, LDK>(acc, Ks, s, l32, hh);
  }
  if (valid) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 32 * dt + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (d < D) dQ[(int64_t)qrow * p.sdqn + (int64_t)d * p.sdqd] = acc[dt][i] * p.scale;
      }
  }
}

// Key-stationary dK, dV: S = Q K^T and dP = dO V^T with the keys as the
// columns (lane = key, registers = queries), dV^T += dO^T P, dK^T += Q^T dS.
template <int DP>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_f32_kernel(const BwdParams p, int causal) {
  constexpr int BK = 128, BM = 32, DT = DP / 32, LDQ = DP + 4;
  __shared__ __attribute__((aligned(16))) float Qs[BM * LDQ];
  __shared__ __attribute__((aligned(16))) float dOs[BM * LDQ];
  __shared__ float Ls[BM], Ds[BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D, off = nk - nq;
  const int k0 = blockIdx.x * BK;
  const float* Q = (const float*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const float* K = (const float*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const float* V = (const float*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const float* dO = (const float*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  float* dK = (float*)p.dk + (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
  float* dV = (float*)p.dv + (int64_t)b * p.sdvb + (int64_t)h * p.sdvh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float* Dg = p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh + 1;  // delta of query q at Dg[2q]
  const int kw = k0 + 32 * wave, krow = kw + l32;

  float kreg[DP / 2], vreg[DP / 2];
  load_row_operand<DP>(kreg, K, p.skn, p.skd, krow, nk, D, hh);
  load_row_operand<DP>(vreg, V, p.svn, p.svd, krow, nk, D, hh);
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] = f32x16{};
    dv[dt] = f32x16{};
  }
  const float sl2 = p.scale * kLog2e;
  int q_lo = (causal && k0 < nk) ? max(0, k0 - off) : 0;
  q_lo = (q_lo / BM) * BM;
  const int q_end = k0 < nk ? nq : 0;
  for (int qt = q_lo; qt < q_end; qt += BM) {
    __syncthreads();
    stage_rows<BM, DP, LDQ>(Qs, Q, p.sqn, p.sqd, qt, nq, D, tid, 256);
    stage_rows<BM, DP, LDQ>(dOs, dO, p.sdon, p.sdod, qt, nq, D, tid, 256);
    if (tid < BM) {
      const int q = qt + tid;
      float lv = q < nq ? Lg[(int64_t)q * p.sln] : INFINITY;
      if (lv == -INFINITY) lv = INFINITY;
      Ls[tid] = lv * kLog2e;
      Ds[tid] = q < nq ? Dg[2 * (int64_t)q] : 0.f;
    }
    __syncthreads();
    if (causal && kw > qt + BM - 1 + off) continue;  // wave-uniform: no query of the block sees these keys
    f32x16 s = dim_product<DP, LDQ>(Qs, kreg, l32, hh);
    f32x16 dp = dim_product<DP, LDQ>(dOs, vreg, l32, hh);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 8 * (i >> 2) + 4 * hh + (i & 3), q = qt + r;
      float pr = exp2f(s[i] * sl2 - Ls[r]);
      if (q >= nq || krow >= nk || (causal && krow > q + off)) pr = 0.f;
      s[i] = pr;
      dp[i] = pr * (dp[i] - Ds[r]);
    }
    block_product<DT, LDQ>(dv, dOs, s, l32, hh);
    block_product<DT, LDQ>(dk, Qs, dp, l32, hh);
  }
  if (krow < nk) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = 32 * dt + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (d < D) {
          dK[(int64_t)krow * p.sdkn + (int64_t)d * p.sdkd] = dk[dt][i] * p.scale;
          dV[(int64_t)krow * p.sdvn + (int64_t)d * p.sdvd] = dv[dt][i];
        }
      }
  }
}

template <int DP>
static hipError_t launch_fwd_f32(const FwdParams& p, bool causal, bool varlen, float scale, hipStream_t s) {
  dim3 grid((p.Nq + 127) / 128, p.B * p.Hq);
  if (varlen)
    hipLaunchKernelGGL((fa_fwd_f32_kernel<DP, true>), grid, dim3(256), 0, s, p, (int)causal, scale);
  else
    hipLaunchKernelGGL((fa_fwd_f32_kernel<DP, false>), grid, dim3(256), 0, s, p, (int)causal, scale);
  return hipGetLastError();
}

hipError_t fwd_f32(const FwdParams& p, int dp, bool causal, bool varlen, float scale, hipStream_t s) {
  switch (dp) {
    case 32: return launch_fwd_f32<32>(p, causal, varlen, scale, s);
    case 64: return launch_fwd_f32<64>(p, causal, varlen, scale, s);
    default: return launch_fwd_f32<128>(p, causal, varlen, scale, s);
  }
}

template <int DP>
static hipError_t launch_bwd_f32(const BwdParams& p, bool causal, hipStream_t s) {
  if (p.Nq > 0) {
    hipLaunchKernelGGL((fa_bwd_dq_f32_kernel<DP>), dim3((p.Nq + 127) / 128, p.B * p.H), dim3(256), 0, s, p,
                       (int)causal);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.Nk > 0) {
    hipLaunchKernelGGL((fa_bwd_dkdv_f32_kernel<DP>), dim3((p.Nk + 127) / 128, p.B * p.H), dim3(256), 0, s, p,
                       (int)causal);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t bwd_f32(const BwdParams& p, int dp, bool causal, hipStream_t s) {
  switch (dp) {
    case 32: return launch_bwd_f32<32>(p, causal, s);
    case 64: return launch_bwd_f32<64>(p, causal, s);
    default: return launch_bwd_f32<128>(p, causal, s);
  }
}

}  // namespace lsfa
