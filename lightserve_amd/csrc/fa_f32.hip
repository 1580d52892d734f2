// Exact fp32 FlashAttention (forward and backward) on the vector ALUs.
//
// This is the path for float32 inputs: the reference checks its fp32 results
// against SDPA at 1e-3 and runs gradcheck in fp32
// (kernels/tests/test_flash_attention.py:49-53,
// kernels/tests/test_flash_attention_backward.py:44-65), so nothing here is
// rounded to a narrower type. Arbitrary element strides and any head_dim
// <= 128 are accepted. Each query (or key) row is owned by 4 adjacent lanes
// that split the head dimension (lane part p owns dims 4t+p); dot products are
// reduced with two lane shuffles. Tiles of the other operand are staged in LDS.
//
// Math is the same as the MFMA kernels (kernels/flash_attention.py:135-179,
// kernels/flash_attention_backward.py:290-330) in natural-log units.
#include "fa_common.hpp"

namespace lsfa {

__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x;
}

template <int DP, bool VARLEN>
__global__ __launch_bounds__(256) void fa_fwd_f32_kernel(const FwdParams p, int causal, float scale) {
  constexpr int RQ = 64, BN = 32, PT = DP / 4;
  __shared__ float Ks[BN][DP];
  __shared__ float Vs[BN][DP];
  const int tid = threadIdx.x, qi = tid >> 2, part = tid & 3;
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
  const int q0 = blockIdx.x * RQ;
  if (q0 >= nq) return;
  const int off = nk - nq, D = p.D;
  const float* Q = (const float*)p.q + (VARLEN ? 0 : (int64_t)b * p.sqb) + (int64_t)h * p.sqh + rq0 * p.sqn;
  const float* K = (const float*)p.k + (VARLEN ? 0 : (int64_t)b * p.skb) + (int64_t)hk * p.skh + rk0 * p.skn;
  const float* V = (const float*)p.v + (VARLEN ? 0 : (int64_t)b * p.svb) + (int64_t)hk * p.svh + rk0 * p.svn;
  float* O = (float*)p.o + (VARLEN ? 0 : (int64_t)b * p.sob) + (int64_t)h * p.soh + rq0 * p.son;
  const int qrow = q0 + qi;
  const bool valid = qrow < nq;

  float q[PT], o[PT];
#pragma unroll
  for (int t = 0; t < PT; ++t) {
    const int d = 4 * t + part;
    q[t] = (valid && d < D) ? Q[(int64_t)qrow * p.sqn + (int64_t)d * p.sqd] : 0.f;
    o[t] = 0.f;
  }
  int kv_end = nk;
  if (causal) kv_end = min(nk, q0 + RQ + off);
  float m = -INFINITY, l = 0.f;
  for (int kt = 0; kt < kv_end; kt += BN) {
    __syncthreads();
    for (int idx = tid; idx < BN * DP; idx += 256) {
      const int r = idx / DP, c = idx - r * DP, key = kt + r;
      const bool ok = key < nk && c < D;
      Ks[r][c] = ok ? K[(int64_t)key * p.skn + (int64_t)c * p.skd] : 0.f;
      Vs[r][c] = ok ? V[(int64_t)key * p.svn + (int64_t)c * p.svd] : 0.f;
    }
    __syncthreads();
    float sc[BN];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < BN; ++r) {
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < PT; ++t) s += q[t] * Ks[r][4 * t + part];
      s = quad_sum(s) * scale;
      const int key = kt + r;
      if (key >= nk || (causal && key > qrow + off)) s = -INFINITY;
      sc[r] = s;
      mx = fmaxf(mx, s);
    }
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = expf(m - m_use);
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < PT; ++t) o[t] *= alpha;
#pragma unroll
    for (int r = 0; r < BN; ++r) {
      const float pr = expf(sc[r] - m_use);
      sum += pr;
#pragma unroll
      for (int t = 0; t < PT; ++t) o[t] += pr * Vs[r][4 * t + part];
    }
    l = l * alpha + sum;
    m = m_new;
  }
  if (valid) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int t = 0; t < PT; ++t) {
      const int d = 4 * t + part;
      if (d < D) O[(int64_t)qrow * p.son + (int64_t)d * p.sod] = o[t] * inv;
    }
    if (p.lse != nullptr && part == 0) {
      float* L = p.lse + (VARLEN ? 0 : (int64_t)b * p.slb) + (int64_t)h * p.slh + (rq0 + qrow) * p.sln;
      *L = l > 0.f ? m + logf(l) : -INFINITY;
    }
  }
}

// Query-stationary dQ (and delta = rowsum(dO * O)).
template <int DP>
__global__ __launch_bounds__(256) void fa_bwd_dq_f32_kernel(const BwdParams p, int causal) {
  constexpr int RQ = 64, BN = 32, PT = DP / 4;
  __shared__ float Ks[BN][DP];
  __shared__ float Vs[BN][DP];
  const int tid = threadIdx.x, qi = tid >> 2, part = tid & 3;
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D, off = nk - nq;
  const int q0 = blockIdx.x * RQ;
  const float* Q = (const float*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const float* K = (const float*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const float* V = (const float*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const float* Og = (const float*)p.o + (int64_t)b * p.sob + (int64_t)h * p.soh;
  const float* dO = (const float*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  float* dQ = (float*)p.dq + (int64_t)b * p.sdqb + (int64_t)h * p.sdqh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  float* Dg = p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh + 1;  // delta of query q at Dg[2q]
  const int qrow = q0 + qi;
  const bool valid = qrow < nq;

  float q[PT], dor[PT], dq[PT];
  float dpart = 0.f;
#pragma unroll
  for (int t = 0; t < PT; ++t) {
    const int d = 4 * t + part;
    const bool ok = valid && d < D;
    q[t] = ok ? Q[(int64_t)qrow * p.sqn + (int64_t)d * p.sqd] : 0.f;
    dor[t] = ok ? dO[(int64_t)qrow * p.sdon + (int64_t)d * p.sdod] : 0.f;
    const float ov = ok ? Og[(int64_t)qrow * p.son + (int64_t)d * p.sod] : 0.f;
    dpart += dor[t] * ov;
    dq[t] = 0.f;
  }
  const float delta = quad_sum(dpart);
  float L = valid ? Lg[(int64_t)qrow * p.sln] : INFINITY;
  if (L == -INFINITY) L = INFINITY;
  if (valid && part == 0) Dg[2 * (int64_t)qrow] = delta;

  int kv_end = nk;
  if (causal) kv_end = min(nk, q0 + RQ + off);
  const float scale = p.scale;
  for (int kt = 0; kt < kv_end; kt += BN) {
    __syncthreads();
    for (int idx = tid; idx < BN * DP; idx += 256) {
      const int r = idx / DP, c = idx - r * DP, key = kt + r;
      const bool ok = key < nk && c < D;
      Ks[r][c] = ok ? K[(int64_t)key * p.skn + (int64_t)c * p.skd] : 0.f;
      Vs[r][c] = ok ? V[(int64_t)key * p.svn + (int64_t)c * p.svd] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int r = 0; r < BN; ++r) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int t = 0; t < PT; ++t) {
        s += q[t] * Ks[r][4 * t + part];
        dp += dor[t] * Vs[r][4 * t + part];
      }
      s = quad_sum(s);
      dp = quad_sum(dp);
      const int key = kt + r;
      float pr = expf(s * scale - L);
      if (key >= nk || (causal && key > qrow + off)) pr = 0.f;
      const float ds = pr * (dp - delta);
#pragma unroll
      for (int t = 0; t < PT; ++t) dq[t] += ds * Ks[r][4 * t + part];
    }
  }
  if (valid) {
#pragma unroll
    for (int t = 0; t < PT; ++t) {
      const int d = 4 * t + part;
      if (d < D) dQ[(int64_t)qrow * p.sdqn + (int64_t)d * p.sdqd] = dq[t] * scale;
    }
  }
}

// Key-stationary dK, dV.
template <int DP>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_f32_kernel(const BwdParams p, int causal) {
  constexpr int RK = 64, BM = 32, PT = DP / 4;
  __shared__ float Qs[BM][DP];
  __shared__ float dOs[BM][DP];
  __shared__ float Ls[BM], Ds[BM];
  const int tid = threadIdx.x, ki = tid >> 2, part = tid & 3;
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int nq = p.Nq, nk = p.Nk, D = p.D, off = nk - nq;
  const int k0 = blockIdx.x * RK;
  const float* Q = (const float*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
  const float* K = (const float*)p.k + (int64_t)b * p.skb + (int64_t)h * p.skh;
  const float* V = (const float*)p.v + (int64_t)b * p.svb + (int64_t)h * p.svh;
  const float* dO = (const float*)p.dout + (int64_t)b * p.sdob + (int64_t)h * p.sdoh;
  float* dK = (float*)p.dk + (int64_t)b * p.sdkb + (int64_t)h * p.sdkh;
  float* dV = (float*)p.dv + (int64_t)b * p.sdvb + (int64_t)h * p.sdvh;
  const float* Lg = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
  const float* Dg = p.ld + (int64_t)b * p.sldb + (int64_t)h * p.sldh + 1;  // delta of query q at Dg[2q]
  const int krow = k0 + ki;
  const bool valid = krow < nk;

  float k[PT], v[PT], dk[PT], dv[PT];
#pragma unroll
  for (int t = 0; t < PT; ++t) {
    const int d = 4 * t + part;
    const bool ok = valid && d < D;
    k[t] = ok ? K[(int64_t)krow * p.skn + (int64_t)d * p.skd] : 0.f;
    v[t] = ok ? V[(int64_t)krow * p.svn + (int64_t)d * p.svd] : 0.f;
    dk[t] = 0.f;
    dv[t] = 0.f;
  }
  int q_lo = causal ? max(0, k0 - off) : 0;
  q_lo = (q_lo / BM) * BM;
  const float scale = p.scale;
  for (int qt = q_lo; qt < nq; qt += BM) {
    __syncthreads();
    for (int idx = tid; idx < BM * DP; idx += 256) {
      const int r = idx / DP, c = idx - r * DP, q = qt + r;
      const bool ok = q < nq && c < D;
      Qs[r][c] = ok ? Q[(int64_t)q * p.sqn + (int64_t)c * p.sqd] : 0.f;
      dOs[r][c] = ok ? dO[(int64_t)q * p.sdon + (int64_t)c * p.sdod] : 0.f;
    }
    if (tid < BM) {
      const int q = qt + tid;
      float lv = q < nq ? Lg[(int64_t)q * p.sln] : INFINITY;
      if (lv == -INFINITY) lv = INFINITY;
      Ls[tid] = lv;
      Ds[tid] = q < nq ? Dg[2 * (int64_t)q] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int r = 0; r < BM; ++r) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int t = 0; t < PT; ++t) {
        s += Qs[r][4 * t + part] * k[t];
        dp += dOs[r][4 * t + part] * v[t];
      }
      s = quad_sum(s);
      dp = quad_sum(dp);
      float pr = expf(s * scale - Ls[r]);
      if (causal && krow > qt + r + off) pr = 0.f;
      const float ds = pr * (dp - Ds[r]);
#pragma unroll
      for (int t = 0; t < PT; ++t) {
        dv[t] += pr * dOs[r][4 * t + part];
        dk[t] += ds * Qs[r][4 * t + part];
      }
    }
  }
  if (valid) {
#pragma unroll
    for (int t = 0; t < PT; ++t) {
      const int d = 4 * t + part;
      if (d < D) {
        dK[(int64_t)krow * p.sdkn + (int64_t)d * p.sdkd] = dk[t] * scale;
        dV[(int64_t)krow * p.sdvn + (int64_t)d * p.sdvd] = dv[t];
      }
    }
  }
}

template <int DP>
static hipError_t launch_fwd_f32(const FwdParams& p, bool causal, bool varlen, float scale, hipStream_t s) {
  dim3 grid((p.Nq + 63) / 64, p.B * p.Hq);
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
    hipLaunchKernelGGL((fa_bwd_dq_f32_kernel<DP>), dim3((p.Nq + 63) / 64, p.B * p.H), dim3(256), 0, s, p,
                       (int)causal);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.Nk > 0) {
    hipLaunchKernelGGL((fa_bwd_dkdv_f32_kernel<DP>), dim3((p.Nk + 63) / 64, p.B * p.H), dim3(256), 0, s, p,
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
