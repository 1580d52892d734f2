// Paged-KV decode attention for gfx950 (one new query token per sequence).
//
// The reference's engine keeps per-request block tables of physical KV-cache
// block ids (engine/block_manager.py:56-60: table entry i holds tokens
// [i*block_size, (i+1)*block_size)) and documents the missing kernel: decode
// needs Nq = 1 against a paged Nkv, gathering K/V across the block table
// (engine/README.md, "No decode-shaped attention kernel"; engine/request.py
// is_prefill). A block holds block_size x n_kv_heads x head_dim elements per
// layer for K and for V (engine/config.py:5-7); here the cache tensors are
// [num_blocks, block_size, Hkv, D] with element strides.
//
// The path is HBM-bound (each K/V byte is used by Hq/Hkv query heads: about
// 4 FLOP per byte), so the kernel is built around coalesced streaming:
//   fa_decode_split_kernel: one workgroup per (sequence, KV head, split of
//     the sequence). With D = 128 a wave reads 4 tokens per load
//     instruction: lane (tq, c) = (lane / 16, lane % 16) loads 16 bytes
//     (8 dims) of token tq, so a token's 256-byte row is one contiguous
//     16-lane access. Each lane keeps q for its 8 dims and all G = Hq/Hkv
//     query heads in registers, partial dot products are summed across the
//     16 lanes with butterfly shuffles, and every lane group runs its own
//     online softmax over its tokens (exponent offset raised per 4-token
//     chunk). The split's block-table slice is staged in LDS first. Lane
//     groups merge with shuffles, waves through LDS.
//   fa_decode_combine_kernel: when a sequence is split, merges the splits'
//     normalised partial outputs with their logsumexps.
// K/V rows are read with nontemporal loads: each byte is used once per step.
#include "fa_common.hpp"

namespace lsfa {

constexpr float kDecLn2 = 0.6931471805599453f;

// Sum over the DP/8 lanes that hold one token's row, left in every one of
// them, with DPP row operations (VALU, no LDS round trip). 16-lane groups:
// rotations by 8, 4, 2, 1 within the row. 8-lane groups: mirror within the
// half row, then swaps within quads.
__device__ __forceinline__ float dpp_add(float x, int ctrl_sel) {
  int v = __float_as_int(x);
  int r;
  switch (ctrl_sel) {
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false); break;  // row_ror:8
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false); break;  // row_ror:4
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false); break;  // row_ror:2
    case 3: r = __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false); break;  // row_ror:1
    case 4: r = __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false); break;  // row_half_mirror
    case 5: r = __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false); break;   // quad_perm [2,3,0,1]
    default: r = __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false); break;  // quad_perm [1,0,3,2]
  }
  return x + __int_as_float(r);
}

template <int DP>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (DP == 128) {
    x = dpp_add(x, 0);
    x = dpp_add(x, 1);
    x = dpp_add(x, 2);
    x = dpp_add(x, 3);
  } else {
    x = dpp_add(x, 4);
    x = dpp_add(x, 5);
    x = dpp_add(x, 6);
  }
  return x;
}

__device__ __forceinline__ float dot2(bf16x2 a, bf16x2 b, float c) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false); }
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
// a . b over 8 bf16/f16 elements (fp32 accumulate). The pairs are taken with
// explicit shuffles: bit-casting single 32-bit lanes of a u32x4 to a 2-element
// vector was miscompiled (every pair read the same register).
template <typename X8>
__device__ __forceinline__ float dot8(const X8& a, const X8& b) {
  float d = dot2(__builtin_shufflevector(a, a, 0, 1), __builtin_shufflevector(b, b, 0, 1), 0.f);
  d = dot2(__builtin_shufflevector(a, a, 2, 3), __builtin_shufflevector(b, b, 2, 3), d);
  d = dot2(__builtin_shufflevector(a, a, 4, 5), __builtin_shufflevector(b, b, 4, 5), d);
  return dot2(__builtin_shufflevector(a, a, 6, 7), __builtin_shufflevector(b, b, 6, 7), d);
}

template <typename T, int DP, int G>
__global__ __launch_bounds__(256) void fa_decode_split_kernel(const DecodeParams p) {
  using X8 = typename VecT<T>::x8;
  constexpr int LPT = DP / 8;    // lanes per token row (16 B each)
  constexpr int TPW = 64 / LPT;  // tokens per wave per load instruction
  constexpr int NW = 4;
  constexpr int TPI = NW * TPW;  // tokens per workgroup per load instruction
  constexpr int CH = 4;          // tokens per lane group between offset updates

  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane % LPT, tq = lane / LPT;
  const int seq = min(max(p.seq_lens[b], 0), min(p.max_seq_len, p.max_blocks << p.block_shift));
  const int t0 = split * p.split_tokens;
  const int t1 = min(seq, t0 + p.split_tokens);

  __shared__ int s_blk[kDecodeMaxTableSlots];
  __shared__ float st_m[NW][G], st_l[NW][G];
  __shared__ float st_o[NW][G][DP];

  // The split's slice of the block table (the host keeps it within
  // kDecodeMaxTableSlots entries).
  const int first_slot = t0 >> p.block_shift;
  const int n_slots = t1 > t0 ? ((t1 - 1) >> p.block_shift) - first_slot + 1 : 0;
  const int32_t* table = p.block_tables + (int64_t)b * p.sbt + first_slot;
  for (int i = tid; i < n_slots; i += 256) s_blk[i] = table[i];

  // q of the G query heads of this KV head, dims 8c..8c+7 (scores via
  // v_dot2, fp32 accumulate; the scale is applied after).
  X8 qp[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = hk * G + g;
    u32x4 raw = {0, 0, 0, 0};
    if (8 * c < p.D) raw = ldg16((const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh + 8 * c);
    qp[g] = __builtin_bit_cast(X8, raw);
  }
  const float sl2 = p.scale_log2;
  __syncthreads();

  float m[G], l[G], acc[G][8];  // m in log2 units of scaled scores
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  const T* kbase = (const T*)p.kc + (int64_t)hk * p.skh + 8 * c;
  const T* vbase = (const T*)p.vc + (int64_t)hk * p.svh + 8 * c;
  const bool col_ok = 8 * c < p.D;
  const int bmask = (1 << p.block_shift) - 1;

  // Every lane group (wave, tq) walks its own tokens in chunks of CH; the
  // loads of the next chunk are in flight while the current one is used.
  auto load_chunk = [&](int tb, u32x4* kr, u32x4* vr) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int t = tb + u * TPI;
      kr[u] = u32x4{0, 0, 0, 0};
      vr[u] = u32x4{0, 0, 0, 0};
      const int blk = t < t1 ? s_blk[(t >> p.block_shift) - first_slot] : -1;
      if (t < t1 && col_ok && (unsigned)blk < (unsigned)p.num_blocks) {
        const int slot = t & bmask;
        kr[u] = __builtin_nontemporal_load((const u32x4*)(kbase + (int64_t)blk * p.skb + (int64_t)slot * p.sks));
        vr[u] = __builtin_nontemporal_load((const u32x4*)(vbase + (int64_t)blk * p.svb + (int64_t)slot * p.svs));
      }
    }
  };
  auto use_chunk = [&](int tb, const u32x4* kr, const u32x4* vr) {
    float s[CH][G];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const bool ok = tb + u * TPI < t1;
      const X8 kx = __builtin_bit_cast(X8, kr[u]);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = group_sum<DP>(dot8(qp[g], kx));
        s[u][g] = ok ? d * sl2 : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < CH; ++u) mx = fmaxf(mx, s[u][g]);
      if (mx > m[g]) {  // uniform within the lane group
        const float alpha = fast_exp2(m[g] - mx);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
        m[g] = mx;
      }
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const X8 vv = __builtin_bit_cast(X8, vr[u]);
      float vf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) vf[e] = (float)vv[e];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pv = fast_exp2(s[u][g] - m[g]);  // exp2(-inf) = 0 past the end
        l[g] += pv;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pv, vf[e], acc[g][e]);
      }
    }
  };
  u32x4 ka[CH], va[CH], kb[CH], vb[CH];
  int tb = t0 + wave * TPW + tq;
  if (tb < t1) load_chunk(tb, ka, va);
  while (tb < t1) {
    const int tn = tb + CH * TPI;
    if (tn < t1) load_chunk(tn, kb, vb);
    use_chunk(tb, ka, va);
    if (tn >= t1) break;
    const int tn2 = tn + CH * TPI;
    if (tn2 < t1) load_chunk(tn2, ka, va);
    use_chunk(tn, kb, vb);
    tb = tn2;
  }

  // Merge the wave's TPW lane groups (lanes with equal c) with shuffles, then
  // the NW waves through LDS. States are (m, l, acc) in log2 units; an empty
  // state has m = -inf and contributes weight 0.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = m[g];
#pragma unroll
    for (int msk = LPT; msk < 64; msk <<= 1) M = fmaxf(M, __shfl_xor(M, msk));
    const float w = M == -INFINITY ? 0.f : fast_exp2(m[g] - M);
    float L = w * l[g];
#pragma unroll
    for (int msk = LPT; msk < 64; msk <<= 1) L += __shfl_xor(L, msk);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float o = w * acc[g][e];
#pragma unroll
      for (int msk = LPT; msk < 64; msk <<= 1) o += __shfl_xor(o, msk);
      acc[g][e] = o;
    }
    if (lane == 0) {
      st_m[wave][g] = M;
      st_l[wave][g] = L;
    }
    if (tq == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) st_o[wave][g][8 * c + e] = acc[g][e];
    }
  }
  __syncthreads();

  for (int idx = tid; idx < G * DP; idx += 256) {
    const int g = idx / DP, d = idx % DP;
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < NW; ++r) M = fmaxf(M, st_m[r][g]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int r = 0; r < NW; ++r) {
        const float w = fast_exp2(st_m[r][g] - M);
        L += w * st_l[r][g];
        O += w * st_o[r][g][d];
      }
    }
    const int h = hk * G + g;
    const float on = L > 0.f ? O / L : 0.f;
    const float lse2 = L > 0.f ? M + __log2f(L) : -INFINITY;  // log2 units
    if (p.num_splits == 1) {
      if (d < p.D) ((T*)p.o)[(int64_t)b * p.sob + (int64_t)h * p.soh + d] = (T)on;
      if (d == 0 && p.lse != nullptr) p.lse[(int64_t)b * p.slb + (int64_t)h * p.slh] = lse2 * kDecLn2;
    } else {
      const int64_t row = ((int64_t)b * p.Hq + h) * p.num_splits + split;
      p.o_part[row * DP + d] = on;
      if (d == 0) p.lse_part[row] = lse2;
    }
  }
}

// Merges the splits of one (sequence, query head): o = sum_s w_s o_s / sum_s
// w_s with w_s = 2^(lse_s - max lse); lse = max + log2(sum w) (log2 units in
// the workspace, natural log in the output). The splits' lse values are
// staged in LDS (batches of kCombineBatch, one load per thread, merged with a
// running max), and the partial rows are read eight splits at a time so that
// their loads are in flight together.
constexpr int kCombineBatch = 512;

template <typename T, int DP>
__global__ __launch_bounds__(DP) void fa_decode_combine_kernel(const DecodeParams p) {
  constexpr int U = 8;
  __shared__ float s_w[kCombineBatch];
  __shared__ float s_red[DP / 64];
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t row0 = ((int64_t)b * p.Hq + h) * p.num_splits;
  const int seq = min(max(p.seq_lens[b], 0), min(p.max_seq_len, p.max_blocks << p.block_shift));
  const int ns = min(p.num_splits, (seq + p.split_tokens - 1) / p.split_tokens);
  float M = -INFINITY, W = 0.f, O = 0.f;
  for (int c0 = 0; c0 < ns; c0 += kCombineBatch) {
    const int cn = min(kCombineBatch, ns - c0);
    __syncthreads();  // s_w and s_red of the previous batch are consumed
    float mx = -INFINITY;
    for (int s = d; s < cn; s += DP) {
      const float v = p.lse_part[row0 + c0 + s];
      s_w[s] = v;
      mx = fmaxf(mx, v);
    }
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) mx = fmaxf(mx, __shfl_xor(mx, msk));
    if ((d & 63) == 0) s_red[d >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < DP / 64; ++w) mx = fmaxf(mx, s_red[w]);
    const float Mn = fmaxf(M, mx);
    if (Mn == -INFINITY) continue;  // nothing visible so far
    const float a = fast_exp2(M - Mn);  // 0 while M is still -inf
    W *= a;
    O *= a;
    M = Mn;
    for (int s0 = 0; s0 < cn; s0 += U) {
      float o[U];
#pragma unroll
      for (int u = 0; u < U; ++u) o[u] = s0 + u < cn ? p.o_part[(row0 + c0 + s0 + u) * DP + d] : 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (s0 + u < cn) {
          const float w = fast_exp2(s_w[s0 + u] - M);
          W += w;
          O += w * o[u];
        }
      }
    }
  }
  if (d < p.D) ((T*)p.o)[(int64_t)b * p.sob + (int64_t)h * p.soh + d] = (T)(W > 0.f ? O / W : 0.f);
  if (d == 0 && p.lse != nullptr)
    p.lse[(int64_t)b * p.slb + (int64_t)h * p.slh] = W > 0.f ? (M + __log2f(W)) * kDecLn2 : -INFINITY;
}

template <typename T, int DP, int G>
static hipError_t launch_decode(const DecodeParams& p, hipStream_t s) {
  hipLaunchKernelGGL((fa_decode_split_kernel<T, DP, G>), dim3(p.num_splits, p.Hkv, p.B), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  hipLaunchKernelGGL((fa_decode_combine_kernel<T, DP>), dim3(p.Hq, p.B), dim3(DP), 0, s, p);
  return hipGetLastError();
}

template <typename T, int DP>
static hipError_t dispatch_decode_g(const DecodeParams& p, hipStream_t s) {
  switch (p.Hq / p.Hkv) {
    case 1: return launch_decode<T, DP, 1>(p, s);
    case 2: return launch_decode<T, DP, 2>(p, s);
    case 4: return launch_decode<T, DP, 4>(p, s);
    case 8: return launch_decode<T, DP, 8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Host entry used by the C ABI layer (arguments already validated): dp is 64
// or 128; the group size Hq/Hkv is 1, 2, 4 or 8.
hipError_t decode_gqa(const DecodeParams& p, bool is_bf16, int dp, hipStream_t s) {
  if (is_bf16) return dp == 64 ? dispatch_decode_g<__bf16, 64>(p, s) : dispatch_decode_g<__bf16, 128>(p, s);
  return dp == 64 ? dispatch_decode_g<_Float16, 64>(p, s) : dispatch_decode_g<_Float16, 128>(p, s);
}

}  // namespace lsfa
