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
//   fa_decode_mfma_kernel: group sizes other than 1, 2, 4, 8 (up to 32,
//     caches with blocks of 16 tokens or more); see below.
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
    // P V two tokens at a time on v_dot2 (each pair of V rows interleaved by
    // v_perm_b32, shared by the G heads), with p rounded to the input dtype
    // as the forward's PV operands are. The row sums stay fp32: the offset
    // is the exact running max, so the largest p is 1 and exact, and the
    // rounding moves O by at most ~2^-9 of |v| while L keeps fp32 accuracy.
    typedef __attribute__((ext_vector_type(2))) T T2;
#pragma unroll
    for (int u = 0; u < CH; u += 2) {
      T2 vp[8];  // (token u, token u+1) of dim e
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vp[2 * j] = __builtin_bit_cast(T2, __builtin_amdgcn_perm(vr[u + 1][j], vr[u][j], 0x05040100u));
        vp[2 * j + 1] = __builtin_bit_cast(T2, __builtin_amdgcn_perm(vr[u + 1][j], vr[u][j], 0x07060302u));
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p0 = fast_exp2(s[u][g] - m[g]);  // exp2(-inf) = 0 past the end
        const float p1 = fast_exp2(s[u + 1][g] - m[g]);
        const T2 pp = T2{(T)p0, (T)p1};
        l[g] += p0 + p1;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = dot2(pp, vp[e], acc[g][e]);
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

// MFMA decode for group sizes the lane-group kernel does not cover (up to 32
// query heads per KV head, caches whose block size is a multiple of 16): one
// workgroup per (sequence, KV head, split) as above, but the G query
// heads of the KV head are the columns of S^T = K Q^T and O^T += V^T P^T on
// v_mfma_f32_32x32x16 (q in registers, G <= 32 columns used), and K/V reach
// LDS through buffer_load ... lds, so bytes in flight do not cost registers.
// Each wave streams its own 32-token tiles of the split (tiles w, w+4, ...),
// two stages deep in its own LDS buffers: no workgroup barrier inside the
// loop. A tile is two 16-token pieces, each inside one cache block, so each
// piece takes one buffer descriptor built from one block-table entry (read
// one tile ahead by a scalar load). Each wave keeps an online softmax per
// column (exponent offset raised lazily, as in the forward); the waves merge
// through LDS at the end, and split partials go to the combine kernel.
template <typename T, int DP>
__global__ __launch_bounds__(256) void fa_decode_mfma_kernel(const DecodeParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int NW = 4, BT = 32;        // waves, tokens per wave tile
  constexpr int TB = BT * DP * 2;       // bytes of one K (or V) tile
  constexpr int CPT = TB / 1024;        // 1 KB direct-load chunks per tile
  constexpr int KSTEPS = DP / 16, DT = DP / 32;
  constexpr int STAGES = 2;
  constexpr int SMEM = NW * STAGES * 2 * TB;
  static_assert(CPT >= 2 && CPT % 2 == 0, "a tile is two 16-row pieces of whole chunks");
  static_assert(NW * BT * DP * 4 <= SMEM, "the merge reuses the tile buffers");
  constexpr float kThreshold = 8.0f;  // log2 units

  __shared__ __attribute__((aligned(1024))) char smem_raw[SMEM];
  __shared__ float st_m[NW][32], st_l[NW][32], st_le[NW][32];
  LDS_AS char* smem = (LDS_AS char*)smem_raw;

  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int G = p.Hq / p.Hkv;
  const int seq = min(max(p.seq_lens[b], 0), min(p.max_seq_len, p.max_blocks << p.block_shift));
  const int t0 = split * p.split_tokens;
  const int t1 = min(seq, t0 + p.split_tokens);
  const int ntile = t1 > t0 ? (t1 - t0 + BT - 1) / BT : 0;
  const int D = p.D;
  const float sl2 = p.scale_log2;

  // q as the B operand: lane holds column g = l32 (query head hk*G + g),
  // dims 16kk + 8hh .. +7; zero for g >= G and dims >= D.
  X8 qreg[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    u32x4 raw = {0, 0, 0, 0};
    if (l32 < G && col < D) raw = ldg16((const T*)p.q + (int64_t)b * p.sqb + (int64_t)(hk * G + l32) * p.sqh + col);
    qreg[kk] = __builtin_bit_cast(X8, raw);
  }

  // Direct-load lane offsets inside a 16-row piece (rows of a piece are the
  // cache slots of one block, sks/svs apart); columns at or past D read zero.
  int ko[CPT / 2], vo[CPT / 2];
#pragma unroll
  for (int c = 0; c < CPT / 2; ++c) {
    const int byte = c * 1024 + lane * 16;
    const int row = byte / (DP * 2);  // 0..15
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    ko[c] = seg * 8 < D ? (int)(row * p.sks * 2) + seg * 16 : (int)0x80000000;
    vo[c] = seg * 8 < D ? (int)(row * p.svs * 2) + seg * 16 : (int)0x80000000;
  }
  const __attribute__((address_space(4))) int32_t* table =
      (const __attribute__((address_space(4))) int32_t*)(p.block_tables + (int64_t)b * p.sbt);
  const int bmask = (1 << p.block_shift) - 1;
  // Block of the piece starting at token tok (-1 past the split).
  auto block_of = [&](int tok) -> int { return tok < t1 ? table[tok >> p.block_shift] : -1; };
  // (Captured arrays are read into locals before the builtin call: an array
  // element of a capture inside a builtin's argument list makes clang's host
  // pass silently drop the kernel's launch stub.)
  auto piece_load = [&](int tok, int blk, int kofs, int vofs) {
    LDS_AS char* kdst = smem + kofs;
    LDS_AS char* vdst = smem + vofs;
    const int rows = min(t1 - tok, 16);
    const bool live = rows > 0 && blk >= 0 && blk < p.num_blocks;
    const int slot = tok & bmask;
    const T* ks = (const T*)p.kc + (live ? (int64_t)blk * p.skb + (int64_t)slot * p.sks + (int64_t)hk * p.skh : 0);
    const T* vs = (const T*)p.vc + (live ? (int64_t)blk * p.svb + (int64_t)slot * p.svs + (int64_t)hk * p.svh : 0);
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(ks, live ? (int)(rows * p.sks * 2) : 0);
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(vs, live ? (int)(rows * p.svs * 2) : 0);
#pragma unroll
    for (int c = 0; c < CPT / 2; ++c) {
      const int kc = ko[c], vc = vo[c];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (LDS_AS void*)(kdst + c * 1024), 16, kc, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (LDS_AS void*)(vdst + c * 1024), 16, vc, 0, 0, 0);
    }
  };
  auto kofs = [&](int st) { return ((wave * STAGES + st) * 2) * TB; };
  auto vofs = [&](int st) { return ((wave * STAGES + st) * 2 + 1) * TB; };
  // Tile i of this wave covers tokens t0 + (i*NW + wave)*BT .. +31.
  auto tile_tok = [&](int i) { return t0 + (i * NW + wave) * BT; };
  const int nmine = ntile > wave ? (ntile - wave + NW - 1) / NW : 0;
  auto tile_load = [&](int i, int blk0, int blk1) {
    const int tok = tile_tok(i), st = i % STAGES;
    const int ko0 = kofs(st), vo0 = vofs(st);
    piece_load(tok, blk0, ko0, vo0);
    piece_load(tok + 16, blk1, ko0 + TB / 2, vo0 + TB / 2);
  };

  int koff[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) koff[kk] = swz_off<DP>(l32, 16 * kk + 8 * hh) * 2;
  const int tr_row = 4 * hh + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int voff[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    voff[dt][0] = swz_off<DP>(tr_row, 32 * dt + tr_col) * 2;
    voff[dt][1] = swz_off<DP>(tr_row + 8, 32 * dt + tr_col) * 2;
  }

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  // l_run: sum of the rounded p (normalises O); l_lse: fp32 sum (the lse).
  float m_run = -1e30f, l_run = 0.f, l_lse = 0.f;

  if (nmine > 0) tile_load(0, block_of(tile_tok(0)), block_of(tile_tok(0) + 16));
  if (nmine > 1) tile_load(1, block_of(tile_tok(1)), block_of(tile_tok(1) + 16));
  for (int i = 0; i < nmine; ++i) {
    // Block ids of tile i+2, read while tile i lands.
    const int nb0 = i + 2 < nmine ? block_of(tile_tok(i + 2)) : -1;
    const int nb1 = i + 2 < nmine ? block_of(tile_tok(i + 2) + 16) : -1;
    if (i + 1 < nmine)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * CPT) : "memory");  // tile i+1's loads may stay in flight
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int kso = kofs(i % STAGES), vso = vofs(i % STAGES);
    const LDS_AS char* Ks = smem + kso;
    const LDS_AS char* Vs = smem + vso;
    f32x16 s = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) s = mfma32(*(const LDS_AS X8*)(Ks + koff[kk]), qreg[kk], s);
    // Tokens past the split end (rows 8(i/4) + 4hh + i%4) are masked.
    const int lim = t1 - 1 - tile_tok(i) - 4 * hh;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (8 * (e >> 2) + (e & 3) > lim) s[e] = -INFINITY;
      mx = fmaxf(mx, s[e]);
    }
    mx = half_max(mx);
    const float mxs = mx == -INFINITY ? -INFINITY : mx * sl2;
    if (__builtin_amdgcn_ballot_w64(mxs > m_run + kThreshold) != 0) {
      const float m_new = fmaxf(m_run, mxs);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
      l_lse *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
    }
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = fast_exp2(fmaf(s[e], sl2, -m_run));
      l_lse += s[e];
    }
    X8 pb[2];
    pb[0] = pack8<T>(s, 0);
    pb[1] = pack8<T>(s, 8);
    sum8_into(pb[0], rs);
    sum8_into(pb[1], rs);
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const LDS_AS char* base = Vs + ks * 16 * DP * 2;
        const X8 a = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(base + voff[dt][0])),
                                  lds_read_tr((const LDS_AS T*)(base + voff[dt][1])));
        acc[dt] = mfma32(a, pb[ks], acc[dt]);
      }
    }
    // This stage's LDS reads are consumed before its next transfer is issued.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (i + 2 < nmine) tile_load(i + 2, nb0, nb1);
  }

  // Merge the waves: (m, l) per column through LDS, O^T rows through the
  // (now idle) tile buffers as [wave][column][DP] floats.
  const float lt = half_sum(l_run), le = half_sum(l_lse);
  __syncthreads();
  float* st_o = (float*)smem_raw;
  if (l32 < G) {
    if (hh == 0) {
      st_m[wave][l32] = nmine > 0 ? m_run : -INFINITY;
      st_l[wave][l32] = lt;
      st_le[wave][l32] = le;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st_o[(wave * 32 + l32) * DP + 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3)] = acc[dt][e];
  }
  __syncthreads();
  for (int idx = tid; idx < G * DP; idx += 256) {
    const int g = idx / DP, d = idx % DP;
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < NW; ++r)
      if (st_l[r][g] > 0.f) M = fmaxf(M, st_m[r][g]);
    float L = 0.f, LE = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int r = 0; r < NW; ++r) {
        if (st_l[r][g] > 0.f) {
          const float w = fast_exp2(st_m[r][g] - M);
          L += w * st_l[r][g];
          LE += w * st_le[r][g];
          O += w * st_o[(r * 32 + g) * DP + d];
        }
      }
    }
    const int h = hk * G + g;
    const float on = L > 0.f ? O / L : 0.f;
    const float lse2 = LE > 0.f ? M + __log2f(LE) : -INFINITY;  // log2 units
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

template <typename T, int DP>
static hipError_t launch_decode_mfma(const DecodeParams& p, hipStream_t s) {
  hipLaunchKernelGGL((fa_decode_mfma_kernel<T, DP>), dim3(p.num_splits, p.Hkv, p.B), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  hipLaunchKernelGGL((fa_decode_combine_kernel<T, DP>), dim3(p.Hq, p.B), dim3(DP), 0, s, p);
  return hipGetLastError();
}

// Host entry used by the C ABI layer (arguments already validated): dp is 64
// or 128. Group sizes 1, 2, 4 and 8 take the lane-group kernel (any block
// size); other group sizes up to 32 take the MFMA kernel (block sizes that
// are multiples of 16). The lane-group kernel keeps more K/V bytes in flight
// per CU (in registers, at high occupancy) than the MFMA kernel can in LDS,
// so it is the faster one where both apply.
hipError_t decode_gqa(const DecodeParams& p, bool is_bf16, int dp, hipStream_t s) {
  if (decode_uses_mfma(p.Hq / p.Hkv, p.block_shift)) {
    if (is_bf16) return dp == 64 ? launch_decode_mfma<__bf16, 64>(p, s) : launch_decode_mfma<__bf16, 128>(p, s);
    return dp == 64 ? launch_decode_mfma<_Float16, 64>(p, s) : launch_decode_mfma<_Float16, 128>(p, s);
  }
  if (is_bf16) return dp == 64 ? dispatch_decode_g<__bf16, 64>(p, s) : dispatch_decode_g<__bf16, 128>(p, s);
  return dp == 64 ? dispatch_decode_g<_Float16, 64>(p, s) : dispatch_decode_g<_Float16, 128>(p, s);
}

}  // namespace lsfa
