// Shared device-side helpers for the gfx950 FlashAttention kernels.
//
// Register layouts used throughout (checked on MI355X with an in-bounds lane
// probe of the builtins):
//   v_mfma_f32_32x32x16_{bf16,f16}  C[32x32] += A[32x16] * B[16x32]
//     A: lane l holds A[l%32][8*(l/32) + s], s = 0..7
//     B: lane l holds B[8*(l/32) + s][l%32]
//     C: lane l, register i holds C[8*(i/4) + 4*(l/32) + i%4][l%32]
//   ds_read_b64_tr_b16: inside each group of 16 lanes, lane 4r+e receives, in
//     slot j, element e of the 8 bytes addressed by lane 4j+r of the group.
//   v_permlane32_swap(a, b): lanes 32..63 of a trade places with lanes 0..31
//     of b, so max(r[0], r[1]) of swap(x, x) reduces x across the two halves.
//
// Every kernel computes transposed score tiles S^T = K Q^T (or S = Q K^T in the
// key-stationary backward) so that an accumulator can be converted in
// registers into the B operand of the next MFMA; the matching A operand is
// then read from LDS with the transpose read above.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lsfa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

template <typename T> struct VecT;
template <> struct VecT<__bf16> { using x8 = bf16x8; using x4 = bf16x4; };
template <> struct VecT<_Float16> { using x8 = f16x8; using x4 = f16x4; };

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Transposed 8-byte LDS read (see header comment for the lane mapping).
// Transposed 4 x 16-bit LDS read. The pointer is __restrict__ so that, once
// inlined, the read carries its own alias scope: the compiler then no longer
// waits for every outstanding global->LDS (buffer_load ... lds) transfer
// before it, which it otherwise does because it cannot tell which LDS bytes
// those transfers write. Callers order such transfers against the reads that
// need them with an explicit s_waitcnt vmcnt(0) and a barrier.
__device__ __forceinline__ bf16x4 lds_read_tr(const LDS_AS __bf16* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LDS_AS bf16x4*)p);
}
typedef __fp16 fp16x4_builtin __attribute__((__vector_size__(4 * sizeof(__fp16))));
__device__ __forceinline__ f16x4 lds_read_tr(const LDS_AS _Float16* __restrict__ p) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS fp16x4_builtin*)p));
}

template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 lds_read8(const LDS_AS T* p) {
  return *(const LDS_AS typename VecT<T>::x8*)p;
}

template <typename X8, typename X4>
__device__ __forceinline__ X8 cat4(X4 a, X4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Eight consecutive accumulator registers -> one bf16/f16 MFMA operand (RNE).
template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 pack8(const f32x16& c, int base) {
  typename VecT<T>::x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (T)c[base + s];
  return r;
}

// acc + sum of the 8 elements of a bf16/f16 operand (four v_dot2 with 1.0).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_ones(bf16x2 v, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(v, one, acc, false);
}
__device__ __forceinline__ float dot2_ones(f16x2 v, float acc) {
  const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(v, one, acc, false);
}
template <typename X8>
__device__ __forceinline__ void sum8_into(const X8& v, float (&acc)[4]) {
  acc[0] = dot2_ones(__builtin_shufflevector(v, v, 0, 1), acc[0]);
  acc[1] = dot2_ones(__builtin_shufflevector(v, v, 2, 3), acc[1]);
  acc[2] = dot2_ones(__builtin_shufflevector(v, v, 4, 5), acc[2]);
  acc[3] = dot2_ones(__builtin_shufflevector(v, v, 6, 7), acc[3]);
}

// All-reduce across the two 32-lane halves of a wave.
__device__ __forceinline__ float half_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte segment swizzle of LDS tiles stored [rows][DP]. Rows r..r+15 read
// at one segment (K operand, ds_read_b128) and 4-row x 32-byte blocks
// (transpose reads) both land on distinct banks (64 banks of 4 bytes, i.e.
// 16 segment slots per 256 bytes). With 256-byte rows (DP = 128) every row
// starts at slot 0, so the 16 rows need 16 distinct swizzles. With 128-byte
// rows (DP = 64) rows alternate between slots 0..7 and 8..15, so rows of one
// parity need 8 distinct swizzles, and rows 4q and 4q + 2 (and 4q + 1, 4q + 3)
// must differ in bit 2 so that their 32-byte transpose-read spans do not
// meet: swizzle = bit-rotated (row / 2) % 8. With 64-byte rows (DP = 32) four
// rows share 256 bytes; rows r and r + 4 need distinct swizzles.
template <int DP>
__device__ __forceinline__ int seg_swz(int row) {
  if constexpr (DP == 64) {
    const int e = (row >> 1) & 7;
    return ((e & 1) << 2) | (e >> 1);
  }
  return (((row & 3) << 2) | ((row >> 2) & 3)) & (DP / 8 - 1);
}
// Element offset of (row, col) inside a swizzled [rows][DP] LDS tile; col%8
// is preserved, so 8- and 16-byte accesses stay contiguous.
template <int DP>
__device__ __forceinline__ int swz_off(int row, int col) {
  return row * DP + ((((col >> 3) ^ seg_swz<DP>(row))) << 3) + (col & 7);
}

// Kernel-side argument block (filled by the host dispatcher from the C ABI
// structs; all strides in elements).
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t sqb, sqh, sqn;
  int64_t skb, skh, skn;
  int64_t svb, svh, svn;
  int64_t sob, soh, son;
  int64_t slb, slh, sln;
  int64_t sqd, skd, svd, sod;  // head-dim strides (fp32 path only; 1 on the MFMA path)
  const int32_t* cu_q;
  const int32_t* cu_k;
  // Paged K/V (chunked prefill against a KV cache): k/v are the caches
  // [num_blocks, block_size, Hkv, D] with skb/svb the block stride, skn/svn
  // the slot stride and skh/svh the head stride; keys per sequence come from
  // seq_lens_k and their blocks from block_tables [B, max_blocks].
  const int32_t* block_tables;
  const int32_t* seq_lens_k;
  int64_t sbt;  // block-table row stride
  int block_shift, max_blocks, num_blocks;
  int B, Hq, Hkv, Nq, Nk, D;
  int num_q_tiles;
  int heads_per_group;  // map_tile grouping
  float scale_log2;  // |sm_scale| * log2(e), at least 1e-30
  int neg_q;         // sm_scale < 0: q is negated on load so scale_log2 stays positive
};

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  void* dq;
  void* dk;
  void* dv;
  // Workspace written by the dq kernel's prologue:
  //   ld  : per (b, h) at b*sldb + h*sldh, blocks of 64 queries: 64 values of
  //         lse * log2(e), then 64 of -delta (query q's at 128 (q / 64) + q % 64
  //         and 64 further); +inf stands in for lse where a row sees no key or
  //         q >= Nq. The fp32 kernels keep (lse * log2(e), delta) pairs, query
  //         q's at 2q.
  float* ld;
  int64_t sldb, sldh;
  int nq_pad;  // Nq rounded up to the query-stationary tile (128)
  // Stored-dS path: dS^T rows (input dtype) of heads bh0 .. bh0 + nbh - 1,
  // element (key n, query m) of head bh at (bh - bh0) * ds_sbh + n * ds_ldq + m
  void* ds;
  int64_t ds_sbh, ds_ldq;
  int bh0, nbh;
  int64_t sqb, sqh, sqn;
  int64_t skb, skh, skn;
  int64_t svb, svh, svn;
  int64_t sob, soh, son;
  int64_t sdob, sdoh, sdon;
  int64_t sdqb, sdqh, sdqn;
  int64_t sdkb, sdkh, sdkn;
  int64_t sdvb, sdvh, sdvn;
  int64_t slb, slh, sln;
  int64_t sqd, skd, svd, sod, sdod, sdqd, sdkd, sdvd;  // fp32 path only
  int B, H, Nq, Nk, D;
  int G;             // query heads per KV head (GQA: query head h reads KV head h / G)
  // Varlen (packed [tokens, heads, d] rows; Nq / Nk are the longest
  // sequences): sequence b's rows are cu_q[b] .. cu_q[b+1]-1 (cu_k for keys)
  const int32_t* cu_q;
  const int32_t* cu_k;
  int num_tiles;     // tiles per (b, h) along the kernel's stationary axis
  int heads_per_group;  // map_tile grouping
  float scale;       // sm_scale
  float scale_log2;  // sm_scale * log2(e)
};

// Paged-KV decode (one query token per sequence); strides in elements.
constexpr int kDecodeMaxTableSlots = 512;  // block-table entries one split may span

// Skinny GEMM y[M, N] = x[M, K] @ W[K, N] (M <= 8; element strides; W rows
// contiguous). partial: fp32 workspace [splits][M][N].
struct GemvParams {
  // Up to four weight matrices sharing x and K; their columns are numbered
  // one after another (matrix g holds columns col_off[g] .. col_off[g+1]-1 of
  // a virtual y of N = col_off[groups] columns).
  const void* x;
  const void* xg;  // optional gate: the product reads bf16/fp16(silu(xg) * x), as torch rounds it
  int64_t sxg;
  const void* w[4];
  void* y[4];
  int64_t sw[4], sy[4];
  int col_off[5];
  int groups;
  float* partial;  // [splits][M][N] fp32 (splits > 1)
  int* counters;   // 16 per 256-column block, zero on entry and on exit (splits > 1)
  int64_t sx;
  int M, K, N;
  int kc, splits;  // K-range per split and the number of splits
  // Optional RMSNorm of the input (nw non-null): the products read
  // rmsnorm(x + nr) * nw as fused_add_rmsnorm computes it; the workgroup
  // (0, 0) writes h = x + nr to nh when nh is non-null.
  const void* nw;
  const void* nr;
  void* nh;
  int64_t snr, snh;
  float eps;
};

// Which decode kernel serves a group size Hq/Hkv and block size 2^shift: the
// lane-group kernel for groups 1, 2, 4, 8; the MFMA kernel for other groups
// (up to 32) with blocks of at least 16 tokens.
inline __host__ __device__ bool decode_uses_mfma(int group, int block_shift) {
  return block_shift >= 4 && group != 1 && group != 2 && group != 4 && group != 8;
}
struct DecodeParams {
  const void* q;       // [B, Hq, D]
  const void* kc;      // [num_blocks, block_size, Hkv, D]
  const void* vc;
  void* o;             // [B, Hq, D]
  float* lse;          // [B, Hq] or null
  const int32_t* block_tables;  // [B, max_blocks]
  const int32_t* seq_lens;      // [B]
  float* o_part;       // [B, Hq, num_splits, DP] (split path)
  float* lse_part;     // [B, Hq, num_splits]
  int64_t sqb, sqh;
  int64_t skb, sks, skh;  // k cache: block, slot, head strides
  int64_t svb, svs, svh;
  int64_t sob, soh;
  int64_t slb, slh;
  int64_t sbt;            // block table row stride
  int B, Hq, Hkv, D;
  int block_shift;        // log2(block_size)
  int max_blocks;         // block-table entries per sequence
  int num_blocks;         // blocks in the cache; other ids read as zero
  int max_seq_len;        // sequences are clamped to min(this, max_blocks * block_size)
  int num_splits, split_tokens;  // split_tokens is a multiple of 16
  float scale_log2;       // sm_scale * log2(e)
};

// In-place rotary embedding of q [B, Hq, N, D] and k [B, Hkv, N, D]
// (element strides in b, h, n, d order; packed [tokens, h, d] when
// cu_seqlens is set, then strides[0] is unused and strides[2] is the token
// stride). cos/sin: [max_pos, D] rows of the input dtype.
struct RopeParams {
  void* q;
  void* k;                     // null when Hkv == 0
  const void* cos;
  const void* sin;
  const int32_t* pos0;         // [B] position of each sequence's first token, or null (0)
  const int32_t* cu_seqlens;   // [B + 1] or null
  int64_t sq[4], sk[4];
  int64_t table_stride;
  int B, N, Hq, Hkv, D, max_pos;
  // Optional K/V cache append: rotated k and v rows of token t go to slot
  // slots[t] (skipped outside [0, num_slots)).
  const void* v;
  void* k_cache;
  void* v_cache;
  const int64_t* slots;
  int64_t sv[4];
  int64_t cs_slot, cs_head, num_slots;
  const int32_t* block_tables;  // or slots from the block table and the token's position
  int64_t sbt;
  int block_size, max_blocks;
};

// Fused residual add + RMSNorm over rows of a [rows, cols] matrix (column
// stride 1, row strides in elements). residual and residual_out may be null.
struct NormParams {
  const void* x;
  const void* residual;
  const void* weight;
  void* out;
  void* residual_out;
  int64_t sx, sr, so, sh;
  int rows, cols;
  float eps;
};

// Maps the 1-D launch index to (batch*head, tile). Workgroups are handed to
// the 8 XCDs round-robin by launch index, so consecutive launch indices are
// spread so that each XCD owns a contiguous run of heads (their operands stay
// in that XCD's L2). Within a run, heads go in groups of heads_per_group and
// each group's tiles are issued heaviest-first across the whole group (largest
// causal extent first: all its heads' heaviest tiles, then the next level):
// the late, light tiles of one group overlap the heavy ones of the next, so
// the grid's tail is short, while a group's streamed operands (a few MB)
// stay in L2.
__device__ __forceinline__ void map_tile(int num_tiles, int total, int heads_per_group, int& bh, int& tile,
                                         bool heavy_last_index) {
  const int L = blockIdx.x;
  int W = L;
  if ((total & 7) == 0) W = (L & 7) * (total >> 3) + (L >> 3);
  const int BH = total / num_tiles;
  const int hg = max(heads_per_group, 1);
  const int g0 = (W / (hg * num_tiles)) * hg;  // first head of W's group
  const int gh = min(hg, BH - g0);             // heads in the group
  const int rr = W - g0 * num_tiles;
  const int level = rr / gh;
  bh = g0 + (rr - level * gh);
  tile = heavy_last_index ? (num_tiles - 1 - level) : level;
}

// Heads per map_tile group: as many as keep a group's streamed operands
// (bytes_per_head each: K and V for the query-stationary kernels, Q and dO
// for the key-stationary one) within ~8 MiB, i.e. two XCD L2s, at most 16.
inline int heads_per_group_for(long long bytes_per_head) {
  const long long g = bytes_per_head > 0 ? (8LL << 20) / bytes_per_head : 16;
  return (int)(g < 1 ? 1 : (g > 16 ? 16 : g));
}

__device__ __forceinline__ u32x4 ldg16(const void* p) { return *(const u32x4*)p; }

// Raw buffer descriptor over [base, base + bytes): loads at or past the end
// return zero, and a size below zero is taken as zero (every load returns
// zero). Callers pass wave-uniform values; readfirstlane keeps the size in a
// scalar register even where the compiler computed it with VALU ops (a
// vector descriptor would turn every load into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int bytes) {
  const int n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n > 0 ? n : 0, 0x00020000);
}

// Buffer accesses as device functions (the host compilation pass then
// never meets the builtins inside a kernel's lambdas): a 16-byte-per-lane
// direct global -> LDS load, and 16- / 4-byte stores (lanes whose offset
// falls outside the descriptor are dropped).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, LDS_AS void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void store16(u32x4 v, __amdgpu_buffer_rsrc_t rs, int voff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, 0, 0);
}
__device__ __forceinline__ void store4(float v, __amdgpu_buffer_rsrc_t rs, int voff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, voff, 0, 0);
}

}  // namespace lsfa
