// FlashAttention forward for gfx950: bf16/fp16 operands on
// v_mfma_f32_32x32x16, fp32 online softmax in base 2.
//
// Algorithm (same per-tile order as kernels/flash_attention.py:121-179 and
// kernels/flash_attention_backward.py:129-169): for each key tile, scores are
// computed and scaled, masked to -inf (key beyond the sequence, or causal),
// the running row max is raised, p = exp(s - m) and alpha = exp(m_old - m),
// l = alpha*l + sum(p), acc = alpha*acc + p(cast to the input dtype) @ V; at
// the end o = acc / l and lse = m + ln(l). One difference in bookkeeping, not
// in the result: the exponent offset m is the first tile's row max and is
// only raised where p would come near the input dtype's range (above 2^64 for
// bf16, whose exponent range is fp32's, or 2^15 for fp16), so most tiles need
// neither a row max nor a rescale of acc; m + log(l) is unchanged by the
// choice of offset. A tile's exponentials are computed with the current
// offset and their row sums checked before the PV products use them: a sum
// above the limit (rare: scores above the first tile's max by more than 44 /
// 10 natural-log units) sends the tile through the row max, the rescale and
// its exponentials again.
//
// Work decomposition
//   workgroup = 4 waves = 128 query rows of one (batch, head); wave w owns
//   rows 32w..32w+31, one row per lane pair (l, l+32). At most 256 registers
//   per wave, so two workgroups share a CU and the hardware interleaves one
//   wave's softmax with the other's MFMA work on each SIMD. Long dense
//   sequences and varlen batches with long query runs take 8-wave
//   workgroups (256 rows, one per CU), which halve the K/V bytes streamed
//   into LDS per query row.
//   K/V tiles of 64 keys go global -> LDS with buffer_load ... lds (no
//   register staging; rows past the sequence read as zero through the buffer
//   range check), double-buffered, 16-byte segments XOR-swizzled per row.
//   S^T = K Q^T on MFMA (A = K rows from LDS, B = Q held in registers), so
//   every lane owns one query row: the row max/sum need one permlane32 swap.
//   The fp32 S^T accumulator is rounded in registers into the B operand of
//   O^T += V^T P^T; V^T comes from LDS through ds_read_b64_tr_b16.
//
// Paged K/V (PAGED, with packed varlen queries): the keys of sequence b are
// its seq_lens_k[b] cache slots, found through its block-table row. A 64-key
// tile is loaded as one 16-row (4 waves) or 8-row (8 waves) piece per wave;
// with block sizes that are multiples of 16 each piece lies inside one cache
// block, so every wave
// builds one buffer descriptor per tile from one block-table entry and the
// LDS tile is the same as for contiguous K/V. Block ids outside
// [0, num_blocks) read as zeros.
#include "fa_common.hpp"
#include <atomic>
#include <type_traits>

namespace lsfa {

constexpr float kLn2 = 0.6931471805599453f;
// Largest log2 of p the PV operands may carry: a row's offset is raised once
// its scores (in log2 units) exceed it by more than this.
template <typename T> constexpr float kMaxLog2P = 64.0f;
template <> constexpr float kMaxLog2P<_Float16> = 15.0f;

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Number of a sequence's query tiles (tq of them, BM rows each) whose key
// tile count (64 keys each) exceeds x; the tiles counted are always the last
// ones, as causal work grows with the tile index. x = -1 counts every tile.
template <bool CAUSAL, int BM>
__device__ __forceinline__ int tiles_above(int x, int tq, int nk, int off) {
  if (x < 0) return tq;
  if (tq == 0 || nk <= 64 * x) return 0;  // the last tile sees all nk keys
  if (!CAUSAL) return tq;
  // tile t < tq-1 sees off + BM(t+1) keys: more than 64x iff t >= (64x-off)/BM
  const long long y = 64LL * x - off;
  return y < 0 ? tq : 1 + max(0, tq - 1 - (int)(y / BM));
}

// Longest-first order of a varlen launch's (sequence, query tile) items, so
// that each XCD starts its longest workgroups first and the short ones fill
// the tail: returns the item of the given rank (rank 0 has the most key
// tiles; ties go by sequence, then tile), or b = -1 past the last item.
// Lane i holds sequence i (B <= 64). The key tile count of the item at the
// rank is found by binary search on the number of items above a count, then
// the item among those of that count by a prefix sum over the sequences.
// Wave-uniform result.
template <bool CAUSAL, bool PAGED, int BM>
__device__ __forceinline__ void varlen_item_at(const FwdParams& p, int rank, int lane, int& b_out, int& qt_out) {
  int tq = 0, nk = 0, off = 0;
  if (lane < p.B) {
    const int nq = p.cu_q[lane + 1] - p.cu_q[lane];
    nk = PAGED ? min(max(p.seq_lens_k[lane], 0), p.max_blocks << p.block_shift)
               : p.cu_k[lane + 1] - p.cu_k[lane];
    tq = nq > 0 ? (nq + BM - 1) / BM : 0;
    off = nk - nq;
  }
  b_out = -1;
  qt_out = 0;
  if (rank >= wave_sum_i(tq)) return;
  int kmax = nk > 0 ? (nk + 63) >> 6 : 0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, __shfl_xor(kmax, o));
  int lo = 0, hi = __builtin_amdgcn_readfirstlane(kmax);  // no item exceeds hi
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (__builtin_amdgcn_readfirstlane(wave_sum_i(tiles_above<CAUSAL, BM>(mid, tq, nk, off))) <= rank) hi = mid;
    else lo = mid + 1;
  }
  // rank lies among the items of exactly lo key tiles: tiles
  // [tq - above(lo-1), tq - above(lo)) of each sequence.
  const int a_hi = tiles_above<CAUSAL, BM>(lo - 1, tq, nk, off);
  const int a_lo = tiles_above<CAUSAL, BM>(lo, tq, nk, off);
  const int c = a_hi - a_lo;
  const int k = rank - __builtin_amdgcn_readfirstlane(wave_sum_i(a_lo));
  int inc = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  const int pre = inc - c;
  const unsigned long long hit = __ballot(c > 0 && k >= pre && k < pre + c);
  const int src = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));
  b_out = src;
  qt_out = __builtin_amdgcn_readfirstlane(__shfl(tq - a_hi + k - pre, src));
}

// NW waves per workgroup (NW x 32 query rows): 4 (two workgroups per CU) or,
// for long dense sequences and varlen batches with long query runs,
// 8 (one per CU), so that every K/V tile brought into LDS serves twice the
// rows.
template <typename T, int DP, bool CAUSAL, bool VARLEN, bool LSE, bool PAGED, int NW>
__global__ __launch_bounds__((NW * 64), (8 / NW)) void fa_fwd_kernel(const FwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int BM = NW * 32, BN = 64;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  constexpr int TILE = BN * DP;              // elements of one K or V tile
  constexpr int LDI = TILE * 2 / 1024 / NW;  // 1 KB direct loads per wave per tile
  constexpr int KSTEPS = DP / 16;
  constexpr int DT = DP / 32;
  constexpr int KB = BN / 32;
  static_assert(LDI >= 1, "tile too small for the workgroup");
  static_assert(!PAGED || VARLEN, "paged K/V takes packed varlen queries");
  constexpr int RPW = LDI * 1024 / (DP * 2);  // tile rows each wave loads
  // Paged: a wave's rows must lie in one cache block (blocks hold 16 or more
  // tokens, a power of two).
  static_assert(!PAGED || (RPW * DP * 2 == LDI * 1024 && (RPW == 8 || RPW == 16)), "rows per wave");
  // Dense 8-wave launches: the second wave of each SIMD (waves 4-7) issues
  // the whole tile, 2 LDI chunks each, and waves 0-3 issue none (0.7-2%
  // faster at the config-3/4 shapes than every wave issuing LDI: a wave
  // stalls while the CU's load path takes its chunks, and waves 0-3, which
  // win the SIMD's issue arbitration, then run on). Paged launches keep one
  // cache block per wave's rows, so every wave loads there.
  constexpr bool kSecondLoads = NW == 8 && !PAGED;
  constexpr int LDC = kSecondLoads ? 2 * LDI : LDI;  // 1 KB chunks this wave issues per tile

  __shared__ __attribute__((aligned(1024))) T smem_raw[4 * TILE];  // K0 K1 V0 V1
  LDS_AS T* smem = (LDS_AS T*)smem_raw;
  const LDS_AS char* sbytes = (const LDS_AS char*)smem_raw;
  LDS_AS char* smem_bytes = (LDS_AS char*)smem_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31, hh = lane >> 5;
  const bool loads = !kSecondLoads || wave >= NW / 2;  // wave-uniform
  const int lw = kSecondLoads ? (wave & (NW / 2 - 1)) : wave;  // this wave's chunk group
  int b, h, qt;
  if (VARLEN && p.B <= 64) {
    // Varlen sequences differ in length: workgroup L takes the item of rank
    // L / Hq in longest-first order, for head slot L % Hq. Workgroups go to
    // the XCDs round-robin, so with Hq a multiple of 8 XCD x gets slots
    // x, x+8, ..., mapped to the adjacent heads x*Hq/8 .. (with GQA, query
    // heads that share K/V), every rank in order.
    const int L = blockIdx.x;
    const int rank = L / p.Hq, u = L - rank * p.Hq;
    h = (p.Hq & 7) == 0 ? (u & 7) * (p.Hq >> 3) + (u >> 3) : u;
    varlen_item_at<CAUSAL, PAGED, BM>(p, rank, lane, b, qt);
    if (b < 0) return;  // uniform, before any barrier
  } else {
    int bh;
    map_tile(p.num_q_tiles, gridDim.x, p.heads_per_group, bh, qt, CAUSAL);
    // Longer varlen batches: the (sequence, head) index runs head-major, so
    // each XCD's contiguous run of indices holds a few heads of every
    // sequence instead of all heads of one sequence.
    b = VARLEN ? bh % p.B : bh / p.Hq;
    h = VARLEN ? bh / p.B : bh - b * p.Hq;
  }
  const int hk = h / (p.Hq / p.Hkv);
  int nq = p.Nq, nk = p.Nk;
  int64_t rq0 = 0, rk0 = 0;
  if (VARLEN) {
    rq0 = p.cu_q[b];
    nq = p.cu_q[b + 1] - (int)rq0;
    if (PAGED) {
      nk = min(max(p.seq_lens_k[b], 0), p.max_blocks << p.block_shift);
    } else {
      rk0 = p.cu_k[b];
      nk = p.cu_k[b + 1] - (int)rk0;
    }
  }
  const int q0 = qt * BM;
  if (q0 >= nq) return;  // uniform across the workgroup, before any barrier
  const int off = nk - nq;  // bottom-right causal alignment

  const T* Q = (const T*)p.q + (VARLEN ? 0 : (int64_t)b * p.sqb) + (int64_t)h * p.sqh + rq0 * p.sqn;
  const T* K = PAGED ? (const T*)p.k
                     : (const T*)p.k + (VARLEN ? 0 : (int64_t)b * p.skb) + (int64_t)hk * p.skh + rk0 * p.skn;
  const T* V = PAGED ? (const T*)p.v
                     : (const T*)p.v + (VARLEN ? 0 : (int64_t)b * p.svb) + (int64_t)hk * p.svh + rk0 * p.svn;
  T* O = (T*)p.o + (VARLEN ? 0 : (int64_t)b * p.sob) + (int64_t)h * p.soh + rq0 * p.son;

  int kv_end = nk;
  if (CAUSAL) kv_end = min(nk, q0 + BM + off);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  const int D = p.D;
  const int qw_lo = q0 + wave * 32;
  const int qrow = qw_lo + l32;
  const float sl2 = p.scale_log2;  // > 0 (the host folds a negative scale into neg_q)

  // Q as the B operand of S^T = K Q^T: lane holds row qrow, columns
  // 16kk + 8hh .. +7; zero outside the sequence / head dim.
  X8 qreg[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const int col = 16 * kk + 8 * hh;
    u32x4 raw = {0, 0, 0, 0};
    if (qrow < nq && col < D) raw = ldg16(Q + (int64_t)qrow * p.sqn + col);
    if (p.neg_q) raw ^= 0x80008000u;
    qreg[kk] = __builtin_bit_cast(X8, raw);
  }

  // Direct global -> LDS tile load: a loading wave with chunk group g issues
  // LDC 1 KB chunks; lane t of chunk c lands at tile byte (g*LDC + c)*1024 + 16t
  // = (row, swizzled seg). The buffer descriptor is rebuilt per tile (scalar
  // work) and clipped to the rows that exist, so the per-lane byte offsets
  // are loop-invariant and rows at or past nk (and columns at or past D) read
  // as zero. Paged offsets are relative to the wave's first row.
  int kvo[LDC], vvo[LDC];
#pragma unroll
  for (int c = 0; c < LDC; ++c) {
    const int byte = (lw * LDC + c) * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    const int r = PAGED ? row - RPW * wave : row;
    kvo[c] = seg * 8 < D ? (int)(r * p.skn * 2) + seg * 16 : (int)0x80000000;
    vvo[c] = seg * 8 < D ? (int)(r * p.svn * 2) + seg * 16 : (int)0x80000000;
  }
  // Paged: the cache block holding this wave's RPW rows of tile j (-1 past
  // the sequence). The table is read through the constant address space (it
  // does not change during a launch), so the wave-uniform read is one scalar
  // load into an SGPR, issued one pipelined iteration before the tile load
  // that uses it; it completes under the previous iteration's closing waits.
  auto block_of = [&](int j) -> int {
    if (!PAGED) return 0;
    const int key0 = j * BN + RPW * wave;  // wave-uniform
    if (key0 >= nk) return -1;
    const __attribute__((address_space(4))) int32_t* bt = (const __attribute__((address_space(4))) int32_t*)p.block_tables;
    return bt[(int64_t)b * p.sbt + (key0 >> p.block_shift)];
  };
  auto tile_load = [&](const T* base, int64_t sn, int64_t sblk, int64_t shead, const int* vo, int j, int buf,
                       int blk) {
    if (!loads) return;
    __amdgpu_buffer_rsrc_t rs;
    if (PAGED) {
      const int key0 = j * BN + RPW * wave;  // wave-uniform
      const int rows = min(nk - key0, RPW);
      blk = __builtin_amdgcn_readfirstlane(blk);
      const bool live = rows > 0 && blk >= 0 && blk < p.num_blocks;
      const int slot = key0 & ((1 << p.block_shift) - 1);
      const T* src = live ? base + (int64_t)blk * sblk + (int64_t)slot * sn + (int64_t)hk * shead : base;
      rs = tile_rsrc(src, live ? (int)(rows * sn * 2) : 0);
    } else {
      const int rows = min(nk - j * BN, BN);
      rs = tile_rsrc(base + (int64_t)j * BN * sn, (int)(rows * sn * 2));
    }
    LDS_AS char* dst = (LDS_AS char*)(smem + buf * TILE);
#pragma unroll
    for (int c = 0; c < LDC; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(dst + (lw * LDC + c) * 1024), 16, vo[c], 0, 0, 0);
  };

  // Per-lane LDS byte offsets relative to a tile base. The swizzle depends
  // only on row & 15, so the 32-row key block and 16-row steps are immediates.
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
  // l_run: the sum O is normalised by (bf16: of the rounded p the PV products
  // take, so the weights of the V rows sum to one exactly; fp16: of the fp32
  // p); l_lse: sum of the fp32 p (for the logsumexp output, as the
  // reference's l_i).
  float m_run = -1e30f, l_run = 0.f, l_lse = 0.f;
  const float kTileSumMax = __builtin_exp2f(kMaxLog2P<T>);

  // K tile t lives in buffer t&1 (smem + (t&1)*TILE), V tile t in 2 + (t&1).
  auto kbuf = [&](int t) { return sbytes + (t & 1) * TILE * 2; };
  auto vbuf = [&](int t) { return sbytes + (2 + (t & 1)) * TILE * 2; };

  // LDS operand reads run this many MFMAs ahead of the MFMA that takes them
  // (the compiler's own order reads only one or two ahead, so every pair of
  // MFMAs waited out a full LDS latency).
  constexpr int kReadAhead = 4;
  // S^T = K Q^T for one tile (fp32, unscaled).
  auto scores = [&](const LDS_AS char* Ks, f32x16* s) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s[kb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const X8 a = *(const LDS_AS X8*)(Ks + kb * 32 * DP * 2 + koff[kk]);
        s[kb] = mfma32(a, qreg[kk], s[kb]);
      }
    }
    constexpr int NM = KSTEPS * KB;
#pragma unroll
    for (int i = 0; i < kReadAhead; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // K reads
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA j
      if (j + kReadAhead < NM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  // Row max of a tile in log2 units (both lane halves hold the row's keys).
  auto row_max = [&](const f32x16* s) -> float {
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = half_max(mx);
    return mx == -INFINITY ? -INFINITY : mx * sl2;
  };
  // Exponentials with the current offset, rounded to the input dtype into
  // the PV operands; returns this lane's part of the tile's row sums: x = the
  // sum O is normalised by, y = the fp32 p with LSE (four interleaved partial
  // sums), else 0. s is left as it is. For bf16, x sums the rounded p
  // (v_dot2 with ones), so that O's weights sum to one exactly (8-bit
  // mantissas: normalising by the fp32 sum fails the max-abs gate when one
  // large p dominates a row). fp16 keeps 11 bits, so the fp32 sum moves O by
  // at most ~2^-11 |v|; it is used for x as well, which drops the 16 v_dot2
  // per tile (a v_dot2 holds up the other wave's MFMAs on the SIMD).
  auto softmax = [&](const f32x16* s, X8* pb) -> float2 {
    constexpr bool kF16 = std::is_same<T, _Float16>::value;
    const float neg_m = -m_run;
    // The partial sums start at -0, the additive identity, so that the
    // first add of each folds away (+0 would not: +0 + -0 is +0).
    float rs[4] = {-0.f, -0.f, -0.f, -0.f}, re[4] = {-0.f, -0.f, -0.f, -0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      f32x16 p;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = fast_exp2(fmaf(s[kb][i], sl2, neg_m));
        if constexpr (LSE || kF16) re[i & 3] += p[i];
      }
      pb[2 * kb] = pack8<T>(p, 0);
      pb[2 * kb + 1] = pack8<T>(p, 8);
      if constexpr (!kF16) {
        sum8_into(pb[2 * kb], rs);
        sum8_into(pb[2 * kb + 1], rs);
      }
    }
    float2 r;
    r.y = (LSE || kF16) ? (re[0] + re[1]) + (re[2] + re[3]) : 0.f;
    r.x = kF16 ? r.y : (rs[0] + rs[1]) + (rs[2] + rs[3]);
    return r;
  };
  auto add_sums = [&](float2 ts) {
    l_run += ts.x;
    if constexpr (LSE) l_lse += ts.y;
  };
  // The exponentials of a tile, checked: if some row's sum passes the limit
  // (a p above 2^kMaxLog2P, or inf; wave-uniform branch, taken on few tiles),
  // that row's offset rises to its max in this tile, O and l rescale in
  // place, and the exponentials are computed again.
  auto softmax_checked = [&](const f32x16* s, X8* pb) {
    float2 ts = softmax(s, pb);
    if (__builtin_amdgcn_ballot_w64(ts.x > kTileSumMax) != 0) {
      const float mx = row_max(s);
      if (__builtin_amdgcn_ballot_w64(mx > m_run) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        l_run *= alpha;
        if constexpr (LSE) l_lse *= alpha;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      }
      ts = softmax(s, pb);
    }
    add_sums(ts);
  };
  // O^T += V^T P^T with V^T from transpose reads.
  auto pv = [&](const LDS_AS char* Vs, const X8* pb) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int ks = 0; ks < 2 * KB; ++ks) {
        const LDS_AS char* base = Vs + ks * 16 * DP * 2;
        const X8 a = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(base + voff[dt][0])),
                                  lds_read_tr((const LDS_AS T*)(base + voff[dt][1])));
        acc[dt] = mfma32(a, pb[ks], acc[dt]);
      }
    }
    constexpr int NM = DT * 2 * KB;
#pragma unroll
    for (int i = 0; i < kReadAhead; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // V^T reads
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA j
      if (j + kReadAhead < NM) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };

  // Every key tile runs software-pipelined: while the MFMAs of S for tile t+1
  // issue, the VALU computes tile t's exponentials (with the first tile's
  // offset and the overflow check), then tile t's PV MFMAs issue. A wave
  // skips the tiles it cannot see (causal: keys past its last row's
  // diagonal) and, before their exponentials, masks to -inf the scores of
  // the tiles it sees in part (the diagonal, the sequence end), so that
  // their p are exactly 0. Buffers: K tile t+2 and V tile t+1 load while
  // tile t is processed (K runs one tile ahead of V).
  auto wave_sees = [&](int j) { return !CAUSAL || j * BN <= qw_lo + 31 + off; };
  auto mask_tile = [&](int j, f32x16* s) {
    const int kbase = j * BN;
    if ((kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > qw_lo + off)) {
      // (the empty volatile asm keeps this a branch: the selects below would
      // otherwise be hoisted out of it and run on every tile)
      asm volatile("" ::: "memory");
      int lim = nk - 1 - kbase - 4 * hh;
      if (CAUSAL) lim = min(lim, qrow + off - kbase - 4 * hh);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s[kb][i] = 32 * kb + 8 * (i >> 2) + (i & 3) > lim ? -INFINITY : s[kb][i];
    }
  };

  // blk1, blk2: blocks of tiles t+1 and t+2 for the next pipelined step t.
  const int blk0 = block_of(0);
  int blk1 = block_of(1), blk2 = block_of(2);
  if (ntiles > 0) {
    tile_load(K, p.skn, p.skb, p.skh, kvo, 0, 0, blk0);
    tile_load(V, p.svn, p.svb, p.svh, vvo, 0, 2, blk0);
  }
  if (ntiles > 1) tile_load(K, p.skn, p.skb, p.skh, kvo, 1, 1, blk1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // The offset starts at the first tile's row max (rows that see none of its
  // keys keep -1e30: their first visible tile then takes the check's slow
  // path, which raises the offset to that tile's max).
  f32x16 s0[KB], s1[KB];
  if (ntiles > 0 && wave_sees(0)) {
    scores(kbuf(0), s0);
    mask_tile(0, s0);
    m_run = fmaxf(row_max(s0), -1e30f);
  }
  __syncthreads();  // K buffer 0 is refilled by the first step
  // One pipelined step: tile t's scores are in cur, tile t+1's go to nxt.
  // The V load of dense launches is issued after the S MFMAs: each wave's
  // direct loads queue behind the whole workgroup's in the CU's load path
  // (issuing all of a step's loads at its start stalled every wave for
  // ~400 cycles), and V tile t+1 is first needed one step later.
  auto pipe_step = [&](int t, f32x16* cur, f32x16* nxt) {
    if (t + 2 < ntiles) tile_load(K, p.skn, p.skb, p.skh, kvo, t + 2, t & 1, blk2);
    if (PAGED && t + 1 < ntiles) tile_load(V, p.svn, p.svb, p.svh, vvo, t + 1, 2 + ((t + 1) & 1), blk1);
    if (t + 1 < ntiles && wave_sees(t + 1)) {
      scores(kbuf(t + 1), nxt);
      mask_tile(t + 1, nxt);
    }
    if (!PAGED && t + 1 < ntiles) tile_load(V, p.svn, p.svb, p.svh, vvo, t + 1, 2 + ((t + 1) & 1), blk1);
    if (wave_sees(t)) {
      X8 pb[2 * KB];
      softmax_checked(cur, pb);
      pv(vbuf(t), pb);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (PAGED) {
      // The next step's block id is read after this step's last LDS read:
      // an outstanding scalar load holds up every LDS wait issued after it,
      // so here its latency only overlaps the barrier's own wait.
      blk1 = blk2;
      blk2 = block_of(t + 3);
    }
    __syncthreads();
  };
  int j = 0;
  for (; j + 1 < ntiles; j += 2) {
    pipe_step(j, s0, s1);
    pipe_step(j + 1, s1, s0);
  }
  if (j < ntiles) pipe_step(j, s0, s1);

  const float lt = half_sum(l_run);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  // O leaves through LDS: a lane's accumulators hold 4-column pieces of one
  // query's row, so direct stores would scatter 8-byte pieces over 32 rows
  // per instruction. Each wave writes its 32 rows (swizzled 16-byte
  // segments) into its own LDS region, reads them back row-major and stores
  // 16 bytes per lane, four whole rows per instruction. The last step's
  // closing barrier has retired every K/V read.
  {
    constexpr int BLK = 32 * DP * 2;  // bytes of one wave's 32 rows
    static_assert(NW * BLK <= 4 * TILE * 2, "O staging fits in the K/V buffers");
    LDS_AS char* wb = smem_bytes + wave * BLK;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        X4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)(acc[dt][4 * g + e] * inv);
        *(LDS_AS X4*)(wb + swz_off<DP>(l32, 32 * dt + 8 * g + 4 * hh) * 2) = v;
      }
#pragma unroll
    for (int c = 0; c < BLK / 1024; ++c) {
      const int byte = c * 1024 + lane * 16;
      const int row = byte / (DP * 2), seg = (byte % (DP * 2)) / 16;
      const X8 v = *(const LDS_AS X8*)(wb + row * DP * 2 + ((seg ^ seg_swz<DP>(row)) << 4));
      const int q = qw_lo + row;
      if (q < nq && seg * 8 < D) *(X8*)(O + (int64_t)q * p.son + seg * 8) = v;
    }
  }
  if (qrow < nq) {
    if constexpr (LSE) {
      const float le = half_sum(l_lse);
      if (hh == 0) {
        float* L = p.lse + (VARLEN ? 0 : (int64_t)b * p.slb) + (int64_t)h * p.slh + (rq0 + qrow) * p.sln;
        *L = le > 0.f ? (m_run + __log2f(le)) * kLn2 : -INFINITY;
      }
    }
  }
}

// Items one persistent forward workgroup may take (its LDS item table), and
// the fewest per workgroup for which the fixed split beats the hardware's
// own dispatch of one workgroup per item (measured: 8 per workgroup -2.4%,
// 4 per workgroup -0.5 to -1.1%, 4.5 even, 2.1 per workgroup +31%, where a
// fixed split of so few causal items leaves a long tail).
constexpr int kPersistMaxItems = 64;
constexpr int kPersistMinItems = 4;

// Persistent dense forward: one 8-wave workgroup per CU walks a fixed list
// of (batch, head, 256-row query tile) items, so the per-workgroup start
// (Q rows, the first K/V tiles, the first score tile) overlaps the previous
// item's work instead of idling the CU. The K/V tiles of consecutive items
// form one stream through the double buffer: during an item's last step the
// next item's first K and V tiles load and its first score tile is computed.
// Each wave's next Q rows wait in its own LDS region (loaded during the
// item's first step), which also stages the wave's O rows on the way out.
// Items: the launch's (b, h, tile) list in map_tile's order; workgroup u of
// the PU on XCD x takes, from XCD x's share, positions i PU + u (i even) and
// i PU + PU - 1 - u (i odd), so heavy and light causal tiles pair up.
// Requires (host-checked): dense, 8-wave shapes, Nk > 64, Nk >= Nq when
// causal (every item has at least two key tiles), total items % 8 == 0.
template <typename T, int DP, bool CAUSAL, bool LSE>
__global__ __launch_bounds__(512, 1) void fa_fwd_persist_kernel(const FwdParams p) {
  using X8 = typename VecT<T>::x8;
  using X4 = typename VecT<T>::x4;
  constexpr int NW = 8, BM = NW * 32, BN = 64;
  constexpr int TILE = BN * DP;              // elements of one K or V tile
  constexpr int LDI = TILE * 2 / 1024 / NW;  // 1 KB loads per wave per tile
  constexpr int LDC = 2 * LDI;               // issued by waves 4-7 only
  constexpr int KSTEPS = DP / 16, DT = DP / 32, KB = BN / 32;
  constexpr int QB = 32 * DP * 2;  // bytes of one wave's 32 rows of Q or O
  constexpr int QC = QB / 1024;
  static_assert(LDI >= 1 && QC >= 1, "tile too small for the workgroup");

  // K0 K1 V0 V1 | each wave's Q / O rows | the workgroup's item table
  __shared__ __attribute__((aligned(1024))) char sm_raw[4 * TILE * 2 + NW * QB + kPersistMaxItems * 64];
  LDS_AS char* smb = (LDS_AS char*)sm_raw;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const bool loads = wave >= NW / 2;
  const int lw = wave & (NW / 2 - 1);
  const int nq = p.Nq, nk = p.Nk, off = nk - nq, D = p.D;
  const float sl2 = p.scale_log2;
  LDS_AS char* qst = smb + 4 * TILE * 2 + wave * QB;
  // Arguments used only when an item starts or ends are re-read from the
  // kernel argument segment there (scalar loads through an opaque pointer),
  // instead of occupying scalar registers across the whole loop.
  typedef const __attribute__((address_space(4))) FwdParams* KArgs;
  auto kargs = [&]() __attribute__((always_inline)) -> KArgs {
    KArgs pk = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(pk));
    return pk;
  };

  // The workgroup's items, in order: item i is position j = i PU + u (i
  // even) or i PU + PU - 1 - u (i odd) of XCD x's share of the launch's
  // (b, h, tile) list in map_tile's order. Lane i of wave 0 decodes item i
  // into a 64-byte LDS record {b, h, q0, key tiles | K, V, Q, O, L head
  // pointers} once, before the loop; nt = 0 past the last item.
  struct Item {
    int b, h, q0, nt;
    const T* k;
    const T* v;
  };
  LDS_AS char* itab = smb + 4 * TILE * 2 + NW * QB;
  if (wave == 0) {
    const int xcd = blockIdx.x & 7, u = blockIdx.x >> 3, PU = gridDim.x >> 3;
    const int nqt = p.num_q_tiles, BH = p.B * p.Hq, T8 = (nqt * BH) >> 3;
    const int hg = max(p.heads_per_group, 1);
    const int i = lane;
    const int j = i * PU + ((i & 1) ? PU - 1 - u : u);
    u32x4 r0 = {0u, 0u, 0u, 0u};
    const T *kh = nullptr, *vh = nullptr, *qh = nullptr, *oh = nullptr;
    const float* lh = nullptr;
    if (i < kPersistMaxItems && j < T8) {
      const int W = xcd * T8 + j;
      const int g0 = (W / (hg * nqt)) * hg;
      const int gh = min(hg, BH - g0);
      const int rr = W - g0 * nqt;
      const int level = rr / gh;
      const int bh = g0 + (rr - level * gh);
      const int qt = CAUSAL ? nqt - 1 - level : level;
      const int b = bh / p.Hq, h = bh - b * p.Hq, hk = h / (p.Hq / p.Hkv);
      const int q0 = qt * BM;
      const int kv_end = CAUSAL ? min(nk, q0 + BM + off) : nk;
      r0 = u32x4{(uint32_t)b, (uint32_t)h, (uint32_t)q0, (uint32_t)((kv_end + BN - 1) / BN)};
      kh = (const T*)p.k + (int64_t)b * p.skb + (int64_t)hk * p.skh;
      vh = (const T*)p.v + (int64_t)b * p.svb + (int64_t)hk * p.svh;
      qh = (const T*)p.q + (int64_t)b * p.sqb + (int64_t)h * p.sqh;
      oh = (const T*)p.o + (int64_t)b * p.sob + (int64_t)h * p.soh;
      if (LSE) lh = p.lse + (int64_t)b * p.slb + (int64_t)h * p.slh;
    }
    if (i < kPersistMaxItems) {
      LDS_AS char* rec = itab + i * 64;
      *(LDS_AS u32x4*)rec = r0;
      *(LDS_AS uint64_t*)(rec + 16) = (uint64_t)kh;
      *(LDS_AS uint64_t*)(rec + 24) = (uint64_t)vh;
      *(LDS_AS uint64_t*)(rec + 32) = (uint64_t)qh;
      *(LDS_AS uint64_t*)(rec + 40) = (uint64_t)oh;
      *(LDS_AS uint64_t*)(rec + 48) = (uint64_t)lh;
    }
  }
  __syncthreads();
  // Scalar copies of an item record's fields (uniform LDS reads).
  auto rec_int = [&](int i, int f) __attribute__((always_inline)) -> int {
    return __builtin_amdgcn_readfirstlane(*(const LDS_AS int*)(itab + i * 64 + 4 * f));
  };
  auto rec_ptr = [&](int i, int off) __attribute__((always_inline)) -> const void* {
    const uint64_t v = *(const LDS_AS uint64_t*)(itab + i * 64 + off);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(((uint64_t)hi << 32) | lo);
  };
  auto item_at = [&](int i) __attribute__((always_inline)) -> Item {
    Item it{0, 0, 0, 0, nullptr, nullptr};
    if (i >= kPersistMaxItems) return it;
    it.b = rec_int(i, 0);
    it.h = rec_int(i, 1);
    it.q0 = rec_int(i, 2);
    it.nt = rec_int(i, 3);
    it.k = (const T*)rec_ptr(i, 16);
    it.v = (const T*)rec_ptr(i, 24);
    return it;
  };

  // K/V tile loads (waves 4-7, two chunk groups each; see fa_fwd_kernel).
  int kvo[LDC], vvo[LDC];
#pragma unroll
  for (int c = 0; c < LDC; ++c) {
    const int byte = (lw * LDC + c) * 1024 + lane * 16;
    const int row = byte / (DP * 2);
    const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
    kvo[c] = seg * 8 < D ? (int)(row * p.skn * 2) + seg * 16 : (int)0x80000000;
    vvo[c] = seg * 8 < D ? (int)(row * p.svn * 2) + seg * 16 : (int)0x80000000;
  }
  // This wave's 32 Q rows of an item into its LDS region (row-major,
  // swizzled; rows past nq and columns past D read as zero).
  auto q_load = [&](int i, const Item& it) __attribute__((always_inline)) {
    const int r0 = it.q0 + 32 * wave;
    const KArgs pk = kargs();
    const int64_t sqn = pk->sqn;
    const T* src = (const T*)rec_ptr(i, 32) + (int64_t)r0 * sqn;
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(src, (int)(min(nq - r0, 32) * sqn * 2));
    int ln = lane;  // opaque: the offsets below are recomputed here, not held across the loop
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      const int byte = c * 1024 + ln * 16;
      const int row = byte / (DP * 2);
      const int seg = ((byte % (DP * 2)) / 16) ^ seg_swz<DP>(row);
      const int vo = seg * 8 < D ? (int)(row * sqn * 2) + seg * 16 : (int)0x80000000;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDS_AS void*)(qst + c * 1024), 16, vo, 0, 0, 0);
    }
  };
  X8 qreg[KSTEPS];
  auto q_read = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      u32x4 raw = *(const LDS_AS u32x4*)(qst + swz_off<DP>(l32, 16 * kk + 8 * hh) * 2);
      if (p.neg_q) raw ^= 0x80008000u;
      qreg[kk] = __builtin_bit_cast(X8, raw);
    }
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
  float m_run = -1e30f, l_run = 0.f, l_lse = 0.f;
  const float kTileSumMax = __builtin_exp2f(kMaxLog2P<T>);
  auto kbuf = [&](int t) __attribute__((always_inline)) { return (const LDS_AS char*)smb + (t & 1) * TILE * 2; };
  auto vbuf = [&](int t) __attribute__((always_inline)) { return (const LDS_AS char*)smb + (2 + (t & 1)) * TILE * 2; };

  constexpr int kReadAhead = 4;
  auto scores = [&](const LDS_AS char* Ks, f32x16* s) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s[kb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const X8 a = *(const LDS_AS X8*)(Ks + kb * 32 * DP * 2 + koff[kk]);
        s[kb] = mfma32(a, qreg[kk], s[kb]);
      }
    }
    constexpr int NM = KSTEPS * KB;
#pragma unroll
    for (int i = 0; i < kReadAhead; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (j + kReadAhead < NM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  auto row_max = [&](const f32x16* s) __attribute__((always_inline)) -> float {
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kb][i]);
    mx = half_max(mx);
    return mx == -INFINITY ? -INFINITY : mx * sl2;
  };
  auto softmax = [&](const f32x16* s, X8* pb) __attribute__((always_inline)) -> float2 {
    constexpr bool kF16 = std::is_same<T, _Float16>::value;
    const float neg_m = -m_run;
    float rs[4] = {-0.f, -0.f, -0.f, -0.f}, re[4] = {-0.f, -0.f, -0.f, -0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      f32x16 pp;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pp[i] = fast_exp2(fmaf(s[kb][i], sl2, neg_m));
        if constexpr (LSE || kF16) re[i & 3] += pp[i];
      }
      pb[2 * kb] = pack8<T>(pp, 0);
      pb[2 * kb + 1] = pack8<T>(pp, 8);
      if constexpr (!kF16) {
        sum8_into(pb[2 * kb], rs);
        sum8_into(pb[2 * kb + 1], rs);
      }
    }
    float2 r;
    r.y = (LSE || kF16) ? (re[0] + re[1]) + (re[2] + re[3]) : 0.f;
    r.x = kF16 ? r.y : (rs[0] + rs[1]) + (rs[2] + rs[3]);
    return r;
  };
  auto softmax_checked = [&](const f32x16* s, X8* pb) __attribute__((always_inline)) {
    float2 ts = softmax(s, pb);
    if (__builtin_amdgcn_ballot_w64(ts.x > kTileSumMax) != 0) {
      const float mx = row_max(s);
      if (__builtin_amdgcn_ballot_w64(mx > m_run) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        l_run *= alpha;
        if constexpr (LSE) l_lse *= alpha;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      }
      ts = softmax(s, pb);
    }
    l_run += ts.x;
    if constexpr (LSE) l_lse += ts.y;
  };
  auto pv = [&](const LDS_AS char* Vs, const X8* pb) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int ks = 0; ks < 2 * KB; ++ks) {
        const LDS_AS char* base = Vs + ks * 16 * DP * 2;
        const X8 a = cat4<X8, X4>(lds_read_tr((const LDS_AS T*)(base + voff[dt][0])),
                                  lds_read_tr((const LDS_AS T*)(base + voff[dt][1])));
        acc[dt] = mfma32(a, pb[ks], acc[dt]);
      }
    }
    constexpr int NM = DT * 2 * KB;
#pragma unroll
    for (int i = 0; i < kReadAhead; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (j + kReadAhead < NM) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  // qlo: the first of this wave's 32 query rows in the item.
  auto wave_sees = [&](int qlo, int j) __attribute__((always_inline)) { return !CAUSAL || j * BN <= qlo + 31 + off; };
  auto mask_tile = [&](int qlo, int j, f32x16* s) __attribute__((always_inline)) {
    const int kbase = j * BN;
    if ((kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > qlo + off)) {
      asm volatile("" ::: "memory");
      int lim = nk - 1 - kbase - 4 * hh;
      if (CAUSAL) lim = min(lim, qlo + l32 + off - kbase - 4 * hh);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s[kb][i] = 32 * kb + 8 * (i >> 2) + (i & 3) > lim ? -INFINITY : s[kb][i];
    }
  };
  // O (and L) of an item: through this wave's LDS region, four whole rows
  // per store instruction.
  // An item ends in two parts. finish_stage (its last step): O / l goes
  // into this wave's LDS region as the input dtype, and L into a register.
  // finish_store (the start of the next step, so that the global stores
  // complete under that step's work): the rows leave LDS row-major, four
  // whole rows per store instruction, through buffer stores clipped to the
  // rows that exist (rows past nq and columns past D are dropped).
  float lpend = 0.f;
  int st_item = 0, st_qlo = 0;
  bool st_due = false;
  auto finish_stage = [&](int qlo) __attribute__((always_inline)) {
    const float lt = half_sum(l_run);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    // Lane-dependent offsets come from an opaque copy of the lane id, so
    // that the compiler computes them here instead of keeping them in
    // registers across the whole loop.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int l32o = ln & 31, hho = ln >> 5;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        X4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)(acc[dt][4 * g + e] * inv);
        *(LDS_AS X4*)(qst + swz_off<DP>(l32o, 32 * dt + 8 * g + 4 * hho) * 2) = v;
      }
    if constexpr (LSE) {
      const float le = half_sum(l_lse);
      lpend = le > 0.f ? (m_run + __log2f(le)) * kLn2 : -INFINITY;
    }
  };
  auto finish_store = [&]() __attribute__((always_inline)) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const KArgs pk = kargs();
    const int64_t son = pk->son;
    const int rows = min(nq - st_qlo, 32);
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc((const T*)rec_ptr(st_item, 40) + (int64_t)st_qlo * son, (int)(rows * son * 2));
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      const int byte = c * 1024 + ln * 16;
      const int row = byte / (DP * 2), seg = (byte % (DP * 2)) / 16;
      const u32x4 v = *(const LDS_AS u32x4*)(qst + row * DP * 2 + ((seg ^ seg_swz<DP>(row)) << 4));
      store16(v, rs, seg * 8 < D ? (int)(row * son * 2) + seg * 16 : (int)0x80000000);
    }
    if constexpr (LSE) {
      const int64_t sln = pk->sln;
      const __amdgpu_buffer_rsrc_t lr = tile_rsrc((const float*)rec_ptr(st_item, 48) + (int64_t)st_qlo * sln, (int)(rows * sln * 4));
      store4(lpend, lr, (ln >> 5) == 0 ? (int)((ln & 31) * sln * 4) : (int)0x80000000);
    }
  };

  int item = 0;
  Item cur = item_at(0);
  if (cur.nt == 0) return;  // uniform, before any barrier
  Item nxt = item_at(1);
  int qlo = cur.q0 + 32 * wave;
  // Load cursors of the K and V streams: the next tile's first row, the key
  // rows from there to the sequence end (the last tile's descriptor is
  // clipped to them), and the tiles left in the item the cursor is in. A
  // cursor that runs out moves to the next item (items have at least two
  // tiles, and K runs at most two tiles ahead of the computation, so that
  // is always nxt).
  const int64_t kstep = (int64_t)BN * p.skn, vstep = (int64_t)BN * p.svn;
  const int krow2 = (int)(p.skn * 2), vrow2 = (int)(p.svn * 2);
  const T* kp = cur.k;
  const T* vp = cur.v;
  int krows = nk, vrows = nk;  // key rows from the cursor's tile to the sequence end
  int kleft = cur.nt, vleft = cur.nt;
  auto k_next = [&](int buf) __attribute__((always_inline)) {
    if (loads) {
      const __amdgpu_buffer_rsrc_t rs = tile_rsrc(kp, min(krows, BN) * krow2);
      LDS_AS char* dst = smb + buf * TILE * 2;
#pragma unroll
      for (int c = 0; c < LDC; ++c) dma16(rs, (LDS_AS void*)(dst + (lw * LDC + c) * 1024), kvo[c]);
    }
    kp += kstep;
    krows -= BN;
    --kleft;
  };
  auto v_next = [&](int buf) __attribute__((always_inline)) {
    if (loads) {
      const __amdgpu_buffer_rsrc_t rs = tile_rsrc(vp, min(vrows, BN) * vrow2);
      LDS_AS char* dst = smb + buf * TILE * 2;
#pragma unroll
      for (int c = 0; c < LDC; ++c) dma16(rs, (LDS_AS void*)(dst + (lw * LDC + c) * 1024), vvo[c]);
    }
    vp += vstep;
    vrows -= BN;
    --vleft;
  };
  // A cursor that has run out moves to the next item first.
  auto k_issue = [&](int buf) __attribute__((always_inline)) {
    if (kleft == 0) {
      if (nxt.nt == 0) return;
      kp = nxt.k;
      krows = nk;
      kleft = nxt.nt;
    }
    k_next(buf);
  };
  auto v_issue = [&](int buf) __attribute__((always_inline)) {
    if (vleft == 0) {
      if (nxt.nt == 0) return;
      vp = nxt.v;
      vrows = nk;
      vleft = nxt.nt;
    }
    v_next(buf);
  };
  q_load(0, cur);
  k_issue(0);
  v_issue(2);
  k_issue(1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  q_read();
  f32x16 s0[KB], s1[KB];
  if (wave_sees(qlo, 0)) {
    scores(kbuf(0), s0);
    mask_tile(qlo, 0, s0);
    m_run = fmaxf(row_max(s0), -1e30f);
  }
  // The next item's Q rows load during the first step (the region was just read).
  bool q_due = nxt.nt > 0;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();  // K buffer 0 is refilled by the first step
  int t = 0;
  // Steps: tile t of the current item (in buffer PAR, the parity of its
  // position in the workgroup's stream) is finished and the stream's next
  // tile is scored.
  // A step in the middle of an item (1 <= t <= nt - 3): the K and V
  // cursors stay inside the item and nothing changes hands, so the step
  // carries no item bookkeeping.
  auto fast_step = [&](auto par_c, f32x16* sc, f32x16* sn) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par_c)::value;
    k_next(PAR);
    if (wave_sees(qlo, t + 1)) {
      scores(kbuf(PAR ^ 1), sn);
      mask_tile(qlo, t + 1, sn);
    }
    v_next(2 + (PAR ^ 1));
    if (wave_sees(qlo, t)) {
      X8 pb[2 * KB];
      softmax_checked(sc, pb);
      pv(vbuf(PAR), pb);
    }
    ++t;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  // Any other step (an item's first, next-to-last and last): cursors may
  // move to the next item, the next item's Q rows load (first step) or come
  // into registers and its first score tile is computed (last step), and
  // the item is finished. Returns false after the workgroup's last item.
  auto slow_step = [&](auto par_c, f32x16* sc, f32x16* sn) __attribute__((always_inline)) -> bool {
    constexpr int PAR = decltype(par_c)::value;
    const bool last = t + 1 == cur.nt;
    k_issue(PAR);  // K tile two ahead in the stream
    if (st_due) {  // the previous item's O and L rows leave
      finish_store();
      st_due = false;
    }
    if (q_due) {  // the next item's Q rows load into the region just read
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      q_load(item + 1, nxt);
      q_due = false;
    }
    const int jn = last ? 0 : t + 1;
    const bool more = !last || nxt.nt > 0;
    const int qlo_n = last ? nxt.q0 + 32 * wave : qlo;
    if (last && more) q_read();
    const bool s_next = more && wave_sees(qlo_n, jn);
    if (s_next) {
      scores(kbuf(PAR ^ 1), sn);
      mask_tile(qlo_n, jn, sn);
    }
    v_issue(2 + (PAR ^ 1));
    if (wave_sees(qlo, t)) {
      X8 pb[2 * KB];
      softmax_checked(sc, pb);
      pv(vbuf(PAR), pb);
    }
    if (last) {
      const float m_next = s_next ? fmaxf(row_max(sn), -1e30f) : -1e30f;
      finish_stage(qlo);
      st_item = item;
      st_qlo = qlo;
      st_due = true;
      m_run = m_next;
      l_run = 0.f;
      l_lse = 0.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
      ++item;
      cur = nxt;
      qlo = cur.q0 + 32 * wave;
      t = 0;
      if (cur.nt > 0) {
        nxt = item_at(item + 1);
        q_due = nxt.nt > 0;
      }
    } else {
      ++t;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    return cur.nt > 0;
  };
  // Two general steps, then middle-of-item steps in pairs while the item
  // has them (the pair keeps the buffer parity a compile-time constant).
  for (;;) {
    if (!slow_step(std::integral_constant<int, 0>{}, s0, s1)) break;
    if (!slow_step(std::integral_constant<int, 1>{}, s1, s0)) break;
    while (t >= 1 && t + 3 < cur.nt) {
      fast_step(std::integral_constant<int, 0>{}, s0, s1);
      fast_step(std::integral_constant<int, 1>{}, s1, s0);
    }
  }
  if (st_due) finish_store();
}

template <typename T, int DP, bool CAUSAL>
static hipError_t launch_fwd_persist(FwdParams p, int grid, hipStream_t s) {
  p.num_q_tiles = (p.Nq + 255) / 256;
  if (p.lse != nullptr)
    hipLaunchKernelGGL((fa_fwd_persist_kernel<T, DP, CAUSAL, true>), dim3(grid), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((fa_fwd_persist_kernel<T, DP, CAUSAL, false>), dim3(grid), dim3(512), 0, s, p);
  return hipGetLastError();
}

// Compute units of the current device (cached per device id; 0 if unknown).
static int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = -1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n > 0 ? n : 0;
}

// Whether the persistent kernel's fixed split of causal items is balanced
// for this launch: the host replays the kernel's assignment (workgroup u of
// the PU on XCD x takes positions i PU + u, i even, and i PU + PU - 1 - u,
// i odd, of XCD x's share of map_tile's order) and compares the largest
// workgroup's key tiles with the mean. The zigzag pairs heavy with light
// items when a share's rows of PU positions fall on whole levels of the
// grouped order; where they do not (4x32x3072, 4x16x4200: largest
// 1.59-1.74x the mean) the fixed split measured up to 18% slower than the
// dispatcher. (Non-causal items are equal: both splits end after
// ceil(items / CUs) of them.) Replays are memoised per thread (a launch
// shape is usually repeated).
static bool persist_balanced(const FwdParams& p, bool causal, int grid) {
  struct Key {
    int bh, nq, nk, hg, grid;
    bool causal;
  };
  thread_local Key keys[4];
  thread_local bool vals[4];
  thread_local int used = 0, next = 0;
  const int BH = p.B * p.Hq, nq = p.Nq, nk = p.Nk, hg = p.heads_per_group > 1 ? p.heads_per_group : 1;
  for (int i = 0; i < used; ++i)
    if (keys[i].bh == BH && keys[i].nq == nq && keys[i].nk == nk && keys[i].hg == hg && keys[i].grid == grid &&
        keys[i].causal == causal)
      return vals[i];
  const int nqt = (nq + 255) / 256, total = nqt * BH, T8 = total / 8, PU = grid / 8, off = nk - nq;
  long long sum = 0, worst = 0;
  for (int x = 0; x < 8; ++x)
    for (int u = 0; u < PU; ++u) {
      long long w = 0;
      for (int i = 0;; ++i) {
        const int j = i * PU + ((i & 1) ? PU - 1 - u : u);
        if (j >= T8) break;
        const int W = x * T8 + j;
        const int g0 = (W / (hg * nqt)) * hg, gh = BH - g0 < hg ? BH - g0 : hg;
        const int level = (W - g0 * nqt) / gh;
        const int q0 = (causal ? nqt - 1 - level : level) * 256;
        const int kv_end = causal ? (q0 + 256 + off < nk ? q0 + 256 + off : nk) : nk;
        w += (kv_end + 63) / 64;
      }
      sum += w;
      worst = w > worst ? w : worst;
    }
  // at most 2% above the mean
  const bool ok = worst * 8LL * PU * 50 <= sum * 51;
  keys[next] = Key{BH, nq, nk, hg, grid, causal};
  vals[next] = ok;
  next = (next + 1) & 3;
  used = used < 4 ? used + 1 : 4;
  return ok;
}

template <typename T, int DP, bool CAUSAL, bool VARLEN, bool PAGED, int NW>
static hipError_t launch_fwd_nw(FwdParams p, hipStream_t s) {
  p.num_q_tiles = (p.Nq + NW * 32 - 1) / (NW * 32);
  const int total = p.num_q_tiles * p.B * p.Hq;
  if (p.lse != nullptr)
    hipLaunchKernelGGL((fa_fwd_kernel<T, DP, CAUSAL, VARLEN, true, PAGED, NW>), dim3(total), dim3(NW * 64), 0, s, p);
  else
    hipLaunchKernelGGL((fa_fwd_kernel<T, DP, CAUSAL, VARLEN, false, PAGED, NW>), dim3(total), dim3(NW * 64), 0, s, p);
  return hipGetLastError();
}

// 8-wave workgroups, head dims of 64 or more: dense launches with at least
// 4096 queries (measured: config-3 shape -3%, non-causal N=4096 -6%, but +2%
// at N=2048, where one workgroup per CU leaves a longer causal tail), and
// varlen batches (packed or paged K/V) of up to 64 sequences (the
// longest-first ranking) with runs of at least 512 queries (config 5,
// 512-query chunks over 2.4k-7.3k keys: -5%).
// Dense launches from 4096 queries (2048 at head dim 128) with at least
// kPersistMinItems 256-query items per CU run persistent (one workgroup per
// CU streaming its items; bit-identical outputs) when every item has at
// least two key tiles (Nk > 64, and Nk >= Nq if causal), the item count
// splits evenly over the 8 XCDs, no workgroup takes more than
// kPersistMaxItems items and, when causal, the fixed split is balanced
// (persist_balanced).
// At 2048 queries and head dim 128 the persistent kernel beat the 4-wave
// grid (config-2 shape -3.7%, non-causal -4.5%, 8x16 heads -2%); at head
// dim 64 it lost 1.7% there.
template <typename T, int DP, bool CAUSAL, bool VARLEN, bool PAGED = false>
static hipError_t launch_fwd(const FwdParams& p, hipStream_t s) {
  if constexpr (!VARLEN && !PAGED && DP >= 64) {
    if (p.Nq >= (DP >= 128 ? 2048 : 4096)) {
      const int total = ((p.Nq + 255) / 256) * p.B * p.Hq;
      const int grid = (cu_count() / 8) * 8;
      if (grid >= 8 && total >= kPersistMinItems * grid && total % 8 == 0 &&
          (total / 8 + grid / 8 - 1) / (grid / 8) <= kPersistMaxItems && p.Nk > 64 && (!CAUSAL || p.Nk >= p.Nq) &&
          (!CAUSAL || persist_balanced(p, CAUSAL, grid)))
        return launch_fwd_persist<T, DP, CAUSAL>(p, grid, s);
      if (p.Nq >= 4096) return launch_fwd_nw<T, DP, CAUSAL, VARLEN, PAGED, 8>(p, s);
    }
  }
  if constexpr (VARLEN && DP >= 64) {
    if (p.B <= 64 && p.Nq >= 512) return launch_fwd_nw<T, DP, CAUSAL, VARLEN, PAGED, 8>(p, s);
  }
  return launch_fwd_nw<T, DP, CAUSAL, VARLEN, PAGED, 4>(p, s);
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
// dp is the padded head dim (32, 64 or 128). Query tiles are 128 rows.
hipError_t fwd_mfma(FwdParams p, bool is_bf16, int dp, bool causal, bool varlen, hipStream_t s) {
  p.heads_per_group = heads_per_group_for((long long)p.Nk * dp * 2 * 2);  // K and V rows of a head
  if (is_bf16) return dispatch_fwd_t<__bf16>(p, dp, causal, varlen, s);
  return dispatch_fwd_t<_Float16>(p, dp, causal, varlen, s);
}

template <typename T, int DP>
static hipError_t dispatch_paged_dp(const FwdParams& p, bool causal, hipStream_t s) {
  return causal ? launch_fwd<T, DP, true, true, true>(p, s) : launch_fwd<T, DP, false, true, true>(p, s);
}

template <typename T>
static hipError_t dispatch_paged_t(const FwdParams& p, int dp, bool causal, hipStream_t s) {
  switch (dp) {
    case 32: return dispatch_paged_dp<T, 32>(p, causal, s);
    case 64: return dispatch_paged_dp<T, 64>(p, causal, s);
    default: return dispatch_paged_dp<T, 128>(p, causal, s);
  }
}

// Paged K/V forward (arguments validated by the C ABI layer; p.Nq is the
// longest query chunk, block_shift >= 4).
hipError_t fwd_paged(FwdParams p, bool is_bf16, int dp, bool causal, hipStream_t s) {
  p.heads_per_group = heads_per_group_for((long long)p.Nk * dp * 2 * 2);
  if (is_bf16) return dispatch_paged_t<__bf16>(p, dp, causal, s);
  return dispatch_paged_t<_Float16>(p, dp, causal, s);
}

}  // namespace lsfa
