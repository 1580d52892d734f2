// C ABI of liblsfa_gfx950.so: argument validation (host only, no GPU access)
// and kernel selection. See include/lightserve_fa.h for the contract.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/lightserve_fa.h"
#include "fa_common.hpp"

namespace lsfa {
hipError_t fwd_mfma(FwdParams p, bool is_bf16, int dp, bool causal, bool varlen, hipStream_t s);
hipError_t fwd_paged(FwdParams p, bool is_bf16, int dp, bool causal, hipStream_t s);
hipError_t bwd_mfma(const BwdParams& p, bool is_bf16, int dp, bool causal, int phases, hipStream_t s);
hipError_t fwd_f32(const FwdParams& p, int dp, bool causal, bool varlen, float scale, hipStream_t s);
hipError_t bwd_f32(const BwdParams& p, int dp, bool causal, hipStream_t s);
hipError_t decode_gqa(const DecodeParams& p, bool is_bf16, int dp, hipStream_t s);
hipError_t rope_inplace(const RopeParams& p, int dtype, hipStream_t s);
hipError_t add_rmsnorm(const NormParams& p, int dtype, bool vec, hipStream_t s);
hipError_t gemv(const GemvParams& p, bool is_bf16, hipStream_t s);
hipError_t gemv_mfma(const GemvParams& p, bool is_bf16, hipStream_t s);
int gemv_capacity(int m);
hipError_t greedy(const void* logits, int64_t stride, int dtype, int rows, int cols, int64_t* tokens,
                  int32_t* seq_lens, hipStream_t s);
}  // namespace lsfa

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return LSFA_OK;
}

// Padded head dim of the kernels: 32, 64 or 128.
int padded_dim(int d) { return d <= 32 ? 32 : (d <= 64 ? 64 : 128); }
int padded_decode_dim(int d) { return d <= 64 ? 64 : 128; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Layout requirement of the MFMA kernels for one [b, h, n, d] tensor.
int check_fast_layout(const char* name, const void* ptr, const int64_t* st, bool varlen) {
  if (st[3] != 1) return fail(LSFA_ERR_UNSUPPORTED, "%s: head-dim stride must be 1 for bf16/fp16 (got %lld)", name, (long long)st[3]);
  for (int i = varlen ? 1 : 0; i < 3; ++i)
    if (st[i] % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "%s: stride[%d]=%lld is not a multiple of 8 elements", name, i, (long long)st[i]);
  if (!aligned16(ptr)) return fail(LSFA_ERR_UNSUPPORTED, "%s: base pointer is not 16-byte aligned", name);
  // Tile loads address up to 128 rows from a per-tile base with 32-bit byte
  // offsets.
  if (st[2] < 0 || st[2] > (1LL << 22))
    return fail(LSFA_ERR_UNSUPPORTED, "%s: row stride %lld outside 0..2^22 elements", name, (long long)st[2]);
  return LSFA_OK;
}

int check_common(int dtype, int batch, int hq, int hkv, int nq, int nk, int d, float scale) {
  if (dtype != LSFA_DTYPE_FP32 && dtype != LSFA_DTYPE_FP16 && dtype != LSFA_DTYPE_BF16)
    return fail(LSFA_ERR_INVALID, "unknown dtype %d", dtype);
  if (batch < 0 || hq < 0 || hkv < 0 || nq < 0 || nk < 0)
    return fail(LSFA_ERR_INVALID, "negative size (batch=%d heads_q=%d heads_kv=%d seqlen_q=%d seqlen_k=%d)", batch, hq,
                hkv, nq, nk);
  if (hkv == 0 && hq != 0) return fail(LSFA_ERR_INVALID, "heads_kv must be positive");
  if (hkv > 0 && hq % hkv != 0) return fail(LSFA_ERR_INVALID, "heads_q (%d) is not a multiple of heads_kv (%d)", hq, hkv);
  if (d < 1 || d > 128) return fail(LSFA_ERR_UNSUPPORTED, "head_dim %d outside 1..128", d);
  if (!std::isfinite(scale)) return fail(LSFA_ERR_INVALID, "sm_scale is not finite");
  const long long tiles = (long long)((nq + 63) / 64) * batch * hq;
  if (tiles > (1LL << 30)) return fail(LSFA_ERR_UNSUPPORTED, "problem too large for one launch");
  return LSFA_OK;
}

// Backward workspace: (lse*log2e, delta) pairs for every (b, h, query),
// queries padded to a multiple of 128 (the recompute path's dq kernel writes
// whole 128-row tiles). The stored-dS path (LSFA_BWD_STORED_DS, bf16/fp16
// with head_dim above 64) adds, 256-byte aligned, dS of a chunk of heads in
// the input dtype: per head ceil(seqlen_k / 32) rows of ds_ldq / 32 blocks
// of 32 keys x 32 queries (1024 elements), ds_ldq = seqlen_q rounded up to
// the dQ kernel's 256-query tile. A chunk is as many heads as fit in
// kDsChunkBytes (at least one); the backward then runs chunk by chunk. At
// head_dim <= 64 moving dS through HBM costs more than recomputing it, so
// the flag does not apply there.
struct BwdWorkspace {
  int64_t nq_pad = 0;
  uint64_t ld_off = 0, bytes = 0;
  bool stored_ds = false;
  uint64_t ds_off = 0;
  int64_t ds_ldq = 0, ds_sbh = 0;
  int chunk_heads = 0, chunks = 0;
};

constexpr uint64_t kDsChunkBytes = uint64_t(4) << 30;

uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

bool bwd_stored_ds(int dtype, int flags, int head_dim) {
  return dtype != LSFA_DTYPE_FP32 && (flags & LSFA_BWD_STORED_DS) != 0 && padded_dim(head_dim) == 128;
}

BwdWorkspace bwd_workspace(int dtype, int flags, int batch, int heads, int nq, int nk, int head_dim) {
  BwdWorkspace w;
  w.nq_pad = ((int64_t)nq + 127) / 128 * 128;
  const uint64_t rows = (uint64_t)batch * heads * w.nq_pad;
  w.ld_off = 0;
  w.bytes = align256(rows * 8);
  const int64_t bh = (int64_t)batch * heads;
  if (bwd_stored_ds(dtype, flags, head_dim) && bh > 0 && nq > 0 && nk > 0) {
    w.stored_ds = true;
    w.ds_ldq = ((int64_t)nq + 255) / 256 * 256;
    w.ds_sbh = ((int64_t)nk + 31) / 32 * 32 * w.ds_ldq;
    const uint64_t head_bytes = (uint64_t)w.ds_sbh * 2;
    const uint64_t fit = kDsChunkBytes / head_bytes;
    w.chunk_heads = (int)(fit < 1 ? 1 : (fit > (uint64_t)bh ? bh : fit));
    w.chunks = (int)((bh + w.chunk_heads - 1) / w.chunk_heads);
    w.ds_off = w.bytes;
    w.bytes = w.ds_off + align256(head_bytes * w.chunk_heads);
  }
  return w;
}

// Decode split: enough workgroups (batch x kv heads x splits) to fill the
// GPU, splits of a multiple of 64 tokens whose block-table slice fits the
// kernel's LDS table. Partial outputs go to the workspace when split.
struct DecodeSplit {
  int num_splits = 1, split_tokens = 64;
  uint64_t o_off = 0, lse_off = 0, bytes = 0;
};

int log2_exact(int x) {
  int s = 0;
  while ((1 << s) < x) ++s;
  return (1 << s) == x ? s : -1;
}

DecodeSplit decode_split(const lsfa_decode_args* a) {
  DecodeSplit d;
  const int maxs = std::max(a->max_seq_len, 0);
  const long long units = std::max(1LL, (long long)a->batch * a->heads_kv);
  // Lane-group kernel: splits of about 512 tokens while fewer than ~16
  // workgroups per CU exist (sequence lengths vary, and short splits keep the
  // longest sequences from setting the tail). MFMA kernel (one workgroup per
  // CU): splits only below one workgroup per CU, of at least 4096 tokens, so
  // that each workgroup's first-load latency is amortised.
  const int g = a->heads_kv > 0 ? a->heads_q / a->heads_kv : 1;
  const bool mfma = lsfa::decode_uses_mfma(g, std::max(0, log2_exact(std::max(1, a->block_size))));
  const long long target = mfma ? 256 : 4096, min_split = mfma ? 4096 : 512;
  long long ns = 1;
  if (units < target && maxs > min_split)
    ns = std::min<long long>((target + units - 1) / units, (maxs + min_split - 1) / min_split);
  long long st = (maxs + ns - 1) / ns;
  st = std::max(64LL, (st + 63) / 64 * 64);
  const int shift = std::max(0, log2_exact(std::max(1, a->block_size)));
  const long long max_st = ((long long)(lsfa::kDecodeMaxTableSlots - 1) << shift) / 64 * 64;
  st = std::min(st, std::max(64LL, max_st));
  ns = std::max(1LL, (maxs + st - 1) / st);
  d.num_splits = (int)ns;
  d.split_tokens = (int)st;
  if (ns > 1) {
    const uint64_t rows = (uint64_t)a->batch * a->heads_q * ns;
    d.o_off = 0;
    d.lse_off = align256(rows * padded_decode_dim(a->head_dim) * 4);
    d.bytes = d.lse_off + align256(rows * 4);
  }
  return d;
}

}  // namespace

extern "C" {

int lsfa_abi_version(void) { return LSFA_ABI_VERSION; }

const char* lsfa_last_error(void) { return g_last_error.c_str(); }

int lsfa_fwd_check(const lsfa_fwd_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  int rc = check_common(a->dtype, a->batch, a->heads_q, a->heads_kv, a->seqlen_q, a->seqlen_k, a->head_dim, a->sm_scale);
  if (rc) return rc;
  if ((a->cu_seqlens_q == nullptr) != (a->cu_seqlens_k == nullptr))
    return fail(LSFA_ERR_INVALID, "cu_seqlens_q and cu_seqlens_k must both be set or both be NULL");
  const bool empty = (long long)a->batch * a->heads_q * a->seqlen_q == 0;
  if (!empty && (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr))
    return fail(LSFA_ERR_INVALID, "q, k, v and o must be non-NULL");
  const bool varlen = a->cu_seqlens_q != nullptr;
  if (a->dtype != LSFA_DTYPE_FP32 && !empty) {
    if (a->head_dim % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "bf16/fp16 head_dim must be a multiple of 8 (got %d)", a->head_dim);
    if ((rc = check_fast_layout("q", a->q, a->q_stride, varlen))) return rc;
    if ((rc = check_fast_layout("k", a->k, a->k_stride, varlen))) return rc;
    if ((rc = check_fast_layout("v", a->v, a->v_stride, varlen))) return rc;
    if ((rc = check_fast_layout("o", a->o, a->o_stride, varlen))) return rc;
  }
  return ok();
}

int lsfa_fwd(const lsfa_fwd_args* a, void* stream) {
  int rc = lsfa_fwd_check(a);
  if (rc) return rc;
  if ((long long)a->batch * a->heads_q * a->seqlen_q == 0) return ok();
  lsfa::FwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.o = a->o;
  p.lse = a->lse;
  p.sqb = a->q_stride[0]; p.sqh = a->q_stride[1]; p.sqn = a->q_stride[2]; p.sqd = a->q_stride[3];
  p.skb = a->k_stride[0]; p.skh = a->k_stride[1]; p.skn = a->k_stride[2]; p.skd = a->k_stride[3];
  p.svb = a->v_stride[0]; p.svh = a->v_stride[1]; p.svn = a->v_stride[2]; p.svd = a->v_stride[3];
  p.sob = a->o_stride[0]; p.soh = a->o_stride[1]; p.son = a->o_stride[2]; p.sod = a->o_stride[3];
  p.slb = a->lse_stride[0]; p.slh = a->lse_stride[1]; p.sln = a->lse_stride[2];
  p.cu_q = a->cu_seqlens_q;
  p.cu_k = a->cu_seqlens_k;
  p.B = a->batch; p.Hq = a->heads_q; p.Hkv = a->heads_kv;
  p.Nq = a->seqlen_q; p.Nk = a->seqlen_k; p.D = a->head_dim;
  // The MFMA kernels keep the exponent scale positive (a negative scale is
  // folded into q) and nonzero (a zero scale becomes 1e-30: every score is 0
  // to within fp32 rounding either way).
  p.scale_log2 = fmaxf(fabsf(a->sm_scale) * 1.4426950408889634f, 1e-30f);
  p.neg_q = a->sm_scale < 0.f;
  const bool varlen = a->cu_seqlens_q != nullptr;
  const int dp = padded_dim(a->head_dim);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (a->dtype == LSFA_DTYPE_FP32)
    e = lsfa::fwd_f32(p, dp, a->causal != 0, varlen, a->sm_scale, s);
  else
    e = lsfa::fwd_mfma(p, a->dtype == LSFA_DTYPE_BF16, dp, a->causal != 0, varlen, s);
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_bwd_check(const lsfa_bwd_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  int rc = check_common(a->dtype, a->batch, a->heads_q, a->heads_kv, a->seqlen_q, a->seqlen_k, a->head_dim, a->sm_scale);
  if (rc) return rc;
  if ((a->cu_seqlens_q == nullptr) != (a->cu_seqlens_k == nullptr))
    return fail(LSFA_ERR_INVALID, "cu_seqlens_q and cu_seqlens_k must both be set or both be NULL");
  const bool varlen = a->cu_seqlens_q != nullptr;
  if (varlen && a->dtype == LSFA_DTYPE_FP32)
    return fail(LSFA_ERR_UNSUPPORTED, "the fp32 backward has no varlen (cu_seqlens)");
  if (varlen && (a->flags & LSFA_BWD_STORED_DS))
    return fail(LSFA_ERR_UNSUPPORTED, "LSFA_BWD_STORED_DS has no varlen (cu_seqlens)");
  if (a->heads_kv != a->heads_q && a->dtype == LSFA_DTYPE_FP32)
    return fail(LSFA_ERR_UNSUPPORTED, "the fp32 backward has no GQA (heads_kv != heads_q)");
  if (a->heads_kv != a->heads_q && (a->flags & LSFA_BWD_STORED_DS))
    return fail(LSFA_ERR_UNSUPPORTED, "LSFA_BWD_STORED_DS has no GQA (heads_kv != heads_q)");
  const int phase = a->flags & ~LSFA_BWD_STORED_DS;
  if (phase != 0 && phase != LSFA_BWD_ONLY_DQ && phase != LSFA_BWD_ONLY_DKDV)
    return fail(LSFA_ERR_INVALID, "unknown flags %d", a->flags);
  if (phase != 0 && a->dtype == LSFA_DTYPE_FP32)
    return fail(LSFA_ERR_UNSUPPORTED, "the fp32 backward runs both phases together (no LSFA_BWD_ONLY_* flag)");
  const bool empty = (long long)a->batch * a->heads_q * (a->seqlen_q + a->seqlen_k) == 0;
  if (!empty) {
    if (!a->q || !a->k || !a->v || !a->o || !a->dout || !a->lse || !a->dq || !a->dk || !a->dv)
      return fail(LSFA_ERR_INVALID, "q, k, v, o, dout, lse, dq, dk and dv must be non-NULL");
    const BwdWorkspace w = bwd_workspace(a->dtype, a->flags, a->batch, a->heads_q, a->seqlen_q, a->seqlen_k, a->head_dim);
    if (phase != 0 && w.chunks > 1)
      return fail(LSFA_ERR_UNSUPPORTED,
                  "LSFA_BWD_ONLY_* with LSFA_BWD_STORED_DS needs the stored dS of all heads at once (this "
                  "problem runs in %d chunks)",
                  w.chunks);
    if (w.bytes > 0 && !a->workspace) return fail(LSFA_ERR_INVALID, "workspace must be non-NULL");
    if (a->workspace_bytes < w.bytes)
      return fail(LSFA_ERR_INVALID, "workspace_bytes %llu is below the %llu bytes lsfa_bwd_workspace_size asks for",
                  (unsigned long long)a->workspace_bytes, (unsigned long long)w.bytes);
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
      return fail(LSFA_ERR_INVALID, "workspace is not 256-byte aligned");
    if (a->dtype != LSFA_DTYPE_FP32) {
      if (a->head_dim % 8 != 0)
        return fail(LSFA_ERR_UNSUPPORTED, "bf16/fp16 head_dim must be a multiple of 8 (got %d)", a->head_dim);
      const char* names[8] = {"q", "k", "v", "o", "dout", "dq", "dk", "dv"};
      const void* ptrs[8] = {a->q, a->k, a->v, a->o, a->dout, a->dq, a->dk, a->dv};
      const int64_t* strides[8] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride,
                                   a->do_stride, a->dq_stride, a->dk_stride, a->dv_stride};
      for (int i = 0; i < 8; ++i)
        if ((rc = check_fast_layout(names[i], ptrs[i], strides[i], varlen))) return rc;
    }
  }
  return ok();
}

int lsfa_bwd_workspace_size(const lsfa_bwd_args* a, uint64_t* bytes) {
  if (a == nullptr || bytes == nullptr) return fail(LSFA_ERR_INVALID, "args or bytes is NULL");
  int rc = check_common(a->dtype, a->batch, a->heads_q, a->heads_kv, a->seqlen_q, a->seqlen_k, a->head_dim, a->sm_scale);
  if (rc) return rc;
  *bytes = bwd_workspace(a->dtype, a->flags, a->batch, a->heads_q, a->seqlen_q, a->seqlen_k, a->head_dim).bytes;
  return ok();
}

// Launches the backward for validated arguments (the workspace included).
static int run_bwd(const lsfa_bwd_args* a, void* stream) {
  if ((long long)a->batch * a->heads_q * (a->seqlen_q + a->seqlen_k) == 0) return ok();
  lsfa::BwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o; p.dout = a->dout; p.lse = a->lse;
  p.dq = a->dq; p.dk = a->dk; p.dv = a->dv;
  const BwdWorkspace w = bwd_workspace(a->dtype, a->flags, a->batch, a->heads_q, a->seqlen_q, a->seqlen_k, a->head_dim);
  char* ws = static_cast<char*>(a->workspace);
  p.nq_pad = (int)w.nq_pad;
  p.ld = reinterpret_cast<float*>(ws + w.ld_off);
  p.sldh = 2 * w.nq_pad;
  p.sldb = (int64_t)a->heads_q * p.sldh;
  if (w.stored_ds) {
    p.ds = ws + w.ds_off;
    p.ds_ldq = w.ds_ldq;
    p.ds_sbh = w.ds_sbh;
    p.nbh = w.chunk_heads;
  }
  p.sqb = a->q_stride[0]; p.sqh = a->q_stride[1]; p.sqn = a->q_stride[2]; p.sqd = a->q_stride[3];
  p.skb = a->k_stride[0]; p.skh = a->k_stride[1]; p.skn = a->k_stride[2]; p.skd = a->k_stride[3];
  p.svb = a->v_stride[0]; p.svh = a->v_stride[1]; p.svn = a->v_stride[2]; p.svd = a->v_stride[3];
  p.sob = a->o_stride[0]; p.soh = a->o_stride[1]; p.son = a->o_stride[2]; p.sod = a->o_stride[3];
  p.sdob = a->do_stride[0]; p.sdoh = a->do_stride[1]; p.sdon = a->do_stride[2]; p.sdod = a->do_stride[3];
  p.sdqb = a->dq_stride[0]; p.sdqh = a->dq_stride[1]; p.sdqn = a->dq_stride[2]; p.sdqd = a->dq_stride[3];
  p.sdkb = a->dk_stride[0]; p.sdkh = a->dk_stride[1]; p.sdkn = a->dk_stride[2]; p.sdkd = a->dk_stride[3];
  p.sdvb = a->dv_stride[0]; p.sdvh = a->dv_stride[1]; p.sdvn = a->dv_stride[2]; p.sdvd = a->dv_stride[3];
  p.slb = a->lse_stride[0]; p.slh = a->lse_stride[1]; p.sln = a->lse_stride[2];
  p.B = a->batch; p.H = a->heads_q; p.Nq = a->seqlen_q; p.Nk = a->seqlen_k; p.D = a->head_dim;
  p.G = a->heads_kv > 0 ? a->heads_q / a->heads_kv : 1;
  p.cu_q = a->cu_seqlens_q;
  p.cu_k = a->cu_seqlens_k;
  p.scale = a->sm_scale;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  const int dp = padded_dim(a->head_dim);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (a->dtype == LSFA_DTYPE_FP32)
    e = lsfa::bwd_f32(p, dp, a->causal != 0, s);
  else
  {
    const int phase = a->flags & ~LSFA_BWD_STORED_DS;
    e = lsfa::bwd_mfma(p, a->dtype == LSFA_DTYPE_BF16, dp, a->causal != 0,
                       phase == LSFA_BWD_ONLY_DQ ? 1 : (phase == LSFA_BWD_ONLY_DKDV ? 2 : 3), s);
  }
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_bwd(const lsfa_bwd_args* a, void* stream) {
  int rc = lsfa_bwd_check(a);
  if (rc) return rc;
  return run_bwd(a, stream);
}

// Allocation-free backward: the workspace is this file's device array
// `scratch` (every GPU holds its own copy while the library is loaded). Host
// code never uses the array's name as an address: each device's address comes
// from hipGetSymbolAddress, resolved once per device on that device's first
// call (with the device current) and kept in scratch_ptr.
static __device__ __attribute__((aligned(256))) char scratch[LSFA_BWD_SCRATCH_BYTES];

}  // extern "C"

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(LSFA_ERR_UNSUPPORTED, "device index %d above %d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(LSFA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return LSFA_OK;
}
}  // namespace

extern "C" {

int lsfa_bwd_noalloc(const lsfa_bwd_args* args, void* stream) {
  if (args == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  // The recompute kernels: their workspace is the per-row pairs alone.
  lsfa_bwd_args r = *args;
  r.flags &= ~LSFA_BWD_STORED_DS;
  const lsfa_bwd_args* a = &r;
  uint64_t need = 0;
  int rc = lsfa_bwd_workspace_size(a, &need);
  if (rc) return rc;
  if (need > (uint64_t)LSFA_BWD_SCRATCH_BYTES)
    return fail(LSFA_ERR_UNSUPPORTED,
                "lsfa_bwd_noalloc: this problem needs %llu bytes of workspace, above the %d bytes of the library's "
                "scratch array (batch * heads * seqlen_q rounded up to 128 must be at most %d); use lsfa_bwd",
                (unsigned long long)need, LSFA_BWD_SCRATCH_BYTES, LSFA_BWD_SCRATCH_BYTES / 8);
  // Every argument is checked (host only) before any GPU query: the
  // workspace fields first stand for the array (an aligned placeholder that
  // the check never dereferences), then get its address on this device.
  lsfa_bwd_args b = *a;
  b.workspace = reinterpret_cast<void*>(uintptr_t{256});
  b.workspace_bytes = LSFA_BWD_SCRATCH_BYTES;
  if ((rc = lsfa_bwd_check(&b))) return rc;
  b.workspace = nullptr;
  if ((long long)a->batch * a->heads_q * (a->seqlen_q + a->seqlen_k) != 0 && need > 0)
    if ((rc = scratch_for_current_device(&b.workspace))) return rc;
  return run_bwd(&b, stream);
}

int lsfa_decode_check(const lsfa_decode_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(a->dtype == LSFA_DTYPE_FP32 ? LSFA_ERR_UNSUPPORTED : LSFA_ERR_INVALID,
                "decode supports bf16 and fp16 (dtype %d)", a->dtype);
  if (a->batch < 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->num_blocks < 0 || a->max_blocks_per_seq < 0 ||
      a->max_seq_len < 0)
    return fail(LSFA_ERR_INVALID, "negative size or no heads (batch=%d heads_q=%d heads_kv=%d num_blocks=%d "
                "max_blocks_per_seq=%d max_seq_len=%d)", a->batch, a->heads_q, a->heads_kv, a->num_blocks,
                a->max_blocks_per_seq, a->max_seq_len);
  if (a->heads_q % a->heads_kv != 0) return fail(LSFA_ERR_INVALID, "heads_q (%d) is not a multiple of heads_kv (%d)", a->heads_q, a->heads_kv);
  if (a->head_dim < 8 || a->head_dim > 128 || a->head_dim % 8 != 0)
    return fail(LSFA_ERR_UNSUPPORTED, "decode head_dim must be a multiple of 8 in 8..128 (got %d)", a->head_dim);
  if (a->block_size < 1 || log2_exact(a->block_size) < 0)
    return fail(LSFA_ERR_UNSUPPORTED, "block_size must be a power of two (got %d)", a->block_size);
  // Blocks of 16 tokens or more take the MFMA kernel (query heads are MFMA
  // columns: up to 32 per KV head); smaller blocks the lane-group kernel.
  const int g = a->heads_q / a->heads_kv;
  if (a->block_size >= 16 ? g > 32 : (g != 1 && g != 2 && g != 4 && g != 8))
    return fail(LSFA_ERR_UNSUPPORTED, "heads_q / heads_kv = %d; decode supports up to 32 with block_size >= 16, "
                "else 1, 2, 4 and 8", g);
  if (!std::isfinite(a->sm_scale)) return fail(LSFA_ERR_INVALID, "sm_scale is not finite");
  if (a->batch == 0) return ok();
  if (!a->q || !a->k_cache || !a->v_cache || !a->o || !a->block_tables || !a->seq_lens)
    return fail(LSFA_ERR_INVALID, "q, k_cache, v_cache, o, block_tables and seq_lens must be non-NULL");
  if (a->q_stride[2] != 1 || a->o_stride[2] != 1 || a->k_stride[3] != 1 || a->v_stride[3] != 1)
    return fail(LSFA_ERR_UNSUPPORTED, "head-dim strides must be 1");
  for (int i = 0; i < 2; ++i)
    if (a->q_stride[i] % 8 != 0 || a->o_stride[i] % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "q/o strides must be multiples of 8 elements");
  for (int i = 0; i < 3; ++i)
    if (a->k_stride[i] % 8 != 0 || a->v_stride[i] % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be multiples of 8 elements");
  if (!aligned16(a->q) || !aligned16(a->o) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return fail(LSFA_ERR_UNSUPPORTED, "q, o, k_cache and v_cache must be 16-byte aligned");
  if (a->block_table_stride < a->max_blocks_per_seq)
    return fail(LSFA_ERR_INVALID, "block_table_stride %lld is below max_blocks_per_seq %d",
                (long long)a->block_table_stride, a->max_blocks_per_seq);
  const DecodeSplit d = decode_split(a);
  if (d.bytes > 0) {
    if (!a->workspace) return fail(LSFA_ERR_INVALID, "workspace must be non-NULL");
    if (a->workspace_bytes < d.bytes)
      return fail(LSFA_ERR_INVALID, "workspace_bytes %llu is below the %llu bytes lsfa_decode_workspace_size asks for",
                  (unsigned long long)a->workspace_bytes, (unsigned long long)d.bytes);
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
      return fail(LSFA_ERR_INVALID, "workspace is not 256-byte aligned");
  }
  return ok();
}

int lsfa_decode_workspace_size(const lsfa_decode_args* a, uint64_t* bytes) {
  if (a == nullptr || bytes == nullptr) return fail(LSFA_ERR_INVALID, "args or bytes is NULL");
  *bytes = decode_split(a).bytes;
  return ok();
}

int lsfa_decode(const lsfa_decode_args* a, void* stream) {
  int rc = lsfa_decode_check(a);
  if (rc) return rc;
  if (a->batch == 0) return ok();
  const DecodeSplit d = decode_split(a);
  lsfa::DecodeParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.kc = a->k_cache; p.vc = a->v_cache; p.o = a->o; p.lse = a->lse;
  p.block_tables = a->block_tables; p.seq_lens = a->seq_lens;
  if (d.bytes > 0) {
    char* ws = static_cast<char*>(a->workspace);
    p.o_part = reinterpret_cast<float*>(ws + d.o_off);
    p.lse_part = reinterpret_cast<float*>(ws + d.lse_off);
  }
  p.sqb = a->q_stride[0]; p.sqh = a->q_stride[1];
  p.skb = a->k_stride[0]; p.sks = a->k_stride[1]; p.skh = a->k_stride[2];
  p.svb = a->v_stride[0]; p.svs = a->v_stride[1]; p.svh = a->v_stride[2];
  p.sob = a->o_stride[0]; p.soh = a->o_stride[1];
  p.slb = a->lse_stride[0]; p.slh = a->lse_stride[1];
  p.sbt = a->block_table_stride;
  p.B = a->batch; p.Hq = a->heads_q; p.Hkv = a->heads_kv; p.D = a->head_dim;
  p.block_shift = log2_exact(a->block_size);
  p.max_blocks = a->max_blocks_per_seq;
  p.num_blocks = a->num_blocks;
  p.max_seq_len = a->max_seq_len;
  p.num_splits = d.num_splits;
  p.split_tokens = d.split_tokens;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  hipError_t e = lsfa::decode_gqa(p, a->dtype == LSFA_DTYPE_BF16, padded_decode_dim(a->head_dim),
                                  reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "decode launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_prefill_paged_check(const lsfa_prefill_paged_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(a->dtype == LSFA_DTYPE_FP32 ? LSFA_ERR_UNSUPPORTED : LSFA_ERR_INVALID,
                "paged prefill supports bf16 and fp16 (dtype %d)", a->dtype);
  if (a->batch < 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->num_blocks < 0 || a->max_blocks_per_seq < 0 ||
      a->max_seqlen_q < 0)
    return fail(LSFA_ERR_INVALID, "negative size or no heads (batch=%d heads_q=%d heads_kv=%d num_blocks=%d "
                "max_blocks_per_seq=%d max_seqlen_q=%d)", a->batch, a->heads_q, a->heads_kv, a->num_blocks,
                a->max_blocks_per_seq, a->max_seqlen_q);
  if (a->heads_q % a->heads_kv != 0)
    return fail(LSFA_ERR_INVALID, "heads_q (%d) is not a multiple of heads_kv (%d)", a->heads_q, a->heads_kv);
  if (a->head_dim < 8 || a->head_dim > 128 || a->head_dim % 8 != 0)
    return fail(LSFA_ERR_UNSUPPORTED, "paged prefill head_dim must be a multiple of 8 in 8..128 (got %d)", a->head_dim);
  if (a->block_size < 16 || log2_exact(a->block_size) < 0)
    return fail(LSFA_ERR_UNSUPPORTED, "paged prefill needs a power-of-two block_size of at least 16 (got %d)",
                a->block_size);
  if (!std::isfinite(a->sm_scale)) return fail(LSFA_ERR_INVALID, "sm_scale is not finite");
  const long long tiles = (long long)((a->max_seqlen_q + 127) / 128) * a->batch * a->heads_q;
  if (tiles > (1LL << 30)) return fail(LSFA_ERR_UNSUPPORTED, "problem too large for one launch");
  if (a->batch == 0 || a->max_seqlen_q == 0) return ok();
  if (!a->q || !a->k_cache || !a->v_cache || !a->o || !a->cu_seqlens_q || !a->seq_lens_k || !a->block_tables)
    return fail(LSFA_ERR_INVALID, "q, k_cache, v_cache, o, cu_seqlens_q, seq_lens_k and block_tables must be non-NULL");
  for (int i = 0; i < 2; ++i)
    if (a->q_stride[i] % 8 != 0 || a->o_stride[i] % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "q/o strides must be multiples of 8 elements");
  for (int i = 0; i < 3; ++i)
    if (a->k_stride[i] % 8 != 0 || a->v_stride[i] % 8 != 0)
      return fail(LSFA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be multiples of 8 elements");
  // 16 slots of one block are addressed from a per-wave base with 32-bit byte offsets.
  if (a->k_stride[1] < 0 || a->k_stride[1] > (1LL << 22) || a->v_stride[1] < 0 || a->v_stride[1] > (1LL << 22))
    return fail(LSFA_ERR_UNSUPPORTED, "cache slot strides must lie in 0..2^22 elements");
  if (!aligned16(a->q) || !aligned16(a->o) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return fail(LSFA_ERR_UNSUPPORTED, "q, o, k_cache and v_cache must be 16-byte aligned");
  if (a->block_table_stride < a->max_blocks_per_seq)
    return fail(LSFA_ERR_INVALID, "block_table_stride %lld is below max_blocks_per_seq %d",
                (long long)a->block_table_stride, a->max_blocks_per_seq);
  return ok();
}

int lsfa_prefill_paged(const lsfa_prefill_paged_args* a, void* stream) {
  int rc = lsfa_prefill_paged_check(a);
  if (rc) return rc;
  if (a->batch == 0 || a->max_seqlen_q == 0) return ok();
  lsfa::FwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.k = a->k_cache; p.v = a->v_cache; p.o = a->o; p.lse = a->lse;
  p.sqn = a->q_stride[0]; p.sqh = a->q_stride[1];
  p.skb = a->k_stride[0]; p.skn = a->k_stride[1]; p.skh = a->k_stride[2];
  p.svb = a->v_stride[0]; p.svn = a->v_stride[1]; p.svh = a->v_stride[2];
  p.son = a->o_stride[0]; p.soh = a->o_stride[1];
  p.slh = a->lse_stride[0]; p.sln = a->lse_stride[1];
  p.cu_q = a->cu_seqlens_q;
  p.block_tables = a->block_tables;
  p.seq_lens_k = a->seq_lens_k;
  p.sbt = a->block_table_stride;
  p.block_shift = log2_exact(a->block_size);
  p.max_blocks = a->max_blocks_per_seq;
  p.num_blocks = a->num_blocks;
  p.B = a->batch; p.Hq = a->heads_q; p.Hkv = a->heads_kv;
  p.Nq = a->max_seqlen_q; p.Nk = 0; p.D = a->head_dim;
  p.scale_log2 = fmaxf(fabsf(a->sm_scale) * 1.4426950408889634f, 1e-30f);
  p.neg_q = a->sm_scale < 0.f;
  hipError_t e = lsfa::fwd_paged(p, a->dtype == LSFA_DTYPE_BF16, padded_dim(a->head_dim), a->causal != 0,
                                 reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "paged prefill launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"

namespace {

// Skinny GEMM split: about 1024 workgroups (256 columns x one K-range each)
// with K-ranges of at least 128 rows (multiples of 8; measured on MI355X in
// graph replays: 1024 workgroups with 128-row minimum beat 256-4096
// workgroups and 32-256-row minimums on the decode projections, the narrow
// ones gaining most from fewer splits) and at most what keeps
// x's range within 32 KB of LDS at the kernel's row capacity (2048 rows up to
// 4 rows, 1024 at 8). Workspace (only with more than one split): the int32
// arrival counters, 16 per 256-column block, in a region of fixed size
// (LSFA_GEMV_COUNTER_BYTES, so that no call's partials overlap another call's
// counters in a shared workspace), then the fp32 partials [splits][m][n].
struct GemvSplit {
  int kc = 8, splits = 1;
  uint64_t counter_bytes = 0, bytes = 0;
};

// The MFMA kernel (fa_gemv_mfma.hip) serves 3..32 rows when every matrix's
// width is a multiple of 128 and the input is x or x with a SwiGLU gate (not a
// fused norm): K-ranges of at most 256 rows (four 64-row tiles per
// workgroup), 128-column blocks.
bool gemv_uses_mfma(const lsfa_gemv_group_args* a) {
  if (a->m < 3 || a->m > 32 || a->norm_weight || a->k % 8 != 0 || a->x_stride % 8 != 0 || !aligned16(a->x))
    return false;
  if (a->x_gate && (a->x_gate_stride % 8 != 0 || !aligned16(a->x_gate))) return false;
  long long n = 0;
  for (int i = 0; i < a->count; ++i) {
    if (a->n[i] % 128 != 0) return false;
    n += a->n[i];
  }
  return n / 128 <= LSFA_GEMV_COUNTER_BYTES / 64;
}

GemvSplit gemv_split_mfma(long long M, long long K, long long N) {
  GemvSplit g;
  M = std::max(M, 0LL); K = std::max(K, 0LL); N = std::max(N, 0LL);
  g.kc = (int)std::min(256LL, std::max(64LL, (K + 63) / 64 * 64));
  g.splits = (int)std::max(1LL, (K + g.kc - 1) / g.kc);
  if (g.splits > 1) {
    g.counter_bytes = LSFA_GEMV_COUNTER_BYTES;
    g.bytes = g.counter_bytes + align256((uint64_t)g.splits * M * N * 4);
  }
  return g;
}

GemvSplit gemv_split(long long M, long long K, long long N) {
  GemvSplit g;
  M = std::max(M, 0LL); K = std::max(K, 0LL); N = std::max(N, 0LL);
  const long long col_blocks = std::max(1LL, (N + 255) / 256);
  const long long kc_max = std::min(2048LL, 8192LL / lsfa::gemv_capacity((int)std::min(std::max(M, 1LL), 8LL)));
  long long splits = std::max(1LL, std::min((1024 + col_blocks - 1) / col_blocks, (K + 127) / 128));
  long long kc = std::max(8LL, ((K + splits - 1) / splits + 7) / 8 * 8);
  kc = std::min(kc, kc_max);
  splits = std::max(1LL, (K + kc - 1) / kc);
  g.kc = (int)kc;
  g.splits = (int)splits;
  if (splits > 1) {
    g.counter_bytes = LSFA_GEMV_COUNTER_BYTES;
    g.bytes = g.counter_bytes + align256((uint64_t)splits * M * N * 4);
  }
  return g;
}

lsfa_gemv_group_args gemv_as_group(const lsfa_gemv_args* a) {
  lsfa_gemv_group_args gr;
  memset(&gr, 0, sizeof(gr));
  gr.x = a->x; gr.workspace = a->workspace; gr.workspace_bytes = a->workspace_bytes; gr.x_stride = a->x_stride;
  gr.w[0] = a->w; gr.y[0] = a->y; gr.w_stride[0] = a->w_stride; gr.y_stride[0] = a->y_stride; gr.n[0] = a->n;
  gr.dtype = a->dtype; gr.m = a->m; gr.k = a->k; gr.count = 1;
  return gr;
}

long long gemv_total_n(const lsfa_gemv_group_args* a) {
  long long n = 0;
  for (int i = 0; i < std::min(std::max(a->count, 0), LSFA_GEMV_MAX_GROUP); ++i) n += std::max(a->n[i], 0);
  return n;
}

}  // namespace

extern "C" {

int lsfa_gemv_group_check(const lsfa_gemv_group_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(a->dtype == LSFA_DTYPE_FP32 ? LSFA_ERR_UNSUPPORTED : LSFA_ERR_INVALID,
                "gemv supports bf16 and fp16 (dtype %d)", a->dtype);
  if (a->count < 1 || a->count > LSFA_GEMV_MAX_GROUP)
    return fail(LSFA_ERR_INVALID, "count must be 1..%d (count=%d)", LSFA_GEMV_MAX_GROUP, a->count);
  if (a->m < 0 || a->k < 0) return fail(LSFA_ERR_INVALID, "negative size (m=%d k=%d)", a->m, a->k);
  if (a->m > 8 && !gemv_uses_mfma(a))
    return fail(LSFA_ERR_UNSUPPORTED, "gemv takes at most 8 rows, or 32 without a fused norm, widths that are multiples of "
                "128 and 16-byte aligned x rows (m=%d)", a->m);
  for (int i = 0; i < a->count; ++i) {
    if (a->n[i] < 0) return fail(LSFA_ERR_INVALID, "negative size (n=%d)", a->n[i]);
    if (a->n[i] % 8 != 0) return fail(LSFA_ERR_UNSUPPORTED, "gemv needs n %% 8 == 0 (n=%d)", a->n[i]);
  }
  const long long N = gemv_total_n(a);
  if (N > (long long)LSFA_GEMV_COUNTER_BYTES / 64 * 256)
    return fail(LSFA_ERR_UNSUPPORTED, "gemv takes at most %d columns (n=%lld)", LSFA_GEMV_COUNTER_BYTES / 64 * 256, N);
  if (a->m == 0 || N == 0) return ok();
  if (!a->x) return fail(LSFA_ERR_INVALID, "x, w and y must be non-NULL");
  if (a->x_stride < a->k) return fail(LSFA_ERR_INVALID, "x_stride must be >= k");
  if (a->x_gate && a->x_gate_stride < a->k) return fail(LSFA_ERR_INVALID, "x_gate_stride must be >= k");
  if (a->norm_weight) {
    if (a->x_gate) return fail(LSFA_ERR_INVALID, "norm_weight and x_gate exclude each other");
    if (!(a->eps >= 0.f) || !std::isfinite(a->eps)) return fail(LSFA_ERR_INVALID, "eps must be finite and >= 0");
    if (a->k % 8 != 0 || a->x_stride % 8 != 0 || !aligned16(a->x) || !aligned16(a->norm_weight))
      return fail(LSFA_ERR_UNSUPPORTED, "the fused RMSNorm needs k %% 8 == 0, x rows 16-byte aligned");
    if (a->residual && (a->residual_stride < a->k || a->residual_stride % 8 != 0 || !aligned16(a->residual)))
      return fail(LSFA_ERR_UNSUPPORTED, "residual rows must be 16-byte aligned with residual_stride >= k");
    if (a->residual_out) {
      if (a->residual_out_stride < a->k || a->residual_out_stride % 8 != 0 || !aligned16(a->residual_out))
        return fail(LSFA_ERR_UNSUPPORTED, "residual_out rows must be 16-byte aligned with residual_out_stride >= k");
      const int esz = 2;
      auto span = [&](const void* base, int64_t stride) {
        const uintptr_t b = reinterpret_cast<uintptr_t>(base);
        return std::make_pair(b, b + ((uint64_t)std::max(a->m - 1, 0) * stride + a->k) * esz);
      };
      const auto o = span(a->residual_out, a->residual_out_stride);
      const auto xs = span(a->x, a->x_stride);
      if (o.first < xs.second && xs.first < o.second)
        return fail(LSFA_ERR_INVALID, "residual_out overlaps x (other workgroups still read it)");
      if (a->residual) {
        const auto rs = span(a->residual, a->residual_stride);
        if (o.first < rs.second && rs.first < o.second)
          return fail(LSFA_ERR_INVALID, "residual_out overlaps residual (other workgroups still read it)");
      }
    }
  }
  for (int i = 0; i < a->count; ++i) {
    if (a->n[i] == 0) continue;
    if (!a->w[i] || !a->y[i]) return fail(LSFA_ERR_INVALID, "x, w and y must be non-NULL");
    if (a->w_stride[i] < a->n[i] || a->w_stride[i] % 8 != 0 || !aligned16(a->w[i]))
      return fail(LSFA_ERR_UNSUPPORTED, "w rows must be 16-byte aligned with w_stride >= n and a multiple of 8");
    if (a->y_stride[i] < a->n[i]) return fail(LSFA_ERR_INVALID, "y_stride must be >= n");
  }
  const GemvSplit g = gemv_uses_mfma(a) ? gemv_split_mfma(a->m, a->k, N) : gemv_split(a->m, a->k, N);
  if (g.splits > 65535) return fail(LSFA_ERR_UNSUPPORTED, "k too large for one launch");
  if (g.bytes > 0) {
    if (!a->workspace) return fail(LSFA_ERR_INVALID, "workspace must be non-NULL");
    if (a->workspace_bytes < g.bytes)
      return fail(LSFA_ERR_INVALID, "workspace_bytes %llu is below the %llu bytes lsfa_gemv_workspace_size asks for",
                  (unsigned long long)a->workspace_bytes, (unsigned long long)g.bytes);
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
      return fail(LSFA_ERR_INVALID, "workspace is not 256-byte aligned");
  }
  return ok();
}

int lsfa_gemv_group_workspace_size(const lsfa_gemv_group_args* a, uint64_t* bytes) {
  if (a == nullptr || bytes == nullptr) return fail(LSFA_ERR_INVALID, "args or bytes is NULL");
  const long long N = gemv_total_n(a);
  *bytes = (gemv_uses_mfma(a) ? gemv_split_mfma(a->m, a->k, N) : gemv_split(a->m, a->k, N)).bytes;
  return ok();
}

int lsfa_gemv_group(const lsfa_gemv_group_args* a, void* stream) {
  int rc = lsfa_gemv_group_check(a);
  if (rc) return rc;
  const long long N = gemv_total_n(a);
  if (a->m == 0 || N == 0) return ok();
  const bool mfma = gemv_uses_mfma(a);
  const GemvSplit g = mfma ? gemv_split_mfma(a->m, a->k, N) : gemv_split(a->m, a->k, N);
  lsfa::GemvParams p;
  memset(&p, 0, sizeof(p));
  p.x = a->x;
  p.xg = a->x_gate;
  p.sxg = a->x_gate_stride;
  p.nw = a->norm_weight;
  p.nr = a->residual;
  p.nh = a->residual_out;
  p.snr = a->residual_stride;
  p.snh = a->residual_out_stride;
  p.eps = a->eps;
  int off = 0;
  for (int i = 0; i < 4; ++i) {
    p.col_off[i] = off;
    if (i < a->count) {
      p.w[i] = a->w[i]; p.y[i] = a->y[i]; p.sw[i] = a->w_stride[i]; p.sy[i] = a->y_stride[i];
      off += a->n[i];
    }
  }
  p.col_off[4] = off;
  for (int i = a->count; i < 4; ++i) p.col_off[i] = off;  // unused matrices own no column
  p.groups = a->count;
  if (g.splits > 1) {
    p.counters = static_cast<int*>(a->workspace);
    p.partial = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + g.counter_bytes);
  }
  p.sx = a->x_stride;
  p.M = a->m; p.K = a->k; p.N = (int)N;
  p.kc = g.kc; p.splits = g.splits;
  hipError_t e = mfma ? lsfa::gemv_mfma(p, a->dtype == LSFA_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream))
                      : lsfa::gemv(p, a->dtype == LSFA_DTYPE_BF16, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "gemv launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_gemv_check(const lsfa_gemv_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  const lsfa_gemv_group_args gr = gemv_as_group(a);
  return lsfa_gemv_group_check(&gr);
}

int lsfa_gemv_workspace_size(const lsfa_gemv_args* a, uint64_t* bytes) {
  if (a == nullptr || bytes == nullptr) return fail(LSFA_ERR_INVALID, "args or bytes is NULL");
  const lsfa_gemv_group_args gr = gemv_as_group(a);
  return lsfa_gemv_group_workspace_size(&gr, bytes);
}

int lsfa_gemv(const lsfa_gemv_args* a, void* stream) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  const lsfa_gemv_group_args gr = gemv_as_group(a);
  return lsfa_gemv_group(&gr, stream);
}

int lsfa_greedy_check(const lsfa_greedy_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP32 && a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(LSFA_ERR_INVALID, "unknown dtype %d", a->dtype);
  if (a->rows < 0 || a->cols < 0) return fail(LSFA_ERR_INVALID, "negative size (rows=%d cols=%d)", a->rows, a->cols);
  if (a->rows > 65535) return fail(LSFA_ERR_UNSUPPORTED, "at most 65535 rows per call (rows=%d)", a->rows);
  if (a->rows == 0) return ok();
  if (a->cols == 0) return fail(LSFA_ERR_INVALID, "argmax of an empty row");
  if (!a->logits || !a->tokens) return fail(LSFA_ERR_INVALID, "logits and tokens must be non-NULL");
  if (a->logits_stride < a->cols) return fail(LSFA_ERR_INVALID, "logits_stride must be >= cols");
  return ok();
}

int lsfa_greedy(const lsfa_greedy_args* a, void* stream) {
  int rc = lsfa_greedy_check(a);
  if (rc) return rc;
  hipError_t e = lsfa::greedy(a->logits, a->logits_stride, a->dtype, a->rows, a->cols, a->tokens, a->seq_lens,
                              reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "greedy launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_rope_check(const lsfa_rope_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP32 && a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(LSFA_ERR_INVALID, "unknown dtype %d", a->dtype);
  if (a->batch < 0 || a->seqlen < 0 || a->heads_q < 0 || a->heads_kv < 0 || a->max_pos < 0)
    return fail(LSFA_ERR_INVALID, "negative size (batch=%d seqlen=%d heads_q=%d heads_kv=%d max_pos=%d)",
                a->batch, a->seqlen, a->heads_q, a->heads_kv, a->max_pos);
  const int vec = a->dtype == LSFA_DTYPE_FP32 ? 4 : 8;
  if (a->head_dim <= 0 || a->head_dim % (2 * vec) != 0 || a->head_dim > 1024)
    return fail(LSFA_ERR_UNSUPPORTED, "rope head_dim must be a multiple of %d in %d..1024 (got %d)", 2 * vec,
                2 * vec, a->head_dim);
  if (a->batch == 0 || a->seqlen == 0 || a->heads_q + a->heads_kv == 0) return ok();
  if (a->max_pos <= 0) return fail(LSFA_ERR_INVALID, "max_pos must be positive");
  if (!a->cos || !a->sin) return fail(LSFA_ERR_INVALID, "cos and sin must be non-NULL");
  if (a->heads_q > 0 && !a->q) return fail(LSFA_ERR_INVALID, "q is NULL with heads_q > 0");
  if (a->heads_kv > 0 && !a->k) return fail(LSFA_ERR_INVALID, "k is NULL with heads_kv > 0");
  if (a->table_stride < a->head_dim || a->table_stride % vec != 0)
    return fail(LSFA_ERR_UNSUPPORTED, "table_stride %lld must be >= head_dim and a multiple of %d",
                (long long)a->table_stride, vec);
  if (!aligned16(a->cos) || !aligned16(a->sin)) return fail(LSFA_ERR_UNSUPPORTED, "cos/sin must be 16-byte aligned");
  const bool varlen = a->cu_seqlens != nullptr;
  for (int t = 0; t < 2; ++t) {
    const int64_t* st = t == 0 ? a->q_stride : a->k_stride;
    const void* ptr = t == 0 ? a->q : a->k;
    if ((t == 0 ? a->heads_q : a->heads_kv) == 0) continue;
    const char* name = t == 0 ? "q" : "k";
    if (st[3] != 1) return fail(LSFA_ERR_UNSUPPORTED, "%s: head-dim stride must be 1 (got %lld)", name, (long long)st[3]);
    for (int i = varlen ? 1 : 0; i < 3; ++i)
      if (st[i] % vec != 0)
        return fail(LSFA_ERR_UNSUPPORTED, "%s: stride[%d]=%lld is not a multiple of %d elements", name, i,
                    (long long)st[i], vec);
    if (!aligned16(ptr)) return fail(LSFA_ERR_UNSUPPORTED, "%s: base pointer is not 16-byte aligned", name);
  }
  if (a->k_cache != nullptr) {
    if (a->heads_kv == 0 || !a->v || !a->v_cache || (!a->slots && !a->block_tables))
      return fail(LSFA_ERR_INVALID, "a K/V cache append needs heads_kv > 0, non-NULL v and v_cache, and slots "
                  "or block_tables");
    if (a->block_tables && (a->block_size <= 0 || a->max_blocks_per_seq < 0 ||
                            a->block_table_stride < a->max_blocks_per_seq))
      return fail(LSFA_ERR_INVALID, "block_tables needs block_size > 0 and block_table_stride >= max_blocks_per_seq");
    if (a->num_slots < 0) return fail(LSFA_ERR_INVALID, "num_slots must be >= 0");
    if (a->v_stride[3] != 1 || !aligned16(a->v))
      return fail(LSFA_ERR_UNSUPPORTED, "v: head-dim stride must be 1 and the pointer 16-byte aligned");
    for (int i = varlen ? 1 : 0; i < 3; ++i)
      if (a->v_stride[i] % vec != 0)
        return fail(LSFA_ERR_UNSUPPORTED, "v: stride[%d] is not a multiple of %d elements", i, vec);
    if (a->cache_stride[0] < (int64_t)a->heads_kv * a->head_dim || a->cache_stride[1] < a->head_dim ||
        a->cache_stride[0] % vec != 0 || a->cache_stride[1] % vec != 0 || !aligned16(a->k_cache) ||
        !aligned16(a->v_cache))
      return fail(LSFA_ERR_UNSUPPORTED, "caches: slot/head strides must cover a row and be multiples of %d "
                  "elements, pointers 16-byte aligned", vec);
  }
  return ok();
}

int lsfa_rope(const lsfa_rope_args* a, void* stream) {
  int rc = lsfa_rope_check(a);
  if (rc) return rc;
  if (a->batch == 0 || a->seqlen == 0 || a->heads_q + a->heads_kv == 0) return ok();
  lsfa::RopeParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.k = a->k; p.cos = a->cos; p.sin = a->sin;
  p.pos0 = a->positions; p.cu_seqlens = a->cu_seqlens;
  for (int i = 0; i < 4; ++i) {
    p.sq[i] = a->q_stride[i];
    p.sk[i] = a->k_stride[i];
  }
  p.table_stride = a->table_stride;
  p.B = a->batch; p.N = a->seqlen; p.Hq = a->heads_q; p.Hkv = a->heads_kv; p.D = a->head_dim;
  p.max_pos = a->max_pos;
  if (a->k_cache != nullptr) {
    p.v = a->v; p.k_cache = a->k_cache; p.v_cache = a->v_cache; p.slots = a->slots;
    for (int i = 0; i < 4; ++i) p.sv[i] = a->v_stride[i];
    p.cs_slot = a->cache_stride[0]; p.cs_head = a->cache_stride[1]; p.num_slots = a->num_slots;
    p.block_tables = a->block_tables; p.sbt = a->block_table_stride;
    p.block_size = a->block_size; p.max_blocks = a->max_blocks_per_seq;
  }
  hipError_t e = lsfa::rope_inplace(p, a->dtype, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "rope launch failed: %s", hipGetErrorString(e));
  return ok();
}

int lsfa_rmsnorm_check(const lsfa_rmsnorm_args* a) {
  if (a == nullptr) return fail(LSFA_ERR_INVALID, "args is NULL");
  if (a->dtype != LSFA_DTYPE_FP32 && a->dtype != LSFA_DTYPE_FP16 && a->dtype != LSFA_DTYPE_BF16)
    return fail(LSFA_ERR_INVALID, "unknown dtype %d", a->dtype);
  if (a->rows < 0 || a->cols < 0) return fail(LSFA_ERR_INVALID, "negative size (rows=%d cols=%d)", a->rows, a->cols);
  if (!(a->eps >= 0.f) || !std::isfinite(a->eps)) return fail(LSFA_ERR_INVALID, "eps must be finite and >= 0");
  if (a->rows == 0 || a->cols == 0) return ok();
  if (!a->x || !a->weight || !a->out) return fail(LSFA_ERR_INVALID, "x, weight and out must be non-NULL");
  if (a->x_stride < a->cols || a->out_stride < a->cols || (a->residual && a->residual_stride < a->cols) ||
      (a->residual_out && a->residual_out_stride < a->cols))
    return fail(LSFA_ERR_INVALID, "row strides must be at least cols (%d)", a->cols);
  return ok();
}

int lsfa_rmsnorm(const lsfa_rmsnorm_args* a, void* stream) {
  int rc = lsfa_rmsnorm_check(a);
  if (rc) return rc;
  if (a->rows == 0 || a->cols == 0) return ok();
  lsfa::NormParams p;
  memset(&p, 0, sizeof(p));
  p.x = a->x; p.residual = a->residual; p.weight = a->weight; p.out = a->out; p.residual_out = a->residual_out;
  p.sx = a->x_stride; p.sr = a->residual_stride; p.so = a->out_stride; p.sh = a->residual_out_stride;
  p.rows = a->rows; p.cols = a->cols; p.eps = a->eps;
  // 16-byte path: width and every row stride a multiple of 16 bytes, aligned
  // pointers, and the row fits 8 groups per thread.
  const int vec = a->dtype == LSFA_DTYPE_FP32 ? 4 : 8;
  bool v = a->cols % vec == 0 && a->cols <= 256 * vec * 8 && a->x_stride % vec == 0 && a->out_stride % vec == 0 &&
           aligned16(a->x) && aligned16(a->out) && aligned16(a->weight);
  if (a->residual) v = v && a->residual_stride % vec == 0 && aligned16(a->residual);
  if (a->residual_out) v = v && a->residual_out_stride % vec == 0 && aligned16(a->residual_out);
  hipError_t e = lsfa::add_rmsnorm(p, a->dtype, v, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(LSFA_ERR_LAUNCH, "rmsnorm launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
