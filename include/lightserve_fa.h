/*
 * lightserve_fa.h -- C ABI of the gfx950 (MI355X) FlashAttention library
 * (liblsfa_gfx950.so).
 *
 * This boundary replaces the Triton launches of lightserve's attention hot
 * path. Every entry point takes plain device pointers, element strides and
 * sizes (no framework types), enqueues work on the caller's stream, never
 * allocates, frees or synchronises, and picks its kernel as a pure function
 * of (dtype, head_dim, causal, varlen). That keeps it safe under stream/graph
 * capture (the reference captures the forward inside torch.cuda.graph,
 * model/cuda_graph_decode.py:137-139).
 *
 * Conventions shared by all entry points
 *   - Layout of q/k/v/o/do/dq/dk/dv: [batch, heads, seqlen, head_dim] with
 *     arbitrary element strides (index 0..3 = b, h, n, d), as the reference
 *     passes all four strides per tensor (kernels/flash_attention.py:211-218).
 *     The fast path requires stride[3] == 1, the other strides and head_dim to
 *     be multiples of 8 elements, and 16-byte aligned base pointers; other
 *     layouts are rejected with LSFA_ERR_UNSUPPORTED (the Python layer makes
 *     a packed copy first).
 *   - Varlen ("packed THD") mode: cu_seqlens_q / cu_seqlens_k are device
 *     int32 arrays of batch+1 prefix offsets. Tensors are then [total_tokens,
 *     heads, head_dim]; stride[0] is ignored, stride[1] is the head stride and
 *     stride[2] the token stride. seqlen_q / seqlen_k give the maximum
 *     per-sequence lengths. lse is [heads, total_q] (lse_stride[1] = head
 *     stride, lse_stride[2] = token stride).
 *   - Causal masking is bottom-right aligned: query i of a sequence with
 *     Nq queries and Nk keys sees keys j <= i + (Nk - Nq). With Nq == Nk this
 *     is the reference's `offs_m >= offs_n` (kernels/flash_attention.py:152).
 *   - Scores are S = (q . k) * sm_scale in fp32; lse = m + ln(l) per query row
 *     in natural-log, scaled-score units (kernels/flash_attention_backward.py:162).
 *     A row that sees no key gets o = 0 and lse = -inf.
 *   - GQA: query head h reads kv head h / (heads_q / heads_kv).
 *   - Return value: LSFA_OK (0) or a negative lsfa_status; the message of the
 *     last failure on the calling thread is returned by lsfa_last_error().
 */
#ifndef LIGHTSERVE_FA_H
#define LIGHTSERVE_FA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSFA_ABI_VERSION 9

typedef enum {
  LSFA_DTYPE_FP32 = 0,
  LSFA_DTYPE_FP16 = 1,
  LSFA_DTYPE_BF16 = 2
} lsfa_dtype;

typedef enum {
  LSFA_OK = 0,
  LSFA_ERR_INVALID = -1,     /* malformed arguments (null pointer, bad sizes) */
  LSFA_ERR_UNSUPPORTED = -2, /* valid but outside what the kernels implement */
  LSFA_ERR_LAUNCH = -3       /* the HIP runtime refused the launch */
} lsfa_status;

/* Forward arguments. lse may be NULL (inference forward, which the reference
 * returns without logsumexp: kernels/flash_attention.py:182-222). */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t lse_stride[3];
  const int32_t* cu_seqlens_q; /* NULL unless varlen */
  const int32_t* cu_seqlens_k; /* NULL unless varlen */
  int32_t dtype;               /* lsfa_dtype; q, k, v and o share it */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t seqlen_q;            /* varlen: max_seqlen_q */
  int32_t seqlen_k;            /* varlen: max_seqlen_k */
  int32_t head_dim;            /* 1..128 */
  int32_t causal;
  float sm_scale;
  int32_t reserved;
} lsfa_fwd_args;

/* Backward arguments. workspace is caller-allocated device memory of at
 * least lsfa_bwd_workspace_size() bytes, 256-byte aligned; its contents on
 * entry do not matter and are scratch afterwards. It receives what the
 * reference's preprocess kernel computes (delta = rowsum(dO * O),
 * kernels/flash_attention_backward.py:202-229, stored negated) with
 * L*log2(e) per query row.
 * By default a query-stationary kernel produces dq and a key-stationary one
 * dk and dv, each computing S and dP itself. With LSFA_BWD_STORED_DS (bf16 /
 * fp16 at head_dim above 64) the key-stationary kernel also stores dS (in
 * the input dtype) into the workspace and dq = scale * dS K is a GEMM over
 * the stored values, so S and dP are computed once per (query, key): the
 * dS region is (seqlen_k rounded up to 32) x (seqlen_q rounded up to 256)
 * elements per head for as many heads as fit in 4 GiB (at least one), and
 * larger problems run chunk by chunk. dq/dk/dv are written in the input
 * dtype (no fp32 dq staging buffer and no atomics, so results are
 * deterministic). */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  void* dq;
  void* dk;
  void* dv;
  void* workspace;
  uint64_t workspace_bytes;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  int64_t do_stride[4];
  int64_t dq_stride[4];
  int64_t dk_stride[4];
  int64_t dv_stride[4];
  int64_t lse_stride[3];
  const int32_t* cu_seqlens_q; /* NULL, or packed varlen as in lsfa_fwd_args (bf16/fp16 without
                                  LSFA_BWD_STORED_DS): q/o/dout/dq rows of sequence b at
                                  cu_seqlens_q[b] .., k/v/dk/dv rows at cu_seqlens_k[b] .., strides
                                  [0, head, row, 1], lse [heads_q, total_q], seqlen_q / seqlen_k the
                                  longest sequences (longer ones are clamped to them) */
  const int32_t* cu_seqlens_k;
  int32_t dtype;
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;            /* divides heads_q; below heads_q (GQA: query head h reads KV head
                                  h / (heads_q / heads_kv), and dk / dv [batch, heads_kv, seqlen_k,
                                  head_dim] sum over the heads_q / heads_kv query heads of their group)
                                  only for bf16/fp16 without LSFA_BWD_STORED_DS */
  int32_t seqlen_q;
  int32_t seqlen_k;
  int32_t head_dim;
  int32_t causal;
  float sm_scale;
  int32_t flags;               /* 0, or LSFA_BWD_ONLY_* and / or LSFA_BWD_STORED_DS */
} lsfa_bwd_args;

/* lsfa_bwd_args.flags: at most one LSFA_BWD_ONLY_* phase, for timing the
 * kernels of a bf16/fp16 backward one at a time (a profiler or benchmark;
 * without one every kernel runs, in order), optionally with
 * LSFA_BWD_STORED_DS.
 * Default path: LSFA_BWD_ONLY_DQ runs the query-stationary kernel alone (it
 * writes dq and the per-row values); LSFA_BWD_ONLY_DKDV runs the
 * key-stationary kernel alone and reads those values, so it needs a
 * workspace that an earlier full or ONLY_DQ call filled.
 * Stored-dS path (LSFA_BWD_STORED_DS at head_dim above 64; the flag is
 * ignored elsewhere): LSFA_BWD_ONLY_DKDV runs the per-row preprocess and the
 * key-stationary kernel (dk, dv, and dS into the workspace);
 * LSFA_BWD_ONLY_DQ runs the dq GEMM alone over the dS that an earlier full
 * or ONLY_DKDV call with the same arguments and workspace left (problems
 * that run in more than one chunk of heads take no ONLY_* flag).
 * The fp32 path takes no ONLY_* flag. */
#define LSFA_BWD_ONLY_DQ 1
#define LSFA_BWD_ONLY_DKDV 2
#define LSFA_BWD_STORED_DS 4

/* Paged-KV decode arguments: one new query token per sequence against a KV
 * cache addressed through block tables. The reference has no such kernel;
 * its engine documents it as the missing decode path (engine/README.md,
 * "No decode-shaped attention kernel": Nq = 1 against a paged Nkv, gathering
 * K/V across a request's block_table).
 *   q          [batch, heads_q, head_dim]
 *   k_cache,
 *   v_cache    [num_blocks, block_size, heads_kv, head_dim] (a block holds
 *              block_size x n_kv_heads x head_dim elements per layer,
 *              engine/config.py:5-7)
 *   block_tables int32 [batch, max_blocks_per_seq]; entry i holds the
 *              physical block of tokens [i*block_size, (i+1)*block_size)
 *              (engine/block_manager.py:56-60)
 *   seq_lens   int32 [batch]: cached tokens per sequence, the new token's K/V
 *              included; clamped on the device to max_seq_len and to
 *              max_blocks_per_seq * block_size
 *   o          like q; lse fp32 [batch, heads_q] (natural log) or NULL
 * Query head h reads KV head h / (heads_q / heads_kv). Block ids outside
 * [0, num_blocks) read as zeros. workspace: lsfa_decode_workspace_size()
 * bytes, 256-byte aligned (0 bytes when no sequence is split). */
typedef struct {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* o;
  float* lse;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  void* workspace;
  uint64_t workspace_bytes;
  int64_t q_stride[3];         /* batch, head, dim */
  int64_t k_stride[4];         /* block, slot, head, dim */
  int64_t v_stride[4];
  int64_t o_stride[3];
  int64_t lse_stride[2];
  int64_t block_table_stride;  /* elements between consecutive sequences' tables */
  int32_t dtype;               /* bf16 or fp16 */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;            /* heads_q / heads_kv <= 32 (block_size >= 16), else in {1, 2, 4, 8} */
  int32_t head_dim;            /* multiple of 8, at most 128 */
  int32_t block_size;          /* power of two */
  int32_t num_blocks;
  int32_t max_blocks_per_seq;
  int32_t max_seq_len;         /* upper bound of seq_lens (sets the split) */
  float sm_scale;
} lsfa_decode_args;

/* Rotary position embedding, applied in place to q and k in one launch.
 * Replaces the reference's apply_rope (model/minimal_llama.py:163-173):
 * for each token at position pos and each head,
 *   x[..., :D/2] <- x1 * cos[pos, :D/2] - x2 * sin[pos, :D/2]
 *   x[..., D/2:] <- x2 * cos[pos, D/2:] + x1 * sin[pos, D/2:]
 * with x1 = x[..., :D/2], x2 = x[..., D/2:] (x * cos + rotate_half(x) * sin),
 * computed in fp32 and rounded once to the tensor's dtype.
 *   q          [batch, heads_q, seqlen, head_dim], element strides (b, h, n, d)
 *   k          [batch, heads_kv, seqlen, head_dim], or NULL with heads_kv = 0
 *   cos, sin   [max_pos, head_dim] rows in q's dtype (the reference's
 *              precompute_rope tables, model/minimal_llama.py:144-156);
 *              table_stride = elements between rows
 *   positions  int32 [batch]: position of each sequence's first token, or
 *              NULL for 0 (prefill from the start); token n sits at
 *              positions[b] + n, clamped on the device to [0, max_pos)
 *   cu_seqlens int32 [batch + 1] or NULL: packed [total_tokens, heads,
 *              head_dim] tensors as in lsfa_fwd_args (stride[0] ignored,
 *              stride[1] head, stride[2] token); seqlen = max tokens per
 *              sequence
 * head_dim must be even with head_dim/2 a multiple of 8 (bf16/fp16) or 4
 * (fp32) elements; stride[3] == 1, other strides multiples of 8 (bf16/fp16)
 * or 4 (fp32) elements, 16-byte aligned pointers.
 * Optional K/V cache append (k_cache non-NULL; the reference model has no
 * cache, its engine's block layout is engine/block_manager.py:56-60): the
 * rotated k row and v's row of token t are also stored at slot slots[t] of
 * k_cache / v_cache ([num_blocks, block_size, heads_kv, head_dim] caches
 * addressed as slots; cache_stride = elements between slots and between
 * heads, head-dim stride 1). t = b * seqlen + n, or the packed index with
 * cu_seqlens. Slots outside [0, num_slots) are skipped (a negative slot marks
 * a padding token). v has k's shape, v_stride its strides. Instead of slots,
 * block_tables (int32 [batch, max_blocks_per_seq], row stride
 * block_table_stride) may name them: token n of sequence b at position
 * p = positions[b] + n goes to block_tables[b, p / block_size] * block_size +
 * p % block_size (the engine's paging, engine/block_manager.py:56-60);
 * positions past the table or block ids outside [0, num_slots / block_size)
 * are skipped. */
typedef struct {
  void* q;
  void* k;
  const void* cos;
  const void* sin;
  const int32_t* positions;
  const int32_t* cu_seqlens;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t table_stride;
  int32_t dtype;
  int32_t batch;
  int32_t seqlen;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;
  int32_t max_pos;
  int32_t reserved;
  const void* v;
  void* k_cache;
  void* v_cache;
  const int64_t* slots;
  int64_t v_stride[4];
  int64_t cache_stride[2];
  int64_t num_slots;
  const int32_t* block_tables;
  int64_t block_table_stride;
  int32_t block_size;
  int32_t max_blocks_per_seq;
} lsfa_rope_args;

/* Fused residual add + RMSNorm over the rows of [rows, cols] matrices
 * (column stride 1; row strides in elements). Replaces the reference's
 * fused_add_rmsnorm launch (kernels/fused_rmsnorm_residual.py:73-118):
 *   h   = x + residual            (rounded to the dtype; residual_out <- h)
 *   out = h * rsqrt(mean(h^2) + eps) * weight   (fp32 statistics, rounded once)
 * residual = NULL gives plain RMSNorm (h = x); residual_out = NULL skips
 * writing h. out and residual_out may alias x or residual with the same row
 * stride (each element is read before it is written, by the same thread).
 * weight: [cols]. */
typedef struct {
  const void* x;
  const void* residual;
  const void* weight;
  void* out;
  void* residual_out;
  int64_t x_stride;
  int64_t residual_stride;
  int64_t out_stride;
  int64_t residual_out_stride;
  int32_t dtype;
  int32_t rows;
  int32_t cols;
  float eps;
} lsfa_rmsnorm_args;

/* Chunked prefill against a paged KV cache: a chunk of new query tokens per
 * sequence attends to that sequence's cached keys (its earlier chunks and,
 * written into the cache beforehand, the chunk itself). The reference's
 * engine documents this as its missing prefill path (engine/request.py:86-93,
 * engine/scheduler.py:34-44: num_scheduled_tokens > 1 has no kernel); the
 * cache layout and block tables are its engine's (engine/config.py:5-7,
 * engine/block_manager.py:56-60).
 *   q          packed [total_q, heads_q, head_dim]; sequence b owns rows
 *              cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1
 *   k_cache,
 *   v_cache    [num_blocks, block_size, heads_kv, head_dim]
 *   block_tables int32 [batch, max_blocks_per_seq]
 *   seq_lens_k int32 [batch]: cached keys of sequence b, the chunk included;
 *              clamped on the device to max_blocks_per_seq * block_size
 *   o          like q; lse fp32 [heads_q, total_q] (natural log) or NULL
 * Causal masking is bottom-right aligned: query i of a chunk of n sits at
 * position seq_lens_k[b] - n + i. Query head h reads KV head
 * h / (heads_q / heads_kv). Block ids outside [0, num_blocks) read as zeros.
 * block_size is a power of two and at least 16. */
typedef struct {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* o;
  float* lse;
  const int32_t* cu_seqlens_q;
  const int32_t* seq_lens_k;
  const int32_t* block_tables;
  int64_t q_stride[2];         /* token, head (head-dim stride 1) */
  int64_t k_stride[3];         /* block, slot, head */
  int64_t v_stride[3];
  int64_t o_stride[2];
  int64_t lse_stride[2];       /* head, token */
  int64_t block_table_stride;
  int32_t dtype;               /* bf16 or fp16 */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;            /* multiple of 8, at most 128 */
  int32_t block_size;
  int32_t num_blocks;
  int32_t max_blocks_per_seq;
  int32_t max_seqlen_q;        /* upper bound of the chunk lengths (sets the grid) */
  int32_t causal;
  float sm_scale;
  int32_t reserved;
} lsfa_prefill_paged_args;

/* Skinny GEMM for decode-time projections: y[M, N] = x[M, K] @ w[K, N] with
 * M <= 8 (up to 32 when every width is a multiple of 128, x rows are 16-byte
 * aligned and the input is x or x with a gate, not a norm: those run on
 * MFMA), w in the reference
 * model's [in, out] row-major weight layout
 * (model/minimal_llama.py: every Linear is x @ w), bf16 or fp16, fp32
 * accumulate, one rounding. The reference calls its tiled GEMM for these
 * (kernels/tiled_matmul.py:135-164, through model/minimal_llama.py:178-182);
 * this entry point serves the rows-per-call of a decode step, where a GEMM's
 * tiles are mostly empty and the product is one HBM pass over w.
 *   x [M, K], y [M, N]: row strides in elements, columns contiguous
 *   w [K, N]: row stride w_stride >= N, columns contiguous; N % 8 == 0
 *   workspace: lsfa_gemv_workspace_size() bytes (0 when K needs no split),
 *   256-byte aligned: the first LSFA_GEMV_COUNTER_BYTES hold int32 arrival
 *   counters (16 per 256 columns of y, hence n <= 1048576), then the fp32
 *   partial sums of the K-splits. The counter bytes must be zero the first
 *   time a workspace is used; every call leaves them zero, so calls in stream
 *   order, of any shape, may reuse one workspace. Calls that can run at the
 *   same time need workspaces of their own. */
#define LSFA_GEMV_COUNTER_BYTES 262144
typedef struct {
  const void* x;
  const void* w;
  void* y;
  void* workspace;
  uint64_t workspace_bytes;
  int64_t x_stride;
  int64_t w_stride;
  int64_t y_stride;
  int32_t dtype;
  int32_t m;
  int32_t k;
  int32_t n;
} lsfa_gemv_args;

/* Grouped skinny GEMM: y_i = x @ w_i for count <= LSFA_GEMV_MAX_GROUP weight
 * matrices that share x (and so K), e.g. a decoder's q/k/v or gate/up
 * projections, as one launch over their concatenated columns. Each w_i / y_i
 * follows the rules of lsfa_gemv_args; the workspace (counters, then partials
 * of all columns) follows them for n = n[0] + ... + n[count-1].
 * x_gate (optional, NULL for none; [M, K] with row stride x_gate_stride):
 * the products read silu(x_gate) * x instead of x, each rounded to the dtype
 * as torch rounds F.silu(gate) * up (the SwiGLU input of a down projection,
 * model/minimal_llama.py's mlp).
 * norm_weight (optional, NULL for none; [K]): the products read
 * rmsnorm(x + residual) * norm_weight, computed exactly as lsfa_rmsnorm
 * computes out (fp32 statistics; the reference's fused_add_rmsnorm,
 * kernels/fused_rmsnorm_residual.py:30-70), so the norm before a projection
 * needs no launch of its own. residual (optional, [M, K], row stride
 * residual_stride) is added first; residual_out (optional, [M, K]) receives
 * h = x + residual and must not overlap x or residual. Needs K % 8 == 0,
 * 16-byte aligned rows and row strides that are multiples of 8 elements;
 * excludes x_gate. */
#define LSFA_GEMV_MAX_GROUP 4
typedef struct {
  const void* x;
  void* workspace;
  uint64_t workspace_bytes;
  int64_t x_stride;
  const void* x_gate;
  int64_t x_gate_stride;
  const void* w[LSFA_GEMV_MAX_GROUP];
  void* y[LSFA_GEMV_MAX_GROUP];
  int64_t w_stride[LSFA_GEMV_MAX_GROUP];
  int64_t y_stride[LSFA_GEMV_MAX_GROUP];
  int32_t n[LSFA_GEMV_MAX_GROUP];
  int32_t dtype;
  int32_t m;
  int32_t k;
  int32_t count;
  const void* norm_weight;
  const void* residual;
  void* residual_out;
  int64_t residual_stride;
  int64_t residual_out_stride;
  float eps;
  int32_t reserved;
} lsfa_gemv_group_args;

/* Greedy next token of a decode step: tokens[r] = argmax over logits[r, :]
 * (comparison as torch's argmax: NaN beats every number, ties go to the
 * lower index) and, when seq_lens is non-NULL, seq_lens[r] += 1. Replaces the
 * reference's torch argmax and length update after each step
 * (model/cuda_graph_decode.py:114, :145).
 *   logits [rows, cols] fp32/fp16/bf16, row stride in elements, columns
 *   contiguous; tokens int64 [rows]; seq_lens int32 [rows] or NULL */
typedef struct {
  const void* logits;
  int64_t* tokens;
  int32_t* seq_lens;
  int64_t logits_stride;
  int32_t dtype;
  int32_t rows;
  int32_t cols;
  int32_t reserved;
} lsfa_greedy_args;

/* ABI version of the loaded library (LSFA_ABI_VERSION). */
int lsfa_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* lsfa_last_error(void);

/* Host-only validation of forward arguments; never touches the GPU.
 * Mirrors the reference's argument checks (kernels/flash_attention.py:192-199)
 * plus the layout requirements of the gfx950 kernels. */
int lsfa_fwd_check(const lsfa_fwd_args* args);

/* Forward: o = softmax(q k^T * sm_scale) v, and lse if requested.
 * Replaces the launch of _flash_attn_fwd_kernel (kernels/flash_attention.py:210-221)
 * and of _flash_attn_fwd_lse_kernel (kernels/flash_attention_backward.py:186-198).
 * stream is a hipStream_t (NULL = the default stream). */
int lsfa_fwd(const lsfa_fwd_args* args, void* stream);

/* Host-only validation of backward arguments; never touches the GPU. */
int lsfa_bwd_check(const lsfa_bwd_args* args);

/* Workspace bytes lsfa_bwd needs for these arguments (only dtype, flags,
 * batch, heads_q, seqlen_q, seqlen_k and head_dim matter: head_dim decides
 * whether LSFA_BWD_STORED_DS applies); no GPU work. */
int lsfa_bwd_workspace_size(const lsfa_bwd_args* args, uint64_t* bytes);

/* Backward: delta, then dk, dv and dq. Replaces the preprocess launch
 * (kernels/flash_attention_backward.py:341-350), the backward launch
 * (:363-381) and the fp32->dtype cast of dq (:382). */
int lsfa_bwd(const lsfa_bwd_args* args, void* stream);

/* Allocation-free backward. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * training or serving loops that forbid allocation). Same arguments, kernels
 * and results as lsfa_bwd with LSFA_BWD_STORED_DS cleared from flags (the
 * default kernels need only the per-row values), except that workspace and
 * workspace_bytes are ignored: the workspace is a device array of
 * LSFA_BWD_SCRATCH_BYTES inside the library (one per GPU, held while the
 * library is loaded), so problems needing more (batch * heads_q * seqlen_q
 * rounded up to 128 above 2097152 rows) are rejected with
 * LSFA_ERR_UNSUPPORTED. Calls share their GPU's array: two calls that can run
 * at the same time on one GPU (different streams) race; calls in stream order
 * do not. Nothing in the array needs clearing between calls (each call
 * writes the per-row values before reading them; an LSFA_BWD_ONLY_DKDV call
 * reads what the last full or ONLY_DQ call on that GPU left). The first call
 * on a device looks up that device's copy of the array (a host query, not a
 * stream operation). */
#define LSFA_BWD_SCRATCH_BYTES 16777216
int lsfa_bwd_noalloc(const lsfa_bwd_args* args, void* stream);

/* Host-only validation of decode arguments; never touches the GPU. */
int lsfa_decode_check(const lsfa_decode_args* args);

/* Workspace bytes lsfa_decode needs (split partial outputs); no GPU work. */
int lsfa_decode_workspace_size(const lsfa_decode_args* args, uint64_t* bytes);

/* Paged-KV decode: o = softmax(q K^T * sm_scale) V over each sequence's
 * seq_lens[b] cached tokens (and lse if requested). No reference
 * counterpart (see lsfa_decode_args). */
int lsfa_decode(const lsfa_decode_args* args, void* stream);

/* Host-only validation of RoPE arguments; never touches the GPU. */
int lsfa_rope_check(const lsfa_rope_args* args);

/* In-place RoPE of q and k (see lsfa_rope_args). */
int lsfa_rope(const lsfa_rope_args* args, void* stream);

/* Host-only validation of paged-prefill arguments; never touches the GPU. */
int lsfa_prefill_paged_check(const lsfa_prefill_paged_args* args);

/* Chunked prefill over a paged KV cache (see lsfa_prefill_paged_args): the
 * forward kernel of lsfa_fwd with K/V tiles gathered through the block
 * tables. No reference counterpart. */
int lsfa_prefill_paged(const lsfa_prefill_paged_args* args, void* stream);

/* Host-only validation of skinny-GEMM arguments; never touches the GPU. */
int lsfa_gemv_check(const lsfa_gemv_args* args);

/* Workspace bytes lsfa_gemv needs (m, k and n matter); no GPU work. */
int lsfa_gemv_workspace_size(const lsfa_gemv_args* args, uint64_t* bytes);

/* y = x @ w for m <= 8 rows (see lsfa_gemv_args): one launch on the stream,
 * a K-split pass over w whose last-arriving workgroup per column block sums
 * the splits (in split order: deterministic) and rounds once into y. */
int lsfa_gemv(const lsfa_gemv_args* args, void* stream);

/* The grouped form (lsfa_gemv_group_args): validation, workspace size, launch. */
int lsfa_gemv_group_check(const lsfa_gemv_group_args* args);
int lsfa_gemv_group_workspace_size(const lsfa_gemv_group_args* args, uint64_t* bytes);
int lsfa_gemv_group(const lsfa_gemv_group_args* args, void* stream);

/* Host-only validation of greedy-token arguments; never touches the GPU. */
int lsfa_greedy_check(const lsfa_greedy_args* args);

/* Greedy next token (see lsfa_greedy_args): one launch, one workgroup per row. */
int lsfa_greedy(const lsfa_greedy_args* args, void* stream);

/* Host-only validation of RMSNorm arguments; never touches the GPU. */
int lsfa_rmsnorm_check(const lsfa_rmsnorm_args* args);

/* Fused residual add + RMSNorm (see lsfa_rmsnorm_args). */
int lsfa_rmsnorm(const lsfa_rmsnorm_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LIGHTSERVE_FA_H */
