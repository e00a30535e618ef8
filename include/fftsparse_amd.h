/*
 * fftsparse_amd -- C ABI of the MI355X (gfx950) FFTSparse prefill path.
 *
 * Plain pointers, sizes and strides only.  Every pointer named "device" is
 * device memory owned by the caller; every entry point is stream-ordered on
 * the given hipStream_t (passed as void*), launches kernels only, allocates
 * nothing and never synchronises the host.  Return value: FS_OK (0) or a
 * negative status; fs_last_error() then describes the failure (thread-local).
 *
 * Reference interfaces replaced (paths relative to the FFTSparse repository):
 *   fs_pool      block_mean_pool              attn_src/fft_attn/my_attn_v7.py:105-114 (call :553-555)
 *   fs_rope_pool the rotary embedding before the call (eval/LongBench/pred.py:195, transformers
 *                apply_rotary_pos_emb) fused with block_mean_pool (my_attn_v7.py:105-114)
 *   fs_corr      batch_fft_cross_correlation  my_attn_v7.py:117-157
 *                + threshold lag selection     my_attn_v7.py:190-208 (create_correlation_block_mask)
 *   fs_stats     compute_stripe_variance      my_attn_v7.py:301-363 (diagonal statistics)
 *                create_column_block_mask     my_attn_v7.py:390-447 (column scores + top-n)
 *                create_last_block_query_mask my_attn_v7.py:54-72
 *   fs_scores    fs_corr + fs_stats for bf16/f16 inputs, from MFMA tiles of
 *                the block scores (the same reference lines)
 *   fs_select    mask composition             my_attn_v7.py:542-550, 588-641 (prior | dynamic | column)
 *                create_qk_topk_block_mask    my_attn_v7.py:256-294 (diffuse heads)
 *                create_deterministic_block_mask attn_src/fix_mask_attn/my_attn.py:39-79 (fixed role)
 *                The dense [1,H,N,N] bool mask the reference hands to the
 *                kernel (my_attn_v7.py:710,780) is kept as a row bitmask (see
 *                "Block masks" below): the same mask, one bit per block.
 *   fs_xattn     XAttention's selector        attn_src/xattn/src/Xattention.py:14-303 (xattn_estimate),
 *                                            utils.py:44-200 (find_blocks_chunked); the mask its
 *                                            Xattention_prefill (:306-406) hands to block_sparse_attn_func
 *   fs_flex      FlexPrefill's selector       attn_src/Flexprefill.py:946-1061 (get_active_blocks), the
 *                                            block index sets its Flexprefill_prefill (:1063-1098) attends
 *   fs_bsattn    block_sparse_attn_func call  my_attn_v7.py:775-786, fix_mask_attn/my_attn.py:196-207
 *                flash_attn_func(causal=True) my_attn_v7.py:509-519 (blk_cnt == NULL: dense causal)
 */
#ifndef FFTSPARSE_AMD_H
#define FFTSPARSE_AMD_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define FS_API __attribute__((visibility("default")))
#else
#define FS_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum { FS_DTYPE_F32 = 0, FS_DTYPE_BF16 = 1, FS_DTYPE_F16 = 2 };

enum {
  FS_OK = 0,
  FS_ERR_ARG = -1,          /* invalid argument (shape, stride, null pointer) */
  FS_ERR_UNSUPPORTED = -2,  /* valid but not implemented (dtype, head dim, size) */
  FS_ERR_LAUNCH = -3        /* the HIP runtime rejected a launch */
};

/* ---- Block masks ---------------------------------------------------------
 * Every selector writes, and fs_bsattn reads, the block mask as a row
 * bitmask plus a count per row:
 *   blk_bits[(h * N + i) * NW + w], NW = ceil(Nk / 64), 64-bit words: bit b of
 *     word w is set iff query-block row i of head h selects key block 64 w + b
 *     (bits at 64 w + b >= Nk are 0);
 *   blk_cnt[h * N + i] = the number of set bits of the row.
 * It is the reference's base_blockmask bool [1, H, N, N] (my_attn_v7.py:710,
 * 780) with one bit per block: N * NW * 8 bytes per head (4 MiB for 32 heads at
 * N = 1024, 256 MiB at N = 8192), whatever the number of selected blocks, and
 * rows are written independently (no prefix sum over rows, no host sync). */
#define FS_MASK_WORDS(Nk) (((Nk) + 63) / 64)

/* ---- block pooling (my_attn_v7.py:105-114) ------------------------------
 * q: [Hq, L, D] view with element strides (q_sh, q_sl), d contiguous.
 * k: [Hk, L, D] likewise.  Outputs q_b [Hq][N][D], k_b [Hk][N][D] in dtype,
 * N = ceil(L / bs): mean of each bs-token block, zero padding, divisor bs. */
typedef struct {
  const void* q; int64_t q_sh, q_sl;
  const void* k; int64_t k_sh, k_sl;
  int dtype, Hq, Hk, L, D, bs;
  void* q_b;
  void* k_b;
} fs_pool_args;
FS_API int fs_pool(const fs_pool_args* a, void* stream);

/* ---- rotary embedding + block pooling in one pass -----------------------
 * Replaces the attention forward's RoPE step (eval/LongBench/pred.py:195,
 * transformers models/llama/modeling_llama.py apply_rotary_pos_emb) followed by
 * block_mean_pool of the rotated states (my_attn_v7.py:105-114, call :553-555).
 * q: pre-RoPE [Hq, L, D] view (element strides q_sh, q_sl; d contiguous), k
 * likewise [Hk, L, D]; cos / sin: [L, D] rows (row stride cs_sl) in dtype, the
 * caller's position embeddings of these L positions.  Writes the rotated
 *   out[d] = rnd(rnd(x[d] * cos[d]) + rnd(r[d] * sin[d])),  r = (-x[D/2:], x[:D/2]),
 * (each step in fp32, rounded to dtype, as the reference's elementwise ops)
 * to q_out / k_out (own strides), and to q_b [Hq][N][D] / k_b [Hk][N][D] the
 * block means fs_pool would compute from q_out / k_out (bit-identical).
 * D / (16 / sizeof(dtype)) must be a power of two <= 64 (D = 128 for every dtype). */
typedef struct {
  const void* q; int64_t q_sh, q_sl;
  const void* k; int64_t k_sh, k_sl;
  const void* cos; const void* sin; int64_t cs_sl;
  void* q_out; int64_t qo_sh, qo_sl;
  void* k_out; int64_t ko_sh, ko_sl;
  int dtype, Hq, Hk, L, D, bs;
  void* q_b;
  void* k_b;
} fs_rope_pool_args;
FS_API int fs_rope_pool(const fs_rope_pool_args* a, void* stream);

/* ---- FFT lag correlation + lag selection (my_attn_v7.py:117-208) --------
 * For query head h (key head h / (Hq/Hk)):
 *   corr_sum[h][t] = sum_i <q_b[h][i], k_b[hk][i-t]>  via zero-padded FFTs,
 *   corr[h][t]     = post-processed value (my_attn_v7.py:134-155),
 *   keep_tau[h][t] = 1 iff t >= remote_start and, by corr_mode,
 *     0 "threshold" (:205-208): corr[h][t] / max(max_{t'>=rs} corr[h][t'], 1e-6) >= corr_threshold;
 *     1 "topk" (:196-203): corr[h][t] >= the corr_quantile quantile of corr[h][rs..N-1]
 *       (torch.quantile, linear interpolation; corr_quantile = 1 - correlation_topk_ratio in fp32).
 * work: fs_corr_work_bytes(Hq, N, D) bytes of device scratch.  N <= 4096
 * (one LDS FFT of length 2N). */
typedef struct {
  const void* q_b; const void* k_b;
  int dtype, Hq, Hk, N, D;
  int local_window, keep_sink, remote_start;
  float corr_threshold;
  int corr_mode;        /* 0 threshold, 1 topk */
  float corr_quantile;  /* topk mode */
  void* work;
  float* corr;          /* [Hq][N] */
  float* corr_sum;      /* [Hq][N] */
  uint8_t* keep_tau;    /* [Hq][N] */
} fs_corr_args;
FS_API size_t fs_corr_work_bytes(int Hq, int N, int D);
FS_API int fs_corr(const fs_corr_args* a, void* stream);

/* ---- per-head statistics (my_attn_v7.py:301-363, 390-447, 54-72) --------
 * diag_var[h][s]  = var(diff(diag_{tau_s}[:-1])) / clamp(mean|diag_{tau_s}[:-1]|, 1e-6)
 *                   over S = q_b k_b^T / sqrt(D), unbiased variance;
 * col_mean[h][j]  = (sum_{i=j}^{N-2} q_b[h][i]) . k_b[hk][j] / sqrt(D) / max(1, N-j-1);
 * col_sel[h][j]   = 1 for the n_cols largest col_mean in [col_start, col_end);
 * last_scores[h][j] = <q_b[h][N-1], k_b[hk][j]> rounded to dtype;
 * last_sel[h][j]  = 1 for the last_k largest last_scores.
 * Ties in the top-n selections go to the lower index.
 * sample_taus: device int32[n_samples]; n_samples == 0 skips diag_var;
 * n_cols == 0 skips the columns; last_k == 0 skips the last row. */
typedef struct {
  const void* q_b; const void* k_b;
  int dtype, Hq, Hk, N, D;
  const int32_t* sample_taus; int n_samples;
  int col_start, col_end, n_cols;
  int last_k;
  float* diag_var;       /* [Hq][n_samples] */
  float* col_mean;       /* [Hq][N] */
  uint8_t* col_sel;      /* [Hq][N] */
  float* last_scores;    /* [Hq][N] */
  uint8_t* last_sel;     /* [Hq][N] */
} fs_stats_args;
FS_API int fs_stats(const fs_stats_args* a, void* stream);

/* ---- correlation + statistics from MFMA block-score tiles (16-bit inputs)
 * One call producing what fs_corr and fs_stats produce, for dtype bf16/f16,
 * D % 16 == 0, D <= 128, N <= 8192 (my_attn_v7.py:117-157, 190-208,
 * 301-363, 390-447, 54-72).  The tiles of S = q_b k_b^T (i >= j) are formed
 * on MFMA and every statistic is a fixed-order sum over them: the lag sums
 * corr_sum[h][t] = sum_i S[i][i-t] (the reference's FFT computes the same
 * sums), the column scores from sum_{i=j}^{N-2} S[i][j] (the reference's
 * suffix sums of q_b give the same sums), the sampled diagonals and the last
 * row.  Fields and outputs mean what they mean in fs_corr_args and
 * fs_stats_args; keep_tau == NULL skips the correlation outputs.
 * work: fs_scores_work_bytes(Hq, N, n_samples) bytes of device scratch. */
typedef struct {
  const void* q_b; const void* k_b;
  int dtype, Hq, Hk, N, D;
  int local_window, keep_sink, remote_start;
  float corr_threshold;
  int corr_mode;         /* 0 threshold, 1 topk (as in fs_corr_args) */
  float corr_quantile;
  float* corr;           /* [Hq][N] */
  float* corr_sum;       /* [Hq][N] or NULL */
  uint8_t* keep_tau;     /* [Hq][N] or NULL */
  const int32_t* sample_taus; int n_samples;
  int col_start, col_end, n_cols;
  int last_k;
  float* diag_var;       /* [Hq][n_samples] */
  float* col_mean;       /* [Hq][N] or NULL */
  uint8_t* col_sel;      /* [Hq][N] */
  float* last_scores;    /* [Hq][N] */
  uint8_t* last_sel;     /* [Hq][N] */
  void* work;
} fs_scores_args;
FS_API size_t fs_scores_work_bytes(int Hq, int N, int n_samples);
FS_API int fs_scores(const fs_scores_args* a, void* stream);

/* ---- fs_scores without a workspace ---------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc): fs_scores with its per-tile partials in a static device array of
 * FS_SCORES_STATIC_BYTES (32 MiB) that each GPU the library runs on holds
 * until the process ends; a->work is ignored (may be NULL).  Same outputs as
 * fs_scores, bit for bit.  A call whose fs_scores_work_bytes(Hq, N, n_samples)
 * exceeds the array is rejected with FS_ERR_UNSUPPORTED before any launch
 * (BASELINE shapes need <= 11 MiB: Hq = 32, N = 1024, 64 samples).  Calls
 * on one GPU share its array: calls that overlap on one GPU (several streams
 * or threads) race; order them on one stream.  The first call on a device
 * looks the array's device address up (no allocation). */
#define FS_SCORES_STATIC_BYTES ((size_t)32 << 20)
FS_API int fs_scores_noalloc(const fs_scores_args* a, void* stream);

/* ---- mask composition -> block mask --------------------------------------
 * Row i of head h selects key block j (0 <= j < Nk, and j <= i if mask_causal) iff
 *   prior:  j < keep_sink || j >= Nk - keep_recent || (local_window > 0 && |i-j| <= local_window)
 *   last:   last_sel && i == N-1 && last_sel[h][j]
 *   dyn_mode 1, stripe head:  t = i-j >= remote_start && j >= keep_sink && keep_tau[h][t]
 *   dyn_mode 1, diffuse head: S[h][i][j] among the top k_i of S[h][i][0..i],
 *                             k_i = max(1, trunc(float(i+1) * qk_topk_ratio)), ties -> lower j
 *   column: col_mode 2, or col_mode 1 and stripe head: col_sel[h][j] && j <= i
 * with is_stripe[h] = mean_s(diag_var[h][s]) <= stripe_threshold (false when
 * stripe_all_diffuse or the mean is nan).  Output: the block mask blk_bits
 * [Hq][N][FS_MASK_WORDS(Nk)] and blk_cnt [Hq][N] (every word of every row is
 * written).  N <= 8192 (D <= 256 with dyn_mode 1). */
typedef struct {
  const void* q_b; const void* k_b;
  int dtype, Hq, Hk, N, Nk, D;
  int mask_causal;
  int keep_sink, keep_recent, local_window, remote_start;
  int dyn_mode;                 /* 0: none, 1: stripe -> lags, diffuse -> qk top-k */
  int stripe_all_diffuse;
  const float* diag_var; int n_samples; float stripe_threshold;
  const uint8_t* keep_tau;
  float qk_topk_ratio;
  int col_mode;                 /* 0: none, 1: stripe heads, 2: all heads */
  const uint8_t* col_sel;
  const uint8_t* last_sel;      /* NULL: no last-row mask */
  float* mean_var;              /* [Hq] out (may be NULL) */
  uint8_t* is_stripe;           /* [Hq] out (may be NULL) */
  int32_t* blk_cnt;             /* [Hq][N] */
  uint64_t* blk_bits;           /* [Hq][N][FS_MASK_WORDS(Nk)] */
} fs_select_args;
FS_API int fs_select(const fs_select_args* a, void* stream);

/* ---- XAttention block selection ------------------------------------------
 * The reference's other selector (attn_src/xattn/src/Xattention.py:14-303
 * xattn_estimate; Triton path kernels.py:5-156, 195-234; torch path
 * Xattention.py:72-135, 170-258; find_blocks_chunked utils.py:44-200), block
 * size 128.  For query head h (key head h / (Hq/Hk)), stride S, reshaped row m
 * and key n (tokens zero past L):
 *   A[m][n]  = sum_{j<S} q[m QS + o_j] . k'[nS+j]  rounded to dtype;
 * Triton path (torch_path 0: the callers' use_triton=True): o_j = S-1-j,
 * QS = S, k' = k, x = A log2(e) / sqrt(D) / S / norm, p = exp2(x - max_m) /
 * sum_m over the keys row m sees (causal: n <= m; non_causal: every key of the
 * sequence zero-padded to whole chunks of `chunk` tokens), rows m >= ceil(L/S)
 * zero, sums[h][I][J] = sum of p over the reshaped rows / keys of blocks I, J,
 * rounded to dtype.  Torch path (use_triton=False): select_mode 0 inverse
 * (o_j = S-1-j, QS = S kdb), 1 slash (o_j = j), 2 random (o_j = perm[j]),
 * 3 double / 4 triple (o_j = S-1-j; k' the neighbouring-chunk sums of k in
 * dtype); x = A / sqrt(D) / S / norm, each division rounded to dtype; causal
 * row m sees keys n <= m kdb + kdb - 1 (those of its own chunk only when the
 * sequence needs no padding, as the reference's mask does); p = softmax (float32; or exp with no_softmax) rounded to dtype; the
 * last padded rows zeroed; sums = two sums rounded to dtype (a block's keys,
 * then its rows).  Then per block row I, in float64: causal: the blocks 0 and
 * I, and the other blocks in decreasing order of sums while sums(0) + sums(I)
 * + (mass of the larger others) < row total * threshold[h]; non_causal: every
 * block of the chunk-padded row in decreasing order while the mass before it
 * < row total * threshold[h], and block 0 (ties: lower index first).  Outputs
 * the block mask blk_bits [Hq][N][FS_MASK_WORDS(N)], blk_cnt [Hq][N] of the
 * N = ceil(L/bs) real blocks (causal: the tril; keep_sink: row 0 selects every
 * block; keep_recent: the diagonal) and sums [Hq][N][N] (causal: its lower
 * triangle).  threshold: device array of Hq float64 values.  work:
 * fs_xattn_work_bytes(a) bytes of device scratch: the row statistics, K' for
 * double / triple and the rounded scores A of the keys each row sees, for
 * head_group heads at a time (about (L/S)^2 bytes per head causal, twice
 * that non-causal: 8.7 / 17.2 GB for 32 heads at L = 131072, S = 8).  Zero-initialised trailing fields give the
 * Triton causal path.  bf16/f16, D = 128, bs = 128, stride 4, 8 or 16,
 * N <= 4096 and chunk-padded blocks <= 4096. */
typedef struct {
  const void* q; int64_t q_sh, q_sl;
  const void* k; int64_t k_sh, k_sl;
  int dtype, Hq, Hk, L, D, stride, bs;
  float norm;
  const double* threshold;
  int keep_sink;
  float* sums;
  int32_t* blk_cnt;
  uint64_t* blk_bits;
  void* work;
  int non_causal;       /* causal=False */
  int torch_path;       /* use_triton=False */
  int select_mode;      /* torch path: 0 inverse, 1 slash, 2 random, 3 double, 4 triple */
  int perm[16];         /* random: the query token offset of chunk j (torch.randperm(stride) in the reference) */
  int kdb;              /* torch path: every kdb-th reshaped query row (0 or 1: all) */
  int no_softmax;       /* torch path: softmax=False */
  int chunk;            /* chunk_size in tokens (non-causal and torch path; 0: none) */
  int keep_recent;
  int head_group;       /* heads whose scores the workspace holds at once (0: all): the score
                           and block-sum passes run group by group, bounding the workspace */
} fs_xattn_args;
FS_API size_t fs_xattn_work_bytes(const fs_xattn_args* a);
FS_API int fs_xattn(const fs_xattn_args* a, void* stream);

/* ---- FlexPrefill block selection -----------------------------------------
 * The reference's third selector (attn_src/Flexprefill.py:946-1061,
 * get_active_blocks; budgets as Flexprefill_prefill :1080-1096 derives them).
 * For query head h (key head h / (Hq/Hk), or h % Hk with gqa_interleave):
 * the last bs queries / sqrt(D) against every key (scores in dtype, the last
 * block causal, fp32 softmax); vertical = mean over those rows, slash = sums
 * along the diagonals ending at each column of the last row / bs; budgets
 * (#descending prefix sums <= gamma, + 1) / 128 + 1 clamped to
 * [min_blocks, max_blocks]; heads whose square-root JS divergence between the
 * softmax of (row-mean last query) . (K block means) and the pooled vertical
 * is below tau take min_blocks and, in addition, the cover of gamma * N of
 * their block-level causal attention; the top pooled vertical columns (block 0
 * forced) in every row at or after them and the top pooled slash offsets
 * (offset 0 forced) as block diagonals (ties: lower index).  Outputs the block
 * mask blk_bits [Hq][N][FS_MASK_WORDS(N)], blk_cnt [Hq][N] (N = ceil(L/bs)), optionally
 * head_info [Hq][4] (vertical budget, slash budget, sparse, 0), head_js [Hq]
 * and the per-token vertical / slash profiles [Hq][L] (fp32).
 * work: fs_flex_work_bytes(Hq, Hk, L, bs, tau) bytes, with the tau of the
 * call (tau <= 0, the reference's default, makes no head sparse and needs no
 * room for the block-level attention and covers).  bf16/f16, D = 128,
 * bs 16, 32, 64 or 128, L > bs, N <= 8192. */
typedef struct {
  const void* q; int64_t q_sh, q_sl;
  const void* k; int64_t k_sh, k_sl;
  int dtype, Hq, Hk, L, D, bs;
  float gamma, tau;
  int min_blocks, max_blocks;
  int gqa_interleave;
  int32_t* blk_cnt;
  uint64_t* blk_bits;
  int32_t* head_info;
  float* head_js;
  float* vertical;
  float* slash;
  void* work;
} fs_flex_args;
FS_API size_t fs_flex_work_bytes(int Hq, int Hk, int L, int bs, float tau);
FS_API int fs_flex(const fs_flex_args* a, void* stream);

/* ---- block-sparse attention prefill --------------------------------------
 * out[b][t][h] = softmax(q[b][h][t] . k[b][hk][s] * scale) v[b][hk][s] over the
 * key tokens s of the selected key blocks of query block t / bs (and s <= t +
 * Lk - Lq when is_causal).  The selected key blocks of query block r of head
 * h are the set bits of row (h, r) of the block mask blk_bits [Hq][Nq][NW]
 * (NW = FS_MASK_WORDS(Nk); bits past the causal limit are ignored); blk_cnt
 * [Hq][Nq] (the rows' bit counts) only orders the work, largest first.
 * blk_cnt == NULL selects every key block up to the
 * causal limit (dense causal attention).  Supported: dtype bf16/f16, D in {64, 128},
 * bs in {16, 32, 64, 128} (16 and 32: FlexPrefill's block sizes; their masks
 * are attended 128 queries at a time over the union of 128 / bs rows,
 * up to 8192 key blocks).  All tensors are
 * strided views with d contiguous.
 * work: fs_bsattn_work_bytes(a) bytes of device scratch (V is staged there
 * transposed, and the work items' longest-first order and the counters from
 * which the attention kernel's workgroups take their work items are formed
 * there, before the attention kernel runs).  Calls that overlap on one
 * workspace race; the results do not depend on which workgroup takes
 * which item. */
typedef struct {
  const void* q; int64_t q_sb, q_sh, q_sl;
  const void* k; int64_t k_sb, k_sh, k_sl;
  const void* v; int64_t v_sb, v_sh, v_sl;
  void* out; int64_t o_sb, o_sh, o_sl;
  int dtype, B, Hq, Hk, Lq, Lk, D, bs;
  int is_causal;
  float softmax_scale;
  int gqa_interleave;           /* query head h reads KV head h % Hk (else h / (Hq / Hk)) */
  const int32_t* blk_cnt;       /* [Hq][Nq] or NULL (B must be 1 when non-NULL) */
  const uint64_t* blk_bits;     /* [Hq][Nq][FS_MASK_WORDS(Nk)] */
  void* work;
} fs_attn_args;
FS_API size_t fs_bsattn_work_bytes(const fs_attn_args* a);
/* The whole stage-2 call: fs_bsattn_prepare then fs_bsattn_run. */
FS_API int fs_bsattn(const fs_attn_args* a, void* stream);
/* The two halves of fs_bsattn, for callers that time or reuse them apart.
 * prepare: writes V^T of every KV head into work (depends on v, and on bs
 * and whether block lists are given: 16- and 32-token lists take V^T block
 * by block).  run: the longest-first order pass (block lists only) and the
 * attention kernel; reads V^T from work, so a prepare with the same v, Lk,
 * bs, lists (present or not) and work must precede it on the stream.  Both replace the same reference call as
 * fs_bsattn (my_attn_v7.py:775-786). */
FS_API int fs_bsattn_prepare(const fs_attn_args* a, void* stream);
FS_API int fs_bsattn_run(const fs_attn_args* a, void* stream);

/* Description of the last failure on this thread ("" if none). */
FS_API const char* fs_last_error(void);
/* sizeof the argument struct: 0 pool, 1 corr, 2 stats, 3 select, 4 attn, 5 scores, 6 rope_pool, 7 xattn,
 * 8 flex
 * (lets a foreign-function binding check its struct layout). */
FS_API size_t fs_sizeof_args(int which);
/* ABI version of this library (increments on any struct change). */
FS_API int fs_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FFTSPARSE_AMD_H */
