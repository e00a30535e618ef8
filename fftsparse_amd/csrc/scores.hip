// Block-score statistics of the selection stage from tiles of
// S = q_b k_b^T on bf16/f16 MFMA, in place of the FFT correlation and the
// per-head statistics kernels for 16-bit inputs:
//   lag sums        corr_sum[t] = sum_i S[i][i-t]          (my_attn_v7.py:117-157; the
//                   reference takes them from zero-padded FFTs, these are the same
//                   sums added directly in fp32)
//   lag selection   post-processing + threshold             (:134-155, :190-208)
//   diagonal stats  var(diff(S[j+t][j] / sqrt(D))) / mean|.| (:301-363)
//   column scores   sum_{i=j}^{N-2} S[i][j] / sqrt(D) / max(1, N-j-1) (:390-447; the
//                   reference forms the suffix sums of q_b first, which is the same sum)
//   last row        S[N-1][j] rounded to the input dtype    (:54-72)
//
// scores_kernel: one workgroup (4 waves) per (head, 128 x 64 column half of a
// 128 x 128 tile I >= J of the lower triangle).  Wave w computes rows
// 32w .. 32w+31 of the half with v_mfma_f32_32x32x16 (the half's 64 K rows
// staged in LDS), the half goes through LDS in two quarters of 32 columns
// (20 KiB of LDS and 80 registers per lane, so six workgroups fit a CU), and
// fixed-order partials are written to the work buffer: the 255 diagonal sums
// of each half, the column sums over rows i >= j, i <= N-2, the elements of
// every sampled diagonal that crosses the half, and the last row.  (Whole
// tiles per workgroup, three to a CU: 31.3 against 28.7 us at N = 1024 with
// 32 heads, the 1152 tiles in two rounds of workgroups either way.)
// scores_final_kernel: grid (head, job): job 0 adds the lag partials and
// selects the lags, 2 the column scores and their top-n, 3 the last-row
// top-k, 4 .. 7 the diagonal statistics (one wave per sample; job 1 is
// idle); every sum is in a fixed order (deterministic).
#include <mutex>

#include "common.h"

namespace fs {

constexpr int kScoreTile = 128;
constexpr int kHalf = kScoreTile / 2;           // columns per score workgroup
constexpr int kQuarter = kScoreTile / 4;        // columns per S pass through LDS
constexpr int kScoreThreads = 256;
constexpr int kFinalThreads = 1024;
constexpr int kDiagSlots = 256;                 // 255 local diagonals per tile (+1 pad)
constexpr int kMaxSamples = 1024;               // sampled diagonals per head
constexpr int kDiagJobs = 4;                    // final-kernel workgroups per head for the diagonal statistics
constexpr int kScoresMaxN = 8192;               // the final kernel's per-head row of N floats in LDS

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct ScoreMma;
template <> struct ScoreMma<bf16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
};
template <> struct ScoreMma<f16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
};

// tile index t of the lower triangle -> (I, J), t = I (I + 1) / 2 + J
__device__ __forceinline__ void tile_ij(int t, int& I, int& J) {
  int i = (int)((sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);
  while ((i + 1) * (i + 2) / 2 <= t) ++i;
  while (i * (i + 1) / 2 > t) --i;
  I = i;
  J = t - i * (i + 1) / 2;
}
__device__ __forceinline__ int tile_id(int I, int J) { return I * (I + 1) / 2 + J; }

template <typename T>
__global__ __launch_bounds__(kScoreThreads) __attribute__((amdgpu_waves_per_eu(5))) void scores_kernel(
    fs_scores_args a, int ntiles, float inv_sqrt_d, float* __restrict__ pdiag, float* __restrict__ pcol,
    float* __restrict__ dvs) {
  // The half's K rows (bf16/f16 [64][D], D <= 128: 16 KiB) are staged in the
  // same LDS as the S quarters written after the MFMAs.
  __shared__ __attribute__((aligned(16))) float sl[kScoreTile][kQuarter + 1];
  __shared__ short rel[kMaxSamples];               // the sampled diagonals that cross this half
  __shared__ int nrel;
  __shared__ float csum[4][kHalf];                 // per-wave column partials
  uint16_t* kt = reinterpret_cast<uint16_t*>(&sl[0][0]);
  // Workgroup w runs on XCD w % 8.  XCD x takes the contiguous range of
  // (head, tile, half) items [x per, (x + 1) per): a head's tiles (and the
  // heads of one KV group) share one XCD, so the Q_b / K_b panels each tile
  // re-reads are fetched into that XCD's L2 once instead of into all eight.
  const int total = a.Hq * ntiles * 2, per = (total + 7) / 8;
  const int slot = (int)(blockIdx.x >> 3), item = (int)(blockIdx.x & 7) * per + slot;
  if (slot >= per || item >= total) return;
  const int ht = item >> 1, hf = item & 1;
  const int h = ht / ntiles, t = ht - h * ntiles;
  int I, J;
  tile_ij(t, I, J);
  const int N = a.N, D = a.D;
  const int hk = h / (a.Hq / a.Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const uint16_t* qb = static_cast<const uint16_t*>(a.q_b) + (int64_t)h * N * D;
  const uint16_t* kb = static_cast<const uint16_t*>(a.k_b) + (int64_t)hk * N * D;
  const int i0 = I * kScoreTile, jt0 = J * kScoreTile;     // first row and column of the tile
  const int c0 = hf * kHalf;                               // first tile column of this half
  const int j0 = jt0 + c0;                                 // first column of this half

  // ---- S half: A = q rows (row i), B = k rows as columns (col j), K = d
  f32x16_t acc[2];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[jt][r] = 0.f;
  // Every global load of the half is issued before the first wait: this
  // wave's Q operands (all D/16 steps, in registers) and the K rows (to LDS,
  // rows past N zero).
  constexpr int kMaxSteps = 128 / 16;              // D <= 128
  const int qi = i0 + wave * 32 + l32;
  const uint16_t* qrow = qb + (int64_t)min(qi, N - 1) * D + hi * 8;
  const bool qok = qi < N;
  uint4 qv[kMaxSteps];
#pragma unroll
  for (int st = 0; st < kMaxSteps; ++st)
    qv[st] = (qok && st < D / 16) ? *reinterpret_cast<const uint4*>(qrow + st * 16) : make_uint4(0, 0, 0, 0);
  const int cpr = D / 8;                           // 16-byte chunks per row
  // K rows are stored with 16-byte chunk c of row r at c ^ (r & sw): the 32
  // lanes of an MFMA operand read take one row each, and without the swizzle
  // every row's chunk would sit in the same banks
  const int sw = (cpr & (cpr - 1)) == 0 ? cpr - 1 : 0;
  constexpr int kMaxChunks = kHalf * (128 / 8) / kScoreThreads;   // per thread, D <= 128
  uint4 kv[kMaxChunks];
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    const int c = tid + u * kScoreThreads, r = c / cpr, cc = c - r * cpr;
    kv[u] = (c < kHalf * cpr && j0 + r < N) ? *reinterpret_cast<const uint4*>(kb + (int64_t)(j0 + r) * D + cc * 8)
                                            : make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) nrel = 0;
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    const int c = tid + u * kScoreThreads, r = c / cpr, cc = c - r * cpr;
    if (c < kHalf * cpr) *reinterpret_cast<uint4*>(kt + r * D + ((cc ^ (r & sw)) * 8)) = kv[u];
  }
  __syncthreads();
#pragma unroll
  for (int st = 0; st < kMaxSteps; ++st) {
    if (st >= D / 16) break;
    const uint4 av = qv[st];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      const int kr = jt * 32 + l32;
      const uint4 bv = *reinterpret_cast<const uint4*>(kt + kr * D + (((2 * st + hi) ^ (kr & sw)) * 8));
      acc[jt] = ScoreMma<T>::mma(av, bv, acc[jt]);
    }
  }
  // the sampled diagonals tau = i - j that cross the half, i - j in
  // [i0 - j0 - 63, i0 - j0 + 127] (their order in rel is arbitrary: each
  // one's elements go to fixed places)
  for (int e = tid; e < a.n_samples; e += kScoreThreads) {
    const int tau = a.sample_taus[e];
    if (tau >= 0 && tau < N && tau >= i0 - j0 - (kHalf - 1) && tau <= i0 - j0 + (kScoreTile - 1))
      rel[atomicAdd(&nrel, 1)] = (short)e;
  }

  // The S half goes through LDS in two quarters of 32 columns (a smaller LDS
  // footprint, so more workgroups per CU).  C layout: lane holds row
  // (r/4)*8 + hi*4 + r%4, column l32 of each 32x32 block.
  const int64_t tb = (int64_t)h * ntiles + t;
  const bool diag_tile = I == J;
  // ---- column sums over rows i >= j, i <= N-2, from the accumulators: the
  // lane's 16 rows, then the other lane half (rows hi * 4 ..), then the four
  // waves in order (through LDS)
  if (a.n_cols > 0) {
    const int ie = min(kScoreTile - 1, N - 2 - i0);
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      const int jl = c0 + jt * 32 + l32;             // tile column
      float c = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int il = wave * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
        if (il <= ie && (!diag_tile || il >= jl)) c += acc[jt][r];
      }
      c += __shfl_xor(c, 32, 64);
      if (hi == 0) csum[wave][jt * 32 + l32] = c;
    }
  }
  const int dl = tid - (kScoreTile - 1);           // this thread's local diagonal iloc - jloc
  const bool lag_on = a.keep_tau != nullptr && tid < 2 * kScoreTile - 1 && !(diag_tile && dl < 0);
  float lag = 0.f;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int cq = c0 + qt * kQuarter;             // first tile column of this quarter
    __syncthreads();                               // K rows / previous quarter consumed
#pragma unroll
    for (int r = 0; r < 16; ++r) sl[wave * 32 + (r >> 2) * 8 + hi * 4 + (r & 3)][l32] = acc[qt][r];
    __syncthreads();
    // ---- lag sums along the local diagonal, rows ascending (this quarter's columns)
    if (lag_on) {
      const int ib = max(0, dl + cq), ie = min(kScoreTile - 1, dl + cq + kQuarter - 1);
#pragma unroll 8
      for (int il = ib; il <= ie; ++il) lag += sl[il][il - dl - cq];
    }
    // ---- sampled diagonals crossing the quarter: S[j + tau][j] / sqrt(D) for j < N - tau - 1
    const int nr = nrel;
    for (int e = tid; e < nr * kQuarter; e += kScoreThreads) {
      const int s = rel[e / kQuarter], jq = e % kQuarter;
      const int tau = a.sample_taus[s];
      const int j = jt0 + cq + jq, i = j + tau;
      if (tau < 0 || tau >= N || j >= N - tau - 1) continue;
      const int il = i - i0;
      if (il < 0 || il >= kScoreTile) continue;
      dvs[((int64_t)h * a.n_samples + s) * N + j] = sl[il][jq] * inv_sqrt_d;
    }
    // ---- last row, rounded to the input dtype
    if (a.last_k > 0 && i0 <= N - 1 && N - 1 < i0 + kScoreTile && tid < kQuarter && jt0 + cq + tid < N)
      a.last_scores[(int64_t)h * N + jt0 + cq + tid] = Conv<T>::round(sl[N - 1 - i0][tid]);
  }
  if (a.keep_tau != nullptr && tid < 2 * kScoreTile - 1) pdiag[(tb * 2 + hf) * kDiagSlots + tid] = lag;
  if (a.n_cols > 0 && tid < kHalf)
    pcol[tb * kScoreTile + c0 + tid] =
        (j0 + tid < N) ? ((csum[0][tid] + csum[1][tid]) + csum[2][tid]) + csum[3][tid] : 0.f;
}


__global__ __launch_bounds__(kFinalThreads) void scores_final_kernel(fs_scores_args a, int ntiles, float inv_sqrt_d,
                                                                     const float* __restrict__ pdiag,
                                                                     const float* __restrict__ pcol,
                                                                     const float* __restrict__ dvs) {
  extern __shared__ float fsm[];                   // [N]: cv, colv or lastv by job
  __shared__ float red[32];
  __shared__ int ired[kTopkScratch];
  // blockIdx.y: 0 lag sums + selection, 2 columns, 3 last row, 4.. diagonal statistics
  const int h = blockIdx.x, job = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.N;
  const int NT = (N + kScoreTile - 1) / kScoreTile;
  const int64_t hb = (int64_t)h * ntiles;
  float* cv = fsm;
  float* colv = fsm;
  float* lastv = fsm;

  // ---- lag sums and the v7 post-processing (my_attn_v7.py:134-155, 193-208)
  if (job == 0 && a.keep_tau != nullptr) {
    const int ex = a.local_window + 1;
    const int st = N - a.keep_sink - 5;
    const int es = min(ex, N);
    const int ss = st >= 0 ? min(st, N) : max(0, N + st);
    for (int t = tid; t < N; t += kFinalThreads) {
      float cs = 0.f;
      const int d0 = t / kScoreTile;
      for (int dd = d0; dd <= d0 + 1 && dd < NT; ++dd) {     // tile diagonals I - J = dd
        const int dl = t - dd * kScoreTile;                  // local diagonal
        if (dl < -(kScoreTile - 1) || dl > kScoreTile - 1) continue;
#pragma unroll 8
        for (int J = 0; J + dd < NT; ++J) {
          const float* pd = pdiag + (hb + tile_id(J + dd, J)) * 2 * kDiagSlots + dl + kScoreTile - 1;
          cs += pd[0];
          cs += pd[kDiagSlots];
        }
      }
      if (a.corr_sum) a.corr_sum[(int64_t)h * N + t] = cs;
      float v = cs / (float)max(N - t, 1);
      if (t < es || t >= ss) v = 0.f;
      cv[t] = v;
    }
    __syncthreads();
    if (ex < st) {
      float mn = INFINITY;
      for (int t = ex + tid; t < st; t += kFinalThreads) mn = fminf(mn, cv[t]);
      mn = block_min(mn, red);
      const float den = clamp_min_nan(log10f((float)(N - ex)), 1e-6f);
      for (int t = ex + tid; t < st; t += kFinalThreads) {
        const float pw = log10f((float)(N - t)) / den;
        cv[t] = (cv[t] - mn) * pw;
      }
      __syncthreads();
    }
    for (int t = tid; t < N; t += kFinalThreads) a.corr[(int64_t)h * N + t] = cv[t];
    const int rs = a.remote_start;
    if (a.corr_mode == 1) {                       // "topk": quantile of the remote lags (:196-203)
      const float qv = block_quantile(cv + rs, N - rs, a.corr_quantile, ired);
      for (int t = tid; t < N; t += kFinalThreads) a.keep_tau[(int64_t)h * N + t] = (t >= rs && cv[t] >= qv) ? 1 : 0;
    } else {                                      // "threshold" (:205-208)
      float mx = -INFINITY;
      for (int t = rs + tid; t < N; t += kFinalThreads) mx = fmaxf(mx, cv[t]);
      mx = clamp_min_nan(block_max(mx, red), 1e-6f);
      for (int t = tid; t < N; t += kFinalThreads)
        a.keep_tau[(int64_t)h * N + t] = (t >= rs && cv[t] / mx >= a.corr_threshold) ? 1 : 0;
    }
  }

  // ---- diagonal statistics, one wave per sample, jobs 4 .. 4+kDiagJobs-1 (:342-349):
  // var(diff(d)) / max(mean|d|, 1e-6) over d = S[j + tau][j] / sqrt(D), j < N - tau - 1.
  // Diagonals of up to 1024 elements are read into registers in one round of
  // loads; the sums run over j = lane, lane + 64, .. in order either way.
  for (int s = (job - 4) * (kFinalThreads / 64) + wave; job >= 4 && s < a.n_samples;
       s += kDiagJobs * (kFinalThreads / 64)) {
    const int tau = a.sample_taus[s];
    const int nd = (tau >= 0 && tau < N) ? N - tau - 1 : 0;
    const float* dv = dvs + ((int64_t)h * a.n_samples + s) * N;
    const int ne = nd - 1;
    float sabs = 0.f, se = 0.f, sq = 0.f, mean_abs, mean_e;
    constexpr int kReg = 16;
    if (nd <= 64 * kReg) {
      float x[kReg], y[kReg];
#pragma unroll
      for (int k = 0; k < kReg; ++k) {             // every load issued (indices clamped), then the sums
        const int j = lane + 64 * k;
        x[k] = dv[max(min(j, nd - 1), 0)];
        y[k] = dv[max(min(j + 1, nd - 1), 0)];
      }
#pragma unroll
      for (int k = 0; k < kReg; ++k) {
        const int j = lane + 64 * k;
        if (j < nd) {
          sabs += fabsf(x[k]);
          if (j + 1 < nd) se += y[k] - x[k];
        }
      }
      mean_abs = wave_sum(sabs) / (float)nd;
      mean_e = wave_sum(se) / (float)ne;
#pragma unroll
      for (int k = 0; k < kReg; ++k) {
        const int j = lane + 64 * k;
        if (j < ne) {
          const float e = (y[k] - x[k]) - mean_e;
          sq += e * e;
        }
      }
    } else {
#pragma unroll 4
      for (int j = lane; j < nd; j += 64) {
        sabs += fabsf(dv[j]);
        if (j + 1 < nd) se += dv[j + 1] - dv[j];
      }
      mean_abs = wave_sum(sabs) / (float)nd;
      mean_e = wave_sum(se) / (float)ne;
#pragma unroll 4
      for (int j = lane; j < ne; j += 64) {
        const float e = (dv[j + 1] - dv[j]) - mean_e;
        sq += e * e;
      }
    }
    const float var = wave_sum(sq) / (float)(ne - 1);
    if (lane == 0) a.diag_var[(int64_t)h * a.n_samples + s] = var / clamp_min_nan(mean_abs, 1e-6f);
  }

  // ---- column scores and their top-n (:404-438)
  if (job == 2 && a.n_cols > 0) {
    for (int j = tid; j < N; j += kFinalThreads) {
      const int Jt = j / kScoreTile, jl = j - Jt * kScoreTile;
      float s = 0.f;
#pragma unroll 8
      for (int It = Jt; It < NT; ++It) s += pcol[(hb + tile_id(It, Jt)) * kScoreTile + jl];
      const float c = (s * inv_sqrt_d) / (float)max(1, N - j - 1);
      colv[j] = c;
      if (a.col_mean) a.col_mean[(int64_t)h * N + j] = c;
      if (j < a.col_start || j >= a.col_end) a.col_sel[(int64_t)h * N + j] = 0;
    }
    __syncthreads();
    block_topk_select(colv + a.col_start, a.col_end - a.col_start, a.n_cols,
                      a.col_sel + (int64_t)h * N + a.col_start, ired);
  }
  // ---- last-row top-k (:61-70)
  if (job == 3 && a.last_k > 0) {
    for (int j = tid; j < N; j += kFinalThreads) lastv[j] = a.last_scores[(int64_t)h * N + j];
    __syncthreads();
    block_topk_select(lastv, N, a.last_k, a.last_sel + (int64_t)h * N, ired);
  }
}

static size_t part_offsets(int Hq, int N, int n_samples, size_t* o_col, size_t* o_dv) {
  const int NT = (N + kScoreTile - 1) / kScoreTile;
  const size_t ntiles = (size_t)NT * (NT + 1) / 2;
  const size_t diag = (size_t)Hq * ntiles * 2 * kDiagSlots * sizeof(float);
  const size_t col = (size_t)Hq * ntiles * kScoreTile * sizeof(float);
  const size_t dv = (size_t)Hq * n_samples * N * sizeof(float);
  if (o_col) *o_col = diag;
  if (o_dv) *o_dv = diag + col;
  return diag + col + dv;
}

template <typename T>
static int launch_scores(const fs_scores_args& a, hipStream_t s) {
  const int NT = (a.N + kScoreTile - 1) / kScoreTile;
  const int ntiles = NT * (NT + 1) / 2;
  size_t o_col, o_dv;
  part_offsets(a.Hq, a.N, a.n_samples, &o_col, &o_dv);
  char* w = static_cast<char*>(a.work);
  float* pdiag = reinterpret_cast<float*>(w);
  float* pcol = reinterpret_cast<float*>(w + o_col);
  float* dvs = reinterpret_cast<float*>(w + o_dv);
  const float inv_sqrt_d = 1.0f / (float)sqrt((double)a.D);
  scores_kernel<T><<<(a.Hq * ntiles * 2 + 7) / 8 * 8, kScoreThreads, 0, s>>>(a, ntiles, inv_sqrt_d, pdiag, pcol, dvs);
  if (int rc = fs_host::launch_status("fs_scores (tiles)")) return rc;
  const size_t smem = (size_t)a.N * sizeof(float);
  if (int rc = fs_host::allow_dynamic_lds(scores_final_kernel, smem, "fs_scores")) return rc;
  scores_final_kernel<<<dim3(a.Hq, 4 + kDiagJobs), kFinalThreads, smem, s>>>(a, ntiles, inv_sqrt_d, pdiag, pcol, dvs);
  return fs_host::launch_status("fs_scores (final)");
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_scores_work_bytes(int Hq, int N, int n_samples) {
  if (Hq <= 0 || N <= 0 || n_samples < 0) return 0;
  return part_offsets(Hq, N, n_samples, nullptr, nullptr);
}

// Argument checks of fs_scores and fs_scores_noalloc (fn: the caller's name;
// with_work: the caller passes the workspace).
static int check_scores(const fs_scores_args* a, const char* fn, bool with_work) {
  FS_CHECK_ARG(a != nullptr, "%s: null args", fn);
  FS_CHECK_ARG(a->q_b && a->k_b && (a->work || !with_work), "%s: null pointer", fn);
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "%s: Hq=%d must be a multiple of Hk=%d", fn,
               a->Hq, a->Hk);
  FS_CHECK_ARG(a->N >= 1 && a->D >= 16, "%s: bad sizes", fn);
  FS_CHECK_ARG(((uintptr_t)a->q_b % 16) == 0 && ((uintptr_t)a->k_b % 16) == 0, "%s: unaligned pooled tensors", fn);
  FS_CHECK_ARG(a->keep_tau == nullptr || (a->corr && a->remote_start >= 0 && a->local_window >= 0),
               "%s: bad correlation arguments", fn);
  FS_CHECK_ARG(a->keep_tau == nullptr || a->corr_mode == 0 ||
                   (a->corr_mode == 1 && a->remote_start < a->N && a->corr_quantile >= 0.f && a->corr_quantile <= 1.f),
               "%s: corr_mode must be 0 or 1; topk mode needs remote_start < N and a quantile in [0, 1]", fn);
  FS_CHECK_ARG(a->n_samples >= 0 && (a->n_samples == 0 || (a->sample_taus && a->diag_var)),
               "%s: sample arrays missing", fn);
  FS_CHECK_ARG(a->n_cols <= 0 || (a->col_sel && a->col_start >= 0 && a->col_end <= a->N &&
                                  a->col_end > a->col_start && a->n_cols <= a->col_end - a->col_start),
               "%s: bad column range", fn);
  FS_CHECK_ARG(a->last_k <= 0 || (a->last_sel && a->last_scores && a->last_k <= a->N),
               "%s: bad last-row arguments", fn);
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16,
                     "%s: dtype %d unsupported (bf16/f16; fp32 uses fs_corr and fs_stats)", fn, a->dtype);
  // the staged K tile (128 * D 16-bit values) shares the S tile's LDS; D <= 128
  FS_CHECK_SUPPORTED(a->D % 16 == 0 && a->D <= 128, "%s: head_dim %d unsupported", fn, a->D);
  FS_CHECK_SUPPORTED(a->N <= kScoresMaxN, "%s: N=%d > %d", fn, a->N, kScoresMaxN);
  FS_CHECK_SUPPORTED(a->n_samples <= kMaxSamples, "%s: %d diagonal samples > %d", fn, a->n_samples, kMaxSamples);
  return FS_OK;
}

extern "C" int fs_scores(const fs_scores_args* a, void* stream) {
  if (int rc = check_scores(a, "fs_scores", true)) return rc;
  hipStream_t s = (hipStream_t)stream;
  return a->dtype == FS_DTYPE_BF16 ? launch_scores<bf16_t>(*a, s) : launch_scores<f16_t>(*a, s);
}

// ---- fs_scores without a workspace --------------------------------------
// The per-tile partials go to `scratch`, a static device array that every GPU
// the library runs on holds until the process ends.  In host code `scratch`
// names a host-side stand-in, not device memory: its device address is taken
// once per device with hipGetSymbolAddress (that device current) and only that
// address is handed to the kernels.  Every call on a GPU shares its array:
// calls that overlap on one GPU race.  Nothing in it must start at zero: each
// call's tile kernel writes every partial its final kernel reads.
constexpr size_t kScoresStaticBytes = (size_t)32 << 20;   // FS_SCORES_STATIC_BYTES
static __device__ __align__(256) unsigned char scratch[kScoresStaticBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];                 // device address of `scratch`, per device

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fs_host::set_error("fs_scores_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return FS_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fs_host::set_error("fs_scores_noalloc: device %d out of range (< %d)", dev, kMaxDevices);
    return FS_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      fs_host::set_error("fs_scores_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                         hipGetErrorString(e));
      return FS_ERR_LAUNCH;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return FS_OK;
}
}  // namespace

extern "C" int fs_scores_noalloc(const fs_scores_args* a, void* stream) {
  if (int rc = check_scores(a, "fs_scores_noalloc", false)) return rc;
  const size_t need = part_offsets(a->Hq, a->N, a->n_samples, nullptr, nullptr);
  FS_CHECK_SUPPORTED(need <= kScoresStaticBytes,
                     "fs_scores_noalloc: %zu bytes of partials (Hq=%d, N=%d, n_samples=%d) exceed the static "
                     "buffer of %zu bytes; use fs_scores with a workspace",
                     need, a->Hq, a->N, a->n_samples, kScoresStaticBytes);
  void* ptr = nullptr;
  if (int rc = scratch_address(&ptr)) return rc;
  fs_scores_args b = *a;
  b.work = ptr;
  hipStream_t s = (hipStream_t)stream;
  return b.dtype == FS_DTYPE_BF16 ? launch_scores<bf16_t>(b, s) : launch_scores<f16_t>(b, s);
}
