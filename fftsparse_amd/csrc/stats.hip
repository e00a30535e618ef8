// Per-head statistics on the pooled blocks:
//   diagonal statistics for the stripe/diffuse test  (my_attn_v7.py:301-363)
//   column scores and their top-n                     (my_attn_v7.py:390-447)
//   last-query-row scores and their top-k             (my_attn_v7.py:54-72)
//
// Grid (Hq, 2 + n_samples), 1024 threads: y == 0 is the column task, y == 1
// the last-row task and y >= 2 the diagonal sample y - 2.  Row dot products
// are computed by groups of 16 lanes (16-byte loads, four whole rows per wave
// load); all arithmetic is fp32 with a fixed accumulation order.  Top-k / top-n
// use the block radix select of common.h.
#include "common.h"

namespace fs {

constexpr int kStatThreads = 1024;
constexpr int kStatWaves = kStatThreads / 64;

template <typename T>
__global__ __launch_bounds__(kStatThreads) void stats_kernel(fs_stats_args a, float inv_sqrt_d) {
  extern __shared__ float sm[];          // [N] values, then [kStatWaves][D] run sums
  __shared__ float red[32];
  __shared__ int ired[kTopkScratch];
  const int h = blockIdx.x, task = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int N = a.N, D = a.D;
  const int hk = h / (a.Hq / a.Hk);
  const T* qb = static_cast<const T*>(a.q_b) + (int64_t)h * N * D;
  const T* kb = static_cast<const T*>(a.k_b) + (int64_t)hk * N * D;

  if (task == 0) {
    // ---- column scores (:404-420):
    //   col[j] = (total - cumsum[j-1]) . k_b[j] / sqrt(D) / max(1, N-j-1),  total = cumsum[N-2],
    // the difference being 0 for j = N-1 (:414).  Wave w owns rows [w R, (w+1) R),
    // lane l owns dims l, l+64, ... (D <= 256).
    if (a.n_cols <= 0) return;
    float* colv = sm;                               // [N]
    float* runs = sm + N;                           // [kStatWaves][D]
    const int R = (N + kStatWaves - 1) / kStatWaves;
    const int r0 = min(N, wave * R), r1 = min(N, r0 + R);
    const int nd = (D + 63) / 64;
    for (int k = 0; k < nd; ++k) {
      const int d = lane + 64 * k;
      if (d >= D) break;
      float s = 0.f;
      for (int i = r0; i < min(r1, N - 1); ++i) s += to_f32(qb[(int64_t)i * D + d]);
      runs[wave * D + d] = s;
    }
    __syncthreads();
    float run[4], tot[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      run[k] = 0.f;
      tot[k] = 0.f;
      const int d = lane + 64 * k;
      if (k < nd && d < D) {
        for (int w = 0; w < kStatWaves; ++w) {
          const float v = runs[w * D + d];
          if (w < wave) run[k] += v;
          tot[k] += v;
        }
      }
    }
    for (int j = r0; j < r1; ++j) {
      float dot = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int d = lane + 64 * k;
        if (k < nd && d < D) {
          const float partial = (j == N - 1) ? 0.f : tot[k] - run[k];
          dot += partial * to_f32(kb[(int64_t)j * D + d]);
          run[k] += to_f32(qb[(int64_t)j * D + d]);
        }
      }
      dot = wave_sum(dot);
      if (lane == 0) colv[j] = (dot * inv_sqrt_d) / (float)max(1, N - j - 1);
    }
    __syncthreads();
    for (int j = tid; j < N; j += kStatThreads) {
      if (a.col_mean) a.col_mean[(int64_t)h * N + j] = colv[j];
      if (j < a.col_start || j >= a.col_end) a.col_sel[(int64_t)h * N + j] = 0;
    }
    const int cs = a.col_start, nv = a.col_end - a.col_start;
    block_topk_select(colv + cs, nv, a.n_cols, a.col_sel + (int64_t)h * N + cs, ired);
    return;
  }
  if (task == 1) {
    // ---- last query row (:61-70): einsum in the input dtype, top-k
    if (a.last_k <= 0) return;
    float* lv = sm;
    const T* ql = qb + (int64_t)(N - 1) * D;
    const int g = lane >> 4, sub = lane & 15;
    for (int j0 = wave * 4; j0 < N; j0 += kStatWaves * 4) {
      const int j = j0 + g;
      float d = 0.f;
      if (j < N) d = row_dot_part(ql, kb + (int64_t)j * D, D, sub);
      d = group16_sum(d);
      if (sub == 0 && j < N) {
        const float s = Conv<T>::round(d);
        lv[j] = s;
        a.last_scores[(int64_t)h * N + j] = s;
      }
    }
    __syncthreads();
    block_topk_select(lv, N, a.last_k, a.last_sel + (int64_t)h * N, ired);
    return;
  }
  // ---- diagonal sample (:342-349)
  const int si = task - 2;
  if (si >= a.n_samples) return;
  const int tau = a.sample_taus[si];
  float* dv = sm;
  // diagonal length minus the dropped last element; an out-of-range lag reads nothing
  const int nd = (tau >= 0 && tau < N) ? N - tau - 1 : 0;
  {
    const int g = lane >> 4, sub = lane & 15;
    for (int j0 = wave * 4; j0 < nd; j0 += kStatWaves * 4) {
      const int j = j0 + g;
      float d = 0.f;
      if (j < nd) d = row_dot_part(qb + (int64_t)(j + tau) * D, kb + (int64_t)j * D, D, sub);
      d = group16_sum(d);
      if (sub == 0 && j < nd) dv[j] = d * inv_sqrt_d;
    }
  }
  __syncthreads();
  float sabs = 0.f;
  for (int j = tid; j < nd; j += kStatThreads) sabs += fabsf(dv[j]);
  const float mean_abs = block_sum(sabs, red) / (float)nd;
  const int ne = nd - 1;
  float se = 0.f;
  for (int j = tid; j < ne; j += kStatThreads) se += dv[j + 1] - dv[j];
  const float mean_e = block_sum(se, red) / (float)ne;
  float sq = 0.f;
  for (int j = tid; j < ne; j += kStatThreads) {
    const float e = (dv[j + 1] - dv[j]) - mean_e;
    sq += e * e;
  }
  const float var = block_sum(sq, red) / (float)(ne - 1);
  if (tid == 0) a.diag_var[(int64_t)h * a.n_samples + si] = var / clamp_min_nan(mean_abs, 1e-6f);
}

template <typename T>
static int launch_stats(const fs_stats_args& a, dim3 grid, size_t smem, float inv_sqrt_d, hipStream_t s) {
  if (int rc = fs_host::allow_dynamic_lds(stats_kernel<T>, smem, "fs_stats")) return rc;
  stats_kernel<T><<<grid, kStatThreads, smem, s>>>(a, inv_sqrt_d);
  return 0;
}

}  // namespace fs

using namespace fs;

extern "C" int fs_stats(const fs_stats_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_stats: null args");
  FS_CHECK_ARG(a->q_b && a->k_b, "fs_stats: null pooled pointer");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "fs_stats: bad head counts");
  FS_CHECK_ARG(a->N >= 1 && a->D >= 8 && a->D <= 256 && a->D % 8 == 0, "fs_stats: bad sizes");
  FS_CHECK_ARG(((uintptr_t)a->q_b % 16) == 0 && ((uintptr_t)a->k_b % 16) == 0, "fs_stats: unaligned pooled tensors");
  FS_CHECK_ARG(a->n_samples >= 0 && (a->n_samples == 0 || (a->sample_taus && a->diag_var)),
               "fs_stats: sample arrays missing");
  FS_CHECK_ARG(a->n_cols <= 0 || (a->col_sel && a->col_start >= 0 && a->col_end <= a->N &&
                                  a->col_end > a->col_start && a->n_cols <= a->col_end - a->col_start),
               "fs_stats: bad column range");
  FS_CHECK_ARG(a->last_k <= 0 || (a->last_sel && a->last_scores && a->last_k <= a->N),
               "fs_stats: bad last-row arguments");
  FS_CHECK_SUPPORTED(a->N <= 4096, "fs_stats: N=%d > 4096", a->N);
  const float inv_sqrt_d = 1.0f / (float)sqrt((double)a->D);
  const size_t smem = (size_t)(a->N + kStatWaves * a->D) * sizeof(float);
  dim3 grid(a->Hq, 2 + a->n_samples);
  hipStream_t s = (hipStream_t)stream;
  int rc = 0;
  switch (a->dtype) {
    case FS_DTYPE_F32: rc = launch_stats<float>(*a, grid, smem, inv_sqrt_d, s); break;
    case FS_DTYPE_BF16: rc = launch_stats<bf16_t>(*a, grid, smem, inv_sqrt_d, s); break;
    case FS_DTYPE_F16: rc = launch_stats<f16_t>(*a, grid, smem, inv_sqrt_d, s); break;
    default: fs_host::set_error("fs_stats: dtype %d unsupported", a->dtype); return FS_ERR_UNSUPPORTED;
  }
  if (rc) return rc;
  return fs_host::launch_status("fs_stats");
}
