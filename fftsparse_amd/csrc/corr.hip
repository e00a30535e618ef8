// FFT lag correlation and lag selection
// (reference: attn_src/fft_attn/my_attn_v7.py:117-157 and :190-208).
//
//   corr_sum[h][t] = sum_d sum_i q_b[h][i][d] k_b[hk][i-t][d],   0 <= t < N
//
// computed in the frequency domain.  For every (head, dim) the real sequences
// x = q_b[h][:,d] and y = k_b[hk][:,d], zero padded to M = next_pow2(2N) >= 2N-1
// (so the circular correlation equals the linear one for t < N), are packed
// into one complex sequence z = x + i y and transformed by one radix-2 FFT in
// LDS.  X = (Z[f] + conj Z[M-f]) / 2 and Y = (Z[f] - conj Z[M-f]) / 2i give
// the cross spectrum X conj(Y), summed over d in registers.
//
// Kernel 1 (grid Hq x ceil(D/dpg)): each workgroup loads dpg dims of one head
// (dpg M <= 16384 complex values: 8 dims up to N = 1024) from the pooled rows
// (16-byte loads) straight into the bit-reversed order of dpg transforms in
// LDS, runs their radix-2 stages together (one barrier per stage) and writes
// its partial cross spectrum (M/2+1 bins) to the work buffer.
// Kernel 2 (grid Hq): sums the partials, inverts with one FFT per head, and
// applies the reference's post-processing and threshold in the same kernel.
#include <algorithm>

#include "common.h"

namespace fs {

constexpr int kFftThreads = 1024;              // 4 waves per SIMD hide the LDS latency of the butterflies
constexpr int kMaxLogM = 13;                              // M <= 8192, N <= 4096

__device__ __forceinline__ int bitrev(int x, int logM) { return (int)(__brev((uint32_t)x) >> (32 - logM)); }

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// tw[k] = exp(-2 pi i k / M), k < M/2 (single-precision sincospi, exact argument).
__device__ void fill_twiddles(float2* tw, int M) {
  for (int k = threadIdx.x; k < M / 2; k += blockDim.x) {
    float s, c;
    sincospif(-2.0f * (float)k / (float)M, &s, &c);
    tw[k] = make_float2(c, s);
  }
}

// In-place radix-2 decimation-in-time FFT; buf holds the input in bit-reversed order.
__device__ void fft_dit(float2* buf, const float2* tw, int M, int logM) {
  for (int s = 1; s <= logM; ++s) {
    const int half = 1 << (s - 1);
    const int tws = M >> s;
    for (int b = threadIdx.x; b < M / 2; b += blockDim.x) {
      const int grp = b >> (s - 1);
      const int pos = b & (half - 1);
      const int i0 = (grp << s) + pos, i1 = i0 + half;
      const float2 t = cmul(buf[i1], tw[pos * tws]);
      const float2 u = buf[i0];
      buf[i0] = make_float2(u.x + t.x, u.y + t.y);
      buf[i1] = make_float2(u.x - t.x, u.y - t.y);
    }
    __syncthreads();
  }
}

// Radix-2 DIT stages over nf transforms of length M stored back to back in
// buf (each in bit-reversed order); one barrier per stage for all of them.
__device__ void fft_dit_batch(float2* buf, const float2* tw, int M, int logM, int nf) {
  const int hm = M / 2;
  for (int s = 1; s <= logM; ++s) {
    const int half = 1 << (s - 1);
    const int tws = M >> s;
    for (int b = threadIdx.x; b < nf * hm; b += blockDim.x) {
      const int f = b / hm, bb = b - f * hm;
      const int grp = bb >> (s - 1);
      const int pos = bb & (half - 1);
      float2* x = buf + f * M;
      const int i0 = (grp << s) + pos, i1 = i0 + half;
      const float2 t = cmul(x[i1], tw[pos * tws]);
      const float2 u = x[i0];
      x[i0] = make_float2(u.x + t.x, u.y + t.y);
      x[i1] = make_float2(u.x - t.x, u.y - t.y);
    }
    __syncthreads();
  }
}

template <typename T>
__global__ __launch_bounds__(kFftThreads) void corr_partial_kernel(fs_corr_args a, int M, int logM, int dpg,
                                                                   float2* part) {
  extern __shared__ float2 smem[];
  float2* tw = smem;                                // [M/2] twiddles
  float2* buf = smem + M / 2;                       // [dpg][M] transforms of z = q + i k
  const int h = blockIdx.x, g = blockIdx.y, G = gridDim.y;
  const int hk = h / (a.Hq / a.Hk);
  const int N = a.N, D = a.D, tid = threadIdx.x;
  const T* qb = static_cast<const T*>(a.q_b) + (int64_t)h * N * D;
  const T* kb = static_cast<const T*>(a.k_b) + (int64_t)hk * N * D;
  fill_twiddles(tw, M);
  // load the group's dims of every row (contiguous in the row) into the
  // bit-reversed positions of the dpg transforms; rows past N are zero
  const int d0 = g * dpg;
  const int nd = min(dpg, D - d0);
  constexpr int V = 16 / sizeof(T);
  const bool vec = (nd % V) == 0 && (d0 % V) == 0 && (D % V) == 0;
  for (int n = tid; n < M; n += kFftThreads) {
    const int p = bitrev(n, logM);
    if (n >= N) {
      for (int e = 0; e < nd; ++e) buf[e * M + p] = make_float2(0.f, 0.f);
    } else if (vec) {
      for (int c = 0; c < nd; c += V) {
        const uint4 rq = *reinterpret_cast<const uint4*>(qb + (int64_t)n * D + d0 + c);
        const uint4 rk = *reinterpret_cast<const uint4*>(kb + (int64_t)n * D + d0 + c);
        const T* eq = reinterpret_cast<const T*>(&rq);
        const T* ek = reinterpret_cast<const T*>(&rk);
#pragma unroll
        for (int e = 0; e < V; ++e) buf[(c + e) * M + p] = make_float2(to_f32(eq[e]), to_f32(ek[e]));
      }
    } else {
      for (int e = 0; e < nd; ++e)
        buf[e * M + p] = make_float2(to_f32(qb[(int64_t)n * D + d0 + e]), to_f32(kb[(int64_t)n * D + d0 + e]));
    }
  }
  __syncthreads();
  fft_dit_batch(buf, tw, M, logM, nd);
  // X conj(Y) summed over the group's dims, in dim order
  const int nb = M / 2 + 1;
  float2* out = part + ((int64_t)h * G + g) * nb;
  for (int f = tid; f < nb; f += kFftThreads) {
    float2 acc = make_float2(0.f, 0.f);
    for (int e = 0; e < nd; ++e) {
      const float2 A = buf[e * M + f];
      const float2 Bc = buf[e * M + ((M - f) & (M - 1))];   // B = conj(Bc)
      // X conj(Y) = (A + B) conj(A - B) * i / 4
      const float2 P = make_float2(A.x + Bc.x, A.y - Bc.y);
      const float2 Qc = make_float2(A.x - Bc.x, -(A.y + Bc.y));
      const float2 pr = cmul(P, Qc);
      acc.x += -0.25f * pr.y;
      acc.y += 0.25f * pr.x;
    }
    out[f] = acc;
  }
}

__global__ __launch_bounds__(kFftThreads) void corr_final_kernel(fs_corr_args a, int M, int logM, int G,
                                                                 const float2* part) {
  extern __shared__ float2 smem[];
  float2* buf = smem;
  float2* tw = smem + M;
  float* cv = reinterpret_cast<float*>(smem + M + M / 2);
  __shared__ float red[32];
  __shared__ int ired[kTopkScratch];
  const int h = blockIdx.x, tid = threadIdx.x, N = a.N;
  const int nb = M / 2 + 1;
  fill_twiddles(tw, M);
  const float2* ph = part + (int64_t)h * G * nb;
  // conj of the Hermitian-completed spectrum, bit-reversed for the DIT FFT
  for (int f = tid; f < M; f += kFftThreads) {
    const int src = f <= M / 2 ? f : M - f;
    float2 c = make_float2(0.f, 0.f);
    for (int gi = 0; gi < G; ++gi) {
      const float2 p = ph[(int64_t)gi * nb + src];
      c.x += p.x;
      c.y += p.y;
    }
    if (f > M / 2) c.y = -c.y;
    buf[bitrev(f, logM)] = make_float2(c.x, -c.y);
  }
  __syncthreads();
  fft_dit(buf, tw, M, logM);
  const float invM = 1.0f / (float)M;
  // my_attn_v7.py:134-141: divide by the pair count, zero the excluded lags
  const int ex = a.local_window + 1;
  const int st = N - a.keep_sink - 5;
  const int es = min(ex, N);
  const int ss = st >= 0 ? min(st, N) : max(0, N + st);
  for (int t = tid; t < N; t += kFftThreads) {
    const float cs = buf[t].x * invM;
    if (a.corr_sum) a.corr_sum[(int64_t)h * N + t] = cs;
    float v = cs / (float)max(N - t, 1);
    if (t < es || t >= ss) v = 0.f;
    cv[t] = v;
  }
  __syncthreads();
  // :144-155: shift the band [ex, st) to a zero minimum, weight by log10 pair count
  if (ex < st) {
    float mn = INFINITY;
    for (int t = ex + tid; t < st; t += kFftThreads) mn = fminf(mn, cv[t]);
    mn = block_min(mn, red);
    const float den = clamp_min_nan(log10f((float)(N - ex)), 1e-6f);
    for (int t = ex + tid; t < st; t += kFftThreads) {
      const float pw = log10f((float)(N - t)) / den;
      cv[t] = (cv[t] - mn) * pw;
    }
    __syncthreads();
  }
  for (int t = tid; t < N; t += kFftThreads) a.corr[(int64_t)h * N + t] = cv[t];
  const int rs = a.remote_start;
  if (a.corr_mode == 1) {
    // :196-203 ("topk"): the quantile of the remote lags
    const float qv = block_quantile(cv + rs, N - rs, a.corr_quantile, ired);
    for (int t = tid; t < N; t += kFftThreads) a.keep_tau[(int64_t)h * N + t] = (t >= rs && cv[t] >= qv) ? 1 : 0;
  } else {
    // :205-208 ("threshold"): threshold on the max-normalised remote lags
    float mx = -INFINITY;
    for (int t = rs + tid; t < N; t += kFftThreads) mx = fmaxf(mx, cv[t]);
    mx = clamp_min_nan(block_max(mx, red), 1e-6f);
    for (int t = tid; t < N; t += kFftThreads)
      a.keep_tau[(int64_t)h * N + t] = (t >= rs && cv[t] / mx >= a.corr_threshold) ? 1 : 0;
  }
}

template <typename T>
static int launch_partial(const fs_corr_args& a, dim3 grid, size_t smem, int M, int logM, int dpg,
                          float2* part, hipStream_t s) {
  if (int rc = fs_host::allow_dynamic_lds(corr_partial_kernel<T>, smem, "fs_corr")) return rc;
  corr_partial_kernel<T><<<grid, kFftThreads, smem, s>>>(a, M, logM, dpg, part);
  return 0;
}

// dims per workgroup: dpg transforms of M complex values fill at most 128 KiB of LDS
static int dims_per_group(int N) {
  int logM = 1;
  while ((1 << logM) < 2 * N) ++logM;
  return std::min(8, 16384 >> logM);
}

static int corr_logM(int N) {
  int logM = 1;
  while ((1 << logM) < 2 * N) ++logM;
  return logM;
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_corr_work_bytes(int Hq, int N, int D) {
  if (Hq <= 0 || N <= 0 || D <= 0) return 0;
  const int M = 1 << corr_logM(N);
  const int dpg = dims_per_group(N);
  const int G = (D + dpg - 1) / dpg;
  return (size_t)Hq * G * (M / 2 + 1) * sizeof(float2);
}

extern "C" int fs_corr(const fs_corr_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_corr: null args");
  FS_CHECK_ARG(a->q_b && a->k_b && a->work && a->corr && a->keep_tau, "fs_corr: null pointer");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "fs_corr: Hq=%d must be a multiple of Hk=%d",
               a->Hq, a->Hk);
  FS_CHECK_ARG(a->N >= 1 && a->D >= 1, "fs_corr: bad sizes");
  FS_CHECK_ARG(a->remote_start >= 0 && a->local_window >= 0, "fs_corr: bad lag parameters");
  FS_CHECK_ARG(a->corr_mode == 0 || (a->corr_mode == 1 && a->remote_start < a->N && a->corr_quantile >= 0.f &&
                                     a->corr_quantile <= 1.f),
               "fs_corr: corr_mode must be 0 or 1; topk mode needs remote_start < N and a quantile in [0, 1]");
  const int logM = corr_logM(a->N);
  FS_CHECK_SUPPORTED(logM <= kMaxLogM, "fs_corr: N=%d exceeds the LDS FFT limit (N <= %d)", a->N,
                     1 << (kMaxLogM - 1));
  const int M = 1 << logM;
  const int dpg = dims_per_group(a->N);
  const int G = (a->D + dpg - 1) / dpg;
  hipStream_t s = (hipStream_t)stream;
  float2* part = static_cast<float2*>(a->work);
  const size_t sm_fft = (size_t)(M + M / 2) * sizeof(float2);
  const size_t sm1 = (size_t)(M / 2 + (size_t)dpg * M) * sizeof(float2);
  dim3 g1(a->Hq, G);
  int rc = 0;
  switch (a->dtype) {
    case FS_DTYPE_F32: rc = launch_partial<float>(*a, g1, sm1, M, logM, dpg, part, s); break;
    case FS_DTYPE_BF16: rc = launch_partial<bf16_t>(*a, g1, sm1, M, logM, dpg, part, s); break;
    case FS_DTYPE_F16: rc = launch_partial<f16_t>(*a, g1, sm1, M, logM, dpg, part, s); break;
    default: fs_host::set_error("fs_corr: dtype %d unsupported", a->dtype); return FS_ERR_UNSUPPORTED;
  }
  if (rc) return rc;
  rc = fs_host::launch_status("fs_corr partial");
  if (rc) return rc;
  const size_t sm2 = sm_fft + (size_t)a->N * sizeof(float);
  if ((rc = fs_host::allow_dynamic_lds(corr_final_kernel, sm2, "fs_corr"))) return rc;
  corr_final_kernel<<<a->Hq, kFftThreads, sm2, s>>>(*a, M, logM, G, part);
  return fs_host::launch_status("fs_corr final");
}
