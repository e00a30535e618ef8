// Block-mask composition into the row bitmask (FS_MASK_WORDS words per row)
// (reference: attn_src/fft_attn/my_attn_v7.py:542-550 prior, :558-560 last
// row, :588-612 stripe/diffuse dynamic mask, :256-294 qk top-k, :623-641
// columns; attn_src/fix_mask_attn/my_attn.py:39-79 for the fixed mask).
//
// One launch serves every head.  One workgroup (4 waves) owns RPW consecutive
// query-block rows of one head and decides from diag_var whether the head is
// a stripe or a diffuse head.  N <= 8192.  Stripe / fixed rows (Nk <= 4096)
// are built word-parallel: a lane forms the 64-bit membership mask of 64 key
// blocks (range masks for the prior, columns and causal limit; a
// funnel-shifted window of the bit-reversed lag mask for the lag diagonals)
// and stores it as word w of the row.  A diffuse head computes its score
// panel S[rows][0..last row] into LDS (fp32 dot products, fixed order) in
// passes of a few rows, so the LDS the launch reserves for the panel stays
// small enough for four workgroups per CU.  Each wave then walks one row at a
// time: for a diffuse row it finds the k_i-th largest score by a 32-step
// bisection on the ordered float key with wave-wide counts, and in a single
// ascending pass over the key blocks it evaluates the membership rule 64
// blocks at a time, the ballot of each pass being the row's next word.
#include <algorithm>

#include "common.h"

namespace fs {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kMaxWords = 64;                       // word-parallel path: Nk <= 4096
constexpr int kSelMaxN = 8192;                      // per-row path: flag bytes + a one-row score panel fit the LDS budget
constexpr int kMaxPanelRows = 16;                   // rows of a diffuse head's score panel per pass
constexpr size_t kSelLdsBudget = 52 * 1024;         // flag bytes + score panel + q rows (three workgroups per CU)

// LDS of the word-parallel path (the start of the launch's dynamic LDS)
struct WordRowsLds {
  uint64_t rkw[2 * kMaxWords + 2];                  // bit x: keep_tau[N-1-x] (x < N), 0 beyond
  uint64_t colw[kMaxWords], lastw[kMaxWords];
  uint32_t fk[4096 / 4], fc[4096 / 4], fl[4096 / 4];   // the staged flag bytes
};

// bits of word w (blocks 64w .. 64w+63) that lie in [lo, hi)
__device__ __forceinline__ uint64_t range_bits(int w, int lo, int hi) {
  const int b0 = max(lo - 64 * w, 0), b1 = min(hi - 64 * w, 64);
  if (b1 <= b0) return 0;
  const uint64_t upto = b1 == 64 ? ~0ull : ((1ull << b1) - 1);
  return upto & ~((1ull << b0) - 1);
}

// panel_rows: rows of a diffuse head's score panel per pass (0 without the
// dynamic mask).  Dynamic LDS: WordRowsLds (word-parallel rows) or, for the
// per-row path, the head's flag bytes [N], then the panel [panel_rows][N] and
// the pass's q rows [panel_rows][D].
template <typename T>
__global__ __launch_bounds__(kSelThreads) void select_kernel(fs_select_args a, int rows_per_wave, int panel_rows,
                                                             float inv_sqrt_d) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sel_lds[];
  const int RPW = rows_per_wave * kSelWaves;
  const int N = a.N, Nk = a.Nk, D = a.D;
  const int chunks = (N + RPW - 1) / RPW;
  const int h = blockIdx.x / chunks;
  const int r0 = (blockIdx.x - h * chunks) * RPW;
  const int hk = h / (a.Hq / a.Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NW = (Nk + 63) >> 6;                   // 64-block words per row
  const bool word_rows = NW <= kMaxWords;          // stripe / fixed rows are built word-parallel (below)

  // The word-parallel path stages the head's lag / column / last-row flags.
  // Their loads are issued here, before the decision's, so that one wait
  // covers both: flag bytes j = 4 w .. 4 w + 3 of word w = tid + 256 u.
  constexpr int kFlagWords = 4096 / 4 / kSelThreads;
  uint32_t fkr[kFlagWords], fcr[kFlagWords], flr[kFlagWords];
  const int nw4 = (N + 3) >> 2;
  if (word_rows) {                                 // (loaded for a diffuse head too: the decision comes later)
    const int64_t hb = (int64_t)h * N;
    const bool v4 = (N & 3) == 0;                  // row starts 4-byte aligned (buffers are)
#pragma unroll
    for (int u = 0; u < kFlagWords; ++u) {
      const int w4 = tid + u * kSelThreads;
      fkr[u] = fcr[u] = flr[u] = 0;
      if (w4 >= nw4) continue;
      if (v4) {
        if (a.keep_tau) fkr[u] = reinterpret_cast<const uint32_t*>(a.keep_tau + hb)[w4];
        if (a.col_sel) fcr[u] = reinterpret_cast<const uint32_t*>(a.col_sel + hb)[w4];
        if (a.last_sel) flr[u] = reinterpret_cast<const uint32_t*>(a.last_sel + hb)[w4];
      } else {
        for (int b = 0; b < 4 && 4 * w4 + b < N; ++b) {
          const int64_t j = hb + 4 * w4 + b;
          if (a.keep_tau) fkr[u] |= (uint32_t)a.keep_tau[j] << (8 * b);
          if (a.col_sel) fcr[u] |= (uint32_t)a.col_sel[j] << (8 * b);
          if (a.last_sel) flr[u] |= (uint32_t)a.last_sel[j] << (8 * b);
        }
      }
    }
  }

  // ---- stripe / diffuse decision (:359-363); identical in every workgroup of the head
  bool stripe = false;
  if (a.dyn_mode == 1) {
    float mv;
    if (a.stripe_all_diffuse) {
      mv = INFINITY;
    } else {
      // every wave forms the same sum (butterfly order is lane-independent)
      float s = 0.f;
      for (int i = lane; i < a.n_samples; i += 64) s += a.diag_var[(int64_t)h * a.n_samples + i];
      s = wave_sum(s);
      mv = s / (float)a.n_samples;
      stripe = mv <= a.stripe_threshold;        // false for nan
    }
    if (r0 == 0 && tid == 0) {
      if (a.mean_var) a.mean_var[h] = mv;
      if (a.is_stripe) a.is_stripe[h] = stripe ? 1 : 0;
    }
  }
  const bool diffuse = a.dyn_mode == 1 && !stripe;
  const bool words = word_rows && !diffuse;
  const bool use_lags = a.dyn_mode == 1 && stripe;
  const bool use_cols = a.col_mode == 2 || (a.col_mode == 1 && stripe);
  const int rend = min(N, r0 + RPW);

  const int lw = a.local_window;
  const bool has_last = a.last_sel != nullptr;
  if (words) {
    // ---- word-parallel rows: lane (row g, word w) builds the membership of
    // blocks 64w .. 64w+63 of its row as a 64-bit mask from per-head masks
    // staged in LDS and stores it as word w of the row; the row's count is
    // the sum of its words' popcounts.
    WordRowsLds& wl = *reinterpret_cast<WordRowsLds*>(sel_lds);
    uint64_t* rkw = wl.rkw;
    uint64_t* colw = wl.colw;
    uint64_t* lastw = wl.lastw;
    uint32_t* fk = wl.fk;
    uint32_t* fc = wl.fc;
    uint32_t* fl = wl.fl;
#pragma unroll
    for (int u = 0; u < kFlagWords; ++u) {
      const int w4 = tid + u * kSelThreads;
      if (w4 < nw4) {
        fk[w4] = fkr[u];
        fc[w4] = fcr[u];
        fl[w4] = flr[u];
      }
    }
    __syncthreads();
    auto flag = [](const uint32_t* f, int j) { return ((f[j >> 2] >> (8 * (j & 3))) & 255u) != 0; };
    for (int q = wave; q < 2 * NW + 2; q += kSelWaves) {
      const int x = 64 * q + lane;
      const bool kb = use_lags && x < N && flag(fk, N - 1 - x);
      const uint64_t m = __ballot(kb);
      if (lane == 0) rkw[q] = m;
      if (q < NW) {
        const bool cb = use_cols && x < N && flag(fc, x);
        const bool lb = has_last && x < N && flag(fl, x);
        const uint64_t mc = __ballot(cb), ml = __ballot(lb);
        if (lane == 0) {
          colw[q] = mc;
          lastw[q] = ml;
        }
      }
    }
    __syncthreads();
    int lpr = 1;                                   // lanes per row (power of two >= NW)
    while (lpr < NW) lpr <<= 1;
    const int rpi = 64 / lpr;                      // rows per wave pass
    const int w = lane & (lpr - 1), g = lane / lpr;
    for (int rr0 = wave * rpi; rr0 < RPW; rr0 += kSelWaves * rpi) {
      const int rr = rr0 + g;
      const int i = r0 + rr;
      const bool row_ok = rr < RPW && i < N;
      uint64_t m = 0;
      if (row_ok && w < NW) {
        const int jlim = a.mask_causal ? min(i + 1, Nk) : Nk;
        // prior (:83-95): sink | recent | local window
        m = range_bits(w, 0, a.keep_sink) | range_bits(w, Nk - a.keep_recent, Nk);
        if (lw > 0) m |= range_bits(w, i - lw, i + lw + 1);
        if (has_last && i == N - 1) m |= lastw[w];
        if (use_lags) {
          // bit b <-> lag t = i - 64w - b <-> rkw bit p0 + b, p0 = N-1-i+64w >= 0
          const int p0 = N - 1 - i + 64 * w;
          const int qw = p0 >> 6, sh = p0 & 63;
          uint64_t win = rkw[qw] >> sh;
          if (sh) win |= rkw[qw + 1] << (64 - sh);
          m |= win & range_bits(w, a.keep_sink, i - a.remote_start + 1);   // t >= rs, j >= keep_sink
        }
        if (use_cols) m |= colw[w] & range_bits(w, 0, i + 1);
        m &= range_bits(w, 0, jlim);
      }
      int c = __popcll(m);
      for (int o = lpr >> 1; o > 0; o >>= 1) c += __shfl_xor(c, o, lpr);
      if (row_ok) {
        if (w < NW) a.blk_bits[((int64_t)h * N + i) * NW + w] = m;
        if (w == 0) a.blk_cnt[(int64_t)h * N + i] = c;
      }
    }
    return;
  }
  // ---- per-head lag / column / last-row flags, staged in LDS (bit 0 lag, 1 column, 2 last row)
  uint8_t* flags = sel_lds;
  float* panel = reinterpret_cast<float*>(sel_lds + ((N + 15) & ~15));   // [panel_rows][N]
  float* qrows = panel + (size_t)panel_rows * N;                           // [panel_rows][D]
  for (int j = tid; j < N; j += kSelThreads) {
    uint8_t f = 0;
    if (a.keep_tau && a.keep_tau[(int64_t)h * N + j]) f |= 1;
    if (a.col_sel && a.col_sel[(int64_t)h * N + j]) f |= 2;
    if (a.last_sel && a.last_sel[(int64_t)h * N + j]) f |= 4;
    flags[j] = f;
  }
  __syncthreads();

  // rows r0 + p0 .. r0 + pend - 1 per pass: a diffuse head's panel holds
  // panel_rows rows; other heads take all their rows in one pass
  const int P = diffuse ? panel_rows : RPW;
  const int nrows = min(RPW, N - r0);
  for (int p0 = 0; p0 < nrows; p0 += P) {
    const int pend = min(nrows, p0 + P);
    if (diffuse) {
      // ---- score panel S[i][j] = (q_b[i] . k_b[j]) * (1/sqrt(D)), j <= last row of the pass (:234-249)
      const T* qb = static_cast<const T*>(a.q_b) + (int64_t)h * N * D;
      const T* kb = static_cast<const T*>(a.k_b) + (int64_t)hk * N * D;
      __syncthreads();                             // the previous pass is done with the panel
      for (int e = tid; e < P * D; e += kSelThreads) {
        const int rr = e / D, d = e - rr * D;
        qrows[e] = (p0 + rr < pend) ? to_f32(qb[(int64_t)(r0 + p0 + rr) * D + d]) : 0.f;
      }
      __syncthreads();
      const int jmax = r0 + pend;                  // columns 0 .. the pass's last row
      for (int j = tid; j < jmax; j += kSelThreads) {
        float acc[kMaxPanelRows];
#pragma unroll
        for (int rr = 0; rr < kMaxPanelRows; ++rr) acc[rr] = 0.f;
        const T* kr = kb + (int64_t)j * D;
        for (int d = 0; d < D; ++d) {
          const float kv = to_f32(kr[d]);
#pragma unroll
          for (int rr = 0; rr < kMaxPanelRows; ++rr)
            if (rr < P) acc[rr] += qrows[rr * D + d] * kv;
        }
#pragma unroll
        for (int rr = 0; rr < kMaxPanelRows; ++rr)
          if (rr < P) panel[(size_t)rr * N + j] = acc[rr] * inv_sqrt_d;
      }
      __syncthreads();
    }
    for (int rr = p0 + wave; rr < pend; rr += kSelWaves) {
      const int i = r0 + rr;
      const int jlim = a.mask_causal ? min(i + 1, Nk) : Nk;
      const float* srow = panel + (size_t)(rr - p0) * N;
      // ---- diffuse row: k_i-th largest of S[i][0..i] (:271-276)
      uint32_t thr = 0;
      int need = 0;
      if (diffuse) {
        int k = (int)((float)(i + 1) * a.qk_topk_ratio);
        if (k < 1) k = 1;
        const int n = i + 1;
        if (k > n) k = n;
        uint32_t prefix = 0;
        for (int b = 31; b >= 0; --b) {
          const uint32_t cand = prefix | (1u << b);
          int c = 0;
          for (int j0 = 0; j0 < n; j0 += 64) c += wave_count(j0 + lane < n && order_key(srow[j0 + lane]) >= cand);
          if (c >= k) prefix = cand;
        }
        int gt = 0;
        for (int j0 = 0; j0 < n; j0 += 64) gt += wave_count(j0 + lane < n && order_key(srow[j0 + lane]) > prefix);
        thr = prefix;
        need = k - gt;
      }
      // ---- membership in ascending block order, one word per 64 blocks
      uint64_t* out = a.blk_bits + ((int64_t)h * N + i) * NW;
      int cnt = 0, eq_seen = 0;
      for (int j0 = 0; j0 < jlim; j0 += 64) {
        const int j = j0 + lane;
        const bool valid = j < jlim;
        bool in = false;
        bool eq = false;
        if (valid) {
          // prior (:83-95): sink | recent | local window
          in = j < a.keep_sink || j >= Nk - a.keep_recent || (lw > 0 && abs(i - j) <= lw);
          const uint8_t fj = j < N ? flags[j] : 0;
          if (has_last && i == N - 1 && (fj & 4)) in = true;
          if (use_lags) {
            const int t = i - j;
            if (t >= a.remote_start && j >= a.keep_sink && (flags[t] & 1)) in = true;
          }
          if (diffuse && j <= i) {
            const uint32_t key = order_key(srow[j]);
            if (key > thr) in = true;
            eq = key == thr;
          }
          if (use_cols && j <= i && (fj & 2)) in = true;
        }
        if (diffuse) {
          const uint64_t me = __ballot(eq);
          if (eq && eq_seen + rank_below(me) < need) in = true;
          eq_seen += __popcll(me);
        }
        const uint64_t m = __ballot(in);
        if (lane == 0) out[j0 >> 6] = m;
        cnt += __popcll(m);
      }
      for (int w = ((jlim + 63) >> 6) + lane; w < NW; w += 64) out[w] = 0ull;   // words past the causal limit
      if (lane == 0) a.blk_cnt[(int64_t)h * N + i] = cnt;
    }
  }
}

template <typename T>
static int launch_select(const fs_select_args& a, unsigned grid, size_t smem, int rows_per_wave, int panel_rows,
                         float inv_sqrt_d, hipStream_t s) {
  if (int rc = fs_host::allow_dynamic_lds(select_kernel<T>, smem, "fs_select")) return rc;
  select_kernel<T><<<grid, kSelThreads, smem, s>>>(a, rows_per_wave, panel_rows, inv_sqrt_d);
  return 0;
}

}  // namespace fs

using namespace fs;

extern "C" int fs_select(const fs_select_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_select: null args");
  FS_CHECK_ARG(a->blk_cnt && a->blk_bits, "fs_select: null output");
  FS_CHECK_ARG(((uintptr_t)a->blk_bits & 7) == 0, "fs_select: blk_bits must be 8-byte aligned");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "fs_select: bad head counts");
  FS_CHECK_ARG(a->N >= 1 && a->Nk >= 1 && a->Nk <= 65535, "fs_select: bad block counts");
  FS_CHECK_ARG(a->dyn_mode == 0 || a->dyn_mode == 1, "fs_select: bad dyn_mode");
  FS_CHECK_ARG(a->col_mode >= 0 && a->col_mode <= 2, "fs_select: bad col_mode");
  FS_CHECK_ARG(a->dyn_mode == 0 || (a->q_b && a->k_b && a->keep_tau &&
                                    (a->stripe_all_diffuse || (a->diag_var && a->n_samples > 0))),
               "fs_select: dynamic mask inputs missing");
  FS_CHECK_ARG(a->col_mode == 0 || a->col_sel, "fs_select: col_sel missing");
  FS_CHECK_ARG(a->col_mode != 1 || a->dyn_mode == 1, "fs_select: col_mode 1 needs dyn_mode 1");
  FS_CHECK_ARG((a->dyn_mode == 0 && a->col_mode == 0 && a->last_sel == nullptr) || a->N == a->Nk,
               "fs_select: dynamic, column and last-row masks need N == Nk");
  FS_CHECK_SUPPORTED(a->N <= kSelMaxN && (a->dyn_mode == 0 || a->D <= 256), "fs_select: N=%d > %d or D=%d > 256",
                     a->N, kSelMaxN, a->D);
  // rows per wave: 16 word-parallel rows of <= 1024 blocks (four rows per
  // pass of 16 lanes each), fewer for longer rows; one on the per-row path
  const int NW = (a->Nk + 63) / 64;
  const int rows_per_wave = NW <= 16 ? 16 : (NW <= 32 ? 8 : (NW <= kMaxWords ? 4 : 1));
  const int RPW = rows_per_wave * kSelWaves;
  const int chunks = (a->N + RPW - 1) / RPW;
  const float inv_sqrt_d = a->D > 0 ? 1.0f / (float)sqrt((double)a->D) : 1.0f;
  // dynamic LDS: the word-parallel path's, or flag bytes + a diffuse head's
  // panel of panel_rows rows (a multiple of 4 rows when 4 fit) + its q rows
  const size_t flag_bytes = ((size_t)a->N + 15) & ~(size_t)15;
  int panel_rows = 0;
  if (a->dyn_mode == 1) {
    const size_t per_row = (size_t)(a->N + a->D) * sizeof(float);
    panel_rows = (int)std::min<size_t>((kSelLdsBudget - flag_bytes) / per_row, (size_t)std::min(RPW, kMaxPanelRows));
    if (panel_rows >= 4) panel_rows &= ~3;
    panel_rows = std::max(panel_rows, 1);
  }
  size_t smem = flag_bytes + (size_t)panel_rows * (a->N + a->D) * sizeof(float);
  if (NW <= kMaxWords) smem = std::max(smem, sizeof(WordRowsLds));
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = (unsigned)(a->Hq * chunks);
  const int dt = a->dyn_mode == 1 ? a->dtype : FS_DTYPE_F32;
  int rc = 0;
  switch (dt) {
    case FS_DTYPE_F32: rc = launch_select<float>(*a, grid, smem, rows_per_wave, panel_rows, inv_sqrt_d, s); break;
    case FS_DTYPE_BF16: rc = launch_select<bf16_t>(*a, grid, smem, rows_per_wave, panel_rows, inv_sqrt_d, s); break;
    case FS_DTYPE_F16: rc = launch_select<f16_t>(*a, grid, smem, rows_per_wave, panel_rows, inv_sqrt_d, s); break;
    default: fs_host::set_error("fs_select: dtype %d unsupported", a->dtype); return FS_ERR_UNSUPPORTED;
  }
  if (rc) return rc;
  return fs_host::launch_status("fs_select");
}
