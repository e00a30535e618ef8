// FlexPrefill block selection on gfx950 -- the reference's third selector
// (attn_src/Flexprefill.py:946-1061 get_active_blocks, with the budget
// arithmetic of Flexprefill_prefill :1063-1098), emitting the per-row block
// lists of the shared block-sparse attention kernel.
//
// flex_lastq_kernel<T, PASS, BS>: one workgroup (4 waves) per (head, chunk of
// kFChunk key columns).  The last bs queries, q / sqrt(D) rounded to T, are
// the B operand of v_mfma_f32_32x32x16 (wave w: row group w % (bs/32), column
// group w / (bs/32)); the 128-key K tiles are staged in swizzled LDS.  Scores
// are rounded to T (the reference's bf16 einsum), the last bs columns causal.
//  PASS 1: each row's max and sum of exp(x - max) over the chunk (partials).
//  PASS 2: the partials combined per row in a fixed order, p = exp(x - M) / S
//  written to an LDS tile [bs][128]; column sums (vertical) and the sums along
//  the diagonals ending at each column of the last row (slash), carried from
//  tile to tile (a diagonal spans bs columns), each / bs.  A chunk starts one
//  tile early so its first diagonals get their carry.
//  The block size is a template parameter: with a run-time sub-tile count the
//  MFMA chain holds branches, and on the path that leaves it after the first
//  32x32x16 the compiler's wait before reading that result's last accumulator
//  register was found too short (the read saw the value before the last MFMA).
// flex_kpool_kernel: block means of K over each block's real rows, in T.
// cut_pass_kernel<P> (four launches per cut): the mass cut of the descending
//   prefix sums at gamma (score_cover_topk / score_cover_idx) over many
//   workgroups: pass P histograms the P-th 8-bit digit of the order-preserving
//   key among the elements carrying the digits found so far, with exact
//   integer masses; jobs are the heads' vertical and slash profiles (budgets)
//   and, later, the sparse heads' block attention (covers).
// flex_head_kernel: one workgroup (1024 threads) per head:
//   budgets       the profiles' cover counts n + 1 (replayed from their cut
//                 histograms), // 128 + 1, clamped to the block budgets;
//   pooled        block sums of vertical / slash; the bs-row mean of the
//                 scaled last queries against the K block means (T), softmax;
//   js            square-root Jensen-Shannon divergence to the pooled vertical
//                 (a zero probability gives nan, as in the reference);
//   sparse heads  js < tau: both budgets become min_budget;
//   choice        the top budgets of pooled vertical (block 0 forced) and
//                 pooled slash (offset 0 forced), ties by the lower index, as
//                 bit masks.
// flex_cover_rows_kernel: for each sparse head, the block-level causal
//   attention softmax(avg_q / sqrt(D) avg_k^T) (block means of q, the last one
//   rescaled to its real rows); its cut at gamma * N by cut_pass_kernel, and
//   flex_cover_emit_kernel writes the kept entries as an N x N bit mask.
// flex_lists_kernel: per (head, block row r): the vertical columns <= r, the
//   diagonals r - s of the chosen slash offsets, the sparse cover's row, as an
//   ascending list (64-bit words, popcount offsets).
#include <algorithm>

#include "common.h"

namespace fs {

constexpr int kFD = 128;
constexpr int kFThreads = 256;
constexpr int kFTile = 128;                      // key columns per tile
constexpr int kFChunk = 2048;                    // key columns per workgroup
constexpr int kFHeadThreads = 1024;
constexpr int kFMaxBlocks = 8192;
constexpr int kFWords = kFMaxBlocks / 64;

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct FMma;
template <> struct FMma<bf16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
};
template <> struct FMma<f16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
};

constexpr float kLog2e = 1.4426950408889634f;

// floats of the region shared by the K tile and PASS 2's p tile [bs][kFTile + 4]
__host__ __device__ constexpr int flex_tile_floats(int bs) {
  return bs * (kFTile + 4) > kFTile * kFD / 2 ? bs * (kFTile + 4) : kFTile * kFD / 2;
}

// 2^x by the hardware exponential (v_exp_f32); exp(y) is taken as 2^(y log2 e)
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct FlexK {
  const uint16_t* q;            // [Hq][L][D] view (strides q_sh, q_sl)
  const uint16_t* k;
  int64_t q_sh, q_sl, k_sh, k_sl;
  int Hq, Hk, L, bs, nb, gqa_interleave, nchunk;
  float sqrt_d;
  float* part;                  // [Hq][nchunk][bs][2] (max, sum) per chunk
  float* vert;                  // [Hq][L]
  float* slash;                 // [Hq][L]
  uint64_t* p_hm;               // the cut histograms, zeroed here (PASS 1, chunk 0 of each head):
  uint32_t* p_hc;               //   profiles [4][2 Hq][256]
  uint64_t* c_hm;               //   covers [4][Hq][256]
  uint32_t* c_hc;
};

__device__ __forceinline__ int kv_head(int h, int Hq, int Hk, int interleave) {
  return interleave ? (h % Hk) : (h / (Hq / Hk));
}

template <typename T, int PASS, int BS>
__global__ __launch_bounds__(kFThreads) void flex_lastq_kernel(FlexK a) {
  // dynamic LDS: the K tile (32 KiB), which in PASS 2 shares its region with
  // the p tile (formed after the MFMAs have read K), then PASS 2's carry, row
  // statistics and column half sums (PASS 1: the lane partials after the loop)
  extern __shared__ __attribute__((aligned(16))) float dyn[];
  uint16_t* lk = reinterpret_cast<uint16_t*>(dyn);
  const int h = blockIdx.x / a.nchunk, chunk = blockIdx.x % a.nchunk;
  const int kvh = kv_head(h, a.Hq, a.Hk, a.gqa_interleave);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hi = lane >> 5;
  constexpr int bs = BS;
  const int L = a.L;
  // 32-row groups of the last block's queries; 16-token blocks fill half of
  // one group (rows 16 .. 31 have no query: zero operands, no scores kept)
  constexpr int RG = bs >= 32 ? bs / 32 : 1, CG = 4 / RG;   // row groups, column groups
  const int rg = wave % RG, cg = wave / RG;
  constexpr int nsub = (kFTile / CG) / 32;        // 32-column sub-tiles per wave: 4 / CG
  const int row = rg * 32 + l32;                  // this lane's query row (0 .. bs-1)
  const bool row_ok = row < bs;
  const int qtok = L - bs + (row_ok ? row : 0);
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)kvh * a.k_sh;

  // B operand: q[L-bs+row] / sqrt(D) rounded to T, dims st*16 + hi*8 .. +7
  uint4 qf[kFD / 16];
#pragma unroll
  for (int st = 0; st < kFD / 16; ++st) {
    const uint4 raw = row_ok ? *reinterpret_cast<const uint4*>(qh + (int64_t)qtok * a.q_sl + st * 16 + hi * 8)
                             : make_uint4(0, 0, 0, 0);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = to_f32(T{(uint16_t)(w[e] & 0xffffu)}) / a.sqrt_d;
      const float up = to_f32(T{(uint16_t)(w[e] >> 16)}) / a.sqrt_d;
      o[e] = (uint32_t)__builtin_bit_cast(uint16_t, Conv<T>::store(lo)) |
             ((uint32_t)__builtin_bit_cast(uint16_t, Conv<T>::store(up)) << 16);
    }
    qf[st] = make_uint4(o[0], o[1], o[2], o[3]);
  }

  const int c_begin = chunk * kFChunk;
  const int c_end = min(L, c_begin + kFChunk);
  // PASS 2 starts one tile early (carry of the diagonals that cross into the chunk)
  const int t_first = (PASS == 2 && chunk > 0) ? c_begin - kFTile : c_begin;
  const int lim_causal = L - bs + row;            // the last block: key <= query
  const int c_valid = PASS == 1 ? c_end : L;      // PASS 2 also forms the carry tile before the chunk
  float m_run = -INFINITY, l_run = 0.f;           // PASS 1, per lane, log2 domain (partial over its columns)
  float M2 = 0.f, inv_s = 0.f;                    // PASS 2: the row's max (log2 domain) and 1 / sum
  constexpr int PS = kFTile + 4;                  // p-tile row stride: 16-byte row chunks spread over the banks
  float* ptl = dyn;                               // [bs][PS], over the K tile
  float* carry = dyn + flex_tile_floats(bs);      // [kFTile + bs] diagonal partials in flight
  float* rowstat = carry + kFTile + bs;           // [bs][2]
  float* vpart = rowstat + 2 * bs;                // [kFThreads] column sums of the two row halves
  if (PASS == 1 && chunk == 0) {
    // this head's cut histograms (profiles 2 h, 2 h + 1 and cover h, four passes)
    for (int e = tid; e < 4 * 3 * 256; e += kFThreads) {
      const int p = e / (3 * 256), r = e - p * 3 * 256, jj = r >> 8, d = r & 255;
      if (jj < 2) {
        const int64_t i = ((int64_t)p * 2 * a.Hq + 2 * h + jj) * 256 + d;
        a.p_hm[i] = 0;
        a.p_hc[i] = 0;
      } else {
        const int64_t i = ((int64_t)p * a.Hq + h) * 256 + d;
        a.c_hm[i] = 0;
        a.c_hc[i] = 0;
      }
    }
  }
  if (PASS == 2) {
    // combine the chunk partials of each row in a fixed order
    if (tid < bs) {
      const float* pp = a.part + ((int64_t)h * a.nchunk) * bs * 2;
      float mx = -INFINITY;
      for (int c = 0; c < a.nchunk; ++c) mx = fmaxf(mx, pp[((int64_t)c * bs + tid) * 2]);
      float s = 0.f;
      for (int c = 0; c < a.nchunk; ++c) {
        const float mc = pp[((int64_t)c * bs + tid) * 2], lc = pp[((int64_t)c * bs + tid) * 2 + 1];
        if (mc > -INFINITY) s += lc * fexp2(mc - mx);
      }
      rowstat[tid * 2] = mx;
      rowstat[tid * 2 + 1] = 1.0f / s;
    }
    for (int e = tid; e < kFTile + bs; e += kFThreads) carry[e] = 0.f;
    __syncthreads();
    M2 = row_ok ? rowstat[row * 2] : 0.f;
    inv_s = row_ok ? rowstat[row * 2 + 1] : 0.f;
  }

  for (int t0 = t_first; t0 < c_end; t0 += kFTile) {
    __syncthreads();                               // previous K tile / p tile consumed
    {
      uint4 kv[kFTile * 16 / kFThreads];
#pragma unroll
      for (int u = 0; u < kFTile * 16 / kFThreads; ++u) {
        const int e = tid + u * kFThreads, c = e >> 4, ch = e & 15;
        const int t = t0 + c;
        kv[u] = t < L ? *reinterpret_cast<const uint4*>(kh + (int64_t)t * a.k_sl + ch * 8) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kFTile * 16 / kFThreads; ++u) {
        const int e = tid + u * kFThreads, c = e >> 4, ch = e & 15;
        *reinterpret_cast<uint4*>(lk + c * kFD + ((ch ^ (c & 15)) << 3)) = kv[u];
      }
    }
    __syncthreads();
    f32x16_t acc[nsub];
#pragma unroll
    for (int s = 0; s < nsub; ++s)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[s][r] = 0.f;
#pragma unroll
    for (int st = 0; st < kFD / 16; ++st) {
#pragma unroll
      for (int s = 0; s < nsub; ++s) {
        const int kr = (cg * nsub + s) * 32 + l32;
        const uint4 ak = *reinterpret_cast<const uint4*>(lk + kr * kFD + (((2 * st + hi) ^ (kr & 15)) << 3));
        acc[s] = FMma<T>::mma(ak, qf[st], acc[s]);
      }
    }
    // lane: keys t0 + (cg nsub + s) 32 + (r/4) 8 + hi 4 + r%4 of query row `row`; the
    // scores rounded to T (the reference's einsum output), then to the log2 domain
    float x[nsub][16];
#pragma unroll
    for (int s = 0; s < nsub; ++s)
#pragma unroll
      for (int r = 0; r < 16; ++r) x[s][r] = Conv<T>::round(acc[s][r]) * kLog2e;
    if (PASS == 2) __syncthreads();                // every wave has read the K tile: the p tile overwrites it
    // every column of the tile valid and causal for every row
    const bool interior = t0 + kFTile <= c_valid && t0 + kFTile - 1 <= L - bs;
    auto valid = [&](int c) { return row_ok && (interior || (c < c_valid && c <= lim_causal)); };
    if (PASS == 1) {
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < nsub; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = t0 + (cg * nsub + s) * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
          if (valid(c)) mx = fmaxf(mx, x[s][r]);
        }
      const float m_new = fmaxf(m_run, mx);
      if (m_new > -INFINITY) {
        float sum = 0.f;
#pragma unroll
        for (int s = 0; s < nsub; ++s)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int c = t0 + (cg * nsub + s) * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
            if (valid(c)) sum += fexp2(x[s][r] - m_new);
          }
        l_run = l_run * fexp2(m_run - m_new) + sum;
        m_run = m_new;
      }
    } else {
      // p tile [bs][PS] in LDS, four consecutive columns per 16-byte write
#pragma unroll
      for (int s = 0; s < nsub; ++s)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int cl = (cg * nsub + s) * 32 + g4 * 8 + hi * 4;
          float4 v;
          v.x = valid(t0 + cl + 0) ? fexp2(x[s][g4 * 4 + 0] - M2) * inv_s : 0.f;
          v.y = valid(t0 + cl + 1) ? fexp2(x[s][g4 * 4 + 1] - M2) * inv_s : 0.f;
          v.z = valid(t0 + cl + 2) ? fexp2(x[s][g4 * 4 + 2] - M2) * inv_s : 0.f;
          v.w = valid(t0 + cl + 3) ? fexp2(x[s][g4 * 4 + 3] - M2) * inv_s : 0.f;
          if (row_ok) *reinterpret_cast<float4*>(ptl + row * PS + cl) = v;
        }
      __syncthreads();
      // vertical: each column's rows in two halves (threads tid and tid + kFTile), four running sums each
      if (t0 >= c_begin) {
        const int cl = tid & (kFTile - 1), half = tid / kFTile;
        const float* col = ptl + half * (bs / 2) * PS + cl;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int i = 0; i < bs / 2; i += 4) {
          s0 += col[(i + 0) * PS];
          s1 += col[(i + 1) * PS];
          s2 += col[(i + 2) * PS];
          s3 += col[(i + 3) * PS];
        }
        vpart[tid] = (s0 + s1) + (s2 + s3);
      }
      // slash: diagonal x = t0 + j (ending at column x of the last row) takes
      // p[i][j + i - (bs-1)] for the rows whose column falls in this tile;
      // this tile adds to the diagonals x in [t0, t0 + kFTile + bs - 1)
      float dsum = 0.f;
      if (tid < kFTile + bs - 1) {
        const int j = tid;
        const int ilo = max(0, bs - 1 - j), ihi = min(bs, kFTile + bs - 1 - j);
        const int base = j - (bs - 1);             // row i's element sits at i (PS + 1) + base
        float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
        int i = ilo;
        for (; i + 4 <= ihi; i += 4) {
          d0 += ptl[(i + 0) * (PS + 1) + base];
          d1 += ptl[(i + 1) * (PS + 1) + base];
          d2 += ptl[(i + 2) * (PS + 1) + base];
          d3 += ptl[(i + 3) * (PS + 1) + base];
        }
        for (; i < ihi; ++i) d0 += ptl[i * (PS + 1) + base];
        dsum = (d0 + d1) + (d2 + d3);
      }
      __syncthreads();                             // vpart written; carry read below is rewritten after
      if (tid < kFTile) {
        const int xcol = t0 + tid;
        if (t0 >= c_begin && xcol < c_end) {
          a.vert[(int64_t)h * L + xcol] = (vpart[tid] + vpart[tid + kFTile]) / (float)bs;
          a.slash[(int64_t)h * L + xcol] = (carry[tid] + dsum) / (float)bs;   // complete: no later column reaches x
        }
      }
      __syncthreads();
      if (tid >= kFTile && tid < kFTile + bs - 1) carry[tid - kFTile] = dsum;
      for (int e = bs - 1 + tid; e < kFTile + bs; e += kFThreads) carry[e] = 0.f;
    }
  }
  if (PASS == 1) {
    // combine the row's columns held by the lanes of all column groups and both halves
    __syncthreads();                               // the K tile is dead
    float* red = dyn;                              // [4 waves][64 lanes][2]
    red[(wave * 64 + lane) * 2] = m_run;
    red[(wave * 64 + lane) * 2 + 1] = l_run;
    __syncthreads();
    if (tid < bs) {
      const int rgi = tid / 32, li = tid % 32;
      float mx = -INFINITY;
      for (int c = 0; c < CG; ++c)
        for (int hh = 0; hh < 2; ++hh) mx = fmaxf(mx, red[(((c * RG + rgi) * 64) + hh * 32 + li) * 2]);
      float s = 0.f;
      for (int c = 0; c < CG; ++c)
        for (int hh = 0; hh < 2; ++hh) {
          const int idx = (((c * RG + rgi) * 64) + hh * 32 + li) * 2;
          if (red[idx] > -INFINITY) s += red[idx + 1] * fexp2(red[idx] - mx);
        }
      float* pp = a.part + (((int64_t)h * a.nchunk + chunk) * bs + tid) * 2;
      pp[0] = mx;
      pp[1] = s;
    }
  }
}

// block means of K over each block's real rows (triton_bnhd_pool "avg", Flexprefill.py:656-782)
template <typename T>
__global__ __launch_bounds__(kFThreads) void flex_kpool_kernel(const uint16_t* __restrict__ k, int64_t k_sh,
                                                               int64_t k_sl, int L, int bs, int nb,
                                                               uint16_t* __restrict__ avg_k) {
  const int hk = blockIdx.x / nb, j = blockIdx.x % nb;
  const int t0 = j * bs, rows = min(bs, L - t0);
  const uint16_t* src = k + (int64_t)hk * k_sh;
  for (int d = threadIdx.x; d < kFD; d += kFThreads) {
    float s = 0.f;
    for (int r = 0; r < rows; ++r) s += to_f32(T{src[(int64_t)(t0 + r) * k_sl + d]});
    avg_k[((int64_t)hk * nb + j) * kFD + d] = __builtin_bit_cast(uint16_t, Conv<T>::store(s / (float)rows));
  }
}

// ---- block reductions over 1024 threads (fixed order) ---------------------
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  for (int s = kFHeadThreads / 2; s > 0; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  const double r = red[0];
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum_f(float v, double* red) {
  return (float)block_sum_d((double)v, red);
}
__device__ __forceinline__ float block_max_f(float v, double* red) {
  const int tid = threadIdx.x;
  red[tid] = (double)v;
  __syncthreads();
  for (int s = kFHeadThreads / 2; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmax(red[tid], red[tid + s]);
    __syncthreads();
  }
  const float r = (float)red[0];
  __syncthreads();
  return r;
}

// ---- the K largest by a radix cut on order-preserving keys (one 1024-thread workgroup)
// Four passes over the data, one 8-bit digit of the key per pass (most
// significant first): a histogram of the digit among the elements that share
// the digits found so far, then one wave scans it from the largest digit down
// for the digit where the count of larger elements reaches K.  The histogram is
// kept in kCutCopies copies, one per lane residue, so that at most
// 64 / kCutCopies lanes of a wave add to one address.
constexpr int kCutCopies = 8;                    // histogram copies: lane l adds to copy l % 8

struct CutScratch {
  uint32_t hc[kCutCopies][256]; // count per digit
  int cnt;                      // crossing: count of the elements above its digit
  int digit;                    // crossing digit, -1: none
};

struct CutResult {
  int count;                    // elements in the cut
  uint32_t key;                 // boundary key: every larger key is in the cut
  int take_eq;                  // elements equal to the boundary key in the cut (lowest index first)
  int eq_total;                 // elements equal to the boundary key
};

// the `want` largest of x[0 .. n) (1 <= want; all of them when want >= n)
__device__ CutResult radix_topk(const float* x, int n, int want, CutScratch* cs) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0;
  int cnt_above = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int e = tid; e < kCutCopies * 256; e += kFHeadThreads) (&cs->hc[0][0])[e] = 0;
    if (tid == 0) cs->digit = -1;
    __syncthreads();
    const int copy = tid % kCutCopies;
    for (int i = tid; i < n; i += kFHeadThreads) {
      const uint32_t key = order_key(x[i]);
      if (pass == 0 || (key >> (shift + 8)) == prefix) atomicAdd(&cs->hc[copy][(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l: digits 255 - 4l .. 252 - 4l, largest first
      uint32_t lc[4], scn = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int d = 255 - 4 * tid - t;
        lc[t] = 0;
#pragma unroll
        for (int r = 0; r < kCutCopies; ++r) lc[t] += cs->hc[r][d];
        scn += lc[t];
      }
      uint32_t ic = scn;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t vc = __shfl_up(ic, o, 64);
        if (tid >= o) ic += vc;
      }
      uint32_t runc = (uint32_t)cnt_above + (ic - scn);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t prevc = runc;
        runc += lc[t];
        if (prevc < (uint32_t)want && runc >= (uint32_t)want) {
          cs->digit = 255 - 4 * tid - t;
          cs->cnt = (int)prevc;
        }
      }
    }
    __syncthreads();
    const int d = cs->digit;
    if (d < 0) {                                   // want >= n: everything (first pass only)
      __syncthreads();
      return {n, 0u, 0, 0};
    }
    prefix = (prefix << 8) | (uint32_t)d;
    cnt_above = cs->cnt;
    uint32_t eq = 0;
    for (int r = 0; r < kCutCopies; ++r) eq += cs->hc[r][d];
    __syncthreads();                               // cs is rewritten by the next pass / call
    if (pass == 3) return {want, prefix, want - cnt_above, (int)eq};
  }
  return {n, 0u, 0, 0};                            // not reached
}

// Writes, in out, the bits of the elements of a cut: every key above cut.key
// and the first cut.take_eq elements equal to it in index order.  Element i of
// a row of row_len elements is bit i % row_len of row i / row_len, rows kFWords
// words apart; every word of the rows' first ceil(row_len / 64) is written (one
// ballot per word, no atomics).  Each wave owns a contiguous range of words;
// when the cut splits the elements equal to its key, a fixed-order prefix of
// the waves' tie counts ranks them.
// Words wb .. we-1 only, with base_rank ties before them, when given.
__device__ void emit_cut(const float* x, int rows, int row_len, const CutResult& cut, uint64_t* out, int* scan,
                         int wb = 0, int we = -1, int base_rank = 0) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = kFHeadThreads / 64;
  const int wpr = (row_len + 63) >> 6;             // words per row
  if (we < 0) we = rows * wpr;
  const int per = (we - wb + kWaves - 1) / kWaves;
  const int w0 = min(we, wb + wave * per), w1 = min(we, w0 + per);
  const bool ranked = cut.take_eq > 0 && cut.take_eq < cut.eq_total;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;   // lanes under this one
  int rank = base_rank;
  if (ranked) {
    int cnt = 0;
    for (int w = w0; w < w1; ++w) {
      const int r = w / wpr, c = (w - r * wpr) * 64 + lane;
      const bool eq = c < row_len && order_key(x[(int64_t)r * row_len + c]) == cut.key;
      cnt += __popcll(__ballot(eq));
    }
    if (lane == 0) scan[wave] = cnt;
    __syncthreads();
    for (int v = 0; v < wave; ++v) rank += scan[v];
    __syncthreads();                               // scan is reused by the caller
  }
  for (int w = w0; w < w1; ++w) {
    const int r = w / wpr, c = (w - r * wpr) * 64 + lane;
    bool in = false, eq = false;
    if (c < row_len) {
      const uint32_t k = order_key(x[(int64_t)r * row_len + c]);
      in = k > cut.key;
      eq = k == cut.key;
    }
    if (ranked) {
      const uint64_t eqm = __ballot(eq);
      in = in || (eq && rank + __popcll(eqm & below) < cut.take_eq);
      rank += __popcll(eqm);
    } else {
      in = in || (eq && cut.take_eq > 0);
    }
    const uint64_t word = __ballot(in);
    if (lane == 0) out[(int64_t)r * kFWords + (w - r * wpr)] = word;
  }
}

// ---- the same mass cuts over many workgroups -----------------------------
// A job is one array to cut: a head's vertical or slash profile (the budgets)
// or a sparse head's N x N block attention (its cover).  Pass p is one launch
// over (job, slice) workgroups: each histograms the p-th key digit of its
// slice's elements that carry the digits found by passes < p (replayed from
// those passes' global histograms by one wave) and adds its histogram to the
// job's global one with integer atomics (exact, so independent of order).
constexpr int kCutSliceThreads = 256;

struct CutJobs {
  const float* x0;              // kind 0 data of head h at x0 + h * stride
  const float* x1;              // kind 1 data (kinds == 2)
  int64_t stride;
  int n;                        // elements per job
  int kinds;                    // jobs per head (1 or 2)
  int jobs, slices;
  int scale_exp;                // masses as integers x * 2^scale_exp
  double g;                     // mass bound of the cut
  const int32_t* info;          // [Hq][4]: only the jobs of sparse heads run (null: every job)
  uint64_t* hm;                 // [4][jobs][256] mass per digit (zeroed before pass 0)
  uint32_t* hc;                 // [4][jobs][256] count per digit
};

__device__ __forceinline__ const float* job_data(const CutJobs& c, int j) {
  const int h = j / c.kinds, kind = j - h * c.kinds;
  return (kind ? c.x1 : c.x0) + (int64_t)h * c.stride;
}
__device__ __forceinline__ bool job_live(const CutJobs& c, int j) {
  return c.info == nullptr || c.info[(j / c.kinds) * 4 + 2] != 0;
}

struct CutState {
  uint64_t above, mass;         // mass above the digits found so far; crossing scratch
  uint32_t prefix, eq;          // digits found so far; elements equal to the boundary key
  int cnt_above, cnt, digit;
  int all;                      // 1: everything is in the cut
};

// Replays passes 0 .. npass-1 of job j from the global histograms into st (LDS);
// every thread of the workgroup calls it, lanes 0-63 scan.
__device__ void cut_replay(const CutJobs& c, int j, int npass, CutState* st) {
  const int tid = threadIdx.x;
  const uint64_t G = (uint64_t)(c.g * ldexp(1.0, c.scale_exp));
  __syncthreads();                                 // st of an earlier call has been read
  if (tid == 0) {
    st->prefix = 0;
    st->above = 0;
    st->cnt_above = 0;
    st->all = 0;
    st->eq = 0;
  }
  __syncthreads();
  for (int p = 0; p < npass; ++p) {
    if (tid == 0) st->digit = -1;
    __syncthreads();
    if (tid < 64 && !st->all) {
      const uint64_t* hm = c.hm + ((int64_t)p * c.jobs + j) * 256;
      const uint32_t* hc = c.hc + ((int64_t)p * c.jobs + j) * 256;
      uint64_t lm[4], sm = 0;
      uint32_t lc[4], scn = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int d = 255 - 4 * tid - t;
        lm[t] = hm[d];
        lc[t] = hc[d];
        sm += lm[t];
        scn += lc[t];
      }
      uint64_t im = sm;
      uint32_t ic = scn;
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t vm = __shfl_up(im, o, 64);
        const uint32_t vc = __shfl_up(ic, o, 64);
        if (tid >= o) {
          im += vm;
          ic += vc;
        }
      }
      uint64_t run = st->above + (im - sm);
      uint32_t runc = (uint32_t)st->cnt_above + (ic - scn);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint64_t prev = run;
        const uint32_t prevc = runc;
        run += lm[t];
        runc += lc[t];
        if (prev <= G && run > G) {
          st->digit = 255 - 4 * tid - t;
          st->mass = prev;
          st->cnt = (int)prevc;
          st->eq = lc[t];
        }
      }
    }
    __syncthreads();
    if (tid == 0 && !st->all) {
      if (st->digit < 0) {
        st->all = 1;
      } else {
        st->prefix = (st->prefix << 8) | (uint32_t)st->digit;
        st->above = st->mass;
        st->cnt_above = st->cnt;
      }
    }
    __syncthreads();
  }
}

// the cut after the four passes
__device__ CutResult cut_result(const CutJobs& c, const CutState& st) {
  if (st.all) return {c.n, 0u, 0, 0};
  const double sc = ldexp(1.0, c.scale_exp);
  const uint64_t G = (uint64_t)(c.g * sc);
  const uint64_t mv = (uint64_t)((double)key_to_f32(st.prefix) * sc);   // > 0: it pushed the sum past G
  const uint64_t fit = mv ? (G - st.above) / mv : (uint64_t)st.eq;
  const int take = (int)(fit < (uint64_t)st.eq ? fit : (uint64_t)st.eq);
  return {st.cnt_above + take, st.prefix, take, (int)st.eq};
}

template <int PASS>
__global__ __launch_bounds__(kCutSliceThreads) void cut_pass_kernel(CutJobs c) {
  __shared__ uint64_t lhm[kCutCopies][256];
  __shared__ uint32_t lhc[kCutCopies][256];
  __shared__ CutState st;
  const int j = blockIdx.x / c.slices, sl = blockIdx.x - j * c.slices;
  if (!job_live(c, j)) return;
  const int tid = threadIdx.x;
  cut_replay(c, j, PASS, &st);
  if (st.all) return;
  for (int e = tid; e < kCutCopies * 256; e += kCutSliceThreads) {
    (&lhm[0][0])[e] = 0;
    (&lhc[0][0])[e] = 0;
  }
  __syncthreads();
  const float* x = job_data(c, j);
  const int per = (c.n + c.slices - 1) / c.slices;
  const int i0 = sl * per, i1 = min(c.n, i0 + per);
  const double sc = ldexp(1.0, c.scale_exp);
  constexpr int shift = 24 - 8 * PASS;
  const uint32_t prefix = st.prefix;
  const int copy = tid % kCutCopies;
  for (int i = i0 + tid; i < i1; i += kCutSliceThreads) {
    const float v = x[i];
    const uint32_t key = order_key(v);
    if (PASS == 0 || (key >> (shift + 8)) == prefix) {
      const uint32_t d = (key >> shift) & 255u;
      const uint64_t m = (uint64_t)((double)v * sc);
      if (m) atomicAdd(reinterpret_cast<unsigned long long*>(&lhm[copy][d]), (unsigned long long)m);
      atomicAdd(&lhc[copy][d], 1u);
    }
  }
  __syncthreads();
  uint64_t* hm = c.hm + ((int64_t)PASS * c.jobs + j) * 256;
  uint32_t* hc = c.hc + ((int64_t)PASS * c.jobs + j) * 256;
  for (int d = tid; d < 256; d += kCutSliceThreads) {
    uint64_t m = 0;
    uint32_t k = 0;
#pragma unroll
    for (int r = 0; r < kCutCopies; ++r) {
      m += lhm[r][d];
      k += lhc[r][d];
    }
    if (k) {
      atomicAdd(reinterpret_cast<unsigned long long*>(&hm[d]), (unsigned long long)m);
      atomicAdd(&hc[d], k);
    }
  }
}

struct FlexHeadK {
  const uint16_t* q;
  int64_t q_sh, q_sl;
  const uint16_t* avg_k;        // [Hk][nb][D]
  const float* vert;            // [Hq][L]
  const float* slash;
  int Hq, Hk, L, bs, nb, gqa_interleave, min_b, max_b;
  float sqrt_d, gamma, tau;
  uint64_t* vmask;              // [Hq][kFWords] chosen vertical blocks
  uint64_t* smask;              // [Hq][kFWords] chosen slash offsets
  int32_t* info;                // [Hq][4]: num_vertical, num_slash, sparse, cover counts packed below
  float* js;                    // [Hq]
  CutJobs pcut;                 // the profiles' cuts (jobs 2 h, 2 h + 1), histograms complete
};

// the K largest of v[0 .. n) (ties: lower index first) as bits of out[kFWords]
__device__ void topk_bits(const float* v, int n, int K, uint64_t* out, CutScratch* cs, int* scan) {
  const int tid = threadIdx.x;
  for (int w = tid; w < kFWords; w += kFHeadThreads) out[w] = 0;
  __syncthreads();
  if (K <= 0) return;
  const CutResult cut = radix_topk(v, n, K, cs);
  emit_cut(v, 1, n, cut, out, scan);
  __syncthreads();
}

template <typename T>
__global__ __launch_bounds__(kFHeadThreads) void flex_head_kernel(FlexHeadK a) {
  __shared__ double red[kFHeadThreads];
  __shared__ float lqm[kFD];
  __shared__ CutScratch cs;
  extern __shared__ float pooled[];                // pv, ps, pk: [nb] each
  float* pv = pooled;
  float* ps = pooled + a.nb;
  float* pk = pooled + 2 * a.nb;
  int* scan = reinterpret_cast<int*>(red);         // the tie ranks reuse the reduction buffer
  const int h = blockIdx.x, tid = threadIdx.x;
  const int L = a.L, bs = a.bs, nb = a.nb;
  const float* vt = a.vert + (int64_t)h * L;
  const float* st = a.slash + (int64_t)h * L;
  const int kvh = kv_head(h, a.Hq, a.Hk, a.gqa_interleave);

  // cover counts (score_cover_topk) -> block budgets
  __shared__ CutState cst;
  cut_replay(a.pcut, 2 * h, 4, &cst);
  int nv = cut_result(a.pcut, cst).count + 1;
  cut_replay(a.pcut, 2 * h + 1, 4, &cst);
  int ns = cut_result(a.pcut, cst).count + 1;
  nv = nv / 128 + 1;
  ns = ns / 128 + 1;
  nv = min(max(nv, a.min_b), a.max_b);
  ns = min(max(ns, a.min_b), a.max_b);

  // pooled vertical / slash (block sums in order; the loads of 8 entries are
  // issued before they are added; entries past L read as 0)
  for (int j = tid; j < nb; j += kFHeadThreads) {
    float sv = 0.f, ss = 0.f;
    for (int c0 = j * bs; c0 < (j + 1) * bs; c0 += 8) {
      float xv[8], xs[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const bool in = c0 + u < L;
        xv[u] = in ? vt[c0 + u] : 0.f;
        xs[u] = in ? st[c0 + u] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        sv += xv[u];
        ss += xs[u];
      }
    }
    pv[j] = sv;
    ps[j] = ss;
  }
  // mean over the bs rows of the scaled last queries, in T (8 loads issued at a time)
  if (tid < kFD) {
    const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
    float s = 0.f;
    for (int i0 = 0; i0 < bs; i0 += 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = to_f32(T{qh[(int64_t)(L - bs + i0 + u) * a.q_sl + tid]}) / a.sqrt_d;
#pragma unroll
      for (int u = 0; u < 8; ++u) s += Conv<T>::round(x[u]);
    }
    lqm[tid] = Conv<T>::round(s / (float)bs);
  }
  __syncthreads();
  // avg_qk (T) and its softmax over the blocks (a K block mean in two halves of
  // 8 loads of 8 dims)
  float mx = -INFINITY;
  for (int j = tid; j < nb; j += kFHeadThreads) {
    const uint4* kr = reinterpret_cast<const uint4*>(a.avg_k + ((int64_t)kvh * nb + j) * kFD);
    float s = 0.f;
#pragma unroll 1
    for (int c0 = 0; c0 < kFD / 8; c0 += 8) {
      uint4 kv[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) kv[c] = kr[c0 + c];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t w[4] = {kv[c].x, kv[c].y, kv[c].z, kv[c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) s += lqm[8 * (c0 + c) + e] * to_f32(T{(uint16_t)(w[e >> 1] >> (16 * (e & 1)))});
      }
    }
    pk[j] = Conv<T>::round(s);
    mx = fmaxf(mx, pk[j]);
  }
  mx = block_max_f(mx, red);
  float se = 0.f;
  for (int j = tid; j < nb; j += kFHeadThreads) {
    pk[j] = expf(pk[j] - mx);
    se += pk[j];
  }
  se = block_sum_f(se, red);
  // square-root JS divergence (nan when a probability is 0, as the reference's p log(p/m))
  float t1 = 0.f, t2 = 0.f;
  for (int j = tid; j < nb; j += kFHeadThreads) {
    const float p = pk[j] / se, qq = pv[j];
    const float m = (p + qq) / 2.f;
    t1 += p * logf(p / m);
    t2 += qq * logf(qq / m);
  }
  t1 = block_sum_f(t1, red);
  t2 = block_sum_f(t2, red);
  const float js = sqrtf(0.5f * t1 + 0.5f * t2);
  const bool sparse = js < a.tau;
  if (sparse) nv = ns = a.min_b;
  if (tid == 0) {
    pv[0] = INFINITY;
    ps[nb - 1] = INFINITY;
  }
  __syncthreads();
  topk_bits(pv, nb, min(nv, nb), a.vmask + (int64_t)h * kFWords, &cs, scan);
  // slash: top ns pooled entries j -> offsets nb - 1 - j
  __shared__ uint64_t sb[kFWords];
  topk_bits(ps, nb, min(ns, nb), sb, &cs, scan);
  // word w of the offsets: bit b is offset 64 w + b = entry x - b, x = nb - 1 - 64 w,
  // so the word is entries x - 63 .. x reversed (entries below 0 read as 0)
  for (int w = tid; w < kFWords; w += kFHeadThreads) {
    const int x = nb - 1 - 64 * w;
    uint64_t word = 0;
    if (x >= 0) {
      const int lo = x - 63, q = lo >> 6, sh = lo & 63;   // q = floor(lo / 64)
      const uint64_t w0 = q >= 0 ? sb[q] : 0ull;
      const uint64_t w1 = q + 1 < kFWords ? sb[q + 1] : 0ull;
      word = __builtin_bitreverse64(sh ? (w0 >> sh) | (w1 << (64 - sh)) : w0);
    }
    a.smask[(int64_t)h * kFWords + w] = word;
  }
  if (tid == 0) {
    a.info[h * 4 + 0] = nv;
    a.info[h * 4 + 1] = ns;
    a.info[h * 4 + 2] = sparse ? 1 : 0;
    a.info[h * 4 + 3] = 0;
    a.js[h] = js;
  }
}

struct FlexCoverK {
  const uint16_t* q;
  int64_t q_sh, q_sl;
  const uint16_t* avg_k;        // [Hk][nb][D]
  const int32_t* info;          // [Hq][4]
  float* attn;                  // [Hq][nb][nb] work (sparse heads)
  uint64_t* cover;              // [Hq][nb][kFWords]
  int Hq, Hk, L, bs, nb, gqa_interleave;
  float sqrt_d, gamma;
};

// block-level causal attention rows of a sparse head: one workgroup per (head,
// kCoverRows consecutive block rows).  The K block means are staged in LDS 256
// rows at a time (row stride 260 bytes: thread t reads row t, bank (t + d / 2)
// % 64, conflict-free) and each staged row serves all the workgroup's query
// rows.  Per row, as one row per workgroup would: the score of key block j is
// the fp32 sum over d in order, rounded to T; thread t takes the blocks j = t,
// t + 256, ... (its exponential sums in that order), the maxima and sums are
// reduced by the same tree, and the scores and their exponentials pass
// through the row's place in attn.
constexpr int kCoverRows = 8;
constexpr int kCoverStride = kFD + 2;            // staged row: 130 bf16 = 260 bytes
template <typename T>
__global__ __launch_bounds__(kFThreads) void flex_cover_rows_kernel(FlexCoverK a) {
  __shared__ float aq[kCoverRows][kFD];
  __shared__ __attribute__((aligned(16))) uint16_t kst[kFThreads * kCoverStride];
  __shared__ float red[kFThreads];
  // a head's workgroups in order of decreasing row (the longest rows start
  // first); consecutive workgroups (one head's) fall on different XCDs
  const int ngr = (a.nb + kCoverRows - 1) / kCoverRows;
  const int h = blockIdx.x / ngr, i0 = (ngr - 1 - (int)(blockIdx.x % ngr)) * kCoverRows;
  if (a.info[h * 4 + 2] == 0) return;              // not a sparse head
  const int tid = threadIdx.x, bs = a.bs, nb = a.nb, L = a.L;
  const int nr = min(kCoverRows, nb - i0);         // rows of this workgroup
  const int kvh = kv_head(h, a.Hq, a.Hk, a.gqa_interleave);
  const int pad = nb * bs - L;
  // block means of q over bs rows (zero padded), in T; the last block rescaled
  // as (mean * bs) / (bs - pad), each step rounded to T.  Thread t forms the
  // means of dim t % 128 for rows t / 128, t / 128 + 2, ...; the loads of 8
  // tokens of every such row are issued before they are added (in token order).
  {
    constexpr int kPer = kCoverRows * kFD / kFThreads;   // (row, dim) pairs per thread
    const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
    const int d = tid % kFD, rr0 = tid / kFD;
    float sum[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) sum[u] = 0.f;
    for (int r0 = 0; r0 < bs; r0 += 8) {
      float x[kPer][8];
#pragma unroll
      for (int u = 0; u < kPer; ++u)
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int i = i0 + rr0 + 2 * u, t = i * bs + r0 + r;
          x[u][r] = (rr0 + 2 * u < nr && t < L) ? to_f32(T{qh[(int64_t)t * a.q_sl + d]}) : 0.f;
        }
#pragma unroll
      for (int u = 0; u < kPer; ++u)
#pragma unroll
        for (int r = 0; r < 8; ++r) sum[u] += x[u][r];
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int rr = rr0 + 2 * u, i = i0 + rr;
      if (rr >= nr) continue;
      float m = Conv<T>::round(sum[u] / (float)bs);
      if (pad && i == nb - 1) m = Conv<T>::round(Conv<T>::round(m * (float)bs) / (float)(bs - pad));
      aq[rr][d] = Conv<T>::round(m / a.sqrt_d);
    }
  }
  const int last = i0 + nr - 1;                    // the workgroup's last row: keys 0 .. last
  float mx[kCoverRows];
#pragma unroll
  for (int rr = 0; rr < kCoverRows; ++rr) mx[rr] = -INFINITY;
  float* rows = a.attn + ((int64_t)h * nb + i0) * nb;
  const uint16_t* kbase = a.avg_k + (int64_t)kvh * nb * kFD;
  for (int j0 = 0; j0 <= last; j0 += kFThreads) {
    __syncthreads();                               // aq written / the previous tile consumed
    // stage rows j0 .. j0 + 255 (16-byte global loads, 4-byte LDS writes)
    for (int c = tid; c < kFThreads * (kFD / 8); c += kFThreads) {
      const int r = c / (kFD / 8), cc = c - r * (kFD / 8);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (j0 + r <= last) v = *reinterpret_cast<const uint4*>(kbase + (int64_t)(j0 + r) * kFD + cc * 8);
      uint32_t* dst = reinterpret_cast<uint32_t*>(kst + r * kCoverStride + cc * 8);
      dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
    __syncthreads();
    const int j = j0 + tid;
    if (j <= last) {
      float acc[kCoverRows];
#pragma unroll
      for (int rr = 0; rr < kCoverRows; ++rr) acc[rr] = 0.f;
      const uint32_t* kr = reinterpret_cast<const uint32_t*>(kst + tid * kCoverStride);
      for (int d2 = 0; d2 < kFD / 2; ++d2) {
        const uint32_t w = kr[d2];
        const float k0 = to_f32(T{(uint16_t)(w & 0xffffu)}), k1 = to_f32(T{(uint16_t)(w >> 16)});
#pragma unroll
        for (int rr = 0; rr < kCoverRows; ++rr) {
          acc[rr] += aq[rr][2 * d2] * k0;
          acc[rr] += aq[rr][2 * d2 + 1] * k1;
        }
      }
#pragma unroll
      for (int rr = 0; rr < kCoverRows; ++rr) {
        if (rr < nr && j <= i0 + rr) {
          const float v = Conv<T>::round(acc[rr]);
          rows[(int64_t)rr * nb + j] = v;
          mx[rr] = fmaxf(mx[rr], v);
        }
      }
    }
  }
  for (int rr = 0; rr < nr; ++rr) {
    const int i = i0 + rr;
    float* out = rows + (int64_t)rr * nb;
    red[tid] = mx[rr];
    __syncthreads();
    for (int s = kFThreads / 2; s > 0; s >>= 1) {
      if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
      __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    float se = 0.f;
    for (int j = tid; j <= i; j += kFThreads) {
      const float e = expf(out[j] - m);
      out[j] = e;
      se += e;
    }
    red[tid] = se;
    __syncthreads();
    for (int s = kFThreads / 2; s > 0; s >>= 1) {
      if (tid < s) red[tid] += red[tid + s];
      __syncthreads();
    }
    se = red[0];
    __syncthreads();
    for (int j = tid; j < nb; j += kFThreads) out[j] = j <= i ? out[j] / se : 0.f;
  }
}

// the cover of gamma * N over a sparse head's N x N probabilities
// (score_cover_idx) from its finished cut: one launch over (head, slice)
// workgroups, one ballot per 64-entry word; when the cut splits the entries
// equal to its boundary value, the head's first workgroup writes every word,
// ranking those entries in flat index order
// the words of slice sl of a head's cover: a contiguous range, in index order
__device__ __forceinline__ void cover_slice_words(int nb, int slices, int sl, int* wb, int* we) {
  const int nwords = nb * ((nb + 63) >> 6);
  const int per = (nwords + slices - 1) / slices;
  *wb = min(nwords, sl * per);
  *we = min(nwords, *wb + per);
}

// when a sparse head's cut splits the entries equal to its boundary value:
// their number in each slice's words (ties [Hq][slices])
__global__ __launch_bounds__(kFHeadThreads) void flex_cover_ties_kernel(FlexCoverK a, CutJobs c, int* ties) {
  __shared__ CutState st;
  __shared__ int wsum[kFHeadThreads / 64];
  const int h = blockIdx.x / c.slices, sl = blockIdx.x - h * c.slices;
  if (!job_live(c, h)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nb = a.nb;
  cut_replay(c, h, 4, &st);
  const CutResult cut = cut_result(c, st);
  if (!(cut.take_eq > 0 && cut.take_eq < cut.eq_total)) return;
  const float* x = a.attn + (int64_t)h * nb * nb;
  const int wpr = (nb + 63) >> 6;
  int wb, we;
  cover_slice_words(nb, c.slices, sl, &wb, &we);
  int cnt = 0;
  for (int w = wb + wave; w < we; w += kFHeadThreads / 64) {
    const int r = w / wpr, col = (w - r * wpr) * 64 + lane;
    const bool eq = col < nb && order_key(x[(int64_t)r * nb + col]) == cut.key;
    cnt += __popcll(__ballot(eq));
  }
  if (lane == 0) wsum[wave] = cnt;
  __syncthreads();
  if (tid == 0) {
    int t = 0;
    for (int v = 0; v < kFHeadThreads / 64; ++v) t += wsum[v];
    ties[h * c.slices + sl] = t;
  }
}

__global__ __launch_bounds__(kFHeadThreads) void flex_cover_emit_kernel(FlexCoverK a, CutJobs c, const int* ties) {
  __shared__ CutState st;
  __shared__ int scan[kFHeadThreads];
  const int h = blockIdx.x / c.slices, sl = blockIdx.x - h * c.slices;
  if (!job_live(c, h)) return;
  const int tid = threadIdx.x, lane = tid & 63, nb = a.nb;
  cut_replay(c, h, 4, &st);
  const CutResult cut = cut_result(c, st);
  const float* x = a.attn + (int64_t)h * nb * nb;
  uint64_t* cov = a.cover + (int64_t)h * nb * kFWords;
  if (cut.take_eq > 0 && cut.take_eq < cut.eq_total) {
    // ties ranked in flat index order: this slice's words, after the earlier slices' ties
    int base = 0;
    for (int v = 0; v < sl; ++v) base += ties[h * c.slices + v];
    int wb, we;
    cover_slice_words(nb, c.slices, sl, &wb, &we);
    emit_cut(x, nb, nb, cut, cov, scan, wb, we, base);
  } else {
    const int wpr = (nb + 63) >> 6, nwords = nb * wpr;
    const int step = c.slices * (kFHeadThreads / 64);
    for (int w = sl * (kFHeadThreads / 64) + (tid >> 6); w < nwords; w += step) {
      const int r = w / wpr, col = (w - r * wpr) * 64 + lane;
      bool in = false;
      if (col < nb) {
        const uint32_t k = order_key(x[(int64_t)r * nb + col]);
        in = k > cut.key || (k == cut.key && cut.take_eq > 0);
      }
      const uint64_t word = __ballot(in);
      if (lane == 0) cov[(int64_t)r * kFWords + (w - r * wpr)] = word;
    }
  }
  __syncthreads();
  if (sl == 0 && tid == 0) atomicOr(reinterpret_cast<unsigned long long*>(&cov[0]), 1ull);   // entry 0 (the padding value)
}

struct FlexListK {
  const uint64_t* vmask;
  const uint64_t* smask;
  const uint64_t* cover;        // [Hq][nb][kFWords] (rows of sparse heads)
  const int32_t* info;
  int32_t* blk_cnt;
  uint64_t* blk_bits;           // [Hq][nb][ceil(nb / 64)]
  int Hq, nb;
};

// one wave per (head, block row): lane l forms the row's 64-bit membership
// words l and l + 64 and stores them; the row's count is their popcount sum
__global__ __launch_bounds__(64) void flex_lists_kernel(FlexListK a) {
  const int h = blockIdx.x / a.nb, r = blockIdx.x % a.nb;
  const int lane = threadIdx.x, nb = a.nb;
  const int NW = (nb + 63) >> 6;
  const uint64_t* vm = a.vmask + (int64_t)h * kFWords;
  const uint64_t* sm = a.smask + (int64_t)h * kFWords;
  const bool sparse = a.info[h * 4 + 2] != 0;
  auto word = [&](int w) -> uint64_t {
    if (w >= NW) return 0ull;
    // vertical columns v <= r
    uint64_t m = vm[w];
    // slash: column c = r - s for offset s; bit b of word w is c = 64 w + b,
    // s = t - b with t = r - 64 w, so the word is the offset mask's bits
    // t - 63 .. t reversed (offsets below 0 read as 0: columns past r)
    const int t = r - 64 * w;
    if (t < 0) return 0ull;                        // every column of the word is past r
    const int lo = t - 63, q = lo >> 6, sh = lo & 63;   // q = floor(lo / 64)
    const uint64_t w0 = q >= 0 ? sm[q] : 0ull;
    const uint64_t w1 = q + 1 < kFWords ? sm[q + 1] : 0ull;
    const uint64_t win = sh ? (w0 >> sh) | (w1 << (64 - sh)) : w0;   // bit k: offset lo + k
    m |= __builtin_bitreverse64(win);
    if (sparse) m |= a.cover[((int64_t)h * nb + r) * kFWords + w];
    if (t < 63) m &= (1ull << (t + 1)) - 1;        // causal: columns <= r
    return m;
  };
  const uint64_t m0 = word(lane), m1 = word(lane + 64);
  uint64_t* out = a.blk_bits + ((int64_t)h * nb + r) * NW;
  if (lane < NW) out[lane] = m0;
  if (lane + 64 < NW) out[lane + 64] = m1;
  const int total = wave_sum_i(__popcll(m0) + __popcll(m1));
  if (lane == 0) a.blk_cnt[(int64_t)h * nb + r] = total;
}

struct FlexLayout {
  size_t part, vert, slash, avgk, vmask, smask, info, attn, cover, p_hm, p_hc, c_hm, c_hc, ties, total;
};

// sparse: whether any head can take the block-level cover (tau > 0; the
// square-root JS divergence is >= 0, or nan, so js < tau never holds otherwise)
static FlexLayout flex_work(int Hq, int Hk, int L, int bs, bool sparse) {
  const int nb = (L + bs - 1) / bs;
  const int nchunk = (L + kFChunk - 1) / kFChunk;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) & ~(size_t)255;
    return at;
  };
  FlexLayout w;
  w.part = take((size_t)Hq * nchunk * bs * 2 * sizeof(float));
  w.vert = take((size_t)Hq * L * sizeof(float));
  w.slash = take((size_t)Hq * L * sizeof(float));
  w.avgk = take((size_t)Hk * nb * kFD * sizeof(uint16_t));
  w.vmask = take((size_t)Hq * kFWords * sizeof(uint64_t));
  w.smask = take((size_t)Hq * kFWords * sizeof(uint64_t));
  w.info = take((size_t)Hq * 4 * sizeof(int32_t) + (size_t)Hq * sizeof(float));
  w.attn = take(sparse ? (size_t)Hq * nb * nb * sizeof(float) : 0);
  w.cover = take(sparse ? (size_t)Hq * nb * kFWords * sizeof(uint64_t) : 0);
  w.p_hm = take((size_t)4 * 2 * Hq * 256 * sizeof(uint64_t));
  w.p_hc = take((size_t)4 * 2 * Hq * 256 * sizeof(uint32_t));
  w.c_hm = take((size_t)4 * Hq * 256 * sizeof(uint64_t));
  w.c_hc = take((size_t)4 * Hq * 256 * sizeof(uint32_t));
  w.ties = take((size_t)Hq * 256 * sizeof(int));     // [Hq][cover slices <= 256]
  w.total = off;
  return w;
}

template <typename T, int BS>
static int launch_lastq(const FlexK& k, unsigned grid, size_t smem1, size_t smem2, hipStream_t s) {
  if (int rc = fs_host::allow_dynamic_lds(flex_lastq_kernel<T, 1, BS>, smem1, "fs_flex")) return rc;
  if (int rc = fs_host::allow_dynamic_lds(flex_lastq_kernel<T, 2, BS>, smem2, "fs_flex")) return rc;
  flex_lastq_kernel<T, 1, BS><<<grid, kFThreads, smem1, s>>>(k);
  flex_lastq_kernel<T, 2, BS><<<grid, kFThreads, smem2, s>>>(k);
  return 0;
}

static void launch_cut_passes(const CutJobs& c, hipStream_t s) {
  const unsigned grid = (unsigned)(c.jobs * c.slices);
  cut_pass_kernel<0><<<grid, kCutSliceThreads, 0, s>>>(c);
  cut_pass_kernel<1><<<grid, kCutSliceThreads, 0, s>>>(c);
  cut_pass_kernel<2><<<grid, kCutSliceThreads, 0, s>>>(c);
  cut_pass_kernel<3><<<grid, kCutSliceThreads, 0, s>>>(c);
}

template <typename T>
static int launch_flex(const fs_flex_args& a, hipStream_t s) {
  const int nb = (a.L + a.bs - 1) / a.bs;
  const int nchunk = (a.L + kFChunk - 1) / kFChunk;
  const bool sparse = a.tau > 0.f;
  const FlexLayout lay = flex_work(a.Hq, a.Hk, a.L, a.bs, sparse);
  char* w = static_cast<char*>(a.work);
  FlexK k{};
  k.q = static_cast<const uint16_t*>(a.q);
  k.k = static_cast<const uint16_t*>(a.k);
  k.q_sh = a.q_sh; k.q_sl = a.q_sl; k.k_sh = a.k_sh; k.k_sl = a.k_sl;
  k.Hq = a.Hq; k.Hk = a.Hk; k.L = a.L; k.bs = a.bs; k.nb = nb; k.gqa_interleave = a.gqa_interleave;
  k.nchunk = nchunk;
  k.sqrt_d = (float)sqrt((double)a.D);
  k.part = reinterpret_cast<float*>(w + lay.part);
  k.vert = a.vertical ? a.vertical : reinterpret_cast<float*>(w + lay.vert);
  k.slash = a.slash ? a.slash : reinterpret_cast<float*>(w + lay.slash);
  k.p_hm = reinterpret_cast<uint64_t*>(w + lay.p_hm);
  k.p_hc = reinterpret_cast<uint32_t*>(w + lay.p_hc);
  k.c_hm = reinterpret_cast<uint64_t*>(w + lay.c_hm);
  k.c_hc = reinterpret_cast<uint32_t*>(w + lay.c_hc);
  const unsigned grid = (unsigned)(a.Hq * nchunk);
  const size_t smem1 = (size_t)kFTile * kFD * sizeof(uint16_t);
  const size_t smem2 = ((size_t)flex_tile_floats(a.bs) + kFTile + a.bs + (size_t)a.bs * 2 + kFThreads) * sizeof(float);
  if (int rc = a.bs == 16    ? launch_lastq<T, 16>(k, grid, smem1, smem2, s)
               : a.bs == 32 ? launch_lastq<T, 32>(k, grid, smem1, smem2, s)
               : a.bs == 64 ? launch_lastq<T, 64>(k, grid, smem1, smem2, s)
                            : launch_lastq<T, 128>(k, grid, smem1, smem2, s))
    return rc;
  uint16_t* avg_k = reinterpret_cast<uint16_t*>(w + lay.avgk);
  flex_kpool_kernel<T><<<(unsigned)(a.Hk * nb), kFThreads, 0, s>>>(k.k, a.k_sh, a.k_sl, a.L, a.bs, nb, avg_k);
  if (int rc = fs_host::launch_status("fs_flex (scores)")) return rc;
  // the profiles' mass cuts at gamma (each profile adds to one: masses x 2^58)
  CutJobs pc{};
  pc.x0 = k.vert;
  pc.x1 = k.slash;
  pc.stride = a.L;
  pc.n = a.L;
  pc.kinds = 2;
  pc.jobs = 2 * a.Hq;
  pc.slices = std::max(1, std::min(64, (a.L + 8191) / 8192));
  pc.scale_exp = 58;
  pc.g = (double)a.gamma;
  pc.info = nullptr;
  pc.hm = k.p_hm;
  pc.hc = k.p_hc;
  launch_cut_passes(pc, s);
  FlexHeadK hk{};
  hk.q = k.q; hk.q_sh = a.q_sh; hk.q_sl = a.q_sl;
  hk.avg_k = avg_k; hk.vert = k.vert; hk.slash = k.slash;
  hk.Hq = a.Hq; hk.Hk = a.Hk; hk.L = a.L; hk.bs = a.bs; hk.nb = nb; hk.gqa_interleave = a.gqa_interleave;
  hk.min_b = a.min_blocks; hk.max_b = a.max_blocks;
  hk.sqrt_d = k.sqrt_d; hk.gamma = a.gamma; hk.tau = a.tau;
  hk.vmask = reinterpret_cast<uint64_t*>(w + lay.vmask);
  hk.smask = reinterpret_cast<uint64_t*>(w + lay.smask);
  hk.info = a.head_info ? a.head_info : reinterpret_cast<int32_t*>(w + lay.info);
  hk.js = a.head_js ? a.head_js : reinterpret_cast<float*>(w + lay.info + (size_t)a.Hq * 4 * sizeof(int32_t));
  hk.pcut = pc;
  const size_t smem_head = (size_t)3 * nb * sizeof(float);
  // the limit covers the kernel's static LDS as well
  const size_t static_head = sizeof(double) * kFHeadThreads + sizeof(float) * kFD + sizeof(CutScratch) +
                             sizeof(CutState) + sizeof(uint64_t) * kFWords;
  if (int rc = fs_host::allow_dynamic_lds(flex_head_kernel<T>, smem_head + static_head, "fs_flex")) return rc;
  flex_head_kernel<T><<<(unsigned)a.Hq, kFHeadThreads, smem_head, s>>>(hk);
  FlexCoverK ck{};
  ck.q = k.q; ck.q_sh = a.q_sh; ck.q_sl = a.q_sl; ck.avg_k = avg_k; ck.info = hk.info;
  ck.attn = reinterpret_cast<float*>(w + lay.attn);
  ck.cover = reinterpret_cast<uint64_t*>(w + lay.cover);
  ck.Hq = a.Hq; ck.Hk = a.Hk; ck.L = a.L; ck.bs = a.bs; ck.nb = nb; ck.gqa_interleave = a.gqa_interleave;
  ck.sqrt_d = k.sqrt_d; ck.gamma = a.gamma;
  if (sparse) flex_cover_rows_kernel<T><<<(unsigned)(a.Hq * ((nb + kCoverRows - 1) / kCoverRows)), kFThreads, 0, s>>>(ck);
  // the sparse heads' covers: mass cut at gamma N of N^2 entries (rows add to one,
  // total nb <= 2^12: masses x 2^(58 - ceil(log2 nb)))
  CutJobs cc{};
  cc.x0 = ck.attn;
  cc.x1 = nullptr;
  cc.stride = (int64_t)nb * nb;
  cc.n = nb * nb;
  cc.kinds = 1;
  cc.jobs = a.Hq;
  cc.slices = std::max(1, std::min(256, (nb * nb + 16383) / 16384));
  cc.scale_exp = 58;
  for (int t = 1; t < nb; t <<= 1) --cc.scale_exp;
  cc.g = (double)a.gamma * nb;
  cc.info = hk.info;
  cc.hm = k.c_hm;
  cc.hc = k.c_hc;
  if (sparse) {
    launch_cut_passes(cc, s);
    int* ties = reinterpret_cast<int*>(w + lay.ties);
    flex_cover_ties_kernel<<<(unsigned)(a.Hq * cc.slices), kFHeadThreads, 0, s>>>(ck, cc, ties);
    flex_cover_emit_kernel<<<(unsigned)(a.Hq * cc.slices), kFHeadThreads, 0, s>>>(ck, cc, ties);
  }
  if (int rc = fs_host::launch_status("fs_flex (heads)")) return rc;
  FlexListK lk{};
  lk.vmask = hk.vmask; lk.smask = hk.smask; lk.cover = ck.cover; lk.info = hk.info;
  lk.blk_cnt = a.blk_cnt; lk.blk_bits = a.blk_bits; lk.Hq = a.Hq; lk.nb = nb;
  flex_lists_kernel<<<(unsigned)(a.Hq * nb), 64, 0, s>>>(lk);
  return fs_host::launch_status("fs_flex (lists)");
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_flex_work_bytes(int Hq, int Hk, int L, int bs, float tau) {
  if (Hq <= 0 || Hk <= 0 || L <= 0 || bs <= 0) return 0;
  return flex_work(Hq, Hk, L, bs, tau > 0.f).total;
}

extern "C" int fs_flex(const fs_flex_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_flex: null args");
  FS_CHECK_ARG(a->q && a->k && a->blk_cnt && a->blk_bits && a->work, "fs_flex: null pointer");
  FS_CHECK_ARG(((uintptr_t)a->blk_bits & 7) == 0, "fs_flex: blk_bits must be 8-byte aligned");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "fs_flex: Hq=%d must be a multiple of Hk=%d", a->Hq,
               a->Hk);
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16, "fs_flex: dtype %d unsupported (bf16/f16)",
                     a->dtype);
  FS_CHECK_SUPPORTED(a->D == kFD, "fs_flex: head_dim %d unsupported (128 only)", a->D);
  FS_CHECK_SUPPORTED(a->bs == 16 || a->bs == 32 || a->bs == 64 || a->bs == 128,
                     "fs_flex: block size %d unsupported (16, 32, 64, 128)", a->bs);
  FS_CHECK_ARG(a->L > a->bs, "fs_flex: the sequence must be longer than one block");
  FS_CHECK_ARG(a->min_blocks >= 1 && a->max_blocks >= 1, "fs_flex: bad budgets");
  FS_CHECK_ARG(((uintptr_t)a->q % 16) == 0 && ((uintptr_t)a->k % 16) == 0 && a->q_sl % 8 == 0 && a->k_sl % 8 == 0 &&
                   a->q_sh % 8 == 0 && a->k_sh % 8 == 0,
               "fs_flex: q/k must be 16-byte aligned with strides of whole 16-byte chunks");
  const int nb = (a->L + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED(nb <= kFMaxBlocks, "fs_flex: %d blocks > %d", nb, kFMaxBlocks);
  hipStream_t s = (hipStream_t)stream;
  return a->dtype == FS_DTYPE_BF16 ? launch_flex<bf16_t>(*a, s) : launch_flex<f16_t>(*a, s);
}
