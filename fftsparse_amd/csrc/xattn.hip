// XAttention block selection on gfx950 -- the reference's other selector
// (attn_src/xattn/src/Xattention.py:14-303 xattn_estimate + :306-406
// Xattention_prefill; its Triton kernels attn_src/xattn/src/kernels.py:5-97 and
// :195-234; attn_src/xattn/src/utils.py:44-200 find_blocks_chunked), feeding
// the same block-sparse attention kernel as the FFT selector.
//
// Reshaped scores (stride S, "inverse" mode): for reshaped query row r and key
// n,  A[r][n] = sum_{j<S} q[rS + S-1-j] . k[nS + j]  -- a GEMM with an S*D
// reduction whose operands are S token rows each; the fp32 result is rounded
// to the input dtype, as the reference's kernel stores it.  Then, in the exp2
// domain, x = A * log2(e) / sqrt(D) / S / norm, each real row is normalised
// over its causal keys n <= r, and the probabilities are summed over
// (bs/S) x (bs/S) squares: the block sums, rounded to the input dtype.
//
// xattn_scores_kernel<T>: one workgroup (4 waves, 32 reshaped rows each) per
// (head, 128 reshaped rows), longest rows first; key tiles of 128 reshaped keys
// up to the diagonal.  For each tile and each j < S the workgroup copies the
// 128 query token rows rS + S-1-j and the 128 key token rows nS + j into LDS
// with global -> LDS copies (no register staging; rows past L zeroed after;
// 256-byte rows, 16-byte chunk c of row r at c ^ (r & 15)) and accumulates
// S^T = K' Q'^T with v_mfma_f32_32x32x16.  It keeps each row's
// running max and exp2 sum (the reference's first loop) and stores the scores,
// rounded to the input dtype, as the reference's GEMM kernel stores its
// output: the causal part only, row tile by row tile (tile rt holds its 128
// rows x 128 (rt + 1) keys, so it starts 16384 rt (rt + 1) / 2 values in).
// xattn_sums_kernel<T>: one workgroup per (head, 128 reshaped rows) streams
// the stored scores (threads along the keys, rows in order), forms
// p = exp2(x - max) / sum and adds it over each block's rows and, by xor
// shuffles, its keys (the reference's second loop).
//
// xattn_select_kernel: one workgroup per (head, block row I): the causal
// block sums of the row, the forced first and diagonal blocks, the others in
// decreasing order (ties: lower index first) by a bitonic sort in LDS, their
// exclusive prefix masses in fp64, and each other block kept iff
// forced mass + prefix < row total * threshold.  Output: ascending per-row
// block lists (the causal tril; keep_sink fills row 0, keep_recent the
// diagonal).
#include "common.h"

namespace fs {

constexpr int kXD = 128;          // head dim
constexpr int kXRows = 128;       // reshaped rows per workgroup: 4 waves x 32
constexpr int kXKeys = 128;       // reshaped keys per tile
constexpr int kXKK = kXKeys / 32; // 32-key MFMA sub-tiles per tile

// One 1 KiB global -> LDS copy per wave: lane l's 16 bytes, from the
// wave-uniform base plus the lane's byte offset, land at lds_base + 16 l.
__device__ __forceinline__ void xdma16(uint32_t lds_base, const void* sbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_base), "v"(voff), "s"(sbase) : "memory");
}
constexpr int kXThreads = 256;
constexpr int kXSelThreads = 256;
constexpr int kXMaxBlocks = 4096;

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <typename T> struct XMma;
template <> struct XMma<bf16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
};
template <> struct XMma<f16_t> {
  static __device__ __forceinline__ f32x16_t mma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
};

struct XScoreK {
  const uint16_t* q;
  const uint16_t* k;
  int64_t q_sh, q_sl, k_sh, k_sl;
  int Hq, Hk, L, S, Lr, real, rbs, Nb;
  float scale;                  // log2(e) / sqrt(D) / S / norm
  float* m;                     // [Hq][Lr] row max (exp2 domain)
  float* l;                     // [Hq][Lr] row sum
  float* sums;                  // [Hq][Nb][Nb] block sums (values of T), causal part
  uint16_t* scores;             // [Hq][head_stride] the rounded scores, causal row tiles
  int64_t head_stride;
};

// first stored score of row tile rt (every earlier tile is whole)
__host__ __device__ inline int64_t xtile_offset(int rt) { return (int64_t)kXRows * 128 * rt * (rt + 1) / 2; }
// keys stored per row of tile rt: its key tiles up to the diagonal
__host__ __device__ inline int xtile_keys(int rt, int Lr) {
  const int last_row = (rt + 1) * kXRows < Lr ? (rt + 1) * kXRows - 1 : Lr - 1;
  return (last_row / kXKeys + 1) * kXKeys;
}

template <typename T>
__global__ __launch_bounds__(kXThreads) void xattn_scores_kernel(XScoreK a) {
  __shared__ __attribute__((aligned(16))) uint16_t lq[kXRows * kXD];   // Q'_j rows, 32 KiB
  __shared__ __attribute__((aligned(16))) uint16_t lk[kXKeys * kXD];   // K'_j rows
  const int nrt = (a.Lr + kXRows - 1) / kXRows;
  const int rt = nrt - 1 - (int)(blockIdx.x / a.Hq);                 // longest rows first
  const int h = (int)(blockIdx.x % a.Hq);
  const int hk = h / (a.Hq / a.Hk);
  const int r0 = rt * kXRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hi = lane >> 5;
  const int row = r0 + wave * 32 + l32;            // this lane's reshaped row (column of S^T)
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)hk * a.k_sh;
  const int S = a.S;
  const int last_row = min(a.Lr, r0 + kXRows) - 1;
  const int nct = last_row / kXKeys + 1;           // key tiles up to the diagonal
  const bool row_ok = row < a.Lr;

  float m_run = -INFINITY, l_run = 0.f;

  for (int ct = 0; ct < nct; ++ct) {
    const int n0 = ct * kXKeys;
    f32x16_t acc[kXKK];
#pragma unroll
    for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[kk][r] = 0.f;
    for (int j = 0; j < S; ++j) {
      __syncthreads();                             // previous stage consumed
      // 1 KiB regions of 4 LDS rows: lane l fills slot l % 16 of row 4R + l / 16
      // with the token row's chunk (l % 16) ^ (row & 15); rows past L read row
      // L-1 here and are zeroed below
      const uint32_t lq0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lq);
      const uint32_t lk0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lk);
      const int wv = __builtin_amdgcn_readfirstlane(wave);   // wave-uniform: the copies' LDS bases
      constexpr int QR = kXRows / 4 / 4, KR = kXKeys / 4 / 4;   // regions per wave
#pragma unroll
      for (int i = 0; i < QR; ++i) {
        const int R = wv * QR + i, rr = 4 * R + (lane >> 4), c = (lane & 15) ^ (rr & 15);
        const int t = min((r0 + rr) * S + S - 1 - j, a.L - 1);
        xdma16(lq0 + R * 1024, qh, (uint32_t)(t * a.q_sl + c * 8) * 2u);
      }
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        const int R = wv * KR + i, cr = 4 * R + (lane >> 4), c = (lane & 15) ^ (cr & 15);
        const int t = min((n0 + cr) * S + j, a.L - 1);
        xdma16(lk0 + R * 1024, kh, (uint32_t)(t * a.k_sl + c * 8) * 2u);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if ((r0 + kXRows - 1) * S + S - 1 - j >= a.L || (n0 + kXKeys - 1) * S + j >= a.L) {
        // this stage reaches past L: those rows are zero
        for (int e = tid; e < (kXRows + kXKeys) * 16; e += kXThreads) {
          const int r = e >> 4, ch = e & 15;
          if (r < kXRows) {
            if ((r0 + r) * S + S - 1 - j >= a.L) *reinterpret_cast<uint4*>(lq + r * kXD + ch * 8) = make_uint4(0, 0, 0, 0);
          } else {
            const int cr = r - kXRows;
            if ((n0 + cr) * S + j >= a.L) *reinterpret_cast<uint4*>(lk + cr * kXD + ch * 8) = make_uint4(0, 0, 0, 0);
          }
        }
        __syncthreads();
      }

      const int qr = wave * 32 + l32;
#pragma unroll
      for (int st = 0; st < kXD / 16; ++st) {
        const uint4 bq = *reinterpret_cast<const uint4*>(lq + qr * kXD + (((2 * st + hi) ^ (qr & 15)) << 3));
#pragma unroll
        for (int kk = 0; kk < kXKK; ++kk) {
          const int kr = kk * 32 + l32;
          const uint4 ak = *reinterpret_cast<const uint4*>(lk + kr * kXD + (((2 * st + hi) ^ (kr & 15)) << 3));
          acc[kk] = XMma<T>::mma(ak, bq, acc[kk]);
        }
      }
    }

    // ---- epilogue: lane holds keys n0 + 32 kk + (r/4) 8 + hi 4 + r%4 of its row
    // a key of this lane's row is causal; its score in the exp2 domain, from the
    // accumulator (recomputed where used, so no tile-sized arrays stay live)
    auto valid = [&](int kk, int r) { return row_ok && n0 + kk * 32 + (r >> 2) * 8 + hi * 4 + (r & 3) <= row; };
    auto xval = [&](int kk, int r) { return Conv<T>::round(acc[kk][r]) * a.scale; };
    if (row_ok) {
      // the rounded scores of this lane's row: four consecutive keys per 8-byte store
      const int NK = xtile_keys(rt, a.Lr);
      uint16_t* dst = a.scores + (int64_t)h * a.head_stride + xtile_offset(rt) + (int64_t)(row - r0) * NK;
#pragma unroll
      for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t w[2];
#pragma unroll
          for (int e = 0; e < 2; ++e)
            w[e] = (uint32_t)__builtin_bit_cast(uint16_t, Conv<T>::store(acc[kk][g * 4 + 2 * e])) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, Conv<T>::store(acc[kk][g * 4 + 2 * e + 1])) << 16);
          *reinterpret_cast<uint2*>(dst + n0 + kk * 32 + g * 8 + hi * 4) = make_uint2(w[0], w[1]);
        }
    }
    {
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (valid(kk, r)) mx = fmaxf(mx, xval(kk, r));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));      // the row's other keys sit in lane ^ 32
      const float m_new = fmaxf(m_run, mx);
      if (m_new > -INFINITY) {
        float s = 0.f;
#pragma unroll
        for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (valid(kk, r)) s += __builtin_amdgcn_exp2f(xval(kk, r) - m_new);
        l_run = l_run * __builtin_amdgcn_exp2f(m_run - m_new) + s;
        m_run = m_new;
      }
    }
  }
  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  if (row_ok && hi == 0) {
    a.m[(int64_t)h * a.Lr + row] = m_run;
    a.l[(int64_t)h * a.Lr + row] = lt;
  }
}

// pass 2 over the stored scores
template <typename T>
__global__ __launch_bounds__(kXThreads) void xattn_sums_kernel(XScoreK a) {
  __shared__ float rm[kXRows], rinv[kXRows];
  const int nrt = (a.Lr + kXRows - 1) / kXRows;
  const int rt = nrt - 1 - (int)(blockIdx.x / a.Hq);
  const int h = (int)(blockIdx.x % a.Hq);
  const int r0 = rt * kXRows;
  const int nr = min(a.Lr, r0 + kXRows) - r0;       // a multiple of rbs
  const int NK = xtile_keys(rt, a.Lr);
  const int tid = threadIdx.x, rbs = a.rbs;
  if (tid < kXRows) {
    const int row = r0 + tid;
    const bool real = row < a.real;                  // padding rows add nothing
    rm[tid] = row < a.Lr ? a.m[(int64_t)h * a.Lr + row] : 0.f;
    rinv[tid] = real ? 1.0f / a.l[(int64_t)h * a.Lr + row] : 0.f;
  }
  __syncthreads();
  const uint16_t* src = a.scores + (int64_t)h * a.head_stride + xtile_offset(rt);
  // eight consecutive keys per thread (one 16-byte load a row): a key block of
  // rbs >= 8 keys spans rbs / 8 neighbouring lanes
  const int gl = rbs / 8;
  for (int c0 = 0; c0 < NK; c0 += 8 * kXThreads) {
    const int n = c0 + 8 * tid;
    const bool key_ok = n < NK;                      // NK and n are multiples of 8
    float acc = 0.f;
    for (int i = 0; i < nr; ++i) {
      const int row = r0 + i;
      if (key_ok && n <= row && rinv[i] > 0.f) {
        const uint4 w = *reinterpret_cast<const uint4*>(src + (int64_t)i * NK + n);
        const uint32_t pr[4] = {w.x, w.y, w.z, w.w};
        const float mi = rm[i], li = rinv[i];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint16_t e = (uint16_t)((t & 1) ? (pr[t >> 1] >> 16) : (pr[t >> 1] & 0xffffu));
          if (n + t <= row) acc += __builtin_amdgcn_exp2f(to_f32(T{e}) * a.scale - mi) * li;
        }
      }
      if ((i + 1) % rbs == 0) {                      // the end of a block row: add over the block's keys
        float v = acc;
        for (int o = 1; o < gl; o <<= 1) v += __shfl_xor(v, o, 64);
        const int I = row / rbs, J = n / rbs;
        if (key_ok && (tid % gl) == 0 && J <= I && I < a.Nb) a.sums[((int64_t)h * a.Nb + I) * a.Nb + J] = Conv<T>::round(v);
        acc = 0.f;
      }
    }
  }
}

struct XSelK {
  const float* sums;            // [Hq][Nb][Nb]
  const double* thr;            // [Hq]
  int32_t* blk_cnt;             // [Hq][N]
  uint16_t* blk_idx;            // [Hq][N][Nk]
  int Hq, Nb, N, Nk, keep_sink;
};

__global__ __launch_bounds__(kXSelThreads) void xattn_select_kernel(XSelK a) {
  __shared__ uint64_t key[kXMaxBlocks];             // (~value bits) << 32 | index: ascending = value desc, index asc
  __shared__ double part[kXSelThreads];
  __shared__ uint8_t sel[kXMaxBlocks];
  const int h = (int)(blockIdx.x / a.N), I = (int)(blockIdx.x % a.N);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* row = a.sums + ((int64_t)h * a.Nb + I) * a.Nb;
  const int n = I + 1;                              // causal blocks of the row
  int P = 1;
  while (P < n) P <<= 1;

  // keys (the forced blocks enter the sorted list as zeros, as the
  // reference's masked_fill does) and the row total in a fixed order
  double tot = 0.0;
  for (int J = tid; J < P; J += kXSelThreads) {
    uint64_t kk = ~0ull;
    if (J < n) {
      const float v = row[J];
      tot += (double)v;
      const float vo = (J == 0 || J == I) ? 0.f : v;
      kk = ((uint64_t)(~__float_as_uint(vo)) << 32) | (uint32_t)J;
    }
    key[J] = kk;
    sel[J] = 0;
  }
  part[tid] = tot;
  __syncthreads();
  for (int s = kXSelThreads / 2; s > 0; s >>= 1) {
    if (tid < s) part[tid] += part[tid + s];
    __syncthreads();
  }
  const double total = part[0];
  const double forced = (double)row[0] + (I > 0 ? (double)row[I] : 0.0);
  const double required = total * a.thr[h];
  __syncthreads();

  // bitonic sort of key[0 .. P) ascending
  for (int k2 = 2; k2 <= P; k2 <<= 1) {
    for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
      for (int i = tid; i < P; i += kXSelThreads) {
        const int ixj = i ^ j2;
        if (ixj > i) {
          const uint64_t x = key[i], y = key[ixj];
          const bool up = (i & k2) == 0;
          if ((x > y) == up) {
            key[i] = y;
            key[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }

  // exclusive prefix masses of the sorted values: thread t owns positions
  // [t * per, (t + 1) * per), its run summed in order, then a fixed-order scan
  const int per = (P + kXSelThreads - 1) / kXSelThreads;
  const int p0 = tid * per;
  auto value_at = [&](int p) -> double {
    const uint64_t kk = key[p];
    if ((uint32_t)kk >= (uint32_t)n) return 0.0;   // padding
    return (double)__uint_as_float(~(uint32_t)(kk >> 32));
  };
  double run = 0.0;
  for (int p = p0; p < min(P, p0 + per); ++p) run += value_at(p);
  part[tid] = run;
  __syncthreads();
  for (int off = 1; off < kXSelThreads; off <<= 1) {  // inclusive scan (Hillis-Steele, fixed order)
    const double v = tid >= off ? part[tid - off] : 0.0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  double before = forced + (part[tid] - run);
  for (int p = p0; p < min(P, p0 + per); ++p) {
    const uint32_t J = (uint32_t)key[p];
    if (J < (uint32_t)n && before < required) sel[J] = 1;
    before += value_at(p);
  }
  __syncthreads();

  // ascending list: forced blocks, chosen blocks, the causal tril; keep_sink fills row 0
  if (wave == 0) {
    const int limit = (I == 0 && a.keep_sink) ? a.Nk : n;
    uint16_t* out = a.blk_idx + ((int64_t)h * a.N + I) * a.Nk;
    int cnt = 0;
    for (int J0 = 0; J0 < limit; J0 += 64) {
      const int J = J0 + lane;
      bool in = false;
      if (J < limit) in = J >= n || J == 0 || J == I || sel[J];
      const uint64_t m = __ballot(in);
      if (in) out[cnt + rank_below(m)] = (uint16_t)J;
      cnt += __popcll(m);
    }
    if (lane == 0) a.blk_cnt[(int64_t)h * a.N + I] = cnt;
  }
}

// stored scores per head: every row tile's rows x keys up to its diagonal
static int64_t xattn_head_stride(int Lr) {
  const int nrt = (Lr + kXRows - 1) / kXRows;
  return xtile_offset(nrt - 1) + (int64_t)kXRows * xtile_keys(nrt - 1, Lr);
}

// workspace: row max and sum [Hq][Lr] each, then the stored scores
static size_t xattn_stats_bytes(int Hq, int Lr) { return ((size_t)Hq * Lr * 2 * sizeof(float) + 255) & ~(size_t)255; }

static size_t xattn_work(int Hq, int L, int stride, int bs) {
  const int64_t Lp = ((int64_t)L + bs - 1) / bs * bs;
  const int Lr = (int)(Lp / stride);
  return xattn_stats_bytes(Hq, Lr) + (size_t)Hq * xattn_head_stride(Lr) * sizeof(uint16_t);
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_xattn_work_bytes(int Hq, int L, int stride, int bs) {
  if (Hq <= 0 || L <= 0 || stride <= 0 || bs <= 0) return 0;
  return xattn_work(Hq, L, stride, bs);
}

extern "C" int fs_xattn(const fs_xattn_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_xattn: null args");
  FS_CHECK_ARG(a->q && a->k && a->threshold && a->sums && a->blk_cnt && a->blk_idx && a->work,
               "fs_xattn: null pointer");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->Hq % a->Hk == 0, "fs_xattn: Hq=%d must be a multiple of Hk=%d", a->Hq,
               a->Hk);
  FS_CHECK_ARG(a->L > 0, "fs_xattn: empty sequence");
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16, "fs_xattn: dtype %d unsupported (bf16/f16)",
                     a->dtype);
  FS_CHECK_SUPPORTED(a->D == kXD, "fs_xattn: head_dim %d unsupported (128 only)", a->D);
  // the reference asserts block_size == 128 (Xattention.py:360)
  FS_CHECK_SUPPORTED(a->bs == 128, "fs_xattn: block size %d unsupported (128 only)", a->bs);
  FS_CHECK_SUPPORTED(a->stride == 4 || a->stride == 8 || a->stride == 16, "fs_xattn: stride %d unsupported (4, 8, 16)",
                     a->stride);
  FS_CHECK_ARG(a->norm > 0.f, "fs_xattn: norm must be positive");
  FS_CHECK_ARG(((uintptr_t)a->q % 16) == 0 && ((uintptr_t)a->k % 16) == 0 && a->q_sl % 8 == 0 && a->k_sl % 8 == 0 &&
                   a->q_sh % 8 == 0 && a->k_sh % 8 == 0,
               "fs_xattn: q/k must be 16-byte aligned with strides of whole 16-byte chunks");
  const int N = (a->L + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED(N <= kXMaxBlocks, "fs_xattn: %d blocks > %d", N, kXMaxBlocks);
  // the tile copies address a token row by a 32-bit byte offset from the head's base
  FS_CHECK_SUPPORTED((int64_t)a->L * (a->q_sl > a->k_sl ? a->q_sl : a->k_sl) * 2 < ((int64_t)1 << 32),
                     "fs_xattn: sequence x row stride too large");
  XScoreK k{};
  k.q = static_cast<const uint16_t*>(a->q);
  k.k = static_cast<const uint16_t*>(a->k);
  k.q_sh = a->q_sh; k.q_sl = a->q_sl; k.k_sh = a->k_sh; k.k_sl = a->k_sl;
  k.Hq = a->Hq; k.Hk = a->Hk; k.L = a->L; k.S = a->stride;
  k.Lr = N * a->bs / a->stride;
  k.real = (a->L + a->stride - 1) / a->stride;
  k.rbs = a->bs / a->stride;
  k.Nb = N;
  k.scale = (float)(1.4426950408889634 / sqrt((double)a->D) / a->stride / a->norm);
  k.m = static_cast<float*>(a->work);
  k.l = k.m + (size_t)a->Hq * k.Lr;
  k.sums = a->sums;
  k.scores = reinterpret_cast<uint16_t*>(static_cast<char*>(a->work) + xattn_stats_bytes(a->Hq, k.Lr));
  k.head_stride = xattn_head_stride(k.Lr);
  const unsigned grid = (unsigned)(a->Hq * ((k.Lr + kXRows - 1) / kXRows));
  hipStream_t s = (hipStream_t)stream;
  if (a->dtype == FS_DTYPE_BF16) {
    xattn_scores_kernel<bf16_t><<<grid, kXThreads, 0, s>>>(k);
    xattn_sums_kernel<bf16_t><<<grid, kXThreads, 0, s>>>(k);
  } else {
    xattn_scores_kernel<f16_t><<<grid, kXThreads, 0, s>>>(k);
    xattn_sums_kernel<f16_t><<<grid, kXThreads, 0, s>>>(k);
  }
  if (int rc = fs_host::launch_status("fs_xattn (scores)")) return rc;
  XSelK sk{};
  sk.sums = a->sums;
  sk.thr = a->threshold;
  sk.blk_cnt = a->blk_cnt;
  sk.blk_idx = a->blk_idx;
  sk.Hq = a->Hq; sk.Nb = N; sk.N = N; sk.Nk = N; sk.keep_sink = a->keep_sink;
  xattn_select_kernel<<<(unsigned)(a->Hq * N), kXSelThreads, 0, s>>>(sk);
  return fs_host::launch_status("fs_xattn (select)");
}
