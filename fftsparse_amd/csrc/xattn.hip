// XAttention block selection on gfx950 -- the reference's other selector
// (attn_src/xattn/src/Xattention.py:14-303 xattn_estimate + :306-406
// Xattention_prefill; its Triton kernels attn_src/xattn/src/kernels.py:5-156 and
// :195-234; attn_src/xattn/src/utils.py:44-200 find_blocks_chunked), feeding
// the same block-sparse attention kernel as the FFT selector.
//
// Reshaped scores (stride S): for reshaped query row m and key n,
//   A[m][n] = sum_{j<S} q[m QS + o_j] . k'[nS + j]
// -- a GEMM with an S*D reduction whose operands are S token rows each; the
// fp32 result is rounded to the input dtype, as the reference's kernel (and
// its torch matmul) stores it.  The Triton path the callers use has o_j =
// S-1-j ("inverse"), QS = S and k' = k.  The torch path (use_triton=False)
// has o_j = S-1-j (inverse, double, triple), j (slash) or perm[j] (random),
// QS = S kdb for inverse (else S), and k' = k, or for double / triple the
// neighbouring-chunk sums of k rounded to dtype (xattn_kaug_kernel).
//
// Triton path: in the exp2 domain, x = A log2(e) / sqrt(D) / S / norm, each
// row is normalised over the keys it sees (causal: n <= m; non-causal: every
// key of the chunk-padded sequence) and the probabilities are summed over
// (bs/S) x (bs/S) squares: the block sums, rounded to the input dtype.
// Torch path: x = A / sqrt(D) / S / norm with each division rounded to dtype,
// causal rows m see keys n <= m kdb + kdb - 1 (the padding ones too), p is the
// float32 softmax (or exp) rounded to dtype, and the block sums are two sums
// rounded to dtype: over a block's keys, then over its rows.
//
// xattn_scores_wide_kernel<T, TP>: one workgroup (8 waves: 4 groups of 64
// reshaped rows x 2 groups of 128 keys) per (head, 256 reshaped rows), longest
// rows first; key tiles of 256 reshaped keys up to the last one the tile's rows
// see.  For each tile, each j < S and each 64-dim half, the workgroup copies
// the 256 query token rows and the 256 key token rows of that stage into LDS
// with global -> LDS copies (two buffers: the next stage's copies land while
// this stage's MFMAs run; rows past the sequence zeroed after; 128-byte rows,
// 16-byte chunk c of row r at c ^ (r & 7)) and accumulates S^T = K' Q'^T with
// v_mfma_f32_32x32x16.  It keeps each row's running max and exp sum (the
// reference's first loop), merged over the two key halves at the end, and
// stores the scores, rounded to the input dtype, in tiles of 128 rows (row
// tile rt holds its 128 rows x 128 nct(rt) keys).
// xattn_sums_kernel<T, TP>: one workgroup per (head, 128 reshaped rows)
// streams the stored scores (threads along the keys, rows in order), forms p
// and adds it over each block's rows and, by xor shuffles, its keys (the
// reference's second loop).  Non-causal: the keys of the chunk padding past
// the last block score 0; their mass per block row is formed in closed form.
//
// xattn_select_kernel: one workgroup per (head, block row I), in float64.
// Causal: the causal block sums of the row, the forced first and diagonal
// blocks, the others in decreasing order (ties: lower index first) by a
// bitonic sort in LDS, their exclusive prefix masses, and each other block
// kept iff forced mass + prefix < row total * threshold.  Non-causal: every
// block of the chunk-padded row sorted, none forced, and block 0 always kept.
// Output: ascending per-row block lists of the N real blocks (keep_sink fills
// row 0, keep_recent the diagonal).
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

// Rounding to the input dtype by the hardware conversion (round to nearest
// even, as the bit-level one in common.h for every finite value), without the
// per-element NaN branch: the score epilogue rounds 128 values per lane per tile.
template <typename T> struct XCvt;
template <> struct XCvt<bf16_t> {
  static __device__ __forceinline__ float round(float f) { return (float)(__bf16)f; }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
  }
};
template <> struct XCvt<f16_t> {
  static __device__ __forceinline__ float round(float f) { return (float)(_Float16)f; }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
  }
};

struct XScoreK {
  const uint16_t* q;
  const uint16_t* k;            // k, or the K' buffer (double / triple)
  int64_t q_sh, q_sl, k_sh, k_sl;
  int Hq, Hk, S, QS, Lq_tok, Lk_tok;
  uint64_t qorder;              // 4 bits per stage j: o_j
  int Lrq, Lrk, rbs, rpb, Nb;   // query rows, keys, keys per block, query rows per block, blocks
  int causal, kdb, own_chunk;
  int real_rows, npad, softmax;
  float scale;                  // Triton path: log2(e) / sqrt(D) / S / norm
  float inv_sqrt, inv_S, inv_norm;   // torch path: float32 reciprocals of the divisors
  float* m;                     // [nck][Hq][Lrq] row max of each key chunk (exp2 domain on the Triton path)
  float* l;                     // [nck][Hq][Lrq] row sum of each key chunk
  float* sums;                  // [Hq][Nb][Nb] block sums (values of T)
  float* pad_sum;               // [Hq][Nb] non-causal: the sum of every key block of the chunk padding
  uint16_t* scores;             // [hg][head_stride] the rounded scores of heads h0 .. h0+hg-1, row tiles
  int64_t head_stride;
  int h0, hg;                   // the heads of this launch
  int kc, items;                // key tiles (of 256) per score workgroup; workgroups per head
};

__host__ __device__ inline int ximin(int a, int b) { return a < b ? a : b; }
// key tiles of row tile rt: up to the last key its rows see
__host__ __device__ inline int xnct(int rt, int Lrq, int Lrk, int causal, int kdb) {
  const int last_row = ximin(Lrq, (rt + 1) * kXRows) - 1;
  int last_key = Lrk - 1;
  if (causal) last_key = ximin(last_key, last_row * kdb + kdb - 1);
  return last_key < 0 ? 1 : last_key / kXKeys + 1;
}
// 256-key tiles of the 256-row tile R of the score pass, and its key chunks of kc tiles
__host__ __device__ inline int xnct_wide(int R, int Lrq, int Lrk, int causal, int kdb) {
  const int last_row = ximin(Lrq, (R + 1) * 256) - 1;
  int last_key = Lrk - 1;
  if (causal) last_key = ximin(last_key, last_row * kdb + kdb - 1);
  return last_key < 0 ? 1 : last_key / 256 + 1;
}
__host__ __device__ inline int xchunks(int R, int Lrq, int Lrk, int causal, int kdb, int kc) {
  return (xnct_wide(R, Lrq, Lrk, causal, kdb) + kc - 1) / kc;
}
// first stored score of row tile rt (every earlier tile is whole)
__host__ __device__ inline int64_t xoffset(int rt, int Lrq, int Lrk, int causal, int kdb) {
  int64_t o = 0;
  for (int t = 0; t < rt; ++t) o += (int64_t)kXRows * kXKeys * xnct(t, Lrq, Lrk, causal, kdb);
  return o;
}

// whether row sees key (the keys past Lrk -- chunk padding -- are formed in
// closed form); the Triton path has kdb 1 and no own-chunk rule
template <bool TP>
__device__ __forceinline__ bool xkey_ok(const XScoreK& a, int row, int key) {
  if (key >= a.Lrk) return false;
  if (!a.causal) return true;
  if constexpr (!TP) return key <= row;
  if (key > row * a.kdb + a.kdb - 1) return false;
  return a.own_chunk == 0 || key >= (row * a.kdb / a.own_chunk) * a.own_chunk;
}
// the score in the softmax's domain from the fp32 accumulator (or a stored value)
template <typename T, bool TP>
__device__ __forceinline__ float xscaled(const XScoreK& a, float acc) {
  const float r = XCvt<T>::round(acc);
  if constexpr (!TP) return r * a.scale;
  return XCvt<T>::round(XCvt<T>::round(XCvt<T>::round(r * a.inv_sqrt) * a.inv_S) * a.inv_norm);
}
template <bool TP>
__device__ __forceinline__ float xexp(float x) {
  if constexpr (TP) return expf(x);
  return __builtin_amdgcn_exp2f(x);
}

// The score pass: one workgroup of 8 waves per (head, 256 reshaped rows), key
// tiles of 256 reshaped keys up to the last key the rows see.  Wave w computes rows 64 (w % 4) .. +63 against keys 128 (w / 4) .. +127
// of the tile (8 v_mfma_f32_32x32x16 tiles).  Each stage copies the 256 query
// token rows and the 256 key token rows of one token offset j, one 64-dim half
// at a time (128-byte LDS rows, chunk c of row r at c ^ (r & 7)), into one of
// two buffers, so a stage's copies land while the previous stage's MFMAs run;
// a 256 x 256 tile reads half the operand bytes per flop of a 128 x 128 one.
// The scores are stored in tiles of 128 rows (the layout the block-sum pass
// reads), and each row's running max / sum of the two key halves are merged at
// the end.
constexpr int kXWide = 256;
constexpr int kXWideThreads = 512;
constexpr int kXChunkTiles = 8;   // 256-key tiles per score workgroup (2048 reshaped keys)
constexpr int kXBlock = 32;       // consecutive work items per XCD turn (one per CU)
constexpr int kXHalf = 64;
template <typename T, bool TP>
__global__ __launch_bounds__(kXWideThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void xattn_scores_wide_kernel(XScoreK a) {
  // [buffer][Q' rows 0..255, then K' rows 0..255][64 dims]: 2 x 64 KiB
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2][2 * kXWide * kXHalf];
  // Work items (head, 256-row tile R, chunk c of kc key tiles): a head's items
  // run R from the last down and c up; consecutive items go in blocks of
  // kXBlock to one XCD (workgroup w runs on XCD w % 8, blocks dealt in turn),
  // so the XCD's CUs hold a few row tiles x several key chunks of one head at a
  // time and share their Q' and K' stage copies in its L2.
  const int nrt = (a.Lrq + kXWide - 1) / kXWide;
  const int xslot = (int)(blockIdx.x >> 3);
  const int item = ((xslot / kXBlock) * 8 + (int)(blockIdx.x & 7)) * kXBlock + xslot % kXBlock;
  if (item >= a.hg * a.items) return;
  const int hidx = item / a.items;
  int p = item - hidx * a.items, R = nrt - 1;
  for (; R > 0; --R) {
    const int nc = xchunks(R, a.Lrq, a.Lrk, a.causal, a.kdb, a.kc);
    if (p < nc) break;
    p -= nc;
  }
  const int chunk = p;
  const int h = a.h0 + hidx;
  const int hk = h / (a.Hq / a.Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31, hi = lane >> 5;
  const int rg = wave & 3, kg = wave >> 2;          // 64-row group, 128-key group
  const int r0 = R * kXWide, wr0 = r0 + rg * 64;
  const uint16_t* qh = a.q + (int64_t)h * a.q_sh;
  const uint16_t* kh = a.k + (int64_t)hk * a.k_sh;
  const int S = a.S, QS = a.QS;
  const int last_row = min(a.Lrq, r0 + kXWide) - 1;
  int last_key = a.Lrk - 1;
  if (a.causal) last_key = min(last_key, last_row * a.kdb + a.kdb - 1);
  const int nct = last_key / kXWide + 1;           // 256-key tiles of the row tile
  const int ct0 = chunk * a.kc, ct1 = min(nct, ct0 + a.kc);   // this workgroup's key tiles
  if (ct0 >= nct) return;
  // this wave's rows lie in one 128-row tile of the stored layout
  const int rt = wr0 / kXRows;
  const int NK = xnct(rt, a.Lrq, a.Lrk, a.causal, a.kdb) * kXKeys;
  uint16_t* dst_base = a.scores + (int64_t)(h - a.h0) * a.head_stride + xoffset(rt, a.Lrq, a.Lrk, a.causal, a.kdb);
  const bool stats = !TP || a.softmax;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&lds[0][0]);

  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  f32x16_t acc[kXKK][2];
#pragma unroll
  for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[kk][rr][r] = 0.f;

  // stage s = (ct S + j) 2 + dh: key tile ct, token offset j, dims 64 dh .. +63, buffer s & 1.
  // 512 rows of 128 bytes = 64 regions of 1 KiB (8 rows); waves 0-3 copy Q', 4-7 K'
  auto issue = [&](int s) {
    const int dh = s & 1, sj = s >> 1, ct = ct0 + sj / S, j = sj % S;
    const int oj = (int)((a.qorder >> (4 * j)) & 15);
    const uint32_t lb = lds0 + (uint32_t)((s & 1) * 2 * kXWide * kXHalf * 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int Rg = wv * 8 + i, rr = 8 * Rg + (lane >> 3), c = (lane & 7) ^ (rr & 7);
      if (wv < 4) {
        const int t = min((r0 + rr) * QS + oj, a.Lq_tok - 1);
        xdma16(lb + Rg * 1024, qh, (uint32_t)(t * a.q_sl + dh * kXHalf + c * 8) * 2u);
      } else {
        const int t = min((ct * kXWide + rr - kXWide) * S + j, a.Lk_tok - 1);
        xdma16(lb + Rg * 1024, kh, (uint32_t)(t * a.k_sl + dh * kXHalf + c * 8) * 2u);
      }
    }
  };
  auto epilogue = [&](int ct) {
    const int n0 = ct * kXWide + kg * kXKeys;        // this wave's first key
    // the lane's key offsets are formed here from an opaque copy of its half's
    // offset, not hoisted out of the stage loop (64 loop-invariant registers
    // would leave the MFMA loop none to read its operands ahead)
    int h4 = hi * 4;
    asm volatile("" : "+v"(h4));
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int row = wr0 + rr * 32 + l32;
      const bool row_ok = row < a.Lrq;
      // the row's visible keys are one range [klo, khi] (xkey_ok as bounds), so a
      // key's test is two compares with no branch
      int klo = 0, khi = a.Lrk - 1;
      if (a.causal) {
        if constexpr (TP) {
          khi = min(khi, row * a.kdb + a.kdb - 1);
          if (a.own_chunk) klo = (row * a.kdb / a.own_chunk) * a.own_chunk;
        } else {
          khi = min(khi, row);
        }
      }
      if (!row_ok) khi = -1;
      // all ones when the key lies outside [klo, khi] (sign bits; no lane masks held)
      auto outside = [&](int kk, int r) -> uint32_t {
        const int key = n0 + kk * 32 + (r >> 2) * 8 + h4 + (r & 3);
        return (uint32_t)(((khi - key) | (key - klo)) >> 31);
      };
      auto xval = [&](int kk, int r) { return xscaled<T, TP>(a, acc[kk][rr][r]); };
      if (row_ok && n0 < NK) {
        uint16_t* dst = dst_base + (int64_t)(row - rt * kXRows) * NK;
#pragma unroll
        for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t w[2];
#pragma unroll
            for (int e = 0; e < 2; ++e)
              w[e] = XCvt<T>::pack2(acc[kk][rr][g * 4 + 2 * e], acc[kk][rr][g * 4 + 2 * e + 1]);
            *reinterpret_cast<uint2*>(dst + n0 + kk * 32 + g * 8 + h4) = make_uint2(w[0], w[1]);
          }
      }
      if (stats) {
        // the accumulators (stored above) now hold the scaled scores, -inf for an
        // invisible key: it adds nothing to the max, and its exponential is 0
#pragma unroll
        for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const uint32_t o = outside(kk, r);
            acc[kk][rr][r] = __uint_as_float((__float_as_uint(xval(kk, r)) & ~o) | (0xff800000u & o));
          }
        float mx = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[kk][rr][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));    // the row's other keys sit in lane ^ 32
        const float m_new = fmaxf(m_run[rr], mx);
        if (m_new > -INFINITY) {
          float sm = 0.f;
#pragma unroll
          for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
            for (int r = 0; r < 16; ++r) sm += xexp<TP>(acc[kk][rr][r] - m_new);
          l_run[rr] = l_run[rr] * xexp<TP>(m_run[rr] - m_new) + sm;
          m_run[rr] = m_new;
        }
      }
#pragma unroll
      for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[kk][rr][r] = 0.f;
    }
  };

  const int nst = (ct1 - ct0) * S * 2;
  issue(0);
  for (int s = 0; s < nst; ++s) {
    const int dh = s & 1, sj = s >> 1, ct = ct0 + sj / S, j = sj % S;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's copies of stage s
    __syncthreads();                               // every wave's copies landed; stage s-1 done
    if (s + 1 < nst) issue(s + 1);                 // into the buffer stage s-1 used
    const uint16_t* qb = lds[s & 1];
    const uint16_t* kb = lds[s & 1] + kXWide * kXHalf;
    const int oj = (int)((a.qorder >> (4 * j)) & 15);
    if ((r0 + kXWide - 1) * QS + oj >= a.Lq_tok || (ct * kXWide + kXWide - 1) * S + j >= a.Lk_tok) {
      // this stage reaches past the sequence: those rows are zero
      uint16_t* w = lds[s & 1];
      for (int e = tid; e < 2 * kXWide * 8; e += kXWideThreads) {
        const int r = e >> 3, ch = e & 7;
        const bool past = r < kXWide ? (r0 + r) * QS + oj >= a.Lq_tok
                                     : (ct * kXWide + r - kXWide) * S + j >= a.Lk_tok;
        if (past) *reinterpret_cast<uint4*>(w + r * kXHalf + ch * 8) = make_uint4(0, 0, 0, 0);
      }
      __syncthreads();
    }
    // the operands of 16-dim step st + 1 are read while step st's MFMAs run
    // (two register sets), so an MFMA waits only for reads issued a step earlier
    uint4 bq[2][2], ak[2][kXKK];
    auto load_ops = [&](int st, int b) {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int row = rg * 64 + rr * 32 + l32;
        bq[b][rr] = *reinterpret_cast<const uint4*>(qb + row * kXHalf + (((2 * st + hi) ^ (row & 7)) << 3));
      }
#pragma unroll
      for (int kk = 0; kk < kXKK; ++kk) {
        const int key = kg * kXKeys + kk * 32 + l32;
        ak[b][kk] = *reinterpret_cast<const uint4*>(kb + key * kXHalf + (((2 * st + hi) ^ (key & 7)) << 3));
      }
    };
    load_ops(0, 0);
#pragma unroll
    for (int st = 0; st < kXHalf / 16; ++st) {
      if (st + 1 < kXHalf / 16) load_ops(st + 1, (st + 1) & 1);
#pragma unroll
      for (int kk = 0; kk < kXKK; ++kk)
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) acc[kk][rr] = XMma<T>::mma(ak[st & 1][kk], bq[st & 1][rr], acc[kk][rr]);
    }
    {
      // order: step 0's six reads, then each MFMA followed by one read of the
      // next step until they are all issued (a step's reads go out during the
      // previous step's first six MFMAs)
      constexpr int NR = 2 + kXKK, NM = (kXHalf / 16) * kXKK * 2;
      __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i % (2 * kXKK) < NR && i < NM - 2 * kXKK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    if (dh == 1 && j == S - 1) epilogue(ct);
  }

  // ---- each row's two key halves: lanes l and l ^ 32, then the two key-group waves through LDS
  __syncthreads();
  float* xm = reinterpret_cast<float*>(&lds[0][0]);   // [256 rows][2 halves] max, then sum
  float* xl = xm + 2 * kXWide;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int lr = rg * 64 + rr * 32 + l32;
    const float lt = l_run[rr] + __shfl_xor(l_run[rr], 32, 64);
    if (hi == 0) {
      xm[lr * 2 + kg] = m_run[rr];
      xl[lr * 2 + kg] = lt;
    }
  }
  __syncthreads();
  if (kg == 0 && hi == 0) {
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int lr = rg * 64 + rr * 32 + l32, row = r0 + lr;
      if (row >= a.Lrq) continue;
      // this key chunk's row max and sum (the block-sum pass merges the chunks)
      const float m0 = xm[lr * 2], m1 = xm[lr * 2 + 1];
      const float m = fmaxf(m0, m1);
      const float lt = m == -INFINITY ? 0.f : xl[lr * 2] * xexp<TP>(m0 - m) + xl[lr * 2 + 1] * xexp<TP>(m1 - m);
      const int64_t at = ((int64_t)chunk * a.Hq + h) * a.Lrq + row;
      a.m[at] = m;
      a.l[at] = lt;
    }
  }
}

// pass 2 over the stored scores
template <typename T, bool TP>
__global__ __launch_bounds__(kXThreads) void xattn_sums_kernel(XScoreK a) {
  __shared__ float rm[kXRows], rl[kXRows];
  __shared__ int rok[kXRows];
  const int nrt = (a.Lrq + kXRows - 1) / kXRows;
  const int rt = nrt - 1 - (int)(blockIdx.x / a.hg);
  const int h = a.h0 + (int)(blockIdx.x % a.hg);
  const int r0 = rt * kXRows;
  const int nr = min(a.Lrq, r0 + kXRows) - r0;       // a multiple of rpb
  const int NK = xnct(rt, a.Lrq, a.Lrk, a.causal, a.kdb) * kXKeys;
  const int tid = threadIdx.x, rbs = a.rbs, rpb = a.rpb;
  if (tid < kXRows) {
    const int row = r0 + tid;
    const bool ok = row < a.Lrq && row < a.real_rows;   // padding rows add nothing
    float m = 0.f, lv = 0.f;
    if (ok) {
      if (!TP || a.softmax) {
        // the row's key chunks: the max of their maxima, then their sums rescaled to it, in chunk order
        const int nc = xchunks(row / kXWide, a.Lrq, a.Lrk, a.causal, a.kdb, a.kc);
        const int64_t cs = (int64_t)a.Hq * a.Lrq, at = (int64_t)h * a.Lrq + row;
        m = -INFINITY;
        for (int c = 0; c < nc; ++c) m = fmaxf(m, a.m[c * cs + at]);
        if (m != -INFINITY)
          for (int c = 0; c < nc; ++c) lv += a.l[c * cs + at] * xexp<TP>(a.m[c * cs + at] - m);
        if (a.npad > 0) {
          // the chunk padding's keys (zero rows of K) score 0
          const float m2 = fmaxf(m, 0.f);
          lv = lv * xexp<TP>(m - m2) + (float)a.npad * xexp<TP>(-m2);
          m = m2;
        }
      } else {
        lv = 1.f;                                    // no softmax: p = exp(x)
      }
    }
    rok[tid] = ok && lv > 0.f;
    rm[tid] = m;
    rl[tid] = TP ? lv : (lv > 0.f ? 1.0f / lv : 0.f);   // torch path divides, Triton multiplies by 1 / l
  }
  __syncthreads();
  // p of a key with scaled score x in row i: rounded to dtype on the torch path
  auto prob = [&](int i, float x) -> float {
    if constexpr (TP) {
      if (!a.softmax) return Conv<T>::round(expf(x));
      return Conv<T>::round(expf(x - rm[i]) / rl[i]);
    }
    return __builtin_amdgcn_exp2f(x - rm[i]) * rl[i];
  };
  const uint16_t* src =
      a.scores + (int64_t)(h - a.h0) * a.head_stride + xoffset(rt, a.Lrq, a.Lrk, a.causal, a.kdb);
  // eight consecutive keys per thread (one 16-byte load a row): a key block of
  // rbs >= 8 keys spans rbs / 8 neighbouring lanes
  const int gl = rbs / 8;
  for (int c0 = 0; c0 < NK; c0 += 8 * kXThreads) {
    const int n = c0 + 8 * tid;
    const bool key_in = n < NK;                      // NK and n are multiples of 8
    float acc = 0.f;
    for (int i = 0; i < nr; ++i) {
      const int row = r0 + i;
      float v = 0.f;
      // a row's visible keys start and end on multiples of 8 from below (chunk
      // starts are multiples of bs / S >= 8), so n decides whether any is seen
      if (key_in && rok[i] && xkey_ok<TP>(a, row, n)) {
        const uint4 w = *reinterpret_cast<const uint4*>(src + (int64_t)i * NK + n);
        const uint32_t pr[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint16_t e = (uint16_t)((t & 1) ? (pr[t >> 1] >> 16) : (pr[t >> 1] & 0xffffu));
          if (xkey_ok<TP>(a, row, n + t)) v += prob(i, xscaled<T, TP>(a, to_f32(T{e})));
        }
      }
      if constexpr (TP) {
        // the row's sum over the block's keys, rounded to dtype
        for (int o = 1; o < gl; o <<= 1) v += __shfl_xor(v, o, 64);
        acc += Conv<T>::round(v);
      } else {
        acc += v;
      }
      if ((i + 1) % rpb == 0) {                      // the end of a block row
        float tot = acc;
        if constexpr (!TP) for (int o = 1; o < gl; o <<= 1) tot += __shfl_xor(tot, o, 64);
        const int I = row / rpb, J = n / rbs;
        if (key_in && (tid % gl) == 0 && I < a.Nb && J < a.Nb && (!a.causal || J <= I))
          a.sums[((int64_t)h * a.Nb + I) * a.Nb + J] = Conv<T>::round(tot);
        acc = 0.f;
      }
    }
  }
  if (a.npad > 0 && tid < nr / rpb) {
    // non-causal: each key block of the chunk padding holds rbs keys scoring 0
    float acc = 0.f;
    for (int i = tid * rpb; i < (tid + 1) * rpb; ++i) {
      if (!rok[i]) continue;
      if constexpr (TP) acc += Conv<T>::round((float)rbs * prob(i, 0.f));
      else acc += (float)rbs * prob(i, 0.f);
    }
    const int I = (r0 + tid * rpb) / rpb;
    if (I < a.Nb) a.pad_sum[(int64_t)h * a.Nb + I] = Conv<T>::round(acc);
  }
}

// torch path, double / triple: K' [Hk][Lp][D] with token nS + j holding
// round(k[nS+j] + k[nS+(j+1)%S]) (double), then round(K'_j + K'_{(j-1)%S}) (triple)
template <typename T>
__global__ __launch_bounds__(256) void xattn_kaug_kernel(const uint16_t* __restrict__ k, int64_t k_sh, int64_t k_sl,
                                                         int Hk, int L, int Lp, int S, int triple,
                                                         uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // (hk, token, 8-dim chunk)
  if (idx >= (int64_t)Hk * Lp * (kXD / 8)) return;
  const int c = (int)(idx % (kXD / 8));
  const int64_t ht = idx / (kXD / 8);
  const int t = (int)(ht % Lp), hk = (int)(ht / Lp);
  const int n = t / S, j = t - n * S;
  const uint16_t* kh = k + (int64_t)hk * k_sh;
  float r[3][8];                                   // chunks j-1, j, j+1 (mod S)
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const int tt = n * S + (j + d - 1 + S) % S;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (tt < L) w = *reinterpret_cast<const uint4*>(kh + (int64_t)tt * k_sl + c * 8);
    const uint32_t pr[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) r[d][e] = to_f32(T{(uint16_t)((e & 1) ? (pr[e >> 1] >> 16) : (pr[e >> 1] & 0xffffu))});
  }
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = Conv<T>::round(r[1][e] + r[2][e]);                         // chunk j of the doubled key
    if (triple) v = Conv<T>::round(v + Conv<T>::round(r[0][e] + r[1][e]));   // + its chunk j-1
    const uint16_t b = __builtin_bit_cast(uint16_t, Conv<T>::store(v));
    if (e & 1) o[e >> 1] |= (uint32_t)b << 16;
    else o[e >> 1] = b;
  }
  *reinterpret_cast<uint4*>(out + ((int64_t)hk * Lp + t) * kXD + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

struct XSelK {
  const float* sums;            // [Hq][Nb][Nb]
  const float* pad_sum;         // [Hq][Nb] (non-causal)
  const double* thr;            // [Hq]
  int32_t* blk_cnt;             // [Hq][N]
  uint64_t* blk_bits;           // [Hq][N][ceil(Nk / 64)]
  int Hq, Nb, N, Nk, Nbp, causal, keep_sink, keep_recent;
};

__global__ __launch_bounds__(kXSelThreads) void xattn_select_kernel(XSelK a) {
  __shared__ uint64_t key[kXMaxBlocks];             // (~value bits) << 32 | index: ascending = value desc, index asc
  __shared__ double part[kXSelThreads];
  __shared__ uint8_t sel[kXMaxBlocks];
  const int h = (int)(blockIdx.x / a.N), I = (int)(blockIdx.x % a.N);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* row = a.sums + ((int64_t)h * a.Nb + I) * a.Nb;
  const int n = a.causal ? I + 1 : a.Nbp;           // blocks of the row
  const float vpad = a.causal ? 0.f : a.pad_sum[(int64_t)h * a.Nb + I];
  auto val = [&](int J) { return J < a.Nb ? row[J] : vpad; };
  int P = 1;
  while (P < n) P <<= 1;

  // keys (causal: the forced blocks enter the sorted list as zeros, as the
  // reference's masked_fill does) and the row total in a fixed order
  double tot = 0.0;
  for (int J = tid; J < P; J += kXSelThreads) {
    uint64_t kk = ~0ull;
    if (J < n) {
      const float v = val(J);
      tot += (double)v;
      const float vo = (a.causal && (J == 0 || J == I)) ? 0.f : v;
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
  const double forced = a.causal ? (double)row[0] + (I > 0 ? (double)row[I] : 0.0) : 0.0;
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

  // the row's mask words over the real blocks: the chosen ones, the forced ones (causal),
  // block 0 (non-causal: the reference's unselected positions scatter to it),
  // row 0 whole with keep_sink, the diagonal with keep_recent
  if (wave == 0) {
    const int limit = (I == 0 && a.keep_sink) || !a.causal ? a.Nk : n;
    const int NW = (a.Nk + 63) >> 6;
    uint64_t* out = a.blk_bits + ((int64_t)h * a.N + I) * NW;
    int cnt = 0;
    for (int J0 = 0; J0 < NW * 64; J0 += 64) {
      const int J = J0 + lane;
      bool in = false;
      if (J < limit)
        in = (I == 0 && a.keep_sink) || J == 0 || sel[J] || (a.causal && J == I) || (a.keep_recent && J == I);
      const uint64_t m = __ballot(in);
      if (lane == 0) out[J0 >> 6] = m;
      cnt += __popcll(m);
    }
    if (lane == 0) a.blk_cnt[(int64_t)h * a.N + I] = cnt;
  }
}

// Geometry of one call (host)
struct XGeom {
  int N, S, rbs, kdb, QS, Lrq, Lrk, Lp_blk, Lpc, Nbp, real_rows, own_chunk, npad, causal, aug;
  uint64_t qorder;
  int64_t head_stride;
};

static int xgeom(const fs_xattn_args* a, XGeom& g) {
  g.N = (a->L + a->bs - 1) / a->bs;
  g.S = a->stride;
  g.rbs = a->bs / a->stride;
  g.kdb = a->torch_path && a->kdb > 1 ? a->kdb : 1;
  g.causal = a->non_causal ? 0 : 1;
  const bool inverse = !a->torch_path || a->select_mode == 0;
  g.QS = inverse ? g.S * g.kdb : g.S;
  g.aug = a->torch_path && (a->select_mode == 3 || a->select_mode == 4) ? a->select_mode - 2 : 0;
  g.qorder = 0;
  for (int j = 0; j < g.S; ++j) {
    int o = g.S - 1 - j;                                           // inverse, double, triple
    if (a->torch_path && a->select_mode == 1) o = j;               // slash
    if (a->torch_path && a->select_mode == 2) o = a->perm[j];      // random
    g.qorder |= (uint64_t)o << (4 * j);
  }
  g.Lp_blk = g.N * a->bs;
  const int chunk = a->chunk > 0 ? a->chunk : g.Lp_blk;
  g.Lpc = (int)(((int64_t)a->L + chunk - 1) / chunk * chunk);
  g.Nbp = g.Lpc / a->bs;
  g.Lrk = g.N * g.rbs;
  g.Lrq = g.Lrk / g.kdb;
  g.npad = g.causal ? 0 : g.Lpc / g.S - g.Lrk;
  const int k_pad_r = (g.Lpc - a->L) / g.S;                       // k_num_to_pad // stride
  if (a->torch_path) {
    // rows zeroed at the end (Xattention.py:248-249): the last q_pad_r // kdb of
    // the Lpc / (S kdb); when that is 0 with some padding, [-0:] zeroes the last chunk
    int z = k_pad_r / g.kdb;
    if (z == 0 && k_pad_r != 0) z = chunk / g.S / g.kdb;
    g.real_rows = g.Lpc / (g.S * g.kdb) - z;
    // the padding key columns' marks (Xattention.py:205) lie in the last chunk,
    // whose own square (:206-217) is written over them: a row of that chunk sees
    // a padding key at or before its mask row; with no padding the slice [-0:]
    // marks every column first and only the row's own chunk is cleared again
    g.own_chunk = (g.causal && k_pad_r == 0) ? chunk / g.S : 0;
  } else {
    g.real_rows = (a->L + g.S - 1) / g.S;
    g.own_chunk = 0;
  }
  const int nrt = (g.Lrq + kXRows - 1) / kXRows;
  g.head_stride = xoffset(nrt, g.Lrq, g.Lrk, g.causal, g.kdb);
  return 0;
}

// workspace: row max and sum of each key chunk [nck][Hq][Lrq] each, pad sums [Hq][N], K' [Hk][Lp][D]
// (double / triple), the stored scores
static size_t xalign(size_t n) { return (n + 255) & ~(size_t)255; }
// key chunks of the longest row tile (the most any row has)
static int xattn_max_chunks(const XGeom& g) {
  const int nrt = (g.Lrq + kXWide - 1) / kXWide;
  int mx = 1;
  for (int R = 0; R < nrt; ++R) {
    const int c = xchunks(R, g.Lrq, g.Lrk, g.causal, g.kdb, kXChunkTiles);
    mx = c > mx ? c : mx;
  }
  return mx;
}
static size_t xattn_stats_bytes(int Hq, const XGeom& g) {
  return xalign((size_t)xattn_max_chunks(g) * Hq * g.Lrq * 2 * sizeof(float) + (size_t)Hq * g.N * sizeof(float));
}
static size_t xattn_kaug_bytes(int Hk, const XGeom& g) { return g.aug ? xalign((size_t)Hk * g.Lp_blk * kXD * 2) : 0; }
// heads whose scores the workspace holds at once (the passes run head group by head group)
static int xattn_head_group(const fs_xattn_args* a) {
  return a->head_group > 0 && a->head_group < a->Hq ? a->head_group : a->Hq;
}
static size_t xattn_work(const fs_xattn_args* a, const XGeom& g) {
  return xattn_stats_bytes(a->Hq, g) + xattn_kaug_bytes(a->Hk, g) +
         (size_t)xattn_head_group(a) * g.head_stride * sizeof(uint16_t);
}

}  // namespace fs

using namespace fs;

static int xattn_check(const fs_xattn_args* a, bool need_buffers) {
  FS_CHECK_ARG(a != nullptr, "fs_xattn: null args");
  if (need_buffers)
    FS_CHECK_ARG(a->q && a->k && a->threshold && a->sums && a->blk_cnt && a->blk_bits && a->work,
                 "fs_xattn: null pointer");
  FS_CHECK_ARG(((uintptr_t)a->blk_bits & 7) == 0, "fs_xattn: blk_bits must be 8-byte aligned");
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
  FS_CHECK_ARG(a->select_mode >= 0 && a->select_mode <= 4, "fs_xattn: select_mode %d unknown", a->select_mode);
  FS_CHECK_ARG(a->head_group >= 0, "fs_xattn: negative head_group");
  if (a->torch_path && a->select_mode == 2) {
    unsigned seen = 0;
    for (int j = 0; j < a->stride; ++j) {
      FS_CHECK_ARG(a->perm[j] >= 0 && a->perm[j] < a->stride && !(seen >> a->perm[j] & 1u),
                   "fs_xattn: perm is not a permutation of 0..%d", a->stride - 1);
      seen |= 1u << a->perm[j];
    }
  }
  const int kdb = a->kdb > 1 ? a->kdb : 1;
  FS_CHECK_ARG(a->torch_path || kdb == 1, "use_triton and kdb cannot be used together");   // Xattention.py:144
  FS_CHECK_ARG(a->chunk >= 0 && (a->chunk == 0 || (a->chunk % a->bs == 0 && (a->chunk / a->stride) % kdb == 0)),
               "fs_xattn: chunk %d must be a multiple of the block size and of stride x kdb", a->chunk);
  FS_CHECK_ARG((a->bs / a->stride) % kdb == 0, "fs_xattn: kdb %d must divide the reshaped block size %d", kdb,
               a->bs / a->stride);
  FS_CHECK_ARG(!(a->non_causal || a->torch_path) || a->chunk > 0,
               "fs_xattn: the non-causal and torch paths need the chunk size");
  const int N = (a->L + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED(N <= kXMaxBlocks, "fs_xattn: %d blocks > %d", N, kXMaxBlocks);
  XGeom g;
  xgeom(a, g);
  FS_CHECK_SUPPORTED(g.Nbp <= kXMaxBlocks, "fs_xattn: %d chunk-padded blocks > %d", g.Nbp, kXMaxBlocks);
  // the tile copies address a token row by a 32-bit byte offset from the head's base
  FS_CHECK_SUPPORTED((int64_t)g.Lpc * (a->q_sl > a->k_sl ? a->q_sl : a->k_sl) * 2 < ((int64_t)1 << 32) &&
                         (int64_t)g.Lp_blk * kXD * 2 < ((int64_t)1 << 32),
                     "fs_xattn: sequence x row stride too large");
  FS_CHECK_ARG(((uintptr_t)a->q % 16) == 0 && ((uintptr_t)a->k % 16) == 0 && a->q_sl % 8 == 0 && a->k_sl % 8 == 0 &&
                   a->q_sh % 8 == 0 && a->k_sh % 8 == 0,
               "fs_xattn: q/k must be 16-byte aligned with strides of whole 16-byte chunks");
  return FS_OK;
}

extern "C" size_t fs_xattn_work_bytes(const fs_xattn_args* a) {
  if (!a || a->Hq <= 0 || a->Hk <= 0 || a->L <= 0 || a->stride <= 0 || a->bs <= 0 || a->bs % a->stride) return 0;
  XGeom g;
  xgeom(a, g);
  return xattn_work(a, g);
}

extern "C" int fs_xattn(const fs_xattn_args* a, void* stream) {
  if (int rc = xattn_check(a, true)) return rc;
  XGeom g;
  xgeom(a, g);
  XScoreK k{};
  k.q = static_cast<const uint16_t*>(a->q);
  k.q_sh = a->q_sh; k.q_sl = a->q_sl;
  k.Hq = a->Hq; k.Hk = a->Hk; k.S = g.S; k.QS = g.QS;
  k.Lq_tok = a->L;
  k.qorder = g.qorder;
  k.Lrq = g.Lrq; k.Lrk = g.Lrk; k.rbs = g.rbs; k.rpb = g.rbs / g.kdb; k.Nb = g.N;
  k.causal = g.causal; k.kdb = g.kdb; k.own_chunk = g.own_chunk;
  k.real_rows = g.real_rows; k.npad = g.npad; k.softmax = a->no_softmax ? 0 : 1;
  k.scale = (float)(1.4426950408889634 / sqrt((double)a->D) / a->stride / a->norm);
  k.inv_sqrt = 1.0f / (float)sqrt((double)a->D);
  k.inv_S = 1.0f / (float)a->stride;
  k.inv_norm = 1.0f / a->norm;
  char* w = static_cast<char*>(a->work);
  const int nck = xattn_max_chunks(g);
  k.m = reinterpret_cast<float*>(w);
  k.l = k.m + (size_t)nck * a->Hq * g.Lrq;
  k.pad_sum = k.l + (size_t)nck * a->Hq * g.Lrq;
  k.kc = kXChunkTiles;
  k.items = 0;
  for (int R = 0; R < (g.Lrq + kXWide - 1) / kXWide; ++R) k.items += xchunks(R, g.Lrq, g.Lrk, g.causal, g.kdb, k.kc);
  k.sums = a->sums;
  uint16_t* kaug = reinterpret_cast<uint16_t*>(w + xattn_stats_bytes(a->Hq, g));
  k.scores = reinterpret_cast<uint16_t*>(w + xattn_stats_bytes(a->Hq, g) + xattn_kaug_bytes(a->Hk, g));
  k.head_stride = g.head_stride;
  hipStream_t s = (hipStream_t)stream;
  const bool bf = a->dtype == FS_DTYPE_BF16;
  if (g.aug) {
    const int64_t n = (int64_t)a->Hk * g.Lp_blk * (kXD / 8);
    const unsigned blocks = (unsigned)((n + 255) / 256);
    const int triple = g.aug == 2;
    if (bf) xattn_kaug_kernel<bf16_t><<<blocks, 256, 0, s>>>(static_cast<const uint16_t*>(a->k), a->k_sh, a->k_sl,
                                                                a->Hk, a->L, g.Lp_blk, g.S, triple, kaug);
    else xattn_kaug_kernel<f16_t><<<blocks, 256, 0, s>>>(static_cast<const uint16_t*>(a->k), a->k_sh, a->k_sl, a->Hk,
                                                          a->L, g.Lp_blk, g.S, triple, kaug);
    if (int rc = fs_host::launch_status("fs_xattn (keys)")) return rc;
    k.k = kaug;
    k.k_sh = (int64_t)g.Lp_blk * kXD;
    k.k_sl = kXD;
    k.Lk_tok = g.Lp_blk;
  } else {
    k.k = static_cast<const uint16_t*>(a->k);
    k.k_sh = a->k_sh; k.k_sl = a->k_sl;
    k.Lk_tok = a->L;
  }
  // the score and block-sum passes, head group by head group through the same scores buffer
  const int hg = xattn_head_group(a);
  for (int h0 = 0; h0 < a->Hq; h0 += hg) {
    k.h0 = h0;
    k.hg = a->Hq - h0 < hg ? a->Hq - h0 : hg;
    const unsigned grid = (unsigned)(k.hg * ((g.Lrq + kXRows - 1) / kXRows));
    const int64_t nblk = ((int64_t)k.hg * k.items + kXBlock - 1) / kXBlock;   // blocks of work items
    const unsigned wgrid = (unsigned)((nblk + 7) / 8 * 8 * kXBlock);
    if (a->torch_path) {
      if (bf) {
        xattn_scores_wide_kernel<bf16_t, true><<<wgrid, kXWideThreads, 0, s>>>(k);
        xattn_sums_kernel<bf16_t, true><<<grid, kXThreads, 0, s>>>(k);
      } else {
        xattn_scores_wide_kernel<f16_t, true><<<wgrid, kXWideThreads, 0, s>>>(k);
        xattn_sums_kernel<f16_t, true><<<grid, kXThreads, 0, s>>>(k);
      }
    } else {
      if (bf) {
        xattn_scores_wide_kernel<bf16_t, false><<<wgrid, kXWideThreads, 0, s>>>(k);
        xattn_sums_kernel<bf16_t, false><<<grid, kXThreads, 0, s>>>(k);
      } else {
        xattn_scores_wide_kernel<f16_t, false><<<wgrid, kXWideThreads, 0, s>>>(k);
        xattn_sums_kernel<f16_t, false><<<grid, kXThreads, 0, s>>>(k);
      }
    }
    if (int rc = fs_host::launch_status("fs_xattn (scores)")) return rc;
  }
  XSelK sk{};
  sk.sums = a->sums;
  sk.pad_sum = k.pad_sum;
  sk.thr = a->threshold;
  sk.blk_cnt = a->blk_cnt;
  sk.blk_bits = a->blk_bits;
  sk.Hq = a->Hq; sk.Nb = g.N; sk.N = g.N; sk.Nk = g.N; sk.Nbp = g.causal ? g.N : g.Nbp;
  sk.causal = g.causal; sk.keep_sink = a->keep_sink; sk.keep_recent = a->keep_recent;
  xattn_select_kernel<<<(unsigned)(a->Hq * g.N), kXSelThreads, 0, s>>>(sk);
  return fs_host::launch_status("fs_xattn (select)");
}
