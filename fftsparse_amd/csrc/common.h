// Shared device helpers for the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fftsparse_amd.h"

namespace fs {

// ---- element types --------------------------------------------------------
struct bf16_t { uint16_t u; };
struct f16_t { uint16_t u; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float((uint32_t)x.u << 16); }
__device__ __forceinline__ float to_f32(f16_t x) {
  _Float16 h;
  __builtin_memcpy(&h, &x.u, 2);
  return (float)h;
}

// fp32 -> bf16, round to nearest even (nan kept quiet).  Written as a select
// of the two results, so that unrolled code rounds without a branch per value.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

template <typename T> struct Conv;
template <> struct Conv<float> {
  __device__ static float store(float f) { return f; }
  __device__ static float round(float f) { return f; }
};
template <> struct Conv<bf16_t> {
  __device__ static bf16_t store(float f) { return bf16_t{f32_to_bf16_bits(f)}; }
  __device__ static float round(float f) { return to_f32(bf16_t{f32_to_bf16_bits(f)}); }
};
template <> struct Conv<f16_t> {
  __device__ static f16_t store(float f) { return f16_t{f32_to_f16_bits(f)}; }
  __device__ static float round(float f) { return to_f32(f16_t{f32_to_f16_bits(f)}); }
};

// Order-preserving map float -> uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- wave helpers (wave64) --------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// Number of lanes of the wave for which p holds (wave-uniform: a ballot and a
// scalar popcount, no cross-lane data movement).  Call in uniform control flow.
__device__ __forceinline__ int wave_count(bool p) { return (int)__popcll(__ballot(p)); }

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

// Number of set bits of a 64-bit lane mask below this lane.
__device__ __forceinline__ int rank_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// nan-propagating clamp(x, min=lo) (torch.clamp keeps nan).
__device__ __forceinline__ float clamp_min_nan(float x, float lo) { return x < lo ? lo : x; }

// ---- block reductions (blockDim.x threads, scratch >= 32 floats) ----------
template <typename F>
__device__ float block_reduce(float v, float* scratch, F op, float ident) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = ident;
  for (int i = 0; i < nw; ++i) r = op(r, scratch[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum(float v, float* s) {
  return block_reduce(v, s, [](float a, float b) { return a + b; }, 0.0f);
}
__device__ __forceinline__ float block_max(float v, float* s) {
  return block_reduce(v, s, [](float a, float b) { return fmaxf(a, b); }, -INFINITY);
}
__device__ __forceinline__ float block_min(float v, float* s) {
  return block_reduce(v, s, [](float a, float b) { return fminf(a, b); }, INFINITY);
}
__device__ __forceinline__ int block_sum_i(int v, int* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_sum_i(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  int r = 0;
  for (int i = 0; i < nw; ++i) r += scratch[i];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float key_to_f32(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Block-wide top-k over vals[0..n): writes sel[i] = 1 for the k largest
// values (ties to the lower index) and 0 elsewhere; returns the k-th largest
// value.  k is clamped to [0, n].  The k-th largest order-preserving key is
// found by a radix select, 8 bits per pass from the top: each pass
// histograms the digits of the keys that match the digits chosen so far and
// wave 0 picks the digit that holds the (remaining) k-th key.  Equal keys are
// then ranked in index order by wave 0 with ballots.  hist needs kTopkScratch
// ints; all threads of the block must call.
constexpr int kTopkScratch = 256 + 2;
// Order-preserving key of the k-th largest of vals[0..n), 1 <= k <= n (radix
// select, 8 bits per pass from the top).  All threads of the block must call.
__device__ inline uint32_t block_kth_key(const float* vals, int n, int k, int* hist) {
  const int tid = threadIdx.x, nt = blockDim.x;
  uint32_t prefix = 0, mask = 0;
  int kk = k;                                      // rank wanted among keys matching prefix under mask
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += nt) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += nt) {
      const uint32_t key = order_key(vals[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l owns digits 4l .. 4l+3; inc = keys with digit >= 4l
      const int c0 = hist[4 * tid], c1 = hist[4 * tid + 1], c2 = hist[4 * tid + 2], c3 = hist[4 * tid + 3];
      const int tot = c0 + c1 + c2 + c3;
      int inc = tot;
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_down(inc, off, 64);
        if (tid + off < 64) inc += v;
      }
      const int above = inc - tot;                 // keys with digit >= 4l + 4
      if (inc >= kk && above < kk) {
        int d = 4 * tid + 3, s = above + c3;
        int prev = above;
        if (s < kk) { prev = s; s += c2; d = 4 * tid + 2; }
        if (s < kk) { prev = s; s += c1; d = 4 * tid + 1; }
        if (s < kk) { prev = s; s += c0; d = 4 * tid; }
        hist[256] = d;
        hist[257] = kk - prev;                     // rank within digit d
      }
    }
    __syncthreads();
    prefix |= (uint32_t)hist[256] << shift;
    mask |= 255u << shift;
    kk = hist[257];
    __syncthreads();
  }
  return prefix;
}

__device__ inline float block_topk_select(const float* vals, int n, int k, uint8_t* sel, int* hist) {
  const int tid = threadIdx.x, nt = blockDim.x;
  if (k > n) k = n;
  if (k <= 0) {
    for (int i = tid; i < n; i += nt) sel[i] = 0;
    __syncthreads();
    return NAN;
  }
  const uint32_t prefix = block_kth_key(vals, n, k, hist);
  int gt = 0;
  for (int i = tid; i < n; i += nt) {
    const bool g = order_key(vals[i]) > prefix;
    gt += g;
    sel[i] = g;
  }
  gt = block_sum_i(gt, hist);
  const int need = k - gt;
  if (tid < 64) {
    int base = 0;
    for (int c0 = 0; c0 < n && base < need; c0 += 64) {
      const int i = c0 + tid;
      const bool eq = i < n && order_key(vals[i]) == prefix;
      const uint64_t m = __ballot(eq);
      if (eq && base + rank_below(m) < need) sel[i] = 1;
      base += __popcll(m);
    }
  }
  __syncthreads();
  return key_to_f32(prefix);
}

// torch.quantile(vals[0..n), q) with linear interpolation (n >= 1): the fp32
// rank q (n - 1), the order statistics at its floor and ceiling, and torch's
// two-sided lerp between them.  All threads of the block must call.
__device__ inline float block_quantile(const float* vals, int n, float q, int* hist) {
  const float rank = q * (float)(n - 1);
  const int lo = (int)rank, hi = (int)ceilf(rank);
  const float w = rank - (float)lo;
  const float below = key_to_f32(block_kth_key(vals, n, n - lo, hist));     // ascending index lo
  const float above = hi == lo ? below : key_to_f32(block_kth_key(vals, n, n - hi, hist));
  const float d = above - below;
  return fabsf(w) < 0.5f ? below + w * d : above - d * (1.0f - w);
}

// Partial dot product of two rows of D elements (D * sizeof(T) a multiple of
// 16 bytes) held by a group of 16 lanes: lane `sub` takes the 16-byte chunks
// sub, sub + 16, ...; group16_sum then adds the group's partials.  A wave so
// reads four whole rows per load instruction.
template <typename T>
__device__ __forceinline__ float row_dot_part(const T* a, const T* b, int D, int sub) {
  constexpr int V = 16 / sizeof(T);
  float s = 0.f;
  for (int c = sub; c * V < D; c += 16) {
    const uint4 ra = *reinterpret_cast<const uint4*>(a + c * V);
    const uint4 rb = *reinterpret_cast<const uint4*>(b + c * V);
    const T* ea = reinterpret_cast<const T*>(&ra);
    const T* eb = reinterpret_cast<const T*>(&rb);
#pragma unroll
    for (int e = 0; e < V; ++e) s += to_f32(ea[e]) * to_f32(eb[e]);
  }
  return s;
}
__device__ __forceinline__ float group16_sum(float v) {
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Bit position of the r-th (from 0) set bit of x; r < popcount(x).
__device__ __forceinline__ int nth_set_bit(uint64_t x, int r) {
  int p = 0;
  for (int s = 32; s > 0; s >>= 1) {
    const int c = __popcll(x & ((1ull << s) - 1));
    if (r >= c) {
      r -= c;
      x >>= s;
      p += s;
    }
  }
  return p;
}

// Ascending block list of one row written in 16-byte chunks.  The row's G
// membership words (G a power of two) are in LDS: word w (blocks 64 w + bit) at
// wm[w], and the number of entries in the lower words at wp[w]; T is the row's
// entry count.  Chunk c (entries PER c .. PER c + PER - 1, PER = 16 /
// sizeof(E)) is formed by one lane: the word holding its first entry is the
// last one whose prefix is <= PER c, found by binary search over the
// prefixes, and the entries follow from that word's set bits onwards; entry
// (word ws, bit b) is value(ws, b).  The calling lane writes chunks c0, c0 +
// step, ...  Slots past T in the last chunk hold 0.  out must be 16-byte
// aligned with room for PER ceil(T / PER) entries.  One store per chunk,
// instead of one per entry, keeps the write within the memory pipeline's
// address rate.
template <typename E, typename F>
__device__ __forceinline__ void list_chunks_from_lds(E* out, int T, int G, int c0, int step, const uint64_t* wm,
                                                     const int* wp, F value) {
  constexpr int PER = 16 / sizeof(E);
  const int nch = (T + PER - 1) / PER;
  for (int c = c0; c < nch; c += step) {
    const int e0 = PER * c;
    int ws = 0;                                    // the last word whose prefix is <= e0
    for (int st = G >> 1; st > 0; st >>= 1)
      if (ws + st < G && wp[ws + st] <= e0) ws += st;
    uint64_t x = wm[ws];
    x &= ~((1ull << nth_set_bit(x, e0 - wp[ws])) - 1);
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      uint32_t v = 0;
      if (e0 + k < T) {
        while (x == 0 && ws + 1 < G) x = wm[++ws];
        v = x ? (uint32_t)value(ws, __builtin_ctzll(x)) : 0u;
        x &= x - 1;
      }
      if constexpr (PER == 8) pk[k >> 1] |= v << (16 * (k & 1));
      else pk[k] = v;
    }
    *reinterpret_cast<uint4*>(out + e0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
}
// Wave-level form: the row's words are held one per lane by a group of G lanes
// (lane w of the group: word w in m, its prefix in pos; the group's first lane
// is gbase); every lane of the wave puts them in its slot of the wave's LDS
// arrays wm[64] / wp[64], then lane w of the group writes chunks w, w + G, ...
template <typename E, typename F>
__device__ __forceinline__ void write_list_chunks(E* out, uint64_t m, int pos, int T, int G, int w, int gbase,
                                                  uint64_t* wm, int* wp, F value) {
  const int lane = (int)__lane_id();
  wm[lane] = m;
  wp[lane] = pos;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  list_chunks_from_lds(out, T, G, w, G, wm + gbase, wp + gbase, value);
}
// The plain list: entry = block index 64 ws + b.
__device__ __forceinline__ void write_list_chunks(uint16_t* out, uint64_t m, int pos, int T, int G, int w,
                                                  int gbase, uint64_t* wm, int* wp) {
  write_list_chunks(out, m, pos, T, G, w, gbase, wm, wp, [](int ws, int b) { return 64 * ws + b; });
}

}  // namespace fs

// host side ----------------------------------------------------------------
namespace fs_host {
void set_error(const char* fmt, ...);
int launch_status(const char* what);

// Allow a kernel more than the default 64 KiB of dynamic LDS (gfx950: 160 KiB).
template <typename K>
int allow_dynamic_lds(K kernel, size_t bytes, const char* what) {
  if (bytes <= 65536) return 0;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) {
    set_error("%s: cannot reserve %zu bytes of LDS: %s", what, bytes, hipGetErrorString(e));
    return FS_ERR_LAUNCH;
  }
  return 0;
}
}  // namespace fs_host

#define FS_CHECK_ARG(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      fs_host::set_error(__VA_ARGS__);          \
      return FS_ERR_ARG;                        \
    }                                           \
  } while (0)
#define FS_CHECK_SUPPORTED(cond, ...)           \
  do {                                          \
    if (!(cond)) {                              \
      fs_host::set_error(__VA_ARGS__);          \
      return FS_ERR_UNSUPPORTED;                \
    }                                           \
  } while (0)
