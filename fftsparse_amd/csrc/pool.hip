// Q/K block mean pooling (reference: attn_src/fft_attn/my_attn_v7.py:105-114),
// alone (fs_pool) or fused with the rotary embedding that precedes the path
// (fs_rope_pool: the attention forward's apply_rotary_pos_emb,
// eval/LongBench/pred.py:177-195, transformers models/llama/modeling_llama.py
// rotate_half / apply_rotary_pos_emb).
//
// One workgroup reduces one (head, block) tile of bs tokens x D dims.  Each
// thread streams 16-byte vectors of one token row (bs/RPP rows per thread,
// all loads issued before the adds), accumulates in fp32, and the RPP row
// groups are combined through LDS in a fixed order.  The mean is sum * (1/bs)
// (the divisor is bs for a partial last block, as with the reference's zero
// padding), rounded to the input dtype.  Q and K tiles share one launch.
//
// The fused form rotates each loaded row before it is added: the partner
// half of the row (d +- D/2) comes from lane ^ (TPR/2) by a shuffle, the row
// is rotated with the reference's elementwise arithmetic in the input dtype,
//   out = rnd(rnd(x * cos) + rnd(rotate_half(x) * sin)),  rotate_half(x) = (-x2, x1)
// (each product and the sum formed in fp32 and rounded once, as torch's
// 16-bit elementwise ops do; fp32 inputs are not rounded), written out, and
// accumulated exactly as fs_pool accumulates the rotated tensor, so the
// block means are bit-identical to fs_pool applied to the output.  Its grid
// is XCD-aware: the Hq + Hk tiles of one token block run on one XCD, where
// the block's cos / sin rows are read once and then hit that XCD's L2.
#include "common.h"

namespace fs {

constexpr int kPoolThreads = 256;
// rows in flight per thread in the fused pass (4: 0.594 ms at L = 131072 with
// 32 + 8 heads, against 0.600 with 2 and 0.611 with 8)
constexpr int kRopeU = 4;

template <typename T>
struct alignas(16) Vec16 {
  T e[16 / sizeof(T)];
};

// Internal argument block of both entry points.
struct PoolK {
  const void* q; int64_t q_sh, q_sl;
  const void* k; int64_t k_sh, k_sl;
  void* q_b; void* k_b;
  int Hq, Hk, L, D, bs;
  // fused rotary embedding only
  const void* cos; const void* sin; int64_t cs_sl;
  void* q_out; int64_t qo_sh, qo_sl;
  void* k_out; int64_t ko_sh, ko_sl;
};

// Pairs of fp32 values rounded to T (round to nearest even) and back, with
// the pair's storage bits; bf16 uses gfx950's packed conversion
// (v_cvt_pk_bf16_f32), which rounds as the reference's elementwise ops do for
// every finite value.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T> struct Round2;
template <> struct Round2<float> {
  static __device__ __forceinline__ f32x2_t go(f32x2_t v, uint32_t*) { return v; }
};
template <> struct Round2<bf16_t> {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ f32x2_t go(f32x2_t v, uint32_t* bits) {
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
    if (bits) *bits = u;
    return f32x2_t{__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u)};
  }
};
template <> struct Round2<f16_t> {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ f32x2_t go(f32x2_t v, uint32_t* bits) {
    const h2 h = __builtin_convertvector(v, h2);
    if (bits) *bits = __builtin_bit_cast(uint32_t, h);
    return __builtin_convertvector(h, f32x2_t);
  }
};

// x * c + rot * s for two elements, each step rounded to T as the
// reference's separate elementwise ops round (no contraction into an fma);
// bits receives the rounded pair in T's storage (16-bit types)
template <typename T>
__device__ __forceinline__ f32x2_t rope_pair(f32x2_t x, f32x2_t rot, f32x2_t c, f32x2_t s, uint32_t* bits) {
#pragma clang fp contract(off)
  const f32x2_t a = Round2<T>::go(f32x2_t{x[0] * c[0], x[1] * c[1]}, nullptr);
  const f32x2_t b = Round2<T>::go(f32x2_t{rot[0] * s[0], rot[1] * s[1]}, nullptr);
  return Round2<T>::go(f32x2_t{a[0] + b[0], a[1] + b[1]}, bits);
}

// Block means are stored non-temporally: interleaved with the read stream,
// plain write-back stores of the 256-byte results cost the pass 9% of its
// time (209 against 191 us for 1.34 GB with the stores dropped); streaming
// stores bring that to 203 us.
__device__ __forceinline__ void store_mean(float* p, float v) { __builtin_nontemporal_store(v, p); }
template <typename T>
__device__ __forceinline__ void store_mean(T* p, float v) {
  __builtin_nontemporal_store(Conv<T>::store(v).u, reinterpret_cast<uint16_t*>(p));
}

template <typename T, bool ROPE>
__global__ __launch_bounds__(kPoolThreads) void pool_kernel(PoolK a, int N) {
  constexpr int VEC = 16 / sizeof(T);
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int D = a.D, bs = a.bs;
  const int tpr = D / VEC;                 // threads per token row
  const int rpp = kPoolThreads / tpr;      // rows per pass
  const int tid = threadIdx.x;
  const int row_in_pass = tid / tpr, ci = tid % tpr, col = ci * VEC;
  const int H = a.Hq + a.Hk;

  int hh, n;
  if (ROPE) {
    // XCD x (= blockIdx % 8) takes token blocks n = x, x + 8, ..., all heads of a block in a row
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int nn = slot / H;
    hh = slot - nn * H;
    n = nn * 8 + x;
    if (n >= N) return;
  } else {
    hh = blockIdx.x / N;
    n = blockIdx.x - hh * N;
  }
  const T* src;
  int64_t sl;
  T* dst;
  T* rot_out = nullptr;
  int64_t ro_sl = 0;
  if (hh < a.Hq) {
    src = static_cast<const T*>(a.q) + (int64_t)hh * a.q_sh;
    sl = a.q_sl;
    dst = static_cast<T*>(a.q_b) + ((int64_t)hh * N + n) * D;
    if (ROPE) {
      rot_out = static_cast<T*>(a.q_out) + (int64_t)hh * a.qo_sh;
      ro_sl = a.qo_sl;
    }
  } else {
    hh -= a.Hq;
    src = static_cast<const T*>(a.k) + (int64_t)hh * a.k_sh;
    sl = a.k_sl;
    dst = static_cast<T*>(a.k_b) + ((int64_t)hh * N + n) * D;
    if (ROPE) {
      rot_out = static_cast<T*>(a.k_out) + (int64_t)hh * a.ko_sh;
      ro_sl = a.ko_sl;
    }
  }
  const int t0 = n * bs;
  const int rows = min(bs, a.L - t0);

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;

  if (row_in_pass < rpp) {
    // non-temporal loads: the streamed rows are not re-read from the caches
    constexpr int U = ROPE ? kRopeU : 8;
    for (int r0 = row_in_pass; r0 < rows; r0 += U * rpp) {
      Vec16<T> v[U];
      Vec16<T> cs[ROPE ? U : 1], sn[ROPE ? U : 1];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u * rpp;
        if (r < rows) {
          v[u] = __builtin_bit_cast(
              Vec16<T>, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (int64_t)(t0 + r) * sl + col)));
          if constexpr (ROPE) {
            const int64_t co = (int64_t)(t0 + r) * a.cs_sl + col;
            cs[u] = *reinterpret_cast<const Vec16<T>*>(static_cast<const T*>(a.cos) + co);
            sn[u] = *reinterpret_cast<const Vec16<T>*>(static_cast<const T*>(a.sin) + co);
          }
        }
      }
      if constexpr (ROPE) {
        // partner half of the row: lane ^ (tpr / 2) holds d +- D/2 (tpr divides 64,
        // so a row's lanes share a wave); every lane of the wave takes part
        // sign bits of every element of a 32-bit word, flipped for the lower half
        const uint32_t sflip = ci < tpr / 2 ? (sizeof(T) == 2 ? 0x80008000u : 0x80000000u) : 0u;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int r = r0 + u * rpp;
          const u32x4 w = __builtin_bit_cast(u32x4, v[u]);
          u32x4 p;
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] = (unsigned)__shfl_xor((int)w[j], tpr / 2, 64) ^ sflip;
          if (r < rows) {
            const Vec16<T> pv = __builtin_bit_cast(Vec16<T>, p);   // rotate_half(x): partner, negated in the lower half
            Vec16<T> o;
            uint32_t ob[4];
            float of[VEC];
#pragma unroll
            for (int e = 0; e < VEC; e += 2) {
              const f32x2_t y = rope_pair<T>(f32x2_t{to_f32(v[u].e[e]), to_f32(v[u].e[e + 1])},
                                             f32x2_t{to_f32(pv.e[e]), to_f32(pv.e[e + 1])},
                                             f32x2_t{to_f32(cs[u].e[e]), to_f32(cs[u].e[e + 1])},
                                             f32x2_t{to_f32(sn[u].e[e]), to_f32(sn[u].e[e + 1])},
                                             VEC == 8 ? &ob[e / 2] : nullptr);
              of[e] = y[0];
              of[e + 1] = y[1];
            }
            if constexpr (VEC == 8) {
              o = __builtin_bit_cast(Vec16<T>, u32x4{ob[0], ob[1], ob[2], ob[3]});
            } else {
#pragma unroll
              for (int e = 0; e < VEC; ++e) o.e[e] = Conv<T>::store(of[e]);
            }
            *reinterpret_cast<Vec16<T>*>(rot_out + (int64_t)(t0 + r) * ro_sl + col) = o;
            // the same adds, in the same order, as the plain pass below makes on the rotated rows
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] += of[e];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < (ROPE ? 0 : U); ++u) {
        const int r = r0 + u * rpp;
        if (r < rows) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] += to_f32(v[u].e[e]);
        }
      }
    }
  }

  __shared__ float red[kPoolThreads * 8];  // rpp * D <= 256 * 8 floats
  if (row_in_pass < rpp) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[row_in_pass * D + col + e] = acc[e];
  }
  __syncthreads();
  const float inv = 1.0f / (float)bs;
  for (int d = tid; d < D; d += kPoolThreads) {
    float s = 0.f;
    for (int r = 0; r < rpp; ++r) s += red[r * D + d];
    store_mean(&dst[d], s * inv);
  }
}

// The plain pass reserves LDS it does not use so that at most five
// workgroups share a CU: fewer concurrent streams of 32 KiB reads keep the
// DRAM accesses more local (C2 pooling 198-200 -> 196 us, A/B over two
// boxes; three per CU measured 207 us, six or eight 198-200 us).  Blocks of
// fewer than 128 tokens read half as much per workgroup or less, and six
// workgroups per CU keep more bytes in flight (64-token blocks, 65536 tokens
// of 28 + 4 heads: 99.3 -> 82.2-83.2 us; eight per CU 84.6-85.2).
constexpr size_t kPoolLdsReserve = 24 * 1024;     // + the kernel's 8 KiB
constexpr size_t kPoolLdsReserveSmall = 16 * 1024;

template <bool ROPE>
static int launch_pool(const PoolK& k, int dtype, hipStream_t s, const char* what) {
  const int N = (k.L + k.bs - 1) / k.bs;
  const int H = k.Hq + k.Hk;
  const int64_t blocks = ROPE ? (int64_t)((N + 7) / 8) * 8 * H : (int64_t)N * H;
  FS_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", what);
  const size_t lds = ROPE ? 0 : (k.bs >= 128 ? kPoolLdsReserve : kPoolLdsReserveSmall);
  switch (dtype) {
    case FS_DTYPE_F32: pool_kernel<float, ROPE><<<(unsigned)blocks, kPoolThreads, lds, s>>>(k, N); break;
    case FS_DTYPE_BF16: pool_kernel<bf16_t, ROPE><<<(unsigned)blocks, kPoolThreads, lds, s>>>(k, N); break;
    default: pool_kernel<f16_t, ROPE><<<(unsigned)blocks, kPoolThreads, lds, s>>>(k, N); break;
  }
  return fs_host::launch_status(what);
}

}  // namespace fs

using namespace fs;

extern "C" int fs_pool(const fs_pool_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_pool: null args");
  FS_CHECK_ARG(a->q && a->k && a->q_b && a->k_b, "fs_pool: null tensor pointer");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->L > 0 && a->bs > 0, "fs_pool: bad sizes");
  FS_CHECK_SUPPORTED(a->D > 0 && a->D % 8 == 0 && a->D <= 256, "fs_pool: D=%d unsupported", a->D);
  const int esz = a->dtype == FS_DTYPE_F32 ? 4 : 2;
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_F32 || a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16,
                     "fs_pool: dtype %d unsupported", a->dtype);
  FS_CHECK_ARG(((uintptr_t)a->q % 16) == 0 && ((uintptr_t)a->k % 16) == 0,
               "fs_pool: q/k must be 16-byte aligned");
  FS_CHECK_ARG((a->q_sl * esz) % 16 == 0 && (a->q_sh * esz) % 16 == 0 && (a->k_sl * esz) % 16 == 0 &&
                   (a->k_sh * esz) % 16 == 0,
               "fs_pool: strides must be multiples of 16 bytes");
  PoolK k{};
  k.q = a->q; k.q_sh = a->q_sh; k.q_sl = a->q_sl;
  k.k = a->k; k.k_sh = a->k_sh; k.k_sl = a->k_sl;
  k.q_b = a->q_b; k.k_b = a->k_b;
  k.Hq = a->Hq; k.Hk = a->Hk; k.L = a->L; k.D = a->D; k.bs = a->bs;
  return launch_pool<false>(k, a->dtype, (hipStream_t)stream, "fs_pool");
}

extern "C" int fs_rope_pool(const fs_rope_pool_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_rope_pool: null args");
  FS_CHECK_ARG(a->q && a->k && a->cos && a->sin && a->q_out && a->k_out && a->q_b && a->k_b,
               "fs_rope_pool: null tensor pointer");
  FS_CHECK_ARG(a->Hq > 0 && a->Hk > 0 && a->L > 0 && a->bs > 0, "fs_rope_pool: bad sizes");
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_F32 || a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16,
                     "fs_rope_pool: dtype %d unsupported", a->dtype);
  const int esz = a->dtype == FS_DTYPE_F32 ? 4 : 2;
  const int vec = 16 / esz;
  // a row's 16-byte chunks (D / vec threads) must be a power of two dividing
  // the wave, so that the partner half is one shuffle away inside the wave
  const int tpr = a->D / vec;
  FS_CHECK_SUPPORTED(a->D > 0 && a->D % vec == 0 && tpr >= 2 && tpr <= 64 && (tpr & (tpr - 1)) == 0,
                     "fs_rope_pool: D=%d unsupported for dtype %d", a->D, a->dtype);
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->cos, (uintptr_t)a->sin,
                            (uintptr_t)a->q_out, (uintptr_t)a->k_out};
  for (uintptr_t p : ptrs) FS_CHECK_ARG(p % 16 == 0, "fs_rope_pool: tensors must be 16-byte aligned");
  const int64_t strides[] = {a->q_sh, a->q_sl, a->k_sh, a->k_sl, a->cs_sl, a->qo_sh, a->qo_sl, a->ko_sh, a->ko_sl};
  for (int64_t st : strides)
    FS_CHECK_ARG((st * esz) % 16 == 0, "fs_rope_pool: strides must be multiples of 16 bytes");
  PoolK k{};
  k.q = a->q; k.q_sh = a->q_sh; k.q_sl = a->q_sl;
  k.k = a->k; k.k_sh = a->k_sh; k.k_sl = a->k_sl;
  k.q_b = a->q_b; k.k_b = a->k_b;
  k.Hq = a->Hq; k.Hk = a->Hk; k.L = a->L; k.D = a->D; k.bs = a->bs;
  k.cos = a->cos; k.sin = a->sin; k.cs_sl = a->cs_sl;
  k.q_out = a->q_out; k.qo_sh = a->qo_sh; k.qo_sl = a->qo_sl;
  k.k_out = a->k_out; k.ko_sh = a->ko_sh; k.ko_sl = a->ko_sl;
  return launch_pool<true>(k, a->dtype, (hipStream_t)stream, "fs_rope_pool");
}
