// Q/K block mean pooling (reference: attn_src/fft_attn/my_attn_v7.py:105-114).
//
// One workgroup reduces one (head, block) tile of bs tokens x D dims.  Each
// thread streams 16-byte vectors of one token row (bs/RPP rows per thread,
// all loads issued before the adds), accumulates in fp32, and the RPP row
// groups are combined through LDS in a fixed order.  The mean is sum * (1/bs)
// (the divisor is bs for a partial last block, as with the reference's zero
// padding), rounded to the input dtype.  Q and K tiles share one launch.
#include "common.h"

namespace fs {

constexpr int kPoolThreads = 256;

template <typename T>
struct alignas(16) Vec16 {
  T e[16 / sizeof(T)];
};

template <typename T>
__global__ __launch_bounds__(kPoolThreads) void pool_kernel(fs_pool_args a, int N) {
  constexpr int VEC = 16 / sizeof(T);
  const int D = a.D, bs = a.bs;
  const int tpr = D / VEC;                 // threads per token row
  const int rpp = kPoolThreads / tpr;      // rows per pass
  const int tid = threadIdx.x;
  const int row_in_pass = tid / tpr, col = (tid % tpr) * VEC;

  int hh = blockIdx.x / N;
  const int n = blockIdx.x - hh * N;
  const T* src;
  int64_t sl;
  T* dst;
  if (hh < a.Hq) {
    src = static_cast<const T*>(a.q) + (int64_t)hh * a.q_sh;
    sl = a.q_sl;
    dst = static_cast<T*>(a.q_b) + ((int64_t)hh * N + n) * D;
  } else {
    hh -= a.Hq;
    src = static_cast<const T*>(a.k) + (int64_t)hh * a.k_sh;
    sl = a.k_sl;
    dst = static_cast<T*>(a.k_b) + ((int64_t)hh * N + n) * D;
  }
  const int t0 = n * bs;
  const int rows = min(bs, a.L - t0);

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;

  if (row_in_pass < rpp) {
    // non-temporal loads: the streamed rows are not re-read from the caches
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    constexpr int U = 8;
    for (int r0 = row_in_pass; r0 < rows; r0 += U * rpp) {
      Vec16<T> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u * rpp;
        if (r < rows)
          v[u] = __builtin_bit_cast(
              Vec16<T>, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (int64_t)(t0 + r) * sl + col)));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
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
    dst[d] = Conv<T>::store(s * inv);
  }
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
  const int N = (a->L + a->bs - 1) / a->bs;
  const int64_t blocks = (int64_t)N * (a->Hq + a->Hk);
  FS_CHECK_SUPPORTED(blocks < (1ll << 31), "fs_pool: grid too large");
  hipStream_t s = (hipStream_t)stream;
  switch (a->dtype) {
    case FS_DTYPE_F32: pool_kernel<float><<<(unsigned)blocks, kPoolThreads, 0, s>>>(*a, N); break;
    case FS_DTYPE_BF16: pool_kernel<bf16_t><<<(unsigned)blocks, kPoolThreads, 0, s>>>(*a, N); break;
    default: pool_kernel<f16_t><<<(unsigned)blocks, kPoolThreads, 0, s>>>(*a, N); break;
  }
  return fs_host::launch_status("fs_pool");
}
