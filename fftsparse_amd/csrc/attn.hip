// Block-sparse causal GQA flash-attention prefill on bf16/f16 MFMA (gfx950).
// Role: block_sparse_attn_func (my_attn_v7.py:775-786) and, with no block
// list, flash_attn_func(causal=True) (my_attn_v7.py:509-519).
//
// Work item = (batch, query head, query block of BS tokens).  A workgroup of
// BS/32 waves owns one item; wave w owns query rows q0 + 32w .. q0 + 32w + 31
// and keeps them in registers as the B operand of S^T = K Q^T, so every lane
// owns one query column of S^T and of O^T: the softmax statistics and the
// output rescale stay inside the lane (plus one exchange with lane ^ 32).
// Per selected key block the workgroup stages K [BS][D] row-major and V^T
// [D][BS] in LDS (padded rows against bank conflicts), then each wave runs
//   S^T (BS x 32)  = K . Q^T      : (BS/32) x (D/16) v_mfma_f32_32x32x16
//   online softmax in fp32, exp2 domain
//   O^T (D x 32)  += V^T . P^T    : (D/32) x (BS/16) v_mfma_f32_32x32x16
// P^T is fed to the second MFMA straight from the S^T accumulators: the
// MFMA reduction slot k of lane half hi carries key (k/4)*8 + hi*4 + k%4 of
// each 16-key group, and V^T is read with the same key order.
//
// Scheduling: items are mapped XCD-major (workgroup w runs on XCD w % 8) so
// that one XCD walks a contiguous range of (kv head, query block, head in
// group); query blocks are visited last-first so the longest rows start first.
#include "common.h"

namespace fs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct MfmaOps;
template <> struct MfmaOps<bf16_t> {
  using V8 = bf16x8_t;
  static __device__ __forceinline__ f32x16_t mma(V8 a, V8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ V8 pack(const float* x) {
    V8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)x[i];
    return r;
  }
  static __device__ __forceinline__ uint16_t bits(float x) {
    __bf16 b = (__bf16)x;
    return __builtin_bit_cast(uint16_t, b);
  }
};
template <> struct MfmaOps<f16_t> {
  using V8 = f16x8_t;
  static __device__ __forceinline__ f32x16_t mma(V8 a, V8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ V8 pack(const float* x) {
    V8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)x[i];
    return r;
  }
  static __device__ __forceinline__ uint16_t bits(float x) {
    _Float16 b = (_Float16)x;
    return __builtin_bit_cast(uint16_t, b);
  }
};

constexpr int kD = 128;

template <int BS, typename T>
__global__ __launch_bounds__(BS * 2, 2) void bsattn_kernel(fs_attn_args a, int Nq, int Nk, int total, int per_xcd) {
  using Ops = MfmaOps<T>;
  using V8 = typename Ops::V8;
  constexpr int NT = BS * 2;          // threads
  constexpr int KT = BS / 32;         // 32-key sub-tiles per block
  constexpr int KPAD = kD + 8;        // K row stride (elements)
  constexpr int VPAD = BS + 4;        // V^T row stride (elements)
  __shared__ __attribute__((aligned(16))) uint16_t Ks[BS * KPAD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * VPAD];

  const int wg = blockIdx.x;
  const int li = (wg & 7) * per_xcd + (wg >> 3);
  if (li >= total) return;
  const int g = a.Hq / a.Hk;
  const int per_b = a.Hk * Nq * g;
  const int b = li / per_b;
  int rem = li - b * per_b;
  const int hk = rem / (Nq * g);
  rem -= hk * (Nq * g);
  const int qi = rem / g;
  const int h = hk * g + (rem - qi * g);
  const int qb = Nq - 1 - qi;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vp = static_cast<const uint16_t*>(a.v) + b * a.v_sb + hk * a.v_sh;
  const int q0 = qb * BS;
  const int qrow = q0 + wave * 32 + l32;
  const int off = a.Lk - a.Lq;

  // Q^T fragments: lane holds query qrow, dims st*16 + hi*8 .. +7
  V8 qf[kD / 16];
#pragma unroll
  for (int st = 0; st < kD / 16; ++st) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (qrow < a.Lq) raw = *reinterpret_cast<const uint4*>(qp + (int64_t)qrow * a.q_sl + st * 16 + hi * 8);
    qf[st] = __builtin_bit_cast(V8, raw);
  }

  int cnt;
  const uint16_t* lst = nullptr;
  if (a.blk_cnt) {
    cnt = a.blk_cnt[(int64_t)h * Nq + qb];
    lst = a.blk_idx + ((int64_t)h * Nq + qb) * Nk;
  } else {
    const int last_key = a.is_causal ? min(a.Lk - 1, q0 + BS - 1 + off) : a.Lk - 1;
    cnt = last_key < 0 ? 0 : last_key / BS + 1;
  }

  const float sc = a.softmax_scale * 1.44269504088896340736f;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[kD / 32];
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;

  const int qlast_wg = q0 + BS - 1 + off;          // last query of the item, in key coordinates
  const int qlast_w = q0 + wave * 32 + 31 + off;   // last query of this wave
  const int qfirst_w = q0 + wave * 32 + off;

  for (int t = 0; t < cnt; ++t) {
    const int kb = lst ? (int)lst[t] : t;
    const int k0 = kb * BS;
    if (a.is_causal && k0 > qlast_wg) continue;     // block above the diagonal
    __syncthreads();
    // ---- stage K (row-major) and V^T
#pragma unroll
    for (int c = tid; c < BS * 16; c += NT) {
      const int r = c >> 4, cc = (c & 15) * 8;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (k0 + r < a.Lk) val = *reinterpret_cast<const uint4*>(kp + (int64_t)(k0 + r) * a.k_sl + cc);
      *reinterpret_cast<uint4*>(&Ks[r * KPAD + cc]) = val;
    }
#pragma unroll
    for (int c = tid; c < (BS / 2) * 16; c += NT) {
      const int r = (c >> 4) * 2, cc = (c & 15) * 8;
      uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
      if (k0 + r < a.Lk) v0 = *reinterpret_cast<const uint4*>(vp + (int64_t)(k0 + r) * a.v_sl + cc);
      if (k0 + r + 1 < a.Lk) v1 = *reinterpret_cast<const uint4*>(vp + (int64_t)(k0 + r + 1) * a.v_sl + cc);
      const uint32_t w0[4] = {v0.x, v0.y, v0.z, v0.w};
      const uint32_t w1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = (w0[e] & 0xffffu) | (w1[e] << 16);
        const uint32_t hi2 = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(&Vt[(cc + 2 * e) * VPAD + r]) = lo;
        *reinterpret_cast<uint32_t*>(&Vt[(cc + 2 * e + 1) * VPAD + r]) = hi2;
      }
    }
    __syncthreads();
    if (a.is_causal && k0 > qlast_w) continue;      // whole wave above the diagonal

    // ---- S^T = K Q^T
    f32x16_t s[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int st = 0; st < kD / 16; ++st) {
        const uint4 raw = *reinterpret_cast<const uint4*>(&Ks[(kt * 32 + l32) * KPAD + st * 16 + hi * 8]);
        s[kt] = Ops::mma(__builtin_bit_cast(V8, raw), qf[st], s[kt]);
      }
    }
    // ---- mask, online softmax (exp2 domain)
    const bool need_mask = (k0 + BS > a.Lk) || (a.is_causal && k0 + BS - 1 > qfirst_w);
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[kt][r] * sc;
        if (need_mask) {
          const int key = k0 + kt * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
          if (key >= a.Lk || (a.is_causal && key > qrow + off)) x = -INFINITY;
        }
        s[kt][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[kt][r] - m_use);
        s[kt][r] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32, 64);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;

    // ---- O^T += V^T P^T
#pragma unroll
    for (int kk = 0; kk < BS / 16; ++kk) {
      const int kt = kk >> 1, half = kk & 1;
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = s[kt][8 * half + j];
      const V8 pb = Ops::pack(pv);
      const int key0 = kt * 32 + half * 16 + hi * 4;
#pragma unroll
      for (int dt = 0; dt < kD / 32; ++dt) {
        const uint16_t* vr = &Vt[(dt * 32 + l32) * VPAD + key0];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi8 = *reinterpret_cast<const uint2*>(vr + 8);
        const uint4 raw = make_uint4(lo.x, lo.y, hi8.x, hi8.y);
        o[dt] = Ops::mma(__builtin_bit_cast(V8, raw), pb, o[dt]);
      }
    }
  }

  if (qrow >= a.Lq) return;
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.out) + b * a.o_sb + (int64_t)qrow * a.o_sl + h * a.o_sh;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = dt * 32 + g4 * 8 + hi * 4;
      uint2 w;
      w.x = (uint32_t)Ops::bits(o[dt][g4 * 4 + 0] * inv) | ((uint32_t)Ops::bits(o[dt][g4 * 4 + 1] * inv) << 16);
      w.y = (uint32_t)Ops::bits(o[dt][g4 * 4 + 2] * inv) | ((uint32_t)Ops::bits(o[dt][g4 * 4 + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + d0) = w;
    }
}

template <int BS, typename T>
static void launch_attn(const fs_attn_args& a, int Nq, int Nk, hipStream_t s) {
  const int total = a.B * a.Hq * Nq;
  const int per_xcd = (total + 7) / 8;
  bsattn_kernel<BS, T><<<per_xcd * 8, BS * 2, 0, s>>>(a, Nq, Nk, total, per_xcd);
}

}  // namespace fs

using namespace fs;

extern "C" int fs_bsattn(const fs_attn_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_bsattn: null args");
  FS_CHECK_ARG(a->q && a->k && a->v && a->out, "fs_bsattn: null tensor pointer");
  FS_CHECK_ARG(a->B >= 1 && a->Hq >= 1 && a->Hk >= 1 && a->Hq % a->Hk == 0,
               "fs_bsattn: Hq=%d must be a multiple of Hk=%d", a->Hq, a->Hk);
  FS_CHECK_ARG(a->Lq >= 1 && a->Lk >= 1, "fs_bsattn: empty sequence");
  FS_CHECK_SUPPORTED(a->D == kD, "fs_bsattn: head_dim %d unsupported (128 only)", a->D);
  FS_CHECK_SUPPORTED(a->bs == 64 || a->bs == 128, "fs_bsattn: block size %d unsupported", a->bs);
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16,
                     "fs_bsattn: dtype %d unsupported (bf16/f16)", a->dtype);
  FS_CHECK_ARG(a->blk_cnt == nullptr || (a->blk_idx != nullptr && a->B == 1),
               "fs_bsattn: block lists need blk_idx and B == 1");
  const int64_t strides[] = {a->q_sb, a->q_sh, a->q_sl, a->k_sb, a->k_sh, a->k_sl,
                             a->v_sb, a->v_sh, a->v_sl, a->o_sb, a->o_sh, a->o_sl};
  for (int64_t st : strides) FS_CHECK_ARG(st % 8 == 0, "fs_bsattn: strides must be multiples of 8 elements");
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->v, (uintptr_t)a->out};
  for (uintptr_t p : ptrs) FS_CHECK_ARG(p % 16 == 0, "fs_bsattn: tensors must be 16-byte aligned");
  const int Nq = (a->Lq + a->bs - 1) / a->bs;
  const int Nk = (a->Lk + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED((int64_t)a->B * a->Hq * Nq < (1ll << 30), "fs_bsattn: grid too large");
  hipStream_t s = (hipStream_t)stream;
  if (a->bs == 128) {
    if (a->dtype == FS_DTYPE_BF16) launch_attn<128, bf16_t>(*a, Nq, Nk, s);
    else launch_attn<128, f16_t>(*a, Nq, Nk, s);
  } else {
    if (a->dtype == FS_DTYPE_BF16) launch_attn<64, bf16_t>(*a, Nq, Nk, s);
    else launch_attn<64, f16_t>(*a, Nq, Nk, s);
  }
  return fs_host::launch_status("fs_bsattn");
}
