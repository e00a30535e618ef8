// Block-sparse causal GQA flash-attention prefill on bf16/f16 MFMA (gfx950).
// Role: block_sparse_attn_func (my_attn_v7.py:775-786) and, with no block
// list, flash_attn_func(causal=True) (my_attn_v7.py:509-519).
//
// Pre-pass (vt_kernel): V [Lk][D] of every KV head is rewritten once per call
// as V^T [D][Lp] (Lp = Nk * BS, zero padded) with the keys of every group of
// 16 stored in the order 0-3, 8-11, 4-7, 12-15.  That order is exactly the
// key order in which an S^T accumulator of v_mfma_f32_32x32x16 hands P to the
// next MFMA (lane half hi owns keys hi*4..hi*4+3 and 8+hi*4..8+hi*4+3 of each
// 16-key group), so every MFMA operand of the main kernel is one
// ds_read_b128 from a row-major LDS tile.
//
// Main kernel: one workgroup per (batch, query head, query block of BS
// tokens); BS/32 x 2 waves, two waves per SIMD so one wave's softmax runs
// while the other's MFMAs issue.  Wave (qq, kh) owns query rows
// qq*32 .. qq*32+31 of the block (Q held in registers as the B operand of
// S^T = K Q^T) and key columns kh*BS/2 .. of every key tile (split-K inside
// the workgroup: each wave keeps its own running max / sum / O^T, merged
// through LDS at the end).  Per selected key block the workgroup copies
// K [BS][D] and V^T [D][BS] into LDS with global_load_lds_dwordx4 (no
// register staging); tiles are double-buffered, the copy of tile t+1 is in
// flight while tile t is consumed.
// LDS rows are 256 B with the 16-byte chunk c of row r stored at c ^ (r & 15)
// so the 8 lanes of a ds_read_b128 phase hit distinct banks.
//
// Scheduling: workgroup w runs on XCD w % 8; XCD x owns every 8th
// query-block row (last rows first) of every head, which balances the work
// of unevenly sparse heads across XCDs.
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

// position of key k inside its 16-key group in the V^T layout (an involution)
__device__ __forceinline__ int vt_pos(int k) {
  const int q = (k >> 2) & 3;
  return (k & ~15) | (((q == 1) ? 2 : (q == 2) ? 1 : q) << 2) | (k & 3);
}

// ---- V -> V^T pre-pass: one workgroup per (b, hk, 64-key slab) -------------
__global__ __launch_bounds__(256) void vt_kernel(const uint16_t* __restrict__ v, int64_t v_sb, int64_t v_sh,
                                                 int64_t v_sl, uint16_t* __restrict__ vt, int Hk, int Lk,
                                                 int Lp) {
  __shared__ uint16_t tile[64][kD + 2];
  const int slabs = Lp / 64;
  const int bh = blockIdx.x / slabs, slab = blockIdx.x - bh * slabs;
  const int b = bh / Hk, hk = bh - b * Hk;
  const uint16_t* src = v + b * v_sb + hk * v_sh;
  uint16_t* dst = vt + (int64_t)bh * kD * Lp;
  const int k0 = slab * 64;
  const int tid = threadIdx.x;
  for (int c = tid; c < 64 * 16; c += 256) {
    const int r = c >> 4, cc = (c & 15) * 8;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (k0 + r < Lk) val = *reinterpret_cast<const uint4*>(src + (int64_t)(k0 + r) * v_sl + cc);
    const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[r][cc + 2 * e] = (uint16_t)(w[e] & 0xffffu);
      tile[r][cc + 2 * e + 1] = (uint16_t)(w[e] >> 16);
    }
  }
  __syncthreads();
  // write 128 rows (d) x 64 keys: each thread emits 8 keys (16 bytes)
  for (int c = tid; c < kD * 8; c += 256) {
    const int d = c >> 3, p0 = (c & 7) * 8;     // 8 stored positions p0 .. p0+7
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ka = vt_pos(p0 + 2 * e), kb = vt_pos(p0 + 2 * e + 1);
      w[e] = (uint32_t)tile[ka][d] | ((uint32_t)tile[kb][d] << 16);
    }
    *reinterpret_cast<uint4*>(dst + (int64_t)d * Lp + k0 + p0) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---- main kernel -------------------------------------------------------------
template <int BS>
struct AttnCfg {
  static constexpr int QW = BS / 32;          // query waves (32 queries each)
  static constexpr int NW = QW * 2;           // waves (x2 key halves)
  static constexpr int NT = NW * 64;          // threads
  static constexpr int KH = BS / 2;           // keys per wave per tile
  static constexpr int KT = KH / 32;          // 32-key sub-tiles per wave
  static constexpr int TILE = BS * kD;        // elements of one K (or V^T) tile
  static constexpr int REGIONS = TILE * 2 / 1024;   // 1 KiB DMA regions per tile
  static constexpr int DMA_PER_WAVE = 2 * REGIONS / NW;
};

// element offset of 16-byte chunk c of 256-byte row r, swizzled
__device__ __forceinline__ int swz(int r, int c) { return r * kD + ((c ^ (r & 15)) << 3); }

// One 1 KiB global -> LDS copy per wave: lane l's 16 bytes land at lds_base + 16 l.
__device__ __forceinline__ void dma16(uint32_t lds_base, const void* gptr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_base), "v"(gptr) : "memory");
}

template <int BS, typename T>
__global__ __launch_bounds__(AttnCfg<BS>::NT) void bsattn_kernel(fs_attn_args a, const uint16_t* __restrict__ vt,
                                                                 int Nq, int Nk, int Lp, int total, int per_xcd) {
  using C = AttnCfg<BS>;
  using Ops = MfmaOps<T>;
  using V8 = typename Ops::V8;
  // double-buffered [K | V^T] tiles; 256-byte rows with swizzled 16-byte chunks
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2][2][C::TILE];

  // Workgroup wg runs on XCD wg % 8.  XCD x takes the query-block rows
  // r = x, x + 8, x + 16, ... (counted from the last query block, so long
  // rows start first) of every head: each XCD gets an even share of every
  // head's work, and the heads of one GQA group at one query block run back
  // to back on the same XCD (shared K/V tiles in its L2).
  const int wg = blockIdx.x;
  const int x = wg & 7, slot = wg >> 3;
  const int per_row = a.Hq;                       // items per row: (hk, head in group)
  const int r = x + 8 * (slot / per_row);
  if (r >= total) return;                         // total = B * Nq rows
  const int g = a.Hq / a.Hk;
  const int hsel = slot % per_row;
  const int hk = hsel / g;
  const int h = hsel;                             // heads of group hk are hk*g .. hk*g+g-1
  const int b = r / Nq;
  const int qb = Nq - 1 - (r - b * Nq);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hi = lane >> 5;
  const int qq = wave % C::QW, kh = wave / C::QW;
  const int kbase = kh * C::KH;
  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vtp = vt + (int64_t)(b * a.Hk + hk) * kD * Lp;
  const int q0 = qb * BS;
  const int off = a.Lk - a.Lq;
  const int qw0 = q0 + qq * 32;                 // first query of this wave
  const int qrow = qw0 + l32;                   // this lane's query

  // Q^T fragments (B operand of S^T = K Q^T): dims st*16 + hi*8 .. +7
  V8 qf[kD / 16];
#pragma unroll
  for (int st = 0; st < kD / 16; ++st) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (qrow < a.Lq) raw = *reinterpret_cast<const uint4*>(qp + (int64_t)qrow * a.q_sl + st * 16 + hi * 8);
    qf[st] = __builtin_bit_cast(V8, raw);
  }

  // Block lists are read through the scalar unit (constant address space):
  // their completion is tracked by lgkmcnt, so reading the next index never
  // waits on the tile copies in flight (vmcnt).
  typedef const __attribute__((address_space(4))) uint32_t* cptr32;
  int cnt;
  const bool listed = a.blk_cnt != nullptr;
  int64_t lbase = 0;
  if (listed) {
    cnt = (int)((cptr32)(uintptr_t)a.blk_cnt)[(int64_t)h * Nq + qb];
    lbase = ((int64_t)h * Nq + qb) * Nk;
  } else {
    const int last_key = a.is_causal ? min(a.Lk - 1, q0 + BS - 1 + off) : a.Lk - 1;
    cnt = last_key < 0 ? 0 : last_key / BS + 1;
  }
  auto block_at = [&](int t) -> int {
    if (!listed) return t;
    const int64_t gi = lbase + t;
    const uint32_t w = ((cptr32)(uintptr_t)a.blk_idx)[gi >> 1];
    return (int)((gi & 1) ? (w >> 16) : (w & 0xffffu));
  };
  // drop trailing blocks entirely above the diagonal (lists are ascending)
  if (a.is_causal) {
    while (cnt > 0 && block_at(cnt - 1) * BS > q0 + BS - 1 + off) --cnt;
  }

  // ---- tile DMA: wave w copies regions w*DPW/2 .. of the K tile and of the V^T tile
  const uint32_t lds0 = (uint32_t)(uintptr_t)&lds[0][0][0];
  auto issue = [&](int kb, int buf) {
    kb = min(kb, Nk - 1);                          // out-of-range entries are skipped at compute
    const int k0 = kb * BS;
    const int row = lane >> 4, slot = lane & 15;
#pragma unroll
    for (int i = 0; i < C::DMA_PER_WAVE / 2; ++i) {
      const int R = wave * (C::DMA_PER_WAVE / 2) + i;          // region: LDS rows 4R .. 4R+3
      const int r = 4 * R + row;
      const int c = slot ^ (r & 15);
      // K rows past Lk are clamped to the last row (their scores are masked)
      const int key = min(k0 + r, a.Lk - 1);
      dma16(__builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(((buf * 2 + 0) * C::TILE + R * 512) * 2)),
            kp + (int64_t)key * a.k_sl + c * 8);
      int d, kc;
      if (BS == 128) {
        d = r;
        kc = c;
      } else {                                     // two 64-key d rows per 256-byte LDS row
        d = 2 * r + (c >> 3);
        kc = c & 7;
      }
      dma16(__builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(((buf * 2 + 1) * C::TILE + R * 512) * 2)),
            vtp + (int64_t)d * Lp + k0 + kc * 8);
    }
  };
  auto vt_slot = [](int d, int chunk) {
    return BS == 128 ? swz(d, chunk) : swz(d >> 1, (d & 1) * 8 + chunk);
  };

  // Running max is kept in the exp2 domain of raw scores times sc; it is only
  // raised (and O rescaled) when a new score exceeds it by more than 2^8, so
  // p = 2^(s*sc - m) <= 256 and most tiles skip the rescale.
  const float sc = a.softmax_scale * 1.44269504088896340736f;
  constexpr float kSlack = 8.0f;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[kD / 32];
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;

  // Retire the Q loads here, through a wait the compiler sees: otherwise it
  // guards their first use inside the loop with a vmcnt(0) on every iteration,
  // which would also wait for the tile copy in flight.
  __builtin_amdgcn_s_waitcnt(0);
  // Pipeline per iteration t: wait for the copy of tile t, one barrier (tile t
  // visible; every wave is past tile t-1, so its buffer may be refilled),
  // start the copy of tile t+1, touch tile t+2 into L2 (one dword per
  // 128-byte line and thread), compute tile t.  The touch loads land in a
  // register that stays live until a later wait has retired them.
  auto touch = [&](int kb) -> uint32_t {
    kb = min(kb, Nk - 1);
    const int k0 = kb * BS;
    const uint16_t* p;
    if (tid < BS * 2) {                            // K: two 128-byte lines per 256-byte row
      const int key = min(k0 + (tid >> 1), a.Lk - 1);
      p = kp + (int64_t)key * a.k_sl + (tid & 1) * 64;
    } else {                                       // V^T: BS/64 lines per d row
      const int v = tid - BS * 2;
      p = vtp + (int64_t)(v / (BS / 64)) * Lp + k0 + (v % (BS / 64)) * 64;
    }
    uint32_t x;
    asm volatile("global_load_dword %0, %1, off" : "=v"(x) : "v"(p) : "memory");
    return x;
  };
  static_assert(AttnCfg<BS>::NT == BS * 2 + kD * (BS / 64), "one touch line per thread");
  uint32_t pf_prev = 0, pf_cur = 0;
  int kb_cur = cnt > 0 ? block_at(0) : 0;
  if (cnt > 0) issue(kb_cur, 0);
  if (cnt > 1) pf_cur = touch(block_at(1));
  for (int t = 0; t < cnt; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < cnt;
    if (more) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");   // the touch of t+1 may stay in flight
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("" :: "v"(pf_prev));             // touch of tile t retired: release its register
    pf_prev = pf_cur;
    __builtin_amdgcn_s_barrier();
    const int kb = kb_cur;
    if (more) {
      kb_cur = block_at(t + 1);
      issue(kb_cur, buf ^ 1);
    }
    if (t + 2 < cnt) pf_cur = touch(block_at(t + 2));
    const int k0 = kb * BS;
    const int kw0 = k0 + kbase;                   // first key of this wave
    const bool active = kb < Nk && kw0 < a.Lk && !(a.is_causal && kw0 > qw0 + 31 + off);
    if (active) {
      const uint16_t* Kt = lds[buf][0];
      const uint16_t* Vt = lds[buf][1];
      // ---- S^T = K Q^T  (this wave's KH keys x 32 queries)
      f32x16_t s[C::KT];
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int st = 0; st < kD / 16; ++st)
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
          const int row = kbase + kt * 32 + l32;
          const V8 ka = __builtin_bit_cast(V8, *reinterpret_cast<const uint4*>(&Kt[swz(row, st * 2 + hi)]));
          s[kt] = Ops::mma(ka, qf[st], s[kt]);
        }
      // ---- mask, online softmax (exp2 domain)
      if ((kw0 + C::KH > a.Lk) || (a.is_causal && kw0 + C::KH - 1 > qw0 + off)) {
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kw0 + kt * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
            if (key >= a.Lk || (a.is_causal && key > qrow + off)) s[kt][r] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * sc;
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kSlack) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], sc, -m_use));
          s[kt][r] = p;
          rs += p;
        }
      l_run += rs + __shfl_xor(rs, 32, 64);
      // ---- O^T += V^T P^T over this wave's keys
#pragma unroll
      for (int kk = 0; kk < C::KH / 16; ++kk) {
        const int kt = kk >> 1, half = kk & 1;
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = s[kt][8 * half + j];
        const V8 pb = Ops::pack(pv);
        const int ch = ((kbase + kk * 16) >> 3) + hi;    // 16-byte chunk of this lane's 8 keys
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt) {
          const V8 va = __builtin_bit_cast(V8, *reinterpret_cast<const uint4*>(&Vt[vt_slot(dt * 32 + l32, ch)]));
          o[dt] = Ops::mma(va, pb, o[dt]);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" :: "v"(pf_prev), "v"(pf_cur) : "memory");
  __syncthreads();

  // ---- merge the two key halves through LDS, normalise, store
  float* red = reinterpret_cast<float*>(&lds[0][0][0]);   // [QW][PER][64]
  constexpr int PER = (kD / 32) * 16 + 2;
  if (kh == 1) {
    float* dst = red + (size_t)qq * PER * 64;
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(dt * 16 + r) * 64 + lane] = o[dt][r];
    dst[(PER - 2) * 64 + lane] = m_run;
    dst[(PER - 1) * 64 + lane] = l_run;
  }
  __syncthreads();
  if (kh == 1 || qrow >= a.Lq) return;
  const float* src = red + (size_t)qq * PER * 64;
  const float m1 = src[(PER - 2) * 64 + lane];
  const float l1 = src[(PER - 1) * 64 + lane];
  const float m = fmaxf(m_run, m1);
  const float mu = m == -INFINITY ? 0.f : m;
  const float f0 = __builtin_amdgcn_exp2f(m_run - mu);
  const float f1 = __builtin_amdgcn_exp2f(m1 - mu);
  const float l = l_run * f0 + l1 * f1;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.out) + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_sl;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = g4 * 4 + e;
        v4[e] = (o[dt][r] * f0 + src[(dt * 16 + r) * 64 + lane] * f1) * inv;
      }
      const int d0 = dt * 32 + g4 * 8 + hi * 4;
      uint2 w;
      w.x = (uint32_t)Ops::bits(v4[0]) | ((uint32_t)Ops::bits(v4[1]) << 16);
      w.y = (uint32_t)Ops::bits(v4[2]) | ((uint32_t)Ops::bits(v4[3]) << 16);
      *reinterpret_cast<uint2*>(op + d0) = w;
    }
}

template <int BS, typename T>
static int launch_attn(const fs_attn_args& a, int Nq, int Nk, hipStream_t s) {
  const int Lp = Nk * BS;
  uint16_t* vt = static_cast<uint16_t*>(a.work);
  const int slabs = Lp / 64;
  vt_kernel<<<a.B * a.Hk * slabs, 256, 0, s>>>(static_cast<const uint16_t*>(a.v), a.v_sb, a.v_sh, a.v_sl, vt,
                                               a.Hk, a.Lk, Lp);
  if (int rc = fs_host::launch_status("fs_bsattn (V^T)")) return rc;
  const int rows = a.B * Nq;
  const int per_xcd = (rows + 7) / 8 * a.Hq;
  bsattn_kernel<BS, T><<<per_xcd * 8, AttnCfg<BS>::NT, 0, s>>>(a, vt, Nq, Nk, Lp, rows, per_xcd);
  return fs_host::launch_status("fs_bsattn");
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_bsattn_work_bytes(int B, int Hk, int Lk, int D, int bs) {
  if (B <= 0 || Hk <= 0 || Lk <= 0 || D <= 0 || bs <= 0) return 0;
  const int64_t Nk = (Lk + bs - 1) / bs;
  return (size_t)B * Hk * D * Nk * bs * 2;
}

extern "C" int fs_bsattn(const fs_attn_args* a, void* stream) {
  FS_CHECK_ARG(a != nullptr, "fs_bsattn: null args");
  FS_CHECK_ARG(a->q && a->k && a->v && a->out && a->work, "fs_bsattn: null tensor pointer");
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
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->v, (uintptr_t)a->out,
                            (uintptr_t)a->work};
  for (uintptr_t p : ptrs) FS_CHECK_ARG(p % 16 == 0, "fs_bsattn: tensors must be 16-byte aligned");
  const int Nq = (a->Lq + a->bs - 1) / a->bs;
  const int Nk = (a->Lk + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED((int64_t)a->B * a->Hq * Nq < (1ll << 30) && (int64_t)a->B * a->Hk * Nk * a->bs / 64 < (1ll << 31),
                     "fs_bsattn: grid too large");
  hipStream_t s = (hipStream_t)stream;
  if (a->bs == 128) {
    return a->dtype == FS_DTYPE_BF16 ? launch_attn<128, bf16_t>(*a, Nq, Nk, s) : launch_attn<128, f16_t>(*a, Nq, Nk, s);
  }
  return a->dtype == FS_DTYPE_BF16 ? launch_attn<64, bf16_t>(*a, Nq, Nk, s) : launch_attn<64, f16_t>(*a, Nq, Nk, s);
}
