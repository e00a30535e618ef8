// Block-sparse causal GQA flash-attention prefill on bf16/f16 MFMA (gfx950).
// Role: block_sparse_attn_func (my_attn_v7.py:775-786) and, with no block
// list, flash_attn_func(causal=True) (my_attn_v7.py:509-519).
//
// Pre-pass (vt_kernel): V [Lk][D] of every KV head is rewritten once per call
// as V^T [D][Lp] (Lp = Nk * BS rounded up to 64, zero padded) with the keys of every group of
// 16 stored in the order 0-3, 8-11, 4-7, 12-15.  With 16- or 32-token block
// lists (union mode) V^T is stored block by block instead, [Lp / bs][D][bs]:
// the copy of one listed block is then one contiguous run of D * bs keys
// rather than D pieces of bs keys (64 or 32 bytes) strided by Lp.  That order is exactly the
// key order in which an S^T accumulator of v_mfma_f32_32x32x16 hands P to the
// next MFMA (lane half hi owns keys hi*4..hi*4+3 and 8+hi*4..8+hi*4+3 of each
// 16-key group), so every MFMA operand of the main kernel is one
// ds_read_b128 from a row-major LDS tile.
//
// Main kernel: one workgroup per (batch, query head, query block of BS
// tokens).  Keys are consumed in LDS tiles of TK keys: K [TK][D] and
// V^T [D][TK] copied with global_load_lds_dwordx4 (no register staging),
// double-buffered so the copies of the next tiles are in flight while one is
// consumed.  Wave (qq, kh) owns query rows qq*32 .. qq*32+31 of the block (Q
// held in registers as the B operand of S^T = K Q^T) and keys kh*TK/KG .. of
// every tile, with its own running max / sum / O^T.
//  - BS = 128 uses TK = 64: 4 waves, each over all 64 keys of a tile (no
//    split), 64 KiB of LDS, so two workgroups share a CU and the two waves
//    on a SIMD belong to independent workgroups (one's softmax or barrier
//    wait overlaps the other's MFMAs).
//  - BS = 64 uses TK = 64 split between two key groups (4 waves), merged
//    through LDS at the end.
//  - 16- and 32-token block lists run in union mode: a workgroup of 128
//    queries walks the union of its 128 / bs rows' lists (see below), with the
//    BS = 128 layout.  Dense calls at those block sizes take the BS = 128 kernel.
// LDS rows are 256 B with the 16-byte chunk c of row r stored at c ^ (r & 15)
// so the 8 lanes of a ds_read_b128 phase hit distinct banks.
//
// Scheduling: workgroup w runs on XCD w % 8.  With block lists, the query
// blocks of a head are grouped in runs of consecutive blocks; a counting sort
// (order_kernel) ranks the runs KV group by KV group (one KV head's K and V^T
// then stay in the last-level cache while its query heads run) and, inside a
// group, by decreasing tile count; the runs are dealt round-robin to the XCDs
// in that order, the blocks of a run in consecutive slots of one XCD
// (neighbouring query blocks select shifted copies of the same lag diagonals
// and the same columns, which then hit that XCD's L2).
// The dense path gives XCD x every 8th query-block row (last rows first) of
// every head.
#include <atomic>
#include <climits>
#include <type_traits>

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
  // acc + sum of the 8 elements (v_dot2_f32_bf16 against ones)
  static __device__ __forceinline__ float sum8(V8 p, float acc) {
    typedef __bf16 x2 __attribute__((ext_vector_type(2)));
    const x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2_f32_bf16(x2{p[2 * i], p[2 * i + 1]}, one, acc, false);
    return acc;
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
  static __device__ __forceinline__ float sum8(V8 p, float acc) {
    typedef _Float16 x2 __attribute__((ext_vector_type(2)));
    const x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(x2{p[2 * i], p[2 * i + 1]}, one, acc, false);
    return acc;
  }
};

constexpr int kD = 128;

// position of key k inside its 16-key group in the V^T layout (an involution)
__device__ __forceinline__ int vt_pos(int k) {
  const int q = (k >> 2) & 3;
  return (k & ~15) | (((q == 1) ? 2 : (q == 2) ? 1 : q) << 2) | (k & 3);
}

// ---- V -> V^T pre-pass: one workgroup per (b, hk, 64-key slab) -------------
// lb = 0: rows of Lp keys; lb = 16 or 32: blocks of lb keys, [Lp / lb][D][lb].
template <int D>
__global__ __launch_bounds__(256) void vt_kernel(const uint16_t* __restrict__ v, int64_t v_sb, int64_t v_sh,
                                                 int64_t v_sl, uint16_t* __restrict__ vt, int Hk, int Lk,
                                                 int Lp, int lb) {
  constexpr int CPR = D / 8;                     // 16-byte chunks per key row
  __shared__ uint16_t tile[64][D + 2];
  const int slabs = Lp / 64;
  const int bh = blockIdx.x / slabs, slab = blockIdx.x - bh * slabs;
  const int b = bh / Hk, hk = bh - b * Hk;
  const uint16_t* src = v + b * v_sb + hk * v_sh;
  uint16_t* dst = vt + (int64_t)bh * D * Lp;
  const int k0 = slab * 64;
  const int tid = threadIdx.x;
  for (int c = tid; c < 64 * CPR; c += 256) {
    const int r = c / CPR, cc = (c % CPR) * 8;
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
  // write D rows (d) x 64 keys: each thread emits 8 keys (16 bytes)
  for (int c = tid; c < D * 8; c += 256) {
    const int d = c >> 3, p0 = (c & 7) * 8;     // 8 stored positions p0 .. p0+7
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ka = vt_pos(p0 + 2 * e), kb = vt_pos(p0 + 2 * e + 1);
      w[e] = (uint32_t)tile[ka][d] | ((uint32_t)tile[kb][d] << 16);
    }
    const int k = k0 + p0;                       // 8 keys of one block (lb is a multiple of 8)
    const int64_t o = lb ? ((int64_t)(k / lb) * D + d) * lb + k % lb : (int64_t)d * Lp + k;
    *reinterpret_cast<uint4*>(dst + o) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---- main kernel -------------------------------------------------------------
// BS: query / key block size of the block lists; TK: keys per LDS tile
// (BS, or BS / 2 for two tiles per key block).
template <int BS, int TK, int D = kD>
struct AttnCfg {
  static constexpr int QW = BS / 32;          // query waves (32 queries each)
  // key groups: waves sharing the keys of a tile (2 or 1)
  static constexpr int KG = 2 * TK / BS;
  static constexpr int NW = QW * KG;          // waves
  static constexpr int NT = NW * 64;          // threads
  static constexpr int KH = TK / KG;          // keys per wave per tile
  static constexpr int KT = KH / 32;          // 32-key sub-tiles per wave
  static constexpr int TPB = BS >= TK ? BS / TK : 1;   // tiles per key block
  static constexpr int TILE = TK * D;         // elements of one K (or V^T) tile
  static constexpr int REGIONS = TILE * 2 / 1024;   // 1 KiB DMA regions per tile
  static constexpr int DMA_PER_WAVE = 2 * REGIONS / NW;
  static_assert(KG == 1 || KG == 2, "tile is a block or half a block");
};

// V^T row length: the key blocks, zero padded to whole 64-key slabs
__host__ __device__ inline int vt_len(int Nk, int bs) { return (Nk * bs + 63) / 64 * 64; }


// One 1 KiB global -> LDS copy per wave: lane l's 16 bytes land at lds_base + 16 l.
__device__ __forceinline__ void dma16(uint32_t lds_base, const void* gptr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_base), "v"(gptr) : "memory");
}
// Same, addressed as a wave-uniform base (scalar registers) plus a 32-bit lane offset.
__device__ __forceinline__ void dma16s(uint32_t lds_base, const void* sbase, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_base), "v"(voff), "s"(sbase) : "memory");
}

// Arguments of the main kernel: the subset of fs_attn_args it reads, with the
// per-row strides narrowed to 32 bits (checked on the host).
struct AttnKArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  uint16_t* out;
  const int32_t* blk_cnt;       // work order only (non-null: block masks given)
  const uint64_t* blk_bits;     // [Hq][Nq][NWk] block mask rows (64-token and longer blocks)
  const uint32_t* u_idx;        // union mode: [Hq][Nq][Nk] union entries (block | rows << 16)
  const int32_t* order;
  int64_t q_sb, q_sh, k_sb, k_sh, o_sb, o_sh;
  int q_sl, k_sl, o_sl;
  int Hq, Hk, Lq, Lk, Nq, Nk, NWk, Lp, total, is_causal;
  int run;                      // query blocks per scheduling unit (block lists)
  float scale;
  int gqa_interleave;           // KV head h % Hk (else h / (Hq / Hk))
  // dynamic assignment (block lists, null: the static one): ticket counters
  // [8 XCDs + 1 shared pool], zeroed by the order pass; the first
  // static_units units of the order are dealt to the XCDs round-robin, the
  // last pool_units are taken by whichever XCD asks first
  int32_t* ctr;
  int static_units, pool_units;
};

// 16-byte LDS operand at byte offset off of base
__device__ __forceinline__ uint4 lds16(const char* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(base + off);
}

// LB < BS (union mode, BS = 128): the block lists are at LB-token granularity
// and a workgroup covers BS / LB consecutive list rows (128 queries).  It walks
// the ascending union of their lists (union_kernel), each entry a key block
// with the set of the group's rows that selected it; a lane's scores of a key
// block its row did not select are masked.  A tile of TK keys holds TK / LB
// union entries, so every K / V^T tile copy serves 128 queries and every wave
// does 32 x TK per barrier, as with 128-token blocks.
template <int BS, int TK, typename T, int LB = BS, int D = kD>
__global__ __launch_bounds__((AttnCfg<BS, TK, D>::NT)) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bsattn_kernel(AttnKArgs a) {
  using C = AttnCfg<BS, TK, D>;
  static_assert(D == 64 || D == 128, "head dim 64 or 128");
  // K tiles: rows of D * 2 bytes, CPR 16-byte chunks each, chunk c of row r
  // stored at c ^ (r & SWM); a 1 KiB copy region holds RPR rows
  constexpr int ROWB = D * 2, CPR = D / 8, SWM = CPR - 1, RPR = 1024 / ROWB, LCPR = D == 128 ? 4 : 3;
  constexpr bool UNION = LB < BS;
  constexpr int EPT = UNION ? TK / LB : 1;         // union entries per tile
  static_assert(!UNION || (BS == 128 && TK == 64 && (LB == 16 || LB == 32)), "union mode: 16- or 32-token lists");
  using Ops = MfmaOps<T>;
  using V8 = typename Ops::V8;
  // [K | V^T][buffer] tiles; 256-byte rows with swizzled 16-byte chunks
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2][2][C::TILE];

  // Workgroup wg runs on XCD wg % 8.
  typedef const __attribute__((address_space(4))) uint32_t* cptr32;
  const int wg = blockIdx.x;
  const int x = wg & 7, slot = wg >> 3;
  const int g = a.Hq / a.Hk;
  int b, h, qb;
  if (a.order != nullptr) {
    // block lists: units of `run` consecutive query blocks of one head, in
    // decreasing tile count, dealt round-robin to the XCDs; a unit's query
    // blocks take consecutive slots of one XCD, so they run side by side and
    // share the K/V tiles of their (shifted) lag diagonals and columns in its L2
    int unit, j;
    if (a.ctr != nullptr) {
      // Dynamic assignment: the workgroup takes the next ticket of its XCD's
      // share (the share's units in order, `run` consecutive tickets per unit,
      // so a unit's query blocks still run side by side on one XCD); once the
      // share is used up, the next ticket of the shared pool (the shortest
      // units).  Measured per workgroup, the XCDs of one launch differ in
      // time per tile by up to 10%, and a static deal left the faster ones
      // idle for the last 5-10% of the kernel; the pool lets them take more.
      // Every ticket is taken exactly once; workgroups past the last ticket
      // return at once.
      __shared__ int pick[2];
      if (threadIdx.x == 0) {
        int u = -1, jj = 0;
        const int sx = a.static_units > x ? (a.static_units - x + 7) / 8 : 0;   // units x, x+8, .. of the share
        const int i = atomicAdd(&a.ctr[x], 1);
        if (i < sx * a.run) {
          u = a.order[(i / a.run) * 8 + x];
          jj = i % a.run;
        } else {
          const int t = atomicAdd(&a.ctr[8], 1);
          if (t < a.pool_units * a.run) {
            u = a.order[a.static_units + t / a.run];
            jj = t % a.run;
          }
        }
        pick[0] = u;
        pick[1] = jj;
      }
      __syncthreads();
      unit = __builtin_amdgcn_readfirstlane(pick[0]);
      j = __builtin_amdgcn_readfirstlane(pick[1]);
      if (unit < 0) return;
    } else {
      const int unit_slot = slot / a.run;
      j = slot - unit_slot * a.run;
      const int p = unit_slot * 8 + x;
      if (p >= a.total) return;                   // total = Hq * ceil(Nq / run) units
      unit = (int)((cptr32)(uintptr_t)a.order)[p];
    }
    const int nc = (a.Nq + a.run - 1) / a.run;
    b = 0;
    h = unit / nc;
    qb = (unit - h * nc) * a.run + j;
    if (qb >= a.Nq) return;
  } else {
    // dense: XCD x takes the query-block rows r = x, x + 8, ... (counted from
    // the last query block, so long rows start first) of every head; the heads
    // of one GQA group at one query block run back to back on one XCD and
    // share their K/V tiles in its L2
    const int r = x + 8 * (slot / a.Hq);
    if (r >= a.total) return;                     // total = B * Nq rows
    h = slot % a.Hq;
    b = r / a.Nq;
    qb = a.Nq - 1 - (r - b * a.Nq);
  }
  const int hk = a.gqa_interleave ? h % a.Hk : h / g;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar register)
  const int l32 = lane & 31, hi = lane >> 5;
  const int qq = wave % C::QW, kh = wave / C::QW;
  const int kbase = kh * C::KH;
  const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vtp = a.vt + (int64_t)(b * a.Hk + hk) * D * a.Lp;
  const int q0 = qb * BS;
  const int off = a.Lk - a.Lq;
  const int qw0 = q0 + qq * 32;                 // first query of this wave
  const int qrow = qw0 + l32;                   // this lane's query

  // Q^T fragments (B operand of S^T = K Q^T): dims st*16 + hi*8 .. +7
  V8 qf[D / 16];
#pragma unroll
  for (int st = 0; st < D / 16; ++st) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (qrow < a.Lq) raw = *reinterpret_cast<const uint4*>(qp + (int64_t)qrow * a.q_sl + st * 16 + hi * 8);
    qf[st] = __builtin_bit_cast(V8, raw);
  }

  // Block masks are read through the scalar unit (constant address space):
  // their completion is tracked by lgkmcnt, so reading the next word never
  // waits on the tile copies in flight (vmcnt).
  typedef const __attribute__((address_space(4))) uint64_t* cptr64;
  const bool listed = a.blk_cnt != nullptr;
  int64_t lbase = 0;
  int cnt;                                         // key tiles of this query block
  int nb_listed = 0;                               // union entries
  // Row mask walk (64- and 128-token blocks): the set bits of the row in
  // ascending order; it_cur holds the unread bits of word it_w.
  int64_t rbase = 0;
  int it_w = -1, it_blk = 0;
  uint64_t it_cur = 0;
  auto next_block = [&]() -> int {
    while (it_cur == 0 && it_w + 1 < a.NWk) it_cur = ((cptr64)(uintptr_t)a.blk_bits)[rbase + ++it_w];
    if (it_cur == 0) return a.Nk;                  // past the row (not reached: cnt counts the bits)
    const int b = __builtin_ctzll(it_cur);
    it_cur &= it_cur - 1;
    return 64 * it_w + b;
  };
  if (UNION && listed) {
    // the group's union list: 32-bit entries (block | rows << 16), no trim
    const int nb = min(max((int)((cptr32)(uintptr_t)a.blk_cnt)[(int64_t)h * a.Nq + qb], 0), a.Nk);
    lbase = ((int64_t)h * a.Nq + qb) * a.Nk;
    cnt = (nb + EPT - 1) / EPT;
    nb_listed = nb;
  } else if (listed) {
    // the selected blocks up to the causal limit (blocks kb with kb * BS <=
    // the last visible key) and below Nk: the row's words counted lane-parallel
    rbase = ((int64_t)h * a.Nq + qb) * a.NWk;
    const int last_key = q0 + BS - 1 + off;
    const int kb_lim = !a.is_causal ? a.Nk : (last_key < 0 ? 0 : min(a.Nk, last_key / BS + 1));
    const int nwl = (kb_lim + 63) >> 6;
    int c = 0;
    for (int w = lane; w < nwl; w += 64) {
      uint64_t x = a.blk_bits[rbase + w];
      if (w == nwl - 1 && (kb_lim & 63)) x &= (1ull << (kb_lim & 63)) - 1;
      c += __popcll(x);
    }
    const int nb = __builtin_amdgcn_readfirstlane(wave_sum_i(c));
    cnt = nb * C::TPB;
  } else {
    const int last_key = a.is_causal ? min(a.Lk - 1, q0 + BS - 1 + off) : a.Lk - 1;
    cnt = last_key < 0 ? 0 : last_key / TK + 1;
  }
  // first key of tile t (-1: an out-of-range entry, skipped)
  const int nlisted = nb_listed;
  auto uent = [&](int i) -> uint32_t {            // union entry i, all ones past the end
    if (i >= nlisted) return 0xffffffffu;
    return ((cptr32)(uintptr_t)a.u_idx)[lbase + i];
  };
  // Union mode: the entries of tiles t, t+1 and t+2 are held in scalar
  // registers (u0, u1, u2) and those of tile t+3 are loaded during iteration
  // t, so neither a copy nor a mask waits on a list load.
  struct TileEnt {
    uint32_t e[EPT];
  };
  TileEnt u0{}, u1{}, u2{}, u3{};
  auto load_tile = [&](int t) -> TileEnt {
    TileEnt u;
#pragma unroll
    for (int ie = 0; ie < EPT; ++ie) u.e[ie] = uent(t * EPT + ie);
    return u;
  };
  auto key_of = [&](int t) -> int {
    if constexpr (UNION) {
      if (listed) return t;                        // union mode: copies and masks look the tile's entries up
    }
    if (!listed) return t * TK;
    // called for t = 0, 1, 2, ... in order: a new block every TPB tiles
    if (t % C::TPB == 0) it_blk = next_block();
    return it_blk < a.Nk ? it_blk * BS + (t % C::TPB) * TK : -1;
  };

  // ---- tile DMA: wave w copies 1 KiB regions w*NR .. w*NR+NR-1 of the K tile
  // and of the V^T tile.  koff / voff are this lane's byte offsets inside a
  // K / V^T tile in global memory (fixed for the loop); each copy adds them to
  // a wave-uniform tile origin held in scalar registers.
  constexpr int NR = C::DMA_PER_WAVE / 2;
  uint32_t koff[NR], voff[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int R = wave * NR + i;                   // region R of the K tile and of the V^T tile
    const int r = 4 * R + (lane >> 4);             // V^T: 256-byte LDS rows 4R .. 4R+3
    const int c = (lane & 15) ^ (r & 15);
    int rk = r, ck = c;                            // K: rows RPR R .. RPR R + RPR - 1
    if constexpr (D != 128) {
      rk = RPR * R + (lane >> LCPR);
      ck = (lane & SWM) ^ (rk & SWM);
    }
    if constexpr (UNION) {
      // K rows relative to this wave's 16 rows of the tile; V^T: the key
      // offset of the lane's 8 keys inside their union entry
      koff[i] = (uint32_t)((rk - wave * RPR * NR) * a.k_sl + ck * 8) * 2u;
      voff[i] = (uint32_t)((2 * r + (c >> 3)) * LB + (((c & 7) * 8) % LB)) * 2u;   // V^T stored block by block
    } else {
      koff[i] = (uint32_t)(rk * a.k_sl + ck * 8) * 2u;
      voff[i] = (TK == 128 ? (uint32_t)(r * a.Lp + c * 8)                          // d = r
                           : (uint32_t)((2 * r + (c >> 3)) * a.Lp + (c & 7) * 8))  // two d rows per LDS row
                * 2u;
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&lds[0][0][0]);
  auto issue_k = [&](int key0, int buf, TileEnt ue) {
    const uint32_t lk = lds0 + (uint32_t)(buf * C::TILE * 2 + wave * NR * 1024);
    if constexpr (UNION) {
      if (listed) {
        // key0 is the tile index, ue its entries: this wave's 16 rows belong to entry 16 wave / LB
        const int wsel = (16 * wave) / LB;
        uint32_t es = ue.e[0];
#pragma unroll
        for (int ie = 1; ie < EPT; ++ie) es = wsel == ie ? ue.e[ie] : es;
        const uint32_t e = __builtin_amdgcn_readfirstlane(es);   // wave-uniform: the copy base is scalar
        const int blk = (int)(e & 0xffffu);
        key0 = blk < a.Nk ? blk * LB + (16 * wave) % LB : -1;
      }
    }
    if constexpr (UNION) {
      // this wave's 16 rows of the tile from key0
      const int kc = min(max(key0, 0), a.Lk - 1);
      const uint16_t* base = kp + (int64_t)kc * a.k_sl;
      if (key0 >= 0 && key0 + RPR * NR <= a.Lk) {
#pragma unroll
        for (int i = 0; i < NR; ++i) dma16s(lk + i * 1024, base, koff[i]);
      } else {
        // rows past Lk (or of a missing block) read row Lk-1 instead (their scores are masked)
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const int rr = RPR * i + (ln >> LCPR);     // row within this wave's block
          const int c = (ln & SWM) ^ ((RPR * (wave * NR + i) + (ln >> LCPR)) & SWM);
          dma16s(lk + i * 1024, base, (uint32_t)(min(rr, a.Lk - 1 - kc) * a.k_sl + c * 8) * 2u);
        }
      }
      return;
    }
    if (key0 >= 0 && key0 + TK <= a.Lk) {
      const uint16_t* base = kp + (int64_t)key0 * a.k_sl;
#pragma unroll
      for (int i = 0; i < NR; ++i) dma16s(lk + i * 1024, base, koff[i]);
    } else {
      // a tile reaching past Lk, or an out-of-range entry: rows past Lk read
      // row Lk-1 instead (their scores are masked)
      const int kc = min(max(key0, 0), a.Lk - 1);
      const uint16_t* base = kp + (int64_t)kc * a.k_sl;
      int ln = lane;
      asm volatile("" : "+v"(ln));                 // keep this rare path's offsets out of the loop preheader
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const int r = RPR * (wave * NR + i) + (ln >> LCPR);
        const int c = (ln & SWM) ^ (r & SWM);
        dma16s(lk + i * 1024, base, (uint32_t)(min(r, a.Lk - 1 - kc) * a.k_sl + c * 8) * 2u);
      }
    }
  };
  auto issue_v = [&](int key0, int buf, TileEnt ue) {
    const uint32_t lv = lds0 + (uint32_t)((2 + buf) * C::TILE * 2 + wave * NR * 1024);
    if constexpr (UNION) {
      if (listed) {
        // key0 is the tile index; lane chunk c holds keys of entry ((c & 7) * 8) / LB
        uint32_t ek[EPT];
#pragma unroll
        for (int ie = 0; ie < EPT; ++ie) {
          const int blk = (int)(ue.e[ie] & 0xffffu);
          ek[ie] = (uint32_t)(blk < a.Nk ? blk * D * LB : 0) * 2u;
        }
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const int r = 4 * (wave * NR + i) + (lane >> 4);
          const int c = (lane & 15) ^ (r & 15);
          const int sel = ((c & 7) * 8) / LB;
          uint32_t k = ek[0];
#pragma unroll
          for (int ie = 1; ie < EPT; ++ie) k = sel == ie ? ek[ie] : k;
          dma16s(lv + i * 1024, vtp, voff[i] + k);
        }
        return;
      }
    }
    const uint16_t* base = vtp + max(key0, 0);     // V^T is zero padded to Lp
#pragma unroll
    for (int i = 0; i < NR; ++i) dma16s(lv + i * 1024, base, voff[i]);
  };

  // MFMA operand addressing.  A lane reads row l32 of a group of 32 rows and
  // chunk hi of a pair of 16-byte chunks.  The swizzle XORs the chunk with
  // (row & 15); the group origin R0 is a multiple of 16 and the pair origin C0
  // is even, so the operand at (R0, C0) of a tile is at byte
  //   tile + R0 * 256 + (lane_off ^ (C0 << 4)),   lane_off = l32 * 256 + ((hi ^ (l32 & 15)) << 4).
  // For V^T tiles of 64 keys an LDS row holds two d rows (d = 2 r + (chunk >> 3)):
  // the lane's d row dt * 32 + l32 sits in LDS row dt * 16 + (l32 >> 1), chunk
  // (l32 & 1) * 8 + C0 + hi.
  const uint32_t lane_off = (uint32_t)(l32 * ROWB + ((hi ^ (l32 & SWM)) << 4));   // K tile rows
  const uint32_t lane_off_vr = (uint32_t)(l32 * 256 + ((hi ^ (l32 & 15)) << 4));   // 256-byte V^T rows
  const uint32_t lane_off_v =
      TK == 128 ? lane_off_vr
                : (uint32_t)((l32 >> 1) * 256 + (((((l32 & 1) << 3) | hi) ^ (l32 >> 1)) << 4));
  constexpr int VROW = TK == 128 ? 32 * 256 : 16 * 256;   // bytes per 32 d rows of V^T

  // Running max (per query row) is kept in the exp2 domain of raw scores
  // times sc; it is only raised (and O rescaled) when a new score exceeds it
  // by more than 2^8, so p = 2^(s*sc - m) <= 256 and most tiles skip the rescale.
  const float sc = a.scale * 1.44269504088896340736f;
  constexpr float kSlack = 8.0f;
  // Split tiles (block 64, two key groups of 16 MFMAs per wave) take their
  // exponentials against the running max with no row max: a tile whose row
  // sum exceeds 2^64 (or is inf / nan, as on a row's first tile) is redone
  // with the raised max.  Against the row max: C3a -4.6%; at block 128 (32
  // MFMAs per wave) the row max is kept, the other form measured 3.5% slower.
  constexpr bool kRowMax = C::KG == 1;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16_t o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;

  // S^T = K Q^T for this wave's keys of the K tile in buffer kbuf
  auto compute_s = [&](int kbuf, f32x16_t* s) {
    const char* kt_base = reinterpret_cast<const char*>(lds[0][kbuf]) + kbase * ROWB;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      const uint32_t lo = lane_off ^ (uint32_t)(st << 5);
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt) {
        const V8 ka = __builtin_bit_cast(V8, lds16(kt_base + kt * 32 * ROWB, lo));
        s[kt] = Ops::mma(ka, qf[st], s[kt]);
      }
    }
  };
  // whether any key of this wave's half of tile kb is visible to its queries
  auto active_for = [&](int key0) {
    const int kw0 = key0 + kbase;
    return key0 >= 0 && kw0 < a.Lk && !(a.is_causal && kw0 > qw0 + 31 + off);
  };

  // Masking (diagonal / partial / invisible half tiles only) of the tile kb
  // whose scores are in s; the running max is taken later, beside the
  // exponentials of that tile.
  auto mask_only = [&](int key0, f32x16_t* s, TileEnt ue) {
    if constexpr (UNION) {
      if (listed) {
        // key0 is the tile index.  Lane row jq of the group; a key of entry ie
        // is kept iff the entry is real, row jq selected it, and it is below Lk
        // and (causal) at or before the lane's query.  Fast path: every row of
        // this wave selected every entry and no key needs the causal / Lk cut.
        const int jq = (qq * 32 + l32) / LB;
        constexpr uint32_t kWaveRows = (1u << (32 / LB)) - 1;
        const uint32_t wrows = kWaveRows << ((qq * 32) / LB);
        uint32_t ents[EPT];
        bool full = true;
#pragma unroll
        for (int ie = 0; ie < EPT; ++ie) {
          ents[ie] = ue.e[ie];
          const int blk = (int)(ents[ie] & 0xffffu);
          if (blk >= a.Nk || ((ents[ie] >> 16) & wrows) != wrows || blk * LB + LB > a.Lk ||
              (a.is_causal && blk * LB + LB - 1 > qw0 + off))
            full = false;
        }
        if (!full) {
#pragma unroll
          for (int ie = 0; ie < EPT; ++ie) {
            const int blk = (int)(ents[ie] & 0xffffu);
            const bool mine = blk < a.Nk && ((ents[ie] >> (16 + jq)) & 1u);
            int lim = a.Lk - blk * LB;
            if (a.is_causal) lim = min(lim, qrow + off - blk * LB + 1);
            lim = mine ? lim - hi * 4 : INT_MIN;
            // registers of entry ie: sub-tile kt = ie * LB / 32, and at LB = 16 the half r >> 3
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kt = (ie * LB) / 32;
              if (LB == 16 && (r >> 3) != (ie & 1)) continue;
              const int local = (((r >> 2) * 8) % LB) + (r & 3);
              if (local >= lim) s[kt][r] = -INFINITY;
            }
          }
        }
        return;
      }
    }
    const int kw0 = key0 + kbase;
    const bool act = active_for(key0);
    if (!act || (kw0 + C::KH > a.Lk) || (a.is_causal && kw0 + C::KH - 1 > qw0 + off)) {
      int lim = a.Lk - kw0 - hi * 4;
      if (a.is_causal) lim = min(lim, qrow + off - kw0 - hi * 4 + 1);
      if (!act) lim = INT_MIN;
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = kt * 32 + (r >> 2) * 8 + (r & 3);
          if (c >= lim) s[kt][r] = -INFINITY;
        }
    }
  };
  // P = 2^(s sc - m) with m = m_use, packed to the MFMA input type; returns
  // the row sum of the rounded P over this lane's keys
  auto exp_part = [&](const f32x16_t* s, V8* pb, float m_use) -> float {
    float rs = 0.f;
#pragma unroll
    for (int kk = 0; kk < C::KH / 16; ++kk) {
      const int kt = kk >> 1, half = kk & 1;
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][8 * half + j], sc, -m_use));
      pb[kk] = Ops::pack(pv);
      rs = Ops::sum8(pb[kk], rs);
    }
    return rs;
  };
  // v and the value of the lane 32 apart (the same query's other keys): one
  // v_permlane32_swap, both operand orders identical in the two halves
  auto halves = [](float v, float& lo, float& hi_) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(r[0]);
    hi_ = __uint_as_float(r[1]);
  };
  auto row_max = [&](const f32x16_t* s) -> float {
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][r]);
    return mx;
  };
  // O^T += V^T P^T for the V^T tile in buffer vbuf
  auto pv_mma = [&](int vbuf, const V8* pb) {
    const char* vt_base = reinterpret_cast<const char*>(lds[1][vbuf]);
#pragma unroll
    for (int kk = 0; kk < C::KH / 16; ++kk) {
      const uint32_t lo = lane_off_v ^ (uint32_t)(((kbase >> 3) + 2 * kk) << 4);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const V8 va = __builtin_bit_cast(V8, lds16(vt_base + dt * VROW, lo));
        o[dt] = Ops::mma(va, pb[kk], o[dt]);
      }
    }
  };
  auto scale_o = [&](float alpha) {
    if (alpha != 1.0f) {                             // per query row (lane); rare
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
  };
  // Pipeline with P V deferred by one tile.  Iteration t: wait for K(t+1)
  // and V(t-1), one barrier, copy K(t+2) (into the buffer of K(t)) and V(t)
  // (into that of V(t-2)); then one straight-line block with S(t+1) and
  // P V(t-1) on the MFMA pipe interleaved with the row max, running-max raise
  // and exponentials of tile t on the VALU (independent work); then the O
  // rescale of a raise (rare) and the masking of tile t+1 (diagonal and
  // partial tiles only).
  f32x16_t sa[C::KT], sb[C::KT];
  V8 pa[C::KH / 16], pb[C::KH / 16];
  int kb0 = 0, kb1 = 0, kb2 = 0;                   // first keys of tiles t, t+1, t+2
  typedef std::integral_constant<bool, true> yes;
  typedef std::integral_constant<bool, false> no;
  auto iter = [&](int t, f32x16_t* s_next, f32x16_t* s_cur, V8* p_prev, V8* p_cur, auto hasS, auto hasPV,
                  auto hasE) {
    // a wave waiting here yields issue priority to the other workgroup's
    // wave on its SIMD, which is in its MFMA block (priority raised below)
    __builtin_amdgcn_s_setprio(0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (t + 2 < cnt) {
      kb2 = key_of(t + 2);
      issue_k(kb2, t & 1, u2);
    }
    if (t < cnt) issue_v((UNION && listed) ? t : kb0, t & 1, u0);
    if constexpr (UNION) {
      if (listed) u3 = load_tile(t + 3);
    }
    __builtin_amdgcn_s_setprio(2);
    // The row max of tile t, the raise of the running max and the
    // exponentials of tile t are VALU work independent of the MFMAs of S(t+1)
    // and P V(t-1), so all of it goes into the interleaved block; only the
    // rescale of O, which must follow P V(t-1), is left after it (rare).
    float rs = 0.f, al = 1.0f;
    if constexpr (decltype(hasS)::value) compute_s((t + 1) & 1, s_next);
    if constexpr (decltype(hasPV)::value) pv_mma((t - 1) & 1, p_prev);
    if constexpr (decltype(hasE)::value) {
      if constexpr (kRowMax) {
        float mx = row_max(s_cur), m0, m1;
        halves(mx, m0, m1);
        mx = fmaxf(m0, m1) * sc;
        // a row raises its running max only when a score exceeds it by more than the slack
        const bool up = mx > m_run + kSlack;
        al = up ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;
        m_run = up ? mx : m_run;
        rs = exp_part(s_cur, p_cur, m_run == -INFINITY ? 0.f : m_run);
      } else {
        // exponentials against the running max with no row max; a row whose
        // sum overflows (or the first tile, m_run = -inf: inf / nan) is redone below
        rs = exp_part(s_cur, p_cur, m_run);
      }
    }
    if constexpr (decltype(hasS)::value && decltype(hasPV)::value && decltype(hasE)::value) {
      // Steady state: the scheduler interleaves one MFMA with three VALU
      // instructions (a wave issues in order, so MFMAs issued back to back
      // would hold its exponentials until the last one), the LDS operand
      // reads running six MFMAs ahead (measured best of 2 .. 8; three VALU
      // per MFMA against two: C2 -2.4%, C3a -4.6%, C3b -1.5%).
      constexpr int NM = C::KT * (D / 16) + (C::KH / 16) * (D / 32);
      constexpr int LA = 6;
      constexpr int VPM = 3;
      __builtin_amdgcn_sched_group_barrier(0x100, LA, 0);        // DS reads
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
        if (i + LA < NM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);     // VALU
      }
    }
    if constexpr (decltype(hasE)::value) {
      float r0, r1;
      halves(rs, r0, r1);
      if constexpr (kRowMax) {
        l_run = l_run * al + (r0 + r1);
        if (__builtin_amdgcn_ballot_w64(al != 1.0f) != 0) scale_o(al);   // O holds P V up to t-1 now
      } else {
        float tot = r0 + r1;
        const bool bad = !(tot <= 0x1p64f);            // p above 2^64 somewhere, inf or nan
        if (__builtin_amdgcn_ballot_w64(bad) != 0) {   // rare: the row's max, raised running max, exps again
          // the first pass's P stays defined before the branch (else its packing sinks out of the MFMA block)
#pragma unroll
          for (int kk = 0; kk < C::KH / 16; ++kk) asm volatile("" : "+v"(p_cur[kk]));
          float mx = row_max(s_cur), m0, m1;
          halves(mx, m0, m1);
          mx = fmaxf(m0, m1) * sc;
          const float mnew = bad ? fmaxf(m_run, mx) : m_run;
          al = (!bad || m_run == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run - mnew);
          m_run = mnew;
          rs = exp_part(s_cur, p_cur, m_run == -INFINITY ? 0.f : m_run);
          halves(rs, r0, r1);
          tot = r0 + r1;
          scale_o(al);                                 // O holds P V up to t-1 now
        }
        l_run = l_run * al + tot;
      }
    }
    if constexpr (decltype(hasS)::value) mask_only(kb1, s_next, u1);
    kb0 = kb1;
    kb1 = kb2;
    if constexpr (UNION) {
      u0 = u1;
      u1 = u2;
      u2 = u3;
    }
  };
  // The first two K tiles are requested before the Q loads are waited for,
  // so the two latencies overlap; one wait then retires both (the loop's own
  // waits then find no register load of Q outstanding).
  if constexpr (UNION) {
    if (listed) {
      u0 = load_tile(0);
      u1 = load_tile(1);
      u2 = load_tile(2);
    }
  }
  if (cnt > 0) {
    kb0 = key_of(0);
    issue_k(kb0, 0, u0);
    if (cnt > 1) {
      kb1 = key_of(1);
      issue_k(kb1, 1, u1);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (cnt > 0) {
    __builtin_amdgcn_s_barrier();
    compute_s(0, sa);
    mask_only(kb0, sa, u0);
    // t = 0: S(1) if it exists, exponentials of tile 0, no P V yet
    if (cnt > 1) iter(0, sb, sa, pb, pa, yes(), no(), yes());
    else iter(0, sb, sa, pb, pa, no(), no(), yes());
    int t = 1;
    for (; t + 2 < cnt; t += 2) {                    // steady state: t and t+1 both have S(t+1)
      iter(t, sa, sb, pa, pb, yes(), yes(), yes());
      iter(t + 1, sb, sa, pb, pa, yes(), yes(), yes());
    }
    // remaining iterations t .. cnt: at most one more steady step, the last
    // tile (no S(t+1)) and the final P V
    if (t + 1 < cnt) {                               // t odd, t+1 = cnt-1 even
      iter(t, sa, sb, pa, pb, yes(), yes(), yes());
      iter(t + 1, sb, sa, pb, pa, no(), yes(), yes());
      iter(t + 2, sa, sb, pa, pb, no(), yes(), no());
    } else if (t < cnt) {                            // t = cnt-1, odd
      iter(t, sa, sb, pa, pb, no(), yes(), yes());
      iter(t + 1, sb, sa, pb, pa, no(), yes(), no());
    } else {                                         // t = cnt (cnt == 1): the final P V
      iter(t, sa, sb, pa, pb, no(), yes(), no());
    }
  }
  // ---- merge the two key halves through LDS (split tiles), normalise, store
  float f0 = 1.0f, f1 = 0.0f, l = l_run;
  constexpr int PER = (D / 32) * 16 + 2;
  const float* src = reinterpret_cast<const float*>(&lds[0][0][0]) + (size_t)qq * PER * 64;   // [QW][PER][64]
  if constexpr (C::KG == 2) {
    __syncthreads();
    if (kh == 1) {
      float* dst = reinterpret_cast<float*>(&lds[0][0][0]) + (size_t)qq * PER * 64;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(dt * 16 + r) * 64 + lane] = o[dt][r];
      dst[(PER - 2) * 64 + lane] = m_run;
      dst[(PER - 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (kh == 1 || qrow >= a.Lq) return;
    const float m1 = src[(PER - 2) * 64 + lane];
    const float l1 = src[(PER - 1) * 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float mu = m == -INFINITY ? 0.f : m;
    f0 = __builtin_amdgcn_exp2f(m_run - mu);
    f1 = __builtin_amdgcn_exp2f(m1 - mu);
    l = l_run * f0 + l1 * f1;
  }
  if (qrow >= a.Lq) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t* op = a.out + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_sl;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = g4 * 4 + e;
        float acc = o[dt][r] * f0;
        if constexpr (C::KG == 2) acc += src[(dt * 16 + r) * 64 + lane] * f1;
        v4[e] = acc * inv;
      }
      const int d0 = dt * 32 + g4 * 8 + hi * 4;
      uint2 w;
      w.x = (uint32_t)Ops::bits(v4[0]) | ((uint32_t)Ops::bits(v4[1]) << 16);
      w.y = (uint32_t)Ops::bits(v4[2]) | ((uint32_t)Ops::bits(v4[3]) << 16);
      *reinterpret_cast<uint2*>(op + d0) = w;
    }
}

// ---- order of the scheduling units (run consecutive query blocks of one
// head): KV group by KV group, and inside a group longest first.  One KV
// head's K and V^T (64 MiB at L = 131072) then stay in the last-level cache
// while its query heads run, instead of every KV head's streaming at once.
// Counting sort of key = hk * nbc + (nbc - 1 - (tile count >> shift)).
constexpr int kOrderThreads = 1024;
constexpr int kTicketCounters = 9;               // 8 XCD shares + the shared pool
constexpr int kPoolPercent = 10;                 // share of the work units (the shortest) in the shared pool
constexpr int kOrderMaxBins = 8192;
constexpr int kOrderKeysPerThread = 8;           // keys kept in registers between the two passes
// kvmajor = 0: one longest-first order over all units (the KV group left out of the key).
__global__ __launch_bounds__(kOrderThreads) void order_kernel(const int32_t* __restrict__ cnt, int Hq, int Hk,
                                                              int gqa_interleave, int Nq, int run, int Nk, int shift,
                                                              int32_t* __restrict__ order, int kvmajor,
                                                              int32_t* __restrict__ ctr) {
  __shared__ int hist[kOrderMaxBins];
  if (ctr != nullptr && threadIdx.x < kTicketCounters) ctr[threadIdx.x] = 0;   // the attention kernel's tickets
  __shared__ int part[kOrderThreads];
  const int tid = threadIdx.x;
  const int nc = (Nq + run - 1) / run;
  const int units = Hq * nc;
  const int g = Hq / Hk;
  const int nbc = ((run * Nk) >> shift) + 1;       // count bins 0 .. (run Nk) >> shift
  const int nb = Hk * nbc;                         // keys
  auto key_of = [&](int u) {
    const int h = u / nc, q0 = (u - h * nc) * run;
    const int32_t* c0 = cnt + (int64_t)h * Nq + q0;
    const int n = min(run, Nq - q0);
    // the count loads of a unit are issued together (16 at a time), then added
    int c = 0;
    for (int j0 = 0; j0 < n; j0 += 16) {
      int v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = j0 + j < n ? c0[j0 + j] : 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) c += min(max(v[j], 0), Nk);
    }
    const int hk = kvmajor ? (gqa_interleave ? h % Hk : h / g) : 0;
    return hk * nbc + (nbc - 1 - (c >> shift));
  };
  // this thread's units u = tid + k * kOrderThreads; their keys stay in registers
  // when there are at most kOrderKeysPerThread of them, else they are formed again
  const bool held = units <= kOrderKeysPerThread * kOrderThreads;
  int keys[kOrderKeysPerThread];
#pragma unroll
  for (int k = 0; k < kOrderKeysPerThread; ++k) {
    const int u = tid + k * kOrderThreads;
    keys[k] = (held && u < units) ? key_of(u) : 0;
  }
  for (int i = tid; i < nb; i += kOrderThreads) hist[i] = 0;
  __syncthreads();
  if (held) {
#pragma unroll
    for (int k = 0; k < kOrderKeysPerThread; ++k)
      if (tid + k * kOrderThreads < units) atomicAdd(&hist[keys[k]], 1);
  } else {
    for (int u = tid; u < units; u += kOrderThreads) atomicAdd(&hist[key_of(u)], 1);
  }
  __syncthreads();
  // start[k] = number of units with a smaller key: thread tid scans keys tid*per ..
  const int per = (nb + kOrderThreads - 1) / kOrderThreads;
  const int k0 = tid * per;
  int local = 0;
  for (int k = 0; k < per; ++k)
    if (k0 + k < nb) local += hist[k0 + k];
  part[tid] = local;
  __syncthreads();
  for (int off = 1; off < kOrderThreads; off <<= 1) {   // inclusive scan of chunk sums
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int acc = part[tid] - local;                     // exclusive prefix of this chunk
  for (int k = 0; k < per; ++k) {
    if (k0 + k < nb) {
      const int h = hist[k0 + k];
      hist[k0 + k] = acc;
      acc += h;
    }
  }
  __syncthreads();
  if (held) {
#pragma unroll
    for (int k = 0; k < kOrderKeysPerThread; ++k) {
      const int u = tid + k * kOrderThreads;
      if (u < units) order[atomicAdd(&hist[keys[k]], 1)] = u;
    }
  } else {
    for (int u = tid; u < units; u += kOrderThreads) order[atomicAdd(&hist[key_of(u)], 1)] = u;
  }
}

// ---- union lists of groups of R consecutive mask rows (union mode) -------
// One wave per (head, group): the rows' mask words in LDS (lane l: words l and
// l + 64, blocks 64 w .. 64 w + 63), their OR word by word, a prefix of the
// popcounts, and the union written in ascending order as
// block | (rows that selected it) << 16.  Nk <= 8192, R <= 8.
constexpr int kUnionMaxRows = 8;
__global__ __launch_bounds__(64) void union_kernel(const uint64_t* __restrict__ mask, int Nq, int Nk, int R, int Ng,
                                                   int32_t* __restrict__ u_cnt, uint32_t* __restrict__ u_idx) {
  constexpr int kW = 2 * 64;                       // words per row: Nk <= 8192
  __shared__ unsigned long long bits[kUnionMaxRows][kW];
  const int h = blockIdx.x / Ng, grp = blockIdx.x - h * Ng;
  const int lane = threadIdx.x;
  const int NW = (Nk + 63) >> 6;
  // words past Nk's last word, and rows past Nq, are empty
  for (int j = 0; j < kUnionMaxRows; ++j) {
    const int row = grp * R + j;
    const uint64_t* mr = mask + ((int64_t)h * Nq + row) * NW;
    const bool ok = j < R && row < Nq;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int w = lane + 64 * k;
      uint64_t x = (ok && w < NW) ? mr[w] : 0ull;
      if (w == NW - 1 && (Nk & 63)) x &= (1ull << (Nk & 63)) - 1;
      bits[j][w] = x;
    }
  }
  __syncthreads();
  unsigned long long any0 = 0ull, any1 = 0ull;
  for (int j = 0; j < R; ++j) {
    any0 |= bits[j][lane];
    any1 |= bits[j][lane + 64];
  }
  const int c0 = __popcll(any0), c1 = __popcll(any1);
  int i0 = c0, i1 = c1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v0 = __shfl_up(i0, o, 64), v1 = __shfl_up(i1, o, 64);
    if (lane >= o) {
      i0 += v0;
      i1 += v1;
    }
  }
  const int t0 = __shfl(i0, 63, 64);
  const int total = t0 + __shfl(i1, 63, 64);
  uint32_t* out = u_idx + ((int64_t)h * Ng + grp) * Nk;
  // entry: block | (rows of the group that selected it) << 16
  auto entry = [&](int wd, int b) -> uint32_t {
    uint32_t rows = 0;
    for (int j = 0; j < R; ++j) rows |= (uint32_t)((bits[j][wd] >> b) & 1ull) << j;
    return (uint32_t)(64 * wd + b) | (rows << 16);
  };
  if ((Nk & 3) == 0 && ((uintptr_t)u_idx & 15) == 0) {
    // 16-byte stores of 4 entries
    __shared__ uint64_t stw[kW];
    __shared__ int stp[kW];
    stw[lane] = any0;
    stp[lane] = i0 - c0;
    stw[lane + 64] = any1;
    stp[lane + 64] = t0 + i1 - c1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    list_chunks_from_lds(out, total, kW, lane, 64, stw, stp, entry);
  } else {
    int pos = i0 - c0;
    for (unsigned long long m = any0; m; m &= m - 1) out[pos++] = entry(lane, __builtin_ctzll(m));
    pos = t0 + i1 - c1;
    for (unsigned long long m = any1; m; m &= m - 1) out[pos++] = entry(lane + 64, __builtin_ctzll(m));
  }
  if (lane == 0) u_cnt[(int64_t)h * Ng + grp] = total;
}

// Work units go KV group by KV group (one KV head's K and V^T then stay in
// the last-level cache while its query heads run) when a group's workgroups
// fill at least 4 rounds of the device's workgroup slots (two per CU);
// with fewer, the group boundaries leave partly filled rounds and one
// longest-first order over all units balances better (config 1: 2 rounds
// per group, attention 2.03 -> 1.90 ms; configs 2 and 3 have 7 to 14 and
// keep the grouped order, 2.2% and 0.8% faster with it).
static int kv_major(const fs_attn_args& a, int Nq) {
  // CU count per device, read once; host threads may race to fill an entry,
  // so it is atomic (they store the same value)
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 1;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  const int64_t per_group = (int64_t)(a.Hq / a.Hk) * Nq;   // workgroups of one KV group
  return per_group >= 4 * 2 * (int64_t)n ? 1 : 0;
}

static size_t vt_bytes(const fs_attn_args& a) {
  const int Nk = (a.Lk + a.bs - 1) / a.bs;
  return ((size_t)a.B * a.Hk * a.D * vt_len(Nk, a.bs) * 2 + 255) & ~(size_t)255;
}
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
// workspace after V^T: the order [Hq * Nq] (+ union mode: u_cnt [Hq * Ng], u_idx [Hq * Ng * Nk])
static size_t order_bytes(const fs_attn_args& a) {
  const int64_t Nq = (a.Lq + a.bs - 1) / a.bs;
  return align256((size_t)a.Hq * Nq * sizeof(int32_t)) + 256;   // + the ticket counters
}
// Ticket assignment of `total` ordered work units of `run` workgroups: the
// last kPoolPercent% of the units (the shortest) form the shared pool, XCD x's
// share is units x, x+8, .. of the rest.  Each XCD gets enough workgroups for
// its share and twice its even part of the pool; the ones that find no ticket
// left return at once.  Returns the grid.
static unsigned deal_units(int total, int run, int& static_units, int& pool_units) {
  pool_units = (int)((int64_t)total * kPoolPercent / 100);
  static_units = total - pool_units;
  const int64_t per_xcd = (int64_t)(static_units + 7) / 8 * run + 2 * (((int64_t)pool_units * run + 7) / 8);
  return (unsigned)(8 * per_xcd);
}
static int32_t* ticket_counters(const fs_attn_args& a) {
  const int64_t Nq = (a.Lq + a.bs - 1) / a.bs;
  return reinterpret_cast<int32_t*>(static_cast<char*>(a.work) + vt_bytes(a) +
                                    align256((size_t)a.Hq * Nq * sizeof(int32_t)));
}
static bool union_mode(const fs_attn_args& a) { return a.blk_cnt != nullptr && a.bs < 64; }
static int union_groups(const fs_attn_args& a) {
  const int Nq = (a.Lq + a.bs - 1) / a.bs;
  const int R = 128 / a.bs;
  return (Nq + R - 1) / R;
}

// order pass (block lists only) and the main kernel, reading V^T from the workspace
template <int BS, int TK, typename T, int D>
static int launch_run(const fs_attn_args& a, int Nq, int Nk, hipStream_t s, int Lp = 0) {
  if (Lp == 0) Lp = vt_len(Nk, BS);                // else: V^T laid out for another block size
  const uint16_t* vt = static_cast<const uint16_t*>(a.work);
  int32_t* order = nullptr;
  int32_t* ctr = nullptr;
  int static_units = 0, pool_units = 0;
  int total;
  unsigned grid;
  // Scheduling units of `run` consecutive query blocks: at C2 (Nq = 1024) a
  // run of 16 halves the K/V bytes fetched beyond L2 (166 -> 83 GB) and
  // still leaves 2048 units for longest-first balance over 256 CUs.
  const int run = min(16, max(1, Nq / 64));
  if (a.blk_cnt) {
    int shift = 0;
    while ((int64_t)a.Hk * (((run * Nk) >> shift) + 1) > kOrderMaxBins) ++shift;
    order = reinterpret_cast<int32_t*>(static_cast<char*>(a.work) + vt_bytes(a));
    total = a.Hq * ((Nq + run - 1) / run);
    ctr = ticket_counters(a);
    order_kernel<<<1, kOrderThreads, 0, s>>>(a.blk_cnt, a.Hq, a.Hk, a.gqa_interleave ? 1 : 0, Nq, run, Nk, shift,
                                             order, kv_major(a, Nq), ctr);
    if (int rc = fs_host::launch_status("fs_bsattn (order)")) return rc;
    grid = deal_units(total, run, static_units, pool_units);
  } else {
    total = a.B * Nq;
    grid = (unsigned)((total + 7) / 8 * a.Hq * 8);
  }
  AttnKArgs k;
  k.q = static_cast<const uint16_t*>(a.q);
  k.k = static_cast<const uint16_t*>(a.k);
  k.vt = vt;
  k.out = static_cast<uint16_t*>(a.out);
  k.blk_cnt = a.blk_cnt;
  k.blk_bits = a.blk_bits;
  k.u_idx = nullptr;
  k.order = order;
  k.q_sb = a.q_sb; k.q_sh = a.q_sh; k.k_sb = a.k_sb; k.k_sh = a.k_sh; k.o_sb = a.o_sb; k.o_sh = a.o_sh;
  k.q_sl = (int)a.q_sl; k.k_sl = (int)a.k_sl; k.o_sl = (int)a.o_sl;
  k.Hq = a.Hq; k.Hk = a.Hk; k.Lq = a.Lq; k.Lk = a.Lk;
  k.Nq = Nq; k.Nk = Nk; k.NWk = (Nk + 63) / 64; k.Lp = Lp; k.total = total; k.is_causal = a.is_causal;
  k.run = run;
  k.scale = a.softmax_scale;
  k.gqa_interleave = a.gqa_interleave ? 1 : 0;
  k.ctr = ctr;
  k.static_units = static_units;
  k.pool_units = pool_units;
  bsattn_kernel<BS, TK, T, BS, D><<<grid, AttnCfg<BS, TK, D>::NT, 0, s>>>(k);
  return fs_host::launch_status("fs_bsattn");
}

// union mode (16- and 32-token lists): union lists, order pass over the
// groups, the 128-query kernel over the unions
template <int LB, typename T, int D>
static int launch_run_union(const fs_attn_args& a, hipStream_t s) {
  constexpr int R = 128 / LB;
  const int NqL = (a.Lq + LB - 1) / LB, NkL = (a.Lk + LB - 1) / LB;
  const int Ng = (NqL + R - 1) / R;
  char* w = static_cast<char*>(a.work);
  int32_t* order = reinterpret_cast<int32_t*>(w + vt_bytes(a));
  int32_t* u_cnt = reinterpret_cast<int32_t*>(w + vt_bytes(a) + order_bytes(a));
  uint32_t* u_idx = reinterpret_cast<uint32_t*>(w + vt_bytes(a) + order_bytes(a) +
                                                align256((size_t)a.Hq * Ng * sizeof(int32_t)));
  union_kernel<<<(unsigned)(a.Hq * Ng), 64, 0, s>>>(a.blk_bits, NqL, NkL, R, Ng, u_cnt, u_idx);
  if (int rc = fs_host::launch_status("fs_bsattn (union lists)")) return rc;
  const int run = min(16, max(1, Ng / 64));
  int shift = 0;
  while ((int64_t)a.Hk * (((run * NkL) >> shift) + 1) > kOrderMaxBins) ++shift;
  const int total = a.Hq * ((Ng + run - 1) / run);
  int32_t* ctr = ticket_counters(a);              // after the order, inside order_bytes
  order_kernel<<<1, kOrderThreads, 0, s>>>(u_cnt, a.Hq, a.Hk, a.gqa_interleave ? 1 : 0, Ng, run, NkL, shift, order,
                                           kv_major(a, Ng), ctr);
  if (int rc = fs_host::launch_status("fs_bsattn (order)")) return rc;
  AttnKArgs k;
  k.q = static_cast<const uint16_t*>(a.q);
  k.k = static_cast<const uint16_t*>(a.k);
  k.vt = static_cast<const uint16_t*>(a.work);
  k.out = static_cast<uint16_t*>(a.out);
  k.blk_cnt = u_cnt;
  k.blk_bits = nullptr;
  k.u_idx = u_idx;
  k.order = order;
  k.q_sb = a.q_sb; k.q_sh = a.q_sh; k.k_sb = a.k_sb; k.k_sh = a.k_sh; k.o_sb = a.o_sb; k.o_sh = a.o_sh;
  k.q_sl = (int)a.q_sl; k.k_sl = (int)a.k_sl; k.o_sl = (int)a.o_sl;
  k.Hq = a.Hq; k.Hk = a.Hk; k.Lq = a.Lq; k.Lk = a.Lk;
  k.Nq = Ng; k.Nk = NkL; k.NWk = 0; k.Lp = vt_len(NkL, LB); k.total = total; k.is_causal = a.is_causal;
  k.run = run;
  k.scale = a.softmax_scale;
  k.ctr = ctr;
  k.gqa_interleave = a.gqa_interleave ? 1 : 0;
  const unsigned grid = deal_units(total, run, k.static_units, k.pool_units);
  bsattn_kernel<128, 64, T, LB, D><<<grid, AttnCfg<128, 64, D>::NT, 0, s>>>(k);
  return fs_host::launch_status("fs_bsattn");
}

}  // namespace fs

using namespace fs;

extern "C" size_t fs_bsattn_work_bytes(const fs_attn_args* a) {
  if (!a || a->B <= 0 || a->Hq <= 0 || a->Hk <= 0 || a->Lq <= 0 || a->Lk <= 0 || a->D <= 0 || a->bs <= 0) return 0;
  size_t n = vt_bytes(*a) + order_bytes(*a);
  if (union_mode(*a)) {
    const size_t Ng = (size_t)union_groups(*a), Nk = (size_t)(a->Lk + a->bs - 1) / a->bs;
    n += align256((size_t)a->Hq * Ng * sizeof(int32_t)) + (size_t)a->Hq * Ng * Nk * sizeof(uint32_t);
  }
  return n;
}

// Argument checks shared by the three attention entry points.
static int check_attn(const fs_attn_args* a, const char* fn) {
  FS_CHECK_ARG(a != nullptr, "%s: null args", fn);
  FS_CHECK_ARG(a->q && a->k && a->v && a->out && a->work, "%s: null tensor pointer", fn);
  FS_CHECK_ARG(a->B >= 1 && a->Hq >= 1 && a->Hk >= 1 && a->Hq % a->Hk == 0,
               "%s: Hq=%d must be a multiple of Hk=%d", fn, a->Hq, a->Hk);
  FS_CHECK_ARG(a->Lq >= 1 && a->Lk >= 1, "%s: empty sequence", fn);
  FS_CHECK_SUPPORTED(a->D == 128 || a->D == 64, "%s: head_dim %d unsupported (64 or 128)", fn, a->D);
  FS_CHECK_SUPPORTED(a->bs == 16 || a->bs == 32 || a->bs == 64 || a->bs == 128, "%s: block size %d unsupported", fn,
                     a->bs);
  // union mode (16- and 32-token lists): block indices and their rows packed in 32-bit entries
  FS_CHECK_SUPPORTED(!(a->blk_cnt && a->bs < 64) || (a->Lk + a->bs - 1) / a->bs <= 8192,
                     "%s: %d-token lists over more than 8192 key blocks unsupported", fn, a->bs);
  FS_CHECK_SUPPORTED(a->dtype == FS_DTYPE_BF16 || a->dtype == FS_DTYPE_F16,
                     "%s: dtype %d unsupported (bf16/f16)", fn, a->dtype);
  FS_CHECK_SUPPORTED(a->Hk <= 4096, "%s: %d KV heads > 4096", fn, a->Hk);
  FS_CHECK_ARG(a->blk_cnt == nullptr || (a->blk_bits != nullptr && a->B == 1),
               "%s: block masks need blk_bits and B == 1", fn);
  const int64_t strides[] = {a->q_sb, a->q_sh, a->q_sl, a->k_sb, a->k_sh, a->k_sl,
                             a->v_sb, a->v_sh, a->v_sl, a->o_sb, a->o_sh, a->o_sl};
  for (int64_t st : strides) FS_CHECK_ARG(st % 8 == 0, "%s: strides must be multiples of 8 elements", fn);
  const uintptr_t ptrs[] = {(uintptr_t)a->q, (uintptr_t)a->k, (uintptr_t)a->v, (uintptr_t)a->out,
                            (uintptr_t)a->work};
  for (uintptr_t p : ptrs) FS_CHECK_ARG(p % 16 == 0, "%s: tensors must be 16-byte aligned", fn);
  FS_CHECK_ARG((uintptr_t)a->blk_cnt % 4 == 0 && (uintptr_t)a->blk_bits % 8 == 0,
               "%s: blk_cnt / blk_bits must be 4- / 8-byte aligned", fn);
  const int64_t Nq = (a->Lq + a->bs - 1) / a->bs;
  const int64_t Nk = (a->Lk + a->bs - 1) / a->bs;
  FS_CHECK_SUPPORTED((int64_t)a->B * a->Hq * Nq < (1ll << 30) && (int64_t)a->B * a->Hk * Nk * a->bs / 64 < (1ll << 31),
                     "%s: grid too large", fn);
  // per-lane tile-copy offsets are 32-bit byte offsets: 128 rows of a row stride, 128 d rows of V^T
  FS_CHECK_SUPPORTED(a->q_sl < (1 << 23) && a->k_sl < (1 << 23) && a->o_sl < (1 << 23) && vt_len((int)Nk, a->bs) < (1 << 23),
                     "%s: row stride or sequence too large", fn);
  return FS_OK;
}

extern "C" int fs_bsattn_prepare(const fs_attn_args* a, void* stream) {
  if (int rc = check_attn(a, "fs_bsattn_prepare")) return rc;
  const int Nk = (a->Lk + a->bs - 1) / a->bs;
  const int Lp = vt_len(Nk, a->bs);
  auto vt = a->D == 64 ? vt_kernel<64> : vt_kernel<128>;
  vt<<<a->B * a->Hk * (Lp / 64), 256, 0, (hipStream_t)stream>>>(
      static_cast<const uint16_t*>(a->v), a->v_sb, a->v_sh, a->v_sl, static_cast<uint16_t*>(a->work), a->Hk, a->Lk,
      Lp, union_mode(*a) ? a->bs : 0);
  return fs_host::launch_status("fs_bsattn_prepare");
}

// head dim D, element type T: the kernels of one call
template <typename T, int D>
static int run_typed(const fs_attn_args* a, int Nq, int Nk, hipStream_t s) {
  if (a->bs == 128) return launch_run<128, 64, T, D>(*a, Nq, Nk, s);
  if (a->bs < 64) {
    if (a->blk_cnt) {
      // 16- and 32-token lists: unions over groups of 128 queries
      return a->bs == 32 ? launch_run_union<32, T, D>(*a, s) : launch_run_union<16, T, D>(*a, s);
    }
    // dense causal attention does not depend on the block size: the 128-token
    // kernel, reading V^T as it was laid out for this block size
    const int Nq128 = (a->Lq + 127) / 128, Nk128 = (a->Lk + 127) / 128;
    return launch_run<128, 64, T, D>(*a, Nq128, Nk128, s, vt_len(Nk, a->bs));
  }
  return launch_run<64, 64, T, D>(*a, Nq, Nk, s);
}

extern "C" int fs_bsattn_run(const fs_attn_args* a, void* stream) {
  if (int rc = check_attn(a, "fs_bsattn_run")) return rc;
  const int Nq = (a->Lq + a->bs - 1) / a->bs;
  const int Nk = (a->Lk + a->bs - 1) / a->bs;
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 64)
    return a->dtype == FS_DTYPE_BF16 ? run_typed<bf16_t, 64>(a, Nq, Nk, s) : run_typed<f16_t, 64>(a, Nq, Nk, s);
  return a->dtype == FS_DTYPE_BF16 ? run_typed<bf16_t, 128>(a, Nq, Nk, s) : run_typed<f16_t, 128>(a, Nq, Nk, s);
}

extern "C" int fs_bsattn(const fs_attn_args* a, void* stream) {
  if (int rc = check_attn(a, "fs_bsattn")) return rc;
  if (int rc = fs_bsattn_prepare(a, stream)) return rc;
  return fs_bsattn_run(a, stream);
}
