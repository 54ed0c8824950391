// Shared device helpers for the gfx950 causal sliding-window attention kernels.
//
// Conventions used by every kernel in this library
// -------------------------------------------------
// * Tensors q, k, v, o, dO, dq, dk, dv are bf16 in (B, T, H, D) order with unit
//   stride along D and arbitrary (16-byte aligned) strides along B, T, H.
// * lse and delta are fp32 (B, H, T), contiguous.  lse is the natural-log
//   log-sum-exp of the scaled, masked scores of each query row.
// * Query i sees keys j with  i - W < j <= i  (W = window, W >= T means plain
//   causal), the rule of hackable-lm's model.py:143-153.
// * All contractions use v_mfma_f32_32x32x16_bf16.  For one wave (64 lanes):
//     A operand (32 x 16):  lane l holds A[l % 32][8 * (l / 32) + e], e = 0..7
//     B operand (16 x 32):  lane l holds B[8 * (l / 32) + e][l % 32]
//     C/D (32 x 32, fp32):  lane l holds C[8 * i + 4 * (l / 32) + j][l % 32]
//                           in acc[4 * i + j], i, j = 0..3
//   (checked against a host matmul on the MI355X before these kernels were
//   written).
// * "key order" of a 16-wide contraction step: the accumulator values
//   acc[8 t .. 8 t + 7] of a 32-row block, taken as the 8 B-operand values of
//   contraction step t, cover the rows sigma(8 * (l / 32) + e) of the 16-row
//   group 16 t .. 16 t + 15 with sigma = [0,1,2,3,8,9,10,11,4,5,6,7,12,13,14,15].
//   cs_operand_tr() reads the other operand of that contraction in the same
//   order, so the pair contracts over the right rows without any shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hlm {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kNonTemporal = 2;  // cache-policy operand of the buffer builtins: nt
constexpr int kThreads = 256;  // 4 waves of 64

// Backward phases (bit mask): dQ + delta first, then dK/dV, which reads delta.
constexpr int kBwdDq = 1;
constexpr int kBwdDkDv = 2;
constexpr int kBwdAll = kBwdDq | kBwdDkDv;

struct FwdArgs {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  float* lse;
  int64_t sq[3], sk[3], sv[3], so[3];  // (batch, time, head) strides in elements
  int B, T, H, Hkv, W;                 // 1 <= W <= T
  float scale_log2;                    // softmax scale * log2(e)
  // Split-key forward only: nsplit workgroups share one query tile's key
  // range; each writes its unnormalised O rows (fp32, part_o[s][b*H+h][t][D])
  // and per-row (running max in log2 units, row sum) pairs
  // (part_ml[s][b*H+h][t][2]) for the combine kernel.
  float* part_o;
  float* part_ml;
  int nsplit;
};

struct BwdArgs {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* o;
  const bf16* dout;
  const float* lse;
  bf16* dq;
  bf16* dk;
  bf16* dv;
  float* delta;  // 2 x (B, H, T) workspace written by the dq kernel: -lse * log2(e), then -rowsum(dO * O)
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sdq[3], sdk[3], sdv[3];
  int B, T, H, Hkv, W;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
};

// Arguments of the fused q/k RMSNorm + partial rotary kernels (qk_norm_rope.hip).
// Division of 0 <= n < 2^31 by a fixed divisor 1 <= d < 2^31 as a multiply
// and a shift (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994, Thm. 4.2): with l = ceil(log2 d), p = 31 + l and
// mul = ceil(2^p / d) (< 2^32), floor(n / d) = (n * mul) >> p, because
// 2^p <= mul d < 2^p + 2^(p - 31).  The host fills it (fast_div_of).
struct FastDiv {
  unsigned mul;
  int shift;  // p
};
__host__ __device__ inline FastDiv fast_div_of(unsigned d) {
  int l = 0;
  while ((1ull << l) < d) ++l;
  const int p = 31 + l;
  return {(unsigned)(((1ull << p) + d - 1) / d), p};
}
__host__ __device__ __forceinline__ int fast_div(int n, FastDiv f) {
  return (int)(((unsigned long long)(unsigned)n * f.mul) >> f.shift);
}

struct QkNormRopeArgs {
  const bf16* x[2];   // q, k: (B, T, heads, D), unit D stride
  const bf16* g[2];   // backward: gradients of the two outputs, contiguous
  bf16* out[2];       // outputs (forward) or input gradients (backward), contiguous
  int64_t s[2][3];    // (batch, time, head) strides of q and k in elements
  int heads[2];       // H, Hkv
  FastDiv div_heads[2], div_T;  // the same divisors for the row -> (batch, time, head) split
  const void* cos;    // (T, R) rows, fp32 or bf16 (tab_bf16); columns 0 .. R / 2 - 1 are read
  const void* sin;
  int tab_bf16;
  int T, rot;
  float eps;
  int rows_q;  // B * T * H
  int rows;    // B * T * (H + Hkv), < 2^31
  int blocks_q;  // workgroups of q rows (set by the launcher)
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// bf16 round of x * f, elementwise (the backward's operands pre-multiplied by
// scale * log2(e)).
__device__ __forceinline__ bf16x8 scale_bf16x8(bf16x8 x, float f) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)((float)x[e] * f);
  return r;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Workgroup order.  The grid is rank-major: workgroup id = rank * n_units +
// unit, where a unit is one (batch, head) slab and rank 0 is the unit's
// longest tile.  The hardware dispatches ids in increasing order, so the
// longest tiles start first and the short ones fill the tail; and it places
// id on XCD id % 8, so when n_units is a multiple of 8 every tile of a unit
// runs on the same XCD and its neighbouring tiles share that XCD's L2.
struct TileId {
  int rank, unit;
};
__device__ __forceinline__ TileId rank_major(int id, int n_units) { return {id / n_units, id % n_units}; }

// Two-phase order for grids of n_units * n_ranks workgroups where ranks
// 0 .. n_full - 1 all have the unit's full length: each XCD (ids congruent
// mod 8) owns the units congruent to it mod 8 and first runs their
// full-length tiles unit by unit (a unit's neighbouring tiles share L2 while
// they run), then the shorter ranks, longest first, so the short tiles fill
// the tail.  Falls back to rank_major when n_units is not a multiple of 8.
__device__ __forceinline__ TileId tile_order(int id, int n_units, int n_full) {
  if ((n_units & 7) != 0 || n_full <= 0) return rank_major(id, n_units);
  const int xcd = id & 7, slot = id >> 3, per = n_units >> 3;
  if (slot < per * n_full) return {slot % n_full, 8 * (slot / n_full) + xcd};
  const int s2 = slot - per * n_full;
  return {n_full + s2 / per, 8 * (s2 % per) + xcd};
}

typedef __attribute__((address_space(3))) void lds_void;

// Buffer resource over one (batch, head) slab of a (B, T, H, D) tensor: T rows
// of 2*D bytes at a row stride of `st` elements.  Loads beyond the slab's last
// byte return zeros (checked on the MI355X), so tile loads need no bounds
// branches: rows >= T simply arrive as zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slab_rsrc(const bf16* base, int64_t st, int T, int D) {
  const int64_t extent = (int64_t)(T - 1) * st * 2 + 2 * D;  // bytes; < 2^31 (checked by the host)
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)extent, 0x00020000);
}

// Raw buffer of `extent` bytes at `base`: loads past the end return zeros and
// stores past it are dropped.  Built from uniform values it costs a few
// scalar instructions, so loops can move a tile's row offset into the base
// (slab_rsrc from a later row) and keep their per-lane offsets invariant.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t bytes_rsrc(const void* base, int extent) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, extent, 0x00020000);
}

// LDS byte address of a __shared__ location (taken once per kernel; the
// per-tile addresses are then plain 32-bit offsets from it, so the loops carry
// no generic-to-LDS pointer conversions).
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const lds_void*)p);
}

// One LDS DMA instruction: `bytes` (16 or 4) per lane from the buffer at byte
// offset voff into LDS byte address ldsaddr + bytes * lane (lane placement
// checked on the MI355X).  Issued as inline asm on purpose: the compiler then
// does not track these LDS writes, so it inserts no conservative vmcnt waits
// before unrelated LDS reads; every wait for them is explicit (dma_barrier,
// vm_wait_upto).  Vector-memory loads complete in issue order, so the
// compiler's own waits for its loads can only over-wait.
template <int bytes>
__device__ __forceinline__ void lds_dma_at(__amdgpu_buffer_rsrc_t rs, unsigned ldsaddr, int voff) {
  if constexpr (bytes == 16)
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
  else
    asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
}

// Barrier for tiles that arrive by LDS DMA: wait until at most `pending` of
// this wave's vector-memory ops are outstanding (the DMA of newer tiles,
// which complete after the older ones), drain LDS ops, then s_barrier.  A
// plain __syncthreads() would drain every outstanding DMA, which removes the
// prefetch depth.  Callers make sure no stores are in flight when they rely
// on `pending` counting only DMA loads.
template <int pending>
__device__ __forceinline__ void dma_barrier() {
  static_assert(pending >= 0 && pending < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] (0) | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((pending & 15) | (7 << 4) | ((pending >> 4) << 14));
  asm volatile("" ::: "memory");  // no compiler motion of memory ops across the barrier
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// dma_barrier<K * PERW> for the largest K <= min(newer, KMAX): the barrier of
// a ring that has `newer` tiles of PERW copies each in flight behind the one
// being waited for.
template <int PERW, int KMAX>
__device__ __forceinline__ void dma_barrier_upto(int newer) {
  if constexpr (KMAX == 0) {
    dma_barrier<0>();
  } else {
    if (newer >= KMAX)
      dma_barrier<KMAX * PERW>();
    else
      dma_barrier_upto<PERW, KMAX - 1>(newer);
  }
}

// Waits (no barrier) until at most K * PERW vector-memory ops of this wave
// are outstanding, K = min(newer, KMAX).
template <int PERW, int KMAX>
__device__ __forceinline__ void vm_wait_upto(int newer) {
  if constexpr (KMAX == 0) {
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
  } else {
    if (newer >= KMAX) {
      constexpr int p = KMAX * PERW;
      static_assert(p < 64, "vmcnt range");
      __builtin_amdgcn_s_waitcnt((p & 15) | (7 << 4) | (15 << 8) | ((p >> 4) << 14));
      asm volatile("" ::: "memory");
    } else {
      vm_wait_upto<PERW, KMAX - 1>(newer);
    }
  }
}

// Ordinary (compiler-tracked) buffer loads at a byte offset; reads past the
// resource's extent return zeros.
__device__ __forceinline__ bf16x8 buf_load_b128(__amdgpu_buffer_rsrc_t rs, int voff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 0));
}
__device__ __forceinline__ float buf_load_b32(__amdgpu_buffer_rsrc_t rs, int voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, 0, 0));
}

// Buffer resource over n contiguous fp32 values (reads past the end return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* base, int n) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n * 4, 0x00020000);
}

// ---------------------------------------------------------------------------
// "cs" tile layout: R rows x D bf16 in LDS, built for coalesced copies.
//
// A tile is a sequence of 1 KB chunks of RPC = 512 / D whole rows (8 rows of
// 128 B for D = 64, 4 rows of 256 B for D = 128).  Within a chunk, 16-byte unit
// u of row r sits in slot (r % RPC) * U + (u ^ f(r)), U = D / 8 units per row,
// with an XOR pattern f that depends on r % 16.  Hence:
//  * one 1 KB DMA instruction copies RPC whole rows (every lane reads 16 bytes
//    of a row, 8 or 16 lanes cover it contiguously): fully coalesced;
//  * an MFMA operand along the rows (lane l: row 32 rb + l % 32, unit
//    2 s + l / 32; one ds_read_b128) and a transposed operand
//    (ds_read_b64_tr_b16 over 4 rows x 4 units per 32 lanes) are both free of
//    LDS bank conflicts (64 banks of 4 bytes; 16 lanes per b128 pass,
//    32 lanes per b64 pass).
// f: D = 64: bit 2 = bit 1 of r, bits 0-1 = bits 2-3 of r;
//    D = 128: bits 2-3 = bits 0-1 of r, bits 0-1 = bits 2-3 of r.
// ---------------------------------------------------------------------------
template <int D>
struct CS {
  static constexpr int U = D / 8;      // 16-byte units per row
  static constexpr int RPC = 512 / D;  // rows per 1 KB chunk
  static constexpr int ROW32 = 32 * 2 * D;  // bytes of 32 rows
  __device__ __forceinline__ static int f(int r) {
    if constexpr (D == 64)
      return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else
      return ((r & 3) << 2) | ((r >> 2) & 3);
  }
  // Byte offset of unit u of row r.
  __device__ __forceinline__ static int byte(int r, int u) {
    return (r / RPC) * 1024 + ((r % RPC) * U + (u ^ f(r))) * 16;
  }
  // Copy of chunk j: lane l reads 16 bytes of row RPC j + l / U at this byte
  // offset within the row (add (row0 + RPC j + l / U) * row stride).
  __device__ __forceinline__ static int dma_row(int j, int lane) { return RPC * j + lane / U; }
  __device__ __forceinline__ static int dma_col_bytes(int j, int lane) {
    return ((lane % U) ^ f(RPC * j + lane / U)) * 16;
  }
};

// Operand along the rows of a cs tile at LDS byte address `base`: lane l gets
// row 32 rb + l % 32, columns 16 s + 8 (l / 32) .. + 7 (the A/B layout of a
// 32x32x16 MFMA).  `off_s` = CS<D>::byte(l % 32, 2 s + l / 32), precomputed.
template <int D>
__device__ __forceinline__ bf16x8 cs_operand(unsigned base, int off_s, int rb) {
  typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
  return *(const lds_bf16x8*)(uintptr_t)(base + off_s + rb * CS<D>::ROW32);
}

// Per-lane byte offsets of the transposed operand of a cs tile for the 32
// columns c0 = 32 db: the two ds_read_b64_tr_b16 of rows 4 (g / 2) + rr and
// +8 (g = l / 16, rr = (l / 4) % 4), 8-byte piece 16 (g % 2) + 4 (l % 4) of
// the column block.
template <int D>
__device__ __forceinline__ int cs_tr_off(int db, int second, int lane) {
  const int g = lane >> 4, rr = (lane >> 2) & 3, c = lane & 3;
  const int row = 4 * (g >> 1) + rr + 8 * second;
  const int col = 32 * db + 16 * (g & 1) + 4 * c;
  return CS<D>::byte(row, col >> 3) + 8 * ((col >> 2) & 1);
}

// Bit c (0 <= c < 32) set iff lo <= c <= hi: the columns of a 32-wide score
// block that a row can see, as one register (masks then cost a bit test per
// element and no per-element constants).
__device__ __forceinline__ unsigned band_bits(int lo, int hi) {
  const unsigned vhi = hi < 0 ? 0u : hi >= 31 ? ~0u : (2u << hi) - 1u;
  const unsigned vlo = lo <= 0 ? ~0u : lo >= 32 ? 0u : ~0u << lo;
  return vhi & vlo;
}

// cs_tr_off(db, second, lane) from cs_tr_off(0, 0, lane): column block db
// flips bit 2 of the 16-byte unit (byte ^ 64 db); the second 8 rows add one
// (D = 64) or two (D = 128) 1 KB chunks and flip bit 1 of the swizzle
// (byte ^ 32), and neither touches bits the base offset has set.
template <int D>
__device__ __forceinline__ int cs_tr_off_from(int t0, int db, int second) {
  return t0 ^ (64 * db) ^ (second ? ((D == 64 ? 1024 : 2048) | 32) : 0);
}

// Transposed operand of a cs tile, contracting over the 16 rows r0 .. r0 + 15
// (r0 a multiple of 16) for 32 columns: lane l receives the values of column
// l % 32 at rows sigma(8 (l / 32) + e) (the order of lds_operand_tr).  o0, o1 =
// cs_tr_off(db, 0 / 1, lane).
template <int D>
__device__ __forceinline__ bf16x8 cs_operand_tr(unsigned base, int o0, int o1, int r0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const unsigned rb = base + r0 * 2 * D;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)(rb + o0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)(rb + o1));
  const bf16x4 lo_b = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 hi_b = __builtin_bit_cast(bf16x4, hi);
  bf16x8 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = lo_b[e];
    out[4 + e] = hi_b[e];
  }
  return out;
}

// Plain LDS access at a byte address.
__device__ __forceinline__ bf16x8 lds_read_b128(unsigned addr) {
  typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
  return *(const lds_bf16x8*)(uintptr_t)addr;
}
__device__ __forceinline__ void lds_write_b64(unsigned addr, bf16x4 v) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  *(lds_bf16x4*)(uintptr_t)addr = v;
}

}  // namespace hlm
