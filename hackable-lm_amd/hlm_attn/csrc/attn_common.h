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
//   lds_operand_tr() reads the other operand of that contraction in the same
//   order, so the pair contracts over the right rows without any shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace hlm {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kThreads = 256;  // 4 waves of 64

// 32-query blocks per forward wave (1 or 2); a build-time choice.
#ifndef HLM_FWD_QB
#define HLM_FWD_QB 1
#endif
constexpr int kFwdQB = HLM_FWD_QB;

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

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.f;
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

// A/B operand whose 8 contraction values sit contiguously in one LDS row:
// lane l reads x[(l % 32) * stride + 8 * (l / 32) .. + 7].
__device__ __forceinline__ bf16x8 lds_operand(const bf16* x, int stride, int lane) {
  return *reinterpret_cast<const bf16x8*>(x + (lane & 31) * stride + 8 * (lane >> 5));
}

// A/B operand that contracts over the ROWS of a row-major LDS tile x (16 rows
// of one contraction step, 32 columns of the output): lane l receives
// x[sigma(8 * (l / 32) + e) * stride + (l % 32)], e = 0..7, via two
// ds_read_b64_tr_b16.  Within a 16-lane group, lanes 4r..4r+3 supply the four
// 8-byte pieces of row r of a 4 x 16 block and lane i receives column i.
__device__ __forceinline__ bf16x8 lds_operand_tr(const bf16* x, int stride, int lane) {
  const int g = lane >> 4, r = (lane >> 2) & 3, c = lane & 3;
  const bf16* p0 = x + (4 * (g >> 1) + r) * stride + 16 * (g & 1) + 4 * c;
  const bf16* p1 = p0 + 8 * stride;
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  bf16x8 out;
  const bf16x4 lo_b = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 hi_b = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = lo_b[e];
    out[4 + e] = hi_b[e];
  }
  return out;
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

// The same slab seen from row r0 on: rows r0 .. T - 1 of the slab are rows
// 0 .. T - 1 - r0 of the resource and everything past them (and any r0 >= T)
// reads as zeros.  Tile copies use this so that their per-lane offsets do not
// depend on the tile.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slab_rsrc_from(const bf16* base, int64_t st, int T, int D, int r0) {
  const int64_t extent = (int64_t)(T - 1 - r0) * st * 2 + 2 * D;
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)r0 * st), (short)0, extent > 0 ? (int)extent : 0,
                                           0x00020000);
}

// 16 bytes of one row at element column `col` through a slab resource.
__device__ __forceinline__ bf16x8 slab_load(__amdgpu_buffer_rsrc_t rs, int row, int st2, int col) {
  typedef __attribute__((ext_vector_type(4))) int i32x4;
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, row * st2 + col * 2, 0, 0);
  return __builtin_bit_cast(bf16x8, v);
}

// One LDS DMA instruction: `bytes` (16 or 4) per lane from the buffer at byte
// offset voff into lds + bytes * lane (lane placement checked on the MI355X).
// Issued as inline asm on purpose: the compiler then does not track these LDS
// writes, so it inserts no conservative vmcnt waits before unrelated LDS
// reads; every wait for them is explicit (dma_barrier).  Vector-memory loads
// complete in issue order, so the compiler's own waits for its loads can only
// over-wait.
template <int bytes>
__device__ __forceinline__ void lds_dma(__amdgpu_buffer_rsrc_t rs, const void* lds, int voff) {
  const unsigned ldsaddr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const lds_void*)lds);
  if constexpr (bytes == 16)
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
  else
    asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
}

// LDS byte address of a __shared__ location (taken once per kernel; the
// per-tile addresses are then plain 32-bit offsets from it, so the loops carry
// no generic-to-LDS pointer conversions).
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const lds_void*)p);
}

// As lds_dma, to an LDS byte address.
template <int bytes>
__device__ __forceinline__ void lds_dma_at(__amdgpu_buffer_rsrc_t rs, unsigned ldsaddr, int voff) {
  if constexpr (bytes == 16)
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
  else
    asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(ldsaddr));
}

// A buffer resource that walks down a slab tile by tile: `addr` is the byte
// address of the current tile's first row and `bytes` the bytes left in the
// slab from there (<= 0 past the end: every read returns zeros).
struct SlabCursor {
  uint64_t addr;
  int64_t bytes;
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc() const {
    const int n = bytes > 0 ? (int)bytes : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)addr, (short)0, n, 0x00020000);
  }
  __device__ __forceinline__ void advance(int64_t step) {
    addr += step;
    bytes -= step;
  }
};

// Cursor over a (batch, head) slab of T rows of 2*D bytes at row stride st
// elements, positioned at row r0.
__device__ __forceinline__ SlabCursor slab_cursor(const bf16* base, int64_t st, int T, int D, int r0) {
  return {(uint64_t)(uintptr_t)(base + (int64_t)r0 * st), (int64_t)(T - 1 - r0) * st * 2 + 2 * D};
}

// Direct buffer -> LDS copies of a ROWS x D tile starting at row r0 (st2 = row
// stride in bytes).  Each instruction moves 1 KB, and a layout is chosen by
// choosing each lane's source address.  The NW waves of a workgroup split the
// 1 KB pieces among themselves; nothing passes through VGPRs.
//
// Row-major: rows are contiguous (2*D bytes each), for ds_read_b64_tr_b16.
template <int ROWS, int D, int NW>
__device__ __forceinline__ void dma_rows(__amdgpu_buffer_rsrc_t rs, int st2, int r0, bf16* lds, int wave, int lane) {
  constexpr int NI = ROWS * D / 512, LPR = D / 8;  // 1 KB pieces; lanes per row
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
#pragma unroll
  for (int i = 0; i < NI / NW; ++i) {
    const int j = wave + NW * i;
    const int row = r0 + j * (64 / LPR) + lane / LPR;
    lds_dma<16>(rs, lds + j * 512, row * st2 + (lane % LPR) * 16);
  }
}

// Fragment-major: piece f = rb * (D / 16) + s holds, in lane order l, the
// 16 bytes of row 32 rb + l % 32 at columns 16 s + 8 (l / 32) .. + 7 -- exactly
// the A/B operand of one 32x32x16 MFMA -- so an operand read is one contiguous
// 1 KB ds_read_b128 (frag_operand).
template <int ROWS, int D, int NW>
__device__ __forceinline__ void dma_frags(__amdgpu_buffer_rsrc_t rs, int st2, int r0, bf16* lds, int wave, int lane) {
  constexpr int NI = ROWS * D / 512, SPR = D / 16;  // 1 KB pieces; pieces per 32-row block
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
#pragma unroll
  for (int i = 0; i < NI / NW; ++i) {
    const int j = wave + NW * i;
    const int row = r0 + 32 * (j / SPR) + (lane & 31);
    const int col = 16 * (j % SPR) + 8 * (lane >> 5);
    lds_dma<16>(rs, lds + j * 512, row * st2 + col * 2);
  }
}

// Swizzled fragment layout: one LDS copy of a ROWS x D tile that serves both
// operand orientations without bank conflicts.  Piece f = rb * (D / 16) + s
// (1 KB) holds rows 32 rb .. 32 rb + 31, columns 16 s .. 16 s + 15, as 64
// chunks of 16 bytes; chunk p holds half h = p / 32 (columns 16 s + 8 h ..
// + 7) of row 32 rb + ((p % 32) ^ 4 h).
//  * An MFMA operand along the rows (lane l: row l % 32, half l / 32) is one
//    ds_read_b128 per lane; each group of 16 lanes covers 16 distinct chunk
//    slots mod 256 bytes.
//  * A transposed operand (ds_read_b64_tr_b16, 4 rows x both halves per
//    16-lane group) touches 8 chunks whose slots differ mod 256 bytes, because
//    the XOR moves the second half of rows 4 m .. 4 m + 3 by 4 slots.
__device__ __forceinline__ int swz_chunk(int row, int h) { return 32 * h + ((row & 31) ^ (4 * h)); }

template <int ROWS, int D, int NW>
__device__ __forceinline__ void dma_swz(__amdgpu_buffer_rsrc_t rs, int st2, bf16* lds, int wave, int lane) {
  constexpr int NI = ROWS * D / 512, SPR = D / 16;  // 1 KB pieces; pieces per 32-row block
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
  const int h = lane >> 5, r = (lane & 31) ^ (4 * h);
#pragma unroll
  for (int i = 0; i < NI / NW; ++i) {
    const int j = wave + NW * i;
    const int row = 32 * (j / SPR) + r;
    const int col = 16 * (j % SPR) + 8 * h;
    lds_dma<16>(rs, lds + j * 512, row * st2 + col * 2);
  }
}

// dma_swz to the LDS byte address `lds` with the per-lane source offsets
// precomputed by swz_offsets (they depend only on the lane and the row stride).
template <int ROWS, int D, int NW>
struct SwzOffsets {
  int v[ROWS * D / 512 / NW];
};
template <int ROWS, int D, int NW>
__device__ __forceinline__ SwzOffsets<ROWS, D, NW> swz_offsets(int st2, int wave, int lane) {
  constexpr int NI = ROWS * D / 512, SPR = D / 16;
  static_assert(NI % NW == 0, "tile must split evenly over the waves");
  SwzOffsets<ROWS, D, NW> o;
  const int h = lane >> 5, r = (lane & 31) ^ (4 * h);
#pragma unroll
  for (int i = 0; i < NI / NW; ++i) {
    const int j = wave + NW * i;
    o.v[i] = (32 * (j / SPR) + r) * st2 + (16 * (j % SPR) + 8 * h) * 2;
  }
  return o;
}
template <int ROWS, int D, int NW>
__device__ __forceinline__ void dma_swz_at(__amdgpu_buffer_rsrc_t rs, const SwzOffsets<ROWS, D, NW>& o, unsigned lds,
                                           int wave) {
  constexpr int NI = ROWS * D / 512;
#pragma unroll
  for (int i = 0; i < NI / NW; ++i) lds_dma_at<16>(rs, lds + (wave + NW * i) * 1024, o.v[i]);
}

// Operand (rb, s) along the rows of a swizzled tile: lane l gets row
// 32 rb + l % 32, columns 16 s + 8 (l / 32) .. + 7.
template <int D>
__device__ __forceinline__ bf16x8 swz_operand(const bf16* lds, int rb, int s, int lane) {
  const int h = lane >> 5;
  return *reinterpret_cast<const bf16x8*>(lds + (rb * (D / 16) + s) * 512 + swz_chunk(lane & 31, h) * 8);
}

// Transposed operand of a swizzled tile, contracting over 16 rows r0 ..
// r0 + 15 (r0 a multiple of 16) for the 32 columns c0 .. c0 + 31 (c0 a
// multiple of 32): the same values and order as lds_operand_tr on a
// row-major copy.
template <int D>
__device__ __forceinline__ bf16x8 swz_operand_tr(const bf16* lds, int r0, int c0, int lane) {
  const int g = lane >> 4, r = (lane >> 2) & 3, c = lane & 3;
  const int row = r0 + 4 * (g >> 1) + r;
  const int s = c0 / 16 + (g & 1), h = c >> 1;
  const bf16* base = lds + ((row >> 5) * (D / 16) + s) * 512 + 4 * (c & 1);
  const bf16* p0 = base + swz_chunk(row, h) * 8;
  const bf16* p1 = base + swz_chunk(row + 8, h) * 8;
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  bf16x8 out;
  const bf16x4 lo_b = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 hi_b = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = lo_b[e];
    out[4 + e] = hi_b[e];
  }
  return out;
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
  typedef __attribute__((ext_vector_type(4))) int i32x4;
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

// Waits for every outstanding vector-memory op of this wave.  Used once after
// a kernel's prologue loads (and stores), so that inside the DMA-pipelined
// loop the compiler has nothing of its own left to wait for and dma_barrier's
// counts cover exactly the DMA of newer tiles.
__device__ __forceinline__ void drain_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Operand (rb, s) of a fragment-major tile.
template <int D>
__device__ __forceinline__ bf16x8 frag_operand(const bf16* lds, int rb, int s, int lane) {
  return *reinterpret_cast<const bf16x8*>(lds + (rb * (D / 16) + s) * 512 + lane * 8);
}

// Workgroups of a persistent launch: as many as the device holds at once
// (occupancy x compute units), at most n_items, rounded down to a multiple of 8
// (the XCD count) when that is at least 8.  Cached per kernel and device.
inline int persistent_grid(const void* kernel, int block, int64_t n_items) {
  struct Entry {
    const void* kernel;
    int device, grid;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int n_cache = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  int full = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_cache; ++i)
      if (cache[i].kernel == kernel && cache[i].device == dev) full = cache[i].grid;
  }
  if (full == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess || per_cu < 1) per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
    full = per_cu * cus;
    std::lock_guard<std::mutex> lock(mu);
    if (n_cache < 64) cache[n_cache++] = {kernel, dev, full};
  }
  int64_t g = n_items < full ? n_items : full;
  if (g >= 8) g &= ~(int64_t)7;
  return (int)(g > 0 ? g : 1);
}

}  // namespace hlm
