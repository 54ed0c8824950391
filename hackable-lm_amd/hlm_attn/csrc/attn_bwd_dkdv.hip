// Backward pass of causal sliding-window attention for gfx950: the dK/dV
// kernel (the dQ kernel and the phase dispatch are in attn_bwd.hip; the math
// and conventions are described there).
//
// This file is compiled with LLVM's default (max-occupancy) machine
// scheduler, which honours the sched_group_barrier pipeline of the S/dP
// operand reads below within three waves per SIMD at D = 64; the dQ kernel
// keeps the iterative-ILP scheduler, which measured 2-5% faster for it.
#include "attn_common.h"

namespace hlm {

// ---------------------------------------------------------------------------
// dK, dV.  Per wave, lanes own key columns of S = Q K^T and dP = dO V^T (K, pre-
// multiplied by scale * log2(e), and V stay in VGPRs as B operands); the start
// values of the S and dP accumulators, -lse * log2(e) and -delta of the query
// rows, come from LDS.  dV^T += dO^T P and dK^T += Q^T dS read dO^T / Q^T
// transposed from the same cs-layout copies that feed S and dP.
//
// Every global access is coalesced: query tiles (Q, dO: 32 rows) stream
// through an NBUF-slot LDS ring as whole-row DMA in the cs layout; each wave's
// own K and V rows arrive the same way in ring slots the ring does not use yet
// (PRE tiles are in flight in the first slots), and dK, dV leave through LDS
// as whole rows.  The ring is topped up to NBUF - 1 tiles ahead after each
// barrier.
// ---------------------------------------------------------------------------
template <int D, int NBUF, int PRE>
__global__ __launch_bounds__(kThreads, D == 64 ? 3 : 2) void attn_bwd_dkdv_kernel(BwdArgs a) {
  using L = CS<D>;
  constexpr int NW = 4, BNK = NW * 32, BMQ = 32;
  constexpr int NDB = D / 32, NS = D / 16;
  constexpr int TILEB = BMQ * D * 2;     // bytes of one Q or dO tile
  constexpr int SLOTB = 2 * TILEB;       // one ring slot: Q and dO
  constexpr int CPT = TILEB / 1024;      // 1 KB chunks per tile
  constexpr int PER = 2 * CPT / NW + 1;  // DMA instructions per wave per tile: Q and dO pieces, one start-value row
  constexpr int NCH = 32 / L::RPC;       // chunks of a wave's 32 rows
  constexpr int WSTG = 2 * NCH * 1024;   // staging bytes per wave (K and V)
  // D = 64: K and V rows arrive by whole-row DMA into ring slots and are read
  // from there; D = 128: each lane loads its own row pieces (the ring then
  // keeps its slots for query tiles from the start).
  constexpr bool STAGE_KV = D == 64;
  static_assert(CPT % NW == 0, "tile chunks split evenly over the waves");
  static_assert(!STAGE_KV || PRE * SLOTB + NW * WSTG <= NBUF * SLOTB, "staging fits behind the first tiles");
  static_assert(PRE >= 2 && PRE < NBUF, "tiles 0 and 1 are in flight before the loop");
  static_assert(NBUF >= 4, "a barrier every second tile needs two tiles of slack");
  static_assert(NBUF * PER < 64 && 2 * NS + 2 * NCH + PRE * PER < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char ring[NBUF * SLOTB];
  __shared__ __attribute__((aligned(256))) float stbuf[NBUF][128];  // [0, 64): -lse * log2(e), [64, 128): -delta

  const int T = a.T, W = a.W, H = a.H, Hkv = a.Hkv;
  const int G = H / Hkv;
  // Rank-major: every kv head's longest key tiles (the low ones) first.
  const TileId tid_ = rank_major(blockIdx.x, a.B * Hkv);
  const int kt = tid_.rank;
  const int bhk = tid_.unit;
  const int hk = bhk % Hkv, b = bhk / Hkv;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int k0 = kt * BNK, kw0 = k0 + 32 * wave, mykey = kw0 + l32;
  const float c = a.scale_log2;

  const int q_lo = k0;
  const int q_hi = min(T - 1, k0 + BNK - 1 + W - 1);
  const int tq_lo = q_lo / BMQ, tq_hi = q_hi / BMQ;
  const int nq = tq_hi - tq_lo + 1;
  const int n_iter = nq * G;
  const int sq2 = (int)(a.sq[1] * 2), sdo2 = (int)(a.sdo[1] * 2);

  // Start values: waves 0 and 2 copy a tile's -lse*log2(e) row, waves 1 and 3
  // its -delta row, to the same LDS bytes (identical data), so every wave
  // issues the same number of copies per tile and waits on one count.
  const unsigned lring = lds_addr(ring), lst = lds_addr(stbuf) + 256 * (wave & 1);
  const unsigned stg_k = lring + PRE * SLOTB + wave * WSTG, stg_v = stg_k + NCH * 1024;

  // 1. This wave's K and V rows: into the staging area (cs layout), or
  // straight into registers as B operands (lane l: row kw0 + l % 32, columns
  // 16 s + 8 (l / 32) + e).
  bf16x8 kraw[NS], vraw[NS];
  {
    const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
    const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
    const int sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);
    if constexpr (STAGE_KV) {
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int row = kw0 + L::dma_row(k, lane), cb = L::dma_col_bytes(k, lane);
        lds_dma_at<16>(rk, stg_k + k * 1024, row * sk2 + cb);
        lds_dma_at<16>(rv, stg_v + k * 1024, row * sv2 + cb);
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kraw[s] = buf_load_b128(rk, mykey * sk2 + (16 * s + 8 * h32) * 2);
        vraw[s] = buf_load_b128(rv, mykey * sv2 + (16 * s + 8 * h32) * 2);
      }
    }
  }

  // 2. Query tiles, visited head by head (the G query heads of this kv head),
  // tile by tile; each copy goes to ring slot (issue index) % NBUF.
  int ld_g = 0, ld_t = 0, issued = 0, islot = 0;
  // D = 128: query tiles of each head in the rotated order (step t reads the
  // tile congruent to t modulo nq), so that neighbouring key tiles on one XCD
  // stream the same Q and dO rows together: 25-30% fewer L2 misses at W =
  // 1024-2048.  At D = 64 the plain order already misses little and the
  // rotation measured slightly slower.
  const int rot = D == 128 ? (nq - tq_lo % nq) % nq : 0;
  auto qtile_of = [&](int t) __attribute__((always_inline)) {
    const int g = t + rot;
    return g >= nq ? g - nq : g;
  };
  const int qstep = BMQ * sq2, dostep = BMQ * sdo2;  // bytes per query tile (< 2^31: the host bounds each slab)
  const int64_t plane = (wave & 1) == 0 ? 0 : (int64_t)(a.B * H) * T;  // -lse*log2(e) or -delta rows
  // Per query head: buffer resources over its Q, dO and workspace rows from
  // row tq_lo * BMQ on (reads past the last row return zeros); a tile's copy
  // adds only its byte offset to each lane's fixed offset.
  __amdgpu_buffer_rsrc_t rq, rdo, rst;
  auto start_head = [&]() __attribute__((always_inline)) {
    const int hq = hk * G + ld_g, qs = tq_lo * BMQ;
    rq = slab_rsrc(a.q + b * a.sq[0] + hq * a.sq[2] + (int64_t)qs * a.sq[1], a.sq[1], T - qs, D);
    rdo = slab_rsrc(a.dout + b * a.sdo[0] + hq * a.sdo[2] + (int64_t)qs * a.sdo[1], a.sdo[1], T - qs, D);
    rst = row_rsrc(a.delta + plane + ((int64_t)b * H + hq) * T + qs, T - qs);
  };
  start_head();
  int qof[CPT / NW], dof[CPT / NW];
#pragma unroll
  for (int i = 0; i < CPT / NW; ++i) {
    const int j = wave + NW * i;
    qof[i] = L::dma_row(j, lane) * sq2 + L::dma_col_bytes(j, lane);
    dof[i] = L::dma_row(j, lane) * sdo2 + L::dma_col_bytes(j, lane);
  }
  auto load_tile = [&]() __attribute__((always_inline)) {
    const unsigned sb = lring + (unsigned)islot * SLOTB;
    const int rt = qtile_of(ld_t);
    const int tq = rt * qstep, tdo = rt * dostep;
#pragma unroll
    for (int i = 0; i < CPT / NW; ++i) {
      const unsigned piece = (unsigned)(wave + NW * i) * 1024;
      lds_dma_at<16>(rq, sb + piece, qof[i] + tq);
      lds_dma_at<16>(rdo, sb + TILEB + piece, dof[i] + tdo);
    }
    lds_dma_at<4>(rst, lst + islot * 512, lane * 4 + rt * (BMQ * 4));  // fp32 rows, 64 lanes x 4 bytes
    ++issued;
    islot = islot == NBUF - 1 ? 0 : islot + 1;
    if (++ld_t == nq) {
      ld_t = 0;
      ++ld_g;
      if (ld_g < G) start_head();
    }
  };
  const int n_pre = min(PRE, n_iter);
  for (int i = 0; i < n_pre; ++i) load_tile();

  // 3. Wait for this wave's K and V rows (the first tiles may be in flight).
  vm_wait_upto<PER, PRE>(n_pre);

  // Operand offsets: kept in registers for D = 64, recomputed per use for
  // D = 128 (whose accumulators leave no room for them).
  constexpr bool KEEP_TRO = D == 64;
  const int rbase = (l32 / L::RPC) * 1024 + (l32 % L::RPC) * L::U * 16, fr = L::f(l32);
  int off_s[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) off_s[s] = KEEP_TRO ? L::byte(l32, 2 * s + h32) : 0;
  auto offs = [&](int s) __attribute__((always_inline)) {
    return KEEP_TRO ? off_s[s] : rbase + (((2 * s + h32) ^ fr) << 4);
  };
  int tro[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tro[db][0] = KEEP_TRO ? cs_tr_off<D>(db, 0, lane) : 0;
    tro[db][1] = KEEP_TRO ? cs_tr_off<D>(db, 1, lane) : 0;
  }
  // K^T (times scale * log2(e)) and V^T as B operands: lane l holds row
  // kw0 + l % 32, columns 16 s + 8 (l / 32) + e.
  bf16x8 kreg[NS], vreg[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if constexpr (STAGE_KV) {
      kraw[s] = cs_operand<D>(stg_k, offs(s), 0);
      vraw[s] = cs_operand<D>(stg_v, offs(s), 0);
    }
    kreg[s] = scale_bf16x8(kraw[s], c);
    vreg[s] = vraw[s];
  }
  if constexpr (!STAGE_KV) {
    // V's registers come straight from ordinary loads and are first read by
    // the loop's dP products.  The compiler's wait for such loads counts only
    // its own loads, so left to itself it puts a vmcnt(0) before that first
    // read inside the loop, which then drains every tile copy in flight on
    // every tile.  Reading them here puts that one wait in the prologue (it
    // also covers the first tiles, which the loop needs next).
#pragma unroll
    for (int s = 0; s < NS; ++s) asm volatile("" : "+v"(vreg[s]));
  }

  f32x16 dkacc[NDB], dvacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dkacc[db] = zero16();
    dvacc[db] = zero16();
  }

  const bool wave_live = kw0 < T;
  const int wk_hi = min(kw0 + 31, T - 1);
  int cp_t = 0;  // query tile (within the current head) of the compute pointer

  // The tile loop is unrolled by the ring depth, so each copy of the body
  // reads a fixed slot: its LDS addresses are a per-lane register (slot 0's
  // address, lane part included, made opaque so it is not re-associated)
  // plus a constant that the ds_read offset field carries.  No address
  // arithmetic is left in the loop (24 VALU instructions per tile fewer at
  // D = 64).  D = 128 has no registers to spare for them and recomputes
  // the lane part, still with the slot constant folded.
  static_assert(NBUF % 2 == 0, "a slot's parity is its tile's parity");
  unsigned ab_s[NS] = {}, atr[NDB][2] = {};
  if constexpr (KEEP_TRO) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      ab_s[s] = lring + (unsigned)off_s[s];
      asm volatile("" : "+v"(ab_s[s]));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        atr[db][k] = lring + (unsigned)tro[db][k];
        asm volatile("" : "+v"(atr[db][k]));
      }
  }
  const unsigned lbase = KEEP_TRO ? 0u : lring;  // the part of the ring address not in ab_s / atr

  for (int it0 = 0; it0 < n_iter; it0 += NBUF)
#pragma unroll
  for (int slot = 0; slot < NBUF; ++slot) {
    const int it = it0 + slot;
    if (it >= n_iter) break;
    // Every second tile: wait for this wave's copies of tiles it and it + 1
    // (newer tiles may stay in flight); the barrier makes every wave's copies
    // visible and frees the slots of tiles it - 2 and it - 1 (and, at it = 0,
    // the staging area); then the ring is topped up to NBUF - 1 tiles past
    // it.  Tile it + 1 then needs no barrier of its own.
    if ((slot & 1) == 0) {
      if (it >= 2 && it + NBUF <= n_iter) {
        // Steady state: tiles it + 2 .. it + NBUF - 3 stay in flight behind
        // tiles it and it + 1, and the two slots just freed take tiles
        // it + NBUF - 2 and it + NBUF - 1.
        static_assert(NBUF % 2 == 0 && NBUF >= 4, "groups of two tiles fill the ring");
        dma_barrier<(NBUF - 4) * PER>();
        load_tile();
        load_tile();
      } else {
        const int need = min(it + 1, n_iter - 1);
        dma_barrier_upto<PER, NBUF - 1>(issued - 1 - need);
        const int want = min(it + NBUF, n_iter);
        while (issued < want) load_tile();
      }
    }

    const unsigned qs_t = lbase + (unsigned)slot * SLOTB, ds_t = qs_t + TILEB;
    const float* st = stbuf[slot];
    const int qs = (tq_lo + qtile_of(cp_t)) * BMQ;
    if (++cp_t == nq) cp_t = 0;
    if (!(wave_live && qs <= wk_hi + W - 1 && qs + BMQ - 1 >= kw0)) continue;
    // Query rows >= T need no mask: their Q, dO and start values arrive as
    // zeros, so they add exactly zero to dK and dV.
    const bool full = (qs >= kw0 + 31) && (qs + BMQ - 1 - kw0 < W);

    // Start values: element x = 4 i + j of the accumulator is query row
    // qs + 8 i + 4 h32 + j.
    f32x16 si, di;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + 8 * i + 4 * h32);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(st + 64 + 8 * i + 4 * h32);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        si[4 * i + j] = l4[j];
        di[4 * i + j] = d4[j];
      }
    }
    if (!full) {
      const int d0 = qs + 4 * h32 - mykey;  // query - key for x = 0
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int cst = 8 * (x >> 2) + (x & 3);
        si[x] = (unsigned)(d0 + cst) < (unsigned)W ? si[x] : -INFINITY;
      }
    }

    f32x16 sacc = si, pacc = di;
    if constexpr (D == 64) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int o = KEEP_TRO ? (int)ab_s[s] : offs(s);
      sacc = mfma32(cs_operand<D>(qs_t, o, 0), kreg[s], sacc);
      pacc = mfma32(cs_operand<D>(ds_t, o, 0), vreg[s], pacc);
    }
    if constexpr (D == 64) {
      // The 8 row-operand reads run two ahead of their products (a ds_read,
      // then alternately one MFMA and the next read): left to itself the
      // scheduler issued each read right before its product and waited for
      // it there, so every S and dP product waited out a full LDS latency.
      // Two operand buffers fit in the 168 VGPRs of three waves per SIMD.
      constexpr int AHEAD = 2;
      __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 2 * NS - AHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the next read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    bf16x8 pb[2], dsb[2];
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const float p = fast_exp2(sacc[x]);
      pb[x >> 3][x & 7] = (bf16)p;
      dsb[x >> 3][x & 7] = (bf16)(p * pacc[x]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int o0 = KEEP_TRO ? (int)atr[db][0] : cs_tr_off<D>(db, 0, lane);
        const int o1 = KEEP_TRO ? (int)atr[db][1] : cs_tr_off<D>(db, 1, lane);
        dvacc[db] = mfma32(cs_operand_tr<D>(ds_t, o0, o1, 16 * kk), pb[kk], dvacc[db]);
        dkacc[db] = mfma32(cs_operand_tr<D>(qs_t, o0, o1, 16 * kk), dsb[kk], dkacc[db]);
      }
  }

  // dK and dV through LDS: every wave is past its last tile, so wave w may use
  // the bytes [64 rows * w, 64 rows * (w + 1)) of the ring for its two blocks.
  dma_barrier<0>();
  // Epilogue addresses from an opaque lane index (computed here, not hoisted).
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int e32 = ln & 31, eh = ln >> 5;
  const unsigned rk_ = lring + wave * (2 * 32 * D * 2), rv_ = rk_ + 32 * D * 2;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x4 k4, v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        k4[j] = (bf16)(dkacc[db][4 * i + j] * a.scale);
        v4[j] = (bf16)dvacc[db][4 * i + j];
      }
      const int ub = L::byte(e32, 4 * db + i) + 8 * eh;
      lds_write_b64(rk_ + ub, k4);
      lds_write_b64(rv_ + ub, v4);
    }
  bf16* dkbase = a.dk + b * a.sdk[0] + hk * a.sdk[2];
  bf16* dvbase = a.dv + b * a.sdv[0] + hk * a.sdv[2];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int row = L::dma_row(k, ln), ub = L::byte(row, ln % L::U);
    const bf16x8 kv = lds_read_b128(rk_ + ub), vv = lds_read_b128(rv_ + ub);
    if (kw0 + row < T) {
      const int64_t r = kw0 + row;
      __builtin_nontemporal_store(kv, reinterpret_cast<bf16x8*>(dkbase + r * a.sdk[1] + 8 * (ln % L::U)));
      __builtin_nontemporal_store(vv, reinterpret_cast<bf16x8*>(dvbase + r * a.sdv[1] + 8 * (ln % L::U)));
    }
  }
}

template <int D>
hipError_t launch_bwd_dkdv(const BwdArgs& a, hipStream_t stream) {
  constexpr int BNK = 4 * 32;
  const int nkt = (a.T + BNK - 1) / BNK;
  const int64_t blocks = (int64_t)nkt * a.Hkv * a.B;
  // D = 64: six slots of 8 KB (three workgroups per CU), the K/V staging in
  // four of them behind two tiles in flight; D = 128: four slots of 16 KB
  // (two per CU), three tiles in flight from the start.
  if constexpr (D == 64)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, 6, 2>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, 4, 3>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template hipError_t launch_bwd_dkdv<64>(const BwdArgs&, hipStream_t);
template hipError_t launch_bwd_dkdv<128>(const BwdArgs&, hipStream_t);

}  // namespace hlm
