// Backward pass of causal sliding-window attention for gfx950.
//
// With S = scale * Q K^T (masked), P = exp(S - lse), the gradients are
//   delta_i = sum_d dO[i,d] O[i,d]
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q
// i.e. the autograd of hackable-lm's `torch` backend (kernels.py:785-800),
// with P recomputed from the saved lse instead of stored.
//
// Two kernels, no atomics (fp32 atomics run at ~1.3 TB/s on the MI355X, far
// too slow to accumulate dQ across key blocks):
//   attn_bwd_dq_kernel    query-stationary, 32 queries per wave, 128 per
//                         workgroup.  Writes dQ and the workspace the next
//                         kernel reads (-lse * log2(e) and -delta per row).
//   attn_bwd_dkdv_kernel  key-stationary, 32 keys per wave, 128 per
//                         workgroup, for one kv head; loops over the query
//                         heads of its group and the 32-row query tiles that
//                         can see its keys, accumulating dK and dV in VGPRs
//                         (attn_bwd_dkdv.hip, compiled with another scheduler).
// Both skip whole tiles outside the causal window, so cost scales with T * W.
//
// Per score element the VALU does two operations (exp2, multiply) plus two
// half bf16 conversions:
// * the stationary operand that meets the moving one in S (Q in the dq kernel,
//   K in the dkdv kernel) is held pre-multiplied by scale * log2(e), rounded
//   to bf16, so S comes out in log2 units;
// * the S and dP accumulators start from -lse * log2(e) and -delta instead of
//   zero, so the MFMAs deliver S - lse and dP - delta directly, and
//   P = exp2(acc), dS = P * acc;
// * on tiles that cross the diagonal or the window edge, masked entries of the
//   S accumulator's start value are set to -inf (P = 0 there), before the
//   MFMAs and independent of them.
//
// Memory: every global access is coalesced (whole rows per instruction).
// Moving tiles stream through an NBUF-slot LDS ring as whole-row DMA in the cs
// layout (attn_common.h), which serves both the operand read along the rows
// and the transposed one (ds_read_b64_tr_b16) from one copy; each wave's own
// rows arrive the same way in ring slots the ring does not use yet; results
// leave through LDS as whole rows.
#include "attn_common.h"

namespace hlm {

__device__ __forceinline__ f32x16 splat16(float v) {
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = v;
  return r;
}

// ---------------------------------------------------------------------------
// dQ (+ the workspace).  Every global access is coalesced.
//  * K/V tiles of 32 keys stream through an NBUF-slot LDS ring in the cs
//    layout (one 1 KB DMA instruction = whole rows); each tile serves the S
//    operand (rows) and the K^T operand of dQ (transposed) from one copy.
//  * Each wave's own Q and dO rows arrive by DMA in the cs layout in ring slots
//    that the ring does not use yet (PRE tiles are already in flight in the
//    first slots), and are read from there into operand registers.
//  * O is read with coalesced loads (whole rows per instruction) only to form
//    delta = rowsum(dO * O) together with the staged dO.
//  * dQ leaves through LDS: each wave writes its 32 x D block into a cs tile
//    and stores whole rows (non-temporal).
// Tile and staging copies are inline asm with explicit waits; the few loads
// into registers are ordinary (compiler-tracked) buffer loads issued before
// them, and no store is issued before the loop ends, so inside the loop the
// vector-memory counter counts tile copies only.
// ---------------------------------------------------------------------------
template <int D, int NBUF, int PRE>
__global__ __launch_bounds__(256, D == 64 ? 3 : 2) void attn_bwd_dq_kernel(BwdArgs a) {
  using L = CS<D>;
  constexpr int NW = 4, BM = NW * 32, BN = 32;
  constexpr int NDB = D / 32, NS = D / 16;
  constexpr int TILEB = BN * D * 2;       // bytes of one K or V tile
  constexpr int SLOTB = 2 * TILEB;        // one ring slot: K and V
  constexpr int CPT = TILEB / 1024;       // 1 KB chunks per tile
  constexpr int PER = 2 * CPT / NW;       // DMA instructions per wave per tile
  constexpr int NCH = 32 / L::RPC;        // chunks of a wave's 32 rows
  constexpr int WSTG = 2 * NCH * 1024;    // staging bytes per wave (Q and dO)
  static_assert(CPT % NW == 0, "tile chunks split evenly over the waves");
  static_assert(PRE >= 1, "the loop waits for tile 0 at its first barrier");
  static_assert(PRE * SLOTB + NW * WSTG <= NBUF * SLOTB, "staging fits behind the first tiles");
  static_assert(NBUF * PER < 64 && 2 * NCH + PRE * PER < 64, "vmcnt range");
  __shared__ __attribute__((aligned(2048))) char ring[NBUF * SLOTB];

  const int T = a.T, W = a.W, H = a.H;
  const int nqt = (T + BM - 1) / BM;
  const TileId tid_ = tile_order(blockIdx.x, a.B * H, nqt - (W - 1 + BM - 1) / BM);
  const int qt = nqt - 1 - tid_.rank;  // longest causal rows first
  const int bh = tid_.unit;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + 32 * wave, myq = qw0 + l32;

  const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + h * a.sq[2], a.sq[1], T, D);
  const __amdgpu_buffer_rsrc_t rdo = slab_rsrc(a.dout + b * a.sdo[0] + h * a.sdo[2], a.sdo[1], T, D);
  const __amdgpu_buffer_rsrc_t ro = slab_rsrc(a.o + b * a.so[0] + h * a.so[2], a.so[1], T, D);
  const __amdgpu_buffer_rsrc_t rl = row_rsrc(a.lse + (int64_t)bh * T, T);
  const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
  const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
  const int sq2 = (int)(a.sq[1] * 2), sdo2 = (int)(a.sdo[1] * 2), so2 = (int)(a.so[1] * 2);
  const int sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);
  const float c = a.scale_log2;

  const unsigned lring = lds_addr(ring);
  const unsigned stg_q = lring + PRE * SLOTB + wave * WSTG, stg_do = stg_q + NCH * 1024;

  // 1. Its Q and dO rows into the staging area (cs layout).
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int row = qw0 + L::dma_row(k, lane), cb = L::dma_col_bytes(k, lane);
    lds_dma_at<16>(rq, stg_q + k * 1024, row * sq2 + cb);
    lds_dma_at<16>(rdo, stg_do + k * 1024, row * sdo2 + cb);
  }
  // 2. The first ring tiles.
  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, n_tiles = key_hi / BN - t_lo + 1;
  // Key tiles in the forward's rotated order (step t reads the tile congruent
  // to t modulo n_tiles), so that the workgroups on one XCD, whose windows
  // are offset by a few tiles each, read the same K/V tiles at the same step.
  const int rot = (n_tiles - t_lo % n_tiles) % n_tiles;
  auto tile_of = [&](int t) __attribute__((always_inline)) {
    const int g = t + rot;
    return t_lo + (g >= n_tiles ? g - n_tiles : g);
  };
  int kof[CPT / NW], vof[CPT / NW];
#pragma unroll
  for (int i = 0; i < CPT / NW; ++i) {
    const int j = wave + NW * i;
    kof[i] = L::dma_row(j, lane) * sk2 + L::dma_col_bytes(j, lane);
    vof[i] = L::dma_row(j, lane) * sv2 + L::dma_col_bytes(j, lane);
  }
  // Copies tile t into the ring slot at LDS address `slot`.
  auto load_tile_at = [&](int t, unsigned slot) __attribute__((always_inline)) {
    const int kb = tile_of(t) * BN * sk2, vb = tile_of(t) * BN * sv2;
#pragma unroll
    for (int i = 0; i < CPT / NW; ++i) {
      const unsigned piece = (unsigned)(wave + NW * i) * 1024;
      lds_dma_at<16>(rk, slot + piece, kb + kof[i]);
      lds_dma_at<16>(rv, slot + TILEB + piece, vb + vof[i]);
    }
  };
  auto load_tile = [&](int t) __attribute__((always_inline)) { load_tile_at(t, lring + (unsigned)(t % NBUF) * SLOTB); };
  const int n_pre = min(PRE, n_tiles);
  for (int t = 0; t < n_pre; ++t) load_tile(t);

  // 3. The wave's O rows (coalesced: chunk k = rows qw0 + RPC k + l / U) and
  // lse, into registers.  Issued after every copy: the compiler waits for
  // these loads with counts that assume no other memory operation is in
  // flight, so issued first, its wait for one of them (it once read the lse
  // register as the unused half of a 64-bit address add) drained all copies
  // issued after them.  Issued last, every wait for them also covers the
  // copies, which the loop needs first anyway.
  bf16x8 oc[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    oc[k] = buf_load_b128(ro, (qw0 + L::dma_row(k, lane)) * so2 + (lane % L::U) * 16);
  float lraw = buf_load_b32(rl, myq * 4);  // 0 for rows >= T

  // 4. Wait for this wave's rows (the first tiles and the O rows may still be
  // in flight: they are newer).
  vm_wait_upto<PER, PRE>(n_pre);

  int off_s[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) off_s[s] = L::byte(l32, 2 * s + h32);
  int tro[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tro[db][0] = cs_tr_off<D>(db, 0, lane);
    tro[db][1] = cs_tr_off<D>(db, 1, lane);
  }

  // Q^T (times scale * log2(e)) and dO^T as B operands: lane l holds row
  // qw0 + l % 32, columns 16 s + 8 (l / 32) + e.
  bf16x8 qreg[NS], doreg[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qreg[s] = scale_bf16x8(cs_operand<D>(stg_q, off_s[s], 0), c);
    doreg[s] = cs_operand<D>(stg_do, off_s[s], 0);
  }
  // delta of row RPC k + l / U: the U lanes of a row hold its 16-byte pieces.
  float dpart[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const bf16x8 d8 = lds_read_b128(stg_do + L::byte(L::dma_row(k, lane), lane % L::U));
    float p = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) p += (float)oc[k][e] * (float)d8[e];
#pragma unroll
    for (int m = 1; m < L::U; m <<= 1) p += __shfl_xor(p, m);
    dpart[k] = p;
  }
  float dsum = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const float t = __shfl(dpart[k], L::U * (l32 % L::RPC));
    dsum = (l32 / L::RPC == k) ? t : dsum;
  }
  const float ndelta = -dsum;
  const float nlse2 = -lraw * kLog2e;

  f32x16 dqacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dqacc[db] = zero16();

  const bool wave_live = qw0 < T;
  const int wq_hi = min(qw0 + 31, T - 1);
  // D = 64 issues all S and dP operand reads of a tile at once (the registers
  // for that fit with 3 waves per SIMD) and keeps the start values splatted;
  // D = 128 reads the operands as it goes.
  [[maybe_unused]] const f32x16 slse = splat16(nlse2), sdel = splat16(ndelta);

  // D = 64 synchronises every second tile (tiles it and it + 1 behind one
  // barrier); D = 128, whose staging leaves only one tile in flight at the
  // start, every tile.
  constexpr int KG = D == 64 ? 2 : 1;
  static_assert(PRE >= KG && NBUF >= 2 * KG + 1, "the first group is in flight before the loop");
  if constexpr (D == 64) {
    // Unrolled by the ring depth like the D = 128 loop below: fixed slots per
    // copy, ring base folded into two per-lane registers.  Their XOR variants
    // (valid with the base included: the ring is 2 KB aligned and the XORed
    // bits 5, 6 and 10 lie below that, as do the offsets they act on) are
    // formed per tile from copies made opaque in each iteration, so they are
    // not hoisted into registers of their own.
    static_assert(NBUF % KG == 0, "a group never straddles two passes of the unrolled loop");
    const unsigned ab0 = lring + (unsigned)off_s[0], at00 = lring + (unsigned)tro[0][0];
    int issued_hi = n_pre - 1;
    for (int it0 = 0; it0 < n_tiles; it0 += NBUF)
#pragma unroll
    for (int slot = 0; slot < NBUF; ++slot) {
      const int it = it0 + slot;
      if (it >= n_tiles) break;
      if (slot % KG == 0) {
        if (it >= KG && it + NBUF - 1 <= n_tiles - 1) {
          dma_barrier<(NBUF - 2 * KG) * PER>();
#pragma unroll
          for (int m = 0; m < KG; ++m)  // slots of tiles it - KG .. it - 1
            load_tile_at(++issued_hi, lring + (unsigned)((slot - KG + m + NBUF) % NBUF) * SLOTB);
        } else {
          dma_barrier_upto<PER, NBUF - 1>(issued_hi - min(it + KG - 1, n_tiles - 1));
          const int want = min(it + NBUF - 1, n_tiles - 1);
          while (issued_hi < want) load_tile(++issued_hi);
        }
      }
      const unsigned kt = (unsigned)slot * SLOTB, vt = kt + TILEB;  // constants; the base is in ab / tb
      const int k0 = tile_of(it) * BN;
      if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) continue;
      const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + 32 - W);
      // All operand reads of S and dP are issued before the first MFMA.
      bf16x8 kop[NS], vop[NS];
      unsigned ab = ab0, tb = at00;
      asm volatile("" : "+v"(ab), "+v"(tb));
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kop[s] = cs_operand<D>(kt, (int)(ab ^ (32u * s)), 0);
        vop[s] = cs_operand<D>(vt, (int)(ab ^ (32u * s)), 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x16 sacc;
      if (full) {
        sacc = mfma32(kop[0], qreg[0], slse);
      } else {
        // Column c = 4 h32 + 8 (x / 4) + x % 4 of the tile is key k0 + c; it is
        // visible to row myq iff d0 - W < c <= d0 with d0 = myq - k0 - 4 h32.
        const int d0 = myq - k0 - 4 * h32;
        const unsigned vis = band_bits(d0 - W + 1, d0);
        f32x16 st = slse;
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int cst = 8 * (x >> 2) + (x & 3);
          st[x] = ((vis >> cst) & 1u) ? st[x] : -INFINITY;
        }
        sacc = mfma32(kop[0], qreg[0], st);
      }
      f32x16 pacc = mfma32(vop[0], doreg[0], sdel);
#pragma unroll
      for (int s = 1; s < NS; ++s) {
        sacc = mfma32(kop[s], qreg[s], sacc);
        pacc = mfma32(vop[s], doreg[s], pacc);
      }
      bf16x8 dsb[2];
      // dQ's K^T operands are read right after the S and dP products issue
      // (into the registers their operands free), so the LDS latency hides
      // under the softmax; placed by the compiler, half of them were read
      // after it and waited for just before their products.
      bf16x8 ktr[2][NDB];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          ktr[kk][db] = cs_operand_tr<D>(kt, cs_tr_off_from<D>((int)tb, db, 0), cs_tr_off_from<D>((int)tb, db, 1), 16 * kk);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int x = 0; x < 16; ++x) dsb[x >> 3][x & 7] = (bf16)(fast_exp2(sacc[x]) * pacc[x]);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int db = 0; db < NDB; ++db) dqacc[db] = mfma32(ktr[kk][db], dsb[kk], dqacc[db]);
    }
  } else {
    // D = 128 (one tile per group): the loop unrolled by the ring depth, so
    // each copy reads and refills fixed slots -- per-lane address registers
    // with the ring base included (opaque, not re-associated) plus constants
    // that the ds_read offset field carries; no address arithmetic in the
    // loop.  (D = 64 has no registers to spare for this.)
    unsigned ab_s[NS], atr[NDB][2];
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
    static_assert(KG == 1, "one tile per group");
    int issued_hi = n_pre - 1;
    for (int it0 = 0; it0 < n_tiles; it0 += NBUF)
#pragma unroll
    for (int slot = 0; slot < NBUF; ++slot) {
      const int it = it0 + slot;
      if (it >= n_tiles) break;
      // As above with groups of one tile: in the steady state the slot of
      // tile it - 1 is refilled right after the barrier.
      if (it >= 1 && it + NBUF - 1 <= n_tiles - 1) {
        dma_barrier<(NBUF - 2) * PER>();
        load_tile_at(++issued_hi, lring + (unsigned)((slot + NBUF - 1) % NBUF) * SLOTB);
      } else {
        dma_barrier_upto<PER, NBUF - 1>(issued_hi - it);
        const int want = min(it + NBUF - 1, n_tiles - 1);
        while (issued_hi < want) load_tile(++issued_hi);
      }
      const unsigned kt = (unsigned)slot * SLOTB, vt = kt + TILEB;  // constants; the base is in ab_s / atr
      const int k0 = tile_of(it) * BN;
      if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) continue;
      const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + 32 - W);
      f32x16 sacc = splat16(nlse2), pacc = splat16(ndelta);
      if (!full) {
        // key = k0 + 4 h32 + 8 (x / 4) + x % 4 is visible iff 0 <= myq - key < W.
        const int d0 = myq - k0 - 4 * h32;
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int cst = 8 * (x >> 2) + (x & 3);
          sacc[x] = (unsigned)(d0 - cst) < (unsigned)W ? sacc[x] : -INFINITY;
        }
      }
      // As in the D = 128 forward, the wave raises its priority while it
      // issues its products (two waves per SIMD; 1% faster at windows of
      // 1024 and 2048 keys).
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        sacc = mfma32(cs_operand<D>(kt, (int)ab_s[s], 0), qreg[s], sacc);
        pacc = mfma32(cs_operand<D>(vt, (int)ab_s[s], 0), doreg[s], pacc);
      }
      __builtin_amdgcn_s_setprio(0);
      bf16x8 dsb[2];
#pragma unroll
      for (int x = 0; x < 16; ++x) dsb[x >> 3][x & 7] = (bf16)(fast_exp2(sacc[x]) * pacc[x]);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          dqacc[db] = mfma32(cs_operand_tr<D>(kt, (int)atr[db][0], (int)atr[db][1], 16 * kk), dsb[kk], dqacc[db]);
      __builtin_amdgcn_s_setprio(0);
    }
  }

  // dQ through LDS: every wave is past its last tile, so wave w may use the
  // bytes [32 rows * w, 32 rows * (w + 1)) of the ring for its block.
  dma_barrier<0>();
  // The epilogue's addresses derive from a lane index that the compiler cannot
  // see through, so they are computed here rather than hoisted (and kept live)
  // above the loop.
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int e32 = ln & 31, eh = ln >> 5;
  const unsigned reg = lring + wave * (32 * D * 2);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x4 v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = (bf16)(dqacc[db][4 * i + j] * a.scale);
      lds_write_b64(reg + L::byte(e32, 4 * db + i) + 8 * eh, v4);
    }
  bf16* dqbase = a.dq + b * a.sdq[0] + h * a.sdq[2];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int row = L::dma_row(k, ln);
    const bf16x8 v = lds_read_b128(reg + L::byte(row, ln % L::U));
    bf16x8* dst = reinterpret_cast<bf16x8*>(dqbase + (int64_t)(qw0 + row) * a.sdq[1] + 8 * (ln % L::U));
    if (qw0 + row < T) __builtin_nontemporal_store(v, dst);
  }
  if (myq < T && h32 == 0) {
    a.delta[(int64_t)bh * T + myq] = nlse2;
    a.delta[(int64_t)(a.B * H + bh) * T + myq] = ndelta;
  }
}

// attn_bwd_dkdv.hip
template <int D>
hipError_t launch_bwd_dkdv(const BwdArgs& a, hipStream_t stream);

template <int D>
hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream, int phases) {
  if (phases & kBwdDq) {
    constexpr int BM = 128;
    const int nqt = (a.T + BM - 1) / BM;
    const int64_t blocks = (int64_t)nqt * a.H * a.B;
    // D = 64: 6 slots of 8 KB, two tiles in flight while the staging (4 slots) is used;
    // D = 128: 5 slots of 16 KB, one tile in flight.
    if constexpr (D == 64)
      hipLaunchKernelGGL((attn_bwd_dq_kernel<D, 6, 2>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_bwd_dq_kernel<D, 5, 1>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (phases & kBwdDkDv) return launch_bwd_dkdv<D>(a, stream);
  return hipSuccess;
}

template hipError_t launch_bwd<64>(const BwdArgs&, hipStream_t, int);
template hipError_t launch_bwd<128>(const BwdArgs&, hipStream_t, int);

}  // namespace hlm
