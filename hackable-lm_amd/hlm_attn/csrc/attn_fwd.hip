// Forward pass of causal sliding-window attention for gfx950.
//
// Computes, per (batch, head) and query row i,
//   O[i]   = sum_j softmax_j(scale * q_i . k_j) v_j     over keys i - W < j <= i
//   lse[i] = log sum_j exp(scale * q_i . k_j)
// which is the math of hackable-lm's `torch` attention backend
// (kernels.py:785-800) with the window mask of model.py:143-153, evaluated in
// fp32 with bf16 inputs, as the FlashAttention-2 path (kernels.py:836-841)
// receives them.
//
// Work split: one workgroup (4 waves) per tile of 128 queries of one (batch,
// head); each wave owns 32 consecutive queries.  A wave keeps its Q^T slice in
// VGPRs as the B operand of S^T = K Q^T, so every lane owns one query column of
// each score block and the softmax statistics are lane-local (plus one swap
// with lane l ^ 32).
//
// K/V tiles of 64 keys (in a rotated order, below) stream through an
// NBUF-slot LDS ring as whole-row (coalesced) DMA in the cs layout
// (attn_common.h): K is read along its rows,
// V transposed with ds_read_b64_tr_b16, both without bank conflicts.  Each
// wave's Q rows arrive the same way in a slot the ring does not use yet, and O
// leaves through LDS as whole rows.  Key tiles outside [q0 - W + 1, q_last]
// are never loaded, so the cost is proportional to T * W; only tiles that
// cross the diagonal or the window edge evaluate the mask per element.
//
// Softmax: exponentials are base 2 with scale * log2(e) folded into one FMA,
// taken against the running row max m.  A tile is first exponentiated against
// the current m with no max pass at all; only if some row's tile sum leaves
// [0, 2^64] (a new max more than 64 log2-units above m, or the first tile) does
// the wave take the exact path: tile max, rescale of O and the row sum, and a
// second exponentiation.  The row sum adds fp32 probabilities (their bf16
// roundings feed only the P V product), which keeps lse within 1e-3 even for
// windows of a few keys.
#include "attn_common.h"

namespace hlm {

constexpr float kSumLimit = 0x1p64f;  // a tile's row sum above this (or NaN) forces the exact path

template <int D, int NBUF, int PRE, bool SPLIT>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(FwdArgs a) {
  using L = CS<D>;
  constexpr int NW = 4, BM = NW * 32, BN = 64;
  constexpr int NDB = D / 32, NS = D / 16;
  constexpr int TILEB = BN * D * 2;   // bytes of one K or V tile
  constexpr int SLOTB = 2 * TILEB;    // one ring slot: K and V
  constexpr int CPT = TILEB / 1024;   // 1 KB chunks per tile
  constexpr int PER = 2 * CPT / NW;   // DMA instructions per wave per tile
  constexpr int NCH = 32 / L::RPC;    // chunks of a wave's 32 rows
  constexpr int WSTG = NCH * 1024;    // staging bytes per wave (its Q rows)
  static_assert(CPT % NW == 0, "tile chunks split evenly over the waves");
  static_assert(PRE >= 1 && PRE * SLOTB + NW * WSTG <= NBUF * SLOTB, "staging fits behind the first tiles");
  static_assert(NBUF * PER < 64 && NCH + PRE * PER < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char ring[NBUF * SLOTB];

  const int T = a.T, W = a.W, H = a.H;
  const int nqt = (T + BM - 1) / BM;
  // Split-key launches repeat the grid of tiles nsplit times, split index
  // outermost (so the XCD grouping of tile_order holds within each repeat).
  int bid = blockIdx.x, split = 0;
  if constexpr (SPLIT) {
    const int units = nqt * a.B * H;
    split = bid / units;
    bid -= split * units;
  }
  // Query tiles with q0 >= W - 1 see a full window: they are ranks 0 .. n_full - 1.
  const TileId tid_ = tile_order(bid, a.B * H, nqt - (W - 1 + BM - 1) / BM);
  const int qt = nqt - 1 - tid_.rank;  // longest causal rows first
  const int bh = tid_.unit;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + 32 * wave;

  const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + h * a.sq[2], a.sq[1], T, D);
  const char* kslab = reinterpret_cast<const char*>(a.k + b * a.sk[0] + hk * a.sk[2]);
  const char* vslab = reinterpret_cast<const char*>(a.v + b * a.sv[0] + hk * a.sv[2]);
  const int sq2 = (int)(a.sq[1] * 2), sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);
  // Slab extents in bytes (< 2^31, checked by the host): rows >= T read as zeros.
  const int kext = (T - 1) * sk2 + 2 * D, vext = (T - 1) * sv2 + 2 * D;

  const unsigned lring = lds_addr(ring);
  const unsigned stg_q = lring + PRE * SLOTB + wave * WSTG;

  // The key tiles this workgroup visits: all that meet [q0 - W + 1, q_last],
  // or with split-key launches the split-th of nsplit equal runs of them.
  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  int t_lo = key_lo / BN, n_tiles = key_hi / BN - t_lo + 1;
  if constexpr (SPLIT) {
    const int per = (n_tiles + a.nsplit - 1) / a.nsplit;
    t_lo += split * per;
    n_tiles = min(per, n_tiles - split * per);
    if (n_tiles <= 0) {  // nothing to visit: rows marked empty (sum 0) for the combine
      const int myq = qw0 + l32;
      if (myq < T && h32 == 0) {
        const int64_t prow = ((int64_t)split * a.B * H + bh) * T + myq;
        a.part_ml[2 * prow] = -INFINITY;
        a.part_ml[2 * prow + 1] = 0.f;
      }
      return;
    }
  }

  // Visiting order: step t reads the key tile of [t_lo, t_lo + n_tiles)
  // that is congruent to t modulo n_tiles (a rotation of the window, not
  // its left-to-right order).  The workgroups resident on one XCD hold
  // neighbouring query tiles whose windows are offset by two key tiles each;
  // left to right they would read ~64 different K/V tiles at any moment
  // (5 MB at W = 2048, D = 128, beyond the XCD's 4 MB L2), rotated they read
  // one or two.  Causal windows (t_lo = 0) keep the plain order.  The split
  // forward keeps the plain order within each split's run.
  const int rot = SPLIT ? 0 : (n_tiles - t_lo % n_tiles) % n_tiles;
  auto tile_of = [&](int t) __attribute__((always_inline)) {
    const int g = t + rot;
    return t_lo + (g >= n_tiles ? g - n_tiles : g);
  };
  // 1. This wave's Q rows into the staging area (cs layout).
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    lds_dma_at<16>(rq, stg_q + k * 1024, (qw0 + L::dma_row(k, lane)) * sq2 + L::dma_col_bytes(k, lane));

  // 2. The first key tiles.  A tile's buffer descriptors start at its first
  // row (scalar arithmetic), so the per-lane offsets are loop-invariant
  // registers (opaque: not recomputed in the loop) and rows >= T still read
  // as zeros.
  int kof[CPT / NW], vof[CPT / NW];
#pragma unroll
  for (int i = 0; i < CPT / NW; ++i) {
    const int j = wave + NW * i;
    kof[i] = L::dma_row(j, lane) * sk2 + L::dma_col_bytes(j, lane);
    vof[i] = L::dma_row(j, lane) * sv2 + L::dma_col_bytes(j, lane);
    asm volatile("" : "+v"(kof[i]), "+v"(vof[i]));
  }
  auto load_tile = [&](int t) __attribute__((always_inline)) {
    const unsigned slot = lring + (unsigned)(t % NBUF) * SLOTB;
    const int row0 = tile_of(t) * BN;  // < T
    const int kskip = row0 * sk2, vskip = row0 * sv2;
    const __amdgpu_buffer_rsrc_t rk = bytes_rsrc(kslab + kskip, kext - kskip);
    const __amdgpu_buffer_rsrc_t rv = bytes_rsrc(vslab + vskip, vext - vskip);
#pragma unroll
    for (int i = 0; i < CPT / NW; ++i) {
      const unsigned piece = (unsigned)(wave + NW * i) * 1024;
      lds_dma_at<16>(rk, slot + piece, kof[i]);
      lds_dma_at<16>(rv, slot + TILEB + piece, vof[i]);
    }
  };
  const int n_pre = min(PRE, n_tiles);
  for (int t = 0; t < n_pre; ++t) load_tile(t);

  // 3. Q^T as the B operand: lane l holds row qw0 + l % 32, columns
  // 16 s + 8 (l / 32) + e (rows >= T arrive as zeros).
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
  bf16x8 qreg[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qreg[s] = cs_operand<D>(stg_q, off_s[s], 0);

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = zero16();
  float m = -INFINITY, lsum = 0.f;  // running max (log2 units) and this lane's share of the row sum

  const bool wave_live = qw0 < T;
  const int wq_hi = min(qw0 + 31, T - 1);
  const float c = a.scale_log2;

  // The tile loop is unrolled by the ring depth, so each copy of the body
  // reads a fixed slot: its LDS addresses are a per-lane register (slot 0's
  // address, lane part included, opaque so that it is not re-associated) plus
  // a constant carried by the ds_read offset field -- no address arithmetic
  // in the loop.
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

  int issued_hi = n_pre - 1;
  for (int it0 = 0; it0 < n_tiles; it0 += NBUF)
#pragma unroll
  for (int slot = 0; slot < NBUF; ++slot) {
    const int it = it0 + slot;
    if (it >= n_tiles) break;
    // Wait for this wave's copies of tile it (newer tiles may stay in flight);
    // the barrier makes every wave's copies visible and frees the slot of tile
    // it - 1 (and, at it = 0, the staging area); then the ring is topped up to
    // NBUF - 1 tiles ahead.
    dma_barrier_upto<PER, NBUF - 1>(issued_hi - it);
    const int want = min(it + NBUF - 1, n_tiles - 1);
    while (issued_hi < want) load_tile(++issued_hi);

    const unsigned kt = (unsigned)slot * SLOTB, vt = kt + TILEB;  // constants; lring is in ab_s / atr
    const int k0 = tile_of(it) * BN;
    if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) continue;
    const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + 32 - W);

    // D = 128 (two waves per SIMD): the wave raises its priority while it
    // issues its products, so the S and P V products of one wave are not held
    // back behind the other wave's softmax instructions (1-2% faster at
    // windows of 1024 and 2048 keys; no change at D = 64, three waves per
    // SIMD).
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
    f32x16 sacc[BN / 32];
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      sacc[kb] = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s) sacc[kb] = mfma32(cs_operand<D>(kt, (int)ab_s[s], kb), qreg[s], sacc[kb]);
    }
    if (!full) {
      // key = k0 + 4 h32 + (32 kb + 8 i + j) is visible iff 0 <= myq - key < W.
      // (Keys >= T fail this for every real query row myq < T.)
      const int d0 = qw0 + l32 - k0 - 4 * h32;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const int cst = 32 * kb + 8 * (x >> 2) + (x & 3);
          sacc[kb][x] = (unsigned)(d0 - cst) < (unsigned)W ? sacc[kb][x] : -INFINITY;
        }
    }

    if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
    bf16x8 pb[BN / 16];
    auto exponentiate = [&](const float mref) __attribute__((always_inline)) {
      float tsum = 0.f;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          const float p = fast_exp2(fmaf(sacc[kb][x], c, -mref));
          tsum += p;
          pb[2 * kb + (x >> 3)][x & 7] = (bf16)p;
        }
      return tsum;
    };
    float tsum = 0.f;
    bool exact = __any(m == -INFINITY);
    if (!exact) {
      tsum = exponentiate(m);
      exact = __any(!(tsum <= kSumLimit));
    }
    if (exact) {
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[kb][x]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32)) * c;
      const float mnew = fmaxf(m, tmax);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = fast_exp2(m - mref);  // 0 while m is -inf (O and the sum are 0 then)
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[db][x] *= alpha;
      tsum = exponentiate(mref);
    }
    lsum += tsum;
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < BN / 16; ++kk)
        oacc[db] = mfma32(cs_operand_tr<D>(vt, (int)atr[db][0], (int)atr[db][1], 16 * kk), pb[kk], oacc[db]);
    if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
  }

  if constexpr (SPLIT) {
    // Unnormalised O (fp32) and the row's (max, sum): lane (l32, h32) holds
    // O[qw0 + l32][32 db + 8 i + 4 h32 + j] in oacc[db][4 i + j].  Every
    // issued tile has been waited for inside the loop, so no copy into LDS is
    // still in flight when the wave ends.
    const float ltot = lsum + __shfl_xor(lsum, 32);
    const int myq = qw0 + l32;
    if (myq < T) {
      const int64_t prow = ((int64_t)split * a.B * H + bh) * T + myq;
      float* po = a.part_o + prow * D + 4 * h32;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4 v4;
#pragma unroll
          for (int j = 0; j < 4; ++j) v4[j] = oacc[db][4 * i + j];
          *reinterpret_cast<f32x4*>(po + 32 * db + 8 * i) = v4;
        }
      if (h32 == 0) {
        a.part_ml[2 * prow] = m;
        a.part_ml[2 * prow + 1] = ltot;
      }
    }
    return;
  }

  // O through LDS (whole rows leave with coalesced stores, non-temporal: 1-3%
  // faster than cached ones, here and for dQ, dK, dV); lse from lanes 0..31.
  // O is rounded to bf16, so a 1-ulp reciprocal of the row sum suffices.
  dma_barrier<0>();
  int ln = lane;
  asm volatile("" : "+v"(ln));  // epilogue addresses are computed here, not hoisted above the loop
  const int e32 = ln & 31, eh = ln >> 5;
  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = __builtin_amdgcn_rcpf(ltot);
  const unsigned reg = lring + wave * (32 * D * 2);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x4 v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = (bf16)(oacc[db][4 * i + j] * inv);
      lds_write_b64(reg + L::byte(e32, 4 * db + i) + 8 * eh, v4);
    }
  if (wave_live) {
    // The wave's rows from qw0 on; stores to rows >= T fall past the buffer's
    // end and are dropped.
    const int so2 = (int)(a.so[1] * 2);
    const __amdgpu_buffer_rsrc_t ro =
        bytes_rsrc(a.o + b * a.so[0] + h * a.so[2] + (int64_t)qw0 * a.so[1], (T - 1 - qw0) * so2 + 2 * D);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int row = L::dma_row(k, ln);
      const bf16x8 v = lds_read_b128(reg + L::byte(row, ln % L::U));
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, row * so2 + 16 * (ln % L::U), 0,
                                             kNonTemporal);
    }
  }
  const int myq = qw0 + l32;
  if (myq < T && h32 == 0) a.lse[(int64_t)bh * T + myq] = (m + __log2f(ltot)) * kLn2;
}

// Merges the nsplit partial results of a split-key forward: per query row,
// M = max_s m_s, L = sum_s l_s 2^(m_s - M), O = sum_s O_s 2^(m_s - M) / L and
// lse = (M + log2 L) ln 2.  Splits that saw no visible key (l_s = 0) are
// skipped (their O rows were never written).  One thread per 8 values of a
// row; every row has at least one visible key (itself), so L > 0.
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_combine_kernel(FwdArgs a) {
  constexpr int LPR = D / 8;
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / LPR;
  const int c = (int)(gid % LPR);
  if (row >= rows) return;
  const int64_t split_stride = rows;  // rows per split
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.part_ml[2 * (s * split_stride + row)]);
  float L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const int64_t prow = s * split_stride + row;
    const float l = a.part_ml[2 * prow + 1];
    if (!(l > 0.f)) continue;
    const float w = exp2f(a.part_ml[2 * prow] - M);
    L = fmaf(l, w, L);
    const float* po = a.part_o + prow * D + 8 * c;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(po), hi = *reinterpret_cast<const f32x4*>(po + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = fmaf(lo[e], w, acc[e]);
      acc[e + 4] = fmaf(hi[e], w, acc[e + 4]);
    }
  }
  const float inv = 1.f / L;
  const int t = (int)(row % a.T);
  const int bh = (int)(row / a.T), h = bh % a.H, b = bh / a.H;
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (bf16)(acc[e] * inv);
  *reinterpret_cast<bf16x8*>(a.o + b * a.so[0] + t * a.so[1] + h * a.so[2] + 8 * c) = o;
  if (c == 0) a.lse[row] = (M + __log2f(L)) * kLn2;
}

template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  constexpr int BM = 128;
  const int nqt = (a.T + BM - 1) / BM;
  const int64_t blocks = (int64_t)nqt * a.H * a.B;
  // D = 64: three slots of 16 KB (three workgroups per CU), the Q staging in
  // the third behind two tiles in flight; D = 128: two slots of 32 KB (two
  // per CU), the staging in the second behind one tile in flight.
  if (a.nsplit <= 1) {
    if constexpr (D == 64)
      hipLaunchKernelGGL((attn_fwd_kernel<D, 3, 2, false>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<D, 2, 1, false>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
  }
  const unsigned sblocks = (unsigned)(blocks * a.nsplit);
  if constexpr (D == 64)
    hipLaunchKernelGGL((attn_fwd_kernel<D, 3, 2, true>), dim3(sblocks), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, 2, 1, true>), dim3(sblocks), dim3(kThreads), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int64_t threads = (int64_t)a.B * a.H * a.T * (D / 8);
  hipLaunchKernelGGL((attn_fwd_combine_kernel<D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

// Splits for a small forward grid.  A workgroup alone on a CU runs a key
// tile in about 1 us (latency-bound), three sharing a CU about 2.1 us each,
// and the merge pass costs 4-10 us (measured on the MI355X at B = 1, H = 12,
// D = 64).  So splitting pays only when the longest row is long: 1 (no
// split) when the tiles already occupy half of the workgroup slots or the
// longest row has fewer than 24 key tiles; otherwise one split per 12 key
// tiles of the longest row, at most enough to fill the slots and at most
// kMaxSplit.  (B = 1, T = 2048, causal: 33.7 us unsplit, 28 us in 2 splits;
// with a 512-key window, or at T = 1024, splitting is slower.)
template <int D>
int fwd_split_count(int B, int T, int H, int W) {
  constexpr int BM = 128, BN = 64, kMaxSplit = 16, kMinTiles = 24, kTilesPerSplit = 12;
  const int slots = 256 * (D == 64 ? 3 : 2);  // resident workgroups on the MI355X
  const int64_t units = (int64_t)((T + BM - 1) / BM) * B * H;
  if (units == 0 || 2 * units >= slots) return 1;
  const int longest = (min(T, W + BM - 1) + BN - 1) / BN + 1;  // key tiles of the longest row
  if (longest < kMinTiles) return 1;
  const int fill = (int)((slots + units - 1) / units);
  const int n = min(min(longest / kTilesPerSplit, fill), kMaxSplit);
  return n >= 2 ? n : 1;
}

template int fwd_split_count<64>(int, int, int, int);
template int fwd_split_count<128>(int, int, int, int);

template hipError_t launch_fwd<64>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd<128>(const FwdArgs&, hipStream_t);

}  // namespace hlm
