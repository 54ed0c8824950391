// Single-pass backward of causal sliding-window attention for gfx950 (D = 64).
//
// The same gradients as attn_bwd.hip (the autograd of hackable-lm's `torch`
// backend, kernels.py:785-800), with S and dP formed once per score block
// instead of once in the dq kernel and again in the dkdv kernel:
//
//   attn_bwd_prep_kernel    -lse * log2(e) and -delta = -rowsum(dO * O) of every
//                           query row into the workspace: the values, bit for
//                           bit, that the dq kernel writes there.
//   attn_bwd_fused_kernel   the dkdv kernel's key-stationary loop (128 keys per
//                           workgroup, 32-row query tiles of every query head of
//                           the kv group, dK and dV in VGPRs), which also forms
//                           each query tile's dQ over the workgroup's keys:
//                           every wave writes its dS^T rows to an LDS exchange
//                           buffer, and after the next barrier each wave
//                           contracts one 16-column quarter of dQ^T over all
//                           128 keys with v_mfma_f32_16x16x32_bf16; the tile's
//                           partial (times scale, bf16) leaves through LDS as
//                           whole rows into slot kt % R of the partial buffer.
//   attn_bwd_reduce_kernel  dQ[q] = sum of the partials of the key tiles that
//                           see row q, in increasing key-tile order (fp32 sum,
//                           deterministic), written as bf16.
//
// dK and dV come out bit-identical to the two-kernel backward's (same loop
// arithmetic, same workspace values).  dQ differs from the dq kernel's by
// the bf16 rounding of each partial.
//
// Partial buffer: part[R][B * H][T][D] bf16 with R = the largest number of
// 128-key tiles that one 32-row query tile meets (fused_partial_slots).  The
// key tiles that meet a query tile are consecutive, so kt % R is distinct
// among them, and every slot the reduce reads for a row was written by the
// workgroup of that key tile during the same call.
//
// Compiled with LLVM's default scheduler, which honours the pipelined S/dP
// operand reads (as attn_bwd_dkdv.hip).
//
// Stores inside the tile loop count in vmcnt next to the ring's DMA loads.
// Loads return in issue order, so a wait for "at most N outstanding" still
// guarantees that all but the newest N loads are done; outstanding stores
// only make such a wait stricter.
#include "attn_common.h"

namespace hlm {

namespace {

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two ds_read_b64_tr_b16 at LDS byte addresses a0 and a1, concatenated.  In
// each group of 16 lanes, lane 4 r + c supplies the address of 4 bf16 (row r,
// columns 4 c .. 4 c + 3 of a 4 x 16 block) and lane j receives column j of
// rows 0 .. 3.
__device__ __forceinline__ bf16x8 tr_pair(unsigned a0, unsigned a1) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a0);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)a1);
  const bf16x4 lo_b = __builtin_bit_cast(bf16x4, lo), hi_b = __builtin_bit_cast(bf16x4, hi);
  bf16x8 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = lo_b[e];
    out[4 + e] = hi_b[e];
  }
  return out;
}

// Exchange buffer: one query tile's dS^T, 128 key rows of 32 bf16 (64 bytes),
// 8-byte piece p (queries 4 p .. 4 p + 3) of row rho at rho * 64 + 8 (p ^ x(rho))
// with x = bits 3, 2, 4 of rho as bits 2, 1, 0.  Both the writes (a wave's 32
// rows, one piece each per instruction) and the transposed reads (rows 8 g + r
// of 16-lane groups g) touch 64 distinct banks per 32 lanes.
__device__ __forceinline__ int xswz(int rho) {
  return (((rho >> 3) & 1) << 2) | (((rho >> 2) & 1) << 1) | ((rho >> 4) & 1);
}

}  // namespace

// ---------------------------------------------------------------------------
// Workspace rows: -lse * log2(e) and -rowsum(dO * O).  256 threads cover 32
// rows, D / 8 lanes per row with 16 bytes each; the row sum is formed exactly
// as in attn_bwd_dq_kernel (8 products in order per lane, then a butterfly
// over the row's lanes), so the values are bit-identical to that kernel's.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_kernel(BwdArgs a) {
  constexpr int U = D / 8, ROWS = 256 / U;
  const int T = a.T, H = a.H;
  const int ntile = (T + ROWS - 1) / ROWS;
  const int bh = blockIdx.x / ntile, tile = blockIdx.x - bh * ntile;
  const int h = bh % H, b = bh / H;
  const int row = tile * ROWS + (int)threadIdx.x / U, u = (int)threadIdx.x % U;
  float p = 0.f;
  if (row < T) {
    const bf16x8 o8 =
        *reinterpret_cast<const bf16x8*>(a.o + b * a.so[0] + (int64_t)row * a.so[1] + h * a.so[2] + 8 * u);
    const bf16x8 d8 =
        *reinterpret_cast<const bf16x8*>(a.dout + b * a.sdo[0] + (int64_t)row * a.sdo[1] + h * a.sdo[2] + 8 * u);
#pragma unroll
    for (int e = 0; e < 8; ++e) p += (float)o8[e] * (float)d8[e];
  }
#pragma unroll
  for (int m = 1; m < U; m <<= 1) p += __shfl_xor(p, m);
  if (row < T && u == 0) {
    const float lraw = a.lse[(int64_t)bh * T + row];
    a.delta[(int64_t)bh * T + row] = -lraw * kLog2e;
    a.delta[(int64_t)(a.B * H + bh) * T + row] = -p;
  }
}

// ---------------------------------------------------------------------------
// dK, dV and the dQ partials.  The dK/dV part is attn_bwd_dkdv_kernel<64>:
// lanes own key columns of S = Q K^T and dP = dO V^T, K (times scale *
// log2(e)) and V stay in VGPRs, the start values come from LDS, query tiles
// stream through an NBUF-slot ring of whole-row DMA copies.  Unlike that
// kernel it synchronises on every tile (the dS exchange needs it): at the top
// of iteration it the ring wait and barrier make tile it's copies and every
// wave's dS^T of tile it - 1 visible; the wave then stores the partial rows of
// tile it - 2 (left in LDS during iteration it - 1), runs tile it's dK/dV
// work, writes its dS^T of tile it, and forms its quarter of tile it - 1's
// dQ partial.  Two exchange buffers and two partial buffers alternate by
// tile parity.
// ---------------------------------------------------------------------------
template <int NBUF, int PRE>
__global__ __launch_bounds__(kThreads, 2) void attn_bwd_fused_kernel(BwdArgs a, bf16* part, int R) {
  constexpr int D = 64;
  using L = CS<D>;
  constexpr int NW = 4, BNK = NW * 32, BMQ = 32;
  constexpr int NDB = D / 32, NS = D / 16;
  constexpr int TILEB = BMQ * D * 2;     // bytes of one Q or dO tile
  constexpr int SLOTB = 2 * TILEB;       // one ring slot: Q and dO
  constexpr int CPT = TILEB / 1024;      // 1 KB chunks per tile
  constexpr int PER = 2 * CPT / NW + 1;  // DMA instructions per wave per tile: Q and dO pieces, one start-value row
  constexpr int NCH = 32 / L::RPC;       // chunks of a wave's 32 rows
  constexpr int WSTG = 2 * NCH * 1024;   // staging bytes per wave (K and V)
  constexpr int XB = BNK * BMQ * 2;      // one exchange buffer: 128 key rows of 32 bf16
  constexpr int PB = BMQ * D * 2;        // one partial buffer: 32 query rows of D bf16 (cs layout)
  static_assert(CPT % NW == 0, "tile chunks split evenly over the waves");
  static_assert(PRE * SLOTB + NW * WSTG <= NBUF * SLOTB, "staging fits behind the first tiles");
  static_assert(PRE >= 1 && PRE < NBUF && NBUF % 2 == 0, "ring shape");
  static_assert(NBUF * PER < 64 && 2 * NCH + PRE * PER < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char ring[NBUF * SLOTB];
  __shared__ __attribute__((aligned(256))) float stbuf[NBUF][128];  // [0, 64): -lse * log2(e), [64, 128): -delta
  __shared__ __attribute__((aligned(1024))) char xbuf[2 * XB];
  __shared__ __attribute__((aligned(1024))) char pbuf[2 * PB];

  const int T = a.T, W = a.W, H = a.H, Hkv = a.Hkv;
  const int G = H / Hkv;
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

  const unsigned lring = lds_addr(ring), lst = lds_addr(stbuf) + 256 * (wave & 1);
  const unsigned lx = lds_addr(xbuf), lp = lds_addr(pbuf);
  const unsigned stg_k0 = lring + PRE * SLOTB, stg_k = stg_k0 + wave * WSTG, stg_v = stg_k + NCH * 1024;

  // 1. This wave's K and V rows into the staging area (cs layout).
  {
    const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
    const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
    const int sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int row = kw0 + L::dma_row(k, lane), cb = L::dma_col_bytes(k, lane);
      lds_dma_at<16>(rk, stg_k + k * 1024, row * sk2 + cb);
      lds_dma_at<16>(rv, stg_v + k * 1024, row * sv2 + cb);
    }
  }

  // 2. Query tiles, head by head, tile by tile, into ring slot (issue index) % NBUF.
  int ld_g = 0, ld_t = 0, issued = 0, islot = 0;
  const int qstep = BMQ * sq2, dostep = BMQ * sdo2;
  const int64_t plane = (wave & 1) == 0 ? 0 : (int64_t)(a.B * H) * T;  // -lse*log2(e) or -delta rows
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
    const int tq = ld_t * qstep, tdo = ld_t * dostep;
#pragma unroll
    for (int i = 0; i < CPT / NW; ++i) {
      const unsigned piece = (unsigned)(wave + NW * i) * 1024;
      lds_dma_at<16>(rq, sb + piece, qof[i] + tq);
      lds_dma_at<16>(rdo, sb + TILEB + piece, dof[i] + tdo);
    }
    lds_dma_at<4>(rst, lst + islot * 512, lane * 4 + ld_t * (BMQ * 4));  // fp32 rows, 64 lanes x 4 bytes
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

  // 3. Wait for this wave's K and V rows, then (barrier) for every wave's:
  // the dQ operands need all 128 keys.
  vm_wait_upto<PER, PRE>(n_pre);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  const int g16 = lane >> 4, j16 = lane & 15, r4 = j16 >> 2, c4 = j16 & 3;
  int off_s[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) off_s[s] = L::byte(l32, 2 * s + h32);
  int tro[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    tro[db][0] = cs_tr_off<D>(db, 0, lane);
    tro[db][1] = cs_tr_off<D>(db, 1, lane);
  }
  // K^T (times scale * log2(e)) and V^T as B operands of S and dP: lane l
  // holds row kw0 + l % 32, columns 16 s + 8 (l / 32) + e.
  bf16x8 kreg[NS], vreg[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kreg[s] = scale_bf16x8(cs_operand<D>(stg_k, off_s[s], 0), c);
    vreg[s] = cs_operand<D>(stg_v, off_s[s], 0);
  }
  // K^T (unscaled) as the A operand of this wave's dQ^T quarter, columns
  // 16 wave .. 16 wave + 15 of D, for the 32-key contraction step s (the
  // rows of wave s): lane l holds K[k0 + 32 s + 8 (l / 16) + e][16 wave + l % 16].
  bf16x8 kT[NW];
#pragma unroll
  for (int s = 0; s < NW; ++s) {
    const unsigned sk = stg_k0 + s * WSTG;
    const int col = 16 * wave + 4 * c4;
    const int half = 8 * ((col >> 2) & 1);
    kT[s] = tr_pair(sk + L::byte(8 * g16 + r4, col >> 3) + half, sk + L::byte(8 * g16 + 4 + r4, col >> 3) + half);
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

  // LDS addresses: per-lane registers with the array bases included (opaque,
  // not re-associated), slot and buffer constants in the ds offset field.
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
  // dS^T writes: row rho = 32 wave + l % 32, piece 2 i + l / 32 (i = 0..3).
  const int rho_w = 32 * wave + l32;
  unsigned xw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xw[i] = lx + (unsigned)(rho_w * 64 + 8 * ((2 * i + h32) ^ xswz(rho_w)));
    asm volatile("" : "+v"(xw[i]));
  }
  // dS^T reads for the dQ^T B operand of step s, query half hf, row group sc:
  // lane (g16, r4, c4) addresses row 32 s + 8 g16 + 4 sc + r4, piece 4 hf + c4;
  // the byte offset is (xr ^ (16 sc) ^ (32 hf)) + 256 sc + 2048 s.
  unsigned xr = lx + (unsigned)((8 * g16 + r4) * 64 + 8 * ((c4 ^ (g16 >> 1)) + 4 * (g16 & 1)));
  asm volatile("" : "+v"(xr));
  // dQ^T quarter into the partial buffer: lane (g16, j16) holds rows
  // 16 hf + j16, columns 16 wave + 4 g16 .. + 3.
  unsigned pw = lp + (unsigned)(L::byte(j16, 2 * wave + (g16 >> 1)) + 8 * (g16 & 1));
  asm volatile("" : "+v"(pw));
  // Partial rows out: wave w reads rows 8 w + l / 8, unit l % 8 (cs layout)
  // and stores them at byte (8 w + l / 8) * 2 D + 16 (l % 8) = 1024 w + 16 l
  // of the tile's first row.
  unsigned pr = lp + (unsigned)L::byte(8 * wave + (lane >> 3), lane & 7);
  asm volatile("" : "+v"(pr));
  const int pst_off = 1024 * wave + 16 * lane;
  const float scale = a.scale;

  // Store pointer: the (head, tile) of the next partial rows to store.
  int sp_g = 0, sp_t = 0;
  const int64_t slot_plane = (int64_t)(kt % R) * a.B * H;
  auto store_partial = [&](unsigned pbase) __attribute__((always_inline)) {
    const int hq = hk * G + sp_g, qs = (tq_lo + sp_t) * BMQ;
    // The head's partial rows from row qs on; rows >= T fall past the extent and are dropped.
    const bf16* prow = part + ((slot_plane + (int64_t)b * H + hq) * T + qs) * D;
    const __amdgpu_buffer_rsrc_t rp = bytes_rsrc(prow, (T - qs) * (2 * D));
    const bf16x8 v = lds_read_b128(pbase + pr);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, pst_off, 0, 0);
    if (++sp_t == nq) {
      sp_t = 0;
      ++sp_g;
    }
  };
  // This wave's dQ^T quarter of the tile whose dS^T is in the exchange
  // buffer at byte offset xbase, times scale, into the partial buffer at byte
  // offset pbase (the array bases are in xr and pw).
  auto dq_quarter = [&](unsigned xbase, unsigned pbase) __attribute__((always_inline)) {
    f32x4 acc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) acc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NW; ++s)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const unsigned a0 = (xr ^ (32u * hf)) + 2048u * s, a1 = (xr ^ 16u ^ (32u * hf)) + 256u + 2048u * s;
        acc[hf] = mfma16(kT[s], tr_pair(xbase + a0, xbase + a1), acc[hf]);
      }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      bf16x4 v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = (bf16)(acc[hf][j] * scale);
      lds_write_b64(pbase + pw + 2048u * hf, v4);
    }
  };

  for (int it0 = 0; it0 < n_iter; it0 += NBUF)
#pragma unroll
  for (int slot = 0; slot < NBUF; ++slot) {
    const int it = it0 + slot;
    if (it >= n_iter) break;
    // Wait for this wave's copies of tile it (newer tiles may stay in flight);
    // the barrier makes every wave's copies and dS^T writes visible and frees
    // the slot of tile it - 1 (and, at it = 0, the staging area); then the
    // ring is topped up to NBUF - 1 tiles ahead.
    if (it >= 1 && it + NBUF - 1 <= n_iter - 1) {
      dma_barrier<(NBUF - 2) * PER>();
      load_tile();
    } else {
      dma_barrier_upto<PER, NBUF - 1>(issued - 1 - it);
      const int want = min(it + NBUF, n_iter);
      while (issued < want) load_tile();
    }
    // Buffer parities: NBUF is even and it0 a multiple of NBUF, so they are
    // compile-time constants of each unrolled slot.
    const unsigned xcur = (unsigned)((slot & 1) * XB), xprev = (unsigned)(((slot + 1) & 1) * XB);
    const unsigned pcur = (unsigned)((slot & 1) * PB), pprev = (unsigned)(((slot + 1) & 1) * PB);

    // The partial rows of tile it - 2 (partial buffer (it - 2) & 1 == it & 1).
    if (it >= 2) store_partial(pcur);

    const unsigned qs_t = (unsigned)slot * SLOTB, ds_t = qs_t + TILEB;  // constants; lring is in ab_s / atr
    const float* st = stbuf[slot];
    const int qs = (tq_lo + cp_t) * BMQ;
    if (++cp_t == nq) cp_t = 0;
    bf16x8 dsb[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dsb[0][e] = (bf16)0.f;
      dsb[1][e] = (bf16)0.f;
    }
    if (wave_live && qs <= wk_hi + W - 1 && qs + BMQ - 1 >= kw0) {
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
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        sacc = mfma32(cs_operand<D>(qs_t, (int)ab_s[s], 0), kreg[s], sacc);
        pacc = mfma32(cs_operand<D>(ds_t, (int)ab_s[s], 0), vreg[s], pacc);
      }
      // The row-operand reads run two ahead of their products, as in the
      // dkdv kernel (attn_bwd_dkdv.hip).
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 0; i < 2 * NS - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 pb[2];
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
          dvacc[db] = mfma32(cs_operand_tr<D>(ds_t, (int)atr[db][0], (int)atr[db][1], 16 * kk), pb[kk], dvacc[db]);
          dkacc[db] = mfma32(cs_operand_tr<D>(qs_t, (int)atr[db][0], (int)atr[db][1], 16 * kk), dsb[kk], dkacc[db]);
        }
    }
    // dS^T of tile it (zeros where this wave's keys see none of its rows).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x4 v4;
#pragma unroll
      for (int e = 0; e < 4; ++e) v4[e] = dsb[i >> 1][4 * (i & 1) + e];
      lds_write_b64(xw[i] + xcur, v4);
    }
    // dQ partial of tile it - 1, written before this iteration's barrier.
    if (it >= 1) dq_quarter(xprev, pprev);
  }

  // Drain: every copy has landed and every wave has written the dS^T of the
  // last tile; store tile n - 2's rows, form tile n - 1's partial, and after
  // one more barrier store its rows.
  dma_barrier<0>();
  if (n_iter >= 2) store_partial((unsigned)((n_iter & 1) * PB));
  dq_quarter((unsigned)(((n_iter - 1) & 1) * XB), (unsigned)(((n_iter - 1) & 1) * PB));
  dma_barrier<0>();
  store_partial((unsigned)(((n_iter - 1) & 1) * PB));

  // dK and dV through LDS (the ring is free: every copy has landed and every
  // wave is past its last tile).
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

// ---------------------------------------------------------------------------
// dQ[q] = sum over key tiles kt = kt_lo(q) .. q / 128 of partial slot kt % R,
// kt_lo(q) = max(0, q - W + 1) / 128, in increasing kt.  256 threads cover 32
// rows, D / 8 lanes per row with 16 bytes each.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(BwdArgs a, const bf16* part, int R) {
  constexpr int U = D / 8, ROWS = 256 / U, BNK = 128;
  const int T = a.T, H = a.H, W = a.W;
  const int ntile = (T + ROWS - 1) / ROWS;
  const int bh = blockIdx.x / ntile, tile = blockIdx.x - bh * ntile;
  const int h = bh % H, b = bh / H;
  const int row = tile * ROWS + (int)threadIdx.x / U, u = (int)threadIdx.x % U;
  if (row >= T) return;
  const int kt_hi = row / BNK, kt_lo = max(0, row - W + 1) / BNK;
  const int64_t slot_elems = (int64_t)a.B * H * T * D;
  const bf16* src = part + ((int64_t)bh * T + row) * D + 8 * u;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  int slot = kt_lo % R;
  for (int k = kt_lo; k <= kt_hi; ++k) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(src + slot * slot_elems);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += (float)v[e];
    slot = slot + 1 == R ? 0 : slot + 1;
  }
  bf16x8 out;
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (bf16)acc[e];
  *reinterpret_cast<bf16x8*>(a.dq + b * a.sdq[0] + (int64_t)row * a.sdq[1] + h * a.sdq[2] + 8 * u) = out;
}

// Partial slots R for (T, W): the most 128-key tiles that one 32-row query
// tile meets.
int fused_partial_slots(int T, int W) {
  int r = 1;
  for (int q0 = 0; q0 < T; q0 += 32) r = max(r, q0 / 128 - max(0, q0 - W + 1) / 128 + 1);
  return r;
}

hipError_t launch_bwd_fused(const BwdArgs& a, bf16* part, int R, hipStream_t stream) {
  const int64_t row_blocks = (int64_t)((a.T + 31) / 32) * a.B * a.H;
  hipLaunchKernelGGL((attn_bwd_prep_kernel<64>), dim3((unsigned)row_blocks), dim3(256), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int64_t key_blocks = (int64_t)((a.T + 127) / 128) * a.B * a.Hkv;
  // Six ring slots of 8 KB (the K/V staging in four of them behind two tiles
  // in flight), two exchange and two partial buffers: 75 KB, two workgroups
  // per CU.
  hipLaunchKernelGGL((attn_bwd_fused_kernel<6, 2>), dim3((unsigned)key_blocks), dim3(kThreads), 0, stream, a, part, R);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  hipLaunchKernelGGL((attn_bwd_reduce_kernel<64>), dim3((unsigned)row_blocks), dim3(256), 0, stream, a,
                     (const bf16*)part, R);
  return hipGetLastError();
}

}  // namespace hlm
