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
// K/V tiles of 64 keys stream through an NBUF-slot LDS ring as whole-row
// (coalesced) DMA in the cs layout (attn_common.h): K is read along its rows,
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

template <int D, int NBUF, int PRE>
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
  // Query tiles with q0 >= W - 1 see a full window: they are ranks 0 .. n_full - 1.
  const TileId tid_ = tile_order(blockIdx.x, a.B * H, nqt - (W - 1 + BM - 1) / BM);
  const int qt = nqt - 1 - tid_.rank;  // longest causal rows first
  const int bh = tid_.unit;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + 32 * wave;

  const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + h * a.sq[2], a.sq[1], T, D);
  const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
  const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
  const int sq2 = (int)(a.sq[1] * 2), sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);

  const unsigned lring = lds_addr(ring);
  const unsigned stg_q = lring + PRE * SLOTB + wave * WSTG;

  // 1. This wave's Q rows into the staging area (cs layout).
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    lds_dma_at<16>(rq, stg_q + k * 1024, (qw0 + L::dma_row(k, lane)) * sq2 + L::dma_col_bytes(k, lane));

  // 2. The first key tiles.
  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, n_tiles = key_hi / BN - t_lo + 1;
  int kof[CPT / NW], vof[CPT / NW];
#pragma unroll
  for (int i = 0; i < CPT / NW; ++i) {
    const int j = wave + NW * i;
    kof[i] = L::dma_row(j, lane) * sk2 + L::dma_col_bytes(j, lane);
    vof[i] = L::dma_row(j, lane) * sv2 + L::dma_col_bytes(j, lane);
  }
  auto load_tile = [&](int t) __attribute__((always_inline)) {
    const unsigned slot = lring + (unsigned)(t % NBUF) * SLOTB;
    const int kb = (t_lo + t) * BN * sk2, vb = (t_lo + t) * BN * sv2;
#pragma unroll
    for (int i = 0; i < CPT / NW; ++i) {
      const unsigned piece = (unsigned)(wave + NW * i) * 1024;
      lds_dma_at<16>(rk, slot + piece, kb + kof[i]);
      lds_dma_at<16>(rv, slot + TILEB + piece, vb + vof[i]);
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

  int issued_hi = n_pre - 1;
  for (int it = 0; it < n_tiles; ++it) {
    // Wait for this wave's copies of tile it (newer tiles may stay in flight);
    // the barrier makes every wave's copies visible and frees the slot of tile
    // it - 1 (and, at it = 0, the staging area); then the ring is topped up to
    // NBUF - 1 tiles ahead.
    dma_barrier_upto<PER, NBUF - 1>(issued_hi - it);
    const int want = min(it + NBUF - 1, n_tiles - 1);
    while (issued_hi < want) load_tile(++issued_hi);

    const unsigned kt = lring + (unsigned)(it % NBUF) * SLOTB, vt = kt + TILEB;
    const int k0 = (t_lo + it) * BN;
    if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) continue;
    const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + 32 - W);

    f32x16 sacc[BN / 32];
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      sacc[kb] = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s) sacc[kb] = mfma32(cs_operand<D>(kt, off_s[s], kb), qreg[s], sacc[kb]);
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
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int kk = 0; kk < BN / 16; ++kk)
        oacc[db] = mfma32(cs_operand_tr<D>(vt, tro[db][0], tro[db][1], 16 * kk), pb[kk], oacc[db]);
  }

  // O through LDS (whole rows leave with coalesced stores); lse from lanes 0..31.
  dma_barrier<0>();
  int ln = lane;
  asm volatile("" : "+v"(ln));  // epilogue addresses are computed here, not hoisted above the loop
  const int e32 = ln & 31, eh = ln >> 5;
  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = 1.f / ltot;
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
  bf16* obase = a.o + b * a.so[0] + h * a.so[2];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int row = L::dma_row(k, ln);
    const bf16x8 v = lds_read_b128(reg + L::byte(row, ln % L::U));
    if (qw0 + row < T) *reinterpret_cast<bf16x8*>(obase + (int64_t)(qw0 + row) * a.so[1] + 8 * (ln % L::U)) = v;
  }
  const int myq = qw0 + l32;
  if (myq < T && h32 == 0) a.lse[(int64_t)bh * T + myq] = (m + __log2f(ltot)) * kLn2;
}

template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  constexpr int BM = 128;
  const int nqt = (a.T + BM - 1) / BM;
  const int64_t blocks = (int64_t)nqt * a.H * a.B;
  // D = 64: three slots of 16 KB (three workgroups per CU), the Q staging in
  // the third behind two tiles in flight; D = 128: two slots of 32 KB (two
  // per CU), the staging in the second behind one tile in flight.
  if constexpr (D == 64)
    hipLaunchKernelGGL((attn_fwd_kernel<D, 3, 2>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, 2, 1>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template hipError_t launch_fwd<64>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd<128>(const FwdArgs&, hipStream_t);

}  // namespace hlm
