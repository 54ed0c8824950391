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
// Work split: one workgroup (4 waves) per tile of 4 * 32 * QB queries of one
// (batch, head); each wave owns 32 * QB consecutive queries.  A wave keeps its
// Q^T slice in VGPRs as the B operand of S^T = K Q^T, so every lane owns one
// query column of each score block and the softmax statistics are lane-local
// (plus one swap with lane l ^ 32).
//
// K/V tiles of 64 keys are copied straight from HBM into LDS by buffer DMA
// (no VGPR staging; rows beyond T arrive as zeros) into named buffers, so the
// copies of the next one or two tiles overlap the math of the current one.  K is
// stored fragment-major (each MFMA operand is one contiguous 1 KB LDS read);
// V is stored row-major and read transposed with ds_read_b64_tr_b16.  Each LDS
// operand feeds QB MFMAs.  Key tiles outside [q0 - W + 1, q_last] are never
// loaded, so the cost is proportional to T * W; only tiles that cross the
// diagonal or the window edge evaluate the mask per element.
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

template <int D, int QB, int NBUF>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(FwdArgs a) {
  constexpr int NW = 4, QW = 32 * QB, BM = NW * QW, BN = 64;
  constexpr int TILE = BN * D;              // elements of one K or V tile
  constexpr int PER = 2 * TILE / 512 / NW;  // DMA instructions per wave per tile
  static_assert(NBUF == 2 || NBUF == 3, "double or triple buffering");
  __shared__ __attribute__((aligned(1024))) bf16 kbuf0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 vbuf0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kbuf1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 vbuf1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kbuf2[NBUF == 3 ? TILE : 8];
  __shared__ __attribute__((aligned(1024))) bf16 vbuf2[NBUF == 3 ? TILE : 8];

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
  const int q0 = qt * BM, qw0 = q0 + QW * wave;

  const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + h * a.sq[2], a.sq[1], T, D);
  const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
  const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
  const int sq2 = (int)(a.sq[1] * 2), sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);

  // Q^T as the B operand: lane l of block qb holds q[qw0 + 32 qb + l % 32][16 s + 8 (l / 32) + e].
  bf16x8 qreg[QB][D / 16];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int s = 0; s < D / 16; ++s) qreg[qb][s] = slab_load(rq, qw0 + 32 * qb + l32, sq2, 16 * s + 8 * h32);
  drain_vmem();

  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, t_hi = key_hi / BN;
  auto issue = [&](int t, bf16* kb, bf16* vb) __attribute__((always_inline)) {
    dma_frags<BN, D, NW>(rk, sk2, t * BN, kb, wave, lane);
    dma_rows<BN, D, NW>(rv, sv2, t * BN, vb, wave, lane);
  };
  issue(t_lo, kbuf0, vbuf0);
  if (NBUF == 3 && t_lo + 1 <= t_hi) issue(t_lo + 1, kbuf1, vbuf1);

  f32x16 oacc[QB][D / 32];
  float m[QB], lsum[QB];  // running max (log2 units) and this lane's share of the row sum
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -INFINITY;
    lsum[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) oacc[qb][db] = zero16();
  }

  const bool wave_live = qw0 < T;
  const int wq_hi = min(qw0 + QW - 1, T - 1);
  const float c = a.scale_log2;

  auto tile_step = [&](const int t, const bf16* ks, const bf16* vs) __attribute__((always_inline)) {
    const int k0 = t * BN;
    if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) return;
    const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + QW - W);

    f32x16 sacc[QB][BN / 32];
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = zero16();
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        const bf16x8 kop = frag_operand<D>(ks, kb, s, lane);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma32(kop, qreg[qb][s], sacc[qb][kb]);
      }
    }
    if (!full) {
      // key = k0 + 4 h32 + (32 kb + 8 i + j) is visible iff 0 <= myq - key < W.
      // (Keys >= T fail this for every real query row myq < T.)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int d0 = qw0 + 32 * qb + l32 - k0 - 4 * h32;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int x = 0; x < 16; ++x) {
            const int cst = 32 * kb + 8 * (x >> 2) + (x & 3);
            const bool ok = (unsigned)(d0 - cst) < (unsigned)W;
            sacc[qb][kb][x] = ok ? sacc[qb][kb][x] : -INFINITY;
          }
      }
    }

    bf16x8 pb[QB][BN / 16];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      auto exponentiate = [&](const float mref) __attribute__((always_inline)) {
        float tsum = 0.f;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int x = 0; x < 16; ++x) {
            const float p = fast_exp2(fmaf(sacc[qb][kb][x], c, -mref));
            tsum += p;
            pb[qb][2 * kb + (x >> 3)][x & 7] = (bf16)p;
          }
        return tsum;
      };
      float tsum = 0.f;
      bool exact = __any(m[qb] == -INFINITY);
      if (!exact) {
        tsum = exponentiate(m[qb]);
        exact = __any(!(tsum <= kSumLimit));
      }
      if (exact) {
        float tmax = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[qb][kb][x]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32)) * c;
        const float mnew = fmaxf(m[qb], tmax);
        const float mref = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = fast_exp2(m[qb] - mref);  // 0 while m is -inf (O and the sum are 0 then)
        m[qb] = mnew;
        lsum[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
          for (int x = 0; x < 16; ++x) oacc[qb][db][x] *= alpha;
        tsum = exponentiate(mref);
      }
      lsum[qb] += tsum;
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int kk = 0; kk < BN / 16; ++kk) {
        const bf16x8 vop = lds_operand_tr(vs + 16 * kk * D + 32 * db, D, lane);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = mfma32(vop, pb[qb][kk], oacc[qb][db]);
      }
  };

  // Named buffers, loop unrolled by NBUF.  Before tile t is read, each wave
  // waits for its own copy of tile t (the newer tile t+1 may still be in
  // flight), then the barrier makes every wave's copy visible and frees the
  // buffer of tile t-1, into which tile t+NBUF-1 is issued at once.
  auto stage = [&](int t, const bf16* kb, const bf16* vb, bf16* kn, bf16* vn) __attribute__((always_inline)) {
    if (NBUF == 3 && t + 1 <= t_hi)
      dma_barrier<PER>();
    else
      dma_barrier<0>();
    if (t + NBUF - 1 <= t_hi) issue(t + NBUF - 1, kn, vn);
    tile_step(t, kb, vb);
  };
  if constexpr (NBUF == 3) {
    for (int t = t_lo; t <= t_hi; t += 3) {
      stage(t, kbuf0, vbuf0, kbuf2, vbuf2);
      if (t + 1 > t_hi) break;
      stage(t + 1, kbuf1, vbuf1, kbuf0, vbuf0);
      if (t + 2 > t_hi) break;
      stage(t + 2, kbuf2, vbuf2, kbuf1, vbuf1);
    }
  } else {
    for (int t = t_lo; t <= t_hi; t += 2) {
      stage(t, kbuf0, vbuf0, kbuf1, vbuf1);
      if (t + 1 > t_hi) break;
      stage(t + 1, kbuf1, vbuf1, kbuf0, vbuf0);
    }
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = qw0 + 32 * qb + l32;
    const float ltot = lsum[qb] + __shfl_xor(lsum[qb], 32);
    if (myq < T) {
      const float inv = 1.f / ltot;
      bf16* obase = a.o + b * a.so[0] + (int64_t)myq * a.so[1] + h * a.so[2];
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x4 v4;
#pragma unroll
          for (int j = 0; j < 4; ++j) v4[j] = (bf16)(oacc[qb][db][4 * i + j] * inv);
          *reinterpret_cast<bf16x4*>(obase + 32 * db + 8 * i + 4 * h32) = v4;
        }
      if (h32 == 0) a.lse[(int64_t)bh * T + myq] = (m[qb] + __log2f(ltot)) * kLn2;
    }
  }
}

template <int D, int QB, int NBUF>
hipError_t launch_fwd_cfg(const FwdArgs& a, hipStream_t stream) {
  constexpr int BM = 4 * 32 * QB;
  const int nqt = (a.T + BM - 1) / BM;
  const int64_t blocks = (int64_t)nqt * a.H * a.B;
  hipLaunchKernelGGL((attn_fwd_kernel<D, QB, NBUF>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  // D = 128: two buffers (64 KB) so that two workgroups share a CU's LDS.
  return D == 64 ? launch_fwd_cfg<D, kFwdQB, 3>(a, stream) : launch_fwd_cfg<D, 1, 2>(a, stream);
}

template hipError_t launch_fwd<64>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd<128>(const FwdArgs&, hipStream_t);

}  // namespace hlm
