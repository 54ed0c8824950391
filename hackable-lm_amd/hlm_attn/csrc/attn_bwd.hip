// Backward pass of causal sliding-window attention for gfx950.
//
// With S = scale * Q K^T (masked), P = exp(S - lse), the gradients are
//   delta_i = sum_d dO[i,d] O[i,d]
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q
// i.e. the autograd of hackable-lm's `torch` backend (kernels.py:785-800),
// with P recomputed from the saved lse instead of stored.
//
// Two kernels, no atomics (fp32 atomics run at ~1.36 TB/s on the MI355X,
// far too slow to accumulate dQ across key tiles):
//   attn_bwd_dq_kernel    query-stationary.  Writes delta and lse * log2(e)
//                         (the workspace the next kernel reads) and dQ.
//   attn_bwd_dkdv_kernel  key-stationary: 64 keys per wave, 256 per
//                         workgroup, for one kv head; loops over the query
//                         heads of its group and the query tiles that can see
//                         its keys, accumulating dK and dV in registers.
// Both skip whole tiles outside the causal window, so cost scales with T * W.
// Tiles reach LDS by buffer DMA into named buffers (triple-buffered, loop
// unrolled by three), fragment-major for operands read along their rows and
// row-major for operands read transposed with ds_read_b64_tr_b16.
#include "attn_common.h"

namespace hlm {

// ---------------------------------------------------------------------------
// dQ (+ delta, lse2).  Same orientation as the forward: per wave, lanes own
// query columns of S^T = K Q^T and dP^T = V dO^T, so lse and delta are
// per-lane scalars; dQ^T += K^T dS^T reads K^T transposed from the row-major
// copy of the K tile.
// ---------------------------------------------------------------------------
template <int D, int QB>
__global__ __launch_bounds__(kThreads) void attn_bwd_dq_kernel(BwdArgs a) {
  constexpr int NW = 4, QW = 32 * QB, BM = NW * QW, BN = 64;
  constexpr int TILE = BN * D;
  constexpr int PER = 3 * TILE / 512 / NW;  // DMA instructions per wave per tile
  __shared__ __attribute__((aligned(1024))) bf16 kf0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kr0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 vf0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kf1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kr1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 vf1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kf2[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 kr2[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 vf2[TILE];

  const int T = a.T, W = a.W, H = a.H;
  const int nqt = (T + BM - 1) / BM;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x);
  const int qt = nqt - 1 - tile % nqt;
  const int bh = tile / nqt;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + QW * wave;

  const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + h * a.sq[2], a.sq[1], T, D);
  const __amdgpu_buffer_rsrc_t rdo = slab_rsrc(a.dout + b * a.sdo[0] + h * a.sdo[2], a.sdo[1], T, D);
  const __amdgpu_buffer_rsrc_t ro = slab_rsrc(a.o + b * a.so[0] + h * a.so[2], a.so[1], T, D);
  const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
  const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
  const int sq2 = (int)(a.sq[1] * 2), sdo2 = (int)(a.sdo[1] * 2), so2 = (int)(a.so[1] * 2);
  const int sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);

  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, t_hi = key_hi / BN;
  auto load_tile = [&](int t, bf16* kf, bf16* kr, bf16* vf) __attribute__((always_inline)) {
    dma_frags<BN, D, NW>(rk, sk2, t * BN, kf, wave, lane);
    dma_rows<BN, D, NW>(rk, sk2, t * BN, kr, wave, lane);
    dma_frags<BN, D, NW>(rv, sv2, t * BN, vf, wave, lane);
  };

  bf16x8 qreg[QB][D / 16], doreg[QB][D / 16];
  float delta[QB], lse2[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = qw0 + 32 * qb + l32;
    float dpart = 0.f;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const int col = 16 * s + 8 * h32;
      qreg[qb][s] = slab_load(rq, myq, sq2, col);
      doreg[qb][s] = slab_load(rdo, myq, sdo2, col);
      const bf16x8 o8 = slab_load(ro, myq, so2, col);
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)doreg[qb][s][e] * (float)o8[e];
    }
    delta[qb] = dpart + __shfl_xor(dpart, 32);
    lse2[qb] = myq < T ? a.lse[(int64_t)bh * T + myq] * kLog2e : 0.f;
    if (myq < T && h32 == 0) {
      a.delta[(int64_t)bh * T + myq] = delta[qb];
      a.delta[(int64_t)(a.B * H + bh) * T + myq] = lse2[qb];
    }
  }
  drain_vmem();
  load_tile(t_lo, kf0, kr0, vf0);
  if (t_lo + 1 <= t_hi) load_tile(t_lo + 1, kf1, kr1, vf1);

  f32x16 dqacc[QB][D / 32];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int db = 0; db < D / 32; ++db) dqacc[qb][db] = zero16();

  const bool wave_live = qw0 < T;
  const int wq_hi = min(qw0 + QW - 1, T - 1);
  const float c = a.scale_log2;

  auto tile_step = [&](const int t, const bf16* kf, const bf16* kr, const bf16* vf) __attribute__((always_inline)) {
    const int k0 = t * BN;
    if (!(wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1)) return;
    const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + QW - W);
#pragma unroll
    for (int kb = 0; kb < BN / 32; ++kb) {
      f32x16 sacc[QB], pacc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        sacc[qb] = zero16();
        pacc[qb] = zero16();
      }
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        const bf16x8 kop = frag_operand<D>(kf, kb, s, lane);
        const bf16x8 vop = frag_operand<D>(vf, kb, s, lane);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          sacc[qb] = mfma32(kop, qreg[qb][s], sacc[qb]);
          pacc[qb] = mfma32(vop, doreg[qb][s], pacc[qb]);
        }
      }
      bf16x8 dsb[QB][2];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int d0 = qw0 + 32 * qb + l32 - k0 - 32 * kb - 4 * h32;  // myq - key + (8 i + j)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          float p = fast_exp2(fmaf(sacc[qb][x], c, -lse2[qb]));
          if (!full) {  // visible iff 0 <= myq - key < W (keys >= T fail it for real rows)
            const int cst = 8 * (x >> 2) + (x & 3);
            p = (unsigned)(d0 - cst) < (unsigned)W ? p : 0.f;
          }
          dsb[qb][x >> 3][x & 7] = (bf16)(p * (pacc[qb][x] - delta[qb]));
        }
      }
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 ktop = lds_operand_tr(kr + (32 * kb + 16 * kk) * D + 32 * db, D, lane);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) dqacc[qb][db] = mfma32(ktop, dsb[qb][kk], dqacc[qb][db]);
        }
    }
  };

  // Triple-buffered: see attn_fwd.hip.
  auto stage = [&](int t, const bf16* kf, const bf16* kr, const bf16* vf, bf16* kfn, bf16* krn, bf16* vfn) __attribute__((always_inline)) {
    if (t + 1 <= t_hi)
      dma_barrier<PER>();
    else
      dma_barrier<0>();
    if (t + 2 <= t_hi) load_tile(t + 2, kfn, krn, vfn);
    tile_step(t, kf, kr, vf);
  };
  for (int t = t_lo; t <= t_hi; t += 3) {
    stage(t, kf0, kr0, vf0, kf2, kr2, vf2);
    if (t + 1 > t_hi) break;
    stage(t + 1, kf1, kr1, vf1, kf0, kr0, vf0);
    if (t + 2 > t_hi) break;
    stage(t + 2, kf2, kr2, vf2, kf1, kr1, vf1);
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = qw0 + 32 * qb + l32;
    if (myq < T) {
      bf16* dqrow = a.dq + b * a.sdq[0] + h * a.sdq[2] + (int64_t)myq * a.sdq[1];
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x4 v4;
#pragma unroll
          for (int j = 0; j < 4; ++j) v4[j] = (bf16)(dqacc[qb][db][4 * i + j] * a.scale);
          *reinterpret_cast<bf16x4*>(dqrow + 32 * db + 8 * i + 4 * h32) = v4;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// dK, dV.  Per wave, lanes own key columns of S = Q K^T and dP = dO V^T (K and
// V stay in VGPRs as B operands, 64 keys per wave so each LDS operand feeds two
// MFMAs); lse2 and delta of the query rows come from LDS.  dV^T += dO^T P and
// dK^T += Q^T dS read dO^T / Q^T transposed from row-major copies.
// ---------------------------------------------------------------------------
template <int D, int KB, int BMQ, int NBUF>
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv_kernel(BwdArgs a) {
  constexpr int NW = 4, KW = 32 * KB, BNK = NW * KW;
  constexpr int TILE = BMQ * D;
  static_assert(BMQ == 32, "one 32-row query block per tile");
  __shared__ __attribute__((aligned(1024))) bf16 qf0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 qr0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 df0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 dr0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 qf1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 qr1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 df1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16 dr1[TILE];
  static_assert(NBUF == 2 || NBUF == 3, "double or triple buffering");
  constexpr int TILE3 = NBUF == 3 ? TILE : 8;
  __shared__ __attribute__((aligned(1024))) bf16 qf2[TILE3];
  __shared__ __attribute__((aligned(1024))) bf16 qr2[TILE3];
  __shared__ __attribute__((aligned(1024))) bf16 df2[TILE3];
  __shared__ __attribute__((aligned(1024))) bf16 dr2[TILE3];
  __shared__ __attribute__((aligned(256))) float st0[128];  // [0, 64): lse2, [64, 128): delta
  __shared__ __attribute__((aligned(256))) float st1[128];
  __shared__ __attribute__((aligned(256))) float st2[NBUF == 3 ? 128 : 4];
  constexpr int PER = 4 * TILE / 512 / NW;  // bf16 DMA instructions per wave per tile (+1 on waves 0, 1)

  const int T = a.T, W = a.W, H = a.H, Hkv = a.Hkv;
  const int G = H / Hkv;
  const int nkt = (T + BNK - 1) / BNK;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x);
  const int kt = tile % nkt;  // low key tiles see the most queries: they go first
  const int bhk = tile / nkt;
  const int hk = bhk % Hkv, b = bhk / Hkv;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h32 = lane >> 5;
  const int k0 = kt * BNK, kw0 = k0 + KW * wave;

  // K^T / V^T as B operands: lane l of block kb holds k[kw0 + 32 kb + l % 32][16 s + 8 (l / 32) + e].
  bf16x8 kreg[KB][D / 16], vreg[KB][D / 16];
  {
    const __amdgpu_buffer_rsrc_t rk = slab_rsrc(a.k + b * a.sk[0] + hk * a.sk[2], a.sk[1], T, D);
    const __amdgpu_buffer_rsrc_t rv = slab_rsrc(a.v + b * a.sv[0] + hk * a.sv[2], a.sv[1], T, D);
    const int sk2 = (int)(a.sk[1] * 2), sv2 = (int)(a.sv[1] * 2);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        kreg[kb][s] = slab_load(rk, kw0 + 32 * kb + l32, sk2, 16 * s + 8 * h32);
        vreg[kb][s] = slab_load(rv, kw0 + 32 * kb + l32, sv2, 16 * s + 8 * h32);
      }
  }
  drain_vmem();

  const int q_lo = k0;
  const int q_hi = min(T - 1, k0 + BNK - 1 + W - 1);
  const int tq_lo = q_lo / BMQ, tq_hi = q_hi / BMQ;
  const int nq = tq_hi - tq_lo + 1;
  const int n_iter = nq * G;
  const int sq2 = (int)(a.sq[1] * 2), sdo2 = (int)(a.sdo[1] * 2);

  auto load_tile = [&](int it, bf16* qf, bf16* qr, bf16* df, bf16* dr, float* st) __attribute__((always_inline)) {
    const int hq = hk * G + it / nq;
    const int qs = (tq_lo + it % nq) * BMQ;
    const __amdgpu_buffer_rsrc_t rq = slab_rsrc(a.q + b * a.sq[0] + hq * a.sq[2], a.sq[1], T, D);
    const __amdgpu_buffer_rsrc_t rdo = slab_rsrc(a.dout + b * a.sdo[0] + hq * a.sdo[2], a.sdo[1], T, D);
    dma_frags<BMQ, D, NW>(rq, sq2, qs, qf, wave, lane);
    dma_rows<BMQ, D, NW>(rq, sq2, qs, qr, wave, lane);
    dma_frags<BMQ, D, NW>(rdo, sdo2, qs, df, wave, lane);
    dma_rows<BMQ, D, NW>(rdo, sdo2, qs, dr, wave, lane);
    if (wave < 2) {
      // wave 0: lse2 rows qs.., wave 1: delta rows qs.. (fp32, 64 lanes x 4 bytes; rows >= T read 0)
      const int64_t plane = wave == 0 ? (int64_t)(a.B * H) * T : 0;
      const float* base = a.delta + plane + ((int64_t)b * H + hq) * T;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, T * 4, 0x00020000);
      lds_dma<4>(rs, st + 64 * wave, (qs + lane) * 4);
    }
  };
  load_tile(0, qf0, qr0, df0, dr0, st0);
  if (NBUF == 3 && n_iter > 1) load_tile(1, qf1, qr1, df1, dr1, st1);

  f32x16 dkacc[KB][D / 32], dvacc[KB][D / 32];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      dkacc[kb][db] = zero16();
      dvacc[kb][db] = zero16();
    }

  const bool wave_live = kw0 < T;
  const int wk_hi = min(kw0 + KW - 1, T - 1);
  const float c = a.scale_log2;

  auto tile_step = [&](const int it, const bf16* qf, const bf16* qr, const bf16* df, const bf16* dr,
                       const float* st) __attribute__((always_inline)) {
    const int qs = (tq_lo + it % nq) * BMQ;
    if (!(wave_live && qs <= wk_hi + W - 1 && qs + BMQ - 1 >= kw0)) return;
    // Query rows >= T need no mask: their Q, dO, lse2 and delta arrive as zeros,
    // so they add exactly zero to dK and dV.
    const bool full = (qs >= kw0 + KW - 1) && (qs + BMQ - 1 - W + 1 <= kw0);

    f32x16 sacc[KB], pacc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      sacc[kb] = zero16();
      pacc[kb] = zero16();
    }
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const bf16x8 qop = frag_operand<D>(qf, 0, s, lane);
      const bf16x8 dop = frag_operand<D>(df, 0, s, lane);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sacc[kb] = mfma32(qop, kreg[kb][s], sacc[kb]);
        pacc[kb] = mfma32(dop, vreg[kb][s], pacc[kb]);
      }
    }
    bf16x8 pb[KB][2], dsb[KB][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = 8 * i + 4 * h32;
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + r0);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(st + 64 + r0);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int d0 = qs + r0 - (kw0 + 32 * kb + l32);  // query - key, for j = 0
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float p = fast_exp2(fmaf(sacc[kb][4 * i + j], c, -l4[j]));
          if (!full) p = (unsigned)(d0 + j) < (unsigned)W ? p : 0.f;
          pb[kb][i >> 1][4 * (i & 1) + j] = (bf16)p;
          dsb[kb][i >> 1][4 * (i & 1) + j] = (bf16)(p * (pacc[kb][4 * i + j] - d4[j]));
        }
      }
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8 dtop = lds_operand_tr(dr + 16 * kk * D + 32 * db, D, lane);
        const bf16x8 qtop = lds_operand_tr(qr + 16 * kk * D + 32 * db, D, lane);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          dvacc[kb][db] = mfma32(dtop, pb[kb][kk], dvacc[kb][db]);
          dkacc[kb][db] = mfma32(qtop, dsb[kb][kk], dkacc[kb][db]);
        }
      }
  };

  // Triple-buffered: see attn_fwd.hip.  Waves 0 and 1 also copy the row
  // statistics, one more DMA instruction per tile.
  auto stage = [&](int it, const bf16* qf, const bf16* qr, const bf16* df, const bf16* dr, const float* st,
                   bf16* qfn, bf16* qrn, bf16* dfn, bf16* drn, float* stn) __attribute__((always_inline)) {
    if (NBUF == 3 && it + 1 < n_iter) {
      if (wave < 2)
        dma_barrier<PER + 1>();
      else
        dma_barrier<PER>();
    } else {
      dma_barrier<0>();
    }
    if (it + NBUF - 1 < n_iter) load_tile(it + NBUF - 1, qfn, qrn, dfn, drn, stn);
    tile_step(it, qf, qr, df, dr, st);
  };
  if constexpr (NBUF == 3) {
    for (int it = 0; it < n_iter; it += 3) {
      stage(it, qf0, qr0, df0, dr0, st0, qf2, qr2, df2, dr2, st2);
      if (it + 1 >= n_iter) break;
      stage(it + 1, qf1, qr1, df1, dr1, st1, qf0, qr0, df0, dr0, st0);
      if (it + 2 >= n_iter) break;
      stage(it + 2, qf2, qr2, df2, dr2, st2, qf1, qr1, df1, dr1, st1);
    }
  } else {
    for (int it = 0; it < n_iter; it += 2) {
      stage(it, qf0, qr0, df0, dr0, st0, qf1, qr1, df1, dr1, st1);
      if (it + 1 >= n_iter) break;
      stage(it + 1, qf1, qr1, df1, dr1, st1, qf0, qr0, df0, dr0, st0);
    }
  }

#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int mykey = kw0 + 32 * kb + l32;
    if (mykey < T) {
      bf16* dkrow = a.dk + b * a.sdk[0] + hk * a.sdk[2] + (int64_t)mykey * a.sdk[1];
      bf16* dvrow = a.dv + b * a.sdv[0] + hk * a.sdv[2] + (int64_t)mykey * a.sdv[1];
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x4 k4, v4;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            k4[j] = (bf16)(dkacc[kb][db][4 * i + j] * a.scale);
            v4[j] = (bf16)dvacc[kb][db][4 * i + j];
          }
          *reinterpret_cast<bf16x4*>(dkrow + 32 * db + 8 * i + 4 * h32) = k4;
          *reinterpret_cast<bf16x4*>(dvrow + 32 * db + 8 * i + 4 * h32) = v4;
        }
    }
  }
}

template <int D>
hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream, int phases) {
  constexpr int QB = D == 64 ? 2 : 1;
  constexpr int KB = 2;
  if (phases & kBwdDq) {
    constexpr int BM = 4 * 32 * QB;
    const int nqt = (a.T + BM - 1) / BM;
    const int64_t blocks = (int64_t)nqt * a.H * a.B;
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D, QB>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (phases & kBwdDkDv) {
    constexpr int BNK = 4 * 32 * KB;
    const int nkt = (a.T + BNK - 1) / BNK;
    const int64_t blocks = (int64_t)nkt * a.Hkv * a.B;
    // D = 128 stays double-buffered: the triple-buffered variant at this register
    // pressure crashes the ROCm 7.2 compiler (AMDGPU Rewrite AGPR-Copy-MFMA pass).
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, KB, 32, D == 64 ? 3 : 2>), dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

template hipError_t launch_bwd<64>(const BwdArgs&, hipStream_t, int);
template hipError_t launch_bwd<128>(const BwdArgs&, hipStream_t, int);

}  // namespace hlm
