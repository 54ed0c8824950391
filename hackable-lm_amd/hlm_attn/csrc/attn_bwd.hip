// Backward pass of causal sliding-window attention for gfx950.
//
// With S = scale * Q K^T (masked), P = exp(S - lse), the gradients are
//   delta_i = sum_d dO[i,d] O[i,d]
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q
// i.e. the autograd of hackable-lm's `torch` backend (kernels.py:785-800),
// with P recomputed from the saved lse instead of stored.
//
// Two kernels, no atomics:
//   attn_bwd_dq_kernel    query-stationary: one workgroup per 128-query tile.
//                         Computes delta (written for the next kernel) and dQ.
//   attn_bwd_dkdv_kernel  key-stationary: one workgroup per 128-key tile of one
//                         kv head; loops over the query heads of its group and
//                         the query tiles that can see its keys, accumulating
//                         dK and dV in registers.
// Both skip whole tiles outside the causal window, so cost scales with T * W.
#include "attn_common.h"

namespace hlm {

// ---------------------------------------------------------------------------
// dQ (+ delta).  Same orientation as the forward: per wave, lanes own query
// columns of S^T = K Q^T and dP^T = V dO^T, so lse and delta are per-lane
// scalars; dQ^T += K^T dS^T reads K^T straight from the row-major K tile.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_dq_kernel(BwdArgs a) {
  constexpr int BM = 128, BN = 64, STR = D + 8;
  constexpr int TILE = BN * STR;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * 2 * TILE];  // [buf][K, V]

  const int T = a.T, W = a.W, H = a.H;
  const int nqt = (T + BM - 1) / BM;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x);
  const int qt = nqt - 1 - tile % nqt;
  const int bh = tile / nqt;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + 32 * wave, myq = qw0 + l32;
  const bool qok = myq < T;

  const bf16* qrow = a.q + b * a.sq[0] + h * a.sq[2] + (int64_t)myq * a.sq[1];
  const bf16* dorow = a.dout + b * a.sdo[0] + h * a.sdo[2] + (int64_t)myq * a.sdo[1];
  const bf16* orow = a.o + b * a.so[0] + h * a.so[2] + (int64_t)myq * a.so[1];
  const bf16* kbase = a.k + b * a.sk[0] + hk * a.sk[2];
  const bf16* vbase = a.v + b * a.sv[0] + hk * a.sv[2];

  bf16x8 qreg[D / 16], doreg[D / 16];
  float dpart = 0.f;
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const int d0 = 16 * s + 8 * h32;
    if (qok) {
      qreg[s] = *reinterpret_cast<const bf16x8*>(qrow + d0);
      doreg[s] = *reinterpret_cast<const bf16x8*>(dorow + d0);
      const bf16x8 o8 = *reinterpret_cast<const bf16x8*>(orow + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += (float)doreg[s][e] * (float)o8[e];
    } else {
      qreg[s] = zero_bf16x8();
      doreg[s] = zero_bf16x8();
    }
  }
  const float delta = dpart + __shfl_xor(dpart, 32);
  const float lse2 = qok ? a.lse[(int64_t)bh * T + myq] * kLog2e : 0.f;
  if (qok && h32 == 0) a.delta[(int64_t)bh * T + myq] = delta;

  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, t_hi = key_hi / BN;

  RowTile<BN, D> kt, vt;
  kt.load(kbase, a.sk[1], t_lo * BN, T, tid);
  vt.load(vbase, a.sv[1], t_lo * BN, T, tid);
  kt.store(smem, tid);
  vt.store(smem + TILE, tid);
  __syncthreads();

  f32x16 dqacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) dqacc[db] = zero16();

  const bool wave_live = qw0 < T;
  const int wq_hi = min(qw0 + 31, T - 1);
  const float c = a.scale_log2;

  for (int t = t_lo; t <= t_hi; ++t) {
    const int buf = (t - t_lo) & 1;
    if (t < t_hi) {
      kt.load(kbase, a.sk[1], (t + 1) * BN, T, tid);
      vt.load(vbase, a.sv[1], (t + 1) * BN, T, tid);
    }
    const int k0 = t * BN;
    const bool active = wave_live && k0 <= wq_hi && k0 + BN - 1 >= qw0 - W + 1;
    if (active) {
      const bf16* ks = smem + buf * 2 * TILE;
      const bf16* vs = ks + TILE;
      const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + 31 - W + 1) && (k0 + BN <= T);

      f32x16 sacc[BN / 32], pacc[BN / 32];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
        sacc[kb] = zero16();
        pacc[kb] = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          sacc[kb] = mfma32(lds_operand(ks + 32 * kb * STR + 16 * s, STR, lane), qreg[s], sacc[kb]);
          pacc[kb] = mfma32(lds_operand(vs + 32 * kb * STR + 16 * s, STR, lane), doreg[s], pacc[kb]);
        }
      }
      bf16x8 dsb[BN / 16];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          float p = fast_exp2(fmaf(sacc[kb][x], c, -lse2));
          if (!full) {
            const int key = k0 + 32 * kb + 8 * (x >> 2) + 4 * h32 + (x & 3);
            const bool ok = key <= myq && key > myq - W && key < T;
            p = ok ? p : 0.f;
          }
          dsb[2 * kb + (x >> 3)][x & 7] = (bf16)(p * (pacc[kb][x] - delta));
        }
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int kk = 0; kk < BN / 16; ++kk)
          dqacc[db] = mfma32(lds_operand_tr(ks + 16 * kk * STR + 32 * db, STR, lane), dsb[kk], dqacc[db]);
    }
    if (t < t_hi) {
      kt.store(smem + (buf ^ 1) * 2 * TILE, tid);
      vt.store(smem + (buf ^ 1) * 2 * TILE + TILE, tid);
    }
    __syncthreads();
  }

  if (qok) {
    bf16* dqrow = a.dq + b * a.sdq[0] + h * a.sdq[2] + (int64_t)myq * a.sdq[1];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x4 v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = (bf16)(dqacc[db][4 * i + j] * a.scale);
        *reinterpret_cast<bf16x4*>(dqrow + 32 * db + 8 * i + 4 * h32) = v4;
      }
  }
}

// ---------------------------------------------------------------------------
// dK, dV.  Per wave, lanes own key columns of S = Q K^T and dP = dO V^T (K and
// V stay in VGPRs as B operands); lse and delta of the query rows come from
// LDS.  dV^T += dO^T P and dK^T += Q^T dS read dO^T / Q^T straight from the
// row-major Q / dO tiles.
// ---------------------------------------------------------------------------
template <int D, int BMQ>
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv_kernel(BwdArgs a) {
  constexpr int BN = 128, STR = D + 8;
  constexpr int TILE = BMQ * STR;
  constexpr int BUF = 2 * TILE;  // Q, dO
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * BUF];
  __shared__ __attribute__((aligned(16))) float rowstat[2][2][BMQ];  // [buf][lse2, delta]
  static_assert(2 * BMQ <= kThreads, "one thread per lse/delta value");

  const int T = a.T, W = a.W, H = a.H, Hkv = a.Hkv;
  const int G = H / Hkv;
  const int nkt = (T + BN - 1) / BN;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x);
  const int kt = tile % nkt;  // low key tiles see the most queries: they go first
  const int bhk = tile / nkt;
  const int hk = bhk % Hkv, b = bhk / Hkv;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;
  const int k0 = kt * BN, kw0 = k0 + 32 * wave, mykey = kw0 + l32;
  const bool kok = mykey < T;

  // K^T / V^T as B operands: lane l holds k[mykey][16 s + 8 (l / 32) + e].
  bf16x8 kreg[D / 16], vreg[D / 16];
  {
    const bf16* krow = a.k + b * a.sk[0] + hk * a.sk[2] + (int64_t)mykey * a.sk[1];
    const bf16* vrow = a.v + b * a.sv[0] + hk * a.sv[2] + (int64_t)mykey * a.sv[1];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const int d0 = 16 * s + 8 * h32;
      kreg[s] = kok ? *reinterpret_cast<const bf16x8*>(krow + d0) : zero_bf16x8();
      vreg[s] = kok ? *reinterpret_cast<const bf16x8*>(vrow + d0) : zero_bf16x8();
    }
  }

  const int q_lo = k0;
  const int q_hi = min(T - 1, k0 + BN - 1 + W - 1);
  const int tq_lo = q_lo / BMQ, tq_hi = q_hi / BMQ;
  const int nq = tq_hi - tq_lo + 1;
  const int n_iter = nq * G;

  const bool wave_live = kw0 < T;
  const int wk_hi = min(kw0 + 31, T - 1);
  const float c = a.scale_log2;

  RowTile<BMQ, D> qtl, dotl;
  float stat = 0.f;
  auto load = [&](int it) {
    const int hq = hk * G + it / nq;
    const int qs = (tq_lo + it % nq) * BMQ;
    const int64_t bhq = (int64_t)b * H + hq;
    qtl.load(a.q + b * a.sq[0] + hq * a.sq[2], a.sq[1], qs, T, tid);
    dotl.load(a.dout + b * a.sdo[0] + hq * a.sdo[2], a.sdo[1], qs, T, tid);
    if (tid < 2 * BMQ) {
      const int r = tid % BMQ, qi = qs + r;
      stat = 0.f;
      if (qi < T) stat = tid < BMQ ? a.lse[bhq * T + qi] * kLog2e : a.delta[bhq * T + qi];
    }
  };
  auto store = [&](int buf) {
    qtl.store(smem + buf * BUF, tid);
    dotl.store(smem + buf * BUF + TILE, tid);
    if (tid < 2 * BMQ) rowstat[buf][tid / BMQ][tid % BMQ] = stat;
  };

  f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dkacc[db] = zero16();
    dvacc[db] = zero16();
  }

  load(0);
  store(0);
  __syncthreads();

  for (int it = 0; it < n_iter; ++it) {
    const int buf = it & 1;
    if (it + 1 < n_iter) load(it + 1);
    const int qs = (tq_lo + it % nq) * BMQ;
    const bool active = wave_live && qs <= wk_hi + W - 1 && qs + BMQ - 1 >= kw0;
    if (active) {
      const bf16* qsm = smem + buf * BUF;
      const bf16* dosm = qsm + TILE;
      const float* lse2s = rowstat[buf][0];
      const float* dels = rowstat[buf][1];
      const bool full = (qs >= kw0 + 31) && (qs + BMQ - 1 - W + 1 <= kw0) && (qs + BMQ <= T) && (kw0 + 32 <= T);

      f32x16 sacc[BMQ / 32], pacc[BMQ / 32];
#pragma unroll
      for (int qb = 0; qb < BMQ / 32; ++qb) {
        sacc[qb] = zero16();
        pacc[qb] = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          sacc[qb] = mfma32(lds_operand(qsm + 32 * qb * STR + 16 * s, STR, lane), kreg[s], sacc[qb]);
          pacc[qb] = mfma32(lds_operand(dosm + 32 * qb * STR + 16 * s, STR, lane), vreg[s], pacc[qb]);
        }
      }
      bf16x8 pb[BMQ / 16], dsb[BMQ / 16];
#pragma unroll
      for (int qb = 0; qb < BMQ / 32; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r0 = 32 * qb + 8 * i + 4 * h32;
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2s + r0);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(dels + r0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float p = fast_exp2(fmaf(sacc[qb][4 * i + j], c, -l4[j]));
            if (!full) {
              const int qi = qs + r0 + j;
              const bool ok = mykey <= qi && mykey > qi - W && qi < T;
              p = ok ? p : 0.f;
            }
            const float ds = p * (pacc[qb][4 * i + j] - d4[j]);
            pb[2 * qb + (i >> 1)][4 * (i & 1) + j] = (bf16)p;
            dsb[2 * qb + (i >> 1)][4 * (i & 1) + j] = (bf16)ds;
          }
        }
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int kk = 0; kk < BMQ / 16; ++kk) {
          dvacc[db] = mfma32(lds_operand_tr(dosm + 16 * kk * STR + 32 * db, STR, lane), pb[kk], dvacc[db]);
          dkacc[db] = mfma32(lds_operand_tr(qsm + 16 * kk * STR + 32 * db, STR, lane), dsb[kk], dkacc[db]);
        }
    }
    if (it + 1 < n_iter) store(buf ^ 1);
    __syncthreads();
  }

  if (kok) {
    bf16* dkrow = a.dk + b * a.sdk[0] + hk * a.sdk[2] + (int64_t)mykey * a.sdk[1];
    bf16* dvrow = a.dv + b * a.sdv[0] + hk * a.sdv[2] + (int64_t)mykey * a.sdv[1];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x4 k4, v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          k4[j] = (bf16)(dkacc[db][4 * i + j] * a.scale);
          v4[j] = (bf16)dvacc[db][4 * i + j];
        }
        *reinterpret_cast<bf16x4*>(dkrow + 32 * db + 8 * i + 4 * h32) = k4;
        *reinterpret_cast<bf16x4*>(dvrow + 32 * db + 8 * i + 4 * h32) = v4;
      }
  }
}

template <int D>
hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream, int phases) {
  if (phases & kBwdDq) {
    const int nqt = (a.T + 127) / 128;
    const int64_t dq_blocks = (int64_t)nqt * a.H * a.B;
    hipLaunchKernelGGL(attn_bwd_dq_kernel<D>, dim3((unsigned)dq_blocks), dim3(kThreads), 0, stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (phases & kBwdDkDv) {
    const int nkt = (a.T + 127) / 128;
    const int64_t kv_blocks = (int64_t)nkt * a.Hkv * a.B;
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<D, 64>), dim3((unsigned)kv_blocks), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

template hipError_t launch_bwd<64>(const BwdArgs&, hipStream_t, int);
template hipError_t launch_bwd<128>(const BwdArgs&, hipStream_t, int);

}  // namespace hlm
