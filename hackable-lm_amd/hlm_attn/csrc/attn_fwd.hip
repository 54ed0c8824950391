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
// Work split: one workgroup (4 waves) per 128-query tile of one (batch, head);
// wave w owns queries q0 + 32 w .. + 31.  Each wave keeps its Q^T slice in
// VGPRs as the B operand of S^T = K Q^T, so every lane owns one query column
// of the score block and the row max / row sum are lane-local (plus one swap
// with lane l ^ 32).  K/V tiles of 64 keys are double-buffered through LDS;
// key tiles outside [q0 - W + 1, q0 + 127] are never loaded, so the cost is
// proportional to T * W, and only tiles that cross the diagonal or the window
// edge evaluate the mask per element.
#include "attn_common.h"

namespace hlm {

template <int D>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(FwdArgs a) {
  constexpr int BM = 128, BN = 64, STR = D + 8;
  constexpr int TILE = BN * STR;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * 2 * TILE];  // [buf][K, V]

  const int T = a.T, W = a.W, H = a.H;
  const int nqt = (T + BM - 1) / BM;
  const int tile = xcd_swizzle(blockIdx.x, gridDim.x);
  const int qt = nqt - 1 - tile % nqt;  // longest causal rows first within a head
  const int bh = tile / nqt;
  const int h = bh % H, b = bh / H;
  const int hk = h / (H / a.Hkv);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, h32 = lane >> 5;
  const int q0 = qt * BM, qw0 = q0 + 32 * wave, myq = qw0 + l32;

  const bf16* qbase = a.q + b * a.sq[0] + h * a.sq[2];
  const bf16* kbase = a.k + b * a.sk[0] + hk * a.sk[2];
  const bf16* vbase = a.v + b * a.sv[0] + hk * a.sv[2];

  // Q^T as the B operand: lane l holds q[myq][16 s + 8 (l / 32) + e].
  bf16x8 qreg[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qreg[s] = myq < T ? *reinterpret_cast<const bf16x8*>(qbase + (int64_t)myq * a.sq[1] + 16 * s + 8 * h32)
                      : zero_bf16x8();

  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, t_hi = key_hi / BN;

  RowTile<BN, D> kt, vt;
  kt.load(kbase, a.sk[1], t_lo * BN, T, tid);
  vt.load(vbase, a.sv[1], t_lo * BN, T, tid);
  kt.store(smem, tid);
  vt.store(smem + TILE, tid);
  __syncthreads();

  f32x16 oacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) oacc[db] = zero16();
  float m = -INFINITY;  // running max of scale*log2(e)*s for this lane's query
  float lsum = 0.f;     // this lane's share of the running row sum

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

      f32x16 sacc[BN / 32];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
        sacc[kb] = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s)
          sacc[kb] = mfma32(lds_operand(ks + 32 * kb * STR + 16 * s, STR, lane), qreg[s], sacc[kb]);
      }
      if (!full) {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int key = k0 + 32 * kb + 8 * i + 4 * h32 + j;
              const bool ok = key <= myq && key > myq - W && key < T;
              if (!ok) sacc[kb][4 * i + j] = -INFINITY;
            }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[kb][x]);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
      const float mnew = fmaxf(m, tmax * c);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = fast_exp2(m - mref);
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int x = 0; x < 16; ++x) oacc[db][x] *= alpha;

      bf16x8 pb[BN / 16];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p = fast_exp2(fmaf(sacc[kb][8 * t2 + e], c, -mref));
            lsum += p;
            pb[2 * kb + t2][e] = (bf16)p;
          }
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int kk = 0; kk < BN / 16; ++kk)
          oacc[db] = mfma32(lds_operand_tr(vs + 16 * kk * STR + 32 * db, STR, lane), pb[kk], oacc[db]);
    }
    if (t < t_hi) {
      kt.store(smem + (buf ^ 1) * 2 * TILE, tid);
      vt.store(smem + (buf ^ 1) * 2 * TILE + TILE, tid);
    }
    __syncthreads();
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  if (myq < T) {
    const float inv = 1.f / ltot;
    bf16* obase = a.o + b * a.so[0] + (int64_t)myq * a.so[1] + h * a.so[2];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x4 v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = (bf16)(oacc[db][4 * i + j] * inv);
        *reinterpret_cast<bf16x4*>(obase + 32 * db + 8 * i + 4 * h32) = v4;
      }
    if (h32 == 0) a.lse[(int64_t)bh * T + myq] = (m + __log2f(ltot)) * kLn2;
  }
}

template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  const int nqt = (a.T + 127) / 128;
  const int64_t blocks = (int64_t)nqt * a.H * a.B;
  hipLaunchKernelGGL(attn_fwd_kernel<D>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template hipError_t launch_fwd<64>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd<128>(const FwdArgs&, hipStream_t);

}  // namespace hlm
