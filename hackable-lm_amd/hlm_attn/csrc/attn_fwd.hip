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
// query column of each score block and the row max / row sum are lane-local
// (plus one swap with lane l ^ 32).  Each K / V^T operand fragment read from
// LDS feeds QB MFMAs, which is what keeps the kernel under the LDS bandwidth.
// K/V tiles of 64 keys are double-buffered through LDS; key tiles outside
// [q0 - W + 1, q_last] are never loaded, so the cost is proportional to T * W,
// and only tiles that cross the diagonal or the window edge evaluate the mask
// per element.
//
// Softmax: exponentials are taken in base 2 with scale * log2(e) folded into
// one FMA; the running max only moves (rescaling O and the row sum) when some
// row's tile max exceeds it by more than kRescaleSlack, so most tiles skip the
// rescale.  The row sum adds the fp32 probabilities (the bf16-rounded ones
// feed only the P V product), which keeps lse within 1e-3 even for windows
// of a few keys, where rounding errors of a bf16 sum would not average out.
#include "attn_common.h"

namespace hlm {

// log2 headroom before the running max must move: probabilities are at most
// 2^kRescaleSlack, far inside fp32 / bf16 range.
constexpr float kRescaleSlack = 8.f;

template <int D, int QB>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(FwdArgs a) {
  constexpr int QW = 32 * QB, BM = 4 * QW, BN = 64, STR = D + 8;
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
  const int q0 = qt * BM, qw0 = q0 + QW * wave;

  const bf16* qbase = a.q + b * a.sq[0] + h * a.sq[2];
  const bf16* kbase = a.k + b * a.sk[0] + hk * a.sk[2];
  const bf16* vbase = a.v + b * a.sv[0] + hk * a.sv[2];

  // Q^T as the B operand: lane l of block qb holds q[qw0 + 32 qb + l % 32][16 s + 8 (l / 32) + e].
  bf16x8 qreg[QB][D / 16];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int myq = qw0 + 32 * qb + l32;
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qreg[qb][s] = myq < T ? *reinterpret_cast<const bf16x8*>(qbase + (int64_t)myq * a.sq[1] + 16 * s + 8 * h32)
                            : zero_bf16x8();
  }

  const int key_lo = max(0, q0 - W + 1);
  const int key_hi = min(T, q0 + BM) - 1;
  const int t_lo = key_lo / BN, t_hi = key_hi / BN;

  RowTile<BN, D> kt, vt;
  kt.load(kbase, a.sk[1], t_lo * BN, T, tid);
  vt.load(vbase, a.sv[1], t_lo * BN, T, tid);
  kt.store(smem, tid);
  vt.store(smem + TILE, tid);
  __syncthreads();

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
      const bool full = (k0 + BN - 1 <= qw0) && (k0 >= qw0 + QW - W) && (k0 + BN <= T);

      f32x16 sacc[QB][BN / 32];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          const bf16x8 kop = lds_operand(ks + 32 * kb * STR + 16 * s, STR, lane);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) sacc[qb][kb] = mfma32(kop, qreg[qb][s], sacc[qb][kb]);
        }
      }
      if (!full) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const int myq = qw0 + 32 * qb + l32;
#pragma unroll
          for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
            for (int x = 0; x < 16; ++x) {
              const int key = k0 + 32 * kb + 8 * (x >> 2) + 4 * h32 + (x & 3);
              const bool ok = key <= myq && key > myq - W && key < T;
              if (!ok) sacc[qb][kb][x] = -INFINITY;
            }
        }
      }

      bf16x8 pb[QB][BN / 16];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float tmax = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int x = 0; x < 16; ++x) tmax = fmaxf(tmax, sacc[qb][kb][x]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32)) * c;
        if (__any(tmax > m[qb] + kRescaleSlack)) {
          const float mnew = fmaxf(m[qb], tmax);
          const float alpha = mnew == -INFINITY ? 1.f : fast_exp2(m[qb] - mnew);
          m[qb] = mnew;
          lsum[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int x = 0; x < 16; ++x) oacc[qb][db][x] *= alpha;
        }
        const float mref = m[qb] == -INFINITY ? 0.f : m[qb];
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float p = fast_exp2(fmaf(sacc[qb][kb][8 * t2 + e], c, -mref));
              lsum[qb] += p;
              pb[qb][2 * kb + t2][e] = (bf16)p;
            }
          }
      }
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int kk = 0; kk < BN / 16; ++kk) {
          const bf16x8 vop = lds_operand_tr(vs + 16 * kk * STR + 32 * db, STR, lane);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) oacc[qb][db] = mfma32(vop, pb[qb][kk], oacc[qb][db]);
        }
    }
    if (t < t_hi) {
      kt.store(smem + (buf ^ 1) * 2 * TILE, tid);
      vt.store(smem + (buf ^ 1) * 2 * TILE + TILE, tid);
    }
    __syncthreads();
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

template <int D, int QB>
hipError_t launch_fwd_qb(const FwdArgs& a, hipStream_t stream) {
  constexpr int BM = 4 * 32 * QB;
  const int nqt = (a.T + BM - 1) / BM;
  const int64_t blocks = (int64_t)nqt * a.H * a.B;
  hipLaunchKernelGGL((attn_fwd_kernel<D, QB>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  return launch_fwd_qb<D, kFwdQB>(a, stream);
}

template hipError_t launch_fwd<64>(const FwdArgs&, hipStream_t);
template hipError_t launch_fwd<128>(const FwdArgs&, hipStream_t);

}  // namespace hlm
