// Residual add + RMSNorm (no weight) after the attention output projection
// and the MLP down projection: per row of n values,
//   out    = residual + branch                      (rounded to bf16: the new residual stream)
//   normed = out * rsqrt(mean(out^2) + eps)         (from the rounded out, fp32, rounded once)
// -- hackable-lm's residual_rms_norm (model.py:73-75), used by
// OutputProjection.fwd_torch (model.py:261-264) and DownProjection.fwd_torch
// (model.py:303-304).  Backward, with r = rsqrt(mean(out^2) + eps), z = out r:
//   grad_in = grad_out + r (grad_normed - z mean(grad_normed z))
// which is the gradient of both residual and branch.
//
// Memory-bound: one wave per row, 4 rows per workgroup; a lane holds chunks
// of 8 values (16 bytes) at elements 8 (lane + 64 j), so each wave
// instruction moves 1 KB of one row, coalesced; the row's sums are wave
// shuffles (no LDS, no barrier).  Forward: 2 reads + 2 writes of 2n bytes
// per row; backward: 3 reads + 1 write.  Every byte is touched once, so loads
// and stores are non-temporal (12% faster than cached ones on the MI355X).
#include "attn_common.h"

namespace hlm {

struct ResNormArgs {
  const bf16* a;   // forward: residual; backward: out (the forward's first output)
  const bf16* b;   // forward: branch;   backward: grad_out
  const bf16* c;   // backward: grad_normed
  bf16* y0;        // forward: out;      backward: grad_in
  bf16* y1;        // forward: normed
  int64_t rows;
  int n;           // multiple of 8
  float eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

template <int J, bool BWD>
__global__ __launch_bounds__(256) void residual_rms_norm_kernel(ResNormArgs p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= p.rows) return;  // the whole wave leaves; nothing below synchronises waves
  const int n = p.n;
  const int64_t base = row * n;
  bf16x8 va[J], vb[J], vc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e0 = 8 * (lane + 64 * j);
    va[j] = vb[j] = vc[j] = bf16x8{};
    if (e0 < n) {
      va[j] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p.a + base + e0));
      vb[j] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p.b + base + e0));
      if constexpr (BWD) vc[j] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p.c + base + e0));
    }
  }
  if constexpr (!BWD) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        va[j][e] = (bf16)((float)va[j][e] + (float)vb[j][e]);  // out, rounded as the bf16 add rounds it
        const float o = (float)va[j][e];
        ss = fmaf(o, o, ss);
      }
    const float r = rsqrtf(wave_sum(ss) / (float)n + p.eps);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e0 = 8 * (lane + 64 * j);
      if (e0 >= n) continue;
      bf16x8 z;
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (bf16)((float)va[j][e] * r);
      __builtin_nontemporal_store(va[j], reinterpret_cast<bf16x8*>(p.y0 + base + e0));
      __builtin_nontemporal_store(z, reinterpret_cast<bf16x8*>(p.y1 + base + e0));
    }
  } else {
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float o = (float)va[j][e];
        ss = fmaf(o, o, ss);
        dot = fmaf((float)vc[j][e], o, dot);
      }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    const float r = rsqrtf(ss / (float)n + p.eps);
    // mean(grad_normed * z) = r * dot / n;  grad_in = grad_out + r gn - r^2 out * mean(gn z)
    const float k = r * r * (r * dot / (float)n);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e0 = 8 * (lane + 64 * j);
      if (e0 >= n) continue;
      bf16x8 g;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        g[e] = (bf16)((float)vb[j][e] + fmaf(r, (float)vc[j][e], -k * (float)va[j][e]));
      __builtin_nontemporal_store(g, reinterpret_cast<bf16x8*>(p.y0 + base + e0));
    }
  }
}

template <bool BWD>
hipError_t launch_res_norm(const ResNormArgs& p, hipStream_t stream) {
  const int64_t blocks = (p.rows + 3) / 4;
  const int chunks = (p.n / 8 + 63) / 64;  // 16-byte chunks per lane
  const dim3 grid((unsigned)blocks), block(256);
  if (chunks <= 1)
    hipLaunchKernelGGL((residual_rms_norm_kernel<1, BWD>), grid, block, 0, stream, p);
  else if (chunks <= 2)
    hipLaunchKernelGGL((residual_rms_norm_kernel<2, BWD>), grid, block, 0, stream, p);
  else if (chunks <= 4)
    hipLaunchKernelGGL((residual_rms_norm_kernel<4, BWD>), grid, block, 0, stream, p);
  else if (chunks <= 8)
    hipLaunchKernelGGL((residual_rms_norm_kernel<8, BWD>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((residual_rms_norm_kernel<16, BWD>), grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_residual_rms_norm(const void* a, const void* b, const void* c, void* y0, void* y1, int64_t rows,
                                    int n, float eps, bool backward, hipStream_t stream) {
  ResNormArgs p{static_cast<const bf16*>(a), static_cast<const bf16*>(b), static_cast<const bf16*>(c),
                static_cast<bf16*>(y0), static_cast<bf16*>(y1), rows, n, eps};
  if (rows == 0) return hipSuccess;
  return backward ? launch_res_norm<true>(p, stream) : launch_res_norm<false>(p, stream);
}

}  // namespace hlm
