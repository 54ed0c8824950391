// Cross-entropy rows of the LM head's fused linear + cross-entropy: for each
// row of logits x (V values) and its target t,
//   lse     = log sum_j exp(x_j)
//   loss    = (lse - x_t) / n_tokens
//   x_j    <- (exp(x_j - lse) - [j == t]) / n_tokens      (in place)
// i.e. the per-row loss and the gradient of the mean loss with respect to the
// logits, which the caller multiplies into the two GEMMs of the backward.
// This is hackable-lm's Triton _linear_ce_kernel (kernels.py:286-316, op
// :320-336), computed in fp32 from bf16 or fp32 logits.  A target equal to
// ignore_index (-100, F.cross_entropy's default, as the torch path of
// model.py:333-341 uses) contributes a zero loss and a zero gradient row; any
// other target outside [0, V) yields NaN for the row's loss and gradient (the
// kernel cannot raise).
//
// Memory-bound: one workgroup per row.  When rows are 16-byte aligned (V and
// the row stride multiples of 16 / sizeof(T)), the row is read once into
// registers in 16-byte chunks (chunk k of thread i holds elements
// 16/sizeof(T) * (i + 256 k) ..), reduced (max, then sum of exponentials) with
// wave shuffles and one LDS exchange between the 4 waves, and written once:
// 2 * V * sizeof(T) bytes per row.  Other layouts take a generic path that
// reads the row three times (max, sum, write), one element per lane.
#include "attn_common.h"

namespace hlm {

struct CeArgs {
  void* logits;            // (n_rows, >= V) rows at row_stride elements
  int64_t row_stride;
  const int64_t* targets;  // n_rows
  float* loss;             // n_rows
  int n_rows, V;
  float inv_n;             // 1 / n_tokens
  int ignore_index;
};

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return (float)x;
}

// Block-wide reductions over 256 threads (4 waves): every thread gets the result.
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  v = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return v;
}

// Row status from its target: 0 = valid, 1 = ignored, 2 = out of range.
__device__ __forceinline__ int target_status(int64_t t, int V, int ignore_index) {
  if (t >= 0 && t < V) return 0;
  return t == ignore_index ? 1 : 2;
}

template <typename T, int K>
__global__ __launch_bounds__(256) void ce_rows_vec_kernel(CeArgs a) {
  constexpr int E = 16 / sizeof(T);  // elements per 16-byte chunk
  typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  T* base = static_cast<T*>(a.logits) + (int64_t)row * a.row_stride;
  const int V = a.V;
  const int64_t tgt = a.targets[row];
  const int status = target_status(tgt, V, a.ignore_index);
  // The target's logit, read before any thread of the block stores (the
  // stores follow two block barriers).
  float xt = 0.f;
  if (tid == 0 && status == 0) xt = to_f32(base[tgt]);

  u32x4 raw[K];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int idx = E * (tid + 256 * k);
    raw[k] = u32x4{};
    if (idx < V) raw[k] = *reinterpret_cast<const u32x4*>(base + idx);
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (E * (tid + 256 * k) >= V) continue;
    const T* v = reinterpret_cast<const T*>(&raw[k]);
#pragma unroll
    for (int e = 0; e < E; ++e) m = fmaxf(m, to_f32(v[e]));
  }
  const float M = block_max(m, red);
  const float c = M * kLog2e;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (E * (tid + 256 * k) >= V) continue;
    const T* v = reinterpret_cast<const T*>(&raw[k]);
#pragma unroll
    for (int e = 0; e < E; ++e) s += fast_exp2(fmaf(to_f32(v[e]), kLog2e, -c));
  }
  const float S = block_sum(s, red);
  const float lse = M + __log2f(S) * kLn2;
  if (tid == 0) a.loss[row] = status == 0 ? (lse - xt) * a.inv_n : status == 1 ? 0.f : NAN;
  // gradient: (p_j - [j == t]) / n, p_j = 2^(x_j log2e - c) / S
  const float scale = status == 0 ? a.inv_n / S : status == 1 ? 0.f : NAN;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int idx = E * (tid + 256 * k);
    if (idx >= V) continue;
    const T* v = reinterpret_cast<const T*>(&raw[k]);
    u32x4 outw;
    T* o = reinterpret_cast<T*>(&outw);
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = (T)(fast_exp2(fmaf(to_f32(v[e]), kLog2e, -c)) * scale);
    // The target's gradient, p_t / S - 1 / n, rounded once as above: one test
    // per chunk instead of one per element (the lane holding the target redoes
    // its element; the others skip the branch).
    if (status == 0 && (uint64_t)(tgt - idx) < (uint64_t)E) {
      const int et = (int)(tgt - idx);
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (e == et) o[e] = (T)(fast_exp2(fmaf(to_f32(v[e]), kLog2e, -c)) * scale - a.inv_n);
    }
    *reinterpret_cast<u32x4*>(base + idx) = outw;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ce_rows_generic_kernel(CeArgs a) {
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  T* base = static_cast<T*>(a.logits) + (int64_t)row * a.row_stride;
  const int V = a.V;
  const int64_t tgt = a.targets[row];
  const int status = target_status(tgt, V, a.ignore_index);
  float xt = 0.f;
  if (tid == 0 && status == 0) xt = to_f32(base[tgt]);
  float m = -INFINITY;
  for (int j = tid; j < V; j += 256) m = fmaxf(m, to_f32(base[j]));
  const float M = block_max(m, red);
  const float c = M * kLog2e;
  float s = 0.f;
  for (int j = tid; j < V; j += 256) s += fast_exp2(fmaf(to_f32(base[j]), kLog2e, -c));
  const float S = block_sum(s, red);  // its barriers order every read above before the stores below
  const float lse = M + __log2f(S) * kLn2;
  if (tid == 0) a.loss[row] = status == 0 ? (lse - xt) * a.inv_n : status == 1 ? 0.f : NAN;
  const float scale = status == 0 ? a.inv_n / S : status == 1 ? 0.f : NAN;
  for (int j = tid; j < V; j += 256) {
    float g = fast_exp2(fmaf(to_f32(base[j]), kLog2e, -c)) * scale;
    if (status == 0 && j == tgt) g -= a.inv_n;
    base[j] = (T)g;
  }
}

template <typename T>
hipError_t launch_ce_rows_typed(const CeArgs& a, bool vec, hipStream_t stream) {
  const dim3 grid((unsigned)a.n_rows), block(256);
  if (!vec) {
    hipLaunchKernelGGL((ce_rows_generic_kernel<T>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  constexpr int E = 16 / sizeof(T);
  const int chunks = (a.V + 256 * E - 1) / (256 * E);  // 16-byte chunks per thread
  if (chunks <= 1)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 1>), grid, block, 0, stream, a);
  else if (chunks <= 2)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 2>), grid, block, 0, stream, a);
  else if (chunks <= 4)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 4>), grid, block, 0, stream, a);
  else if (chunks <= 8)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 8>), grid, block, 0, stream, a);
  else if (chunks <= 16)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 16>), grid, block, 0, stream, a);
  else if (chunks <= 32)
    hipLaunchKernelGGL((ce_rows_vec_kernel<T, 32>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((ce_rows_generic_kernel<T>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// Entry from the C ABI: rows are 16-byte aligned when the base, V and the row
// stride allow it (then the register-resident path is used).
hipError_t launch_ce_rows(void* logits, bool bf16_logits, int64_t row_stride, const int64_t* targets, float* loss,
                          int n_rows, int V, float inv_n, int ignore_index, hipStream_t stream) {
  CeArgs a{logits, row_stride, targets, loss, n_rows, V, inv_n, ignore_index};
  if (n_rows == 0) return hipSuccess;
  const int E = bf16_logits ? 8 : 4;
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && V % E == 0 && row_stride % E == 0;
  return bf16_logits ? launch_ce_rows_typed<bf16>(a, vec, stream) : launch_ce_rows_typed<float>(a, vec, stream);
}

}  // namespace hlm
