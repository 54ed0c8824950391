// Fused RMSNorm (no weight) + partial rotary embedding of the q and k rows
// that feed attention: the producer step before the attention kernels.
//
// Per row x (D values of one (batch, time, head) of q or k), in fp32:
//   z = x * rsqrt(mean(x^2) + eps)
//   out[d] = z[d] c - z[d + h] s     d <  h
//   out[d] = z[d] c + z[d - h] s     h <= d < R
//   out[d] = z[d]                    d >= R
// with R the rotary width, h = R / 2, c = cos[t][d mod h], s = sin[t][d mod h]
// -- hackable-lm's QKVProjection.fwd_torch (model.py:101-115) and its Triton
// kernel (kernels.py:441-535).  The backward (kernels.py:541-665, and the
// closed form of kernels.py:703-741) rotates the incoming gradient back,
//   gn[d] = g[d] c + g[d + h] s  (d < h),  g[d] c - g[d - h] s  (h <= d < R),
//   g[d] otherwise,
// and applies the RMSNorm backward  dx = r (gn - z mean(gn z)),  r = rsqrt(...).
//
// Memory-bound: each row is read once (twice with its gradient) and written
// once, and runs at about the speed of a device copy of the same bytes.  A row
// of D bf16 is D / 8 lanes of 16 bytes, so a wave covers 64 / (D/8) whole rows
// per instruction (fully coalesced when the rows are contiguous, as q and k are
// after the projection's view); the row's sum of squares is a shuffle
// reduction over its lanes, and the rotation partner of lane c's 8 values is
// lane c +- h / 8 of the same row (R a multiple of 16).  One row per thread
// keeps the kernel at 8 waves per SIMD, which hides HBM latency better than
// several rows per thread at fewer waves; only the rotary lanes read the
// (L2-resident) tables, in their own element type (fp32 or bf16).  The
// outputs are contiguous (B, T, heads, D) and written with non-temporal
// stores: nothing reads them again before the attention kernels.
#include "attn_common.h"

namespace hlm {

// Cross-lane moves inside a row's lanes by DPP (no LDS round trip):
// quad_perm [1,0,3,2] is lane ^ 1, [2,3,0,1] lane ^ 2; row_half_mirror maps
// lane i of each 8 to 7 - i, row_mirror lane i of each 16 to 15 - i.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Sum over each aligned group of G = 8 or 16 lanes, every lane getting it:
// after the two quad steps each lane holds its quad's sum, and a mirror
// pairs every lane with one of the other quad (then of the other 8).  The
// additions pair the same values as a lane ^ 1, ^ 2, ^ 4 (, ^ 8) butterfly.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 8 || G == 16, "rows of 8 or 16 lanes");
  v += dpp_mov<kDppXor1>(v);
  v += dpp_mov<kDppXor2>(v);
  v += dpp_mov<kDppHalfMirror>(v);
  if constexpr (G == 16) v += dpp_mov<kDppMirror>(v);
  return v;
}

// The rotation partner's value: lane ^ 1 (R = 16) or lane ^ 2 (R = 32) by
// DPP, otherwise lane +- R / 16 through the LDS crossbar.
__device__ __forceinline__ void partner_values(const float (&v)[8], float (&out)[8], int hp, int partner) {
  if (hp == 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = dpp_mov<kDppXor1>(v[e]);
  } else if (hp == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = dpp_mov<kDppXor2>(v[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = __shfl(v[e], partner);
  }
}

template <int D, bool BWD, typename Tab>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QkNormRopeArgs a) {
  constexpr int LPR = D / 8;       // lanes per row
  constexpr int RPB = 256 / LPR;   // rows per block
  const int tid = threadIdx.x, lane = tid & 63;
  const int c = tid % LPR;         // this lane's values: d = 8 c .. 8 c + 7
  const int half = a.rot / 2;
  const bool rotary = 8 * c < a.rot;
  const bool low = 8 * c < half;
  const int partner = lane + (low ? half / 8 : -(half / 8));  // same row (R % 16 == 0)
  // q rows take the first blocks_q workgroups, k rows the rest, so which
  // tensor a workgroup serves is uniform and its arguments are scalar loads.
  const int w = (int)blockIdx.x >= a.blocks_q;
  const int r = ((int)blockIdx.x - (w ? a.blocks_q : 0)) * RPB + tid / LPR;  // < 2^31 (checked by the host)
  const bool live = r < (w ? a.rows - a.rows_q : a.rows_q);

  // 1. Loads: the row's 8 values, its gradient (backward), and for rotary
  //    lanes cos / sin at columns (8 c) mod h .. + 7 of time step t.
  // The table rows stay raw until they are used, so that all of a lane's
  // loads are in flight together.
  bf16x8 xv{}, gv{}, c8{}, s8{};
  f32x4 c0{}, c1{}, s0{}, s1{};
  if (live) {
    // r -> (bt, h) -> (b, t) by multiply-high division: the compiler's
    // division by a runtime value sits in front of every load (8% of the
    // forward's time).
    const int bt = fast_div(r, a.div_heads[w]), h = r - bt * a.heads[w];
    const int b = fast_div(bt, a.div_T), t = bt - b * a.T;
    const bf16x8* xp = reinterpret_cast<const bf16x8*>(a.x[w] + b * a.s[w][0] + t * a.s[w][1] + h * a.s[w][2] + 8 * c);
    // Non-temporal loads measured 4% faster in the backward and 13% slower in
    // the forward (whose rows are strided views of the fused projection).
    xv = BWD ? __builtin_nontemporal_load(xp) : *xp;
    if constexpr (BWD) gv = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(a.g[w] + (int64_t)r * D + 8 * c));
    if (rotary) {
      const int64_t cb = (int64_t)t * a.rot + (8 * c) % half;
      const Tab* cp = static_cast<const Tab*>(a.cos) + cb;
      const Tab* sp = static_cast<const Tab*>(a.sin) + cb;
      if constexpr (sizeof(Tab) == 2) {
        c8 = *reinterpret_cast<const bf16x8*>(cp);
        s8 = *reinterpret_cast<const bf16x8*>(sp);
      } else {
        c0 = *reinterpret_cast<const f32x4*>(cp);
        c1 = *reinterpret_cast<const f32x4*>(cp + 4);
        s0 = *reinterpret_cast<const f32x4*>(sp);
        s1 = *reinterpret_cast<const f32x4*>(sp + 4);
      }
    }
  }

  // 2. Norm, then the rotation (forward) or its transpose + the norm's
  //    backward.  Every lane takes part in the shuffles, live or not.
  float x[8];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = (float)xv[e];
    ss = fmaf(x[e], x[e], ss);
  }
  ss = group_sum<LPR>(ss);
  const float inv = rsqrtf(ss * (1.f / D) + a.eps);
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (sizeof(Tab) == 2) {
      cs[e] = (float)c8[e];
      sn[e] = (float)s8[e];
    } else {
      cs[e] = e < 4 ? c0[e & 3] : c1[e & 3];
      sn[e] = e < 4 ? s0[e & 3] : s1[e & 3];
    }
  }
  const int hp = half / 8;
  float res[8];
  if constexpr (!BWD) {
    float xp[8];  // the partner's raw values (same row, same inv)
    partner_values(x, xp, hp, partner);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = x[e] * inv;
      if (rotary) {
        const float zp = xp[e] * inv;
        res[e] = low ? fmaf(z, cs[e], -zp * sn[e]) : fmaf(z, cs[e], zp * sn[e]);
      } else {
        res[e] = z;
      }
    }
  } else {
    float g[8], gp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = (float)gv[e];
    partner_values(g, gp, hp, partner);
    float gn[8], dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (rotary) {
        gn[e] = low ? fmaf(g[e], cs[e], gp[e] * sn[e]) : fmaf(g[e], cs[e], -gp[e] * sn[e]);
      } else {
        gn[e] = g[e];
      }
      dot = fmaf(gn[e], x[e] * inv, dot);
    }
    dot = group_sum<LPR>(dot);
    dot *= 1.f / D;
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = inv * (gn[e] - x[e] * inv * dot);
  }

  // 3. Store (vector, non-temporal).
  if (live) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)res[e];
    __builtin_nontemporal_store(o, reinterpret_cast<bf16x8*>(a.out[w] + (int64_t)r * D + 8 * c));
  }
}

template <int D, bool BWD>
hipError_t launch_typed(const QkNormRopeArgs& a, unsigned blocks, hipStream_t stream) {
  if (a.tab_bf16)
    hipLaunchKernelGGL((qk_norm_rope_kernel<D, BWD, bf16>), dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_kernel<D, BWD, float>), dim3(blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_qk_norm_rope(const QkNormRopeArgs& a, bool backward, hipStream_t stream) {
  constexpr int RPB = 256 / (D / 8);
  QkNormRopeArgs b = a;
  b.blocks_q = (int)(((int64_t)a.rows_q + RPB - 1) / RPB);
  const int64_t blocks = b.blocks_q + ((int64_t)(a.rows - a.rows_q) + RPB - 1) / RPB;
  if (blocks == 0) return hipSuccess;
  return backward ? launch_typed<D, true>(b, (unsigned)blocks, stream)
                  : launch_typed<D, false>(b, (unsigned)blocks, stream);
}

template hipError_t launch_qk_norm_rope<64>(const QkNormRopeArgs&, bool, hipStream_t);
template hipError_t launch_qk_norm_rope<128>(const QkNormRopeArgs&, bool, hipStream_t);

}  // namespace hlm
