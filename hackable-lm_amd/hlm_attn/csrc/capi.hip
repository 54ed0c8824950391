// extern "C" entry points of libhlm_attn.so (declared in include/hlm_attn.h):
// argument validation, mask normalisation and kernel dispatch by head dim.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "attn_common.h"
#include "../../../include/hlm_attn.h"

namespace hlm {
template <int D>
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream);
template <int D>
int fwd_split_count(int B, int T, int H, int W);
template <int D>
hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream, int phases);
int fused_partial_slots(int T, int W);
hipError_t launch_bwd_fused(const BwdArgs& a, bf16* part, int R, hipStream_t stream);
template <int D>
hipError_t launch_qk_norm_rope(const QkNormRopeArgs& a, bool backward, hipStream_t stream);
hipError_t launch_ce_rows(void* logits, bool bf16_logits, int64_t row_stride, const int64_t* targets, float* loss,
                          int n_rows, int V, float inv_n, int ignore_index, hipStream_t stream);
hipError_t launch_residual_rms_norm(const void* a, const void* b, const void* c, void* y0, void* y1, int64_t rows,
                                    int n, float eps, bool backward, hipStream_t stream);
}  // namespace hlm

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The kernels address rows of one (batch, head) slab through buffer
// resources with 32-bit byte offsets: (T + 512) rows at the time stride must
// stay below 2^31 bytes.  Rows must not overlap (time stride >= D): then every
// row at or beyond T lies outside the slab and reads as zeros, which the
// kernels rely on instead of masking padded rows.
int check_tensor(const char* name, const void* p, const int64_t* s, int T, int D) {
  if (p == nullptr) return fail(HLM_ATTN_EINVAL, "%s is a null pointer", name);
  if (!aligned16(p)) return fail(HLM_ATTN_EINVAL, "%s is not 16-byte aligned", name);
  if (s == nullptr) return fail(HLM_ATTN_EINVAL, "%s strides are a null pointer", name);
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || s[i] % 8 != 0)
      return fail(HLM_ATTN_EINVAL, "%s stride[%d] = %lld must be a non-negative multiple of 8 elements",
                  name, i, (long long)s[i]);
  if (s[1] < D) return fail(HLM_ATTN_EINVAL, "%s time stride %lld is below head_dim %d", name, (long long)s[1], D);
  if (((int64_t)T + 512) * s[1] * 2 >= ((int64_t)1 << 31))
    return fail(HLM_ATTN_EUNSUPPORTED, "%s: T x time stride too large for 32-bit row offsets", name);
  return HLM_ATTN_OK;
}

int check_dims(int B, int T, int H, int Hkv, int D, float scale) {
  if (B < 0 || T < 0 || H <= 0 || Hkv <= 0)
    return fail(HLM_ATTN_EINVAL, "bad shape B=%d T=%d H=%d Hkv=%d", B, T, H, Hkv);
  if (H % Hkv != 0) return fail(HLM_ATTN_EINVAL, "H=%d is not a multiple of Hkv=%d", H, Hkv);
  if (D != 64 && D != 128) return fail(HLM_ATTN_EUNSUPPORTED, "head_dim %d is not supported (64 or 128)", D);
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(HLM_ATTN_EINVAL, "scale must be positive and finite");
  const int64_t tiles = (int64_t)((T + 127) / 128) * H * B;
  if (tiles >= (int64_t)1 << 31) return fail(HLM_ATTN_EUNSUPPORTED, "problem too large for one launch");
  return HLM_ATTN_OK;
}

int effective_window(int window, int T) { return (window <= 0 || window >= T) ? T : window; }

void copy3(int64_t dst[3], const int64_t* src) {
  for (int i = 0; i < 3; ++i) dst[i] = src[i];
}

}  // namespace

extern "C" {

int hlm_attn_abi_version(void) { return 8; }

const char* hlm_attn_last_error(void) { return g_last_error; }

}  // extern "C"

namespace {

int run_fwd(const void* q, const void* k, const void* v, void* o, float* lse, float* ws, int nsplit, int B, int T,
            int H, int Hkv, int D, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
            const int64_t* o_strides, int window, float scale, void* stream) {
  g_last_error[0] = '\0';
  int rc = check_dims(B, T, H, Hkv, D, scale);
  if (rc) return rc;
  if (nsplit < 1 || nsplit > HLM_ATTN_MAX_SPLIT)
    return fail(HLM_ATTN_EINVAL, "nsplit %d is outside [1, %d]", nsplit, HLM_ATTN_MAX_SPLIT);
  if (nsplit > 1 && (ws == nullptr || !aligned16(ws)))
    return fail(HLM_ATTN_EINVAL, "split workspace is null or not 16-byte aligned");
  if (nsplit > 1 && (int64_t)B * H * T * (D / 8) >= ((int64_t)1 << 38))
    return fail(HLM_ATTN_EUNSUPPORTED, "problem too large for a split-key forward");
  if (B == 0 || T == 0) return HLM_ATTN_OK;
  if ((rc = check_tensor("q", q, q_strides, T, D)) || (rc = check_tensor("k", k, k_strides, T, D)) ||
      (rc = check_tensor("v", v, v_strides, T, D)) || (rc = check_tensor("o", o, o_strides, T, D)))
    return rc;
  if (lse == nullptr) return fail(HLM_ATTN_EINVAL, "lse is a null pointer");
  hlm::FwdArgs a;
  a.q = static_cast<const hlm::bf16*>(q);
  a.k = static_cast<const hlm::bf16*>(k);
  a.v = static_cast<const hlm::bf16*>(v);
  a.o = static_cast<hlm::bf16*>(o);
  a.lse = lse;
  copy3(a.sq, q_strides);
  copy3(a.sk, k_strides);
  copy3(a.sv, v_strides);
  copy3(a.so, o_strides);
  a.B = B;
  a.T = T;
  a.H = H;
  a.Hkv = Hkv;
  a.W = effective_window(window, T);
  a.scale_log2 = scale * hlm::kLog2e;
  a.nsplit = nsplit;
  a.part_o = ws;
  a.part_ml = ws == nullptr ? nullptr : ws + (int64_t)nsplit * B * H * T * D;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t err = D == 64 ? hlm::launch_fwd<64>(a, s) : hlm::launch_fwd<128>(a, s);
  if (err != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "forward launch failed: %s", hipGetErrorString(err));
  return HLM_ATTN_OK;
}

}  // namespace

extern "C" {

int hlm_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int T, int H,
                 int Hkv, int D, const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides, int window, float scale,
                 void* stream) {
  return run_fwd(q, k, v, o, lse, nullptr, 1, B, T, H, Hkv, D, q_strides, k_strides, v_strides, o_strides, window,
                 scale, stream);
}

int hlm_attn_fwd_split_count(int B, int T, int H, int D, int window) {
  if (B <= 0 || T <= 0 || H <= 0 || (D != 64 && D != 128)) return 1;
  const int W = effective_window(window, T);
  return D == 64 ? hlm::fwd_split_count<64>(B, T, H, W) : hlm::fwd_split_count<128>(B, T, H, W);
}

int hlm_attn_fwd_split(const void* q, const void* k, const void* v, void* o, float* lse, float* ws, int nsplit,
                       int B, int T, int H, int Hkv, int D, const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides, int window, float scale,
                       void* stream) {
  return run_fwd(q, k, v, o, lse, ws, nsplit, B, T, H, Hkv, D, q_strides, k_strides, v_strides, o_strides, window,
                 scale, stream);
}

}  // extern "C"

namespace {

int check_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
              const void* dq, const void* dk, const void* dv, int B, int T, int H, int Hkv, int D,
              const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
              const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
              const int64_t* dk_strides, const int64_t* dv_strides, float scale) {
  int rc = check_dims(B, T, H, Hkv, D, scale);
  if (rc || B == 0 || T == 0) return rc;
  if ((rc = check_tensor("q", q, q_strides, T, D)) || (rc = check_tensor("k", k, k_strides, T, D)) ||
      (rc = check_tensor("v", v, v_strides, T, D)) || (rc = check_tensor("o", o, o_strides, T, D)) ||
      (rc = check_tensor("dout", dout, do_strides, T, D)) || (rc = check_tensor("dq", dq, dq_strides, T, D)) ||
      (rc = check_tensor("dk", dk, dk_strides, T, D)) || (rc = check_tensor("dv", dv, dv_strides, T, D)))
    return rc;
  if (lse == nullptr) return fail(HLM_ATTN_EINVAL, "lse is a null pointer");
  return HLM_ATTN_OK;
}

// phases: kBwdDq / kBwdDkDv / kBwdAll for the two-kernel backward, or
// kBwdFused (with `part`, `part_bytes`) for the single-pass one.
constexpr int kBwdFused = 4;

int run_bwd(int phases, const void* q, const void* k, const void* v, const void* o, const void* dout,
            const float* lse, void* dq, void* dk, void* dv, float* delta_ws, int B, int T, int H, int Hkv,
            int D, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
            const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
            const int64_t* dk_strides, const int64_t* dv_strides, int window, float scale, void* stream,
            void* part = nullptr, int64_t part_bytes = 0) {
  g_last_error[0] = '\0';
  int rc = check_bwd(q, k, v, o, dout, lse, dq, dk, dv, B, T, H, Hkv, D, q_strides, k_strides, v_strides, o_strides,
                     do_strides, dq_strides, dk_strides, dv_strides, scale);
  if (rc) return rc;
  int R = 0;
  if (phases == kBwdFused) {
    if (D != 64) return fail(HLM_ATTN_EUNSUPPORTED, "the single-pass backward takes head_dim 64 only (got %d)", D);
    if (B == 0 || T == 0) return HLM_ATTN_OK;
    R = hlm::fused_partial_slots(T, effective_window(window, T));
    const int64_t need = (int64_t)R * B * H * T * D * 2;
    if (part == nullptr || !aligned16(part)) return fail(HLM_ATTN_EINVAL, "partial workspace is null or not 16-byte aligned");
    if (part_bytes < need)
      return fail(HLM_ATTN_EINVAL, "partial workspace holds %lld bytes, %lld needed", (long long)part_bytes,
                  (long long)need);
  }
  if (B == 0 || T == 0) return rc;
  if (delta_ws == nullptr) return fail(HLM_ATTN_EINVAL, "delta_ws is a null pointer");
  hlm::BwdArgs a;
  a.q = static_cast<const hlm::bf16*>(q);
  a.k = static_cast<const hlm::bf16*>(k);
  a.v = static_cast<const hlm::bf16*>(v);
  a.o = static_cast<const hlm::bf16*>(o);
  a.dout = static_cast<const hlm::bf16*>(dout);
  a.lse = lse;
  a.dq = static_cast<hlm::bf16*>(dq);
  a.dk = static_cast<hlm::bf16*>(dk);
  a.dv = static_cast<hlm::bf16*>(dv);
  a.delta = delta_ws;
  copy3(a.sq, q_strides);
  copy3(a.sk, k_strides);
  copy3(a.sv, v_strides);
  copy3(a.so, o_strides);
  copy3(a.sdo, do_strides);
  copy3(a.sdq, dq_strides);
  copy3(a.sdk, dk_strides);
  copy3(a.sdv, dv_strides);
  a.B = B;
  a.T = T;
  a.H = H;
  a.Hkv = Hkv;
  a.W = effective_window(window, T);
  a.scale = scale;
  a.scale_log2 = scale * hlm::kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t err = phases == kBwdFused ? hlm::launch_bwd_fused(a, static_cast<hlm::bf16*>(part), R, s)
                         : D == 64           ? hlm::launch_bwd<64>(a, s, phases)
                                             : hlm::launch_bwd<128>(a, s, phases);
  if (err != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "backward launch failed: %s", hipGetErrorString(err));
  return HLM_ATTN_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free backward: the workspace of hlm_attn_bwd (-lse * log2(e) and
// -delta per query row, 2 * B * H * T floats) lives in this file-scope device
// array instead of caller memory.  Every device that runs the library holds
// its own copy (32 MiB) from the module's load until the process ends.  Host
// code never uses the array's name as an address: the device address comes
// from hipGetSymbolAddress, once per device with that device current, and is
// kept per device.  The dq kernel overwrites every workspace value the dkdv
// kernel reads, so nothing needs clearing between calls; two calls that
// overlap on one device (different streams) race on it.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchFloats = (int64_t)1 << 23;  // 32 MiB: B * H * T up to 4,194,304 query rows
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the device that owns `stream`, looked up
// on the first call for that device (made current for the lookup).
int scratch_for_stream(void* stream, float** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev);
  if (e != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(HLM_ATTN_EUNSUPPORTED, "device %d is beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess)
      return fail(HLM_ATTN_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(HLM_ATTN_ELAUNCH, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess && e2 != hipSuccess)
        return fail(HLM_ATTN_ELAUNCH, "hipSetDevice(%d) failed: %s", cur, hipGetErrorString(e2));
    }
    if (e != hipSuccess || p == nullptr)
      return fail(HLM_ATTN_ELAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return HLM_ATTN_OK;
}

}  // namespace

extern "C" {

int hlm_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, void* dq, void* dk, void* dv, int B, int T, int H, int Hkv, int D,
                         const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                         const int64_t* dk_strides, const int64_t* dv_strides, int window, float scale,
                         void* stream) {
  g_last_error[0] = '\0';
  int rc = check_bwd(q, k, v, o, dout, lse, dq, dk, dv, B, T, H, Hkv, D, q_strides, k_strides, v_strides, o_strides,
                     do_strides, dq_strides, dk_strides, dv_strides, scale);
  if (rc) return rc;
  const int64_t need = 2 * (int64_t)B * H * T;
  if (need > kScratchFloats)
    return fail(HLM_ATTN_EUNSUPPORTED,
                "hlm_attn_bwd_noalloc: B * H * T = %lld query rows exceeds its fixed scratch (%lld rows); "
                "use hlm_attn_bwd with a workspace",
                (long long)(need / 2), (long long)(kScratchFloats / 2));
  if (B == 0 || T == 0) return HLM_ATTN_OK;
  float* ws = nullptr;
  if ((rc = scratch_for_stream(stream, &ws))) return rc;
  return run_bwd(hlm::kBwdAll, q, k, v, o, dout, lse, dq, dk, dv, ws, B, T, H, Hkv, D, q_strides, k_strides,
                 v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides, window, scale, stream);
}

}  // extern "C"

#define HLM_BWD_PARAMS                                                                              \
  const void *q, const void *k, const void *v, const void *o, const void *dout, const float *lse,   \
      void *dq, void *dk, void *dv, float *delta_ws, int B, int T, int H, int Hkv, int D,           \
      const int64_t *q_strides, const int64_t *k_strides, const int64_t *v_strides,                 \
      const int64_t *o_strides, const int64_t *do_strides, const int64_t *dq_strides,               \
      const int64_t *dk_strides, const int64_t *dv_strides, int window, float scale, void *stream
#define HLM_BWD_ARGS                                                                                \
  q, k, v, o, dout, lse, dq, dk, dv, delta_ws, B, T, H, Hkv, D, q_strides, k_strides, v_strides,    \
      o_strides, do_strides, dq_strides, dk_strides, dv_strides, window, scale, stream

extern "C" {

int hlm_attn_bwd(HLM_BWD_PARAMS) { return run_bwd(hlm::kBwdAll, HLM_BWD_ARGS); }
int hlm_attn_bwd_dq(HLM_BWD_PARAMS) { return run_bwd(hlm::kBwdDq, HLM_BWD_ARGS); }
int hlm_attn_bwd_dkdv(HLM_BWD_PARAMS) { return run_bwd(hlm::kBwdDkDv, HLM_BWD_ARGS); }

int64_t hlm_attn_bwd_fused_workspace_bytes(int B, int T, int H, int D, int window) {
  g_last_error[0] = '\0';
  if (B < 0 || T < 0 || H <= 0) return fail(HLM_ATTN_EINVAL, "bad shape B=%d T=%d H=%d", B, T, H);
  if (D != 64) return fail(HLM_ATTN_EUNSUPPORTED, "the single-pass backward takes head_dim 64 only (got %d)", D);
  if (B == 0 || T == 0) return 0;
  return (int64_t)hlm::fused_partial_slots(T, effective_window(window, T)) * B * H * T * D * 2;
}

int hlm_attn_bwd_fused(const void* q, const void* k, const void* v, const void* o, const void* dout,
                       const float* lse, void* dq, void* dk, void* dv, float* delta_ws, void* partial_ws,
                       int64_t partial_ws_bytes, int B, int T, int H, int Hkv, int D, const int64_t* q_strides,
                       const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                       const int64_t* do_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                       const int64_t* dv_strides, int window, float scale, void* stream) {
  return run_bwd(kBwdFused, q, k, v, o, dout, lse, dq, dk, dv, delta_ws, B, T, H, Hkv, D, q_strides, k_strides,
                 v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides, window, scale, stream,
                 partial_ws, partial_ws_bytes);
}

}  // extern "C"

namespace {

int run_qk_norm_rope(bool backward, const void* q, const void* k, const void* gq, const void* gk, const void* cos,
                     const void* sin, int table_dtype, void* oq, void* ok, int B, int T, int H, int Hkv, int D, int rot,
                     const int64_t* q_strides, const int64_t* k_strides, float eps, void* stream) {
  g_last_error[0] = '\0';
  if (B < 0 || T < 0 || H <= 0 || Hkv <= 0)
    return fail(HLM_ATTN_EINVAL, "bad shape B=%d T=%d H=%d Hkv=%d", B, T, H, Hkv);
  if (D != 64 && D != 128) return fail(HLM_ATTN_EUNSUPPORTED, "head_dim %d is not supported (64 or 128)", D);
  if (rot < 0 || rot > D || rot % 16 != 0)
    return fail(HLM_ATTN_EUNSUPPORTED, "rotary_dim %d must be a multiple of 16 in [0, %d]", rot, D);
  if (!(eps > 0.f) || !std::isfinite(eps)) return fail(HLM_ATTN_EINVAL, "eps must be positive and finite");
  if (table_dtype != HLM_TABLE_F32 && table_dtype != HLM_TABLE_BF16)
    return fail(HLM_ATTN_EINVAL, "table_dtype %d is neither HLM_TABLE_F32 nor HLM_TABLE_BF16", table_dtype);
  const int64_t rows = (int64_t)B * T * (H + Hkv);
  if (rows >= ((int64_t)1 << 31) - 1024) return fail(HLM_ATTN_EUNSUPPORTED, "too many rows for one launch");
  if (rows == 0) return HLM_ATTN_OK;
  int rc;
  if ((rc = check_tensor("q", q, q_strides, T, D)) || (rc = check_tensor("k", k, k_strides, T, D))) return rc;
  const void* outs[2] = {oq, ok};
  for (int i = 0; i < 2; ++i)
    if (outs[i] == nullptr || !aligned16(outs[i]))
      return fail(HLM_ATTN_EINVAL, "output %d is null or not 16-byte aligned", i);
  if (backward && (gq == nullptr || gk == nullptr || !aligned16(gq) || !aligned16(gk)))
    return fail(HLM_ATTN_EINVAL, "grad_q_out / grad_k_out are null or not 16-byte aligned");
  if (rot > 0 && (cos == nullptr || sin == nullptr || !aligned16(cos) || !aligned16(sin)))
    return fail(HLM_ATTN_EINVAL, "cos / sin are null or not 16-byte aligned");
  hlm::QkNormRopeArgs a;
  a.x[0] = static_cast<const hlm::bf16*>(q);
  a.x[1] = static_cast<const hlm::bf16*>(k);
  a.g[0] = static_cast<const hlm::bf16*>(gq);
  a.g[1] = static_cast<const hlm::bf16*>(gk);
  a.out[0] = static_cast<hlm::bf16*>(oq);
  a.out[1] = static_cast<hlm::bf16*>(ok);
  copy3(a.s[0], q_strides);
  copy3(a.s[1], k_strides);
  a.heads[0] = H;
  a.heads[1] = Hkv;
  a.div_heads[0] = hlm::fast_div_of((unsigned)H);
  a.div_heads[1] = hlm::fast_div_of((unsigned)Hkv);
  a.div_T = hlm::fast_div_of((unsigned)T);
  a.cos = cos;
  a.sin = sin;
  a.tab_bf16 = table_dtype == HLM_TABLE_BF16;
  a.T = T;
  a.rot = rot;
  a.eps = eps;
  a.rows_q = (int)((int64_t)B * T * H);
  a.rows = (int)rows;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t err = D == 64 ? hlm::launch_qk_norm_rope<64>(a, backward, s)
                                 : hlm::launch_qk_norm_rope<128>(a, backward, s);
  if (err != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "qk_norm_rope launch failed: %s", hipGetErrorString(err));
  return HLM_ATTN_OK;
}

}  // namespace

extern "C" {

int hlm_qk_norm_rope_fwd(const void* q, const void* k, const void* cos, const void* sin, int table_dtype,
                         void* q_out, void* k_out, int B, int T, int H, int Hkv, int D, int rotary_dim,
                         const int64_t* q_strides, const int64_t* k_strides, float eps, void* stream) {
  return run_qk_norm_rope(false, q, k, nullptr, nullptr, cos, sin, table_dtype, q_out, k_out, B, T, H, Hkv, D,
                          rotary_dim, q_strides, k_strides, eps, stream);
}

int hlm_qk_norm_rope_bwd(const void* q, const void* k, const void* grad_q_out, const void* grad_k_out,
                         const void* cos, const void* sin, int table_dtype, void* grad_q, void* grad_k, int B,
                         int T, int H, int Hkv, int D, int rotary_dim, const int64_t* q_strides,
                         const int64_t* k_strides, float eps, void* stream) {
  return run_qk_norm_rope(true, q, k, grad_q_out, grad_k_out, cos, sin, table_dtype, grad_q, grad_k, B, T, H, Hkv,
                          D, rotary_dim, q_strides, k_strides, eps, stream);
}

int hlm_ce_rows(void* logits, int logits_dtype, int64_t row_stride, const int64_t* targets, float* loss, int n_rows,
                int n_cols, int64_t n_tokens, int ignore_index, void* stream) {
  g_last_error[0] = '\0';
  if (n_rows < 0 || n_cols <= 0) return fail(HLM_ATTN_EINVAL, "bad shape n_rows=%d n_cols=%d", n_rows, n_cols);
  if (logits_dtype != HLM_DTYPE_F32 && logits_dtype != HLM_DTYPE_BF16)
    return fail(HLM_ATTN_EINVAL, "logits_dtype %d is neither HLM_DTYPE_F32 nor HLM_DTYPE_BF16", logits_dtype);
  if (row_stride < n_cols) return fail(HLM_ATTN_EINVAL, "row_stride %lld is below n_cols %d", (long long)row_stride, n_cols);
  if (n_tokens <= 0) return fail(HLM_ATTN_EINVAL, "n_tokens must be positive");
  if (n_rows == 0) return HLM_ATTN_OK;
  if (logits == nullptr || targets == nullptr || loss == nullptr)
    return fail(HLM_ATTN_EINVAL, "logits, targets or loss is a null pointer");
  const hipError_t err = hlm::launch_ce_rows(logits, logits_dtype == HLM_DTYPE_BF16, row_stride, targets, loss, n_rows,
                                             n_cols, (float)(1.0 / (double)n_tokens), ignore_index,
                                             static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "cross-entropy launch failed: %s", hipGetErrorString(err));
  return HLM_ATTN_OK;
}

}  // extern "C"

namespace {

int run_residual_rms_norm(bool backward, const void* a, const void* b, const void* c, void* y0, void* y1,
                          int64_t rows, int n, float eps, void* stream) {
  g_last_error[0] = '\0';
  if (rows < 0 || n <= 0) return fail(HLM_ATTN_EINVAL, "bad shape rows=%lld n=%d", (long long)rows, n);
  if (n % 8 != 0 || n > 8192)
    return fail(HLM_ATTN_EUNSUPPORTED, "row width %d must be a multiple of 8 and at most 8192", n);
  if (!(eps > 0.f) || !std::isfinite(eps)) return fail(HLM_ATTN_EINVAL, "eps must be positive and finite");
  if ((rows + 3) / 4 >= ((int64_t)1 << 31)) return fail(HLM_ATTN_EUNSUPPORTED, "too many rows for one launch");
  if (rows == 0) return HLM_ATTN_OK;
  const void* ptrs[5] = {a, b, backward ? c : a, y0, backward ? y0 : y1};
  for (const void* q : ptrs)
    if (q == nullptr || !aligned16(q)) return fail(HLM_ATTN_EINVAL, "a tensor is null or not 16-byte aligned");
  const hipError_t err =
      hlm::launch_residual_rms_norm(a, b, c, y0, y1, rows, n, eps, backward, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(HLM_ATTN_ELAUNCH, "residual_rms_norm launch failed: %s", hipGetErrorString(err));
  return HLM_ATTN_OK;
}

}  // namespace

extern "C" {

int hlm_residual_rms_norm_fwd(const void* residual, const void* branch, void* out, void* normed, int64_t rows, int n,
                              float eps, void* stream) {
  return run_residual_rms_norm(false, residual, branch, nullptr, out, normed, rows, n, eps, stream);
}

int hlm_residual_rms_norm_bwd(const void* out, const void* grad_out, const void* grad_normed, void* grad_in,
                              int64_t rows, int n, float eps, void* stream) {
  return run_residual_rms_norm(true, out, grad_out, grad_normed, grad_in, nullptr, rows, n, eps, stream);
}

}  // extern "C"
