// The no-grad attention forward of the evaluation harness's calls
// (lm_eval_hackable_lm.py:134-160,185-207: batch 1, ragged T, one full
// forward per token) as a single C++ call: check q/k/v, allocate O and lse
// through torch's caching allocator, pick the split count and launch through
// the C ABI (include/hlm_attn.h).  At batch 1 and short T the kernel takes a
// few microseconds, so the host work around the launch decides the call
// rate; done in Python it costs about twice the launch.  Host code only,
// linked against libhlm_attn.so in the same directory.  Device memory comes
// from torch (at::empty on q's device); the stream is the caller's current
// stream, passed as its raw handle.
#include <torch/extension.h>

#include <cstdint>
#include <vector>

#include "../../../include/hlm_attn.h"

namespace {

// The kernels' layout: (B, T, H, D) with unit D stride, (batch, time, head)
// strides multiples of 8 elements, rows that do not overlap, 16-byte aligned.
bool kernel_ready(const at::Tensor& t) {
  const auto s = t.strides();
  return s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 && s[0] >= 0 && s[1] >= 0 && s[2] >= 0 &&
         s[1] >= t.size(3) && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
}

// Returns {o, lse}, or an empty list when q, k, v are not bf16 (B, T, H, D)
// tensors on one device with the kernels' layout (the caller then takes its
// general path, which converts or raises).  A launch error raises with the
// C ABI's message.
std::vector<at::Tensor> fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t window,
                            double scale, int64_t stream) {
  if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4) return {};
  if (q.scalar_type() != at::kBFloat16 || k.scalar_type() != at::kBFloat16 || v.scalar_type() != at::kBFloat16)
    return {};
  if (!q.is_cuda() || k.device() != q.device() || v.device() != q.device()) return {};
  if (k.sizes() != v.sizes() || q.size(0) != k.size(0) || q.size(1) != k.size(1) || q.size(3) != k.size(3) ||
      k.size(2) == 0 || q.size(2) % k.size(2) != 0)
    return {};
  if (!kernel_ready(q) || !kernel_ready(k) || !kernel_ready(v)) return {};
  const int64_t B = q.size(0), T = q.size(1), H = q.size(2), Hkv = k.size(2), D = q.size(3);
  if (B > INT32_MAX || T > INT32_MAX || H > INT32_MAX || D > INT32_MAX || window < 0 || window > INT32_MAX) return {};
  const c10::DeviceGuard guard(q.device());
  at::Tensor o = at::empty({B, T, H, D}, q.options());
  at::Tensor lse = at::empty({B, H, T}, q.options().dtype(at::kFloat));
  const int nsplit = hlm_attn_fwd_split_count((int)B, (int)T, (int)H, (int)D, (int)window);
  const int64_t so[3] = {T * H * D, H * D, D};
  const auto sq = q.strides(), sk = k.strides(), sv = v.strides();
  const int64_t sq3[3] = {sq[0], sq[1], sq[2]}, sk3[3] = {sk[0], sk[1], sk[2]}, sv3[3] = {sv[0], sv[1], sv[2]};
  void* st = reinterpret_cast<void*>(static_cast<uintptr_t>(stream));
  int rc;
  if (nsplit > 1) {
    at::Tensor ws = at::empty({nsplit * B * H * T * (D + 2)}, q.options().dtype(at::kFloat));
    rc = hlm_attn_fwd_split(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr<float>(),
                            ws.data_ptr<float>(), nsplit, (int)B, (int)T, (int)H, (int)Hkv, (int)D, sq3, sk3, sv3, so,
                            (int)window, (float)scale, st);
  } else {
    rc = hlm_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr<float>(), (int)B, (int)T,
                      (int)H, (int)Hkv, (int)D, sq3, sk3, sv3, so, (int)window, (float)scale, st);
  }
  TORCH_CHECK(rc == 0, "hip attention failed (code ", rc, "): ", hlm_attn_last_error());
  return {o, lse};
}

}  // namespace

PYBIND11_MODULE(_torch_fwd, m) {
  m.doc() = "No-grad forward of hip attention in one call (allocation and launch in C++).";
  m.def("fwd", &fwd, "fwd(q, k, v, window, scale, stream) -> [o, lse], or [] when the inputs need the general path");
}
