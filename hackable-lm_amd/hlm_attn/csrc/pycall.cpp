// CPython binding of the forward entry points for no-grad calls (the
// evaluation harness's per-token forwards, lm_eval_hackable_lm.py:134-160,
// 185-207).  It passes the same arguments as the ctypes binding to the same
// C ABI (include/hlm_attn.h), in one METH_FASTCALL call: ctypes converts each
// of the ~25 arguments through its own type objects, which costs a few
// microseconds per call -- as much as the kernel at batch 1 and short T.
// Host code only; linked against libhlm_attn.so, which sits in the same
// directory.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <climits>
#include <cstdint>

#include "../../../include/hlm_attn.h"

namespace {

constexpr Py_ssize_t kFwdArgs = 27;

// fwd(q, k, v, o, lse, ws, nsplit, B, T, H, Hkv, D,
//     sq0, sq1, sq2, sk0, sk1, sk2, sv0, sv1, sv2, so0, so1, so2,
//     window, scale, stream) -> int
// Pointers and the stream are Python ints (tensor.data_ptr(), the raw
// hipStream_t); strides are the (batch, time, head) element strides.  nsplit
// > 1 runs hlm_attn_fwd_split with ws as its workspace, else hlm_attn_fwd.
// Returns the C ABI's status code (0 on success; hlm_attn_last_error() then
// describes a failure).
PyObject* py_fwd(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != kFwdArgs) {
    PyErr_Format(PyExc_TypeError, "fwd takes %zd arguments, got %zd", kFwdArgs, nargs);
    return nullptr;
  }
  void* ptr[6];
  for (int i = 0; i < 6; ++i) ptr[i] = PyLong_AsVoidPtr(args[i]);
  // nsplit, B, T, H, Hkv, D and window are C ints: out-of-range values raise
  // instead of wrapping into a different, valid-looking problem.
  int ints[7];
  for (int i = 0; i < 7; ++i) {
    const long v = PyLong_AsLong(args[i == 6 ? 24 : 6 + i]);
    if (v == -1 && PyErr_Occurred()) return nullptr;
    if (v < INT_MIN || v > INT_MAX) {
      PyErr_Format(PyExc_OverflowError, "fwd argument %d (%ld) does not fit a C int", i == 6 ? 24 : 6 + i, v);
      return nullptr;
    }
    ints[i] = (int)v;
  }
  const int nsplit = ints[0], window = ints[6];
  const int* dims = ints + 1;
  int64_t st[4][3];
  for (int i = 0; i < 12; ++i) st[i / 3][i % 3] = (int64_t)PyLong_AsLongLong(args[12 + i]);
  const float scale = (float)PyFloat_AsDouble(args[25]);
  void* stream = PyLong_AsVoidPtr(args[26]);
  if (PyErr_Occurred()) return nullptr;
  int rc;
  if (nsplit > 1)
    rc = hlm_attn_fwd_split(ptr[0], ptr[1], ptr[2], ptr[3], static_cast<float*>(ptr[4]), static_cast<float*>(ptr[5]),
                            nsplit, dims[0], dims[1], dims[2], dims[3], dims[4], st[0], st[1], st[2], st[3],
                            window, scale, stream);
  else
    rc = hlm_attn_fwd(ptr[0], ptr[1], ptr[2], ptr[3], static_cast<float*>(ptr[4]), dims[0], dims[1], dims[2],
                      dims[3], dims[4], st[0], st[1], st[2], st[3], window, scale, stream);
  return PyLong_FromLong(rc);
}

PyMethodDef kMethods[] = {
    {"fwd", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_fwd)), METH_FASTCALL,
     "Forward attention launch through the C ABI (see the module source for the argument list)."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_pycall", "CPython binding of the forward C ABI.", -1, kMethods,
                       nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__pycall(void) { return PyModule_Create(&kModule); }
