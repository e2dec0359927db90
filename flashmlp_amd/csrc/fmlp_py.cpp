// _fmlp_fast: the per-call fast path of flashmlp_fwd / flashmlp_bwd (flashmlp_amd/flashmlp.py).
//
// A CPython module (METH_FASTCALL) over the C ABI of libflashmlp.so for the common case: 16-bit
// inputs on one GPU, dense and 16-byte aligned, a shape the tuned kernels take. It allocates the
// outputs and the workspace with ATen on the inputs' device, launches on torch's current HIP
// stream of that device and returns the C ABI status with the outputs; for any other input it
// returns None and the Python wrapper takes its general path (which also raises the reference's
// errors). Same entry points, same results as the ctypes calls of the general path; only the
// host work per call is smaller (no ctypes argument conversion, allocations from C++).
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <c10/util/Exception.h>
#include <torch/csrc/Exceptions.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>

#include "flashmlp.h"

namespace {

int io_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kHalf: return FMLP_DTYPE_F16;
    case at::kBFloat16: return FMLP_DTYPE_BF16;
    default: return -1;
  }
}

bool dense16(const at::Tensor& t) {
  return t.dim() == 3 && t.is_contiguous() && (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0;
}

// the tensors the tuned kernels take as they are: 16-bit, one GPU, dense, aligned; sets the io
// dtype code
bool eligible(PyObject* const* args, int n, const at::Tensor** ts, int* code) {
  for (int i = 0; i < n; ++i) {
    if (!THPVariable_Check(args[i])) return false;
    ts[i] = &THPVariable_Unpack(args[i]);
  }
  const at::Tensor& x = *ts[0];
  if (!x.is_cuda()) return false;
  const int c = io_code(x);
  if (c < 0) return false;
  for (int i = 0; i < n; ++i) {
    const at::Tensor& t = *ts[i];
    if (t.scalar_type() != x.scalar_type() || t.device() != x.device() || !dense16(t)) return false;
  }
  *code = c;
  return true;
}

PyObject* wrap_or_none(const at::Tensor& t) {
  if (!t.defined()) Py_RETURN_NONE;
  return THPVariable_Wrap(t);
}

at::Tensor bytes_on(const at::Tensor& like, size_t n) {
  return at::empty({(int64_t)n}, like.options().dtype(at::kByte));
}

// fwd(x, w1, w2, act) -> (status, o) or None
PyObject* fast_fwd(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  HANDLE_TH_ERRORS
  if (nargs != 4) {
    PyErr_SetString(PyExc_TypeError, "fwd(x, w1, w2, act)");
    return nullptr;
  }
  const at::Tensor* ts[3];
  int code = 0;
  if (!eligible(args, 3, ts, &code)) Py_RETURN_NONE;
  const at::Tensor &x = *ts[0], &w1 = *ts[1], &w2 = *ts[2];
  const int act = (int)PyLong_AsLong(args[3]);
  if (act == -1 && PyErr_Occurred()) return nullptr;
  const int64_t H = x.size(0), B = x.size(1), D = x.size(2), E = w1.size(2);
  if (!fmlp_shape_tuned(D, E, code)) Py_RETURN_NONE;
  c10::DeviceGuard guard(x.device());
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
  at::Tensor o = at::empty_like(x);
  size_t n = fmlp_fwd_workspace_bytes(H, B, D, E, code);
  at::Tensor ws;
  if (n) {
    try {
      ws = bytes_on(x, n);
    } catch (const c10::OutOfMemoryError&) {  // the kernels then run every tile whole
      n = 0;
    }
  }
  const int st = fmlp_fwd_ws(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), o.data_ptr(), H, B, D, E, code, act,
                             n ? ws.data_ptr() : nullptr, n, stream);
  return Py_BuildValue("(iN)", st, THPVariable_Wrap(o));
  END_HANDLE_TH_ERRORS
}

// bwd(x, w1, w2, do, act, flags) -> (status, dx, dw1, dw2) or None; flags: the backward's flag
// bits (FMLP_DW_HILO, FMLP_BWD_RECOMPUTE, FMLP_BWD_NO_DX, FMLP_BWD_NO_DW), the io dtype is added
PyObject* fast_bwd(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  HANDLE_TH_ERRORS
  if (nargs != 6) {
    PyErr_SetString(PyExc_TypeError, "bwd(x, w1, w2, do, act, flags)");
    return nullptr;
  }
  const at::Tensor* ts[4];
  int code = 0;
  if (!eligible(args, 4, ts, &code)) Py_RETURN_NONE;
  const at::Tensor &x = *ts[0], &w1 = *ts[1], &w2 = *ts[2], &dout = *ts[3];
  const int act = (int)PyLong_AsLong(args[4]);
  if (act == -1 && PyErr_Occurred()) return nullptr;
  int flags = (int)PyLong_AsLong(args[5]);
  if (flags == -1 && PyErr_Occurred()) return nullptr;
  const int64_t H = x.size(0), B = x.size(1), D = x.size(2), E = w1.size(2);
  if (!fmlp_shape_tuned(D, E, code)) Py_RETURN_NONE;
  flags |= code;
  const bool need_dx = (flags & FMLP_BWD_NO_DX) == 0, need_dw = (flags & FMLP_BWD_NO_DW) == 0;
  c10::DeviceGuard guard(x.device());
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
  at::Tensor dx, dw1, dw2, ws;
  if (need_dx) dx = at::empty_like(x);
  if (need_dw) {
    dw1 = at::empty_like(w1);
    dw2 = at::empty_like(w2);
  }
  // the workspace this call's plan needs (one plan lookup, for its own activation)
  auto ws_need = [&](int f) -> size_t {
    int64_t info[9];
    if (fmlp_bwd_plan(H, B, D, E, f, act, info, 9) == FMLP_OK) return (size_t)info[8];
    return fmlp_bwd_workspace_bytes(H, B, D, E, f);
  };
  size_t n = ws_need(flags);
  if (n) {
    try {
      ws = bytes_on(x, n);
    } catch (const c10::OutOfMemoryError&) {
      // the stored-dZ form's workspace does not fit: the recompute form needs at most the fp32
      // dW partials (as the general path does)
      if (flags & FMLP_BWD_RECOMPUTE) throw;
      flags |= FMLP_BWD_RECOMPUTE;
      n = ws_need(flags);
      if (n) ws = bytes_on(x, n);
    }
  }
  const int st = fmlp_bwd(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), dout.data_ptr(),
                          need_dx ? dx.data_ptr() : nullptr, need_dw ? dw1.data_ptr() : nullptr,
                          need_dw ? dw2.data_ptr() : nullptr, H, B, D, E, flags, act, n ? ws.data_ptr() : nullptr, n,
                          stream);
  return Py_BuildValue("(iNNN)", st, wrap_or_none(dx), wrap_or_none(dw1), wrap_or_none(dw2));
  END_HANDLE_TH_ERRORS
}

PyMethodDef kMethods[] = {
    {"fwd", (PyCFunction)(void (*)(void))fast_fwd, METH_FASTCALL, "fwd(x, w1, w2, act) -> (status, o) or None"},
    {"bwd", (PyCFunction)(void (*)(void))fast_bwd, METH_FASTCALL,
     "bwd(x, w1, w2, do, act, flags) -> (status, dx, dw1, dw2) or None"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_fmlp_fast", "fast path of flashmlp_fwd / flashmlp_bwd", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__fmlp_fast() { return PyModule_Create(&kModule); }
