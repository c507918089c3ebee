/* CPython extension `_ccv1d_torch`: the inference forward of causal_conv1d_fn (no autograd node)
 * in one native call. It takes torch tensors, applies the reference's argument checks and
 * canonicalisation (causal_conv1d.py:397-412, :612-617), allocates the outputs with the caching
 * allocator and calls ccv1d_fwd_inference (include/ccv1d.h: ccv1d_fwd's kernels with the store
 * policy of a pass no backward follows) on torch's current stream of x's device. For the autograd
 * node's two passes it also offers `fwd_train` (allocation of out and ccv1d_fwd, on inputs the
 * Python side has checked and canonicalised) and `bwd` (allocation of the gradients and the
 * workspace and ccv1d_bwd, the reference's `_bwd`, causal_conv1d.py:475-541).
 *
 * Why native: an eager decode step (batch 16, one row, state handoff) spends about 2.7 us in the
 * HIP launch and, in Python, 1.4 us reading tensor attributes, 2.6 us in two torch.empty calls and
 * 2 us in checks; here the attribute reads and allocations cost tens of nanoseconds each. Compute
 * is unchanged: the same C ABI and kernels as every other path.
 *
 * It is built with g++ against torch's headers (Makefile), links libccv1d.so from its own
 * directory, and is loaded after `import torch`.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/GradMode.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/python_variable.h>

#include <exception>

#include "ccv1d.h"

namespace {

// The package's error type for a non-zero library status (set by the Python side at import).
PyObject* g_error_type = nullptr;

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return CCV1D_F32;
    case at::kHalf: return CCV1D_F16;
    case at::kBFloat16: return CCV1D_BF16;
    case at::kDouble: return CCV1D_F64;
    default: return -1;
  }
}

PyObject* assertion(const char* msg) {
  PyErr_SetString(PyExc_AssertionError, msg);
  return nullptr;
}

// A plain tensor (torch.Tensor or Parameter) or None. False for anything else, including tensor
// subclasses (fake tensors, wrappers with their own dispatch), which the Python path handles.
bool tensor_or_none(PyObject* o, const at::Tensor** t) {
  if (o == Py_None) {
    *t = nullptr;
    return true;
  }
  if (!THPVariable_CheckExact(o)) return false;
  *t = &THPVariable_Unpack(o);
  return true;
}

bool device_of_x(const at::Tensor* t, int64_t dev) { return !t || t->get_device() == dev; }

PyObject* fwd_impl(PyObject* const* a) {
  const at::Tensor *px, *pw, *pb, *ps, *pi;
  if (!tensor_or_none(a[0], &px) || !tensor_or_none(a[1], &pw) || !tensor_or_none(a[2], &pb) ||
      !tensor_or_none(a[3], &ps) || !tensor_or_none(a[4], &pi) || !px || !pw)
    Py_RETURN_NONE;
  const int ret_final = PyObject_IsTrue(a[5]);
  const int silu = PyObject_IsTrue(a[6]);
  if (ret_final < 0 || silu < 0) return nullptr;
  const at::Tensor& x = *px;
  const at::Tensor& w = *pw;

  // The reference's assertions (causal_conv1d.py:397-408), with the messages of
  // causal_conv1d.py's _check_inputs, including its device checks of the optional tensors.
  if (x.dim() != 3) return assertion("x must be (batch, seqlen, dim)");
  const int64_t B = x.size(0), T = x.size(1), D = x.size(2);
  if (w.dim() != 2 || w.size(0) != D) return assertion("weight must be (dim, width)");
  const int64_t W = w.size(1);
  if (W < 2) return assertion("width must be >= 2");
  if (!x.is_cuda()) return assertion("x must be on a GPU");
  const int64_t dev = x.get_device();
  if (w.get_device() != dev) return assertion("weight must be on the device of x");
  if (pb) {
    if (pb->dim() != 1 || pb->size(0) != D) return assertion("bias must be (dim,)");
    if (!device_of_x(pb, dev)) return assertion("bias must be on the device of x");
  }
  if (pi) {
    if (pi->dim() != 3 || pi->size(0) != B || pi->size(1) != W - 1 || pi->size(2) != D)
      return assertion("initial_states must be (batch, width - 1, dim)");
    if (!device_of_x(pi, dev)) return assertion("initial_states must be on the device of x");
  }
  if (ps) {
    if (ps->dim() != 2 || ps->size(0) != B || ps->size(1) != T)
      return assertion("seq_idx must be (batch, seqlen)");
    if (!device_of_x(ps, dev)) return assertion("seq_idx must be on the device of x");
  }
  const int64_t st = x.stride(1);
  if ((T + W) * (st > D ? st : D) >= (int64_t(1) << 31))
    return assertion("seqlen * dim too large for 32-bit offsets");

  // An input that autograd must track: the Python path records the call through its autograd
  // node.
  if (c10::GradMode::is_enabled() &&
      (x.requires_grad() || w.requires_grad() || (pb && pb->requires_grad()) ||
       (pi && pi->requires_grad())))
    Py_RETURN_NONE;

  // Canonicalisation (causal_conv1d.py:411-412, :612-617): a unit channel stride for x, the rest
  // contiguous, int32 sequence ids.
  const at::Tensor xc = x.stride(2) == 1 ? x : x.contiguous();
  const at::Tensor wc = w.contiguous();
  const at::Tensor bc = pb ? pb->contiguous() : at::Tensor();
  const at::Tensor sc = ps ? ps->to(at::kInt).contiguous() : at::Tensor();
  const at::Tensor ic = pi ? pi->contiguous() : at::Tensor();
  const int xdt = dtype_code(xc.scalar_type()), wdt = dtype_code(wc.scalar_type());
  const int bdt = pb ? dtype_code(bc.scalar_type()) : 0;
  const int idt = pi ? dtype_code(ic.scalar_type()) : 0;
  if (xdt < 0 || wdt < 0 || bdt < 0 || idt < 0) {
    PyErr_SetString(PyExc_TypeError, "unsupported dtype (fp32, fp16, bf16 or fp64 expected)");
    return nullptr;
  }

  at::Tensor out = at::empty({B, T, D}, xc.options());
  at::Tensor fin;
  if (ret_final) fin = at::empty({B, W - 1, D}, xc.options());
  void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = ccv1d_fwd_inference(xc.data_ptr(), xc.stride(0), xc.stride(1), xdt, wc.data_ptr(), wdt,
                 pb ? bc.data_ptr() : nullptr, bdt,
                 ps ? static_cast<const int32_t*>(sc.data_ptr()) : nullptr,
                 pi ? ic.data_ptr() : nullptr, idt, out.data_ptr(),
                 ret_final ? fin.data_ptr() : nullptr, B, T, D, W, silu, (int)dev, stream);
  Py_END_ALLOW_THREADS
  if (rc) {
    PyErr_Format(g_error_type ? g_error_type : PyExc_RuntimeError, "libccv1d error %d: %s", rc,
                 ccv1d_last_error());
    return nullptr;
  }
  PyObject* o = THPVariable_Wrap(std::move(out));
  if (!ret_final || !o) return o;
  PyObject* f = THPVariable_Wrap(std::move(fin));
  if (!f) {
    Py_DECREF(o);
    return nullptr;
  }
  PyObject* r = PyTuple_Pack(2, o, f);
  Py_DECREF(o);
  Py_DECREF(f);
  return r;
}

/* fwd(x, weight, bias, seq_idx, initial_states, return_final_states, silu)
 *   -> out or (out, final_states); None when the call is not for this path (an input autograd must
 *      track, or an argument that is not a plain tensor), which the caller then makes in Python. */
PyObject* native_fwd(PyObject*, PyObject* const* a, Py_ssize_t n) {
  if (n != 7) {
    PyErr_Format(PyExc_TypeError, "fwd() takes 7 arguments (%zd given)", n);
    return nullptr;
  }
  try {
    return fwd_impl(a);
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

PyObject* library_error(int rc) {
  PyErr_Format(g_error_type ? g_error_type : PyExc_RuntimeError, "libccv1d error %d: %s", rc,
               ccv1d_last_error());
  return nullptr;
}

// Wraps a tensor, or None for an undefined one; steals nothing on failure.
PyObject* wrap_or_none(at::Tensor&& t) {
  if (!t.defined()) Py_RETURN_NONE;
  return THPVariable_Wrap(std::move(t));
}

/* fwd_train(x, weight, bias, seq_idx, initial_states, final_states, silu) -> out
 * The training forward (ccv1d_fwd) on tensors the Python side has checked and canonicalised
 * (causal_conv1d_fn), writing final_states when given. None when an argument is not a plain
 * tensor, for the Python path. */
PyObject* fwd_train_impl(PyObject* const* a) {
  const at::Tensor *px, *pw, *pb, *ps, *pi, *pf;
  if (!tensor_or_none(a[0], &px) || !tensor_or_none(a[1], &pw) || !tensor_or_none(a[2], &pb) ||
      !tensor_or_none(a[3], &ps) || !tensor_or_none(a[4], &pi) || !tensor_or_none(a[5], &pf) ||
      !px || !pw)
    Py_RETURN_NONE;
  const int silu = PyObject_IsTrue(a[6]);
  if (silu < 0) return nullptr;
  const at::Tensor& x = *px;
  const at::Tensor& w = *pw;
  const int64_t B = x.size(0), T = x.size(1), D = x.size(2), W = w.size(1);
  const int xdt = dtype_code(x.scalar_type()), wdt = dtype_code(w.scalar_type());
  const int bdt = pb ? dtype_code(pb->scalar_type()) : 0;
  const int idt = pi ? dtype_code(pi->scalar_type()) : 0;
  if (xdt < 0 || wdt < 0 || bdt < 0 || idt < 0) {
    PyErr_SetString(PyExc_TypeError, "unsupported dtype (fp32, fp16, bf16 or fp64 expected)");
    return nullptr;
  }
  const int64_t dev = x.get_device();
  at::Tensor out = at::empty({B, T, D}, x.options());
  void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = ccv1d_fwd(x.data_ptr(), x.stride(0), x.stride(1), xdt, w.data_ptr(), wdt,
                 pb ? pb->data_ptr() : nullptr, bdt,
                 ps ? static_cast<const int32_t*>(ps->data_ptr()) : nullptr,
                 pi ? pi->data_ptr() : nullptr, idt, out.data_ptr(),
                 pf ? pf->data_ptr() : nullptr, B, T, D, W, silu, (int)dev, stream);
  Py_END_ALLOW_THREADS
  if (rc) return library_error(rc);
  return THPVariable_Wrap(std::move(out));
}

/* bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, need_dinit, silu)
 *   -> (dx, dweight, dbias or None, dinitial_states or None)
 * The autograd node's backward (the reference's _bwd, causal_conv1d.py:475-541): x, weight, bias,
 * seq_idx and initial_states as the forward saved them (checked and canonicalised), dout with a
 * unit channel stride, dfinal_states contiguous. Allocates the gradients and the fp32 partial-sum
 * workspace (ccv1d_bwd_workspace_bytes) and calls ccv1d_bwd. None when an argument is not a plain
 * tensor, for the Python path. */
PyObject* bwd_impl(PyObject* const* a) {
  const at::Tensor *px, *pw, *pb, *ps, *pi, *pd, *pf;
  if (!tensor_or_none(a[0], &px) || !tensor_or_none(a[1], &pw) || !tensor_or_none(a[2], &pb) ||
      !tensor_or_none(a[3], &ps) || !tensor_or_none(a[4], &pi) || !tensor_or_none(a[5], &pd) ||
      !tensor_or_none(a[6], &pf) || !px || !pw || !pd)
    Py_RETURN_NONE;
  const int need_dinit = PyObject_IsTrue(a[7]);
  const int silu = PyObject_IsTrue(a[8]);
  if (need_dinit < 0 || silu < 0) return nullptr;
  const at::Tensor& x = *px;
  const at::Tensor& w = *pw;
  const at::Tensor& dy = *pd;
  const int64_t dev = x.get_device();
  // The incoming gradients must sit on x's device and carry x's dtype (causal_conv1d.py's
  // _check_grads and _ffi's checks, with their messages).
  if (dy.get_device() != dev) return assertion("the gradient of out must be on the device of x");
  if (pf && pf->get_device() != dev)
    return assertion("the gradient of final_states must be on the device of x");
  // The library reads batch * seqlen * dim elements of dout and batch * (width - 1) * dim of
  // dfinal_states: a smaller tensor would be read past its end.
  if (dy.sizes() != x.sizes()) return assertion("the gradient of out must have the shape of x");
  if (pf && (pf->dim() != 3 || pf->size(0) != x.size(0) || pf->size(1) != w.size(1) - 1 ||
             pf->size(2) != x.size(2)))
    return assertion("the gradient of final_states must be (batch, width - 1, dim)");
  if (dy.scalar_type() != x.scalar_type() || (pf && pf->scalar_type() != x.scalar_type())) {
    PyErr_SetString(PyExc_TypeError, "the gradients of out and final_states must have x's dtype");
    return nullptr;
  }
  const int64_t B = x.size(0), T = x.size(1), D = x.size(2), W = w.size(1);
  const int xdt = dtype_code(x.scalar_type()), wdt = dtype_code(w.scalar_type());
  const int bdt = pb ? dtype_code(pb->scalar_type()) : 0;
  const int idt = pi ? dtype_code(pi->scalar_type()) : 0;
  if (xdt < 0 || wdt < 0 || bdt < 0 || idt < 0) {
    PyErr_SetString(PyExc_TypeError, "unsupported dtype (fp32, fp16, bf16 or fp64 expected)");
    return nullptr;
  }
  at::Tensor dx = at::empty({B, T, D}, x.options());
  at::Tensor dw = at::empty_like(w);
  at::Tensor db = pb ? at::empty_like(*pb) : at::Tensor();
  at::Tensor di = need_dinit && pi ? at::empty_like(*pi) : at::Tensor();
  // The workspace of the path this call takes (dx is contiguous and the allocation aligned).
  const size_t ws_bytes = ccv1d_bwd_workspace_bytes_for(
      x.data_ptr(), x.stride(0), x.stride(1), xdt,
      ps ? static_cast<const int32_t*>(ps->data_ptr()) : nullptr, dy.data_ptr(), dy.stride(0),
      dy.stride(1), pf ? pf->data_ptr() : nullptr, dx.data_ptr(), B, T, D, W);
  at::Tensor ws = ws_bytes ? at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte))
                           : at::Tensor();
  void* stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = ccv1d_bwd(x.data_ptr(), x.stride(0), x.stride(1), xdt, w.data_ptr(), wdt,
                 pb ? pb->data_ptr() : nullptr, bdt,
                 ps ? static_cast<const int32_t*>(ps->data_ptr()) : nullptr,
                 pi ? pi->data_ptr() : nullptr, idt, dy.data_ptr(), dy.stride(0), dy.stride(1),
                 pf ? pf->data_ptr() : nullptr, dx.data_ptr(),
                 di.defined() ? di.data_ptr() : nullptr, dw.data_ptr(),
                 db.defined() ? db.data_ptr() : nullptr, ws.defined() ? ws.data_ptr() : nullptr,
                 ws_bytes, B, T, D, W, silu, (int)dev, stream);
  Py_END_ALLOW_THREADS
  if (rc) return library_error(rc);
  PyObject* r = PyTuple_New(4);
  if (!r) return nullptr;
  PyObject* items[4] = {THPVariable_Wrap(std::move(dx)), THPVariable_Wrap(std::move(dw)),
                        wrap_or_none(std::move(db)), wrap_or_none(std::move(di))};
  for (int i = 0; i < 4; ++i) {
    if (!items[i]) {
      for (int j = 0; j < 4; ++j) Py_XDECREF(items[j]);
      Py_DECREF(r);
      return nullptr;
    }
  }
  for (int i = 0; i < 4; ++i) PyTuple_SET_ITEM(r, i, items[i]);
  return r;
}

template <PyObject* (*IMPL)(PyObject* const*), Py_ssize_t N>
PyObject* native_call(PyObject*, PyObject* const* a, Py_ssize_t n) {
  if (n != N) {
    PyErr_Format(PyExc_TypeError, "takes %zd arguments (%zd given)", N, n);
    return nullptr;
  }
  try {
    return IMPL(a);
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

PyObject* native_set_error_type(PyObject*, PyObject* t) {
  if (!PyType_Check(t) || !PyType_IsSubtype(reinterpret_cast<PyTypeObject*>(t),
                                            reinterpret_cast<PyTypeObject*>(PyExc_Exception))) {
    PyErr_SetString(PyExc_TypeError, "an exception type is expected");
    return nullptr;
  }
  Py_INCREF(t);
  Py_XDECREF(g_error_type);
  g_error_type = t;
  Py_RETURN_NONE;
}

PyMethodDef methods[] = {
    {"fwd", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(native_fwd)),
     METH_FASTCALL, "inference forward; None when the Python path must make the call"},
    {"fwd_train",
     reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(native_call<fwd_train_impl, 7>)),
     METH_FASTCALL, "training forward on checked, canonicalised tensors; None for the Python path"},
    {"bwd", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(native_call<bwd_impl, 9>)),
     METH_FASTCALL, "backward of the autograd node; None for the Python path"},
    {"set_error_type", native_set_error_type, METH_O, "exception type for library errors"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {
    PyModuleDef_HEAD_INIT, "_ccv1d_torch",
    "causal_conv1d_fn's passes over torch tensors, each in one native call", -1, methods,
    nullptr, nullptr, nullptr, nullptr,
};

}  // namespace

PyMODINIT_FUNC PyInit__ccv1d_torch(void) { return PyModule_Create(&module); }
