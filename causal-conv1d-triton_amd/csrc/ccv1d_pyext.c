/* CPython binding of the two launch entry points of libccv1d.so (include/ccv1d.h), for the
 * Python side of the package (causal_conv1d_triton/_ffi.py). It takes the same arguments as the C
 * ABI, as Python ints (device pointers from Tensor.data_ptr(), None for a null pointer), and
 * returns the C status code; the caller raises on a non-zero code with ccv1d_last_error().
 *
 * It exists to cut the per-call host cost of small calls (decode steps): argument conversion here
 * is one C call per argument, where a ctypes call converts every argument through its own
 * Python-level type machinery (about 1 us for the 20 arguments of ccv1d_fwd on an MI355X host).
 * The GIL is released around the launch, as ctypes does. It links libccv1d.so from its own
 * directory (rpath $ORIGIN), the same file the ctypes binding loads.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "ccv1d.h"

/* None -> NULL, int -> pointer. */
static int arg_ptr(PyObject* o, void** p) {
  if (o == Py_None) {
    *p = NULL;
    return 0;
  }
  *p = PyLong_AsVoidPtr(o);
  return (*p == NULL && PyErr_Occurred()) ? -1 : 0;
}

static int arg_i64(PyObject* o, int64_t* v) {
  const long long x = PyLong_AsLongLong(o);
  if (x == -1 && PyErr_Occurred()) return -1;
  *v = (int64_t)x;
  return 0;
}

static int arg_int(PyObject* o, int* v) {
  const long x = PyLong_AsLong(o);
  if (x == -1 && PyErr_Occurred()) return -1;
  if (x < INT32_MIN || x > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "argument does not fit a C int");
    return -1;
  }
  *v = (int)x;
  return 0;
}

static int arg_count(Py_ssize_t n, Py_ssize_t want, const char* name) {
  if (n == want) return 0;
  PyErr_Format(PyExc_TypeError, "%s() takes %zd arguments (%zd given)", name, want, n);
  return -1;
}

/* fwd(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype, seq_idx,
 *     initial_states, init_dtype, out, final_states, batch, seqlen, dim, width, silu, device,
 *     stream) -> status: the arguments of ccv1d_fwd in order. */
static PyObject* native_fwd(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  void *x, *w, *b, *seq, *init, *out, *fin, *stream;
  int64_t sxb, sxt, B, T, D, W;
  int xdt, wdt, bdt, idt, silu, dev;
  if (arg_count(n, 20, "fwd") || arg_ptr(a[0], &x) || arg_i64(a[1], &sxb) || arg_i64(a[2], &sxt) ||
      arg_int(a[3], &xdt) || arg_ptr(a[4], &w) || arg_int(a[5], &wdt) || arg_ptr(a[6], &b) ||
      arg_int(a[7], &bdt) || arg_ptr(a[8], &seq) || arg_ptr(a[9], &init) || arg_int(a[10], &idt) ||
      arg_ptr(a[11], &out) || arg_ptr(a[12], &fin) || arg_i64(a[13], &B) || arg_i64(a[14], &T) ||
      arg_i64(a[15], &D) || arg_i64(a[16], &W) || arg_int(a[17], &silu) || arg_int(a[18], &dev) ||
      arg_ptr(a[19], &stream))
    return NULL;
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = ccv1d_fwd(x, sxb, sxt, xdt, w, wdt, b, bdt, (const int32_t*)seq, init, idt, out, fin, B, T, D,
                 W, silu, dev, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

/* bwd(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype, seq_idx,
 *     initial_states, init_dtype, dout, dout_stride_b, dout_stride_t, dfinal_states, dx,
 *     dinitial_states, dweight, dbias, workspace, workspace_bytes, batch, seqlen, dim, width, silu,
 *     device, stream) -> status: the arguments of ccv1d_bwd in order. */
static PyObject* native_bwd(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  void *x, *w, *b, *seq, *init, *dy, *dfin, *dx, *dinit, *dw, *db, *ws, *stream;
  int64_t sxb, sxt, syb, syt, wsb, B, T, D, W;
  int xdt, wdt, bdt, idt, silu, dev;
  if (arg_count(n, 28, "bwd") || arg_ptr(a[0], &x) || arg_i64(a[1], &sxb) || arg_i64(a[2], &sxt) ||
      arg_int(a[3], &xdt) || arg_ptr(a[4], &w) || arg_int(a[5], &wdt) || arg_ptr(a[6], &b) ||
      arg_int(a[7], &bdt) || arg_ptr(a[8], &seq) || arg_ptr(a[9], &init) || arg_int(a[10], &idt) ||
      arg_ptr(a[11], &dy) || arg_i64(a[12], &syb) || arg_i64(a[13], &syt) ||
      arg_ptr(a[14], &dfin) || arg_ptr(a[15], &dx) || arg_ptr(a[16], &dinit) ||
      arg_ptr(a[17], &dw) || arg_ptr(a[18], &db) || arg_ptr(a[19], &ws) || arg_i64(a[20], &wsb) ||
      arg_i64(a[21], &B) || arg_i64(a[22], &T) || arg_i64(a[23], &D) || arg_i64(a[24], &W) ||
      arg_int(a[25], &silu) || arg_int(a[26], &dev) || arg_ptr(a[27], &stream))
    return NULL;
  if (wsb < 0) {
    PyErr_SetString(PyExc_ValueError, "negative workspace size");
    return NULL;
  }
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = ccv1d_bwd(x, sxb, sxt, xdt, w, wdt, b, bdt, (const int32_t*)seq, init, idt, dy, syb, syt,
                 dfin, dx, dinit, dw, db, ws, (size_t)wsb, B, T, D, W, silu, dev, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyObject* native_abi_version(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  return PyLong_FromLong(ccv1d_abi_version());
}

static PyMethodDef methods[] = {
    {"fwd", (PyCFunction)(void (*)(void))native_fwd, METH_FASTCALL, "ccv1d_fwd; returns the status"},
    {"bwd", (PyCFunction)(void (*)(void))native_bwd, METH_FASTCALL, "ccv1d_bwd; returns the status"},
    {"abi_version", native_abi_version, METH_NOARGS, "ccv1d_abi_version()"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {
    PyModuleDef_HEAD_INIT, "_ccv1d_native", "CPython binding of libccv1d.so's launch entry points",
    -1, methods, NULL, NULL, NULL, NULL,
};

PyMODINIT_FUNC PyInit__ccv1d_native(void) { return PyModule_Create(&module); }
