/*
 * _slmt_fast: a CPython METH_FASTCALL binding of the two per-layer hot entry
 * points of libslmturbo_hip.so (slmt_quantize_store, slmt_decode_paged_batched).
 * ctypes spends ~3 us converting a dozen arguments per call; this module takes
 * the same arguments as plain Python ints (pointers as integers) and calls the
 * library through function pointers that kernels/_native.py hands it from the
 * loaded library (bind), so the two bindings always reach the same code.
 * Host code only: no device work happens here.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "../../include/slmturbo.h"

typedef __typeof__(slmt_quantize_store) store_fn;
typedef __typeof__(slmt_decode_paged_batched) decode_fn;

static store_fn* g_store = NULL;
static decode_fn* g_decode = NULL;

/* args[i] as a 64-bit integer; -1 with an exception set on failure */
static int take(PyObject* const* args, Py_ssize_t n, long long* v) {
  for (Py_ssize_t i = 0; i < n; ++i) {
    v[i] = PyLong_AsLongLong(args[i]);
    if (v[i] == -1 && PyErr_Occurred()) return -1;
  }
  return 0;
}

static PyObject* bind(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  long long v[2];
  if (n != 2) {
    PyErr_SetString(PyExc_TypeError, "bind(store_address, decode_address)");
    return NULL;
  }
  if (take(args, 2, v)) return NULL;
  if (!v[0] || !v[1]) {
    PyErr_SetString(PyExc_ValueError, "bind: null function address");
    return NULL;
  }
  g_store = (store_fn*)(intptr_t)v[0];
  g_decode = (decode_fn*)(intptr_t)v[1];
  Py_RETURN_NONE;
}

static PyObject* quantize_store(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  long long v[12];
  if (!g_store) {
    PyErr_SetString(PyExc_RuntimeError, "quantize_store: library not bound");
    return NULL;
  }
  if (n != 12) {
    PyErr_SetString(PyExc_TypeError, "quantize_store takes 12 arguments");
    return NULL;
  }
  if (take(args, 12, v)) return NULL;
  const int rc = g_store((const void*)(intptr_t)v[0], (int64_t)v[1], (const void*)(intptr_t)v[2], (int64_t)v[3],
                         (void*)(intptr_t)v[4], (int64_t)v[5], (int)v[6], (const int64_t*)(intptr_t)v[7],
                         (int64_t)v[8], (int)v[9], (int)v[10], (slmt_stream_t)(intptr_t)v[11]);
  return PyLong_FromLong(rc);
}

static PyObject* decode_paged_batched(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  long long v[22];
  if (!g_decode) {
    PyErr_SetString(PyExc_RuntimeError, "decode_paged_batched: library not bound");
    return NULL;
  }
  if (n != 22) {
    PyErr_SetString(PyExc_TypeError, "decode_paged_batched takes 22 arguments");
    return NULL;
  }
  if (take(args, 22, v)) return NULL;
  const int rc = g_decode((const void*)(intptr_t)v[0], (int64_t)v[1], (int64_t)v[2], (const void*)(intptr_t)v[3],
                          (int64_t)v[4], (int)v[5], (const void*)(intptr_t)v[6], (int)v[7], (int64_t)v[8],
                          (const int32_t*)(intptr_t)v[9], (int)v[10], (int)v[11], (int)v[12], (int)v[13],
                          (int)v[14], (void*)(intptr_t)v[15], (int)v[16], (int64_t)v[17], (int64_t)v[18],
                          (void*)(intptr_t)v[19], (int64_t)v[20], (slmt_stream_t)(intptr_t)v[21]);
  return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"bind", (PyCFunction)(void (*)(void))bind, METH_FASTCALL, "bind the library's entry points"},
    {"quantize_store", (PyCFunction)(void (*)(void))quantize_store, METH_FASTCALL, "slmt_quantize_store"},
    {"decode_paged_batched", (PyCFunction)(void (*)(void))decode_paged_batched, METH_FASTCALL,
     "slmt_decode_paged_batched"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_slmt_fast", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__slmt_fast(void) { return PyModule_Create(&module); }
