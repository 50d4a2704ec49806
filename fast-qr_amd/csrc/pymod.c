/*
 * pymod.c — thin CPython binding over the C ABI in include/fastqr.h.
 *
 * It only converts Python ints to the ABI's int64 / pointer arguments
 * (METH_FASTCALL, no argument tuples) and returns the status code; all
 * validation and every launch happen behind the fastqr_* entry points.  It exists so
 * that a call costs well under a microsecond of host time; ctypes over the
 * same library is equivalent and is what the tests use to check the ABI.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "fastqr.h"

static int as_i64(PyObject* o, int64_t* out) {
  long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)v;
  return 0;
}

static int as_ptr(PyObject* o, void** out) {
  unsigned long long v = PyLong_AsUnsignedLongLong(o);
  if (v == (unsigned long long)-1 && PyErr_Occurred()) return -1;
  *out = (void*)(uintptr_t)v;
  return 0;
}

/* geqrf(A, batch, n, as0, as1, as2, H, hs0, hs1, hs2, tau, ts0, ts1, ws, ws_bytes, stream) -> int */
static PyObject* py_geqrf(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 16) {
    PyErr_SetString(PyExc_TypeError, "geqrf expects 16 integer arguments");
    return NULL;
  }
  void *A, *H, *tau, *ws, *stream;
  int64_t b, n, as0, as1, as2, hs0, hs1, hs2, ts0, ts1, wsb;
  if (as_ptr(args[0], &A) || as_i64(args[1], &b) || as_i64(args[2], &n) || as_i64(args[3], &as0) ||
      as_i64(args[4], &as1) || as_i64(args[5], &as2) || as_ptr(args[6], &H) || as_i64(args[7], &hs0) ||
      as_i64(args[8], &hs1) || as_i64(args[9], &hs2) || as_ptr(args[10], &tau) || as_i64(args[11], &ts0) ||
      as_i64(args[12], &ts1) || as_ptr(args[13], &ws) || as_i64(args[14], &wsb) || as_ptr(args[15], &stream))
    return NULL;
  const int rc = fastqr_geqrf_f32((const float*)A, b, n, as0, as1, as2, (float*)H, hs0, hs1, hs2, (float*)tau,
                                  ts0, ts1, ws, (size_t)wsb, stream);
  return PyLong_FromLong(rc);
}

/* orgqr(H, batch, n, hs0, hs1, hs2, tau, ts0, ts1, Q, qs0, qs1, qs2, ws, ws_bytes, stream) -> int */
static PyObject* py_orgqr(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 16) {
    PyErr_SetString(PyExc_TypeError, "orgqr expects 16 integer arguments");
    return NULL;
  }
  void *H, *tau, *Q, *ws, *stream;
  int64_t b, n, hs0, hs1, hs2, ts0, ts1, qs0, qs1, qs2, wsb;
  if (as_ptr(args[0], &H) || as_i64(args[1], &b) || as_i64(args[2], &n) || as_i64(args[3], &hs0) ||
      as_i64(args[4], &hs1) || as_i64(args[5], &hs2) || as_ptr(args[6], &tau) || as_i64(args[7], &ts0) ||
      as_i64(args[8], &ts1) || as_ptr(args[9], &Q) || as_i64(args[10], &qs0) || as_i64(args[11], &qs1) ||
      as_i64(args[12], &qs2) || as_ptr(args[13], &ws) || as_i64(args[14], &wsb) || as_ptr(args[15], &stream))
    return NULL;
  const int rc = fastqr_orgqr_f32((const float*)H, b, n, hs0, hs1, hs2, (const float*)tau, ts0, ts1, (float*)Q, qs0,
                                  qs1, qs2, ws, (size_t)wsb, stream);
  return PyLong_FromLong(rc);
}

/* ormqr(H, batch, m, r, hs0, hs1, hs2, tau, ts0, ts1, C, k, cs0, cs1, cs2, transpose, ws, ws_bytes, stream) -> int */
static PyObject* py_ormqr(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 19) {
    PyErr_SetString(PyExc_TypeError, "ormqr expects 19 integer arguments");
    return NULL;
  }
  void *H, *tau, *C, *ws, *stream;
  int64_t b, m, r, hs0, hs1, hs2, ts0, ts1, k, cs0, cs1, cs2, tr, wsb;
  if (as_ptr(args[0], &H) || as_i64(args[1], &b) || as_i64(args[2], &m) || as_i64(args[3], &r) ||
      as_i64(args[4], &hs0) || as_i64(args[5], &hs1) || as_i64(args[6], &hs2) || as_ptr(args[7], &tau) ||
      as_i64(args[8], &ts0) || as_i64(args[9], &ts1) || as_ptr(args[10], &C) || as_i64(args[11], &k) ||
      as_i64(args[12], &cs0) || as_i64(args[13], &cs1) || as_i64(args[14], &cs2) || as_i64(args[15], &tr) ||
      as_ptr(args[16], &ws) || as_i64(args[17], &wsb) || as_ptr(args[18], &stream))
    return NULL;
  const int rc = fastqr_ormqr_f32((const float*)H, b, m, r, hs0, hs1, hs2, (const float*)tau, ts0, ts1, (float*)C, k,
                                  cs0, cs1, cs2, (int)tr, ws, (size_t)wsb, stream);
  return PyLong_FromLong(rc);
}

/* geqrf_mixed(A, batch, n, as0, as1, as2, H, hs0, hs1, hs2, tau, ts0, ts1, panel_width, precision, flags, ws,
 *             ws_bytes, stream) -> int */
static PyObject* py_geqrf_mixed(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 19) {
    PyErr_SetString(PyExc_TypeError, "geqrf_mixed expects 19 integer arguments");
    return NULL;
  }
  void *A, *H, *tau, *ws, *stream;
  int64_t b, n, as0, as1, as2, hs0, hs1, hs2, ts0, ts1, pw, prec, flags, wsb;
  if (as_ptr(args[0], &A) || as_i64(args[1], &b) || as_i64(args[2], &n) || as_i64(args[3], &as0) ||
      as_i64(args[4], &as1) || as_i64(args[5], &as2) || as_ptr(args[6], &H) || as_i64(args[7], &hs0) ||
      as_i64(args[8], &hs1) || as_i64(args[9], &hs2) || as_ptr(args[10], &tau) || as_i64(args[11], &ts0) ||
      as_i64(args[12], &ts1) || as_i64(args[13], &pw) || as_i64(args[14], &prec) || as_i64(args[15], &flags) ||
      as_ptr(args[16], &ws) || as_i64(args[17], &wsb) || as_ptr(args[18], &stream))
    return NULL;
  const int rc = fastqr_geqrf_mixed_f32((const float*)A, b, n, as0, as1, as2, (float*)H, hs0, hs1, hs2, (float*)tau,
                                        ts0, ts1, pw, (int)prec, (int)flags, ws, (size_t)wsb, stream);
  return PyLong_FromLong(rc);
}

static PyObject* py_geqrf_mixed_workspace_bytes(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  int64_t b, n, pw, flags;
  if (nargs != 4 || as_i64(args[0], &b) || as_i64(args[1], &n) || as_i64(args[2], &pw) || as_i64(args[3], &flags)) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "geqrf_mixed_workspace_bytes(batch, n, panel_width, flags)");
    return NULL;
  }
  return PyLong_FromSize_t(fastqr_geqrf_mixed_workspace_bytes(b, n, pw, (int)flags));
}

static PyObject* py_ormqr_workspace_bytes(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  int64_t b, m, r, k;
  if (nargs != 4 || as_i64(args[0], &b) || as_i64(args[1], &m) || as_i64(args[2], &r) || as_i64(args[3], &k)) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "ormqr_workspace_bytes(batch, m, r, k)");
    return NULL;
  }
  return PyLong_FromSize_t(fastqr_ormqr_workspace_bytes(b, m, r, k));
}

static PyObject* py_orgqr_workspace_bytes(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  int64_t b, n;
  if (nargs != 2 || as_i64(args[0], &b) || as_i64(args[1], &n)) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "orgqr_workspace_bytes(batch, n)");
    return NULL;
  }
  return PyLong_FromSize_t(fastqr_orgqr_workspace_bytes(b, n));
}

static PyObject* py_workspace_bytes(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  int64_t b, n;
  if (nargs != 2 || as_i64(args[0], &b) || as_i64(args[1], &n)) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "workspace_bytes(batch, n)");
    return NULL;
  }
  return PyLong_FromSize_t(fastqr_workspace_bytes(b, n));
}

static PyObject* py_last_error(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  return PyUnicode_FromString(fastqr_last_error());
}

static PyObject* py_path_name(PyObject* self, PyObject* arg) {
  (void)self;
  int64_t n;
  if (as_i64(arg, &n)) return NULL;
  return PyUnicode_FromString(fastqr_path_name(n));
}

static PyObject* py_version(PyObject* self, PyObject* unused) {
  (void)self;
  (void)unused;
  return PyLong_FromLong(fastqr_version());
}

static PyMethodDef methods[] = {
    {"geqrf", (PyCFunction)(void (*)(void))py_geqrf, METH_FASTCALL, "fastqr_geqrf_f32 over raw pointers"},
    {"workspace_bytes", (PyCFunction)(void (*)(void))py_workspace_bytes, METH_FASTCALL, "fastqr_workspace_bytes"},
    {"orgqr", (PyCFunction)(void (*)(void))py_orgqr, METH_FASTCALL, "fastqr_orgqr_f32 over raw pointers"},
    {"orgqr_workspace_bytes", (PyCFunction)(void (*)(void))py_orgqr_workspace_bytes, METH_FASTCALL,
     "fastqr_orgqr_workspace_bytes"},
    {"ormqr", (PyCFunction)(void (*)(void))py_ormqr, METH_FASTCALL, "fastqr_ormqr_f32 over raw pointers"},
    {"ormqr_workspace_bytes", (PyCFunction)(void (*)(void))py_ormqr_workspace_bytes, METH_FASTCALL,
     "fastqr_ormqr_workspace_bytes"},
    {"geqrf_mixed", (PyCFunction)(void (*)(void))py_geqrf_mixed, METH_FASTCALL,
     "fastqr_geqrf_mixed_f32 over raw pointers"},
    {"geqrf_mixed_workspace_bytes", (PyCFunction)(void (*)(void))py_geqrf_mixed_workspace_bytes, METH_FASTCALL,
     "fastqr_geqrf_mixed_workspace_bytes"},
    {"last_error", py_last_error, METH_NOARGS, "fastqr_last_error"},
    {"path_name", py_path_name, METH_O, "fastqr_path_name"},
    {"version", py_version, METH_NOARGS, "fastqr_version"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastqr_py", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fastqr_py(void) { return PyModule_Create(&module); }
