/*
 * _fastcall: CPython fast-call bindings of the C-ABI entry points that the
 * calibration hooks call once per batch (g2ptq_hessian_stage), for callers
 * that deliver many small batches (an MoE block's routed tokens: thousands
 * of add_batch calls per layer).  Each function takes the same arguments as
 * the entry point, as Python integers (pointers and streams as addresses),
 * and returns its status; the caller raises on a nonzero status exactly as
 * for the ctypes binding.  It calls the entry point of libg2ptq_hip.so
 * (linked, resolved next to this module) and adds no logic of its own.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include "../../include/g2ptq_hip.h"

static int as_ptr(PyObject* o, void** out) {
  if (o == Py_None) {
    *out = NULL;
    return 0;
  }
  const unsigned long long v = PyLong_AsUnsignedLongLong(o);
  if (v == (unsigned long long)-1 && PyErr_Occurred()) return -1;
  *out = (void*)(uintptr_t)v;
  return 0;
}

static int as_i64(PyObject* o, int64_t* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)v;
  return 0;
}

/* hessian_stage(stream, X, T, C, ldx, XT, ldt, t_off) -> status */
static PyObject* hessian_stage(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 8) {
    PyErr_SetString(PyExc_TypeError, "hessian_stage takes 8 arguments");
    return NULL;
  }
  void *stream, *X, *XT;
  int64_t T, C, ldx, ldt, t_off;
  if (as_ptr(args[0], &stream) || as_ptr(args[1], &X) || as_i64(args[2], &T) ||
      as_i64(args[3], &C) || as_i64(args[4], &ldx) || as_ptr(args[5], &XT) ||
      as_i64(args[6], &ldt) || as_i64(args[7], &t_off))
    return NULL;
  const int status = g2ptq_hessian_stage(stream, (const uint16_t*)X, T, C, ldx, (uint16_t*)XT,
                                         ldt, t_off);
  return PyLong_FromLong(status);
}

static PyMethodDef methods[] = {
    {"hessian_stage", (PyCFunction)(void (*)(void))hessian_stage, METH_FASTCALL,
     "g2ptq_hessian_stage(stream, X, T, C, ldx, XT, ldt, t_off) -> status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastcall", NULL, -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fastcall(void) { return PyModule_Create(&module); }
