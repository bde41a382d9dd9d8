/* CPython binding of the per-token (small-M) INT4 + LoRA forward entry points.
 *
 * An eager small-M forward spends more time on the host than on the GPU, and
 * ctypes' per-argument conversion is a large share of it. These functions
 * take the same arguments as the C ABI (device pointers as Python ints, NULL
 * as None) through METH_FASTCALL and forward them unchanged; each returns the
 * C function's status or size. They add nothing else: validation, errors
 * (rpx_last_error) and launches are the library's.
 *
 * Built against librepresentax_amd.so in the same directory (rpath $ORIGIN),
 * so the process holds one instance of the library whichever binding it uses.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <stdint.h>

#include "../../include/representax_amd.h"

#define MAX_PROJECTIONS 16
#define PROJECTION_FIELDS 11

static int get_i64(PyObject* o, int64_t* v) {
  long long x = PyLong_AsLongLong(o);
  if (x == -1 && PyErr_Occurred()) return 0;
  *v = (int64_t)x;
  return 1;
}

static int get_int(PyObject* o, int* v) {
  long x = PyLong_AsLong(o);
  if (x == -1 && PyErr_Occurred()) return 0;
  if (x < INT32_MIN || x > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "value does not fit a C int");
    return 0;
  }
  *v = (int)x;
  return 1;
}

static int get_ptr(PyObject* o, void** p) {
  if (o == Py_None) {
    *p = NULL;
    return 1;
  }
  unsigned long long x = PyLong_AsUnsignedLongLong(o);
  if (x == (unsigned long long)-1 && PyErr_Occurred()) return 0;
  *p = (void*)(uintptr_t)x;
  return 1;
}

static int get_f32(PyObject* o, float* v) {
  double x = PyFloat_AsDouble(o);
  if (x == -1.0 && PyErr_Occurred()) return 0;
  *v = (float)x;
  return 1;
}

static int check_nargs(const char* name, Py_ssize_t nargs, Py_ssize_t want) {
  if (nargs == want) return 1;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, want, nargs);
  return 0;
}

/* int4lora_forward(x, dtype, m, k, packed, scale_bits, n, group_size,
 *                  bias_bits, lora_a, lora_b, rank, scaling, y, h,
 *                  workspace, workspace_bytes, stream) -> status */
static PyObject* fast_int4lora_forward(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  void *x, *packed, *scales, *bias, *a, *b, *y, *h, *ws, *stream;
  int dtype;
  int64_t m, k, n, group, rank, ws_bytes;
  float scaling;
  if (!check_nargs("int4lora_forward", nargs, 18)) return NULL;
  if (!get_ptr(args[0], &x) || !get_int(args[1], &dtype) || !get_i64(args[2], &m) ||
      !get_i64(args[3], &k) || !get_ptr(args[4], &packed) || !get_ptr(args[5], &scales) ||
      !get_i64(args[6], &n) || !get_i64(args[7], &group) || !get_ptr(args[8], &bias) ||
      !get_ptr(args[9], &a) || !get_ptr(args[10], &b) || !get_i64(args[11], &rank) ||
      !get_f32(args[12], &scaling) || !get_ptr(args[13], &y) || !get_ptr(args[14], &h) ||
      !get_ptr(args[15], &ws) || !get_i64(args[16], &ws_bytes) || !get_ptr(args[17], &stream))
    return NULL;
  if (ws_bytes < 0) {
    PyErr_SetString(PyExc_ValueError, "workspace_bytes must be non-negative");
    return NULL;
  }
  int status = rpx_int4lora_forward(x, dtype, m, k, (const uint8_t*)packed,
                                    (const uint16_t*)scales, n, group, (const uint16_t*)bias, a, b,
                                    rank, scaling, y, h, ws, (size_t)ws_bytes, stream);
  return PyLong_FromLong(status);
}

/* int4lora_forward_workspace(m, n, k, group_size, rank, dtype) -> bytes */
static PyObject* fast_int4lora_forward_workspace(PyObject* self, PyObject* const* args,
                                                 Py_ssize_t nargs) {
  (void)self;
  int64_t m, n, k, group, rank;
  int dtype;
  if (!check_nargs("int4lora_forward_workspace", nargs, 6)) return NULL;
  if (!get_i64(args[0], &m) || !get_i64(args[1], &n) || !get_i64(args[2], &k) ||
      !get_i64(args[3], &group) || !get_i64(args[4], &rank) || !get_int(args[5], &dtype))
    return NULL;
  return PyLong_FromSize_t(rpx_int4lora_forward_workspace(m, n, k, group, rank, dtype));
}

/* Fills table[0, count) from a tuple of count x 11 fields in the order of
 * rpx_int4lora_projection: packed, scale_bits, n, group_size, bias_bits,
 * lora_a, lora_b, rank, scaling, y, h. */
static int fill_projections(PyObject* flat, rpx_int4lora_projection* table, int* count) {
  if (!PyTuple_Check(flat)) {
    PyErr_SetString(PyExc_TypeError, "projections must be a flat tuple");
    return 0;
  }
  Py_ssize_t len = PyTuple_GET_SIZE(flat);
  if (len % PROJECTION_FIELDS != 0 || len / PROJECTION_FIELDS > MAX_PROJECTIONS) {
    PyErr_Format(PyExc_ValueError,
                 "projections: expected a multiple of %d fields for at most %d projections",
                 PROJECTION_FIELDS, MAX_PROJECTIONS);
    return 0;
  }
  *count = (int)(len / PROJECTION_FIELDS);
  for (int i = 0; i < *count; ++i) {
    PyObject* const* f = &PyTuple_GET_ITEM(flat, (Py_ssize_t)i * PROJECTION_FIELDS);
    void *packed, *scales, *bias, *a, *b, *y, *h;
    rpx_int4lora_projection* p = &table[i];
    if (!get_ptr(f[0], &packed) || !get_ptr(f[1], &scales) || !get_i64(f[2], &p->n) ||
        !get_i64(f[3], &p->group_size) || !get_ptr(f[4], &bias) || !get_ptr(f[5], &a) ||
        !get_ptr(f[6], &b) || !get_i64(f[7], &p->rank) || !get_f32(f[8], &p->scaling) ||
        !get_ptr(f[9], &y) || !get_ptr(f[10], &h))
      return 0;
    p->packed = (const uint8_t*)packed;
    p->scale_bits = (const uint16_t*)scales;
    p->bias_bits = (const uint16_t*)bias;
    p->lora_a = a;
    p->lora_b = b;
    p->y = y;
    p->h = h;
  }
  return 1;
}

/* int4lora_forward_multi_workspace(m, k, projections, dtype) -> bytes */
static PyObject* fast_int4lora_forward_multi_workspace(PyObject* self, PyObject* const* args,
                                                       Py_ssize_t nargs) {
  (void)self;
  int64_t m, k;
  int dtype, count;
  rpx_int4lora_projection table[MAX_PROJECTIONS];
  if (!check_nargs("int4lora_forward_multi_workspace", nargs, 4)) return NULL;
  if (!get_i64(args[0], &m) || !get_i64(args[1], &k) || !fill_projections(args[2], table, &count) ||
      !get_int(args[3], &dtype))
    return NULL;
  return PyLong_FromSize_t(rpx_int4lora_forward_multi_workspace(m, k, count, table, dtype));
}

/* int4lora_forward_multi(x, dtype, m, k, projections, workspace,
 *                        workspace_bytes, stream) -> status */
static PyObject* fast_int4lora_forward_multi(PyObject* self, PyObject* const* args,
                                             Py_ssize_t nargs) {
  (void)self;
  void *x, *ws, *stream;
  int dtype, count;
  int64_t m, k, ws_bytes;
  rpx_int4lora_projection table[MAX_PROJECTIONS];
  if (!check_nargs("int4lora_forward_multi", nargs, 8)) return NULL;
  if (!get_ptr(args[0], &x) || !get_int(args[1], &dtype) || !get_i64(args[2], &m) ||
      !get_i64(args[3], &k) || !fill_projections(args[4], table, &count) ||
      !get_ptr(args[5], &ws) || !get_i64(args[6], &ws_bytes) || !get_ptr(args[7], &stream))
    return NULL;
  if (ws_bytes < 0) {
    PyErr_SetString(PyExc_ValueError, "workspace_bytes must be non-negative");
    return NULL;
  }
  int status = rpx_int4lora_forward_multi(x, dtype, m, k, count, table, ws, (size_t)ws_bytes,
                                          stream);
  return PyLong_FromLong(status);
}

/* get_tuning(knob) -> value: the library's knob as this binding sees it (the
 * check that both bindings share one loaded library). */
static PyObject* fast_get_tuning(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  int knob;
  if (!check_nargs("get_tuning", nargs, 1)) return NULL;
  if (!get_int(args[0], &knob)) return NULL;
  return PyLong_FromLong(rpx_get_tuning(knob));
}

static PyMethodDef methods[] = {
    {"get_tuning", (PyCFunction)(void (*)(void))fast_get_tuning, METH_FASTCALL, "rpx_get_tuning"},
    {"int4lora_forward", (PyCFunction)(void (*)(void))fast_int4lora_forward, METH_FASTCALL,
     "rpx_int4lora_forward"},
    {"int4lora_forward_workspace", (PyCFunction)(void (*)(void))fast_int4lora_forward_workspace,
     METH_FASTCALL, "rpx_int4lora_forward_workspace"},
    {"int4lora_forward_multi", (PyCFunction)(void (*)(void))fast_int4lora_forward_multi,
     METH_FASTCALL, "rpx_int4lora_forward_multi"},
    {"int4lora_forward_multi_workspace",
     (PyCFunction)(void (*)(void))fast_int4lora_forward_multi_workspace, METH_FASTCALL,
     "rpx_int4lora_forward_multi_workspace"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_rpxfast",
                                    "Fast-call binding of the small-M forward entry points.", -1,
                                    methods};

PyMODINIT_FUNC PyInit__rpxfast(void) { return PyModule_Create(&module); }
