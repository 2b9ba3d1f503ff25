/* Python binding of one layer's GEMM call (host C, CPython API; no torch).
 *
 * _occall.Layer(fn, wbits, in_features, qt, st, scale_dtype, zt, N, K_phys,
 *               group_rows, kmap, kinv)
 * binds the arguments of oc_int4_gemm (wbits 4) or oc_int8_gemm (wbits 8)
 * that stay fixed for a layer: fn is the entry point's address, the tensors
 * are device addresses (None: NULL). Calling the object,
 *   layer(a, lda, a_dtype, M, bias, bias_dtype, c, ldc, workspace,
 *         workspace_bytes, stream) -> status
 * makes the call (regime: automatic) and returns the entry point's status.
 * Arguments arrive through the vectorcall protocol and are converted in
 * place: no tuple and no per-argument foreign-function marshalling. The
 * object holds raw addresses only; the caller keeps the tensors alive. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stddef.h>
#include <stdint.h>

typedef int (*gemm4_t)(const void *, int64_t, int32_t, int32_t, int32_t, const int32_t *, const void *, int32_t,
                       const int32_t *, int32_t, int32_t, int32_t, const int32_t *, const uint16_t *, const void *,
                       int32_t, void *, int64_t, void *, size_t, int32_t, void *);
typedef int (*gemm8_t)(const void *, int64_t, int32_t, int32_t, int32_t, const int32_t *, const void *, int32_t,
                       const int32_t *, int32_t, int32_t, int32_t, const int32_t *, const uint16_t *, const void *,
                       int32_t, void *, int64_t, void *, size_t, void *);

typedef struct {
  PyObject_HEAD
  vectorcallfunc vectorcall;
  void *fn;
  int wbits;
  int32_t in_features, scale_dtype, N, k_phys, group_rows;
  const int32_t *qt, *zt, *kmap;
  const void *st;
  const uint16_t *kinv;
} Layer;

/* None -> NULL, else the integer as an address. */
static int as_ptr(PyObject *o, void **out) {
  if (o == Py_None) {
    *out = NULL;
    return 0;
  }
  *out = PyLong_AsVoidPtr(o);
  return (*out == NULL && PyErr_Occurred()) ? -1 : 0;
}

static int as_i64(PyObject *o, int64_t *out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)v;
  return 0;
}

static PyObject *layer_call(PyObject *self_, PyObject *const *args, size_t nargsf, PyObject *kwnames) {
  Layer *self = (Layer *)self_;
  if (PyVectorcall_NARGS(nargsf) != 11 || (kwnames && PyTuple_GET_SIZE(kwnames) > 0)) {
    PyErr_SetString(PyExc_TypeError,
                    "Layer(a, lda, a_dtype, M, bias, bias_dtype, c, ldc, workspace, workspace_bytes, stream)");
    return NULL;
  }
  void *a, *bias, *c, *ws, *stream;
  int64_t lda, a_dtype, M, bias_dtype, ldc, ws_bytes;
  if (as_ptr(args[0], &a) || as_i64(args[1], &lda) || as_i64(args[2], &a_dtype) || as_i64(args[3], &M) ||
      as_ptr(args[4], &bias) || as_i64(args[5], &bias_dtype) || as_ptr(args[6], &c) || as_i64(args[7], &ldc) ||
      as_ptr(args[8], &ws) || as_i64(args[9], &ws_bytes) || as_ptr(args[10], &stream))
    return NULL;
  if (M < 0 || M > INT32_MAX || ws_bytes < 0) {
    PyErr_SetString(PyExc_ValueError, "M or workspace_bytes out of range");
    return NULL;
  }
  int status;
  if (self->wbits == 4)
    status = ((gemm4_t)self->fn)(a, lda, (int32_t)a_dtype, (int32_t)M, self->in_features, self->qt, self->st,
                                 self->scale_dtype, self->zt, self->N, self->k_phys, self->group_rows, self->kmap,
                                 self->kinv, bias, (int32_t)bias_dtype, c, ldc, ws, (size_t)ws_bytes, 0, stream);
  else
    status = ((gemm8_t)self->fn)(a, lda, (int32_t)a_dtype, (int32_t)M, self->in_features, self->qt, self->st,
                                 self->scale_dtype, self->zt, self->N, self->k_phys, self->group_rows, self->kmap,
                                 self->kinv, bias, (int32_t)bias_dtype, c, ldc, ws, (size_t)ws_bytes, stream);
  return PyLong_FromLong(status);
}

static PyObject *layer_new(PyTypeObject *type, PyObject *args, PyObject *kwds) {
  PyObject *fn, *qt, *st, *zt, *kmap, *kinv;
  int wbits, in_features, scale_dtype, N, k_phys, group_rows;
  static char *kw[] = {"fn", "wbits", "in_features", "qt", "st", "scale_dtype", "zt", "N", "K_phys", "group_rows",
                       "kmap", "kinv", NULL};
  if (!PyArg_ParseTupleAndKeywords(args, kwds, "OiiOOiOiiiOO", kw, &fn, &wbits, &in_features, &qt, &st,
                                   &scale_dtype, &zt, &N, &k_phys, &group_rows, &kmap, &kinv))
    return NULL;
  if (wbits != 4 && wbits != 8) {
    PyErr_SetString(PyExc_ValueError, "wbits must be 4 or 8");
    return NULL;
  }
  Layer *self = (Layer *)type->tp_alloc(type, 0);
  if (!self) return NULL;
  void *p_fn, *p_qt, *p_st, *p_zt, *p_kmap, *p_kinv;
  if (as_ptr(fn, &p_fn) || as_ptr(qt, &p_qt) || as_ptr(st, &p_st) || as_ptr(zt, &p_zt) || as_ptr(kmap, &p_kmap) ||
      as_ptr(kinv, &p_kinv)) {
    Py_DECREF(self);
    return NULL;
  }
  if (!p_fn) {
    Py_DECREF(self);
    PyErr_SetString(PyExc_ValueError, "fn is NULL");
    return NULL;
  }
  self->vectorcall = layer_call;
  self->fn = p_fn;
  self->wbits = wbits;
  self->in_features = in_features;
  self->scale_dtype = scale_dtype;
  self->N = N;
  self->k_phys = k_phys;
  self->group_rows = group_rows;
  self->qt = (const int32_t *)p_qt;
  self->st = p_st;
  self->zt = (const int32_t *)p_zt;
  self->kmap = (const int32_t *)p_kmap;
  self->kinv = (const uint16_t *)p_kinv;
  return (PyObject *)self;
}

static PyTypeObject LayerType = {
    PyVarObject_HEAD_INIT(NULL, 0).tp_name = "_occall.Layer",
    .tp_basicsize = sizeof(Layer),
    .tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_HAVE_VECTORCALL,
    .tp_doc = "One layer's oc_int4_gemm / oc_int8_gemm call with its fixed arguments bound.",
    .tp_new = layer_new,
    .tp_call = PyVectorcall_Call,
    .tp_vectorcall_offset = offsetof(Layer, vectorcall),
};

static struct PyModuleDef occall_module = {PyModuleDef_HEAD_INIT, "_occall",
                                           "Per-layer GEMM calls into libonecomp_hip (CPython binding).", -1, NULL};

PyMODINIT_FUNC PyInit__occall(void) {
  if (PyType_Ready(&LayerType) < 0) return NULL;
  PyObject *m = PyModule_Create(&occall_module);
  if (!m) return NULL;
  Py_INCREF(&LayerType);
  if (PyModule_AddObject(m, "Layer", (PyObject *)&LayerType) < 0) {
    Py_DECREF(&LayerType);
    Py_DECREF(m);
    return NULL;
  }
  return m;
}
