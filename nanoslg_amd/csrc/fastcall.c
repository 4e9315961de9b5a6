/*
 * _nslg_fast: a CPython binding of the C-ABI entry points a forward calls every
 * layer or every step (nslg_kv.h): decode, the planners, append, prefill, page
 * zeroing and copies. Small decode batches and the first chunks of a chunked
 * prefill are paced by the host's Python, not the GPU. Each function takes the entry
 * point's arguments in order, as Python ints (pointers, sizes) and a float (the
 * softmax scale), converts them with the C API's fast-call convention and calls
 * the entry point; it returns the entry point's status. ctypes converts the same
 * 26 arguments of a decode call in ~2.3 us on the host, this binding in a fraction
 * of that. The C ABI is unchanged; this is one more caller of it.
 *
 * Argument codes: p pointer (an int; None for NULL), q int64, i int32, z size_t,
 * f float.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "../../include/nslg_kv.h"

typedef union {
  void* p;
  int64_t q;
  int32_t i;
  size_t z;
  float f;
} arg_t;

#define MAX_ARGS 40

/* Convert args[0..n) by the codes of sig into out; 0, or -1 with a Python error. */
static int parse(const char* name, const char* sig, PyObject* const* args, Py_ssize_t n, arg_t* out) {
  const Py_ssize_t want = (Py_ssize_t)strlen(sig);
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, want, n);
    return -1;
  }
  for (Py_ssize_t k = 0; k < n; ++k) {
    PyObject* o = args[k];
    switch (sig[k]) {
      case 'p':
        if (o == Py_None) {
          out[k].p = NULL;
        } else {
          out[k].p = PyLong_AsVoidPtr(o);
          if (out[k].p == NULL && PyErr_Occurred()) return -1;
        }
        break;
      case 'q': {
        long long v = PyLong_AsLongLong(o);
        if (v == -1 && PyErr_Occurred()) return -1;
        out[k].q = (int64_t)v;
        break;
      }
      case 'z': {
        unsigned long long v = PyLong_AsUnsignedLongLong(o);
        if (v == (unsigned long long)-1 && PyErr_Occurred()) return -1;
        out[k].z = (size_t)v;
        break;
      }
      case 'i': {
        long v = PyLong_AsLong(o);
        if (v == -1 && PyErr_Occurred()) return -1;
        if (v < INT32_MIN || v > INT32_MAX) {
          PyErr_Format(PyExc_OverflowError, "%s: argument %zd out of int32 range", name, k);
          return -1;
        }
        out[k].i = (int32_t)v;
        break;
      }
      case 'f': {
        double v = PyFloat_AsDouble(o);
        if (v == -1.0 && PyErr_Occurred()) return -1;
        out[k].f = (float)v;
        break;
      }
      default:
        PyErr_Format(PyExc_SystemError, "%s: bad signature code", name);
        return -1;
    }
  }
  return 0;
}

static PyObject* paged_decode_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode_append", "pqpqpqppqipppqiiiifipqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode_append(a[0].p, a[1].q, a[2].p, a[3].q, a[4].p, a[5].q, a[6].p, a[7].p, a[8].q,
                                          a[9].i, a[10].p, a[11].p, a[12].p, a[13].q, a[14].i, a[15].i, a[16].i,
                                          a[17].i, a[18].f, a[19].i, a[20].p, a[21].q, a[22].p, a[23].z, a[24].q,
                                          a[25].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_decode_grouped_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode_grouped_append", "pqpqpqppqipppqiiiifipipppqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode_grouped_append(
      a[0].p, a[1].q, a[2].p, a[3].q, a[4].p, a[5].q, a[6].p, a[7].p, a[8].q, a[9].i, a[10].p, a[11].p, a[12].p,
      a[13].q, a[14].i, a[15].i, a[16].i, a[17].i, a[18].f, a[19].i, a[20].p, a[21].i, a[22].p, a[23].p, a[24].p,
      a[25].q, a[26].p, a[27].z, a[28].q, a[29].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_decode(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode", "pqppqipppqiiiifipqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode(a[0].p, a[1].q, a[2].p, a[3].p, a[4].q, a[5].i, a[6].p, a[7].p, a[8].p, a[9].q,
                                   a[10].i, a[11].i, a[12].i, a[13].i, a[14].f, a[15].i, a[16].p, a[17].q, a[18].p,
                                   a[19].z, a[20].q, a[21].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_decode_grouped(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode_grouped", "pqppqipppqiiiifipipppqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode_grouped(a[0].p, a[1].q, a[2].p, a[3].p, a[4].q, a[5].i, a[6].p, a[7].p, a[8].p,
                                           a[9].q, a[10].i, a[11].i, a[12].i, a[13].i, a[14].f, a[15].i, a[16].p,
                                           a[17].i, a[18].p, a[19].p, a[20].p, a[21].q, a[22].p, a[23].z, a[24].q,
                                           a[25].p);
  return PyLong_FromLong(rc);
}

static PyObject* decode_plan_step(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("decode_plan_step", "pppiipppppppppiqiiip", args, n, a)) return NULL;
  const int rc = nslg_decode_plan_step(a[0].p, a[1].p, a[2].p, a[3].i, a[4].i, a[5].p, a[6].p, a[7].p, a[8].p,
                                       a[9].p, a[10].p, a[11].p, a[12].p, a[13].p, a[14].i, a[15].q, a[16].i,
                                       a[17].i, a[18].i, a[19].p);
  return PyLong_FromLong(rc);
}

static PyObject* rope_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("rope_append", "pqpqpqpqppqppqqiiippqip", args, n, a)) return NULL;
  const int rc = nslg_rope_append(a[0].p, a[1].q, a[2].p, a[3].q, a[4].p, a[5].q, a[6].p, a[7].q, a[8].p, a[9].p,
                                  a[10].q, a[11].p, a[12].p, a[13].q, a[14].q, a[15].i, a[16].i, a[17].i, a[18].p,
                                  a[19].p, a[20].q, a[21].i, a[22].p);
  return PyLong_FromLong(rc);
}

static PyObject* append_kv(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("append_kv", "ppqqpippqiiip", args, n, a)) return NULL;
  const int rc = nslg_append_kv(a[0].p, a[1].p, a[2].q, a[3].q, a[4].p, a[5].i, a[6].p, a[7].p, a[8].q, a[9].i,
                                a[10].i, a[11].i, a[12].p);
  return PyLong_FromLong(rc);
}

static PyObject* block_table_csr(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("block_table_csr", "pqpppppqppqip", args, n, a)) return NULL;
  const int rc = nslg_block_table_csr(a[0].p, a[1].q, a[2].p, a[3].p, a[4].p, a[5].p, a[6].p, a[7].q, a[8].p, a[9].p,
                                      a[10].q, a[11].i, a[12].p);
  return PyLong_FromLong(rc);
}

static PyObject* forward_plan(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("forward_plan", "ppppppiiippppp", args, n, a)) return NULL;
  const int rc = nslg_forward_plan(a[0].p, a[1].p, a[2].p, a[3].p, a[4].p, a[5].p, a[6].i, a[7].i, a[8].i, a[9].p,
                                   a[10].p, a[11].p, a[12].p, a[13].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_decode_rope_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode_rope_append", "pqpqpqpppqqppqipppqiiiifipqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode_rope_append(
      a[0].p, a[1].q, a[2].p, a[3].q, a[4].p, a[5].q, a[6].p, a[7].p, a[8].p, a[9].q, a[10].q, a[11].p, a[12].p,
      a[13].q, a[14].i, a[15].p, a[16].p, a[17].p, a[18].q, a[19].i, a[20].i, a[21].i, a[22].i, a[23].f, a[24].i,
      a[25].p, a[26].q, a[27].p, a[28].z, a[29].q, a[30].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_decode_grouped_rope_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_decode_grouped_rope_append", "pqpqpqpppqqppqipppqiiiifipipppqpzqp", args, n, a)) return NULL;
  const int rc = nslg_paged_decode_grouped_rope_append(
      a[0].p, a[1].q, a[2].p, a[3].q, a[4].p, a[5].q, a[6].p, a[7].p, a[8].p, a[9].q, a[10].q, a[11].p, a[12].p,
      a[13].q, a[14].i, a[15].p, a[16].p, a[17].p, a[18].q, a[19].i, a[20].i, a[21].i, a[22].i, a[23].f, a[24].i,
      a[25].p, a[26].i, a[27].p, a[28].p, a[29].p, a[30].q, a[31].p, a[32].z, a[33].q, a[34].p);
  return PyLong_FromLong(rc);
}

static PyObject* forward_plan_csr(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("forward_plan_csr", "pqpppppqppqpppiiippppp", args, n, a)) return NULL;
  const int rc = nslg_forward_plan_csr(a[0].p, a[1].q, a[2].p, a[3].p, a[4].p, a[5].p, a[6].p, a[7].q, a[8].p, a[9].p,
                                       a[10].q, a[11].p, a[12].p, a[13].p, a[14].i, a[15].i, a[16].i, a[17].p,
                                       a[18].p, a[19].p, a[20].p, a[21].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_prefill(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_prefill", "pqpqippqipppiiiifipqpzp", args, n, a)) return NULL;
  const int rc = nslg_paged_prefill(a[0].p, a[1].q, a[2].p, a[3].q, a[4].i, a[5].p, a[6].p, a[7].q, a[8].i, a[9].p,
                                    a[10].p, a[11].p, a[12].i, a[13].i, a[14].i, a[15].i, a[16].f, a[17].i, a[18].p,
                                    a[19].q, a[20].p, a[21].z, a[22].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_prefill_grid(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_prefill_grid", "pqppiqippqipppiiiifipqpzp", args, n, a)) return NULL;
  const int rc = nslg_paged_prefill_grid(a[0].p, a[1].q, a[2].p, a[3].p, a[4].i, a[5].q, a[6].i, a[7].p, a[8].p,
                                         a[9].q, a[10].i, a[11].p, a[12].p, a[13].p, a[14].i, a[15].i, a[16].i,
                                         a[17].i, a[18].f, a[19].i, a[20].p, a[21].q, a[22].p, a[23].z, a[24].p);
  return PyLong_FromLong(rc);
}

static PyObject* paged_prefill_append(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("paged_prefill_append", "pqppiqipqpqppqipppiiiifipqpzp", args, n, a)) return NULL;
  const int rc = nslg_paged_prefill_append(a[0].p, a[1].q, a[2].p, a[3].p, a[4].i, a[5].q, a[6].i, a[7].p, a[8].q,
                                           a[9].p, a[10].q, a[11].p, a[12].p, a[13].q, a[14].i, a[15].p, a[16].p,
                                           a[17].p, a[18].i, a[19].i, a[20].i, a[21].i, a[22].f, a[23].i, a[24].p,
                                           a[25].q, a[26].p, a[27].z, a[28].p);
  return PyLong_FromLong(rc);
}

static PyObject* zero_pages(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("zero_pages", "ppiqiiiipip", args, n, a)) return NULL;
  const int rc = nslg_zero_pages(a[0].p, a[1].p, a[2].i, a[3].q, a[4].i, a[5].i, a[6].i, a[7].i, a[8].p, a[9].i,
                                 a[10].p);
  return PyLong_FromLong(rc);
}

static PyObject* copy_pages(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  arg_t a[MAX_ARGS];
  if (parse("copy_pages", "ppiqiiiippip", args, n, a)) return NULL;
  const int rc = nslg_copy_pages(a[0].p, a[1].p, a[2].i, a[3].q, a[4].i, a[5].i, a[6].i, a[7].i, a[8].p, a[9].p,
                                 a[10].i, a[11].p);
  return PyLong_FromLong(rc);
}

static PyMethodDef methods[] = {
    {"paged_decode_append", (PyCFunction)(void (*)(void))paged_decode_append, METH_FASTCALL,
     "nslg_paged_decode_append: the entry point's arguments in order; returns its status"},
    {"paged_decode_grouped_append", (PyCFunction)(void (*)(void))paged_decode_grouped_append, METH_FASTCALL,
     "nslg_paged_decode_grouped_append: the entry point's arguments in order; returns its status"},
    {"paged_decode", (PyCFunction)(void (*)(void))paged_decode, METH_FASTCALL,
     "nslg_paged_decode: the entry point's arguments in order; returns its status"},
    {"paged_decode_grouped", (PyCFunction)(void (*)(void))paged_decode_grouped, METH_FASTCALL,
     "nslg_paged_decode_grouped: the entry point's arguments in order; returns its status"},
    {"decode_plan_step", (PyCFunction)(void (*)(void))decode_plan_step, METH_FASTCALL,
     "nslg_decode_plan_step: the entry point's arguments in order; returns its status"},
    {"rope_append", (PyCFunction)(void (*)(void))rope_append, METH_FASTCALL,
     "nslg_rope_append: the entry point's arguments in order; returns its status"},
    {"append_kv", (PyCFunction)(void (*)(void))append_kv, METH_FASTCALL,
     "nslg_append_kv: the entry point's arguments in order; returns its status"},
    {"block_table_csr", (PyCFunction)(void (*)(void))block_table_csr, METH_FASTCALL,
     "nslg_block_table_csr: the entry point's arguments in order; returns its status"},
    {"forward_plan", (PyCFunction)(void (*)(void))forward_plan, METH_FASTCALL,
     "nslg_forward_plan: the entry point's arguments in order; returns its status"},
    {"paged_decode_rope_append", (PyCFunction)(void (*)(void))paged_decode_rope_append, METH_FASTCALL,
     "nslg_paged_decode_rope_append: the entry point's arguments in order; returns its status"},
    {"paged_decode_grouped_rope_append", (PyCFunction)(void (*)(void))paged_decode_grouped_rope_append, METH_FASTCALL,
     "nslg_paged_decode_grouped_rope_append: the entry point's arguments in order; returns its status"},
    {"forward_plan_csr", (PyCFunction)(void (*)(void))forward_plan_csr, METH_FASTCALL,
     "nslg_forward_plan_csr: the entry point's arguments in order; returns its status"},
    {"paged_prefill", (PyCFunction)(void (*)(void))paged_prefill, METH_FASTCALL,
     "nslg_paged_prefill: the entry point's arguments in order; returns its status"},
    {"paged_prefill_grid", (PyCFunction)(void (*)(void))paged_prefill_grid, METH_FASTCALL,
     "nslg_paged_prefill_grid: the entry point's arguments in order; returns its status"},
    {"paged_prefill_append", (PyCFunction)(void (*)(void))paged_prefill_append, METH_FASTCALL,
     "nslg_paged_prefill_append: the entry point's arguments in order; returns its status"},
    {"zero_pages", (PyCFunction)(void (*)(void))zero_pages, METH_FASTCALL,
     "nslg_zero_pages: the entry point's arguments in order; returns its status"},
    {"copy_pages", (PyCFunction)(void (*)(void))copy_pages, METH_FASTCALL,
     "nslg_copy_pages: the entry point's arguments in order; returns its status"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_nslg_fast",
                                    "Fast-call binding of the per-step entry points of libnslg_kv", -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__nslg_fast(void) { return PyModule_Create(&module); }
