/*
 * _nslg_host: the host bookkeeping of a forward whose per-token plan is expanded on
 * the device (prefill chunks and other forwards of many new tokens), in one call
 * instead of some sixty small numpy operations (kv_cache.py:575-615 is the reference
 * rule set it follows: write plan, tokens_used, CSR pointers, last-page lengths).
 *
 * plan_forward(states, ntoks, offsets, page_size, ref_count, tokens_used, mark,
 *              zero_pages, out, place)
 *   states      sequence states (objects with num_tokens, n_pages, bt, row, row_cap,
 *               synced)
 *   ntoks       new tokens per sequence (list of int)
 *   offsets     input offsets per sequence (list of int), or None for zeros
 *   ref_count   int64 [P], tokens_used int64 [P] (updated), mark uint8/bool [P]
 *               (all zero on entry and on return)
 *   zero_pages  list of page ids awaiting zero-on-allocation, or None
 *   out         int32 buffer the plan is written to
 *   place       called, in order, with each state whose device row is missing
 *               (row < 0) or shorter than its table (row_cap < n_pages), once the
 *               forward is known to be planned here (it gives the state its device
 *               row: row, row_cap, synced)
 * Returns None when a page the forward writes is shared (copy-on-write is then the
 * caller's; nothing was changed), -n when `out` may need n entries and holds fewer
 * (nothing was changed), else (total, total_pages, patch_entries, zero_entries,
 * shared_first) with shared_first true when some sequence's first page has more than
 * one reference (a decode batch can only have prefix groups then) and out[:total]
 * holding, in order:
 *   kv_indptr [B+1], last_page_len [B], copy sources [0], copy destinations [0],
 *   pages to zero [nz], start [B], new tokens [B], input offsets [B], pages held [B],
 *   device row [B], pages held [B], entries already on the device [B],
 *   patch pointers [B+1], patch (the table entries the device rows lack) [max(np, 1)]
 * and tokens_used raised for every written page to its last written slot + 1. Pages
 * to zero are those of zero_pages that the forward does not write in every slot
 * (a page written whole needs no zeroing: the forward's own write of its rows leaves
 * the same bytes).
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

static PyObject *s_num_tokens, *s_n_pages, *s_bt, *s_row, *s_row_cap, *s_synced;

static int get_i64(PyObject* obj, PyObject* name, int64_t* out) {
  PyObject* v = PyObject_GetAttr(obj, name);
  if (!v) return -1;
  long long x = PyLong_AsLongLong(v);
  Py_DECREF(v);
  if (x == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)x;
  return 0;
}

static int64_t floordiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

typedef struct {
  int64_t start, n_raw, n, off, have, row, syn, p0, plast, cnt;
  Py_buffer bt;
} seq_t;

static int get_buf(PyObject* o, Py_buffer* b, int writable, Py_ssize_t itemsize, const char* what) {
  if (PyObject_GetBuffer(o, b, PyBUF_C_CONTIGUOUS | PyBUF_FORMAT | (writable ? PyBUF_WRITABLE : 0)) < 0) return -1;
  if (b->itemsize != itemsize) {
    PyErr_Format(PyExc_TypeError, "plan_forward: %s must have %zd-byte items", what, itemsize);
    PyBuffer_Release(b);
    return -1;
  }
  return 0;
}

static PyObject* plan_forward(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 10) {
    PyErr_SetString(PyExc_TypeError, "plan_forward takes 10 arguments");
    return NULL;
  }
  PyObject* place = args[9];
  if (!PyCallable_Check(place)) {
    PyErr_SetString(PyExc_TypeError, "plan_forward: place must be callable");
    return NULL;
  }
  PyObject *states = args[0], *ntoks = args[1], *offsets = args[2], *zero = args[7];
  const long ps = PyLong_AsLong(args[3]);
  if (ps == -1 && PyErr_Occurred()) return NULL;
  if (ps <= 0) {
    PyErr_SetString(PyExc_ValueError, "plan_forward: page_size must be positive");
    return NULL;
  }
  if (!PyList_Check(states) || !PyList_Check(ntoks) || (offsets != Py_None && !PyList_Check(offsets)) ||
      (zero != Py_None && !PyList_Check(zero))) {
    PyErr_SetString(PyExc_TypeError, "plan_forward: states, ntoks, offsets and zero_pages must be lists");
    return NULL;
  }
  const Py_ssize_t B = PyList_GET_SIZE(states);
  if (PyList_GET_SIZE(ntoks) != B || (offsets != Py_None && PyList_GET_SIZE(offsets) != B)) {
    PyErr_SetString(PyExc_ValueError, "plan_forward: one count and one offset per sequence");
    return NULL;
  }
  Py_buffer rc = {0}, tu = {0}, mk = {0}, ob = {0};
  seq_t* sq = NULL;
  Py_ssize_t nbt = 0;
  PyObject* result = NULL;
  if (get_buf(args[4], &rc, 0, 8, "ref_count") < 0) return NULL;
  if (get_buf(args[5], &tu, 1, 8, "tokens_used") < 0) goto done;
  if (get_buf(args[6], &mk, 1, 1, "mark") < 0) goto done;
  if (get_buf(args[8], &ob, 1, 4, "out") < 0) goto done;
  const int64_t P = rc.len / 8;
  if (tu.len / 8 != P || mk.len != P) {
    PyErr_SetString(PyExc_ValueError, "plan_forward: ref_count, tokens_used and mark must cover the same pages");
    goto done;
  }
  const int64_t* ref = (const int64_t*)rc.buf;
  int64_t* used = (int64_t*)tu.buf;
  uint8_t* mark = (uint8_t*)mk.buf;
  sq = (seq_t*)PyMem_Calloc(B > 0 ? (size_t)B : 1, sizeof(seq_t));
  if (!sq) {
    PyErr_NoMemory();
    goto done;
  }

  /* pass 1: the sequences' numbers and the written pages' sharing */
  int64_t npatch = 0, held = 0;
  int shared_first = 0;
  for (Py_ssize_t b = 0; b < B; ++b) {
    PyObject* st = PyList_GET_ITEM(states, b);
    seq_t* s = &sq[b];
    if (get_i64(st, s_num_tokens, &s->start) < 0 || get_i64(st, s_n_pages, &s->have) < 0) goto done;
    long long n = PyLong_AsLongLong(PyList_GET_ITEM(ntoks, b));
    if (n == -1 && PyErr_Occurred()) goto done;
    s->n_raw = n;
    s->n = n > 0 ? n : 0;
    s->off = 0;
    if (offsets != Py_None) {
      long long o = PyLong_AsLongLong(PyList_GET_ITEM(offsets, b));
      if (o == -1 && PyErr_Occurred()) goto done;
      s->off = o;
    }
    PyObject* bt = PyObject_GetAttr(st, s_bt);
    if (!bt) goto done;
    int r = get_buf(bt, &s->bt, 0, 4, "a block table");
    Py_DECREF(bt);
    if (r < 0) goto done;
    ++nbt;
    if (s->have < 0 || s->have > s->bt.len / 4) {
      PyErr_SetString(PyExc_ValueError, "plan_forward: a sequence holds more pages than its table");
      goto done;
    }
    /* the plan is int32: positions and lengths below 2^31 */
    if (s->start < 0 || s->start > 0x7fffffffLL || s->n_raw > 0x7fffffffLL || s->start + s->n > 0x7fffffffLL ||
        s->off < -0x7fffffffLL || s->off > 0x7fffffffLL) {
      PyErr_SetString(PyExc_ValueError, "plan_forward: a sequence's tokens, new tokens or offset out of range");
      goto done;
    }
    held += s->have;
    s->p0 = floordiv(s->start, ps);
    s->plast = floordiv(s->start + s->n - 1, ps);
    int64_t c = 0;
    if (s->n > 0) {
      c = (s->plast + 1 < s->have ? s->plast + 1 : s->have) - s->p0;
      if (c < 0) c = 0;
    }
    s->cnt = c;
    const int32_t* t = (const int32_t*)s->bt.buf;
    if (s->have > 0 && t[0] > 0 && t[0] < P && ref[t[0]] > 1) shared_first = 1;
    for (int64_t i = 0; i < c; ++i) {
      const int64_t pid = t[s->p0 + i];
      if (pid < 0 || pid >= P) {
        PyErr_SetString(PyExc_ValueError, "plan_forward: a block table names a page outside the pool");
        goto done;
      }
      if (ref[pid] > 1) { /* a shared page is written: copy-on-write, the caller's path */
        Py_INCREF(Py_None);
        result = Py_None;
        goto done;
      }
    }
  }
  /* the output's size with every table entry in the patch (placing a row can make
     the whole table due): checked before anything changes */
  const Py_ssize_t nzl = zero == Py_None ? 0 : PyList_GET_SIZE(zero);
  const int64_t bound = (B + 1) + B + nzl + 4 * (int64_t)B + 3 * (int64_t)B + (B + 1) + (held > 0 ? held : 1);
  if (ob.len / 4 < bound) {
    result = PyLong_FromLongLong(-(long long)bound);
    goto done;
  }
  for (Py_ssize_t j = 0; j < nzl; ++j) { /* check the ids before anything is written */
    long long z = PyLong_AsLongLong(PyList_GET_ITEM(zero, j));
    if (z == -1 && PyErr_Occurred()) goto done;
    if (z < 0 || z >= P) {
      PyErr_SetString(PyExc_ValueError, "plan_forward: a page to zero lies outside the pool");
      goto done;
    }
  }

  /* the forward is planned here: the device rows (placed where a state has none or
     one too short), then the entries they lack */
  for (Py_ssize_t b = 0; b < B; ++b) {
    PyObject* st = PyList_GET_ITEM(states, b);
    seq_t* s = &sq[b];
    int64_t row0 = 0, cap0 = 0;
    if (get_i64(st, s_row, &row0) < 0 || get_i64(st, s_row_cap, &cap0) < 0) goto done;
    s->row = row0;
    if (row0 < 0 || cap0 < s->have) {
      PyObject* r = PyObject_CallOneArg(place, st);
      if (!r) goto done;
      Py_DECREF(r);
      int64_t have = 0;
      if (get_i64(st, s_row, &s->row) < 0 || get_i64(st, s_n_pages, &have) < 0) goto done;
      if (have != s->have) {
        PyErr_SetString(PyExc_RuntimeError, "plan_forward: place changed a sequence's pages");
        goto done;
      }
    }
    if (get_i64(st, s_synced, &s->syn) < 0) goto done;
    if (s->syn > s->have) s->syn = s->have;
    if (s->syn < 0) s->syn = 0;
    npatch += s->have - s->syn;
  }

  /* pass 2: tokens_used, the pages written whole, the plan arrays */
  int32_t* o = (int32_t*)ob.buf;
  int32_t* indptr = o;
  int32_t* lpl = indptr + (B + 1);
  int32_t* zout = lpl + B; /* copy sources and destinations are empty */
  indptr[0] = 0;
  for (Py_ssize_t b = 0; b < B; ++b) {
    seq_t* s = &sq[b];
    const int32_t* t = (const int32_t*)s->bt.buf;
    const int64_t end = s->start + s->n; /* one past the last written token */
    for (int64_t i = 0; i < s->cnt; ++i) {
      const int64_t pidx = s->p0 + i;
      const int64_t pid = t[pidx];
      const int64_t last = pidx == s->plast ? end - 1 - s->plast * ps : ps - 1;
      if (used[pid] < last + 1) used[pid] = last + 1;
      if (nzl && pidx * ps >= s->start && (pidx + 1) * ps <= end) mark[pid] = 1;
    }
    const int64_t len = s->start + s->n_raw;
    const int64_t npg = len > 0 ? (len + ps - 1) / ps : 0;
    indptr[b + 1] = (int32_t)(indptr[b] + npg);
    lpl[b] = (int32_t)(npg > 0 ? len - (npg - 1) * ps : 0);
  }
  Py_ssize_t nz = 0;
  for (Py_ssize_t j = 0; j < nzl; ++j) {
    const long long z = PyLong_AsLongLong(PyList_GET_ITEM(zero, j));
    if (!mark[z]) zout[nz++] = (int32_t)z;
  }
  if (nzl) { /* clear the marks */
    for (Py_ssize_t b = 0; b < B; ++b) {
      const int32_t* t = (const int32_t*)sq[b].bt.buf;
      for (int64_t i = 0; i < sq[b].cnt; ++i) mark[t[sq[b].p0 + i]] = 0;
    }
  }
  int32_t* w = zout + nz;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].start;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].n_raw;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].off;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].have;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].row;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].have;
  w += B;
  for (Py_ssize_t b = 0; b < B; ++b) w[b] = (int32_t)sq[b].syn;
  w += B;
  int32_t* pip = w;
  pip[0] = 0;
  for (Py_ssize_t b = 0; b < B; ++b) pip[b + 1] = (int32_t)(pip[b] + (sq[b].have - sq[b].syn));
  w += B + 1;
  if (npatch == 0) {
    w[0] = 0;
    ++w;
  } else {
    for (Py_ssize_t b = 0; b < B; ++b) {
      const int32_t* t = (const int32_t*)sq[b].bt.buf;
      const int64_t k = sq[b].have - sq[b].syn;
      memcpy(w, t + sq[b].syn, (size_t)k * 4);
      w += k;
    }
  }
  const int64_t used_total = (int64_t)(w - o);
  result = Py_BuildValue("(LLLnO)", (long long)used_total, (long long)indptr[B], (long long)npatch, nz,
                         shared_first ? Py_True : Py_False);

done:
  if (sq) {
    for (Py_ssize_t b = 0; b < nbt; ++b) PyBuffer_Release(&sq[b].bt);
    PyMem_Free(sq);
  }
  if (ob.obj) PyBuffer_Release(&ob);
  if (mk.obj) PyBuffer_Release(&mk);
  if (tu.obj) PyBuffer_Release(&tu);
  if (rc.obj) PyBuffer_Release(&rc);
  return result;
}

static PyMethodDef methods[] = {
    {"plan_forward", (PyCFunction)(void (*)(void))plan_forward, METH_FASTCALL,
     "Host bookkeeping and plan arrays of a device-planned forward (see the module comment)."},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_nslg_host",
                                    "Host-side forward planning of the KV cache.", -1, methods};

PyMODINIT_FUNC PyInit__nslg_host(void) {
  s_num_tokens = PyUnicode_InternFromString("num_tokens");
  s_n_pages = PyUnicode_InternFromString("n_pages");
  s_bt = PyUnicode_InternFromString("bt");
  s_row = PyUnicode_InternFromString("row");
  s_row_cap = PyUnicode_InternFromString("row_cap");
  s_synced = PyUnicode_InternFromString("synced");
  if (!s_num_tokens || !s_n_pages || !s_bt || !s_row || !s_row_cap || !s_synced) return NULL;
  return PyModule_Create(&module);
}
