/* Host half of a decode step's KV appends, on the manager's own Python objects.
 *
 * mentat_amd.core.paged_kv_cache plans every step's appends on the host: per
 * layer and sequence, a new tail page when the last one is full, copy-on-write
 * of a shared tail, the slot and the new counters (reference
 * core/paged_kv_cache.py:227-284, append_tokens_batched). This module runs the
 * same steps, in the same order, on the same objects: the SequenceState lists
 * (page tables, counters), the allocator's refcount list and its free set,
 * taking ids with PySet_Pop, which is set.pop(). So block ids, refcounts, the
 * free set and every list come out exactly as the Python planner leaves them.
 *
 * Every entry point first checks the objects' types and sizes (lists of ints,
 * an allocator with a set and a list); if anything is not as expected it
 * returns None before changing anything, and the caller runs the Python
 * planner. Errors raised part-way (out of blocks, a release of a free block)
 * leave the state as the Python planner leaves it at the same point.
 *
 *   append_batched(seqs, layer, block_size, allocator, out)
 *       plan_append_batched: out is a writable int32 [7, N] buffer.
 *   step_begin(seqs, num_layers, block_size, allocator, plan)
 *       plan_append_step_begin's layer 0; returns (step state, uniform) or None.
 *   step_layers(state, l0, upto, num_layers, block_size, allocator, plan)
 *       the layers l0 .. upto - 1 of the same step.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static PyObject *s_page_table, *s_tilb, *s_num_tokens, *s_row, *s_free, *s_refcounts, *s_peak, *s_alloc;

/* ---- the allocator ------------------------------------------------------ */

typedef struct {
  PyObject* obj;   /* BlockAllocator (borrowed) */
  PyObject* free;  /* its set of free ids (new reference) */
  PyObject* rc;    /* its refcount list (new reference) */
  Py_ssize_t n;    /* pool size */
  long peak;
  int peak_dirty;
} Alloc;

static void alloc_close(Alloc* a) {
  Py_CLEAR(a->free);
  Py_CLEAR(a->rc);
}

/* 1: usable, 0: not the expected objects (no error set), -1: error */
static int alloc_open(Alloc* a, PyObject* obj) {
  memset(a, 0, sizeof(*a));
  a->obj = obj;
  a->free = PyObject_GetAttr(obj, s_free);
  a->rc = PyObject_GetAttr(obj, s_refcounts);
  PyObject* pk = PyObject_GetAttr(obj, s_peak);
  if (!a->free || !a->rc || !pk) {
    Py_XDECREF(pk);
    alloc_close(a);
    PyErr_Clear();
    return 0;
  }
  int ok = PySet_CheckExact(a->free) && PyList_CheckExact(a->rc) && PyLong_CheckExact(pk);
  if (ok) {
    a->n = PyList_GET_SIZE(a->rc);
    a->peak = PyLong_AsLong(pk);
    if (a->peak == -1 && PyErr_Occurred()) ok = -1;
  }
  Py_DECREF(pk);
  if (ok != 1) alloc_close(a);
  return ok;
}

/* Store the peak back (the allocator's _peak_used), whatever happened. */
static int alloc_finish(Alloc* a) {
  int st = 0;
  if (a->peak_dirty) {
    PyObject *et, *ev, *tb;
    PyErr_Fetch(&et, &ev, &tb);
    PyObject* v = PyLong_FromLong(a->peak);
    if (!v || PyObject_SetAttr(a->obj, s_peak, v) < 0) st = -1;
    Py_XDECREF(v);
    if (et) PyErr_Restore(et, ev, tb);
  }
  alloc_close(a);
  return st;
}

static int rc_get(Alloc* a, long b, long* v) {
  if (b < 0 || b >= a->n) {
    PyErr_Format(PyExc_IndexError, "block id %ld outside the pool", b);
    return -1;
  }
  *v = PyLong_AsLong(PyList_GET_ITEM(a->rc, b));
  return (*v == -1 && PyErr_Occurred()) ? -1 : 0;
}

static int list_set(PyObject* list, Py_ssize_t i, long v) {
  PyObject* o = PyLong_FromLong(v);
  if (!o) return -1;
  return PyList_SetItem(list, i, o); /* steals o */
}

/* BlockAllocator.alloc: set.pop() of the free set, refcount 1, peak. */
static int alloc_one(Alloc* a, long* out) {
  if (PySet_GET_SIZE(a->free) == 0) {
    /* the allocator's own error, with its message */
    PyObject* r = PyObject_CallMethodObjArgs(a->obj, s_alloc, NULL);
    if (r) {
      Py_DECREF(r);
      PyErr_SetString(PyExc_RuntimeError, "PagedKVCache: allocator returned a block from an empty pool");
    }
    return -1;
  }
  PyObject* b = PySet_Pop(a->free);
  if (!b) return -1;
  long blk = PyLong_AsLong(b);
  Py_DECREF(b);
  if (blk == -1 && PyErr_Occurred()) return -1;
  if (blk < 0 || blk >= a->n) {
    PyErr_Format(PyExc_IndexError, "block id %ld outside the pool", blk);
    return -1;
  }
  if (list_set(a->rc, blk, 1) < 0) return -1;
  long used = (long)(a->n - PySet_GET_SIZE(a->free));
  if (used > a->peak) {
    a->peak = used;
    a->peak_dirty = 1;
  }
  *out = blk;
  return 0;
}

/* BlockAllocator.release */
static int release_one(Alloc* a, long blk) {
  long v;
  if (rc_get(a, blk, &v) < 0) return -1;
  if (v <= 0) {
    PyErr_Format(PyExc_AssertionError, "release() on free block %ld", blk);
    return -1;
  }
  if (list_set(a->rc, blk, v - 1) < 0) return -1;
  if (v - 1 == 0) {
    PyObject* o = PyLong_FromLong(blk);
    if (!o) return -1;
    int r = PySet_Add(a->free, o);
    Py_DECREF(o);
    if (r < 0) return -1;
  }
  return 0;
}

/* ---- the sequences ------------------------------------------------------ */

typedef struct {
  PyObject* pt;   /* page_table: list of per-layer lists (new references) */
  PyObject* tilb; /* tokens_in_last_block */
  PyObject* nt;   /* num_tokens */
  long row;
} Seq;

static void seqs_close(Seq* s, Py_ssize_t n) {
  if (!s) return;
  for (Py_ssize_t i = 0; i < n; ++i) {
    Py_XDECREF(s[i].pt);
    Py_XDECREF(s[i].tilb);
    Py_XDECREF(s[i].nt);
  }
  free(s);
}

static int is_int_list(PyObject* l, Py_ssize_t min_len) {
  if (!PyList_CheckExact(l) || PyList_GET_SIZE(l) < min_len) return 0;
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(l); ++i)
    if (!PyLong_CheckExact(PyList_GET_ITEM(l, i))) return 0;
  return 1;
}

/* The sequences' lists, checked: page_table a list of at least `layers`
 * lists, the counters lists of at least `layers` ints, row an int.
 * 1: usable (*out set), 0: not as expected, -1: error. */
static int seqs_open(PyObject* seqs, Py_ssize_t layers, Seq** out, Py_ssize_t* n_out) {
  *out = NULL;
  *n_out = 0;
  if (!PyList_CheckExact(seqs)) return 0;
  const Py_ssize_t n = PyList_GET_SIZE(seqs);
  Seq* s = (Seq*)calloc(n > 0 ? (size_t)n : 1, sizeof(Seq));
  if (!s) {
    PyErr_NoMemory();
    return -1;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* q = PyList_GET_ITEM(seqs, i);
    s[i].pt = PyObject_GetAttr(q, s_page_table);
    s[i].tilb = PyObject_GetAttr(q, s_tilb);
    s[i].nt = PyObject_GetAttr(q, s_num_tokens);
    PyObject* row = PyObject_GetAttr(q, s_row);
    int ok = s[i].pt && s[i].tilb && s[i].nt && row && PyLong_CheckExact(row);
    if (ok) {
      s[i].row = PyLong_AsLong(row);
      ok = !(s[i].row == -1 && PyErr_Occurred());
    }
    Py_XDECREF(row);
    ok = ok && PyList_CheckExact(s[i].pt) && PyList_GET_SIZE(s[i].pt) >= layers && is_int_list(s[i].tilb, layers) &&
         is_int_list(s[i].nt, layers);
    /* (table entries are read as ints where used; only the lists are checked here) */
    for (Py_ssize_t l = 0; ok && l < layers; ++l) ok = PyList_CheckExact(PyList_GET_ITEM(s[i].pt, l));
    if (!ok) {
      PyErr_Clear();
      seqs_close(s, i + 1);
      return 0;
    }
  }
  *out = s;
  *n_out = n;
  return 1;
}

static long lget(PyObject* list, Py_ssize_t i) { return PyLong_AsLong(PyList_GET_ITEM(list, i)); }

/* list[i] = list[0] (the same int object, as a slice assignment of [list[0]] * k stores) */
static void copy_first(PyObject* list, Py_ssize_t i) {
  PyObject* v = PyList_GET_ITEM(list, 0);
  Py_INCREF(v);
  PyObject* old = PyList_GET_ITEM(list, i);
  PyList_SET_ITEM(list, i, v);
  Py_DECREF(old);
}

/* list[i] == list[0] for two lists of ints (checked by seqs_open) */
static int equal_first(PyObject* list, Py_ssize_t i) {
  PyObject *a = PyList_GET_ITEM(list, 0), *b = PyList_GET_ITEM(list, i);
  return a == b || PyLong_AsLong(a) == PyLong_AsLong(b);
}

/* A writable C-contiguous int32 buffer of exactly `count` elements. */
static int get_i32(PyObject* o, Py_buffer* view, Py_ssize_t count) {
  if (PyObject_GetBuffer(o, view, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS | PyBUF_FORMAT) < 0) {
    PyErr_Clear();
    return 0;
  }
  if (view->itemsize != 4 || !view->format || strcmp(view->format, "i") != 0 || view->len != count * 4) {
    PyBuffer_Release(view);
    return 0;
  }
  return 1;
}

/* ---- one layer, as plan_append_batched ---------------------------------- */

/* out: int32 [7][n]; rows dst, slot, cow source, table row, page index, new length, batch index */
static int plan_layer(Seq* s, Py_ssize_t n, Py_ssize_t L, long B, Alloc* a, int32_t* out) {
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* table = PyList_GET_ITEM(s[i].pt, L);
    long slot = lget(s[i].tilb, L);
    if (PyList_GET_SIZE(table) == 0 || slot == B) {
      long b;
      if (alloc_one(a, &b) < 0) return -1;
      PyObject* o = PyLong_FromLong(b);
      if (!o) return -1;
      int r = PyList_Append(table, o);
      Py_DECREF(o);
      if (r < 0 || list_set(s[i].tilb, L, 0) < 0) return -1;
      slot = 0;
    }
    const Py_ssize_t last = PyList_GET_SIZE(table) - 1;
    long tail = lget(table, last), rcv, cow = -1;
    if (rc_get(a, tail, &rcv) < 0) return -1;
    if (rcv > 1) { /* shared tail: copy-on-write */
      long nb;
      if (alloc_one(a, &nb) < 0 || release_one(a, tail) < 0 || list_set(table, last, nb) < 0) return -1;
      cow = tail;
      tail = nb;
    }
    if (list_set(s[i].tilb, L, slot + 1) < 0) return -1;
    const long len = lget(s[i].nt, L) + 1;
    if (list_set(s[i].nt, L, len) < 0) return -1;
    out[0 * n + i] = (int32_t)tail;
    out[1 * n + i] = (int32_t)slot;
    out[2 * n + i] = (int32_t)cow;
    out[3 * n + i] = (int32_t)s[i].row;
    out[4 * n + i] = (int32_t)last;
    out[5 * n + i] = (int32_t)len;
    out[6 * n + i] = (int32_t)i;
  }
  return 0;
}

static PyObject* py_append_batched(PyObject* self, PyObject* args) {
  PyObject *seqs, *alloc_obj, *out_obj;
  Py_ssize_t L;
  long B;
  if (!PyArg_ParseTuple(args, "OnlOO", &seqs, &L, &B, &alloc_obj, &out_obj)) return NULL;
  Seq* s;
  Py_ssize_t n;
  int ok = seqs_open(seqs, L + 1, &s, &n);
  if (ok <= 0) return ok < 0 ? NULL : Py_NewRef(Py_None);
  Alloc a;
  Py_buffer view;
  ok = alloc_open(&a, alloc_obj);
  if (ok <= 0) {
    seqs_close(s, n);
    return ok < 0 ? NULL : Py_NewRef(Py_None);
  }
  if (!get_i32(out_obj, &view, 7 * n)) {
    alloc_close(&a);
    seqs_close(s, n);
    Py_RETURN_NONE;
  }
  int st = plan_layer(s, n, L, B, &a, (int32_t*)view.buf);
  PyBuffer_Release(&view);
  if (alloc_finish(&a) < 0) st = -1;
  seqs_close(s, n);
  if (st < 0) return NULL;
  Py_RETURN_TRUE;
}

/* ---- the step: layer 0 planned, the other layers replay its events ------ */

/* The step state, between step_begin and step_layers: the sequences' lists
 * (references held; nothing else may touch the manager in between), layer
 * 0's tails and their refcounts before the step, each sequence's group (the
 * sequences whose layer-0 tails are one block form a group, numbered in
 * order of first appearance), and layer 0's events. */
typedef struct {
  Seq* s;
  Py_ssize_t n, n_events;
  int uniform, paged, shared0;
  long ngroups0;
  int32_t *tails0, *rc0, *group, *ev; /* ev: pairs (batch index, kind 0 new page / 1 copy-on-write) */
  int32_t *rep, *hash;                /* per-layer scratch: a block per group; open addressing, hcap slots */
  long hcap;
} Step;

static void step_free(Step* st) {
  if (!st) return;
  seqs_close(st->s, st->n);
  free(st->tails0);
  free(st->rc0);
  free(st->group);
  free(st->ev);
  free(st->rep);
  free(st->hash);
  free(st);
}

static void step_capsule_free(PyObject* cap) {
  step_free((Step*)PyCapsule_GetPointer(cap, "mentat_amd._host_plan.step"));
}

static uint32_t hash_slot(int32_t v, long cap) { return ((uint32_t)v * 2654435761u) & (uint32_t)(cap - 1); }

/* Groups of the layer-0 tails (ids >= -1), numbered by first appearance. */
static int group_tails(Step* st) {
  const Py_ssize_t n = st->n;
  int32_t* first = (int32_t*)malloc((size_t)st->hcap * sizeof(int32_t)); /* batch index + 1 of a tail's first holder */
  if (!first) {
    PyErr_NoMemory();
    return -1;
  }
  memset(st->hash, 0, (size_t)st->hcap * sizeof(int32_t));
  long ng = 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const int32_t v = st->tails0[i] + 2; /* >= 1; 0 marks an empty slot */
    uint32_t h = hash_slot(v, st->hcap);
    while (st->hash[h] != 0 && st->hash[h] != v) h = (h + 1) & (uint32_t)(st->hcap - 1);
    if (st->hash[h] == 0) {
      st->hash[h] = v;
      first[h] = (int32_t)ng++;
    }
    st->group[i] = first[h];
  }
  st->ngroups0 = ng;
  free(first);
  return 0;
}

/* tl induces layer 0's partition: one block per group, distinct across groups
 * (len(set(tl)) == len(set(tails0)) == len(set(zip(tails0, tl)))). */
static int same_partition(Step* st, const int32_t* tl) {
  const long ng = st->ngroups0;
  for (long g = 0; g < ng; ++g) st->rep[g] = INT32_MIN;
  for (Py_ssize_t i = 0; i < st->n; ++i) {
    int32_t* r = st->rep + st->group[i];
    if (*r == INT32_MIN)
      *r = tl[i];
    else if (*r != tl[i])
      return 0;
  }
  memset(st->hash, 0, (size_t)st->hcap * sizeof(int32_t));
  for (long g = 0; g < ng; ++g) {
    const int32_t v = st->rep[g] + 2;
    uint32_t h = hash_slot(v, st->hcap);
    while (st->hash[h] != 0) {
      if (st->hash[h] == v) return 0;
      h = (h + 1) & (uint32_t)(st->hcap - 1);
    }
    st->hash[h] = v;
  }
  return 1;
}

/* Layers l0 .. upto - 1 of the step (plan: int32 [num_layers][7][n]). */
static int replay_layers(Step* st, Py_ssize_t l0, Py_ssize_t upto, long B, Alloc* a, int32_t* plan) {
  Seq* s = st->s;
  const Py_ssize_t n = st->n;
  int32_t* tl = (int32_t*)malloc((n > 0 ? (size_t)n : 1) * sizeof(int32_t));
  if (!tl) {
    PyErr_NoMemory();
    return -1;
  }
  const int32_t* p0 = plan;
  int rc = 0;
  for (Py_ssize_t l = l0; l < upto && rc == 0; ++l) {
    int32_t* pl = plan + l * 7 * n;
    int ok = st->uniform;
    for (Py_ssize_t i = 0; ok && i < n; ++i) {
      PyObject* table = PyList_GET_ITEM(s[i].pt, l);
      const Py_ssize_t m = PyList_GET_SIZE(table);
      if (m == 0) {
        if (st->paged) {
          ok = 0; /* an empty table where layer 0 has pages */
          break;
        }
        tl[i] = -1;
      } else {
        const long t = lget(table, m - 1);
        if (t < 0 || t >= a->n) {
          PyErr_Format(PyExc_IndexError, "block id %ld outside the pool", t);
          rc = -1;
          break;
        }
        tl[i] = (int32_t)t;
      }
      long r = 0;
      if (tl[i] >= 0 && rc_get(a, tl[i], &r) < 0) {
        rc = -1;
        break;
      }
      ok = r == st->rc0[i];
    }
    if (rc) break;
    if (ok && st->shared0) ok = same_partition(st, tl);
    if (!ok) {
      rc = plan_layer(s, n, l, B, a, pl);
      continue;
    }
    memcpy(pl + n, p0 + n, (size_t)(6 * n) * sizeof(int32_t));
    for (Py_ssize_t i = 0; i < n; ++i) pl[2 * n + i] = -1;
    for (Py_ssize_t e = 0; e < st->n_events && rc == 0; ++e) {
      const Py_ssize_t i = st->ev[2 * e];
      PyObject* table = PyList_GET_ITEM(s[i].pt, l);
      long b;
      if (st->ev[2 * e + 1] == 0) {
        if (alloc_one(a, &b) < 0) { rc = -1; break; }
        PyObject* o = PyLong_FromLong(b);
        if (!o) { rc = -1; break; }
        const int r = PyList_Append(table, o);
        Py_DECREF(o);
        if (r < 0) { rc = -1; break; }
      } else {
        const Py_ssize_t last = PyList_GET_SIZE(table) - 1;
        const long old = lget(table, last);
        if (alloc_one(a, &b) < 0 || release_one(a, old) < 0 || list_set(table, last, b) < 0) { rc = -1; break; }
        pl[2 * n + i] = (int32_t)old;
      }
      tl[i] = (int32_t)b;
    }
    if (rc) break;
    memcpy(pl, tl, (size_t)n * sizeof(int32_t));
    /* layer 0's counters are the step's counters of a replayed layer */
    for (Py_ssize_t i = 0; i < n; ++i) {
      copy_first(s[i].tilb, l);
      copy_first(s[i].nt, l);
    }
  }
  free(tl);
  return rc;
}

static PyObject* py_step_begin(PyObject* self, PyObject* args) {
  PyObject *seqs, *alloc_obj, *plan_obj;
  Py_ssize_t L;
  long B;
  if (!PyArg_ParseTuple(args, "OnlOO", &seqs, &L, &B, &alloc_obj, &plan_obj)) return NULL;
  if (L < 1) {
    PyErr_SetString(PyExc_ValueError, "step_begin: bad layer counts");
    return NULL;
  }
  Step* st = (Step*)calloc(1, sizeof(Step));
  if (!st) return PyErr_NoMemory();
  int ok = seqs_open(seqs, L, &st->s, &st->n);
  if (ok <= 0) {
    step_free(st);
    return ok < 0 ? NULL : Py_NewRef(Py_None);
  }
  Alloc a;
  ok = alloc_open(&a, alloc_obj);
  if (ok <= 0) {
    step_free(st);
    return ok < 0 ? NULL : Py_NewRef(Py_None);
  }
  const Py_ssize_t n = st->n;
  Seq* s = st->s;
  Py_buffer view;
  if (!get_i32(plan_obj, &view, L * 7 * n)) {
    alloc_close(&a);
    step_free(st);
    Py_RETURN_NONE;
  }
  int32_t* plan = (int32_t*)view.buf;
  const size_t nn = n > 0 ? (size_t)n : 1;
  st->hcap = 16;
  while (st->hcap < 2 * (long)nn) st->hcap *= 2;
  Py_ssize_t* before = (Py_ssize_t*)malloc(nn * sizeof(Py_ssize_t)); /* layer 0's pages before the step */
  PyObject* cap = NULL;
  int rc = -1, uniform = 0;
  if (!before || !(st->tails0 = (int32_t*)malloc(nn * 4)) || !(st->rc0 = (int32_t*)malloc(nn * 4)) ||
      !(st->group = (int32_t*)malloc(nn * 4)) || !(st->rep = (int32_t*)malloc(nn * 4)) ||
      !(st->ev = (int32_t*)malloc(nn * 16)) || !(st->hash = (int32_t*)malloc((size_t)st->hcap * 4))) {
    PyErr_NoMemory();
    goto done;
  }
  /* every layer's counters equal layer 0's (before the step) */
  st->uniform = 1;
  for (Py_ssize_t i = 0; i < n && st->uniform; ++i) {
    for (Py_ssize_t l = 1; l < L; ++l)
      if (!equal_first(s[i].tilb, l) || !equal_first(s[i].nt, l)) {
        st->uniform = 0;
        break;
      }
  }
  st->paged = 1;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* t0 = PyList_GET_ITEM(s[i].pt, 0);
    const Py_ssize_t m = PyList_GET_SIZE(t0);
    long tail = -1, r = 0;
    if (m > 0) {
      tail = lget(t0, m - 1);
      if (rc_get(&a, tail, &r) < 0) goto done;
    } else {
      st->paged = 0;
    }
    st->tails0[i] = (int32_t)tail;
    st->rc0[i] = (int32_t)r;
    st->shared0 |= r > 1;
    before[i] = m;
  }
  if (group_tails(st) < 0) goto done;
  if (plan_layer(s, n, 0, B, &a, plan) < 0) goto done;
  /* layer 0's events in batch order: a new tail page, then a copy-on-write */
  for (Py_ssize_t i = 0; i < n; ++i) {
    if (PyList_GET_SIZE(PyList_GET_ITEM(s[i].pt, 0)) > before[i]) {
      st->ev[2 * st->n_events] = (int32_t)i;
      st->ev[2 * st->n_events + 1] = 0;
      ++st->n_events;
    }
    if (plan[2 * n + i] >= 0) {
      st->ev[2 * st->n_events] = (int32_t)i;
      st->ev[2 * st->n_events + 1] = 1;
      ++st->n_events;
    }
  }
  uniform = st->uniform;
  cap = PyCapsule_New(st, "mentat_amd._host_plan.step", step_capsule_free);
  if (!cap) goto done;
  st = NULL;
  rc = 0;
done:
  free(before);
  step_free(st);
  PyBuffer_Release(&view);
  if (alloc_finish(&a) < 0) rc = -1;
  if (rc < 0) {
    Py_XDECREF(cap);
    return NULL;
  }
  return Py_BuildValue("(NO)", cap, uniform ? Py_True : Py_False); /* (state, uniform) */
}

static PyObject* py_step_layers(PyObject* self, PyObject* args) {
  PyObject *cap, *alloc_obj, *plan_obj;
  Py_ssize_t l0, upto, L;
  long B;
  if (!PyArg_ParseTuple(args, "OnnnlOO", &cap, &l0, &upto, &L, &B, &alloc_obj, &plan_obj)) return NULL;
  Step* st = (Step*)PyCapsule_GetPointer(cap, "mentat_amd._host_plan.step");
  if (!st) return NULL;
  if (l0 < 1 || upto > L || l0 > upto) {
    PyErr_SetString(PyExc_ValueError, "step_layers: bad layer range");
    return NULL;
  }
  if (l0 == upto) Py_RETURN_TRUE;
  Alloc a;
  int ok = alloc_open(&a, alloc_obj);
  if (ok <= 0) {
    if (ok == 0) PyErr_SetString(PyExc_RuntimeError, "step_layers: the allocator changed since step_begin");
    return NULL;
  }
  Py_buffer view;
  if (!get_i32(plan_obj, &view, L * 7 * st->n)) {
    alloc_close(&a);
    PyErr_SetString(PyExc_ValueError, "step_layers: plan must be a writable int32 [num_layers, 7, N] array");
    return NULL;
  }
  int rc = replay_layers(st, l0, upto, B, &a, (int32_t*)view.buf);
  PyBuffer_Release(&view);
  if (alloc_finish(&a) < 0) rc = -1;
  if (rc < 0) return NULL;
  Py_RETURN_TRUE;
}

static PyMethodDef methods[] = {
    {"append_batched", py_append_batched, METH_VARARGS, "plan_append_batched into a [7, N] int32 buffer"},
    {"step_begin", py_step_begin, METH_VARARGS, "layer 0 of a step; returns (state, uniform) or None"},
    {"step_layers", py_step_layers, METH_VARARGS, "the later layers of a step begun by step_begin"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_host_plan", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__host_plan(void) {
  if (!(s_page_table = PyUnicode_InternFromString("page_table")) ||
      !(s_tilb = PyUnicode_InternFromString("tokens_in_last_block")) ||
      !(s_num_tokens = PyUnicode_InternFromString("num_tokens")) || !(s_row = PyUnicode_InternFromString("row")) ||
      !(s_free = PyUnicode_InternFromString("_free")) || !(s_refcounts = PyUnicode_InternFromString("refcounts")) ||
      !(s_peak = PyUnicode_InternFromString("_peak_used")) || !(s_alloc = PyUnicode_InternFromString("alloc")))
    return NULL;
  return PyModule_Create(&module);
}
