/*
 * page_walk.c - CPython extension `helm_amd._page_walk`: the one pass over a
 * layer's page list that perform_streaming_attention makes before it launches
 * anything (helm_amd/runtime/kv_cache.py: walk_pages_py is the same walk in
 * Python, and tests/test_page_walk.py checks that both give the same result).
 *
 * The reference walks its page list in Python to pick what to attend
 * (helm/runtime/kv_cache.py:350-351: pages with used tokens, on the tier their
 * state names); here that walk also sorts the pages into in-place runs, staged
 * chunks and the rest, with the slot arrays the kernels read.  In Python it
 * costs about a microsecond per page, which at a 4K context is as long as the
 * host-link transfer it is meant to overlap; in C it is tens of nanoseconds.
 *
 * classify(pages, gbound, gviews, hbound, hviews, chunk_pages, page_size) ->
 *   (first_active, run_lens, run_meta, chunk_slots, chunk_waits, gpu_rest, cpu_rest)
 * with run_meta and each chunk_slots entry int32 bytes (see PageWalk).
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

static PyObject *s_used, *s_state, *s_device, *s_slot, *s_k, *s_v, *s_cap, *s_ready, *s_type;

typedef struct {
  int32_t* d;
  Py_ssize_t n, cap;
} ibuf;

static int ibuf_push(ibuf* b, long v) {
  if (b->n == b->cap) {
    const Py_ssize_t c = b->cap ? 2 * b->cap : 256;
    int32_t* d = (int32_t*)PyMem_Realloc(b->d, (size_t)c * sizeof(int32_t));
    if (!d) {
      PyErr_NoMemory();
      return -1;
    }
    b->d = d;
    b->cap = c;
  }
  b->d[b->n++] = (int32_t)v;
  return 0;
}

/* Attribute `name` of page `o` (new reference, NULL with an exception set):
   from the instance dict `d` when it holds it (a dataclass page keeps its fields
   there, and no field is shadowed by a data descriptor), else by getattr. */
static PyObject* attr(PyObject* d, PyObject* o, PyObject* name) {
  if (d) {
    PyObject* v = PyDict_GetItemWithError(d, name);
    if (v) {
      Py_INCREF(v);
      return v;
    }
    if (PyErr_Occurred()) return NULL;
  }
  return PyObject_GetAttr(o, name);
}

/* the instance dict of `o` (new reference), or NULL (no exception) when it has none */
static PyObject* inst_dict(PyObject* o) {
  PyObject* d = PyObject_GenericGetDict(o, NULL);
  if (!d) PyErr_Clear();
  else if (!PyDict_Check(d)) {
    Py_DECREF(d);
    d = NULL;
  }
  return d;
}

/* attribute `name` of `o` as a C long; -1 with an exception set on failure */
static int get_long(PyObject* d, PyObject* o, PyObject* name, long* out) {
  PyObject* v = attr(d, o, name);
  if (!v) return -1;
  *out = PyLong_AsLong(v);
  Py_DECREF(v);
  return (*out == -1 && PyErr_Occurred()) ? -1 : 0;
}

/* kv is not None and kv[0] is p.k_tensor and kv[1] is p.v_tensor: 1 / 0, -1 on error */
static int views_match(PyObject* kv, PyObject* d, PyObject* p) {
  if (kv == NULL || kv == Py_None) return 0;
  PyObject* k0 = PySequence_GetItem(kv, 0);
  if (!k0) return -1;
  PyObject* kt = attr(d, p, s_k);
  if (!kt) {
    Py_DECREF(k0);
    return -1;
  }
  const int same_k = k0 == kt;
  Py_DECREF(k0);
  Py_DECREF(kt);
  if (!same_k) return 0;
  PyObject* v1 = PySequence_GetItem(kv, 1);
  if (!v1) return -1;
  PyObject* vt = attr(d, p, s_v);
  if (!vt) {
    Py_DECREF(v1);
    return -1;
  }
  const int same_v = v1 == vt;
  Py_DECREF(v1);
  Py_DECREF(vt);
  return same_v;
}

typedef struct {
  PyObject* chunk_slots;  /* list of int32 bytes */
  PyObject* chunk_waits;  /* list of lists of pages */
  PyObject* waits;        /* the open chunk's pages with an eviction copy in flight */
  ibuf chunk;             /* the open chunk's slots */
  Py_ssize_t closed;
} chunks_t;

static int close_chunk(chunks_t* c) {
  PyObject* b = PyBytes_FromStringAndSize((const char*)c->chunk.d,
                                          c->chunk.n * (Py_ssize_t)sizeof(int32_t));
  if (!b) return -1;
  const int rc = PyList_Append(c->chunk_slots, b);
  Py_DECREF(b);
  if (rc < 0 || PyList_Append(c->chunk_waits, c->waits) < 0) return -1;
  Py_DECREF(c->waits);
  c->waits = PyList_New(0);
  if (!c->waits) return -1;
  c->chunk.n = 0;
  c->closed++;
  return 0;
}

/* close the open run of in-place pages: its slots, then its token count */
static int close_run(ibuf* run, ibuf* meta, PyObject* run_lens, long tokens) {
  for (Py_ssize_t i = 0; i < run->n; ++i)
    if (ibuf_push(meta, run->d[i]) < 0) return -1;
  if (ibuf_push(meta, tokens) < 0) return -1;
  PyObject* len = PyLong_FromSsize_t(run->n);
  if (!len) return -1;
  const int rc = PyList_Append(run_lens, len);
  Py_DECREF(len);
  run->n = 0;
  return rc;
}

static PyObject* classify(PyObject* self, PyObject* args) {
  (void)self;
  PyObject *pages, *gbound, *gviews, *hbound, *hviews;
  int chunk_pages, page_size;
  if (!PyArg_ParseTuple(args, "OO!O!O!O!ii", &pages, &PyDict_Type, &gbound, &PyDict_Type, &gviews,
                        &PyDict_Type, &hbound, &PyDict_Type, &hviews, &chunk_pages, &page_size))
    return NULL;
  if (chunk_pages < 1 || page_size < 1) {
    PyErr_SetString(PyExc_ValueError, "classify: chunk_pages and page_size must be positive");
    return NULL;
  }
  /* a tuple of the pages: the walk holds every page whatever an attribute lookup does */
  PyObject* seq = PySequence_Tuple(pages);
  if (!seq) return NULL;
  const Py_ssize_t n = PyTuple_GET_SIZE(seq);
  PyObject** items = &PyTuple_GET_ITEM(seq, 0);

  PyObject* result = NULL;
  PyObject* run_lens = PyList_New(0);
  PyObject* gpu_rest = PyList_New(0);
  PyObject* cpu_rest = PyList_New(0);
  chunks_t ch = {PyList_New(0), PyList_New(0), PyList_New(0), {NULL, 0, 0}, 0};
  ibuf meta = {NULL, 0, 0}, run = {NULL, 0, 0};
  PyObject* first_active = Py_None;    /* borrowed from the list */
  PyObject* pd = NULL;                 /* the current page's instance dict */
  PyObject* dev_obj[8];                /* devices seen (references held until the end) */
  int dev_cuda[8];
  int n_dev = 0;
  if (!run_lens || !gpu_rest || !cpu_rest || !ch.chunk_slots || !ch.chunk_waits || !ch.waits)
    goto done;

  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* p = items[i];
    Py_XDECREF(pd);
    pd = inst_dict(p);
    long u;
    if (get_long(pd, p, s_used, &u) < 0) goto done;
    if (u <= 0) continue;
    PyObject* state = attr(pd, p, s_state);
    if (!state) goto done;
    const int is_gpu = PyUnicode_Check(state) && PyUnicode_CompareWithASCIIString(state, "GPU") == 0;
    const int is_cpu = !is_gpu && PyUnicode_Check(state) &&
                       PyUnicode_CompareWithASCIIString(state, "CPU") == 0;
    Py_DECREF(state);
    if (!is_gpu && !is_cpu) continue;
    PyObject* dev = attr(pd, p, s_device);
    if (!dev) goto done;
    int cu = -1;
    for (int k = 0; k < n_dev; ++k)
      if (dev_obj[k] == dev) {
        cu = dev_cuda[k];
        break;
      }
    if (cu < 0) {
      PyObject* t = PyObject_GetAttr(dev, s_type);
      if (!t) {
        Py_DECREF(dev);
        goto done;
      }
      cu = PyUnicode_Check(t) && PyUnicode_CompareWithASCIIString(t, "cuda") == 0;
      Py_DECREF(t);
      if (n_dev < 8) {
        Py_INCREF(dev);
        dev_obj[n_dev] = dev;
        dev_cuda[n_dev] = cu;
        ++n_dev;
      }
    }
    Py_DECREF(dev);
    if (cu != is_gpu) continue;   /* a page on the other tier than its state says */
    if (first_active == Py_None) first_active = p;
    PyObject* sl = attr(pd, p, s_slot);
    if (!sl) goto done;
    if (is_gpu) {
      if (ch.chunk.n > 0 && ch.closed < 2 && close_chunk(&ch) < 0) {
        Py_DECREF(sl);
        goto done;
      }
      PyObject* bound = PyDict_GetItemWithError(gbound, sl);
      if (!bound && PyErr_Occurred()) {
        Py_DECREF(sl);
        goto done;
      }
      if (bound == p) {
        PyObject* kv = PyDict_GetItemWithError(gviews, sl);
        if (!kv && PyErr_Occurred()) {
          Py_DECREF(sl);
          goto done;
        }
        Py_XINCREF(kv);
        const int m = views_match(kv, pd, p);
        Py_XDECREF(kv);
        if (m < 0) {
          Py_DECREF(sl);
          goto done;
        }
        if (m) {
          const long slot = PyLong_AsLong(sl);
          Py_DECREF(sl);
          long cap;
          if ((slot == -1 && PyErr_Occurred()) || ibuf_push(&run, slot) < 0 ||
              get_long(pd, p, s_cap, &cap) < 0)
            goto done;
          if (u != cap && close_run(&run, &meta, run_lens, (run.n - 1) * (long)page_size + u) < 0)
            goto done;
          continue;
        }
      }
      Py_DECREF(sl);
      if (PyList_Append(gpu_rest, p) < 0) goto done;
    } else {
      long cap;
      if (get_long(pd, p, s_cap, &cap) < 0) {
        Py_DECREF(sl);
        goto done;
      }
      if (u == cap) {
        PyObject* bound = PyDict_GetItemWithError(hbound, sl);
        if (!bound && PyErr_Occurred()) {
          Py_DECREF(sl);
          goto done;
        }
        if (bound == p) {
          PyObject* kv = PyDict_GetItemWithError(hviews, sl);
          if (!kv && PyErr_Occurred()) {
            Py_DECREF(sl);
            goto done;
          }
          Py_XINCREF(kv);
          const int m = views_match(kv, pd, p);
          Py_XDECREF(kv);
          if (m < 0) {
            Py_DECREF(sl);
            goto done;
          }
          if (m) {
            const long slot = PyLong_AsLong(sl);
            Py_DECREF(sl);
            if ((slot == -1 && PyErr_Occurred()) || ibuf_push(&ch.chunk, slot) < 0) goto done;
            PyObject* ready = attr(pd, p, s_ready);
            if (!ready) goto done;
            const int pending = ready != Py_None;
            Py_DECREF(ready);
            if (pending && PyList_Append(ch.waits, p) < 0) goto done;
            if (ch.chunk.n == chunk_pages && close_chunk(&ch) < 0) goto done;
            continue;
          }
        }
      }
      Py_DECREF(sl);
      if (ch.chunk.n > 0 && ch.closed < 2 && close_chunk(&ch) < 0) goto done;
      if (PyList_Append(cpu_rest, p) < 0) goto done;
    }
  }
  /* every page of an open run is full */
  if (run.n > 0 && close_run(&run, &meta, run_lens, run.n * (long)page_size) < 0) goto done;
  if (ch.chunk.n > 0 && close_chunk(&ch) < 0) goto done;
  {
    PyObject* meta_b = PyBytes_FromStringAndSize((const char*)meta.d, meta.n * (Py_ssize_t)sizeof(int32_t));
    if (!meta_b) goto done;
    result = Py_BuildValue("(OONOOOO)", first_active, run_lens, meta_b, ch.chunk_slots,
                           ch.chunk_waits, gpu_rest, cpu_rest);
  }
done:
  for (int k = 0; k < n_dev; ++k) Py_DECREF(dev_obj[k]);
  Py_XDECREF(pd);
  Py_XDECREF(run_lens);
  Py_XDECREF(gpu_rest);
  Py_XDECREF(cpu_rest);
  Py_XDECREF(ch.chunk_slots);
  Py_XDECREF(ch.chunk_waits);
  Py_XDECREF(ch.waits);
  PyMem_Free(meta.d);
  PyMem_Free(run.d);
  PyMem_Free(ch.chunk.d);
  Py_DECREF(seq);
  return result;
}

static PyMethodDef methods[] = {
    {"classify", classify, METH_VARARGS,
     "classify(pages, gbound, gviews, hbound, hviews, chunk_pages, page_size) -> "
     "(first_active, run_lens, run_meta, chunk_slots, chunk_waits, gpu_rest, cpu_rest)"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_page_walk",
                                    "The page walk of perform_streaming_attention, in C.", -1,
                                    methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__page_walk(void) {
  s_used = PyUnicode_InternFromString("used_tokens");
  s_state = PyUnicode_InternFromString("state");
  s_device = PyUnicode_InternFromString("device");
  s_slot = PyUnicode_InternFromString("slot");
  s_k = PyUnicode_InternFromString("k_tensor");
  s_v = PyUnicode_InternFromString("v_tensor");
  s_cap = PyUnicode_InternFromString("capacity_tokens");
  s_ready = PyUnicode_InternFromString("ready");
  s_type = PyUnicode_InternFromString("type");
  if (!s_used || !s_state || !s_device || !s_slot || !s_k || !s_v || !s_cap || !s_ready || !s_type)
    return NULL;
  return PyModule_Create(&module);
}
