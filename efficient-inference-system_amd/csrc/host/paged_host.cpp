// Native host bookkeeping of a cached HIP-graph step (src/model/graph_decode.py), for the Python
// cache objects of src/cache/paged_kv.py (the reference's API: BatchedPagedKVCache with .pool and
// .states, PagedKVCacheState with .pool, .block_ids and .seq_len, LayerBlockPool with
// .free_block_ids, .k_blocks, .capacity_blocks, .block_size, allocate_block() and
// ensure_initialized()). Each function does exactly what its Python counterpart does, with the
// same checks and errors; only the interpreter overhead of walking every layer's and request's
// objects is gone (about 35 us per decode step of 8 requests x 6 layers in Python).
//
//   lockstep(kv_caches, max_new_blocks) -> bool        graph_decode._lockstep
//   host_append(kv_caches, app, num_heads, head_dim, dtype, device) -> list[int]
//                                                       BatchedPagedKVCache.host_append on every
//                                                       cache; returns the first cache's lengths
//                                                       before the append
//   csr(states, prev, app) -> (bytearray, max_pages)    BatchedPagedKVCache.csr_buffer: int32
//                                                       [offsets B+1 | prev B | app B | block ids]
//   check_tokens(ids, positions, T, vocab, max_pos)     TinyTransformerLM.check_token_inputs for
//                                                       host data: IndexError where the eager
//                                                       embedding lookups would raise
//   max_blocks(states) -> int                           the longest block list of a batch
//   step_metadata(states, rows, prev, app, cur, sel, shadow, shadow_len, desc, layout)
//                                              -> (updates, max_pages)
//                                                       graph_decode._step_metadata_py: the int32
//                                                       part of a step's descriptor for the device
//                                                       block-table mirror (only what changed)
//
// Blocks are allocated through the pool's own allocate_block() (LIFO order, growth and its
// mutation counter unchanged), which a step calls only when a request crosses a block boundary.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <climits>
#include <cstdint>
#include <cstring>
#include <initializer_list>

namespace {

// Owned reference, released at scope exit.
class Ref {
 public:
  explicit Ref(PyObject* o = nullptr) : o_(o) {}
  ~Ref() { Py_XDECREF(o_); }
  Ref(const Ref&) = delete;
  Ref& operator=(const Ref&) = delete;
  PyObject* get() const { return o_; }
  explicit operator bool() const { return o_ != nullptr; }

 private:
  PyObject* o_;
};

struct Names {
  PyObject *pool, *states, *seq_len, *block_ids, *k_blocks, *free_block_ids, *capacity_blocks, *block_size,
      *allocate_block, *ensure_initialized;
};
Names N;

bool init_names() {
  N.pool = PyUnicode_InternFromString("pool");
  N.states = PyUnicode_InternFromString("states");
  N.seq_len = PyUnicode_InternFromString("seq_len");
  N.block_ids = PyUnicode_InternFromString("block_ids");
  N.k_blocks = PyUnicode_InternFromString("k_blocks");
  N.free_block_ids = PyUnicode_InternFromString("free_block_ids");
  N.capacity_blocks = PyUnicode_InternFromString("capacity_blocks");
  N.block_size = PyUnicode_InternFromString("block_size");
  N.allocate_block = PyUnicode_InternFromString("allocate_block");
  N.ensure_initialized = PyUnicode_InternFromString("ensure_initialized");
  return N.pool && N.states && N.seq_len && N.block_ids && N.k_blocks && N.free_block_ids && N.capacity_blocks &&
         N.block_size && N.allocate_block && N.ensure_initialized;
}

// A list attribute (the cache objects keep plain lists); error if it is something else.
PyObject* list_attr(PyObject* o, PyObject* name) {
  PyObject* v = PyObject_GetAttr(o, name);
  if (v != nullptr && !PyList_Check(v)) {
    PyErr_Format(PyExc_TypeError, "%U must be a list", name);
    Py_DECREF(v);
    return nullptr;
  }
  return v;
}

// An attribute as a fast sequence (list or tuple; other iterables are materialised).
PyObject* seq_attr(PyObject* o, PyObject* name) {
  Ref v(PyObject_GetAttr(o, name));
  if (!v) return nullptr;
  return PySequence_Fast(v.get(), "expected a sequence");
}

bool long_attr(PyObject* o, PyObject* name, long long* out) {
  Ref v(PyObject_GetAttr(o, name));
  if (!v) return false;
  *out = PyLong_AsLongLong(v.get());
  return !(*out == -1 && PyErr_Occurred());
}

// 1 if a != b (Python !=), 0 if equal, -1 on error.
int differs(PyObject* a, PyObject* b) { return PyObject_RichCompareBool(a, b, Py_NE); }

PyObject* lockstep(PyObject*, PyObject* args) {
  PyObject* caches_in;
  Py_ssize_t max_new_blocks;
  if (!PyArg_ParseTuple(args, "On", &caches_in, &max_new_blocks)) return nullptr;
  Ref caches(PySequence_Fast(caches_in, "kv_caches must be a sequence"));
  if (!caches) return nullptr;
  const Py_ssize_t L = PySequence_Fast_GET_SIZE(caches.get());
  if (L == 0) {
    PyErr_SetString(PyExc_IndexError, "no caches");
    return nullptr;
  }
  PyObject** cs = PySequence_Fast_ITEMS(caches.get());
  Ref p0(PyObject_GetAttr(cs[0], N.pool));
  if (!p0) return nullptr;
  Ref k0(PyObject_GetAttr(p0.get(), N.k_blocks));
  if (!k0) return nullptr;
  if (k0.get() == Py_None) Py_RETURN_FALSE;
  Ref f0(list_attr(p0.get(), N.free_block_ids));
  if (!f0) return nullptr;
  const Py_ssize_t n0 = PyList_GET_SIZE(f0.get());
  const Py_ssize_t tail0 = max_new_blocks < n0 ? n0 - max_new_blocks : 0;  // first compared free id
  Ref cap0(PyObject_GetAttr(p0.get(), N.capacity_blocks));
  if (!cap0) return nullptr;
  Ref st0(seq_attr(cs[0], N.states));
  if (!st0) return nullptr;
  const Py_ssize_t ns = PySequence_Fast_GET_SIZE(st0.get());
  for (Py_ssize_t i = 1; i < L; ++i) {
    Ref p(PyObject_GetAttr(cs[i], N.pool));
    if (!p) return nullptr;
    Ref k(PyObject_GetAttr(p.get(), N.k_blocks));
    if (!k) return nullptr;
    if (k.get() == Py_None) Py_RETURN_FALSE;
    Ref cap(PyObject_GetAttr(p.get(), N.capacity_blocks));
    if (!cap) return nullptr;
    int d = differs(cap.get(), cap0.get());
    if (d < 0) return nullptr;
    if (d) Py_RETURN_FALSE;
    Ref f(list_attr(p.get(), N.free_block_ids));
    if (!f) return nullptr;
    if (PyList_GET_SIZE(f.get()) != n0) Py_RETURN_FALSE;
    for (Py_ssize_t j = tail0; j < n0; ++j) {
      d = differs(PyList_GET_ITEM(f.get(), j), PyList_GET_ITEM(f0.get(), j));
      if (d < 0) return nullptr;
      if (d) Py_RETURN_FALSE;
    }
    Ref st(seq_attr(cs[i], N.states));
    if (!st) return nullptr;
    if (PySequence_Fast_GET_SIZE(st.get()) != ns) Py_RETURN_FALSE;
    for (Py_ssize_t j = 0; j < ns; ++j) {
      PyObject* a = PySequence_Fast_GET_ITEM(st.get(), j);
      PyObject* b = PySequence_Fast_GET_ITEM(st0.get(), j);
      Ref la(PyObject_GetAttr(a, N.seq_len)), lb(PyObject_GetAttr(b, N.seq_len));
      if (!la || !lb) return nullptr;
      d = differs(la.get(), lb.get());
      if (d < 0) return nullptr;
      if (d) Py_RETURN_FALSE;
      Ref ba(PyObject_GetAttr(a, N.block_ids)), bb(PyObject_GetAttr(b, N.block_ids));
      if (!ba || !bb) return nullptr;
      d = differs(ba.get(), bb.get());
      if (d < 0) return nullptr;
      if (d) Py_RETURN_FALSE;
    }
  }
  Py_RETURN_TRUE;
}

PyObject* host_append(PyObject*, PyObject* args) {
  PyObject *caches_in, *app_in, *heads, *head_dim, *dtype, *device;
  if (!PyArg_ParseTuple(args, "OOOOOO", &caches_in, &app_in, &heads, &head_dim, &dtype, &device)) return nullptr;
  Ref caches(PySequence_Fast(caches_in, "kv_caches must be a sequence"));
  if (!caches) return nullptr;
  Ref app(PySequence_Fast(app_in, "app must be a sequence"));
  if (!app) return nullptr;
  const Py_ssize_t na = PySequence_Fast_GET_SIZE(app.get());
  long long* n = static_cast<long long*>(PyMem_Malloc(sizeof(long long) * (na > 0 ? na : 1)));
  if (n == nullptr) return PyErr_NoMemory();
  bool any = false;
  for (Py_ssize_t b = 0; b < na; ++b) {
    n[b] = PyLong_AsLongLong(PySequence_Fast_GET_ITEM(app.get(), b));
    if (n[b] == -1 && PyErr_Occurred()) {
      PyMem_Free(n);
      return nullptr;
    }
    any = any || n[b] != 0;
  }
  PyObject* first_prev = nullptr;  // owned once set
  const Py_ssize_t L = PySequence_Fast_GET_SIZE(caches.get());
  PyObject** cs = PySequence_Fast_ITEMS(caches.get());
  bool ok = true;
  for (Py_ssize_t i = 0; i < L && ok; ++i) {
    ok = false;
    Ref pool(PyObject_GetAttr(cs[i], N.pool));
    if (!pool) break;
    long long bs;
    if (!long_attr(pool.get(), N.block_size, &bs)) break;
    if (bs <= 0) {
      PyErr_SetString(PyExc_ValueError, "block_size must be positive");
      break;
    }
    if (any) {
      Ref k(PyObject_GetAttr(pool.get(), N.k_blocks));
      if (!k) break;
      if (k.get() == Py_None) {
        Ref r(PyObject_CallMethodObjArgs(pool.get(), N.ensure_initialized, heads, head_dim, dtype, device, nullptr));
        if (!r) break;
      }
    }
    Ref states(seq_attr(cs[i], N.states));
    if (!states) break;
    const Py_ssize_t ns = PySequence_Fast_GET_SIZE(states.get());
    const Py_ssize_t nb = ns < na ? ns : na;  // zip()
    Ref prev(PyList_New(nb));
    if (!prev) break;
    bool inner = true;
    for (Py_ssize_t b = 0; b < nb && inner; ++b) {
      inner = false;
      PyObject* st = PySequence_Fast_GET_ITEM(states.get(), b);
      PyObject* pl = PyObject_GetAttr(st, N.seq_len);
      if (pl == nullptr) break;
      PyList_SET_ITEM(prev.get(), b, pl);  // steals the reference
      const long long p = PyLong_AsLongLong(pl);
      if (p == -1 && PyErr_Occurred()) break;
      if (n[b] <= 0) {
        inner = true;
        continue;
      }
      Ref sp(PyObject_GetAttr(st, N.pool));
      if (!sp) break;
      if (sp.get() != pool.get()) {
        PyErr_SetString(PyExc_ValueError, "all states of a BatchedPagedKVCache must share its pool");
        break;
      }
      Ref ids(list_attr(st, N.block_ids));
      if (!ids) break;
      const long long have = PyList_GET_SIZE(ids.get());
      const long long need_now = (p + bs - 1) / bs;  // Python floor division; p >= 0 here
      if (have != need_now) {
        PyErr_Format(PyExc_ValueError, "block_ids (%lld blocks) does not match seq_len %lld at block size %lld", have,
                     p, bs);
        break;
      }
      const long long want = (p + n[b] + bs - 1) / bs;
      bool alloc_ok = true;
      for (long long k = have; k < want; ++k) {
        Ref blk(PyObject_CallMethodNoArgs(pool.get(), N.allocate_block));
        if (!blk || PyList_Append(ids.get(), blk.get()) < 0) {
          alloc_ok = false;
          break;
        }
      }
      if (!alloc_ok) break;
      Ref nl(PyLong_FromLongLong(p + n[b]));
      if (!nl || PyObject_SetAttr(st, N.seq_len, nl.get()) < 0) break;
      inner = true;
    }
    if (!inner) break;
    if (i == 0) {
      first_prev = prev.get();
      Py_INCREF(first_prev);
    }
    ok = true;
  }
  PyMem_Free(n);
  if (!ok) {
    Py_XDECREF(first_prev);
    return nullptr;
  }
  if (first_prev == nullptr) return PyList_New(0);
  return first_prev;
}

bool as_i32(PyObject* o, int32_t* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return false;
  if (v < INT32_MIN || v > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "value out of int32 range");
    return false;
  }
  *out = static_cast<int32_t>(v);
  return true;
}

PyObject* csr(PyObject*, PyObject* args) {
  PyObject *states_in, *prev_in, *app_in;
  if (!PyArg_ParseTuple(args, "OOO", &states_in, &prev_in, &app_in)) return nullptr;
  Ref states(PySequence_Fast(states_in, "states must be a sequence"));
  Ref prev(PySequence_Fast(prev_in, "prev must be a sequence"));
  Ref app(PySequence_Fast(app_in, "app must be a sequence"));
  if (!states || !prev || !app) return nullptr;
  const Py_ssize_t B = PySequence_Fast_GET_SIZE(states.get());
  if (PySequence_Fast_GET_SIZE(prev.get()) != B || PySequence_Fast_GET_SIZE(app.get()) != B) {
    PyErr_SetString(PyExc_ValueError, "prev and app need one entry per state");
    return nullptr;
  }
  // block lists (borrowed through the owned tuple below)
  Ref lists(PyTuple_New(B));
  if (!lists) return nullptr;
  Py_ssize_t total = 0, max_pages = 0;
  for (Py_ssize_t b = 0; b < B; ++b) {
    PyObject* ids = list_attr(PySequence_Fast_GET_ITEM(states.get(), b), N.block_ids);
    if (ids == nullptr) return nullptr;
    PyTuple_SET_ITEM(lists.get(), b, ids);  // steals
    const Py_ssize_t c = PyList_GET_SIZE(ids);
    total += c;
    max_pages = c > max_pages ? c : max_pages;
  }
  const Py_ssize_t words = 3 * B + 1 + total;
  Ref buf(PyByteArray_FromStringAndSize(nullptr, words * (Py_ssize_t)sizeof(int32_t)));
  if (!buf) return nullptr;
  int32_t* w = reinterpret_cast<int32_t*>(PyByteArray_AS_STRING(buf.get()));
  w[0] = 0;
  Py_ssize_t pos = 3 * B + 1, off = 0;
  for (Py_ssize_t b = 0; b < B; ++b) {
    PyObject* ids = PyTuple_GET_ITEM(lists.get(), b);
    const Py_ssize_t c = PyList_GET_SIZE(ids);
    off += c;
    if (off > INT32_MAX) {
      PyErr_SetString(PyExc_OverflowError, "value out of int32 range");
      return nullptr;
    }
    w[1 + b] = static_cast<int32_t>(off);
    if (!as_i32(PySequence_Fast_GET_ITEM(prev.get(), b), &w[B + 1 + b])) return nullptr;
    if (!as_i32(PySequence_Fast_GET_ITEM(app.get(), b), &w[2 * B + 1 + b])) return nullptr;
    for (Py_ssize_t j = 0; j < c; ++j)
      if (!as_i32(PyList_GET_ITEM(ids, j), &w[pos + j])) return nullptr;
    pos += c;
  }
  return Py_BuildValue("(On)", buf.get(), max_pages);
}

// Writable C-contiguous buffer of int32 words, released at scope exit.
class Words {
 public:
  ~Words() {
    if (ok_) PyBuffer_Release(&v_);
  }
  bool get(PyObject* o, const char* what) {
    if (PyObject_GetBuffer(o, &v_, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS) < 0) return false;
    ok_ = true;
    if (v_.itemsize != 4) {
      PyErr_Format(PyExc_TypeError, "%s must hold 4-byte words", what);
      return false;
    }
    return true;
  }
  int32_t* data() const { return static_cast<int32_t*>(v_.buf); }
  Py_ssize_t size() const { return v_.len / 4; }

 private:
  Py_buffer v_{};
  bool ok_ = false;
};

bool seq_i32(PyObject* seq, Py_ssize_t i, int32_t* out) { return as_i32(PySequence_Fast_GET_ITEM(seq, i), out); }

PyObject* step_metadata(PyObject*, PyObject* args) {
  PyObject *states_in, *rows_in, *prev_in, *app_in, *cur_in, *sel_in, *shadow_in, *shadow_len_in, *desc_in;
  Py_ssize_t o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, stride;
  if (!PyArg_ParseTuple(args, "OOOOOOOOO(nnnnnnnnn)", &states_in, &rows_in, &prev_in, &app_in, &cur_in, &sel_in,
                        &shadow_in, &shadow_len_in, &desc_in, &o_cur, &o_sel, &o_mrow, &o_first, &o_npages,
                        &o_prev, &o_app, &o_upd, &stride))
    return nullptr;
  Ref states(PySequence_Fast(states_in, "states must be a sequence"));
  Ref rows(PySequence_Fast(rows_in, "rows must be a sequence"));
  Ref prev(PySequence_Fast(prev_in, "prev must be a sequence"));
  Ref app(PySequence_Fast(app_in, "app must be a sequence"));
  Ref cur(PySequence_Fast(cur_in, "cur must be a sequence"));
  Ref sel(PySequence_Fast(sel_in, "sel must be a sequence"));
  if (!states || !rows || !prev || !app || !cur || !sel) return nullptr;
  const Py_ssize_t B = PySequence_Fast_GET_SIZE(states.get());
  if (PySequence_Fast_GET_SIZE(rows.get()) != B || PySequence_Fast_GET_SIZE(prev.get()) != B ||
      PySequence_Fast_GET_SIZE(app.get()) != B || PySequence_Fast_GET_SIZE(cur.get()) != B ||
      PySequence_Fast_GET_SIZE(sel.get()) != B) {
    PyErr_SetString(PyExc_ValueError, "rows, prev, app, cur and sel need one entry per state");
    return nullptr;
  }
  Words shadow, shadow_len, desc;
  if (!shadow.get(shadow_in, "shadow") || !shadow_len.get(shadow_len_in, "shadow_len") || !desc.get(desc_in, "desc"))
    return nullptr;
  const Py_ssize_t R = shadow_len.size();
  if (R <= 0 || shadow.size() % R != 0) {
    PyErr_SetString(PyExc_ValueError, "shadow must be [rows, width] with one length per row");
    return nullptr;
  }
  const Py_ssize_t W = shadow.size() / R;
  const Py_ssize_t n_desc = desc.size();
  for (Py_ssize_t o : {o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app}) {
    if (o < 0 || o + B > n_desc) {
      PyErr_SetString(PyExc_ValueError, "descriptor layout outside the buffer");
      return nullptr;
    }
  }
  if (o_upd < 0 || stride < 0 || o_upd + B * stride > n_desc) {
    PyErr_SetString(PyExc_ValueError, "descriptor layout outside the buffer");
    return nullptr;
  }
  int32_t* d = desc.data();
  int32_t* sh = shadow.data();
  int32_t* shl = shadow_len.data();
  Py_ssize_t n_upd = 0, max_pages = 0;
  for (Py_ssize_t b = 0; b < B; ++b) {
    int32_t row;
    if (!seq_i32(rows.get(), b, &row)) return nullptr;
    if (row < 0 || row >= R) {
      PyErr_Format(PyExc_ValueError, "mirror row %d outside [0, %zd)", row, R);
      return nullptr;
    }
    if (!seq_i32(prev.get(), b, &d[o_prev + b]) || !seq_i32(app.get(), b, &d[o_app + b]) ||
        !seq_i32(cur.get(), b, &d[o_cur + b]) || !seq_i32(sel.get(), b, &d[o_sel + b]))
      return nullptr;
    d[o_mrow + b] = row;
    Ref ids(list_attr(PySequence_Fast_GET_ITEM(states.get(), b), N.block_ids));
    if (!ids) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(ids.get());
    if (n > W) {
      PyErr_Format(PyExc_ValueError, "a request holds %zd blocks, more than the mirror width %zd", n, W);
      return nullptr;
    }
    max_pages = n > max_pages ? n : max_pages;
    int32_t* srow = sh + (Py_ssize_t)row * W;
    const Py_ssize_t known = shl[row] < 0 ? 0 : (shl[row] < n ? shl[row] : n);
    // first entry that differs from what the row holds; everything from there on is resent
    Py_ssize_t f = 0;
    for (; f < known; ++f) {
      int32_t v;
      if (!as_i32(PyList_GET_ITEM(ids.get(), f), &v)) return nullptr;
      if (v != srow[f]) break;
    }
    if (n - f > stride) {
      PyErr_SetString(PyExc_ValueError, "descriptor update area too small");
      return nullptr;
    }
    int32_t* upd = d + o_upd + b * stride;
    for (Py_ssize_t j = f; j < n; ++j) {
      int32_t v;
      if (!as_i32(PyList_GET_ITEM(ids.get(), j), &v)) return nullptr;
      srow[j] = v;
      upd[j - f] = v;
    }
    n_upd += n - f;
    shl[row] = (int32_t)n;
    d[o_first + b] = (int32_t)f;
    d[o_npages + b] = (int32_t)n;
  }
  return Py_BuildValue("(nn)", n_upd, max_pages);
}

// Smallest and largest value of an int64 host array (buffer of 8-byte items) or of a (nested)
// sequence of ints; count 0 leaves lo/hi untouched.
bool int_range(PyObject* o, long long* lo, long long* hi, Py_ssize_t* count) {
  if (PyLong_Check(o)) {
    const long long v = PyLong_AsLongLong(o);
    if (v == -1 && PyErr_Occurred()) return false;
    *lo = *count ? (v < *lo ? v : *lo) : v;
    *hi = *count ? (v > *hi ? v : *hi) : v;
    ++*count;
    return true;
  }
  if (PyObject_CheckBuffer(o)) {
    Py_buffer v;
    if (PyObject_GetBuffer(o, &v, PyBUF_C_CONTIGUOUS | PyBUF_FORMAT) < 0) return false;
    const bool i64 = v.itemsize == 8 && v.format != nullptr && (v.format[0] == 'q' || v.format[0] == 'l' ||
                                                                 ((v.format[0] == '<' || v.format[0] == '=') &&
                                                                  (v.format[1] == 'q' || v.format[1] == 'l')));
    if (!i64) {
      PyBuffer_Release(&v);
      PyErr_SetString(PyExc_TypeError, "token ids and positions must be int64 arrays or ints");
      return false;
    }
    const long long* d = static_cast<const long long*>(v.buf);
    const Py_ssize_t n = v.len / 8;
    for (Py_ssize_t i = 0; i < n; ++i) {
      *lo = *count ? (d[i] < *lo ? d[i] : *lo) : d[i];
      *hi = *count ? (d[i] > *hi ? d[i] : *hi) : d[i];
      ++*count;
    }
    PyBuffer_Release(&v);
    return true;
  }
  Ref seq(PySequence_Fast(o, "token ids and positions must be int64 arrays, sequences or ints"));
  if (!seq) return false;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq.get());
  for (Py_ssize_t i = 0; i < n; ++i)
    if (!int_range(PySequence_Fast_GET_ITEM(seq.get(), i), lo, hi, count)) return false;
  return true;
}

PyObject* check_tokens(PyObject*, PyObject* args) {
  PyObject *ids, *pos;
  long long T, V, P;
  if (!PyArg_ParseTuple(args, "OOLLL", &ids, &pos, &T, &V, &P)) return nullptr;
  long long lo = 0, hi = 0, plo = 0, phi = 0;
  Py_ssize_t n = 0, np_ = 0;
  if (!int_range(ids, &lo, &hi, &n) || !int_range(pos, &plo, &phi, &np_)) return nullptr;
  if (n && (lo < 0 || hi >= V)) {
    PyErr_Format(PyExc_IndexError, "token id out of range [0, %lld): min %lld, max %lld", V, lo, hi);
    return nullptr;
  }
  if (np_ && T > 0 && (plo < 0 || phi + T - 1 >= P)) {
    PyErr_Format(PyExc_IndexError, "positions %lld..%lld outside the position table [0, %lld)", plo, phi + T - 1, P);
    return nullptr;
  }
  Py_RETURN_NONE;
}

PyObject* max_blocks(PyObject*, PyObject* states_in) {
  Ref states(PySequence_Fast(states_in, "states must be a sequence"));
  if (!states) return nullptr;
  Py_ssize_t best = 0;
  const Py_ssize_t B = PySequence_Fast_GET_SIZE(states.get());
  for (Py_ssize_t b = 0; b < B; ++b) {
    Ref ids(list_attr(PySequence_Fast_GET_ITEM(states.get(), b), N.block_ids));
    if (!ids) return nullptr;
    best = PyList_GET_SIZE(ids.get()) > best ? PyList_GET_SIZE(ids.get()) : best;
  }
  return PyLong_FromSsize_t(best);
}

PyMethodDef methods[] = {
    {"lockstep", lockstep, METH_VARARGS, "Whether every layer's cache holds the same states and free-list tail."},
    {"host_append", host_append, METH_VARARGS, "Per-layer append bookkeeping; returns the first cache's lengths."},
    {"csr", csr, METH_VARARGS, "int32 CSR metadata buffer of a batch's block lists, and its max pages."},
    {"check_tokens", check_tokens, METH_VARARGS, "IndexError for token ids or positions the embeddings do not hold."},
    {"max_blocks", max_blocks, METH_O, "Length of the longest block list of a batch's states."},
    {"step_metadata", step_metadata, METH_VARARGS,
     "int32 part of a graph step's descriptor: block-list updates against the device mirror's shadow."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_paged_host", "Native host bookkeeping of cached graph steps.", -1,
                      methods, nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__paged_host(void) {
  if (!init_names()) return nullptr;
  return PyModule_Create(&module);
}
