// Native host loop of the GPU batch packer (CPython extension _hostpack).
//
// DeviceBatchPacker.build (auto_infer_amd/packing.py) walks every scheduled
// request of a step: look up its device-table slot, compare its block row
// with what the device table already holds, queue the new block ids / token
// ids / drafts for upload, and append the request's 8-int row descriptor and
// its cu_seqlens_q / seqlens_kv / sample_idx / decode_splice entries.  That
// is the reference's per-request packing loop (auto_infer/worker/
// model_runner.py:126-166) minus everything the packing kernel does on the
// device.  In Python it costs 1-2 us per request; this is the same loop over
// the same Python objects through the CPython API.  The request table's
// state stays in its Python dicts; the rare paths (a request seen for the
// first time, pool growth) call back into the table's Python methods, so the
// two implementations cannot drift apart on them.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <cstdint>

#include <hip/hip_runtime_api.h>

namespace {

struct Ref {            // owned reference
  PyObject* p;
  explicit Ref(PyObject* o = nullptr) : p(o) {}
  ~Ref() { Py_XDECREF(p); }
  Ref(const Ref&) = delete;
  Ref& operator=(const Ref&) = delete;
  PyObject* get() const { return p; }
  PyObject* release() { PyObject* o = p; p = nullptr; return o; }
  explicit operator bool() const { return p != nullptr; }
};

long long as_ll(PyObject* o, bool* err) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) *err = true;
  return v;
}

bool append_ll(PyObject* list, long long v) {
  Ref x(PyLong_FromLongLong(v));
  return x && PyList_Append(list, x.get()) == 0;
}

long long attr_ll(PyObject* o, PyObject* name, bool* err) {
  Ref v(PyObject_GetAttr(o, name));
  if (!v) { *err = true; return 0; }
  return as_ll(v.get(), err);
}

// int attribute of the table that may change when the table grows
bool table_caps(PyObject* table, PyObject* n_blocks, PyObject* n_tokens, long long* cb,
                long long* ct) {
  bool err = false;
  *cb = attr_ll(table, n_blocks, &err);
  *ct = attr_ll(table, n_tokens, &err);
  return !err;
}

PyObject* build_rows(PyObject*, PyObject* args) {
  PyObject *table, *scheduled, *get_request, *tables, *upd, *live;
  long long bs;
  if (!PyArg_ParseTuple(args, "OOOOLOO", &table, &scheduled, &get_request, &tables, &bs, &upd,
                        &live))
    return nullptr;
  // interned attribute names
  static PyObject *s_rid, *s_n, *s_prefill, *s_ncomp, *s_ids, *s_nprompt, *s_draft, *s_slot,
      *s_blocks, *s_ntok, *s_last, *s_step, *s_capb, *s_capt, *s_slot_for, *s_grow, *s_rows,
      *s_ts, *s_ti, *s_tv, *s_bs_, *s_bi, *s_bv, *s_ubr, *s_ube;
  if (!s_rid) {
    s_rid = PyUnicode_InternFromString("request_id");
    s_n = PyUnicode_InternFromString("num_tokens_to_compute");
    s_prefill = PyUnicode_InternFromString("is_prefill");
    s_ncomp = PyUnicode_InternFromString("num_computed_tokens");
    s_ids = PyUnicode_InternFromString("all_token_ids");
    s_nprompt = PyUnicode_InternFromString("num_prompt_tokens");
    s_draft = PyUnicode_InternFromString("spec_draft");
    s_slot = PyUnicode_InternFromString("_slot");
    s_blocks = PyUnicode_InternFromString("_blocks");
    s_ntok = PyUnicode_InternFromString("_ntok");
    s_last = PyUnicode_InternFromString("_last_use");
    s_step = PyUnicode_InternFromString("_step");
    s_capb = PyUnicode_InternFromString("_cap_blocks");
    s_capt = PyUnicode_InternFromString("_cap_tokens");
    s_slot_for = PyUnicode_InternFromString("_slot_for");
    s_grow = PyUnicode_InternFromString("_grow");
    s_rows = PyUnicode_InternFromString("rows");
    s_ts = PyUnicode_InternFromString("tok_slot");
    s_ti = PyUnicode_InternFromString("tok_idx");
    s_tv = PyUnicode_InternFromString("tok_val");
    s_bs_ = PyUnicode_InternFromString("blk_slot");
    s_bi = PyUnicode_InternFromString("blk_idx");
    s_bv = PyUnicode_InternFromString("blk_val");
    s_ubr = PyUnicode_InternFromString("uploaded_block_rows");
    s_ube = PyUnicode_InternFromString("uploaded_block_elements");
  }
  Ref slot_d(PyObject_GetAttr(table, s_slot)), blocks_d(PyObject_GetAttr(table, s_blocks)),
      ntok_d(PyObject_GetAttr(table, s_ntok)), last_d(PyObject_GetAttr(table, s_last)),
      step_o(PyObject_GetAttr(table, s_step));
  Ref rows(PyObject_GetAttr(upd, s_rows)), ts(PyObject_GetAttr(upd, s_ts)),
      ti(PyObject_GetAttr(upd, s_ti)), tv(PyObject_GetAttr(upd, s_tv)),
      bsl(PyObject_GetAttr(upd, s_bs_)), bi(PyObject_GetAttr(upd, s_bi)),
      bv(PyObject_GetAttr(upd, s_bv));
  if (!slot_d || !blocks_d || !ntok_d || !last_d || !step_o || !rows || !ts || !ti || !tv ||
      !bsl || !bi || !bv)
    return nullptr;
  long long capb, capt;
  if (!table_caps(table, s_capb, s_capt, &capb, &capt)) return nullptr;
  bool err = false;
  long long up_rows = attr_ll(table, s_ubr, &err), up_elems = attr_ll(table, s_ube, &err);
  if (err) return nullptr;

  Ref cu(PyList_New(0)), kv(PyList_New(0)), sample(PyDict_New()), splice(PyList_New(0));
  if (!cu || !kv || !sample || !splice) return nullptr;
  // get_request: the plan's lookup, or its request mapping itself (a plan
  // whose get_request is a plain mapping lookup, as BatchPlan's is), which
  // saves a Python call per request
  const bool by_map = !PyCallable_Check(get_request);
  Ref seq(PySequence_Fast(scheduled, "scheduled must be a sequence"));
  if (!seq) return nullptr;
  const Py_ssize_t count = PySequence_Fast_GET_SIZE(seq.get());
  PyObject** items = PySequence_Fast_ITEMS(seq.get());
  long long qacc = 0, width = 0;
  bool all_decode = true;
  Ref live_set;

  for (Py_ssize_t r = 0; r < count; ++r) {
    PyObject* sr = items[r];
    Ref rid(PyObject_GetAttr(sr, s_rid));
    if (!rid) return nullptr;
    Ref req(by_map ? PyObject_GetItem(get_request, rid.get())
                   : PyObject_CallOneArg(get_request, rid.get()));
    if (!req) return nullptr;
    const long long n = attr_ll(sr, s_n, &err);
    const long long start = attr_ll(req.get(), s_ncomp, &err);
    if (err) return nullptr;
    PyObject* blocks = PyObject_GetItem(tables, rid.get());
    Ref blocks_ref(blocks);
    if (!blocks) return nullptr;
    const Py_ssize_t nb = PyObject_Length(blocks);
    if (nb < 0) return nullptr;
    const long long end = start + n;
    if (end > nb * bs) {
      PyErr_Format(PyExc_ValueError, "request %S: %zd blocks cannot hold position %lld", rid.get(),
                   nb, end - 1);
      return nullptr;
    }
    // drafts (verify rows of a decode request)
    Ref drafts;
    Py_ssize_t ndraft = 0;
    {
      Ref draft(PyObject_GetAttr(req.get(), s_draft));
      if (!draft) { PyErr_Clear(); }
      else {
        const int truthy = PyObject_IsTrue(draft.get());
        if (truthy < 0) return nullptr;
        Ref pre(PyObject_GetAttr(sr, s_prefill));
        if (!pre) return nullptr;
        const int is_pre = PyObject_IsTrue(pre.get());
        if (is_pre < 0) return nullptr;
        if (truthy && !is_pre) {
          drafts.p = PySequence_Tuple(draft.get());
          if (!drafts) return nullptr;
          ndraft = PyTuple_GET_SIZE(drafts.get());
        }
      }
    }
    // ---- table sync (DeviceRequestTable.sync)
    long long slot;
    {
      PyObject* so = PyDict_GetItemWithError(slot_d.get(), rid.get());   // borrowed
      if (!so && PyErr_Occurred()) return nullptr;
      if (!so) {
        if (live == Py_None) {   // the step's request ids, built on first need
          live_set.p = PySet_New(nullptr);
          if (!live_set) return nullptr;
          for (Py_ssize_t k = 0; k < count; ++k) {
            Ref id(PyObject_GetAttr(items[k], s_rid));
            if (!id || PySet_Add(live_set.get(), id.get()) < 0) return nullptr;
          }
          live = live_set.get();
        }
        Ref s(PyObject_CallMethodObjArgs(table, s_slot_for, rid.get(), live, nullptr));
        if (!s) return nullptr;
        slot = as_ll(s.get(), &err);
        // a new slot may have come with a grown pool
        if (!table_caps(table, s_capb, s_capt, &capb, &capt)) return nullptr;
      } else {
        slot = as_ll(so, &err);
        if (PyDict_SetItem(last_d.get(), rid.get(), step_o.get()) < 0) return nullptr;
      }
      if (err) return nullptr;
    }
    if (nb > capb || end > capt) {
      Ref kw(PyDict_New());
      if (!kw) return nullptr;
      if (nb > capb) {
        Ref v(PyLong_FromLongLong(nb > 2 * capb ? nb : 2 * capb));
        if (!v || PyDict_SetItemString(kw.get(), "blocks", v.get()) < 0) return nullptr;
      }
      if (end > capt) {
        Ref v(PyLong_FromLongLong(end > 2 * capt ? end : 2 * capt));
        if (!v || PyDict_SetItemString(kw.get(), "tokens", v.get()) < 0) return nullptr;
      }
      Ref grow(PyObject_GetAttr(table, s_grow));
      Ref empty(PyTuple_New(0));
      if (!grow || !empty) return nullptr;
      Ref res(PyObject_Call(grow.get(), empty.get(), kw.get()));
      if (!res) return nullptr;
      if (!table_caps(table, s_capb, s_capt, &capb, &capt)) return nullptr;
    }
    Py_ssize_t first = 0;
    PyObject* prev = PyDict_GetItemWithError(blocks_d.get(), rid.get());   // borrowed
    if (!prev && PyErr_Occurred()) return nullptr;
    if (prev) {
      const Py_ssize_t np_ = PyObject_Length(prev);
      if (np_ < 0) return nullptr;
      if (np_ == nb) {
        const int eq = PyObject_RichCompareBool(prev, blocks, Py_EQ);
        if (eq < 0) return nullptr;
        if (eq) first = nb;
        else if (PyTuple_Check(blocks)) first = 0;
        else {
          Ref tb(PySequence_Tuple(blocks));
          if (!tb) return nullptr;
          const int eq2 = PyObject_RichCompareBool(prev, tb.get(), Py_EQ);
          if (eq2 < 0) return nullptr;
          first = eq2 ? nb : 0;
        }
      }
      if (first == 0 && np_ <= nb) {
        Ref head(PySequence_GetSlice(blocks, 0, np_));
        if (!head) return nullptr;
        Ref th(PySequence_Tuple(head.get()));
        if (!th) return nullptr;
        const int eq = PyObject_RichCompareBool(th.get(), prev, Py_EQ);
        if (eq < 0) return nullptr;
        if (eq) first = np_;
      }
    }
    if (first < nb) {
      for (Py_ssize_t c = first; c < nb; ++c) {
        Ref b(PySequence_GetItem(blocks, c));
        if (!b || PyList_Append(bv.get(), b.get()) < 0) return nullptr;
        if (!append_ll(bsl.get(), slot) || !append_ll(bi.get(), c)) return nullptr;
      }
      up_rows += 1;
      up_elems += nb - first;
      Ref tb(PySequence_Tuple(blocks));
      if (!tb || PyDict_SetItem(blocks_d.get(), rid.get(), tb.get()) < 0) return nullptr;
    } else if (!prev) {
      Ref tb(PySequence_Tuple(blocks));
      if (!tb || PyDict_SetItem(blocks_d.get(), rid.get(), tb.get()) < 0) return nullptr;
    }
    {
      Ref ids(PyObject_GetAttr(req.get(), s_ids));
      if (!ids) return nullptr;
      const Py_ssize_t nids = PyObject_Length(ids.get());
      if (nids < 0) return nullptr;
      PyObject* ho = PyDict_GetItemWithError(ntok_d.get(), rid.get());
      if (!ho && PyErr_Occurred()) return nullptr;
      long long have = ho ? as_ll(ho, &err) : 0;
      if (err) return nullptr;
      long long real_hi = end - ndraft;
      if (real_hi > nids) real_hi = nids;
      if (real_hi > have) {
        for (long long p = have; p < real_hi; ++p) {
          Ref t(PySequence_GetItem(ids.get(), p));
          if (!t || PyList_Append(tv.get(), t.get()) < 0) return nullptr;
          if (!append_ll(ts.get(), slot) || !append_ll(ti.get(), p)) return nullptr;
        }
        Ref hv(PyLong_FromLongLong(real_hi));
        if (!hv || PyDict_SetItem(ntok_d.get(), rid.get(), hv.get()) < 0) return nullptr;
        have = real_hi;
      }
      if (ndraft) {
        const long long base = end - ndraft;
        for (Py_ssize_t d = 0; d < ndraft; ++d) {
          if (PyList_Append(tv.get(), PyTuple_GET_ITEM(drafts.get(), d)) < 0) return nullptr;
          if (!append_ll(ts.get(), slot) || !append_ll(ti.get(), base + d)) return nullptr;
        }
        // drafted positions are not real tokens: resync them later
        Ref hv(PyLong_FromLongLong(have < base ? have : base));
        if (!hv || PyDict_SetItem(ntok_d.get(), rid.get(), hv.get()) < 0) return nullptr;
      }
    }
    // ---- row descriptor and step lists
    {
      Ref row(Py_BuildValue("(LLLnLLii)", slot, start, n, nb, 0LL, qacc, 0, -1));
      if (!row || PyList_Append(rows.get(), row.get()) < 0) return nullptr;
    }
    const long long npr = attr_ll(req.get(), s_nprompt, &err);
    if (err) return nullptr;
    if (end > npr) {
      for (long long li = (npr - start > 0 ? npr - start : 0); li < n; ++li) {
        Ref e(Py_BuildValue("(LO)", qacc + li, rid.get()));
        if (!e || PyList_Append(splice.get(), e.get()) < 0) return nullptr;
      }
    }
    if (start < npr) all_decode = false;
    qacc += n;
    if (!append_ll(cu.get(), qacc) || !append_ll(kv.get(), end)) return nullptr;
    Ref last(PyLong_FromLongLong(qacc - 1));
    if (!last || PyDict_SetItem(sample.get(), rid.get(), last.get()) < 0) return nullptr;
    if (nb > width) width = nb;
  }
  {
    Ref a(PyLong_FromLongLong(up_rows)), b(PyLong_FromLongLong(up_elems));
    if (!a || !b || PyObject_SetAttr(table, s_ubr, a.get()) < 0 ||
        PyObject_SetAttr(table, s_ube, b.get()) < 0)
      return nullptr;
  }
  return Py_BuildValue("(NNNNOLL)", cu.release(), kv.release(), sample.release(), splice.release(),
                       all_decode ? Py_True : Py_False, qacc, width);
}

// list of ints -> int64 / int32 array; a_width != 0: out[k] = a[k] * a_width + b[k]
// (a and b are lists or tuples: PySequence_Fast_ITEMS reads both)
bool fill_ll(PyObject* a, PyObject* b, long long a_width, long long* out, Py_ssize_t n) {
  bool err = false;
  PyObject** ai = PySequence_Fast_ITEMS(a);
  PyObject** bi = b ? PySequence_Fast_ITEMS(b) : nullptr;
  for (Py_ssize_t k = 0; k < n && !err; ++k) {
    long long v = as_ll(ai[k], &err);
    if (bi) v = v * a_width + as_ll(bi[k], &err);
    out[k] = v;
  }
  return !err;
}

bool fill_i32(PyObject* a, int* out, Py_ssize_t n) {
  bool err = false;
  PyObject** ai = PySequence_Fast_ITEMS(a);
  for (Py_ssize_t k = 0; k < n && !err; ++k) {
    const long long v = as_ll(ai[k], &err);
    if (v < INT32_MIN || v > INT32_MAX) {
      PyErr_SetString(PyExc_OverflowError, "value does not fit int32");
      return false;
    }
    out[k] = (int)v;
  }
  return !err;
}

// Interned attribute names of the per-step update lists.
PyObject *u_ts, *u_ti, *u_tv, *u_bs, *u_bi, *u_bv, *u_rows;
bool intern_update_names() {
  if (u_rows) return true;
  u_ts = PyUnicode_InternFromString("tok_slot");
  u_ti = PyUnicode_InternFromString("tok_idx");
  u_tv = PyUnicode_InternFromString("tok_val");
  u_bs = PyUnicode_InternFromString("blk_slot");
  u_bi = PyUnicode_InternFromString("blk_idx");
  u_bv = PyUnicode_InternFromString("blk_val");
  u_rows = PyUnicode_InternFromString("rows");
  return u_ts && u_ti && u_tv && u_bs && u_bi && u_bv && u_rows;
}

PyObject* get_list(PyObject* o, PyObject* name) {
  PyObject* v = PyObject_GetAttr(o, name);
  if (v && !PyList_Check(v)) {
    Py_DECREF(v);
    PyErr_Format(PyExc_TypeError, "updates.%U must be a list", name);
    return nullptr;
  }
  return v;
}

// Writes one step's uploads into host memory at `h` (the upload layout of
// _Uploader.upload: token pool index / value int64, block pool index int64 /
// value int32, row descriptors int32 x row_ints), at the byte offsets the
// caller computed for these list lengths; reports the lengths.
bool stage_impl(PyObject* upd, char* h, long long tw, long long bw, const long long (&o)[5],
                long long row_ints, Py_ssize_t* nt_out, Py_ssize_t* nb_out, Py_ssize_t* nr_out) {
  if (!intern_update_names()) return false;
  Ref ts(get_list(upd, u_ts)), ti(get_list(upd, u_ti)), tv(get_list(upd, u_tv));
  Ref bsl(get_list(upd, u_bs)), bi(get_list(upd, u_bi)), bv(get_list(upd, u_bv));
  Ref rows(get_list(upd, u_rows));
  if (!ts || !ti || !tv || !bsl || !bi || !bv || !rows) return false;
  const Py_ssize_t nt = PyList_GET_SIZE(ti.get()), nb = PyList_GET_SIZE(bi.get());
  const Py_ssize_t nr = PyList_GET_SIZE(rows.get());
  if (PyList_GET_SIZE(ts.get()) != nt || PyList_GET_SIZE(tv.get()) != nt ||
      PyList_GET_SIZE(bsl.get()) != nb || PyList_GET_SIZE(bv.get()) != nb) {
    PyErr_SetString(PyExc_ValueError, "update lists differ in length");
    return false;
  }
  if (!fill_ll(ts.get(), ti.get(), tw, reinterpret_cast<long long*>(h + o[0]), nt) ||
      !fill_ll(tv.get(), nullptr, 0, reinterpret_cast<long long*>(h + o[1]), nt) ||
      !fill_ll(bsl.get(), bi.get(), bw, reinterpret_cast<long long*>(h + o[2]), nb) ||
      !fill_i32(bv.get(), reinterpret_cast<int*>(h + o[3]), nb))
    return false;
  int* rp = reinterpret_cast<int*>(h + o[4]);
  for (Py_ssize_t r = 0; r < nr; ++r) {
    PyObject* row = PyList_GET_ITEM(rows.get(), r);
    if (!PyTuple_Check(row) || PyTuple_GET_SIZE(row) != row_ints) {
      PyErr_SetString(PyExc_ValueError, "row descriptors must be tuples of row_ints ints");
      return false;
    }
    if (!fill_i32(row, rp + r * row_ints, row_ints)) return false;
  }
  *nt_out = nt; *nb_out = nb; *nr_out = nr;
  return true;
}

PyObject* stage(PyObject*, PyObject* args) {
  PyObject* upd;
  unsigned long long base;
  long long tw, bw, row_ints, o[5];
  if (!PyArg_ParseTuple(args, "OKLLLLLLLL", &upd, &base, &tw, &bw, &o[0], &o[1], &o[2], &o[3],
                        &o[4], &row_ints))
    return nullptr;
  Py_ssize_t nt, nb, nr;
  if (!stage_impl(upd, reinterpret_cast<char*>(base), tw, bw, o, row_ints, &nt, &nb, &nr))
    return nullptr;
  Py_RETURN_NONE;
}

// aia_pack_rows (include/auto_infer_amd.h), reached through the address the
// Python side reads from the loaded library.
typedef int (*PackRowsFn)(const int64_t*, const int64_t*, int32_t, const int64_t*, const int32_t*,
                          int32_t, int64_t*, int64_t, int32_t*, int64_t, const int32_t*, int32_t,
                          int32_t, int32_t, int64_t*, int64_t*, int32_t*, int32_t*, int32_t*,
                          int32_t*, int64_t*, int64_t*, int32_t, int32_t, void*);

constexpr int kHipError = -1000;   // returned (negated HIP code added) on a runtime failure

// One step's upload and pack launch, the native form of _Uploader.upload +
// _launch: wait for the event of the last copy that read this staging
// buffer (if any), stage the updates into it at the caller's offsets, copy
// the `total` bytes to the device buffer and record the event on `stream`,
// then call aia_pack_rows on the staged arrays.  Returns aia_pack_rows'
// status, or kHipError - code when a runtime call fails.
PyObject* upload_pack(PyObject*, PyObject* args) {
  PyObject* upd;
  unsigned long long fn, host, dev, wait_ev, rec_ev, stream, token_pool, block_pool;
  unsigned long long token_ids, positions, slot_mapping, block_table, cu, kv, last_rows, sample_rows;
  long long tw, bw, total, o[5], row_ints, tp_stride, bp_stride;
  int block_size, bt_width, sample_count, sample_cap;
  if (!PyArg_ParseTuple(args, "OKKKKKKLLLLLLLLLKLKLiiKKKKKKKKii", &upd, &fn, &host, &dev, &wait_ev,
                        &rec_ev, &stream, &tw, &bw, &total, &o[0], &o[1], &o[2], &o[3], &o[4],
                        &row_ints, &token_pool, &tp_stride, &block_pool, &bp_stride, &block_size,
                        &bt_width, &token_ids, &positions, &slot_mapping, &block_table, &cu, &kv,
                        &last_rows, &sample_rows, &sample_count, &sample_cap))
    return nullptr;
  if (wait_ev) {
    const hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(wait_ev));
    if (e != hipSuccess) return PyLong_FromLong(kHipError - (int)e);
  }
  Py_ssize_t nt, nb, nr;
  if (!stage_impl(upd, reinterpret_cast<char*>(host), tw, bw, o, row_ints, &nt, &nb, &nr))
    return nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(dev), reinterpret_cast<const void*>(host),
                                (size_t)total, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipEventRecord(reinterpret_cast<hipEvent_t>(rec_ev), st);
  if (e != hipSuccess) return PyLong_FromLong(kHipError - (int)e);
  char* d = reinterpret_cast<char*>(dev);
  const int rc = reinterpret_cast<PackRowsFn>(fn)(
      reinterpret_cast<const int64_t*>(d + o[0]), reinterpret_cast<const int64_t*>(d + o[1]),
      (int32_t)nt, reinterpret_cast<const int64_t*>(d + o[2]), reinterpret_cast<const int32_t*>(d + o[3]),
      (int32_t)nb, reinterpret_cast<int64_t*>(token_pool), tp_stride,
      reinterpret_cast<int32_t*>(block_pool), bp_stride, reinterpret_cast<const int32_t*>(d + o[4]),
      (int32_t)nr, block_size, bt_width, reinterpret_cast<int64_t*>(token_ids),
      reinterpret_cast<int64_t*>(positions), reinterpret_cast<int32_t*>(slot_mapping),
      reinterpret_cast<int32_t*>(block_table), reinterpret_cast<int32_t*>(cu),
      reinterpret_cast<int32_t*>(kv), reinterpret_cast<int64_t*>(last_rows),
      reinterpret_cast<int64_t*>(sample_rows), sample_count, sample_cap,
      reinterpret_cast<void*>(stream));
  return PyLong_FromLong(rc);
}

// aia_pack_rows_inline, reached through the address the Python side reads.
typedef int (*PackInlineFn)(const void*, int32_t, int32_t, int32_t, int64_t*, int64_t, int32_t*,
                            int64_t, int32_t, int32_t, int64_t*, int64_t*, int32_t*, int32_t*,
                            int32_t*, int32_t*, int64_t*, int64_t*, int32_t, int32_t, void*);
constexpr long long kInlineBytes = 3072;   // AIA_PACK_INLINE_BYTES

// A small step's pack without a staging copy: the updates and rows are
// staged into a local buffer in the layout aia_pack_rows_inline takes (token
// indices, token values, block indices, block values padded to a word, rows)
// and handed to it, which passes them in the kernel launch.  Returns its
// status, or kInlineTooLarge (nothing launched) when the step does not fit
// kInlineBytes; raises ValueError (from staging) on malformed updates.
// Positional arguments, taken without a format string (METH_FASTCALL): the
// call sits on every decode step's host path.
constexpr int kInlineTooLarge = 1;
PyObject* pack_inline(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 22) {
    PyErr_SetString(PyExc_TypeError, "pack_inline takes 22 arguments");
    return nullptr;
  }
  PyObject* upd = args[0];
  long long v[21];
  for (int i = 1; i < 22; ++i) {
    v[i - 1] = PyLong_AsLongLong(args[i]);
    if (v[i - 1] == -1 && PyErr_Occurred()) {
      PyErr_Clear();      // addresses above 2^63 arrive as unsigned
      v[i - 1] = (long long)PyLong_AsUnsignedLongLong(args[i]);
      if (PyErr_Occurred()) return nullptr;
    }
  }
  const unsigned long long fn = v[0], stream = v[1];
  const long long tw = v[2], bw = v[3], row_ints = v[4];
  const unsigned long long token_pool = v[5];
  const long long tp_stride = v[6];
  const unsigned long long block_pool = v[7];
  const long long bp_stride = v[8];
  const int block_size = (int)v[9], bt_width = (int)v[10];
  const unsigned long long token_ids = v[11], positions = v[12], slot_mapping = v[13],
                           block_table = v[14], cu = v[15], kv = v[16], last_rows = v[17],
                           sample_rows = v[18];
  const int sample_count = (int)v[19], sample_cap = (int)v[20];
  if (!intern_update_names()) return nullptr;
  Ref ti(get_list(upd, u_ti)), bi(get_list(upd, u_bi)), rows(get_list(upd, u_rows));
  if (!ti || !bi || !rows) return nullptr;
  const long long nt = PyList_GET_SIZE(ti.get()), nb = PyList_GET_SIZE(bi.get());
  const long long nr = PyList_GET_SIZE(rows.get());
  const long long o[5] = {0, 8 * nt, 16 * nt, 16 * nt + 8 * nb, 16 * nt + 8 * nb + 8 * ((nb + 1) / 2)};
  const long long total = o[4] + nr * row_ints * 4;
  if (total > kInlineBytes) return PyLong_FromLong(kInlineTooLarge);
  alignas(16) char h[kInlineBytes];
  Py_ssize_t snt, snb, snr;
  if (!stage_impl(upd, h, tw, bw, o, row_ints, &snt, &snb, &snr)) return nullptr;
  const int rc = reinterpret_cast<PackInlineFn>(fn)(
      h, (int32_t)snt, (int32_t)snb, (int32_t)snr, reinterpret_cast<int64_t*>(token_pool), tp_stride,
      reinterpret_cast<int32_t*>(block_pool), bp_stride, block_size, bt_width,
      reinterpret_cast<int64_t*>(token_ids), reinterpret_cast<int64_t*>(positions),
      reinterpret_cast<int32_t*>(slot_mapping), reinterpret_cast<int32_t*>(block_table),
      reinterpret_cast<int32_t*>(cu), reinterpret_cast<int32_t*>(kv),
      reinterpret_cast<int64_t*>(last_rows), reinterpret_cast<int64_t*>(sample_rows), sample_count,
      sample_cap, reinterpret_cast<void*>(stream));
  return PyLong_FromLong(rc);
}

PyMethodDef methods[] = {
    {"pack_inline", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(pack_inline)),
     METH_FASTCALL,
     "pack_inline(updates, pack_rows_inline_fn, stream, token_width, block_width, row_ints, "
     "token_pool, token_pool_stride, block_pool, block_pool_stride, block_size, bt_width, "
     "token_ids, positions, slot_mapping, block_table, cu, kv, last_rows, sample_rows, "
     "sample_count, sample_cap) -> status (1: the step does not fit the launch, nothing done)"},
    {"upload_pack", upload_pack, METH_VARARGS,
     "upload_pack(updates, pack_rows_fn, host, dev, wait_event, record_event, stream, token_width, "
     "block_width, total, 5 offsets, row_ints, token_pool, token_pool_stride, block_pool, "
     "block_pool_stride, block_size, bt_width, token_ids, positions, slot_mapping, block_table, "
     "cu, kv, last_rows, sample_rows, sample_count, sample_cap) -> status"},
    {"stage", stage, METH_VARARGS,
     "stage(updates, host_address, token_width, block_width, off_tok_idx, off_tok_val, "
     "off_blk_idx, off_blk_val, off_rows, row_ints) -> None"},
    {"build_rows", build_rows, METH_VARARGS,
     "build_rows(table, scheduled, get_request, block_tables, block_size, updates, live) "
     "(live: the step's request ids, or None to build them only if a new slot is needed) -> "
     "(cu_seqlens_q, seqlens_kv, sample_idx, decode_splice, all_decode, tokens, width)"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_hostpack",
                      "Native per-request loop of DeviceBatchPacker.build.", -1, methods};

}  // namespace

PyMODINIT_FUNC PyInit__hostpack(void) { return PyModule_Create(&module); }
