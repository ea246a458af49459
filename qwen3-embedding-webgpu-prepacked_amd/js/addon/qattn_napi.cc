// qattn_napi.cc -- Node N-API binding of libqattn.so (C ABI: include/qattn.h).
//
// This is the seam the reference engine reaches through WebGPU (src/webgpu/device.ts,
// src/webgpu/ops.ts:318-345): device context, device buffers, the attention operator
// (createRun / encode / destroy), the mask check and the producer kernels.  Device resources are
// N-API externals; every failure of the C ABI becomes a thrown JavaScript Error carrying
// qattn_last_error() (the reference throws synchronously on contract violations, model.ts:114).
// synchronizeAsync() waits for the context stream on a worker thread and returns a Promise, so
// the engine's run() stays asynchronous like the reference's mapAsync readback (model.ts:135).
#include <node_api.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstring>
#include <set>
#include <string>
#include <vector>

#include "../../../include/qattn.h"

namespace {

#define NAPI_OK(env, call)                                                       \
  do {                                                                           \
    if ((call) != napi_ok) {                                                     \
      const napi_extended_error_info* info_ = nullptr;                           \
      napi_get_last_error_info((env), &info_);                                   \
      napi_throw_error((env), nullptr,                                           \
                       info_ && info_->error_message ? info_->error_message      \
                                                     : "N-API call failed");    \
      return nullptr;                                                            \
    }                                                                            \
  } while (0)

// Lifetime.  A context's JS handle, and every buffer and run made from it, each hold one
// reference on its Ctx; the Ctx is deleted when the last of them is finalized, whatever order the
// garbage collector (or environment teardown) finalizes them in.  The device context itself
// (qattn_ctx) lives until destroyContext() or the last reference: destroyContext() first releases
// every run and buffer still alive on it (runs synchronize on the context stream, so they go
// before the context), and their handles then report "destroyed" instead of touching freed memory.
struct Buf;
struct Run;
struct Model;
struct Plan;
struct Evt;
struct Ctx {
  qattn_ctx* ctx = nullptr;
  int refs = 1;  // the context handle's own reference
  std::set<Buf*> bufs;
  std::set<Run*> runs;
  std::set<Model*> models;
  std::set<Plan*> plans;
  std::set<Evt*> evts;
  int async_busy = 0;  // synchronizeAsync / readAfterAsync waits on worker threads
};
// An event on the context stream (marks the end of one submitted batch).  While a readAfterAsync
// waits on it on a worker thread, destroying it is deferred to the end of that wait.
struct Evt {
  Ctx* owner = nullptr;
  qattn_event_t ev = nullptr;
  int waiters = 0;
  bool destroy_pending = false;
};
struct Buf {
  Ctx* owner = nullptr;
  void* ptr = nullptr;
  size_t bytes = 0;
  int reads_in_flight = 0;  // readAfterAsync copies from this buffer not yet settled
};
// A run holds a reference on each buffer bound to it (so none is collected before the run), and
// the largest token / sequence counts those buffers can take (updateRun checks new batches
// against them).
struct Run {
  Ctx* owner = nullptr;
  qattn_run* run = nullptr;
  std::vector<napi_ref> bound_refs;
  std::vector<const Buf*> bound;
  int64_t max_tokens = 0;
  int64_t max_seqs = 0;  // o_last rows (no limit without o_last)
};

// A model (qattn_model over uploaded weight buffers) holds a reference on each weight buffer; an
// execution plan made from it points back at it.  Destroying or collecting a model first destroys
// the device side of its plans (their handles then report "destroyed").
struct Model {
  Ctx* owner = nullptr;
  qattn_model* model = nullptr;
  std::vector<napi_ref> bound_refs;
  std::set<Plan*> plans;
};
struct Plan {
  Ctx* owner = nullptr;
  Model* model = nullptr;
  qattn_model_plan* plan = nullptr;
  napi_ref model_ref = nullptr;  // keeps the model's handle alive while the plan is
  int64_t max_tokens = 0, max_seqs = 0;
};

void release_device(Ctx* c);
void unref(Ctx* c) {
  if (--c->refs == 0) {
    release_device(c);
    delete c;
  }
}

napi_value throw_qattn(napi_env env, int rc, const qattn_ctx* ctx) {
  std::string msg = "qattn error " + std::to_string(rc) + ": " + qattn_last_error(ctx);
  napi_throw_error(env, std::to_string(rc).c_str(), msg.c_str());
  return nullptr;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

template <typename T>
T* get_external(napi_env env, napi_value v, const char* what) {
  void* data = nullptr;
  if (napi_get_value_external(env, v, &data) != napi_ok || !data) {
    napi_throw_type_error(env, nullptr, (std::string("expected ") + what).c_str());
    return nullptr;
  }
  return static_cast<T*>(data);
}

bool get_i64(napi_env env, napi_value v, int64_t* out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_number) return false;
  return napi_get_value_int64(env, v, out) == napi_ok;
}

bool prop(napi_env env, napi_value obj, const char* name, napi_value* out) {
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return false;
  if (napi_get_named_property(env, obj, name, out) != napi_ok) return false;
  napi_valuetype t;
  napi_typeof(env, *out, &t);
  return t != napi_undefined && t != napi_null;
}

// Typed array (or Buffer) view: data pointer and byte length.
bool typed_bytes(napi_env env, napi_value v, void** data, size_t* bytes) {
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  if (is_ta) {
    napi_typedarray_type type;
    size_t length = 0, offset = 0;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &type, &length, data, &ab, &offset) != napi_ok) return false;
    size_t elem = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: elem = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
      default: elem = 1;
    }
    *bytes = length * elem;
    return true;
  }
  bool is_buf = false;
  napi_is_buffer(env, v, &is_buf);
  if (is_buf) return napi_get_buffer_info(env, v, data, bytes) == napi_ok;
  return false;
}

// Runs, then buffers, then the device context: everything still alive on `c`.
void release_device(Ctx* c) {
  if (!c->ctx) return;
  for (Evt* e : c->evts)
    if (e->ev && e->waiters == 0) {
      qattn_event_destroy(e->ev);
      e->ev = nullptr;
    }
  for (Plan* p : c->plans)
    if (p->plan) {
      qattn_model_plan_destroy(p->plan);
      p->plan = nullptr;
    }
  for (Model* m : c->models)
    if (m->model) {
      qattn_model_destroy(m->model);
      m->model = nullptr;
    }
  for (Run* r : c->runs)
    if (r->run) {
      qattn_run_destroy(r->run);
      r->run = nullptr;
    }
  for (Buf* b : c->bufs)
    if (b->ptr) {
      qattn_buffer_free(c->ctx, b->ptr);
      b->ptr = nullptr;
    }
  qattn_destroy(c->ctx);
  c->ctx = nullptr;
}

void finalize_ctx(napi_env, void* data, void*) { unref(static_cast<Ctx*>(data)); }
void finalize_buf(napi_env, void* data, void*) {
  // Device memory is released by free(); a collected handle that was never freed is released
  // here while its context is still alive.
  auto* b = static_cast<Buf*>(data);
  Ctx* c = b->owner;
  if (b->ptr && c->ctx) qattn_buffer_free(c->ctx, b->ptr);
  c->bufs.erase(b);
  delete b;
  unref(c);
}
void drop_bound(napi_env env, Run* r) {
  for (napi_ref ref : r->bound_refs) napi_delete_reference(env, ref);
  r->bound_refs.clear();
  r->bound.clear();
}
void finalize_run(napi_env env, void* data, void*) {
  auto* r = static_cast<Run*>(data);
  Ctx* c = r->owner;
  if (r->run && c->ctx) qattn_run_destroy(r->run);
  drop_bound(env, r);
  c->runs.erase(r);
  delete r;
  unref(c);
}

napi_value args_of(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc < want) {
    napi_throw_type_error(env, nullptr, "missing arguments");
    return nullptr;
  }
  return undefined(env);
}

// createContext(device) -> external
napi_value CreateContext(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  int64_t device = 0;
  if (!get_i64(env, argv[0], &device)) {
    napi_throw_type_error(env, nullptr, "device must be a number");
    return nullptr;
  }
  qattn_ctx* ctx = nullptr;
  int rc = qattn_create((int)device, &ctx);
  if (rc) return throw_qattn(env, rc, nullptr);
  auto* c = new Ctx{ctx};
  napi_value out;
  NAPI_OK(env, napi_create_external(env, c, finalize_ctx, nullptr, &out));
  return out;
}

napi_value DestroyContext(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Ctx* c = get_external<Ctx>(env, argv[0], "context");
  if (!c) return nullptr;
  if (c->async_busy > 0) {
    napi_throw_error(env, nullptr, "context has asynchronous waits in flight; await them first");
    return nullptr;
  }
  release_device(c);
  return undefined(env);
}

Ctx* live_ctx(napi_env env, napi_value v) {
  Ctx* c = get_external<Ctx>(env, v, "context");
  if (c && !c->ctx) {
    napi_throw_error(env, nullptr, "context was destroyed");
    return nullptr;
  }
  return c;
}

// deviceName(ctx) -> {name, computeUnits}
napi_value DeviceName(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  char name[256];
  int cus = 0;
  int rc = qattn_device_name(c->ctx, name, sizeof(name), &cus);
  if (rc) return throw_qattn(env, rc, c->ctx);
  napi_value out, n, u;
  NAPI_OK(env, napi_create_object(env, &out));
  NAPI_OK(env, napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &n));
  NAPI_OK(env, napi_create_int32(env, cus, &u));
  NAPI_OK(env, napi_set_named_property(env, out, "name", n));
  NAPI_OK(env, napi_set_named_property(env, out, "computeUnits", u));
  return out;
}

// alloc(ctx, bytes) -> external device buffer
napi_value Alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args_of(env, info, 2, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  int64_t bytes = 0;
  if (!c) return nullptr;
  if (!get_i64(env, argv[1], &bytes) || bytes < 0) {
    napi_throw_range_error(env, nullptr, "bytes must be a non-negative number");
    return nullptr;
  }
  void* ptr = nullptr;
  int rc = qattn_buffer_alloc(c->ctx, (size_t)bytes, &ptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  auto* b = new Buf{c, ptr, (size_t)bytes};
  c->bufs.insert(b);
  ++c->refs;
  napi_value out;
  NAPI_OK(env, napi_create_external(env, b, finalize_buf, nullptr, &out));
  return out;
}

napi_value Free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Buf* b = get_external<Buf>(env, argv[0], "device buffer");
  if (!b) return nullptr;
  if (b->reads_in_flight > 0) {
    // a worker thread would copy from freed (or reallocated) device memory
    napi_throw_error(env, nullptr, "device buffer has asynchronous reads in flight; await them first");
    return nullptr;
  }
  if (b->ptr && b->owner->ctx) {
    int rc = qattn_buffer_free(b->owner->ctx, b->ptr);
    if (rc) return throw_qattn(env, rc, b->owner->ctx);
  }
  b->ptr = nullptr;
  return undefined(env);
}

Buf* live_buf(napi_env env, napi_value v) {
  Buf* b = get_external<Buf>(env, v, "device buffer");
  if (b && (!b->ptr || !b->owner->ctx)) {
    napi_throw_error(env, nullptr, "device buffer was freed");
    return nullptr;
  }
  return b;
}

// write(buf, typedArray, byteOffset=0) / read(buf, typedArray, byteOffset=0)
napi_value Copy(napi_env env, napi_callback_info info, bool to_device) {
  napi_value argv[3];
  size_t argc = 3;
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc < 2) {
    napi_throw_type_error(env, nullptr, "missing arguments");
    return nullptr;
  }
  Buf* b = live_buf(env, argv[0]);
  if (!b) return nullptr;
  void* host = nullptr;
  size_t bytes = 0;
  if (!typed_bytes(env, argv[1], &host, &bytes)) {
    napi_throw_type_error(env, nullptr, "expected a TypedArray or Buffer");
    return nullptr;
  }
  int64_t offset = 0;
  if (argc > 2 && !get_i64(env, argv[2], &offset)) offset = 0;
  if (offset < 0 || (size_t)offset + bytes > b->bytes) {
    napi_throw_range_error(env, nullptr, "copy exceeds the device buffer");
    return nullptr;
  }
  int rc = to_device ? qattn_buffer_write(b->owner->ctx, b->ptr, (size_t)offset, host, bytes)
                     : qattn_buffer_read(b->owner->ctx, b->ptr, (size_t)offset, host, bytes);
  if (rc) return throw_qattn(env, rc, b->owner->ctx);
  return undefined(env);
}
napi_value Write(napi_env env, napi_callback_info info) { return Copy(env, info, true); }
napi_value Read(napi_env env, napi_callback_info info) { return Copy(env, info, false); }

bool get_i32_array(napi_env env, napi_value v, std::vector<int32_t>* out) {
  void* data = nullptr;
  size_t bytes = 0;
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  if (is_ta) {
    napi_typedarray_type type;
    size_t length = 0, offset = 0;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &type, &length, &data, &ab, &offset) != napi_ok) return false;
    if (type == napi_int32_array || type == napi_uint32_array) {
      out->assign(static_cast<int32_t*>(data), static_cast<int32_t*>(data) + length);
      return true;
    }
    return false;
  }
  bool is_arr = false;
  napi_is_array(env, v, &is_arr);
  if (!is_arr) return false;
  uint32_t n = 0;
  napi_get_array_length(env, v, &n);
  out->resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    int64_t x = 0;
    napi_get_element(env, v, i, &e);
    if (!get_i64(env, e, &x)) return false;
    (*out)[i] = (int32_t)x;
  }
  (void)bytes;
  return true;
}

// Fills a qattn_run_desc from a JS descriptor object.  Device tensors are buffer externals of
// context `owner` with optional byte offsets (qOffsetBytes, ...), strides in elements.  With a
// device, every tensor's extent -- the bytes the kernels can touch, from its offset, strides and
// the token count -- is checked against its buffer (RangeError), as WebGPU validates bindings.
struct Binding {
  const Buf* buf = nullptr;
  int64_t off = 0;
  napi_value js = nullptr;
};
struct Bindings {
  Binding q, k, v, o, last;
};
bool read_desc(napi_env env, napi_value d, qattn_run_desc* desc, std::vector<int32_t>* cu,
               const Ctx* owner, Bindings* bindings = nullptr) {
  const bool need_device = owner != nullptr;
  std::memset(desc, 0, sizeof(*desc));
  napi_value v;
  auto ptr_of = [&](const char* name, const char* off_name, const void** out, bool required,
                    Binding* bind) {
    if (!prop(env, d, name, &v)) {
      if (required) napi_throw_type_error(env, nullptr, (std::string("missing ") + name).c_str());
      return !required;
    }
    if (!need_device) {
      // host-only planning: any non-null stand-in address is fine
      *out = reinterpret_cast<const void*>(uintptr_t(0x100000));
      return true;
    }
    Buf* b = live_buf(env, v);
    if (!b) return false;
    if (b->owner != owner) {
      napi_throw_error(env, nullptr, (std::string(name) + " belongs to another context").c_str());
      return false;
    }
    int64_t off = 0;
    napi_value ov;
    if (prop(env, d, off_name, &ov) && !get_i64(env, ov, &off)) off = -1;
    if (off < 0 || (uint64_t)off >= b->bytes || off % 16 != 0) {
      napi_throw_range_error(env, nullptr,
                             (std::string(off_name) + " must be a multiple of 16 inside the buffer").c_str());
      return false;
    }
    *out = static_cast<const char*>(b->ptr) + off;
    bind->buf = b;
    bind->off = off;
    bind->js = v;
    return true;
  };
  const void *q, *k, *vv, *o, *ol = nullptr;
  Bindings local;
  Bindings& bb = bindings ? *bindings : local;
  Binding &bq = bb.q, &bk = bb.k, &bv = bb.v, &bo = bb.o, &bl = bb.last;
  if (!ptr_of("q", "qOffsetBytes", &q, true, &bq) || !ptr_of("k", "kOffsetBytes", &k, true, &bk) ||
      !ptr_of("v", "vOffsetBytes", &vv, true, &bv) || !ptr_of("o", "oOffsetBytes", &o, true, &bo) ||
      !ptr_of("oLast", "oLastOffsetBytes", &ol, false, &bl))
    return false;
  desc->q = q;
  desc->k = k;
  desc->v = vv;
  desc->o = const_cast<void*>(o);
  desc->o_last = const_cast<void*>(ol);
  auto num = [&](const char* name, int64_t dflt) {
    int64_t x = dflt;
    if (prop(env, d, name, &v)) get_i64(env, v, &x);
    return x;
  };
  desc->q_row_stride = num("qRowStride", 2048);
  desc->k_row_stride = num("kRowStride", 1024);
  desc->v_row_stride = num("vRowStride", 1024);
  desc->o_row_stride = num("oRowStride", 2048);
  desc->v_offset = num("vOffset", 0);
  desc->mask = (int32_t)num("mask", QATTN_MASK_PREFIX_LOCAL);
  desc->prefix = (int32_t)num("prefix", 176);
  desc->window = (int32_t)num("window", 432);
  desc->flags = (int32_t)num("flags", 0);
  if (!prop(env, d, "cuSeqlens", &v) || !get_i32_array(env, v, cu) || cu->size() < 2) {
    napi_throw_type_error(env, nullptr, "cuSeqlens must be an Int32Array of nseq+1 offsets");
    return false;
  }
  desc->cu_seqlens = cu->data();
  desc->nseq = (int32_t)cu->size() - 1;
  if (!need_device) return true;
  // Extents.  Strides below the head widths, bad cu_seqlens etc. are the C ABI's to reject (with
  // its message); here only what would let a valid-looking descriptor reach past a buffer.
  const int64_t T = cu->back();
  for (int32_t i = 0; i < desc->nseq; ++i)
    if ((*cu)[i + 1] < (*cu)[i] || (*cu)[i] < 0) return true;  // the C ABI rejects it
  if (T <= 0) return true;
  if (desc->q_row_stride < 0 || desc->k_row_stride < 0 || desc->v_row_stride < 0 ||
      desc->o_row_stride < 0 || desc->v_offset < 0 || T > ((int64_t)1 << 31))
    return true;  // rejected by the C ABI
  auto fits = [&](const Binding& b, int64_t elems, const char* name) {
    if ((uint64_t)b.off + 2 * (uint64_t)elems > b.buf->bytes) {
      napi_throw_range_error(env, nullptr,
                             (std::string(name) + ": rows x stride exceed the device buffer").c_str());
      return false;
    }
    return true;
  };
  if (!fits(bq, (T - 1) * desc->q_row_stride + 2048, "q") ||
      !fits(bk, (T - 1) * desc->k_row_stride + 1024, "k") ||
      !fits(bv, desc->v_offset + (T - 1) * desc->v_row_stride + 1024, "v") ||
      !fits(bo, (T - 1) * desc->o_row_stride + 2048, "o"))
    return false;
  if (ol && !fits(bl, (int64_t)desc->nseq * 2048, "oLast")) return false;
  return true;
}

napi_value info_object(napi_env env, const qattn_run_info& i) {
  napi_value out, x;
  napi_create_object(env, &out);
  auto set = [&](const char* n, double val) {
    napi_create_double(env, val, &x);
    napi_set_named_property(env, out, n, x);
  };
  set("tokens", (double)i.tokens);
  set("pairs", (double)i.pairs);
  set("flops", (double)i.flops);
  set("bytes", (double)i.bytes);
  set("workItems", i.work_items);
  set("blockQueries", i.block_queries);
  set("tilePairs", (double)i.tile_pairs);
  set("slots", i.slots);
  set("splitItems", i.split_items);
  return out;
}

// createRun(ctx, desc) -> external run  (reference: CausalAttentionKernel.createRun)
napi_value CreateRun(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args_of(env, info, 2, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  qattn_run_desc desc;
  std::vector<int32_t> cu;
  Bindings bind;
  if (!read_desc(env, argv[1], &desc, &cu, c, &bind)) return nullptr;
  qattn_run* run = nullptr;
  int rc = qattn_run_create(c->ctx, &desc, &run);
  if (rc) return throw_qattn(env, rc, c->ctx);
  auto* r = new Run{c, run};
  // Capacity: the most rows every bound tensor can hold at its offset and stride.
  auto rows_fit = [](const Binding& b, int64_t stride, int64_t extra, int64_t width) {
    const int64_t avail = (int64_t)b.buf->bytes / 2 - b.off / 2 - extra - width;
    return avail < 0 ? 0 : avail / std::max<int64_t>(stride, 1) + 1;
  };
  r->max_tokens = std::min(std::min(rows_fit(bind.q, desc.q_row_stride, 0, 2048), rows_fit(bind.k, desc.k_row_stride, 0, 1024)),
                           std::min(rows_fit(bind.v, desc.v_row_stride, desc.v_offset, 1024),
                                    rows_fit(bind.o, desc.o_row_stride, 0, 2048)));
  r->max_seqs = desc.o_last ? (int64_t)(bind.last.buf->bytes - bind.last.off) / 4096 : INT64_MAX;
  for (const Binding* b : {&bind.q, &bind.k, &bind.v, &bind.o, &bind.last}) {
    if (!b->buf) continue;
    napi_ref ref;
    NAPI_OK(env, napi_create_reference(env, b->js, 1, &ref));
    r->bound_refs.push_back(ref);
    r->bound.push_back(b->buf);
  }
  c->runs.insert(r);
  ++c->refs;
  napi_value out;
  NAPI_OK(env, napi_create_external(env, r, finalize_run, nullptr, &out));
  return out;
}

Run* live_run(napi_env env, napi_value v) {
  Run* r = get_external<Run>(env, v, "attention run");
  if (r && (!r->run || !r->owner->ctx)) {
    napi_throw_error(env, nullptr, r->run ? "context was destroyed" : "attention run was destroyed");
    return nullptr;
  }
  if (r)
    for (const Buf* b : r->bound)
      if (!b->ptr) {
        napi_throw_error(env, nullptr, "a device buffer bound to this run was freed");
        return nullptr;
      }
  return r;
}

// updateRun(run, cuSeqlens)  -- a new batch for the same tensors (qattn_run_update)
napi_value UpdateRun(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args_of(env, info, 2, argv)) return nullptr;
  Run* r = live_run(env, argv[0]);
  if (!r) return nullptr;
  std::vector<int32_t> cu;
  if (!get_i32_array(env, argv[1], &cu) || cu.size() < 2) {
    napi_throw_type_error(env, nullptr, "cuSeqlens must be an Int32Array of nseq+1 offsets");
    return nullptr;
  }
  if ((int64_t)cu.back() > r->max_tokens || (int64_t)cu.size() - 1 > r->max_seqs) {
    napi_throw_range_error(env, nullptr, "the batch exceeds the buffers bound to this run");
    return nullptr;
  }
  int rc = qattn_run_update(r->run, cu.data(), (int32_t)cu.size() - 1);
  if (rc) return throw_qattn(env, rc, r->owner->ctx);
  return undefined(env);
}

// encode(run)  (reference: CausalAttentionKernel.encode(pass, run))
napi_value Encode(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Run* r = live_run(env, argv[0]);
  if (!r) return nullptr;
  int rc = qattn_run_encode(r->run, nullptr);
  if (rc) return throw_qattn(env, rc, nullptr);
  return undefined(env);
}

napi_value DestroyRun(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Run* r = get_external<Run>(env, argv[0], "attention run");
  if (!r) return nullptr;
  if (r->run && r->owner->ctx) qattn_run_destroy(r->run);
  r->run = nullptr;
  drop_bound(env, r);
  return undefined(env);
}

napi_value RunInfo(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Run* r = live_run(env, argv[0]);
  if (!r) return nullptr;
  qattn_run_info i{};
  int rc = qattn_run_get_info(r->run, &i);
  if (rc) return throw_qattn(env, rc, nullptr);
  return info_object(env, i);
}

// planDescribe(desc) -> {items: Int32Array (n*8 entries), info}; host only, no device needed.
napi_value PlanDescribe(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  qattn_run_desc desc;
  std::vector<int32_t> cu;
  if (!read_desc(env, argv[0], &desc, &cu, nullptr)) return nullptr;
  int32_t n = 0;
  qattn_run_info i{};
  int rc = qattn_plan_describe(&desc, nullptr, 0, &n, &i);
  if (rc) return throw_qattn(env, rc, nullptr);
  napi_value ab, arr, out;
  void* data = nullptr;
  NAPI_OK(env, napi_create_arraybuffer(env, (size_t)n * 32, &data, &ab));
  if (n) {
    rc = qattn_plan_describe(&desc, static_cast<int32_t*>(data), n, &n, nullptr);
    if (rc) return throw_qattn(env, rc, nullptr);
  }
  NAPI_OK(env, napi_create_typedarray(env, napi_int32_array, (size_t)n * 8, ab, 0, &arr));
  NAPI_OK(env, napi_create_object(env, &out));
  NAPI_OK(env, napi_set_named_property(env, out, "items", arr));
  NAPI_OK(env, napi_set_named_property(env, out, "info", info_object(env, i)));
  return out;
}

// planMask(L, mask, prefix, window) -> Uint32Array (host evaluation of the kernel iteration)
// debugMask(ctx, L, mask, prefix, window) -> Uint32Array (device)
napi_value MaskCommon(napi_env env, napi_callback_info info, bool device) {
  napi_value argv[5];
  const size_t want = device ? 5 : 4;
  if (!args_of(env, info, want, argv)) return nullptr;
  int off = device ? 1 : 0;
  int64_t L = 0, mask = 1, prefix = 176, window = 432;
  if (!get_i64(env, argv[off], &L) || !get_i64(env, argv[off + 1], &mask) ||
      !get_i64(env, argv[off + 2], &prefix) || !get_i64(env, argv[off + 3], &window) || L < 0) {
    napi_throw_type_error(env, nullptr, "expected (L, mask, prefix, window) numbers");
    return nullptr;
  }
  const size_t words = (size_t)((L + 31) / 32) * (size_t)L;
  napi_value ab, arr;
  void* data = nullptr;
  NAPI_OK(env, napi_create_arraybuffer(env, words * 4, &data, &ab));
  int rc;
  if (device) {
    Ctx* c = live_ctx(env, argv[0]);
    if (!c) return nullptr;
    rc = qattn_debug_mask(c->ctx, (int32_t)L, (int32_t)mask, (int32_t)prefix, (int32_t)window,
                          static_cast<uint32_t*>(data));
    if (rc) return throw_qattn(env, rc, c->ctx);
  } else {
    rc = qattn_plan_mask((int32_t)L, (int32_t)mask, (int32_t)prefix, (int32_t)window,
                         static_cast<uint32_t*>(data));
    if (rc) return throw_qattn(env, rc, nullptr);
  }
  NAPI_OK(env, napi_create_typedarray(env, napi_uint32_array, words, ab, 0, &arr));
  return arr;
}
napi_value PlanMask(napi_env env, napi_callback_info info) { return MaskCommon(env, info, false); }
napi_value DebugMask(napi_env env, napi_callback_info info) { return MaskCommon(env, info, true); }

// genQkv(ctx, config, layer, cuSeqlens, q, k, v)  (compact layouts)
napi_value GenQkv(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  if (!args_of(env, info, 7, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  int64_t config = 0, layer = 0;
  std::vector<int32_t> cu;
  if (!get_i64(env, argv[1], &config) || !get_i64(env, argv[2], &layer) ||
      !get_i32_array(env, argv[3], &cu) || cu.size() < 2) {
    napi_throw_type_error(env, nullptr, "expected (ctx, config, layer, cuSeqlens, q, k, v)");
    return nullptr;
  }
  Buf *q = live_buf(env, argv[4]), *k = q ? live_buf(env, argv[5]) : nullptr,
      *v = k ? live_buf(env, argv[6]) : nullptr;
  if (!v) return nullptr;
  const int64_t T = cu.back();
  if (T < 0 || (uint64_t)T * 4096 > q->bytes || (uint64_t)T * 2048 > k->bytes || (uint64_t)T * 2048 > v->bytes) {
    napi_throw_range_error(env, nullptr, "tokens x head widths exceed the q/k/v buffers");
    return nullptr;
  }
  int rc = qattn_gen_qkv(c->ctx, (uint32_t)config, (uint32_t)layer, cu.data(), (int32_t)cu.size() - 1,
                         q->ptr, 2048, k->ptr, 1024, v->ptr, 1024, nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// fillTokenRows(ctx, dst, ids(device buffer), rows, rowElems, rowStride, seedHi, seedLo)
napi_value FillTokenRows(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  if (!args_of(env, info, 8, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  Buf *dst = live_buf(env, argv[1]), *ids = dst ? live_buf(env, argv[2]) : nullptr;
  if (!ids) return nullptr;
  int64_t rows, elems, stride, hi, lo;
  if (!get_i64(env, argv[3], &rows) || !get_i64(env, argv[4], &elems) ||
      !get_i64(env, argv[5], &stride) || !get_i64(env, argv[6], &hi) || !get_i64(env, argv[7], &lo)) {
    napi_throw_type_error(env, nullptr, "expected numbers");
    return nullptr;
  }
  if (rows < 0 || elems < 0 || elems > stride || (size_t)rows * 4 > ids->bytes ||
      (rows > 0 && (size_t)((rows - 1) * stride + elems) * 2 > dst->bytes)) {
    napi_throw_range_error(env, nullptr, "rows exceed the buffers");
    return nullptr;
  }
  const uint64_t seed = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
  int rc = qattn_fill_token_rows(c->ctx, dst->ptr, static_cast<const int32_t*>(ids->ptr), rows,
                                 elems, stride, seed, nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// qkNormRope(ctx, x, rowStride, col0, heads, cuSeqlens, eps, theta)
// qkNormRopeQkv(ctx, qkv, qkvStride, q, qStride, k, kStride, cuSeqlens, eps, theta)
// (reference: QKNormRopeKernel.createRun + dispatch, ops.ts:104-166; unit gains)
napi_value QkNormRopeQkv(napi_env env, napi_callback_info info) {
  napi_value argv[10];
  if (!args_of(env, info, 10, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  Buf* qkv = live_buf(env, argv[1]);
  Buf* q = qkv ? live_buf(env, argv[3]) : nullptr;
  Buf* k = q ? live_buf(env, argv[5]) : nullptr;
  if (!k) return nullptr;
  int64_t s_qkv, s_q, s_k;
  double eps = 1e-6, theta = 1e6;
  std::vector<int32_t> cu;
  if (!get_i64(env, argv[2], &s_qkv) || !get_i64(env, argv[4], &s_q) || !get_i64(env, argv[6], &s_k) ||
      !get_i32_array(env, argv[7], &cu) || cu.size() < 2 || napi_get_value_double(env, argv[8], &eps) != napi_ok ||
      napi_get_value_double(env, argv[9], &theta) != napi_ok) {
    napi_throw_type_error(env, nullptr,
                          "expected (ctx, qkv, qkvStride, q, qStride, k, kStride, cuSeqlens, eps, theta)");
    return nullptr;
  }
  const int64_t T = cu.back();
  auto fits = [&](const Buf* b, int64_t stride, int64_t width) {
    return stride >= width && (T <= 0 || (uint64_t)((T - 1) * stride + width) * 2 <= b->bytes);
  };
  if (!fits(qkv, s_qkv, 3072) || !fits(q, s_q, 2048) || !fits(k, s_k, 1024)) {
    napi_throw_range_error(env, nullptr, "rows x stride exceed a device buffer");
    return nullptr;
  }
  int rc = qattn_qk_norm_rope_qkv(c->ctx, qkv->ptr, s_qkv, q->ptr, s_q, k->ptr, s_k, cu.data(),
                                  (int32_t)cu.size() - 1, nullptr, nullptr, eps, theta, nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

napi_value QkNormRope(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  if (!args_of(env, info, 8, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  Buf* x = live_buf(env, argv[1]);
  if (!x) return nullptr;
  int64_t stride, col0, heads;
  double eps = 1e-6, theta = 1e6;
  std::vector<int32_t> cu;
  if (!get_i64(env, argv[2], &stride) || !get_i64(env, argv[3], &col0) ||
      !get_i64(env, argv[4], &heads) || !get_i32_array(env, argv[5], &cu) || cu.size() < 2 ||
      napi_get_value_double(env, argv[6], &eps) != napi_ok ||
      napi_get_value_double(env, argv[7], &theta) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected (ctx, x, rowStride, col0, heads, cuSeqlens, eps, theta)");
    return nullptr;
  }
  if ((size_t)cu.back() * (size_t)stride * 2 > x->bytes) {
    napi_throw_range_error(env, nullptr, "rows exceed the buffer");
    return nullptr;
  }
  int rc = qattn_qk_norm_rope(c->ctx, x->ptr, stride, col0, (int32_t)heads, cu.data(),
                              (int32_t)cu.size() - 1, nullptr, eps, theta, nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// q4Matmul(ctx, x, ldx, rows, k, w, wBytes, n, y, ldy): y = x W^T over a tile32-compact Q4_0
// tensor (qattn_q4_matmul).
napi_value Q4Matmul(napi_env env, napi_callback_info info) {
  napi_value argv[10];
  if (!args_of(env, info, 10, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  Buf* x = live_buf(env, argv[1]);
  Buf* w = x ? live_buf(env, argv[5]) : nullptr;
  Buf* y = w ? live_buf(env, argv[8]) : nullptr;
  if (!y) return nullptr;
  int64_t ldx, rows, k, wbytes, n, ldy;
  if (!get_i64(env, argv[2], &ldx) || !get_i64(env, argv[3], &rows) || !get_i64(env, argv[4], &k) ||
      !get_i64(env, argv[6], &wbytes) || !get_i64(env, argv[7], &n) || !get_i64(env, argv[9], &ldy) || rows < 0 ||
      rows > INT32_MAX || k < 0 || k > INT32_MAX || n < 0 || n > INT32_MAX) {
    napi_throw_type_error(env, nullptr, "expected (ctx, x, ldx, rows, k, w, wBytes, n, y, ldy)");
    return nullptr;
  }
  if ((size_t)rows * (size_t)ldx * 2 > x->bytes || (size_t)rows * (size_t)ldy * 2 > y->bytes || (size_t)wbytes > w->bytes) {
    napi_throw_range_error(env, nullptr, "rows exceed the buffers");
    return nullptr;
  }
  int rc = qattn_q4_matmul(c->ctx, x->ptr, ldx, (int32_t)rows, (int32_t)k, w->ptr, wbytes, (int32_t)n, y->ptr, ldy,
                           nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// poolLastL2(ctx, x, rowStride, width, cuSeqlens, out): out (f32 rows of `width`) receives the
// L2-normalised last row of each sequence of x (fp16 rows of rowStride elements).
napi_value PoolLastL2(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!args_of(env, info, 6, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  Buf* x = live_buf(env, argv[1]);
  if (!x) return nullptr;
  Buf* out = live_buf(env, argv[5]);
  if (!out) return nullptr;
  int64_t stride, width;
  std::vector<int32_t> cu;
  if (!get_i64(env, argv[2], &stride) || !get_i64(env, argv[3], &width) || !get_i32_array(env, argv[4], &cu) ||
      cu.size() < 2 || width < 1 || width > INT32_MAX) {
    napi_throw_type_error(env, nullptr, "expected (ctx, x, rowStride, width, cuSeqlens, out)");
    return nullptr;
  }
  if ((size_t)cu.back() * (size_t)stride * 2 > x->bytes || (cu.size() - 1) * (size_t)width * 4 > out->bytes) {
    napi_throw_range_error(env, nullptr, "rows exceed the buffers");
    return nullptr;
  }
  int rc = qattn_pool_last_l2(c->ctx, x->ptr, stride, (int32_t)width, cu.data(), (int32_t)cu.size() - 1,
                              static_cast<float*>(out->ptr), width, nullptr);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// ---- the model forward (Qwen3WebGPUModel / Qwen3ExecutionPlan, model.ts:49-255) --------------

void drop_model_plans(Model* m) {
  for (Plan* p : m->plans) {
    if (p->plan) qattn_model_plan_destroy(p->plan);
    p->plan = nullptr;
    p->model = nullptr;
  }
  m->plans.clear();
}
void finalize_model(napi_env env, void* data, void*) {
  auto* m = static_cast<Model*>(data);
  Ctx* c = m->owner;
  if (c->ctx) {
    drop_model_plans(m);
    if (m->model) qattn_model_destroy(m->model);
  }
  for (napi_ref ref : m->bound_refs) napi_delete_reference(env, ref);
  for (Plan* p : m->plans) p->model = nullptr;
  c->models.erase(m);
  delete m;
  unref(c);
}
void finalize_plan(napi_env env, void* data, void*) {
  auto* p = static_cast<Plan*>(data);
  Ctx* c = p->owner;
  if (p->plan && c->ctx) qattn_model_plan_destroy(p->plan);
  if (p->model) p->model->plans.erase(p);
  if (p->model_ref) napi_delete_reference(env, p->model_ref);
  c->plans.erase(p);
  delete p;
  unref(c);
}

// createModel(ctx, {tokenEmbd, outputNorm, layers: [{attnNorm, attnQkv, attnQNorm, attnKNorm,
// attnOutput, ffnNorm, ffnGateUp, ffnDown}], eps, ropeTheta, mask, prefix, window, batchInvariant})
// -> external.  Every tensor is a device buffer of this context holding exactly that tensor's
// bytes (a compact projection's size is its buffer's); norm gains must hold their width of f32.
napi_value CreateModel(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args_of(env, info, 2, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  napi_value d = argv[1], v;
  std::vector<napi_value> bound;
  auto tensor = [&](napi_value obj, const char* name, size_t min_bytes, const void** ptr, int64_t* bytes) {
    if (!prop(env, obj, name, &v)) {
      napi_throw_type_error(env, nullptr, (std::string("missing ") + name).c_str());
      return false;
    }
    Buf* b = live_buf(env, v);
    if (!b) return false;
    if (b->owner != c) {
      napi_throw_error(env, nullptr, (std::string(name) + " belongs to another context").c_str());
      return false;
    }
    if (b->bytes < min_bytes) {
      napi_throw_range_error(env, nullptr, (std::string(name) + " is smaller than its tensor").c_str());
      return false;
    }
    *ptr = b->ptr;
    if (bytes) *bytes = (int64_t)b->bytes;
    bound.push_back(v);
    return true;
  };
  auto num = [&](const char* name, double dflt) {
    double x = dflt;
    if (prop(env, d, name, &v)) napi_get_value_double(env, v, &x);
    return x;
  };
  qattn_model_desc desc{};
  const void* p = nullptr;
  if (!tensor(d, "tokenEmbd", 0, &desc.token_embd, &desc.token_embd_bytes)) return nullptr;
  if (!tensor(d, "outputNorm", 1024 * 4, &p, nullptr)) return nullptr;
  desc.output_norm = static_cast<const float*>(p);
  napi_value layers;
  bool is_arr = false;
  if (!prop(env, d, "layers", &layers) || napi_is_array(env, layers, &is_arr) != napi_ok || !is_arr) {
    napi_throw_type_error(env, nullptr, "layers must be an array");
    return nullptr;
  }
  uint32_t n = 0;
  napi_get_array_length(env, layers, &n);
  std::vector<qattn_layer_weights> lw(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value l;
    NAPI_OK(env, napi_get_element(env, layers, i, &l));
    qattn_layer_weights& w = lw[i];
    const void *an, *qn, *kn, *fn;
    if (!tensor(l, "attnNorm", 1024 * 4, &an, nullptr) || !tensor(l, "attnQNorm", 128 * 4, &qn, nullptr) ||
        !tensor(l, "attnKNorm", 128 * 4, &kn, nullptr) || !tensor(l, "ffnNorm", 1024 * 4, &fn, nullptr) ||
        !tensor(l, "attnQkv", 0, &w.attn_qkv, &w.attn_qkv_bytes) ||
        !tensor(l, "attnOutput", 0, &w.attn_output, &w.attn_output_bytes) ||
        !tensor(l, "ffnGateUp", 0, &w.ffn_gate_up, &w.ffn_gate_up_bytes) ||
        !tensor(l, "ffnDown", 0, &w.ffn_down, &w.ffn_down_bytes))
      return nullptr;
    w.attn_norm = static_cast<const float*>(an);
    w.attn_q_norm = static_cast<const float*>(qn);
    w.attn_k_norm = static_cast<const float*>(kn);
    w.ffn_norm = static_cast<const float*>(fn);
  }
  desc.n_layers = (int32_t)n;
  desc.layers = lw.data();
  desc.eps = num("eps", 1e-6);
  desc.rope_theta = num("ropeTheta", 1e6);
  desc.mask = (int32_t)num("mask", QATTN_MASK_PREFIX_LOCAL);
  desc.prefix = (int32_t)num("prefix", 176);
  desc.window = (int32_t)num("window", 432);
  bool invariant = true;
  if (prop(env, d, "batchInvariant", &v)) napi_get_value_bool(env, v, &invariant);
  desc.flags = invariant ? QATTN_FLAG_BATCH_INVARIANT : 0;
  qattn_model* model = nullptr;
  int rc = qattn_model_create(c->ctx, &desc, &model);
  if (rc) return throw_qattn(env, rc, c->ctx);
  auto* m = new Model{c, model, {}, {}};
  for (napi_value b : bound) {
    napi_ref ref;
    NAPI_OK(env, napi_create_reference(env, b, 1, &ref));
    m->bound_refs.push_back(ref);
  }
  c->models.insert(m);
  ++c->refs;
  napi_value out;
  NAPI_OK(env, napi_create_external(env, m, finalize_model, nullptr, &out));
  return out;
}

Model* live_model(napi_env env, napi_value v) {
  Model* m = get_external<Model>(env, v, "model");
  if (m && (!m->model || !m->owner->ctx)) {
    napi_throw_error(env, nullptr, "model was destroyed");
    return nullptr;
  }
  return m;
}

napi_value DestroyModel(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Model* m = get_external<Model>(env, argv[0], "model");
  if (!m) return nullptr;
  if (m->owner->ctx) {
    drop_model_plans(m);
    if (m->model) qattn_model_destroy(m->model);
  }
  m->model = nullptr;
  return undefined(env);
}

// createModelPlan(model, maxTokens, maxSeqs) -> external
napi_value CreateModelPlan(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args_of(env, info, 3, argv)) return nullptr;
  Model* m = live_model(env, argv[0]);
  if (!m) return nullptr;
  int64_t max_tokens = 0, max_seqs = 0;
  if (!get_i64(env, argv[1], &max_tokens) || !get_i64(env, argv[2], &max_seqs) || max_tokens < 1 ||
      max_tokens > INT32_MAX || max_seqs < 1 || max_seqs > QATTN_MAX_SEQS) {
    napi_throw_range_error(env, nullptr, "maxTokens / maxSeqs out of range");
    return nullptr;
  }
  qattn_model_plan* plan = nullptr;
  int rc = qattn_model_plan_create(m->model, (int32_t)max_tokens, (int32_t)max_seqs, &plan);
  if (rc) return throw_qattn(env, rc, m->owner->ctx);
  auto* p = new Plan{m->owner, m, plan, nullptr, max_tokens, max_seqs};
  NAPI_OK(env, napi_create_reference(env, argv[0], 1, &p->model_ref));
  m->plans.insert(p);
  m->owner->plans.insert(p);
  ++m->owner->refs;
  napi_value out;
  NAPI_OK(env, napi_create_external(env, p, finalize_plan, nullptr, &out));
  return out;
}

Plan* live_plan(napi_env env, napi_value v) {
  Plan* p = get_external<Plan>(env, v, "model plan");
  if (p && (!p->plan || !p->owner->ctx)) {
    napi_throw_error(env, nullptr, "model plan was destroyed");
    return nullptr;
  }
  return p;
}

napi_value DestroyModelPlan(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Plan* p = get_external<Plan>(env, argv[0], "model plan");
  if (!p) return nullptr;
  if (p->plan && p->owner->ctx) qattn_model_plan_destroy(p->plan);
  p->plan = nullptr;
  return undefined(env);
}

// runModelPlan(plan, ids, cuSeqlens, out) / profileModelPlan(...) -> {stage: ms}: one packed batch
// (ids Int32Array / Uint32Array of cuSeqlens[nseq] token ids) into the f32 [nseq][1024] device
// buffer `out`; enqueued on the context stream (profile waits for it).
napi_value ModelPlanCommon(napi_env env, napi_callback_info info, bool profile) {
  napi_value argv[4];
  if (!args_of(env, info, 4, argv)) return nullptr;
  Plan* p = live_plan(env, argv[0]);
  if (!p) return nullptr;
  std::vector<int32_t> ids, cu;
  if (!get_i32_array(env, argv[1], &ids) || !get_i32_array(env, argv[2], &cu) || cu.size() < 2) {
    napi_throw_type_error(env, nullptr, "ids and cuSeqlens must be Int32Array / Uint32Array / arrays");
    return nullptr;
  }
  Buf* out = live_buf(env, argv[3]);
  if (!out) return nullptr;
  const int64_t nseq = (int64_t)cu.size() - 1;
  if (out->owner != p->owner || out->bytes < (size_t)nseq * 1024 * 4) {
    napi_throw_range_error(env, nullptr, "out must be a buffer of this context holding nseq x 1024 f32");
    return nullptr;
  }
  if (cu.back() < 0 || (size_t)cu.back() > ids.size()) {
    napi_throw_range_error(env, nullptr, "ids holds fewer tokens than cuSeqlens[nseq]");
    return nullptr;
  }
  qattn_ctx* ctx = p->owner->ctx;
  if (!profile) {
    int rc = qattn_model_plan_run(p->plan, ids.data(), cu.data(), (int32_t)nseq, static_cast<float*>(out->ptr), 1024,
                                  nullptr);
    if (rc) return throw_qattn(env, rc, ctx);
    return undefined(env);
  }
  float ms[QATTN_STAGE_COUNT];
  int rc = qattn_model_plan_profile(p->plan, ids.data(), cu.data(), (int32_t)nseq, static_cast<float*>(out->ptr), 1024,
                                    nullptr, ms);
  if (rc) return throw_qattn(env, rc, ctx);
  static const char* names[QATTN_STAGE_COUNT] = {"embedding_norm",      "qkv",         "rope_attention",
                                                 "attention_output",    "post_attention_norm",
                                                 "ffn_up_gate",         "swiglu",      "ffn_down",
                                                 "post_ffn_norm",       "pool"};
  napi_value o;
  NAPI_OK(env, napi_create_object(env, &o));
  for (int s = 0; s < QATTN_STAGE_COUNT; ++s) {
    napi_value x;
    NAPI_OK(env, napi_create_double(env, ms[s], &x));
    NAPI_OK(env, napi_set_named_property(env, o, names[s], x));
  }
  return o;
}
napi_value RunModelPlan(napi_env env, napi_callback_info info) { return ModelPlanCommon(env, info, false); }
napi_value ProfileModelPlan(napi_env env, napi_callback_info info) { return ModelPlanCommon(env, info, true); }

napi_value Synchronize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  int rc = qattn_synchronize(c->ctx);
  if (rc) return throw_qattn(env, rc, c->ctx);
  return undefined(env);
}

// synchronizeAsync(ctx) -> Promise<void>: waits for the context stream off the JS thread.
struct SyncWork {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  Ctx* owner = nullptr;
  qattn_ctx* ctx = nullptr;
  int rc = 0;
  std::string msg;
};
void sync_execute(napi_env, void* data) {
  auto* w = static_cast<SyncWork*>(data);
  w->rc = qattn_synchronize(w->ctx);
  if (w->rc) w->msg = qattn_last_error(w->ctx);
}
void sync_complete(napi_env env, napi_status, void* data) {
  auto* w = static_cast<SyncWork*>(data);
  if (w->rc == 0) {
    napi_resolve_deferred(env, w->deferred, undefined(env));
  } else {
    napi_value m, e;
    std::string s = "qattn error " + std::to_string(w->rc) + ": " + w->msg;
    napi_create_string_utf8(env, s.c_str(), NAPI_AUTO_LENGTH, &m);
    napi_create_error(env, nullptr, m, &e);
    napi_reject_deferred(env, w->deferred, e);
  }
  napi_delete_async_work(env, w->work);
  --w->owner->async_busy;
  unref(w->owner);
  delete w;
}
napi_value SynchronizeAsync(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  auto* w = new SyncWork();
  w->owner = c;
  w->ctx = c->ctx;
  ++c->refs;
  ++c->async_busy;
  napi_value promise, name;
  NAPI_OK(env, napi_create_promise(env, &w->deferred, &promise));
  NAPI_OK(env, napi_create_string_utf8(env, "qattn.synchronize", NAPI_AUTO_LENGTH, &name));
  NAPI_OK(env, napi_create_async_work(env, nullptr, name, sync_execute, sync_complete, w, &w->work));
  NAPI_OK(env, napi_queue_async_work(env, w->work));
  return promise;
}

// createEvent(ctx) / recordEvent(ev) (on the context stream) / destroyEvent(ev).
void finalize_evt(napi_env, void* data, void*) {
  auto* e = static_cast<Evt*>(data);
  Ctx* c = e->owner;
  if (e->ev && c->ctx) qattn_event_destroy(e->ev);
  c->evts.erase(e);
  delete e;
  unref(c);
}
napi_value CreateEvent(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Ctx* c = live_ctx(env, argv[0]);
  if (!c) return nullptr;
  qattn_event_t ev = nullptr;
  int rc = qattn_event_create(c->ctx, &ev);
  if (rc) return throw_qattn(env, rc, c->ctx);
  auto* e = new Evt{c, ev};
  c->evts.insert(e);
  ++c->refs;
  napi_value out;
  NAPI_OK(env, napi_create_external(env, e, finalize_evt, nullptr, &out));
  return out;
}
Evt* live_evt(napi_env env, napi_value v) {
  Evt* e = get_external<Evt>(env, v, "event");
  if (e && (!e->ev || e->destroy_pending || !e->owner->ctx)) {
    napi_throw_error(env, nullptr, "event was destroyed");
    return nullptr;
  }
  return e;
}
napi_value RecordEvent(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Evt* e = live_evt(env, argv[0]);
  if (!e) return nullptr;
  int rc = qattn_event_record(e->ev, qattn_stream(e->owner->ctx));
  if (rc) return throw_qattn(env, rc, e->owner->ctx);
  return undefined(env);
}
napi_value DestroyEvent(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args_of(env, info, 1, argv)) return nullptr;
  Evt* e = get_external<Evt>(env, argv[0], "event");
  if (!e) return nullptr;
  if (e->waiters > 0) {
    e->destroy_pending = true;
  } else if (e->ev && e->owner->ctx) {
    qattn_event_destroy(e->ev);
    e->ev = nullptr;
  }
  return undefined(env);
}

// readAfterAsync(buf, ev, dst) -> Promise<dst>: the readback of one submit -- dst (a typed array,
// at most the buffer's size) receives the buffer's first dst.byteLength bytes once the work
// recorded before ev has finished, copied on the context's readback stream by a worker thread
// (qattn_buffer_read_after), so batches enqueued after ev are not waited for.  The buffer, the
// event and dst stay referenced until the promise settles.
struct ReadWork {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  napi_ref buf_ref = nullptr, evt_ref = nullptr, dst_ref = nullptr;
  Buf* buf = nullptr;  // kept alive by buf_ref
  Evt* evt = nullptr;
  qattn_ctx* ctx = nullptr;
  const void* src = nullptr;
  void* dst = nullptr;
  size_t bytes = 0;
  int rc = 0;
  std::string msg;
};
void read_execute(napi_env, void* data) {
  auto* w = static_cast<ReadWork*>(data);
  w->rc = qattn_buffer_read_after(w->ctx, w->evt->ev, w->src, 0, w->dst, w->bytes);
  if (w->rc) w->msg = qattn_last_error(w->ctx);
}
void read_complete(napi_env env, napi_status, void* data) {
  auto* w = static_cast<ReadWork*>(data);
  Evt* e = w->evt;
  if (--e->waiters == 0 && e->destroy_pending && e->ev && e->owner->ctx) {
    qattn_event_destroy(e->ev);
    e->ev = nullptr;
  }
  if (w->rc == 0) {
    napi_value dst;
    napi_get_reference_value(env, w->dst_ref, &dst);
    napi_resolve_deferred(env, w->deferred, dst);
  } else {
    napi_value m, err;
    std::string s = "qattn error " + std::to_string(w->rc) + ": " + w->msg;
    napi_create_string_utf8(env, s.c_str(), NAPI_AUTO_LENGTH, &m);
    napi_create_error(env, nullptr, m, &err);
    napi_reject_deferred(env, w->deferred, err);
  }
  --w->buf->reads_in_flight;
  napi_delete_reference(env, w->buf_ref);
  napi_delete_reference(env, w->evt_ref);
  napi_delete_reference(env, w->dst_ref);
  napi_delete_async_work(env, w->work);
  --e->owner->async_busy;
  unref(e->owner);
  delete w;
}
napi_value ReadAfterAsync(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args_of(env, info, 3, argv)) return nullptr;
  Buf* b = live_buf(env, argv[0]);
  if (!b) return nullptr;
  Evt* e = live_evt(env, argv[1]);
  if (!e) return nullptr;
  if (e->owner != b->owner) {
    napi_throw_error(env, nullptr, "buffer and event belong to different contexts");
    return nullptr;
  }
  bool is_typed = false;
  napi_is_typedarray(env, argv[2], &is_typed);
  if (!is_typed) {
    napi_throw_type_error(env, nullptr, "dst must be a typed array");
    return nullptr;
  }
  napi_typedarray_type type;
  size_t length = 0, byte_offset = 0;
  void* data = nullptr;
  napi_value ab;
  NAPI_OK(env, napi_get_typedarray_info(env, argv[2], &type, &length, &data, &ab, &byte_offset));
  size_t elem = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: elem = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
    default: elem = 1;
  }
  const size_t bytes = length * elem;
  if (bytes > b->bytes) {
    napi_throw_range_error(env, nullptr, "dst is larger than the buffer");
    return nullptr;
  }
  auto* w = new ReadWork();
  w->buf = b;
  w->evt = e;
  w->ctx = b->owner->ctx;
  w->src = b->ptr;
  w->dst = data;
  w->bytes = bytes;
  NAPI_OK(env, napi_create_reference(env, argv[0], 1, &w->buf_ref));
  NAPI_OK(env, napi_create_reference(env, argv[1], 1, &w->evt_ref));
  NAPI_OK(env, napi_create_reference(env, argv[2], 1, &w->dst_ref));
  ++e->waiters;
  ++b->reads_in_flight;
  ++b->owner->refs;  // the context outlives the wait
  ++b->owner->async_busy;
  napi_value promise, name;
  NAPI_OK(env, napi_create_promise(env, &w->deferred, &promise));
  NAPI_OK(env, napi_create_string_utf8(env, "qattn.readAfter", NAPI_AUTO_LENGTH, &name));
  NAPI_OK(env, napi_create_async_work(env, nullptr, name, read_execute, read_complete, w, &w->work));
  NAPI_OK(env, napi_queue_async_work(env, w->work));
  return promise;
}

napi_value AbiVersion(napi_env env, napi_callback_info) {
  napi_value v;
  napi_create_int32(env, qattn_abi_version(), &v);
  return v;
}

napi_value Init(napi_env env, napi_value exports) {
  struct Fn {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"abiVersion", AbiVersion},     {"createContext", CreateContext},
      {"destroyContext", DestroyContext}, {"deviceName", DeviceName},
      {"alloc", Alloc},               {"free", Free},
      {"write", Write},               {"read", Read},
      {"createRun", CreateRun},       {"encode", Encode},
      {"destroyRun", DestroyRun},     {"runInfo", RunInfo},
      {"planDescribe", PlanDescribe}, {"planMask", PlanMask},
      {"debugMask", DebugMask},       {"genQkv", GenQkv},
      {"fillTokenRows", FillTokenRows}, {"qkNormRope", QkNormRope},
      {"qkNormRopeQkv", QkNormRopeQkv}, {"updateRun", UpdateRun},
      {"poolLastL2", PoolLastL2},     {"q4Matmul", Q4Matmul},
      {"synchronize", Synchronize},   {"synchronizeAsync", SynchronizeAsync},
      {"createModel", CreateModel},   {"destroyModel", DestroyModel},
      {"createModelPlan", CreateModelPlan}, {"destroyModelPlan", DestroyModelPlan},
      {"runModelPlan", RunModelPlan}, {"profileModelPlan", ProfileModelPlan},
      {"createEvent", CreateEvent},   {"recordEvent", RecordEvent},
      {"destroyEvent", DestroyEvent}, {"readAfterAsync", ReadAfterAsync},
  };
  for (const Fn& f : fns) {
    napi_value fn;
    NAPI_OK(env, napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn));
    NAPI_OK(env, napi_set_named_property(env, exports, f.name, fn));
  }
  return exports;
}

}  // namespace

NAPI_MODULE(qattn_napi, Init)
