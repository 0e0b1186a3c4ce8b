/*
 * addon.c -- N-API binding of the q4hip C ABI for the Node.js backend (engine/hip.js).
 *
 * Thin by design: every function converts JavaScript arguments to the C ABI's plain pointers and
 * sizes, calls it, and turns a non-zero status into a thrown Error whose message is
 * q4hip_last_error() and whose `code` is the status.  Calls are synchronous; the JavaScript layer
 * keeps the reference backend's async surface (engine/cpu.js:55-62) on top.
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q4hip.h"

#define NAPI_CALL(env, call)                                          \
  do {                                                                \
    if ((call) != napi_ok) {                                          \
      napi_throw_error((env), NULL, "N-API call failed: " #call);     \
      return NULL;                                                    \
    }                                                                 \
  } while (0)

static napi_value throw_status(napi_env env, int rc) {
  char code[16];
  snprintf(code, sizeof code, "%d", rc);
  napi_throw_error(env, code, q4hip_last_error());
  return NULL;
}

static int get_i32(napi_env env, napi_value v, int32_t* out) {
  return napi_get_value_int32(env, v, out) == napi_ok;
}

/* A context handle is an external over a ctx_slot; its batches are listed there so that
 * destroy() (or the finalizer) releases them first, as q4hip_batch_destroy must precede
 * q4hip_destroy.  A released batch keeps its slot with bt = NULL, and calls on it throw. */
typedef struct batch_slot batch_slot;
typedef struct ctx_slot {
  q4hip* h;
  int head_dim, vocab;
  batch_slot* batches;
} ctx_slot;
struct batch_slot {
  q4hip_batch* bt;
  int B;
  ctx_slot* ctx;      /* NULL once the context is gone */
  batch_slot* next;
};

static void release_batches(ctx_slot* c) {
  for (batch_slot* b = c->batches; b; b = b->next) {
    if (b->bt) q4hip_batch_destroy(b->bt);
    b->bt = NULL;
    b->ctx = NULL;
  }
  c->batches = NULL;
}

static void unlink_batch(batch_slot* b) {
  if (!b->ctx) return;
  for (batch_slot** q = &b->ctx->batches; *q; q = &(*q)->next)
    if (*q == b) { *q = b->next; break; }
  b->ctx = NULL;
}

static ctx_slot* get_slot(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip handle");
    return NULL;
  }
  ctx_slot* c = (ctx_slot*)p;
  if (!c->h) {
    napi_throw_error(env, "5", "context destroyed");
    return NULL;
  }
  return c;
}

static q4hip* get_handle(napi_env env, napi_value v) {
  ctx_slot* c = get_slot(env, v);
  return c ? c->h : NULL;
}

static batch_slot* get_batch(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip batch handle");
    return NULL;
  }
  batch_slot* b = (batch_slot*)p;
  if (!b->bt) {
    napi_throw_error(env, "5", "batch destroyed (or its context)");
    return NULL;
  }
  return b;
}

/* Borrow the bytes of a TypedArray, DataView, Buffer or ArrayBuffer. */
static int get_bytes(napi_env env, napi_value v, void** data, size_t* len) {
  bool is;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type t;
    size_t n, off;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &t, &n, data, &ab, &off) != napi_ok) return 0;
    static const size_t sz[] = {1, 1, 1, 2, 2, 4, 4, 4, 8, 8, 8};
    *len = n * (t <= napi_biguint64_array ? sz[t] : 1);
    return 1;
  }
  if (napi_is_dataview(env, v, &is) == napi_ok && is) {
    napi_value ab;
    size_t off;
    return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is)
    return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
  return 0;
}

static void finalize_handle(napi_env env, void* data, void* hint) {
  (void)env; (void)hint;
  ctx_slot* c = (ctx_slot*)data;
  release_batches(c);
  if (c->h) q4hip_destroy(c->h);
  free(c);
}

static void finalize_batch(napi_env env, void* data, void* hint) {
  (void)env; (void)hint;
  batch_slot* b = (batch_slot*)data;
  if (b->bt) q4hip_batch_destroy(b->bt);
  unlink_batch(b);
  free(b);
}

/* create(dim, layers, ffn, heads, kvHeads, vocab, ctx, mt, eps, device[, kvType]) -> handle;
 * kvType 0 (fp32, the default) or 1 (fp16). */
static napi_value js_create(napi_env env, napi_callback_info info) {
  size_t argc = 11;
  napi_value a[11];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 10) { napi_throw_type_error(env, NULL, "create: 10 arguments"); return NULL; }
  int32_t v[8], dev, kvt = Q4HIP_KV_F32;
  double eps;
  for (int i = 0; i < 8; i++)
    if (!get_i32(env, a[i], &v[i])) { napi_throw_type_error(env, NULL, "create: integer expected"); return NULL; }
  if (napi_get_value_double(env, a[8], &eps) != napi_ok || !get_i32(env, a[9], &dev) ||
      (argc > 10 && !get_i32(env, a[10], &kvt))) {
    napi_throw_type_error(env, NULL, "create: eps, device and kvType expected");
    return NULL;
  }
  q4hip* h = NULL;
  int rc = q4hip_create(&h, v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], (float)eps, dev, kvt);
  if (rc) return throw_status(env, rc);
  ctx_slot* slot = (ctx_slot*)calloc(1, sizeof *slot);
  if (!slot) { q4hip_destroy(h); napi_throw_error(env, NULL, "out of memory"); return NULL; }
  slot->h = h;
  slot->head_dim = v[0] / v[3];
  slot->vocab = v[5];
  napi_value out;
  if (napi_create_external(env, slot, finalize_handle, NULL, &out) != napi_ok) {
    q4hip_destroy(h);
    free(slot);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  return out;
}

/* destroy(handle): frees device memory now (the context's batches first); later calls on the
 * handle or its batches throw. */
static napi_value js_destroy(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value a[1];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  void* p = NULL;
  if (argc < 1 || napi_get_value_external(env, a[0], &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip handle");
    return NULL;
  }
  ctx_slot* c = (ctx_slot*)p;
  release_batches(c);
  if (c->h) { q4hip_destroy(c->h); c->h = NULL; }
  return NULL;
}

/* setTensor(handle, kind, layer, row0, ggmlType, bytes, rows) */
static napi_value js_set_tensor(napi_env env, napi_callback_info info) {
  size_t argc = 7;
  napi_value a[7];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 7) { napi_throw_type_error(env, NULL, "setTensor: 7 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  int32_t kind, layer, row0, type;
  double rows;
  void* data;
  size_t len;
  if (!get_i32(env, a[1], &kind) || !get_i32(env, a[2], &layer) || !get_i32(env, a[3], &row0) ||
      !get_i32(env, a[4], &type) || napi_get_value_double(env, a[6], &rows) != napi_ok) {
    napi_throw_type_error(env, NULL, "setTensor: bad arguments");
    return NULL;
  }
  if (!get_bytes(env, a[5], &data, &len)) { napi_throw_type_error(env, NULL, "setTensor: bytes expected"); return NULL; }
  int rc = q4hip_set_tensor(h, kind, layer, row0, type, data, (int64_t)rows, len);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* setRope(handle, Float32Array table): the library checks the table's float count against
 * ctx * head_dim and reads nothing from a shorter one. */
static napi_value js_set_rope(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value a[2];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 2) { napi_throw_type_error(env, NULL, "setRope: 2 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  void* data;
  size_t len;
  if (!get_bytes(env, a[1], &data, &len)) {
    napi_throw_type_error(env, NULL, "setRope: Float32Array expected");
    return NULL;
  }
  int rc = q4hip_set_rope(h, (const float*)data, (int64_t)(len / 4));
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* forward(handle, Int32Array ids, pos) -> next id */
static napi_value js_forward(napi_env env, napi_callback_info info) {
  size_t argc = 3;
  napi_value a[3];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 3) { napi_throw_type_error(env, NULL, "forward: 3 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  void* data;
  size_t len;
  int32_t pos;
  if (!get_bytes(env, a[1], &data, &len) || !get_i32(env, a[2], &pos)) {
    napi_throw_type_error(env, NULL, "forward: (handle, Int32Array, pos) expected");
    return NULL;
  }
  int next = 0;
  int rc = q4hip_forward(h, (const int*)data, (int)(len / 4), pos, &next);
  if (rc) return throw_status(env, rc);
  napi_value out;
  NAPI_CALL(env, napi_create_int32(env, next, &out));
  return out;
}

/* readLogits(handle, Float32Array out) */
static napi_value js_read_logits(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value a[2];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 2) { napi_throw_type_error(env, NULL, "readLogits: 2 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  void* data;
  size_t len;
  if (!get_bytes(env, a[1], &data, &len)) { napi_throw_type_error(env, NULL, "readLogits: Float32Array expected"); return NULL; }
  int rc = q4hip_read_logits(h, (float*)data, (int)(len / 4));
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* generate(handle, first, pos, Int32Array out) -> fills out (length = steps) */
static napi_value js_generate(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value a[4];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 4) { napi_throw_type_error(env, NULL, "generate: 4 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  int32_t first, pos;
  void* data;
  size_t len;
  if (!get_i32(env, a[1], &first) || !get_i32(env, a[2], &pos) || !get_bytes(env, a[3], &data, &len)) {
    napi_throw_type_error(env, NULL, "generate: bad arguments");
    return NULL;
  }
  int rc = q4hip_generate(h, first, pos, (int)(len / 4), (int*)data);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* profile(handle, token, pos, Float32Array out[Q4HIP_PROF_N]) */
static napi_value js_profile(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value a[4];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 4) { napi_throw_type_error(env, NULL, "profile: 4 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  int32_t token, pos;
  void* data;
  size_t len;
  if (!get_i32(env, a[1], &token) || !get_i32(env, a[2], &pos) || !get_bytes(env, a[3], &data, &len)) {
    napi_throw_type_error(env, NULL, "profile: bad arguments");
    return NULL;
  }
  int rc = q4hip_profile(h, token, pos, (float*)data, (int)(len / 4));
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* setKv(handle, layer, kvHead, pos0, Float32Array k, Float32Array v): n = k.length / head_dim rows
 * of K and of V at positions pos0.. (q4hip_set_kv); k and v must hold whole rows, equally many. */
static int kv_rows(napi_env env, int head_dim, napi_value kv, napi_value vv, void** k, void** v, int* n) {
  size_t kl, vl;
  if (!get_bytes(env, kv, k, &kl) || !get_bytes(env, vv, v, &vl)) {
    napi_throw_type_error(env, NULL, "setKv: Float32Array K and V expected");
    return 0;
  }
  size_t row = (size_t)head_dim * 4;
  if (kl != vl || kl % row || kl / row > 0x7fffffff) {
    napi_throw_range_error(env, NULL, "setKv: K and V must be the same whole number of head_dim rows");
    return 0;
  }
  *n = (int)(kl / row);
  return 1;
}

static napi_value js_set_kv(napi_env env, napi_callback_info info) {
  size_t argc = 6;
  napi_value a[6];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 6) { napi_throw_type_error(env, NULL, "setKv: 6 arguments"); return NULL; }
  ctx_slot* c = get_slot(env, a[0]);
  if (!c) return NULL;
  int32_t layer, kvh, pos0;
  if (!get_i32(env, a[1], &layer) || !get_i32(env, a[2], &kvh) || !get_i32(env, a[3], &pos0)) {
    napi_throw_type_error(env, NULL, "setKv: integer layer, kvHead and pos0 expected");
    return NULL;
  }
  void *k, *v;
  int n;
  if (!kv_rows(env, c->head_dim, a[4], a[5], &k, &v, &n)) return NULL;
  int rc = q4hip_set_kv(c->h, layer, kvh, pos0, n, (const float*)k, (const float*)v);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* setDecodeMode(handle, mode): 0 auto, 1 graph, 2 persistent (q4hip_set_decode_mode). */
static napi_value js_set_decode_mode(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value a[2];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 2) { napi_throw_type_error(env, NULL, "setDecodeMode: 2 arguments"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  int32_t mode;
  if (!get_i32(env, a[1], &mode)) { napi_throw_type_error(env, NULL, "setDecodeMode: integer mode expected"); return NULL; }
  int rc = q4hip_set_decode_mode(h, mode);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* decodeModeUsed(handle) -> 0 (no decode step yet), 1 graph or 2 persistent */
static napi_value js_decode_mode_used(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value a[1];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 1) { napi_throw_type_error(env, NULL, "decodeModeUsed: 1 argument"); return NULL; }
  q4hip* h = get_handle(env, a[0]);
  if (!h) return NULL;
  int mode = 0;
  int rc = q4hip_decode_mode_used(h, &mode);
  if (rc) return throw_status(env, rc);
  napi_value out;
  NAPI_CALL(env, napi_create_int32(env, mode, &out));
  return out;
}

/* batchCreate(handle, B) -> batch handle: B sequences with their own K/V caches, decoded together
 * with the context's weights (q4hip_batch_create).  Released by batchDestroy, by destroy of the
 * context, or when collected. */
static napi_value js_batch_create(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value a[2];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 2) { napi_throw_type_error(env, NULL, "batchCreate: 2 arguments"); return NULL; }
  ctx_slot* c = get_slot(env, a[0]);
  if (!c) return NULL;
  int32_t B;
  if (!get_i32(env, a[1], &B)) { napi_throw_type_error(env, NULL, "batchCreate: integer B expected"); return NULL; }
  q4hip_batch* bt = NULL;
  int rc = q4hip_batch_create(&bt, c->h, B);
  if (rc) return throw_status(env, rc);
  batch_slot* b = (batch_slot*)calloc(1, sizeof *b);
  if (!b) { q4hip_batch_destroy(bt); napi_throw_error(env, NULL, "out of memory"); return NULL; }
  b->bt = bt;
  b->B = B;
  b->ctx = c;
  napi_value out;
  if (napi_create_external(env, b, finalize_batch, NULL, &out) != napi_ok) {
    q4hip_batch_destroy(bt);
    free(b);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  b->next = c->batches;
  c->batches = b;
  return out;
}

/* batchDestroy(batch): frees the batch's caches now; later calls on it throw. */
static napi_value js_batch_destroy(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value a[1];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  void* p = NULL;
  if (argc < 1 || napi_get_value_external(env, a[0], &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip batch handle");
    return NULL;
  }
  batch_slot* b = (batch_slot*)p;
  if (b->bt) q4hip_batch_destroy(b->bt);
  b->bt = NULL;
  unlink_batch(b);
  return NULL;
}

/* batchPrefill(batch, seq, Int32Array ids, pos) -> next id of sequence seq */
static napi_value js_batch_prefill(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value a[4];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 4) { napi_throw_type_error(env, NULL, "batchPrefill: 4 arguments"); return NULL; }
  batch_slot* b = get_batch(env, a[0]);
  if (!b) return NULL;
  int32_t seq, pos;
  void* data;
  size_t len;
  if (!get_i32(env, a[1], &seq) || !get_bytes(env, a[2], &data, &len) || !get_i32(env, a[3], &pos)) {
    napi_throw_type_error(env, NULL, "batchPrefill: (batch, seq, Int32Array, pos) expected");
    return NULL;
  }
  int next = 0;
  int rc = q4hip_batch_prefill(b->bt, seq, (const int*)data, (int)(len / 4), pos, &next);
  if (rc) return throw_status(env, rc);
  napi_value out;
  NAPI_CALL(env, napi_create_int32(env, next, &out));
  return out;
}

/* batchSetKv(batch, seq, layer, kvHead, pos0, Float32Array k, Float32Array v) (as setKv) */
static napi_value js_batch_set_kv(napi_env env, napi_callback_info info) {
  size_t argc = 7;
  napi_value a[7];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 7) { napi_throw_type_error(env, NULL, "batchSetKv: 7 arguments"); return NULL; }
  batch_slot* b = get_batch(env, a[0]);
  if (!b) return NULL;
  int32_t seq, layer, kvh, pos0;
  if (!get_i32(env, a[1], &seq) || !get_i32(env, a[2], &layer) || !get_i32(env, a[3], &kvh) ||
      !get_i32(env, a[4], &pos0)) {
    napi_throw_type_error(env, NULL, "batchSetKv: integer seq, layer, kvHead and pos0 expected");
    return NULL;
  }
  void *k, *v;
  int n;
  if (!kv_rows(env, b->ctx->head_dim, a[5], a[6], &k, &v, &n)) return NULL;
  int rc = q4hip_batch_set_kv(b->bt, seq, layer, kvh, pos0, n, (const float*)k, (const float*)v);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* batchGenerate(batch, Int32Array first[B], Int32Array pos[B], Int32Array out[steps * B]):
 * out[i * B + b] = sequence b's token at position pos[b] + 1 + i (q4hip_batch_generate). */
static napi_value js_batch_generate(napi_env env, napi_callback_info info) {
  size_t argc = 4;
  napi_value a[4];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 4) { napi_throw_type_error(env, NULL, "batchGenerate: 4 arguments"); return NULL; }
  batch_slot* b = get_batch(env, a[0]);
  if (!b) return NULL;
  void *first, *pos, *out;
  size_t fl, pl, ol;
  if (!get_bytes(env, a[1], &first, &fl) || !get_bytes(env, a[2], &pos, &pl) || !get_bytes(env, a[3], &out, &ol)) {
    napi_throw_type_error(env, NULL, "batchGenerate: Int32Array first, pos and out expected");
    return NULL;
  }
  size_t row = (size_t)b->B * 4;
  if (fl != row || pl != row || ol % row || ol / row > 0x7fffffff) {
    napi_throw_range_error(env, NULL, "batchGenerate: first and pos need B entries, out a multiple of B");
    return NULL;
  }
  int rc = q4hip_batch_generate(b->bt, (const int*)first, (const int*)pos, (int)(ol / row), (int*)out);
  if (rc) return throw_status(env, rc);
  return NULL;
}

/* batchReadLogits(batch, Float32Array out[B * vocab]) */
static napi_value js_batch_read_logits(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value a[2];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 2) { napi_throw_type_error(env, NULL, "batchReadLogits: 2 arguments"); return NULL; }
  batch_slot* b = get_batch(env, a[0]);
  if (!b) return NULL;
  void* data;
  size_t len;
  if (!get_bytes(env, a[1], &data, &len)) {
    napi_throw_type_error(env, NULL, "batchReadLogits: Float32Array expected");
    return NULL;
  }
  int rc = q4hip_batch_read_logits(b->bt, (float*)data, (int64_t)(len / 4));
  if (rc) return throw_status(env, rc);
  return NULL;
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int n = 0;
  int rc = q4hip_device_count(&n);
  if (rc) return throw_status(env, rc);
  napi_value out;
  NAPI_CALL(env, napi_create_int32(env, n, &out));
  return out;
}

static napi_value init(napi_env env, napi_value exports) {
  napi_property_descriptor p[] = {
      {"create", NULL, js_create, NULL, NULL, NULL, napi_enumerable, NULL},
      {"destroy", NULL, js_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"setTensor", NULL, js_set_tensor, NULL, NULL, NULL, napi_enumerable, NULL},
      {"setRope", NULL, js_set_rope, NULL, NULL, NULL, napi_enumerable, NULL},
      {"forward", NULL, js_forward, NULL, NULL, NULL, napi_enumerable, NULL},
      {"readLogits", NULL, js_read_logits, NULL, NULL, NULL, napi_enumerable, NULL},
      {"generate", NULL, js_generate, NULL, NULL, NULL, napi_enumerable, NULL},
      {"profile", NULL, js_profile, NULL, NULL, NULL, napi_enumerable, NULL},
      {"setKv", NULL, js_set_kv, NULL, NULL, NULL, napi_enumerable, NULL},
      {"setDecodeMode", NULL, js_set_decode_mode, NULL, NULL, NULL, napi_enumerable, NULL},
      {"decodeModeUsed", NULL, js_decode_mode_used, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchCreate", NULL, js_batch_create, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchDestroy", NULL, js_batch_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchPrefill", NULL, js_batch_prefill, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchSetKv", NULL, js_batch_set_kv, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchGenerate", NULL, js_batch_generate, NULL, NULL, NULL, napi_enumerable, NULL},
      {"batchReadLogits", NULL, js_batch_read_logits, NULL, NULL, NULL, napi_enumerable, NULL},
      {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  NAPI_CALL(env, napi_define_properties(env, exports, sizeof p / sizeof p[0], p));
  return exports;
}

NAPI_MODULE(q4hip, init)
