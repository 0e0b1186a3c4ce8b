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

static q4hip* get_handle(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip handle");
    return NULL;
  }
  q4hip** slot = (q4hip**)p;
  if (!*slot) {
    napi_throw_error(env, "5", "context destroyed");
    return NULL;
  }
  return *slot;
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
  q4hip** slot = (q4hip**)data;
  if (*slot) q4hip_destroy(*slot);
  free(slot);
}

/* create(dim, layers, ffn, heads, kvHeads, vocab, ctx, mt, eps, device) -> handle */
static napi_value js_create(napi_env env, napi_callback_info info) {
  size_t argc = 10;
  napi_value a[10];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  if (argc < 10) { napi_throw_type_error(env, NULL, "create: 10 arguments"); return NULL; }
  int32_t v[8], dev;
  double eps;
  for (int i = 0; i < 8; i++)
    if (!get_i32(env, a[i], &v[i])) { napi_throw_type_error(env, NULL, "create: integer expected"); return NULL; }
  if (napi_get_value_double(env, a[8], &eps) != napi_ok || !get_i32(env, a[9], &dev)) {
    napi_throw_type_error(env, NULL, "create: eps and device expected");
    return NULL;
  }
  q4hip* h = NULL;
  int rc = q4hip_create(&h, v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], (float)eps, dev);
  if (rc) return throw_status(env, rc);
  q4hip** slot = (q4hip**)malloc(sizeof *slot);
  if (!slot) { q4hip_destroy(h); napi_throw_error(env, NULL, "out of memory"); return NULL; }
  *slot = h;
  napi_value out;
  if (napi_create_external(env, slot, finalize_handle, NULL, &out) != napi_ok) {
    q4hip_destroy(h);
    free(slot);
    napi_throw_error(env, NULL, "napi_create_external failed");
    return NULL;
  }
  return out;
}

/* destroy(handle): frees device memory now; later calls on the handle throw. */
static napi_value js_destroy(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value a[1];
  NAPI_CALL(env, napi_get_cb_info(env, info, &argc, a, NULL, NULL));
  void* p = NULL;
  if (argc < 1 || napi_get_value_external(env, a[0], &p) != napi_ok || !p) {
    napi_throw_type_error(env, NULL, "expected a q4hip handle");
    return NULL;
  }
  q4hip** slot = (q4hip**)p;
  if (*slot) { q4hip_destroy(*slot); *slot = NULL; }
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
      {"deviceCount", NULL, js_device_count, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  NAPI_CALL(env, napi_define_properties(env, exports, sizeof p / sizeof p[0], p));
  return exports;
}

NAPI_MODULE(q4hip, init)
