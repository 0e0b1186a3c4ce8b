/*
 * q4hip.h -- C ABI of the MI355X Qwen2 Q4_0 token loop.
 *
 * One opaque context per loaded model, bound to one GPU and one HIP stream.
 * Calls on a context are serialized by the caller (one job at a time, as the
 * reference backend's single `pending` slot does, engine/cpu.js:33-50);
 * contexts are independent.  Every entry point returns Q4HIP_OK (0) or an
 * error code; q4hip_last_error() gives the message of the calling thread's
 * last failure ("context full", "kind 0: expected Q4_0", a HIP error ...).
 *
 * Reference paths below are relative to h2-own-inference-engine/.
 */
#ifndef Q4HIP_H
#define Q4HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4HIP_OK 0
#define Q4HIP_EINVAL 1      /* bad argument or configuration                         */
#define Q4HIP_ECONTEXT 2    /* pos + n >= ctx: "context full" (engine/cpu-worker.js:173) */
#define Q4HIP_ETYPE 3       /* tensor of an unsupported GGML type for its kind        */
#define Q4HIP_EHIP 4        /* HIP runtime failure (message names the call)           */
#define Q4HIP_ESTATE 5      /* model not fully loaded, or context destroyed          */

/* GGML tensor types accepted by q4hip_set_tensor (engine/gguf.js:6) */
#define Q4HIP_TYPE_F32 0
#define Q4HIP_TYPE_Q4_0 2
#define Q4HIP_TYPE_Q8_0 8

/* Tensor kinds, numbered as the reference's set_tensor (engine/kernels.c:422):
 * 0 qkv, 1 o, 2 gate+up, 3 down (Q4_0); 4 attn_norm, 5 ffn_norm, 6 qkv bias (F32);
 * 7 token embedding (Q4_0); 8 output head (Q4_0 or Q8_0); 9 output_norm (F32). */
#define Q4HIP_KIND_QKV 0
#define Q4HIP_KIND_O 1
#define Q4HIP_KIND_GU 2
#define Q4HIP_KIND_DOWN 3
#define Q4HIP_KIND_ATTN_NORM 4
#define Q4HIP_KIND_FFN_NORM 5
#define Q4HIP_KIND_BQKV 6
#define Q4HIP_KIND_EMBD 7
#define Q4HIP_KIND_OUTPUT 8
#define Q4HIP_KIND_OUTPUT_NORM 9

typedef struct q4hip q4hip;

/* Message of the calling thread's last failed call ("" if none). */
const char* q4hip_last_error(void);

/* Number of visible HIP devices. */
int q4hip_device_count(int* count);

/* K/V cache element types (q4hip_create's kv_type):
 *   Q4HIP_KV_F32  the reference's fp32 cache (kc/vc of engine/cpu-worker.js:71): results bit-identical
 *                 to the reference's arithmetic
 *   Q4HIP_KV_F16  half the cache bytes: K and V rounded to fp16 (nearest, ties to even) when appended
 *                 or written by q4hip_set_kv, and read back exactly; results bit-identical to the
 *                 reference's arithmetic over a cache holding those rounded values.  Decode steps run
 *                 on the persistent kernel at every context length with either type (past rows
 *                 beyond its staged tile stream through a ring in shared memory). */
#define Q4HIP_KV_F32 0
#define Q4HIP_KV_F16 1

/* Create a context: replaces set_config (engine/kernels.c:418-421) and the memory plan of
 * engine/cpu-worker.js:52-88.  Allocates weights, activations for device passes of up to `mt`
 * tokens (1..1024, capped at ctx; 0 or out of range = 1024: a prompt runs as passes of that many
 * tokens, with results identical to the reference's 16-token chunks), the K/V cache of `kv_type`
 * for `ctx` positions and the token array on `device`.  head_dim = dim/heads. */
int q4hip_create(q4hip** out, int dim, int layers, int ffn, int heads, int kv_heads, int vocab,
                 int ctx, int mt, float eps, int device, int kv_type);

/* Upload one GGUF tensor (or a part of a fused one): replaces set_tensor (engine/kernels.c:423-431)
 * together with copyBlocks (engine/cpu-worker.js:97-124).  `data` holds `rows` rows in GGUF
 * layout (Q4_0 18-byte / Q8_0 34-byte blocks, or F32 values).  `row0` is the first row of the
 * fused tensor they fill: q at 0, k at dim, v at dim + kv_heads*head_dim (kind 0 and its bias 6);
 * gate at 0, up at ffn (kind 2).  For F32 kinds a "row" is one value.  `nbytes` is the size of
 * `data`; a buffer shorter than `rows` rows is rejected. */
int q4hip_set_tensor(q4hip* h, int kind, int layer, int row0, int ggml_type, const void* data,
                     int64_t rows, size_t nbytes);

/* Upload the RoPE table: fp32 [pos][head_dim/2][2] = cos, sin of pos/theta^(2i/head_dim),
 * computed in double by the host as engine/cpu-worker.js:130-135 does.  `n_floats` is the number
 * of floats `table` holds; fewer than ctx * head_dim is rejected (nothing is read). */
int q4hip_set_rope(q4hip* h, const float* table, int64_t n_floats);

/* Run tokens ids[0..n) at positions pos..pos+n-1 and return the greedy next token (first
 * maximum wins): replaces forward() of engine/cpu-worker.js:169-182 with temperature 0, i.e.
 * the chunk loop over run() (engine/kernels.c:454-465) plus sample() (cpu-worker.js:154-158).
 * K/V of those positions are (over)written; logits of the last token stay on the device. */
int q4hip_forward(q4hip* h, const int* ids, int n, int pos, int* next);

/* How single-token decode steps run (forward with n == 1, generate):
 *   AUTO       the persistent kernel when the model and device admit it, else the graph (default)
 *   GRAPH      a captured hipGraph of one launch per operation
 *   PERSISTENT one launch per call that runs all of the call's steps; fails with
 *              Q4HIP_EINVAL if the model (head_dim 64, D <= 1024, ...) or device does not admit it.
 * Both give bit-identical results.  The reference picks among its kernel builds the same way
 * (engine/cpu.js:18-24); this has no other counterpart there. */
#define Q4HIP_DECODE_AUTO 0
#define Q4HIP_DECODE_GRAPH 1
#define Q4HIP_DECODE_PERSISTENT 2
int q4hip_set_decode_mode(q4hip* h, int mode);
/* The path the last decode step took (Q4HIP_DECODE_GRAPH or Q4HIP_DECODE_PERSISTENT; 0 before any). */
int q4hip_decode_mode_used(q4hip* h, int* mode);

/* Copy the last forward's logits (vocab floats) to host memory: readLogits (engine/cpu.js:60-62). */
int q4hip_read_logits(q4hip* h, float* out, int n);

/* Greedy continuation on the device: token `first` at position `pos`, then `steps` decode steps,
 * each feeding back its own argmax; out[i] = token at position pos+1+i.  The same tokens as
 * `steps` calls of forward([t], pos+i) (engine/llm.js:86-97) without a host round trip per step. */
int q4hip_generate(q4hip* h, int first, int pos, int steps, int* out);

/* Per-operation GPU time of one decode step (forward([token], pos)), in microseconds, summed
 * over layers: profile (engine/cpu-worker.js:31-37, engine/kernels.c:481-483).  us[] receives
 * Q4HIP_PROF_N entries in the order of the Q4HIP_PROF_* indices. */
#define Q4HIP_PROF_EMBED 0
#define Q4HIP_PROF_NORM_Q 1
#define Q4HIP_PROF_QKV 2
#define Q4HIP_PROF_ROPE 3
#define Q4HIP_PROF_ATTN 4
#define Q4HIP_PROF_QUANT 5
#define Q4HIP_PROF_O 6
#define Q4HIP_PROF_GU 7
#define Q4HIP_PROF_SWIGLU 8
#define Q4HIP_PROF_DOWN 9
#define Q4HIP_PROF_OUT 10
#define Q4HIP_PROF_SAMPLE 11
#define Q4HIP_PROF_N 12
int q4hip_profile(q4hip* h, int token, int pos, float* us, int n);

/* The same per-class device times for one pass of `ntok` prompt tokens (1..mt) at positions pos.. */
int q4hip_profile_pass(q4hip* h, const int* ids, int ntok, int pos, float* us, int n);

/* Timeline of one persistent decode step (forward([token], pos)), in microseconds from the
 * kernel's start, for (layers + 1) * 16 slots; -1 where nothing was recorded.  Per layer l, slot
 * 16l + k: 0 att received, 1 x after o sent, 2 act received, 3 x after down sent (first o/down
 * workgroup); 4 x received, 5 q/k/v done, 6 att sent (head 0); 7 x received, 8 act sent (first
 * gate/up workgroup); 9 A normalised, 10 gate/up normalised, 11..14 attention after RoPE, max,
 * sum, normalisation (head 0).  Slots 16L + 0..2: head x received, (value, index) sent, token
 * known; slot 16L + 4: the shader clock over the step in MHz; slot 16L + 5: the grid size G.
 * Then, if n allows, 8 * L * G per-workgroup entries [layer][workgroup][k]: o/down workgroups
 * k = 0 att received, 1 x after o sent, 2 act received, 3 x after down sent, 4 o terms formed
 * (wave 0), 5 down terms formed (wave 0), 6 down terms of all waves; attention workgroups 0 x
 * received, 1 att sent, 2 past K scored (streamed), 3 scores exchanged (pair), 4 new K/V received,
 * 5 probabilities formed; K/V workgroups 0 x received, 2 normalised, 3 rows formed, 1 rows sent;
 * gate/up workgroups 0 x received, 2 normalised, 3 rows formed, 1 act sent.  Measured with the
 * device's constant 100 MHz clock and its shader cycle counter. */
int q4hip_profile_persistent(q4hip* h, int token, int pos, float* us, int n);

/* Write the K and V rows of one layer and kv head at positions [pos0, pos0 + n): `k` and `v` are
 * [n][head_dim] fp32 (rounded to fp16 for an fp16 cache).  The reference's cache is memory its host owns and hands to the kernels
 * (kc/vc of set_buffers, engine/kernels.c:433-440); this fills ours directly, e.g. with a cache
 * prefilled from stored activations.  Positions must lie below ctx. */
int q4hip_set_kv(q4hip* h, int layer, int kv_head, int pos0, int n, const float* k, const float* v);

/* Time `steps` greedy decode steps (as q4hip_generate) with HIP events on the context's stream;
 * *ms = elapsed device time of the whole loop. */
int q4hip_time_generate(q4hip* h, int first, int pos, int steps, int* out, float* ms);

/* Launch the output-head matvec alone `iters` times back to back on the context's stream, on the
 * activations of the last forward, and report its mean duration from HIP events. */
int q4hip_time_head(q4hip* h, int iters, float* us_per_launch);

/* Release all device memory of the context. */
void q4hip_destroy(q4hip* h);

/* ---- batched decode -------------------------------------------------------------------------
 * B independent sequences decoded together, one token each per step, with the context's weights.
 * The reference decodes one sequence per backend (engine/cpu.js:33-50, engine/llm.js:86-97); a
 * batch runs B such loops at once, and every sequence's tokens and logits are the ones its own
 * loop would give.  Each sequence has its own K/V cache of the context's ctx positions, of the
 * context's kv_type (fp32 or fp16); the context's activation buffers are shared, so B <= the context's pass size and calls on a batch and
 * on its context are serialized by the caller.  Destroy batches before their context. */
typedef struct q4hip_batch q4hip_batch;
int q4hip_batch_create(q4hip_batch** out, q4hip* h, int B);
void q4hip_batch_destroy(q4hip_batch* bt);
/* Run prompt ids[0..n) of sequence `seq` at positions pos.. (as q4hip_forward, against that
 * sequence's cache) and return its greedy next token. */
int q4hip_batch_prefill(q4hip_batch* bt, int seq, const int* ids, int n, int pos, int* next);
/* Write K and V rows of sequence `seq` (as q4hip_set_kv). */
int q4hip_batch_set_kv(q4hip_batch* bt, int seq, int layer, int kv_head, int pos0, int n, const float* k,
                       const float* v);
/* `steps` greedy steps of every sequence: sequence b starts with token first[b] at position pos[b]
 * (the positions may differ); out[i * B + b] = its token at position pos[b] + 1 + i.  Fails with
 * Q4HIP_ECONTEXT when pos[b] + steps >= ctx for any b. */
int q4hip_batch_generate(q4hip_batch* bt, const int* first, const int* pos, int steps, int* out);
/* The same, timed with HIP events on the context's stream; *ms = device time of all steps. */
int q4hip_batch_time_generate(q4hip_batch* bt, const int* first, const int* pos, int steps, int* out, float* ms);
/* Logits of the last step, [B][vocab] floats; n >= B * vocab. */
int q4hip_batch_read_logits(q4hip_batch* bt, float* out, int64_t n);

/* ---- isolated Q4_0 matvec (the kernel of every projection) ---------------------------------
 * y[n] = W[n] . x for an N x K Q4_0 matrix given in GGUF layout, with x quantized to int8 per
 * 32-block exactly as quantize_row (engine/kernels.c:90-114) and each output accumulated as
 * matmul_q4 does (engine/kernels.c:200-229).  Used by the matvec sweep and its parity tests.
 * A matvec handle owns its device copy of W, x and y. */
typedef struct q4hip_mv q4hip_mv;
int q4hip_mv_create(q4hip_mv** out, int N, int K, const void* gguf_q4_0, int device);
/* Set x (K floats, host), quantize on the device, run once, copy y (N floats) back. */
int q4hip_mv_run(q4hip_mv* m, const float* x, float* y);
/* Run `iters` matvecs on the resident x; *us = mean HIP-event duration per launch. */
int q4hip_mv_time(q4hip_mv* m, int iters, float* us);
/* The same with the weights not in any cache: `iters` launches cycling through device copies of W
 * whose total size is at least `rotate_bytes` (e.g. more than the 256 MB last-level cache);
 * *copies_used (optional) receives the number of copies. */
int q4hip_mv_time_cold(q4hip_mv* m, int64_t rotate_bytes, int iters, float* us, int* copies_used);
void q4hip_mv_destroy(q4hip_mv* m);

/* The matvec of q4hip_mv_run with nothing allocated: no counterpart in the reference.  It is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  x (K floats) and y (N floats) are device memory of the
 * handle's device, checked before anything is launched.  The int8 activation blocks go to a
 * library-owned static device buffer of Q4HIP_NOALLOC_MAX_K / 32 blocks (128 KB per device, held
 * until the process ends); K above Q4HIP_NOALLOC_MAX_K is rejected.  `stream` (a hipStream_t)
 * NULL: the handle's stream, and the call waits for the result; otherwise the work is enqueued
 * on that stream and the call returns at once.  Every call on one device shares the buffer:
 * calls that overlap on one GPU (other streams, other threads, other handles) race. */
#define Q4HIP_NOALLOC_MAX_K 65536
int q4hip_mv_run_noalloc(q4hip_mv* m, const float* x, float* y, void* stream);

/* ---- self-check of the quotient forms ------------------------------------------------------
 * The kernels compute the reference's IEEE binary32 divisions (engine/kernels.c:84, 98-99, 395)
 * by reciprocal products with fused corrections on verified domains.  This runs every input of
 * each form's domain on the device against the IEEE division and writes the mismatch counts:
 * [0] a / 127 (a >= 0), [1] d ? 1/d : 0 (d >= 0), [2] g / (1 + fast_exp(-g)) (every bit pattern),
 * [3] a / 896 (a >= 0), [4] 1 / d (d >= 0).  No counterpart in the reference (a diagnostic). */
int q4hip_check_division(int device, unsigned long long* mismatches, int n);

/* ---- self-check of the attention ring's row bounds (host only, no GPU) ----------------------
 * The persistent decode kernel's attention workgroups stream past K/V rows through a ring in
 * shared memory; loads past the end of a stream are redirected to its last row.  This runs the
 * kernel's row arithmetic on the host for one step at position `pos` (staged tile of kv_tile
 * positions, a ring of ring_slots = 3 or 7 slots, split = two workgroups per head and `half` the
 * one asked for, kv_f16 = an fp16 cache) and writes the lowest and highest row any ring load
 * reads (*lo = 0, *hi = -1 when there is none) and the number of loads.  Every row must be a past
 * position, < pos (the reference reads exactly pos + 1 positions, engine/kernels.c:355-360, the
 * last from the new row).  No counterpart in the reference (a diagnostic). */
int q4hip_attn_ring_rows(int pos, int kv_tile, int ring_slots, int split, int half, int kv_f16, int* lo, int* hi,
                         int* loads);

#ifdef __cplusplus
}
#endif
#endif
