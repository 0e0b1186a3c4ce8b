/*
 * oracle.h -- CPU restatement of the reference's Qwen2 Q4_0 token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  tests/, the smoke check and the CPU-baseline leg
 * of bench.py load this library to compute expected results.  The product (the HIP library, the N-API addon and the JavaScript
 * backend) never links, loads or calls it.
 *
 * It restates, in scalar C with the same floating-point operation order,
 *   h2-own-inference-engine/engine/kernels.c   (plain SIMD128 build, no -DRELAXED)
 * and the host steps of
 *   h2-own-inference-engine/engine/cpu-worker.js (fp16 table, copyBlocks repack,
 *   RoPE table, chunk loop, greedy sample).
 * Every function cites the reference lines it follows.  Compiled with
 * -ffp-contract=off and without fast-math so each binary32 operation rounds
 * exactly once, as in wasm.
 */
#ifndef Q4_ORACLE_H
#define Q4_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_MAXL 64

/* --- elementwise pieces (kernels.c:69-170) ------------------------------ */
float orc_fast_exp(float x);
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps);
void orc_quantize_row(int8_t* q, float* d, float* s, const float* x, int n);
float orc_dot_q4_q8(const uint8_t* wq, const float* wd, const int8_t* xq, const float* xd, int nb);
float orc_dot_q8_q8(const int8_t* wq, const float* wd, const int8_t* xq, const float* xd, int nb);
/* integer part of one block, per lane of the SIMD128 partition (4 int32) */
void orc_block_lanes_q4(const uint8_t* qs16, const int8_t* x32, int32_t out[4]);
/* y[m][n] (op)= W[n]·x[m] for rows [a,b); op 0 STORE, 1 BIAS, 2 ADD (kernels.c:190-273) */
void orc_matmul_q4(const uint8_t* wqs, const float* wd, int K, int N, int a, int b, int M,
                   const int8_t* xq, const float* xd, float* y, int op, const float* bias);
/* one (token, head) attention task over T cached positions (kernels.c:355-377) */
void orc_attend(const float* q, const float* kb, const float* vb, int T, int hd, float* scores, float* out);
/* NEOX RoPE of one head vector in place (kernels.c:340-344) */
void orc_rope_head(float* v, const float* cs, int hd);
/* act = silu(gate)·up (kernels.c:395) */
void orc_swiglu(float* act, const float* gate, const float* up, int n);
/* greedy argmax, first maximum wins (cpu-worker.js:156-157) */
int orc_argmax(const float* logits, int n);
/* one embedding row: dequantize Q4_0 (qs 16 B + fp32 d per block) to dim floats (kernels.c:312-322) */
void orc_embed_row(float* out, const uint8_t* qs, const float* d, int dim);

/* --- host-side steps (cpu-worker.js) ------------------------------------ */
float orc_f16_to_f32(uint16_t h);                                     /* cpu-worker.js:93-96 */
/* GGUF blocks -> separate values + fp32 scale (cpu-worker.js:97-104) */
void orc_copy_blocks(const uint8_t* src, int64_t nblocks, int block_bytes, uint8_t* qs, float* d);
/* fp32 table [ctx][hd/2][2] of cos/sin(pos/theta^(2i/hd)) in double (cpu-worker.js:130-135) */
void orc_rope_table(float* rope, int ctx, int hd, double theta);

/* --- the model ----------------------------------------------------------- */
typedef struct orc_model orc_model;

/* set_config (kernels.c:418-421) + the memory plan (cpu-worker.js:52-88): allocates activations,
 * the fp32 KV cache, the RoPE table and the token array.  threads = CPU threads for row splits. */
orc_model* orc_create(int dim, int layers, int ffn, int heads, int kvh, int vocab, int ctx, int mt,
                      float eps, double rope_theta, int threads);
void orc_destroy(orc_model* m);
/* set_tensor (kernels.c:423-431): kinds 0 qkv, 1 o, 2 gu, 3 down (Q4 qs + fp32 d), 4 attn_norm,
 * 5 ffn_norm, 6 bqkv (f32 in d), 7 embd (Q4), 8 output (Q8), 9 output_norm.  Pointers are borrowed. */
void orc_set_tensor(orc_model* m, int kind, int layer, const void* qs, const float* d);
/* run (kernels.c:454-465): tokens[pos0 .. pos0+M) through the model */
void orc_run(orc_model* m, int pos0, int M, int want_logits);
/* forward (cpu-worker.js:169-182): chunk loop + greedy sample; returns next id, -1 on "context full" */
int orc_forward(orc_model* m, const int* ids, int n, int pos);
void orc_set_threads(orc_model* m, int threads);
const float* orc_logits(const orc_model* m);

/* Numerics variants, for measuring how far other operation orders or a half-precision cache move
 * the results (none is the reference's arithmetic; 0, the default, is):
 *   ORC_V_NORM_TREE   RMSNorm sums of squares as 32 strided partial sums and a pairwise tree
 *   ORC_V_DOT_SPLITK  each projection lane chain split into 4 contiguous block ranges, then added
 *   ORC_V_ATTN_SPLIT  attention over chunks of 256 positions merged by the log-sum-exp rule
 *   ORC_V_KV_F16      K and V rounded to binary16 (ties to even) when appended to the cache: the
 *                     arithmetic of a half-precision KV cache read back exactly into fp32 */
#define ORC_V_NORM_TREE 1
#define ORC_V_DOT_SPLITK 2
#define ORC_V_ATTN_SPLIT 4
#define ORC_V_KV_F16 8
void orc_set_variant(orc_model* m, int flags);
/* Round to the nearest binary16 value (ties to even) and widen back to fp32. */
float orc_round_f16(float x);
float* orc_kcache(orc_model* m);   /* [layers][kvh][ctx][hd] fp32 */
float* orc_vcache(orc_model* m);
float* orc_hidden(orc_model* m);   /* x [mt][dim] */
int* orc_tokens(orc_model* m);

#ifdef __cplusplus
}
#endif
#endif
