/*
 * oracle.c -- CPU restatement of the reference's Qwen2 Q4_0 token loop.
 *
 * TEST INFRASTRUCTURE ONLY: computes the expected results for tests/, the smoke
 * check and the CPU-baseline leg of bench.py.  The product never links or calls it.
 *
 * Follows h2-own-inference-engine/engine/kernels.c (plain SIMD128 build) and
 * h2-own-inference-engine/engine/cpu-worker.js.  Each 128-bit SIMD value of the
 * reference is written here as four scalar lanes, each lane rounding in the
 * same order as the SIMD lane it stands for.  Threads (OpenMP) split rows and
 * (token, head) tasks only, never a reduction, so results do not depend on the
 * thread count -- the same property the reference's thread pool has
 * (kernels.c:63-66, wiki/04-cpu-webassembly.md:75-77).
 *
 * Build: see oracle/Makefile (-O2 -ffp-contract=off, SSE2 binary32, no fast-math).
 */
#include "oracle.h"

#include <emmintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ math helpers */

/* kernels.c:69-78: e^x as 2^n * degree-6 Taylor polynomial of the Cody-Waite reduced r. */
float orc_fast_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  float n = floorf(x * 1.44269504f + 0.5f);
  float r = x - n * 0.693145752f - n * 1.42860677e-6f;
  float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.166666672f + r * (0.0416666679f +
            r * (0.00833333377f + r * 0.00138888892f)))));
  union { float f; uint32_t i; } u = { .f = p };
  u.i += (uint32_t)(int32_t)n << 23;   /* wasm i32.shl: two's complement, mod 2^32 */
  return u.f;
}

/* kernels.c:80-86: four lane sums of x*x (lane j takes i = j mod 4), then ((l0+l1)+l2)+l3. */
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < n; i += 4)
    for (int j = 0; j < 4; j++) s[j] = s[j] + x[i + j] * x[i + j];
  float ss = s[0] + s[1] + s[2] + s[3];
  float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; i++) out[i] = (x[i] * r) * w[i];
}

/* wasm f32x4.nearest (ties to even) then i32x4.trunc_sat_f32x4 */
static inline int32_t nearest_trunc_sat(float v) {
  if (v != v) return 0;
  float r = nearbyintf(v);                 /* default rounding mode: to nearest, ties to even */
  if (r >= 2147483648.0f) return INT32_MAX;
  if (r < -2147483648.0f) return INT32_MIN;
  return (int32_t)r;
}
static inline int8_t sat_i8(int32_t v) {   /* i16x8.narrow_i32x4_s then i8x16.narrow_i16x8_s */
  if (v > 32767) v = 32767;
  if (v < -32768) v = -32768;
  if (v > 127) v = 127;
  if (v < -128) v = -128;
  return (int8_t)v;
}

/* kernels.c:90-114: per 32-block, d = amax/127, id = d ? 1/d : 0, q = sat(nearest(x*id)), s = d*sum(q). */
void orc_quantize_row(int8_t* q, float* d, float* s, const float* x, int n) {
  for (int b = 0; b < n / 32; b++) {
    const float* xb = x + 32 * b;
    float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 32; i += 4)
      for (int j = 0; j < 4; j++) {
        float a = fabsf(xb[i + j]);
        mx[j] = a > mx[j] ? a : mx[j];      /* f32x4.max on non-negative, non-NaN values */
      }
    float amax = mx[0] > mx[1] ? mx[0] : mx[1];
    if (mx[2] > amax) amax = mx[2];
    if (mx[3] > amax) amax = mx[3];
    float dd = amax / 127.0f, id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int32_t sum = 0;
    for (int i = 0; i < 32; i++) {
      int32_t v = nearest_trunc_sat(xb[i] * id);
      q[32 * b + i] = sat_i8(v);
      sum += v;
    }
    d[b] = dd;
    if (s) s[b] = dd * (float)sum;
  }
}

/* The integer part of kernels.c:127-136 (Q4_UNPACK/q4_bdot, :178-185): lane j of the
 * i32x4 sums elements {2j,2j+1, 8+2j,9+2j, 16+2j,17+2j, 24+2j,25+2j} of (nib-8)*xq,
 * where element e < 16 is the low nibble of byte e and element 16+e the high nibble. */
void orc_block_lanes_q4(const uint8_t* qs, const int8_t* x, int32_t p[4]) {
  for (int j = 0; j < 4; j++) {
    int32_t acc = 0;
    const int idx[4] = {2 * j, 2 * j + 1, 8 + 2 * j, 9 + 2 * j};
    for (int t = 0; t < 4; t++) {
      int e = idx[t];
      acc += ((qs[e] & 15) - 8) * x[e];
      acc += ((qs[e] >> 4) - 8) * x[16 + e];
    }
    p[j] = acc;
  }
}

/* The same lane sums with SSE2 (x86-64's baseline): the 32 products as int16, adjacent pairs
 * (e, e+1) summed by pmaddwd, so int32 lane j of the low half holds pair (2j, 2j+1) and of the high
 * half pair (8+2j, 9+2j); lane j of the total is the lane dot above (for int8 weights the same
 * elements of w).  Integer sums are exact in any order, so this equals orc_block_lanes_q4
 * (tests/test_oracle.py compares the dots with a NumPy emulation of the reference's SIMD). */
static inline __m128i sx_lo(__m128i v) { return _mm_unpacklo_epi8(v, _mm_cmpgt_epi8(_mm_setzero_si128(), v)); }
static inline __m128i sx_hi(__m128i v) { return _mm_unpackhi_epi8(v, _mm_cmpgt_epi8(_mm_setzero_si128(), v)); }
static inline __m128i lanes16(__m128i w, __m128i x) {   /* 16 int8 weights x 16 int8 activations */
  return _mm_add_epi32(_mm_madd_epi16(sx_lo(w), sx_lo(x)), _mm_madd_epi16(sx_hi(w), sx_hi(x)));
}
static inline __m128i block_lanes_q4_sse2(const uint8_t* qs, const int8_t* x) {
  const __m128i q = _mm_loadu_si128((const __m128i*)qs), m4 = _mm_set1_epi8(15), e8 = _mm_set1_epi8(8);
  const __m128i lo = _mm_sub_epi8(_mm_and_si128(q, m4), e8);
  const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(q, 4), m4), e8);
  return _mm_add_epi32(lanes16(lo, _mm_loadu_si128((const __m128i*)x)),
                       lanes16(hi, _mm_loadu_si128((const __m128i*)(x + 16))));
}
static inline __m128i block_lanes_q8_sse2(const int8_t* w, const int8_t* x) {
  return _mm_add_epi32(lanes16(_mm_loadu_si128((const __m128i*)w), _mm_loadu_si128((const __m128i*)x)),
                       lanes16(_mm_loadu_si128((const __m128i*)(w + 16)), _mm_loadu_si128((const __m128i*)(x + 16))));
}

/* kernels.c:121-139: acc_lane += f32(p_lane) * (wd*xd), block by block, then hsum (kernels.c:116-118).
 * The four lanes as one SSE vector: cvtdq2ps is exact for these sums (|p| < 2^24), mulps and addps
 * round each lane once, as the reference's f32x4 operations do. */
static inline float lanes_hsum(__m128 acc) {
  float a[4];
  _mm_storeu_ps(a, acc);
  return a[0] + a[1] + a[2] + a[3];
}
float orc_dot_q4_q8(const uint8_t* wq, const float* wd, const int8_t* xq, const float* xd, int nb) {
  __m128 acc = _mm_setzero_ps();
  for (int b = 0; b < nb; b++) {
    const __m128 p = _mm_cvtepi32_ps(block_lanes_q4_sse2(wq + 16 * b, xq + 32 * b));
    acc = _mm_add_ps(acc, _mm_mul_ps(p, _mm_set1_ps(wd[b] * xd[b])));
  }
  return lanes_hsum(acc);
}

/* kernels.c:157-170: same lane partition with int8 weights. */
float orc_dot_q8_q8(const int8_t* wq, const float* wd, const int8_t* xq, const float* xd, int nb) {
  __m128 acc = _mm_setzero_ps();
  for (int b = 0; b < nb; b++) {
    const __m128 p = _mm_cvtepi32_ps(block_lanes_q8_sse2(wq + 32 * b, xq + 32 * b));
    acc = _mm_add_ps(acc, _mm_mul_ps(p, _mm_set1_ps(wd[b] * xd[b])));
  }
  return lanes_hsum(acc);
}

/* kernels.c:190-194 */
static inline void put(float* y, int N, int m, int n, float v, int op, const float* bias) {
  float* o = y + (size_t)m * N + n;
  if (op == 2) *o = *o + v; else if (op == 1) *o = v + bias[n]; else *o = v;
}

/* kernels.c:200-273.  The reference's 4-row (M = 1) and 2x4 (M > 1) tiles and its leftover
 * loops all compute each output with the arithmetic of dot_q4_q8 (kernels.c:217-218, 243-247,
 * 264-271), so one loop over rows and tokens is the same function. */
void orc_matmul_q4(const uint8_t* wqs, const float* wd, int K, int N, int a, int b, int M,
                   const int8_t* xq, const float* xd, float* y, int op, const float* bias) {
  const int nb = K / 32;
  for (int n = a; n < b; n++) {
    const uint8_t* wq = wqs + (size_t)n * nb * 16;
    const float* d = wd + (size_t)n * nb;
    for (int m = 0; m < M; m++)
      put(y, N, m, n, orc_dot_q4_q8(wq, d, xq + (size_t)m * K, xd + (size_t)m * nb, nb), op, bias);
  }
}

/* kernels.c:340-344: NEOX pairs (i, i+hd/2) rotated by the table's cos/sin for this position. */
void orc_rope_head(float* v, const float* cs, int hd) {
  for (int i = 0; i < hd / 2; i++) {
    float c = cs[2 * i], s = cs[2 * i + 1], x0 = v[i], x1 = v[i + hd / 2];
    v[i] = x0 * c - x1 * s;
    v[i + hd / 2] = x1 * c + x0 * s;
  }
}

/* kernels.c:356-376 for one (token, head): scores with 4 lane sums over i = j mod 4, hsum, scale;
 * softmax with fast_exp and a running sum over t; output lane-wise sum over t of (e_t/sum)*v_t. */
void orc_attend(const float* q, const float* kb, const float* vb, int T, int hd, float* sc, float* out) {
  float mx = -1e30f, scale = 1.0f / sqrtf((float)hd);
  for (int t = 0; t < T; t++) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < hd; i += 4)
      for (int j = 0; j < 4; j++) s[j] = s[j] + q[i + j] * kb[(size_t)t * hd + i + j];
    float v = (s[0] + s[1] + s[2] + s[3]) * scale;
    sc[t] = v;
    if (v > mx) mx = v;
  }
  float sum = 0.0f;
  for (int t = 0; t < T; t++) { float e = orc_fast_exp(sc[t] - mx); sc[t] = e; sum += e; }
  for (int i = 0; i < hd; i++) out[i] = 0.0f;
  for (int t = 0; t < T; t++) {
    float p = sc[t] / sum;
    for (int i = 0; i < hd; i++) out[i] = out[i] + p * vb[(size_t)t * hd + i];
  }
}

/* kernels.c:395: gt / (1 + fast_exp(-gt)) * up */
void orc_swiglu(float* act, const float* gate, const float* up, int n) {
  for (int i = 0; i < n; i++) { float gt = gate[i]; act[i] = gt / (1.0f + orc_fast_exp(-gt)) * up[i]; }
}

/* cpu-worker.js:156-157: strict '>' so the first maximum wins */
int orc_argmax(const float* lg, int n) {
  int best = 0;
  for (int i = 1; i < n; i++) if (lg[i] > lg[best]) best = i;
  return best;
}

/* kernels.c:312-322 for one row */
void orc_embed_row(float* xr, const uint8_t* q, const float* d, int D) {
  for (int blk = 0; blk < D / 32; blk++)
    for (int j = 0; j < 16; j++) {
      xr[32 * blk + j] = (float)((q[16 * blk + j] & 15) - 8) * d[blk];
      xr[32 * blk + 16 + j] = (float)((q[16 * blk + j] >> 4) - 8) * d[blk];
    }
}

/* ------------------------------------------------------------------ host-side steps */

/* cpu-worker.js:93-96: exact IEEE half -> binary32 */
float orc_f16_to_f32(uint16_t h) {
  int s = h & 0x8000 ? -1 : 1, e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) return (float)(s * (double)m * ldexp(1.0, -24));
  if (e == 31) return m ? NAN : (float)(s * INFINITY);
  return (float)(s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15));
}

/* cpu-worker.js:97-104: GGUF block = fp16 scale + values; split into values and fp32 scales */
void orc_copy_blocks(const uint8_t* src, int64_t nb, int block_bytes, uint8_t* qs, float* d) {
  const int vb = block_bytes - 2;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* o = src + b * block_bytes;
    d[b] = orc_f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    memcpy(qs + b * vb, o + 2, (size_t)vb);
  }
}

/* cpu-worker.js:130-135 */
void orc_rope_table(float* rope, int ctx, int hd, double theta) {
  for (int pos = 0; pos < ctx; pos++)
    for (int i = 0; i < hd / 2; i++) {
      double a = pos / pow(theta, (2.0 * i) / hd);
      rope[(size_t)pos * hd + 2 * i] = (float)cos(a);
      rope[(size_t)pos * hd + 2 * i + 1] = (float)sin(a);
    }
}

/* ------------------------------------------------------------------ the model (kernels.c:26-41) */

/* ---- numerics variants (not the reference's arithmetic; see oracle.h) ---- */

/* Round to the nearest binary16 value, ties to even, and widen back (IEEE 754 conversion). */
float orc_round_f16(float x) {
  union { float f; uint32_t u; } v = { .f = x };
  const uint32_t sign = v.u & 0x80000000u, a = v.u & 0x7fffffffu;
  if (a >= 0x7f800000u) return x;                          /* inf and NaN stay */
  if (a >= 0x477ff000u) { v.u = sign | 0x7f800000u; return v.f; }   /* >= 65520: to infinity */
  if (a < 0x38800000u) {                                   /* below 2^-14: multiples of 2^-24 */
    union { float f; uint32_t u; } m = { .u = a };
    float q = nearbyintf(m.f * 16777216.0f) * 5.9604644775390625e-8f;
    union { float f; uint32_t u; } r = { .f = q };
    r.u |= sign;
    return r.f;
  }
  uint32_t u = a + 0x0fffu + ((a >> 13) & 1u);              /* round off 13 mantissa bits, ties to even */
  v.u = sign | (u & ~0x1fffu);
  return v.f;
}

/* RMSNorm with the sum of squares reassociated as a GPU block reduction would: 32 strided
 * partial sums (i mod 32), then a pairwise tree. */
static void rmsnorm_tree(float* out, const float* x, const float* w, int n, float eps) {
  float p[32];
  for (int k = 0; k < 32; k++) p[k] = 0.0f;
  for (int i = 0; i < n; i++) p[i & 31] = p[i & 31] + x[i] * x[i];
  for (int w2 = 16; w2 > 0; w2 >>= 1)
    for (int k = 0; k < w2; k++) p[k] = p[k] + p[k + w2];
  float r = 1.0f / sqrtf(p[0] / (float)n + eps);
  for (int i = 0; i < n; i++) out[i] = (x[i] * r) * w[i];
}

/* dot_q4_q8 with each lane's chain over blocks split into 4 contiguous parts (as 4 waves would
 * split the blocks), the parts added in order, then hsum. */
static float dot_q4_q8_splitk(const uint8_t* wq, const float* wd, const int8_t* xq, const float* xd, int nb) {
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int per = (nb + 3) / 4;
  for (int part = 0; part < 4; part++) {
    float pa[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = part * per; b < nb && b < (part + 1) * per; b++) {
      int32_t p[4];
      orc_block_lanes_q4(wq + 16 * b, xq + 32 * b, p);
      float sc = wd[b] * xd[b];
      for (int j = 0; j < 4; j++) pa[j] = pa[j] + (float)p[j] * sc;
    }
    for (int j = 0; j < 4; j++) acc[j] = acc[j] + pa[j];
  }
  return acc[0] + acc[1] + acc[2] + acc[3];
}

/* Attention split over chunks of 256 positions (flash-decoding): per chunk its own maximum, sum and
 * P.V; the chunks merged with the log-sum-exp rule using expf. */
static void attend_split(const float* q, const float* kb, const float* vb, int T, int hd, float* sc, float* out) {
  enum { CH = 256 };
  float scale = 1.0f / sqrtf((float)hd), M = -1e30f, S = 0.0f;
  float acc[256];
  for (int i = 0; i < hd; i++) acc[i] = 0.0f;
  for (int t = 0; t < T; t++) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < hd; i += 4)
      for (int j = 0; j < 4; j++) s[j] = s[j] + q[i + j] * kb[(size_t)t * hd + i + j];
    sc[t] = (s[0] + s[1] + s[2] + s[3]) * scale;
  }
  for (int c0 = 0; c0 < T; c0 += CH) {
    int c1 = c0 + CH < T ? c0 + CH : T;
    float m = -1e30f, sum = 0.0f, o[256];
    for (int t = c0; t < c1; t++) if (sc[t] > m) m = sc[t];
    for (int i = 0; i < hd; i++) o[i] = 0.0f;
    for (int t = c0; t < c1; t++) {
      float e = orc_fast_exp(sc[t] - m);
      sum += e;
      for (int i = 0; i < hd; i++) o[i] = o[i] + e * vb[(size_t)t * hd + i];
    }
    float nm = m > M ? m : M, a = expf(M - nm), b = expf(m - nm);
    for (int i = 0; i < hd; i++) acc[i] = acc[i] * a + o[i] * b;
    S = S * a + sum * b;
    M = nm;
  }
  for (int i = 0; i < hd; i++) out[i] = acc[i] / S;
}

typedef struct { const uint8_t* qs; const float* d; } Q4;
typedef struct { const int8_t* qs; const float* d; } Q8;
typedef struct { const float *attn_norm, *ffn_norm, *bqkv; Q4 qkv, o, gu, down; } Layer;

struct orc_model {
  int dim, layers, ffn, heads, kvh, hd, vocab, ctx, mt, threads;
  int variant;     /* ORC_V_* bits; 0 = the reference's arithmetic */
  float eps;
  Q4 embd; Q8 out; const float* out_norm;
  Layer L[ORC_MAXL];
  float* rope;
  float *x, *xn, *qkv, *att, *gu, *act, *logits, *kc, *vc, *scores;
  int8_t* aq; float *ad, *as;
  int* tokens;
};

orc_model* orc_create(int dim, int layers, int ffn, int heads, int kvh, int vocab, int ctx, int mt,
                      float eps, double rope_theta, int threads) {
  if (layers > ORC_MAXL || heads <= 0 || dim % heads || (dim / heads) % 4 || dim % 32 || ffn % 32) return NULL;
  orc_model* g = (orc_model*)calloc(1, sizeof(orc_model));
  if (!g) return NULL;
  g->dim = dim; g->layers = layers; g->ffn = ffn; g->heads = heads; g->kvh = kvh; g->hd = dim / heads;
  g->vocab = vocab; g->ctx = ctx; g->mt = mt; g->eps = eps; g->threads = threads > 0 ? threads : 1;
  const int D = dim, F = ffn, HD = g->hd, QKV = D + 2 * kvh * HD, NL = layers, MT = mt;
  /* cpu-worker.js:69-73 */
  g->x = (float*)calloc((size_t)MT * D, 4); g->xn = (float*)calloc((size_t)MT * D, 4);
  g->qkv = (float*)calloc((size_t)MT * QKV, 4); g->att = (float*)calloc((size_t)MT * D, 4);
  g->gu = (float*)calloc((size_t)MT * 2 * F, 4); g->act = (float*)calloc((size_t)MT * F, 4);
  g->logits = (float*)calloc((size_t)vocab, 4);
  g->kc = (float*)calloc((size_t)NL * kvh * ctx * HD, 4); g->vc = (float*)calloc((size_t)NL * kvh * ctx * HD, 4);
  g->scores = (float*)calloc((size_t)g->threads * ctx, 4);
  g->aq = (int8_t*)calloc((size_t)MT * F, 1); g->ad = (float*)calloc((size_t)MT * F / 32, 4);
  g->as = (float*)calloc((size_t)MT * F / 32, 4);
  g->rope = (float*)calloc((size_t)ctx * HD, 4); g->tokens = (int*)calloc((size_t)ctx + 1, 4);
  if (!g->x || !g->xn || !g->qkv || !g->att || !g->gu || !g->act || !g->logits || !g->kc || !g->vc ||
      !g->scores || !g->aq || !g->ad || !g->as || !g->rope || !g->tokens) { orc_destroy(g); return NULL; }
  orc_rope_table(g->rope, ctx, HD, rope_theta);
  return g;
}

void orc_destroy(orc_model* g) {
  if (!g) return;
  free(g->x); free(g->xn); free(g->qkv); free(g->att); free(g->gu); free(g->act); free(g->logits);
  free(g->kc); free(g->vc); free(g->scores); free(g->aq); free(g->ad); free(g->as); free(g->rope);
  free(g->tokens); free(g);
}

void orc_set_threads(orc_model* g, int threads) {
  int t = threads > 0 ? threads : 1;
  if (t > g->threads) { free(g->scores); g->scores = (float*)calloc((size_t)t * g->ctx, 4); }
  g->threads = t;
}

/* kernels.c:423-431 */
void orc_set_tensor(orc_model* g, int kind, int layer, const void* qs, const float* d) {
  Layer* L = &g->L[layer];
  Q4 q4 = { (const uint8_t*)qs, d };
  switch (kind) {
    case 0: L->qkv = q4; break;   case 1: L->o = q4; break;
    case 2: L->gu = q4; break;    case 3: L->down = q4; break;
    case 4: L->attn_norm = d; break;   case 5: L->ffn_norm = d; break;   case 6: L->bqkv = d; break;
    case 7: g->embd = q4; break;
    case 8: g->out.qs = (const int8_t*)qs; g->out.d = d; break;
    case 9: g->out_norm = d; break;
  }
}

static void matmul_mt(orc_model* g, Q4 W, int K, int N, int M, float* y, int op, const float* bias) {
  const int nth = g->threads;
  if (g->variant & ORC_V_DOT_SPLITK) {
    const int nb = K / 32;
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int n = 0; n < N; n++)
      for (int m = 0; m < M; m++)
        put(y, N, m, n, dot_q4_q8_splitk(W.qs + (size_t)n * nb * 16, W.d + (size_t)n * nb, g->aq + (size_t)m * K,
                                         g->ad + (size_t)m * nb, nb), op, bias);
    return;
  }
  /* rows split in contiguous ranges, like split() (kernels.c:63-66) */
  #pragma omp parallel for schedule(static) num_threads(nth)
  for (int t = 0; t < nth; t++) {
    int per = (N + nth - 1) / nth, a = t * per, b = a + per > N ? N : a + per;
    if (a < b) orc_matmul_q4(W.qs, W.d, K, N, a, b, M, g->aq, g->ad, y, op, bias);
  }
}

static void rmsnorm_v(const orc_model* g, float* out, const float* x, const float* w, int n) {
  if (g->variant & ORC_V_NORM_TREE) rmsnorm_tree(out, x, w, n, g->eps);
  else orc_rmsnorm(out, x, w, n, g->eps);
}

/* kernels.c:306-415 */
void orc_run(orc_model* g, int pos0, int M, int want_logits) {
  const int D = g->dim, F = g->ffn, H = g->heads, KVH = g->kvh, HD = g->hd, QKV = D + 2 * KVH * HD;
  const int nth = g->threads;

  /* embedding rows, Q4_0 (kernels.c:312-322) */
  for (int m = 0; m < M; m++) {
    int t = g->tokens[pos0 + m];
    orc_embed_row(g->x + (size_t)m * D, g->embd.qs + (size_t)t * (D / 32) * 16, g->embd.d + (size_t)t * (D / 32), D);
  }

  for (int l = 0; l < g->layers; l++) {
    const Layer* L = &g->L[l];
    for (int m = 0; m < M; m++) {                                          /* :328-331 */
      rmsnorm_v(g, g->xn + (size_t)m * D, g->x + (size_t)m * D, L->attn_norm, D);
      orc_quantize_row(g->aq + (size_t)m * D, g->ad + (size_t)m * (D / 32), g->as + (size_t)m * (D / 32),
                       g->xn + (size_t)m * D, D);
    }
    matmul_mt(g, L->qkv, D, QKV, M, g->qkv, 1, L->bqkv);                    /* :333-334 */
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int task = 0; task < M * (H + KVH); task++) {                     /* :337-352 */
      int m = task / (H + KVH), h = task % (H + KVH), pos = pos0 + m;
      float* v = g->qkv + (size_t)m * QKV + h * HD;
      orc_rope_head(v, g->rope + (size_t)pos * HD, HD);
      if (h >= H) {
        int kh = h - H;
        float* kd = g->kc + (((size_t)l * KVH + kh) * g->ctx + pos) * HD;
        float* vd = g->vc + (((size_t)l * KVH + kh) * g->ctx + pos) * HD;
        const float* vs = g->qkv + (size_t)m * QKV + D + KVH * HD + kh * HD;
        if (g->variant & ORC_V_KV_F16)
          for (int i = 0; i < HD; i++) { kd[i] = orc_round_f16(v[i]); vd[i] = orc_round_f16(vs[i]); }
        else
          for (int i = 0; i < HD; i++) { kd[i] = v[i]; vd[i] = vs[i]; }
      }
    }
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int task = 0; task < M * H; task++) {                             /* :355-377 */
      int m = task / H, h = task % H, T = pos0 + m + 1, kh = h / (H / KVH);
      const float* q = g->qkv + (size_t)m * QKV + h * HD;
      const float* kb = g->kc + ((size_t)l * KVH + kh) * g->ctx * HD;
      const float* vb = g->vc + ((size_t)l * KVH + kh) * g->ctx * HD;
      if (g->variant & ORC_V_ATTN_SPLIT)
        attend_split(q, kb, vb, T, HD, g->scores + (size_t)omp_get_thread_num() * g->ctx, g->att + (size_t)m * D + h * HD);
      else
        orc_attend(q, kb, vb, T, HD, g->scores + (size_t)omp_get_thread_num() * g->ctx,
                   g->att + (size_t)m * D + h * HD);
    }
    for (int m = 0; m < M; m++)                                            /* :379, quantize_tokens :275-277 */
      orc_quantize_row(g->aq + (size_t)m * D, g->ad + (size_t)m * (D / 32), g->as + (size_t)m * (D / 32),
                       g->att + (size_t)m * D, D);
    matmul_mt(g, L->o, D, D, M, g->x, 2, NULL);                             /* :381-382 */
    for (int m = 0; m < M; m++) {                                          /* :385-388 */
      rmsnorm_v(g, g->xn + (size_t)m * D, g->x + (size_t)m * D, L->ffn_norm, D);
      orc_quantize_row(g->aq + (size_t)m * D, g->ad + (size_t)m * (D / 32), g->as + (size_t)m * (D / 32),
                       g->xn + (size_t)m * D, D);
    }
    matmul_mt(g, L->gu, D, 2 * F, M, g->gu, 0, NULL);                       /* :390-391 */
    for (int m = 0; m < M; m++) {                                          /* :393-397 */
      float* gu = g->gu + (size_t)m * 2 * F;
      float* ac = g->act + (size_t)m * F;
      orc_swiglu(ac, gu, gu + F, F);
      orc_quantize_row(g->aq + (size_t)m * F, g->ad + (size_t)m * (F / 32), g->as + (size_t)m * (F / 32), ac, F);
    }
    matmul_mt(g, L->down, F, D, M, g->x, 2, NULL);                          /* :399-400 */
  }

  if (want_logits) {                                                       /* :404-414 */
    rmsnorm_v(g, g->xn, g->x + (size_t)(M - 1) * D, g->out_norm, D);
    orc_quantize_row(g->aq, g->ad, g->as, g->xn, D);
    const int nb = D / 32, V = g->vocab;
    #pragma omp parallel for schedule(static) num_threads(nth)
    for (int n = 0; n < V; n++)
      g->logits[n] = orc_dot_q8_q8(g->out.qs + (size_t)n * D, g->out.d + (size_t)n * nb, g->aq, g->ad, nb);
  }
}

/* cpu-worker.js:169-182 (greedy only): chunk of at most mt tokens per run(), logits from the last chunk */
int orc_forward(orc_model* g, const int* ids, int n, int pos) {
  if (n <= 0 || pos < 0 || pos + n >= g->ctx) return -1;     /* "context full" */
  memcpy(g->tokens + pos, ids, (size_t)n * sizeof(int));
  for (int c = 0; c < n; c += g->mt) {
    int k = n - c < g->mt ? n - c : g->mt;
    orc_run(g, pos + c, k, c + k >= n ? 1 : 0);
  }
  return orc_argmax(g->logits, g->vocab);
}

const float* orc_logits(const orc_model* g) { return g->logits; }
void orc_set_variant(orc_model* g, int flags) { g->variant = flags; }
float* orc_kcache(orc_model* g) { return g->kc; }
float* orc_vcache(orc_model* g) { return g->vc; }
float* orc_hidden(orc_model* g) { return g->x; }
int* orc_tokens(orc_model* g) { return g->tokens; }
