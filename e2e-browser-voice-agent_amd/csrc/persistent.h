// persistent.h -- the decode step as one persistent launch (one or many greedy steps per launch).
//
// A kernel-per-operation step is ~245 dependent launches of 2.5-20 us each.  Here every workgroup
// (one per CU) stays resident and takes one role for the whole launch:
//   OD  (D/16 WGs)   rows 16w..16w+15 of o and down; owns those rows of the residual x
//   A   (heads WGs)  one attention head: its q rows and its kv group's k, v rows (the k/v rows are
//                    recomputed by the heads of a group instead of exchanged), RoPE, K/V append,
//                    attention
//   GU  (F/32 WGs)   gate and up rows of one 32-value block of the SwiGLU activation, quantized
//   all              the output head (rows round-robin), then the greedy argmax
// Four exchanges per layer (att -> OD, x after o -> GU, act -> OD, x after down -> A) and one per
// step (argmax).  Each exchanged value is stored together with the epoch of the phase that wrote it
// in one 8-byte agent-scope store ("LL" store): a reader polls the data itself, so a hand-off is
// one hop, and a thread's entries are all in flight at once.  Every role issues the loads of its
// next weights (and the attention role its past K/V rows) before it waits, so that traffic overlaps
// the waits.  Waits are bounded: a timeout raises State::abort and every workgroup exits.
//
// Arithmetic per output is the one of kernels.h (the reference's lane order), so results are
// bit-identical to the kernel-per-operation path.
#pragma once
#include "kernels.h"

namespace q4 {

struct LayerView {
  Q4Mat qkv, o, gu, down;
  const float* attn_norm;
  const float* ffn_norm;
  const float* bqkv;
};

struct PArgs {
  int D, F, H, KVH, QKV, V, NL, ctx;
  float eps;
  const uint8_t* embd;
  const float* out_norm;
  Q4Mat head;
  const LayerView* layers;
  const float* rope;
  float* kc;
  float* vc;
  float* logits;
  int* tokens;
  State* st;
  uint64_t* ll;   // exchange area: X1[D] X2[D] ATT[D] ACT[F/32*9] ARG[2G] (value, index pairs)
  int steps;
  int nOD, nA, nGU;
  int kv_tile;    // past positions of K and V the attention role stages in shared memory
  unsigned long long* prof;   // optional: phase timestamps of step 0, [(NL + 1) * 16]
};

constexpr int kPThreads = 256;
constexpr int kSpinLimit = 1 << 21;
constexpr int kHD = 64;           // head_dim of the persistent path
constexpr int kKVRow = 68;        // floats per staged K/V row (64 + 4: conflict-free row-per-thread reads)
constexpr int kRecvD = 4;         // LL entries per thread for D-vectors (D <= 1024)
constexpr int kRecvAct = 6;       // LL entries per thread for the quantized activation (9 * F/32 <= 1536)

// ---------------------------------------------------------------- memory helpers

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 GlobalU32x4;
typedef __attribute__((address_space(1))) const f32x4 GlobalF32x4;
typedef __attribute__((address_space(1))) const float GlobalF32;

// Weights and the K/V cache live in global memory; pointers read from the device layer table are
// generic, so load through explicit global-address-space pointers (global_load, not flat_load).
__device__ __forceinline__ uint4 gld(const uint4* p) {
  const u32x4 v = *(GlobalU32x4*)(const void*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gld4f(const float* p) {
  const f32x4 v = *(GlobalF32x4*)(const void*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float gldf(const float* p) { return *(GlobalF32*)(const void*)p; }

__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- LL exchange

__device__ __forceinline__ void ll_put(uint64_t* p, uint32_t payload, uint32_t ep) {
  __hip_atomic_store(p, ((uint64_t)ep << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ll_peek(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait for entries base[tid + 256k] (k < K, index < n) to carry epoch ep.  All K loads are in
// flight together and only the entries still missing are polled again, so a hand-off costs one
// memory round trip however many entries a thread receives.  Bounded: after kSpinLimit polls the
// thread raises st->abort; a raised flag makes every waiter give up (`bad`).
template <int K>
__device__ __forceinline__ void ll_recv(const uint64_t* base, int n, uint32_t ep, State* st, bool& bad,
                                        uint32_t (&out)[K]) {
  uint64_t w[K];
#pragma unroll
  for (int k = 0; k < K; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    w[k] = i < n ? ll_peek(base + i) : ((uint64_t)ep << 32);
  }
  int spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < K; k++) ok = ok && (uint32_t)(w[k] >> 32) == ep;
    if (ok || bad) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < K; k++) {
      const int i = (int)threadIdx.x + 256 * k;
      if (i < n && (uint32_t)(w[k] >> 32) != ep) w[k] = ll_peek(base + i);
    }
    if (++spins > kSpinLimit) {
      bad = true;
      __hip_atomic_store(&st->abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if ((spins & 255) == 0 && __hip_atomic_load(&st->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      bad = true;
    }
  }
#pragma unroll
  for (int k = 0; k < K; k++) out[k] = (uint32_t)w[k];
}

// ---------------------------------------------------------------- register-resident weights

// Groups [g0, g0+ng) (g0 even) of one 16-row group, lane (r, j): word j of 4 blocks per group and
// the fp16 scales of 8 blocks per uint4.
template <int NG>
struct RG {
  uint4 w[NG];
  uint4 s[(NG + 1) / 2];
};

template <int NG>
__device__ __forceinline__ void rg_load(const Q4Mat& W, int rg16, int r, int j, int g0, int ng, RG<NG>& R) {
  const int row = rg16 * 16 + r;
  const int tile = row >> 6, rr = row & 63;
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
#pragma unroll
  for (int g = 0; g < NG; g++) R.w[g] = g < ng ? gld(wq + (size_t)(g0 + g) * 256) : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int c = 0; c < (NG + 1) / 2; c++)
    R.s[c] = 2 * c < ng ? gld(wd + (size_t)(g0 / 2 + c) * 64) : make_uint4(0, 0, 0, 0);
}

// One block's term f32(p_j) * (dw * dx) (kernels.c:137); xv = {A_j, B_j, c_j, dx}.
template <int NG>
__device__ __forceinline__ float rg_term(const RG<NG>& R, int g, int k, uint4 xv) {
  const uint32_t wv = k == 0 ? R.w[g].x : k == 1 ? R.w[g].y : k == 2 ? R.w[g].z : R.w[g].w;
  const uint4 sv = R.s[g >> 1];
  const int hb = ((g & 1) << 2) + k;
  const uint32_t sw = (hb >> 1) == 0 ? sv.x : (hb >> 1) == 1 ? sv.y : (hb >> 1) == 2 ? sv.z : sv.w;
  const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
  int p = sdot4(wv & 0x0F0F0F0Fu, xv.x, (int)xv.z);
  p = sdot4((wv >> 4) & 0x0F0F0F0Fu, xv.y, p);
  return (float)p * (dw * __uint_as_float(xv.w));
}

// The four activation blocks of group g for lane j (zero past nb).
__device__ __forceinline__ void xg_load(const uint4* xs, int g, int nb, int j, uint4 (&xv)[4]) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int b = g * 4 + k;
    xv[k] = b < nb ? xs[b * 4 + j] : make_uint4(0, 0, 0, 0);
  }
}

// acc_i = acc_i + term for N row groups sharing each activation read, blocks of groups
// [g0, g0+ng) in order (kernels.c:217-218); the next group's activation blocks are read ahead.
template <int NG, int N>
__device__ __forceinline__ void rg_dot(const RG<NG> (&R)[N], int g0, int ng, int nb, const uint4* xs, int j,
                                       float (&acc)[N]) {
  uint4 xa[4], xb[4];
  if (ng > 0) xg_load(xs, g0, nb, j, xa);
#pragma unroll
  for (int g = 0; g < NG; g++) {
    if (g < ng) {
      if (g + 1 < ng) xg_load(xs, g0 + g + 1, nb, j, xb);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if ((g0 + g) * 4 + k < nb) {
#pragma unroll
          for (int n = 0; n < N; n++) acc[n] = acc[n] + rg_term(R[n], g, k, xa[k]);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; k++) xa[k] = xb[k];
    }
  }
}

// The same terms written to shared memory, terms[b * 64 + lane], for a serial pass by one wave.
template <int NG>
__device__ __forceinline__ void rg_terms(const RG<NG>& R, int g0, int ng, int nb, const uint4* xs, int j,
                                         float* terms, int lane) {
  uint4 xa[4], xb[4];
  if (ng > 0) xg_load(xs, g0, nb, j, xa);
#pragma unroll
  for (int g = 0; g < NG; g++) {
    if (g < ng) {
      if (g + 1 < ng) xg_load(xs, g0 + g + 1, nb, j, xb);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int b = (g0 + g) * 4 + k;
        if (b < nb) terms[b * 64 + lane] = rg_term(R, g, k, xa[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) xa[k] = xb[k];
    }
  }
}

// ((0 + t_0) + t_1) + ... over the blocks, the accumulation order of one reference lane; loads run
// 8 blocks ahead of the additions.
__device__ __forceinline__ float serial_sum(const float* terms, int nb, int lane) {
  float acc = 0.0f;
  float cur[8], nxt[8];
#pragma unroll
  for (int u = 0; u < 8; u++) cur[u] = u < nb ? terms[u * 64 + lane] : 0.0f;
  for (int b = 0; b < nb; b += 8) {
#pragma unroll
    for (int u = 0; u < 8; u++) nxt[u] = b + 8 + u < nb ? terms[(b + 8 + u) * 64 + lane] : 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (b + u < nb) acc = acc + cur[u];
#pragma unroll
    for (int u = 0; u < 8; u++) cur[u] = nxt[u];
  }
  return acc;
}

// Sum of x[0..n) in index order (n a multiple of 4, x 16-byte aligned), 16 values loaded ahead.
__device__ __forceinline__ float serial_sum_vec(const float* x, int n) {
  const float4* p = reinterpret_cast<const float4*>(x);
  const int n4 = n >> 2;
  float acc = 0.0f;
  float4 cur[4], nxt[4];
#pragma unroll
  for (int u = 0; u < 4; u++) cur[u] = u < n4 ? p[u] : make_float4(0, 0, 0, 0);
  for (int b = 0; b < n4; b += 4) {
#pragma unroll
    for (int u = 0; u < 4; u++) nxt[u] = b + 4 + u < n4 ? p[b + 4 + u] : make_float4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      if (b + u < n4) {
        acc = acc + cur[u].x;
        acc = acc + cur[u].y;
        acc = acc + cur[u].z;
        acc = acc + cur[u].w;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) cur[u] = nxt[u];
  }
  return acc;
}

// Even-aligned split of ng groups over the 4 waves.
__device__ __forceinline__ void wave_range(int ng, int wave, int& g0, int& cnt) {
  const int per = (((ng + 3) >> 2) + 1) & ~1;
  g0 = wave * per;
  cnt = ng - g0 < per ? ng - g0 : per;
  if (cnt < 0) cnt = 0;
}

__device__ __forceinline__ float embed_value(const uint8_t* emb, int D, int t, int i) {
  const uint8_t* bp = emb + ((size_t)t * (D / 32) + (i >> 5)) * 18;
  const float d = half_bits_to_float((uint32_t)bp[0] | ((uint32_t)bp[1] << 8));
  const int e = i & 31;
  const int q = bp[2 + (e & 15)];
  return (float)((e < 16 ? (q & 15) : (q >> 4)) - 8) * d;
}

// ---------------------------------------------------------------- shared memory plan

struct PSmem {
  float* xl;      // (D + 16) floats: a row staged by lane (run stride D/4 + 4), or plain
  uint4* xq;      // activation blocks, max(nbD, nbF) * 4
  float* terms;   // 64 * max(nbD, nbF) floats; attention scores; raw exchange entries
  uint4* tq;      // 4 (GU quantized block)
  float* red;     // 16
  float* qv;      // 3 * 64: q, k, v of one head
  float* own;     // 16 residual rows (OD)
  float* gu;      // 64: gate, up (GU)
  float* argv;    // 256
  int* argi;      // 256
  float* kvt;     // kv_tile * 2 * kKVRow: staged past K and V rows (A)
};

__host__ __device__ inline size_t psmem_base_bytes(int D, int F) {
  const int nbm = (D > F ? D : F) / 32;
  size_t b = (size_t)(D + 16) * 4;
  b += (size_t)nbm * 64;
  b += (size_t)64 * nbm * 4;
  b += (16 + 16 + 192 + 16 + 64 + 256 + 256) * 4;
  return b;
}

__host__ __device__ inline size_t psmem_bytes(int D, int F, int kv_tile) {
  return psmem_base_bytes(D, F) + (size_t)kv_tile * 2 * kKVRow * 4;
}

__device__ __forceinline__ PSmem psmem(unsigned char* base, int D, int F) {
  const int nbm = (D > F ? D : F) / 32;
  PSmem m;
  size_t off = 0;
  m.xl = (float*)(base + off);
  off += (size_t)(D + 16) * 4;
  m.xq = (uint4*)(base + off);
  off += (size_t)nbm * 64;
  m.terms = (float*)(base + off);
  off += (size_t)64 * nbm * 4;
  m.tq = (uint4*)(base + off);
  off += 16 * 4;
  m.red = (float*)(base + off);
  off += 16 * 4;
  m.qv = (float*)(base + off);
  off += 192 * 4;
  m.own = (float*)(base + off);
  off += 16 * 4;
  m.gu = (float*)(base + off);
  off += 64 * 4;
  m.argv = (float*)(base + off);
  off += 256 * 4;
  m.argi = (int*)(base + off);
  off += 256 * 4;
  m.kvt = (float*)(base + off);
  return m;
}

__device__ __forceinline__ uint32_t phase_epoch(uint32_t ep0, int s, int E, int code) {
  return ep0 + (uint32_t)(s * E + code) + 1u;
}

__device__ __forceinline__ int run_stride(int D) { return D / 4 + 4; }

// Wait for the D-vector `src` (epoch ep) and stage it by lane into xl.
__device__ __forceinline__ void recv_x(const uint64_t* src, int D, uint32_t ep, State* st, float* xl, bool& bad) {
  const int stv = run_stride(D);
  uint32_t v[kRecvD];
  ll_recv<kRecvD>(src, D, ep, st, bad, v);
#pragma unroll
  for (int k = 0; k < kRecvD; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    if (i < D) xl[(i & 3) * stv + (i >> 2)] = __uint_as_float(v[k]);
  }
}

// RMSNorm + quantize the staged row into m.xq (kernels.c:80-86, 328-331).  Threads 0..3 run the
// four lane sums of x*x, each over its contiguous run, 16 values loaded ahead.
__device__ __forceinline__ void norm_quant(const PSmem m, int D, const float* w, float eps) {
  const int stv = run_stride(D), tid = threadIdx.x;
  if (tid < 4) {
    const float4* p = reinterpret_cast<const float4*>(m.xl + tid * stv);
    const int n4 = D >> 4;
    float s = 0.0f;
    float4 cur[4], nxt[4];
#pragma unroll
    for (int u = 0; u < 4; u++) cur[u] = u < n4 ? p[u] : make_float4(0, 0, 0, 0);
    for (int b = 0; b < n4; b += 4) {
#pragma unroll
      for (int u = 0; u < 4; u++) nxt[u] = b + 4 + u < n4 ? p[b + 4 + u] : make_float4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        if (b + u < n4) {
          s = s + cur[u].x * cur[u].x;
          s = s + cur[u].y * cur[u].y;
          s = s + cur[u].z * cur[u].z;
          s = s + cur[u].w * cur[u].w;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) cur[u] = nxt[u];
    }
    m.red[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    const float ss = m.red[0] + m.red[1] + m.red[2] + m.red[3];
    m.red[4] = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
  }
  __syncthreads();
  quantize_row_dev<QM_NORM>(nullptr, m.xl, stv, D, w, m.red[4], m.xq, tid, kPThreads);
  __syncthreads();
}

// (value, index) merge with the first-maximum rule of cpu-worker.js:157.
__device__ __forceinline__ void arg_merge(float& bv, int& bi, float v, int i) {
  if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
}

__device__ __forceinline__ void prof_mark(const PArgs a, int s, int slot) {
  if (a.prof && s == 0 && threadIdx.x == 0) a.prof[slot] = wall_clock64();
}

// ---------------------------------------------------------------- the output head + argmax

template <int NGD>
__device__ __forceinline__ void head_rows(const PArgs a, const PSmem m, const RG<NGD> (&R)[1], int rg, int ngD,
                                          int nbD, int r, int j, float& bv, int& bi) {
  float acc[1] = {0.0f};
  rg_dot<NGD, 1>(R, 0, ngD, nbD, m.xq, j, acc);
  const float v = hsum4(acc[0]);
  const int row = rg * 16 + r;
  if (j == 0 && row < a.V) {
    a.logits[row] = v;
    arg_merge(bv, bi, v, row);
  }
}

template <int NGD>
__device__ __forceinline__ int head_phase(const PArgs a, const PSmem m, int s, int pos, uint32_t ep0, int E,
                                          bool& bad) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int G = gridDim.x, wg = blockIdx.x, D = a.D, nbD = D / 32;
  const Q4Mat& W = a.head;
  const int ngD = W.ng;
  const int nRG = W.Np / 16;
  uint64_t* LX2 = a.ll + a.D;
  uint64_t* LARG = a.ll + 3 * a.D + (a.F / 32) * 9;
  const uint32_t epx = phase_epoch(ep0, s, E, 4 * (a.NL - 1) + 3);
  const uint32_t eph = phase_epoch(ep0, s, E, 4 * a.NL);

  // the first two row groups' weights are in flight before waiting for x
  const int stride = 4 * G;
  int rgi = wg + G * wave;
  RG<NGD> R0[1], R1[1], R2[1];
  if (rgi < nRG) rg_load<NGD>(W, rgi, r, j, 0, ngD, R0[0]);
  if (rgi + stride < nRG) rg_load<NGD>(W, rgi + stride, r, j, 0, ngD, R1[0]);
  recv_x(LX2, D, epx, a.st, m.xl, bad);
  if (__syncthreads_or(bad)) return -1;
  prof_mark(a, s, a.NL * 16 + 0);
  norm_quant(m, D, a.out_norm, a.eps);

  float bv = 0.0f;
  int bi = -1;
  // three rotating buffers: two row groups in flight while one is computed
  while (rgi < nRG) {
    if (rgi + 2 * stride < nRG) rg_load<NGD>(W, rgi + 2 * stride, r, j, 0, ngD, R2[0]);
    head_rows<NGD>(a, m, R0, rgi, ngD, nbD, r, j, bv, bi);
    rgi += stride;
    if (rgi >= nRG) break;
    if (rgi + 2 * stride < nRG) rg_load<NGD>(W, rgi + 2 * stride, r, j, 0, ngD, R0[0]);
    head_rows<NGD>(a, m, R1, rgi, ngD, nbD, r, j, bv, bi);
    rgi += stride;
    if (rgi >= nRG) break;
    if (rgi + 2 * stride < nRG) rg_load<NGD>(W, rgi + 2 * stride, r, j, 0, ngD, R1[0]);
    head_rows<NGD>(a, m, R2, rgi, ngD, nbD, r, j, bv, bi);
    rgi += stride;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    arg_merge(bv, bi, ov, oi);
  }
  if (lane == 0) { m.argv[wave] = bv; m.argi[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; w++) arg_merge(bv, bi, m.argv[w], m.argi[w]);
    ll_put(LARG + 2 * wg, __float_as_uint(bv), eph);
    ll_put(LARG + 2 * wg + 1, (uint32_t)bi, eph);
  }
  prof_mark(a, s, a.NL * 16 + 1);
  // everyone reduces everyone's (value, index): the same token in every workgroup
  uint32_t* raw = (uint32_t*)m.terms;
  {
    uint32_t v[2];
    ll_recv<2>(LARG, 2 * G, eph, a.st, bad, v);
    raw[tid] = v[0];
    if (tid + 256 < 2 * G) raw[tid + 256] = v[1];
  }
  if (__syncthreads_or(bad)) return -1;
  bv = 0.0f;
  bi = -1;
  for (int g = tid; g < G; g += kPThreads) arg_merge(bv, bi, __uint_as_float(raw[2 * g]), (int)raw[2 * g + 1]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    arg_merge(bv, bi, ov, oi);
  }
  __syncthreads();
  if (lane == 0) { m.argv[wave] = bv; m.argi[wave] = bi; }
  __syncthreads();
  bv = m.argv[0];
  bi = m.argi[0];
  for (int w = 1; w < 4; w++) arg_merge(bv, bi, m.argv[w], m.argi[w]);
  __syncthreads();
  const int next = bi < 0 ? 0 : bi;
  if (wg == 0 && tid == 0) a.tokens[pos + 1] = next;
  prof_mark(a, s, a.NL * 16 + 2);
  if (a.prof && s == 0 && wg == 0 && tid == 0) a.prof[a.NL * 16 + 5] = clock64();
  return next;
}

// ---------------------------------------------------------------- roles

// o and down rows 16w..16w+15; the residual x of those rows lives in m.own.
template <int NGO, int NGDN, int NGD>
__device__ __forceinline__ void role_od(const PArgs a, const PSmem m, uint32_t ep0, int pos, int tok) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int wg = blockIdx.x, D = a.D, nbD = D / 32, nbF = a.F / 32, E = 4 * a.NL + 1;
  const int row = wg * 16 + r;
  uint64_t* LX1 = a.ll;
  uint64_t* LX2 = a.ll + D;
  uint64_t* LATT = a.ll + 2 * D;
  uint64_t* LACT = a.ll + 3 * D;
  bool bad = false;
  for (int s = 0; s < a.steps; s++, pos++) {
    if (tid < 16) m.own[tid] = embed_value(a.embd, D, tok, wg * 16 + tid);
    for (int l = 0; l < a.NL; l++) {
      const LayerView L = a.layers[l];
      int g0, cnt;
      // ---- o: x1 = x + W_o . quantize(att)
      wave_range(L.o.ng, wave, g0, cnt);
      RG<NGO> ro;
      rg_load<NGO>(L.o, wg, r, j, g0, cnt, ro);
      const uint32_t ep_att = phase_epoch(ep0, s, E, 4 * l + 0);
      {
        uint32_t v[kRecvD];
        ll_recv<kRecvD>(LATT, D, ep_att, a.st, bad, v);
#pragma unroll
        for (int k = 0; k < kRecvD; k++)
          if (tid + 256 * k < D) m.xl[tid + 256 * k] = __uint_as_float(v[k]);
      }
      if (__syncthreads_or(bad)) return;
      if (wg == 0) prof_mark(a, s, l * 16 + 0);
      quantize_row_dev<QM_PLAIN>(m.xl, nullptr, 0, D, nullptr, 0.0f, m.xq, tid, kPThreads);
      __syncthreads();
      rg_terms<NGO>(ro, g0, cnt, nbD, m.xq, j, m.terms, lane);
      __syncthreads();
      if (wave == 0) {
        const float v = hsum4(serial_sum(m.terms, nbD, lane));
        if (j == 0) {
          const float x1 = m.own[r] + v;
          m.own[r] = x1;
          ll_put(LX1 + row, __float_as_uint(x1), phase_epoch(ep0, s, E, 4 * l + 1));
        }
        if (wg == 0) prof_mark(a, s, l * 16 + 1);
      }
      // ---- down: x2 = x1 + W_down . act (act arrives quantized)
      wave_range(L.down.ng, wave, g0, cnt);
      RG<NGDN> rd;
      rg_load<NGDN>(L.down, wg, r, j, g0, cnt, rd);
      const uint32_t ep_act = phase_epoch(ep0, s, E, 4 * l + 2);
      {
        uint32_t v[kRecvAct];
        uint32_t* raw = (uint32_t*)m.terms;
        ll_recv<kRecvAct>(LACT, nbF * 9, ep_act, a.st, bad, v);
        __syncthreads();   // wave 0's serial pass over m.terms has finished
#pragma unroll
        for (int k = 0; k < kRecvAct; k++)
          if (tid + 256 * k < nbF * 9) raw[tid + 256 * k] = v[k];
        if (__syncthreads_or(bad)) return;
        for (int b = tid; b < nbF; b += kPThreads) {
          uint32_t e[9];
#pragma unroll
          for (int k = 0; k < 9; k++) e[k] = raw[b * 9 + k];
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int c = -8 * (sdot4(e[jj], 0x01010101u, 0) + sdot4(e[4 + jj], 0x01010101u, 0));
            m.xq[b * 4 + jj] = make_uint4(e[jj], e[4 + jj], (uint32_t)c, e[8]);
          }
        }
        __syncthreads();
      }
      if (wg == 0) prof_mark(a, s, l * 16 + 2);
      rg_terms<NGDN>(rd, g0, cnt, nbF, m.xq, j, m.terms, lane);
      __syncthreads();
      if (wave == 0) {
        const float v = hsum4(serial_sum(m.terms, nbF, lane));
        if (j == 0) {
          const float x2 = m.own[r] + v;
          m.own[r] = x2;
          ll_put(LX2 + row, __float_as_uint(x2), phase_epoch(ep0, s, E, 4 * l + 3));
        }
        if (wg == 0) prof_mark(a, s, l * 16 + 3);
      }
      __syncthreads();
    }
    tok = head_phase<NGD>(a, m, s, pos, ep0, E, bad);
    if (tok < 0) return;
  }
  if (blockIdx.x == 0 && tid == 0) {
    a.st->pos0 = pos;
    a.st->next = tok;
    a.st->epoch = ep0 + (uint32_t)(a.steps * E) + 1u;
  }
}

// One attention head h: q rows of h and k, v rows of its kv group, RoPE, K/V append (first head of
// the group), attention over the cache (kernels.c:333-377).  Past K/V rows (up to kv_tile of them)
// are staged in shared memory while the role waits for x.
template <int NGD>
__device__ __forceinline__ void role_attn(const PArgs a, const PSmem m, uint32_t ep0, int pos, int tok) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int D = a.D, nbD = D / 32, E = 4 * a.NL + 1;
  const int h = blockIdx.x - a.nOD, grp = a.H / a.KVH, kh = h / grp;
  const bool writer = (h % grp) == 0;
  uint64_t* LX2 = a.ll + D;
  uint64_t* LATT = a.ll + 2 * D;
  const int rq = (h * kHD) / 16 + wave, rk = (D + kh * kHD) / 16 + wave, rv = (D + a.KVH * kHD + kh * kHD) / 16 + wave;
  float* qv = m.qv;
  float* kv = m.qv + 64;
  float* vv = m.qv + 128;
  float* sc = m.terms;
  float* kt = m.kvt;                              // [kv_tile][kKVRow] K
  float* vt = m.kvt + (size_t)a.kv_tile * kKVRow;  // [kv_tile][kKVRow] V
  bool bad = false;
  for (int s = 0; s < a.steps; s++, pos++) {
    const int nt = pos < a.kv_tile ? pos : a.kv_tile;    // staged past positions
    for (int l = 0; l < a.NL; l++) {
      const LayerView L = a.layers[l];
      const int ng = L.qkv.ng;
      RG<NGD> w3[3];
      rg_load<NGD>(L.qkv, rq, r, j, 0, ng, w3[0]);
      rg_load<NGD>(L.qkv, rk, r, j, 0, ng, w3[1]);
      rg_load<NGD>(L.qkv, rv, r, j, 0, ng, w3[2]);
      const size_t cbase = ((size_t)l * a.KVH + kh) * a.ctx * kHD;
      // stage K and V of positions [0, nt) (written by earlier steps or launches)
      for (int idx = tid; idx < nt * 32; idx += kPThreads) {
        const int which = idx >= nt * 16, rem = idx - which * nt * 16, t = rem >> 4, c4 = (rem & 15) * 4;
        const float4 v4 = gld4f((which ? a.vc : a.kc) + cbase + (size_t)t * kHD + c4);
        float* dst = (which ? vt : kt) + t * kKVRow + c4;
        *reinterpret_cast<float4*>(dst) = v4;
      }
      if (l == 0) {
        const int stv = run_stride(D);
        for (int i = tid; i < D; i += kPThreads) m.xl[(i & 3) * stv + (i >> 2)] = embed_value(a.embd, D, tok, i);
      } else {
        recv_x(LX2, D, phase_epoch(ep0, s, E, 4 * (l - 1) + 3), a.st, m.xl, bad);
      }
      if (__syncthreads_or(bad)) return;
      if (h == 0) prof_mark(a, s, l * 16 + 4);
      norm_quant(m, D, L.attn_norm, a.eps);
      float acc[3] = {0.0f, 0.0f, 0.0f};
      rg_dot<NGD, 3>(w3, 0, ng, nbD, m.xq, j, acc);
      const float q = hsum4(acc[0]), k = hsum4(acc[1]), v = hsum4(acc[2]);
      if (j == 0) {
        qv[16 * wave + r] = q + L.bqkv[rq * 16 + r];
        kv[16 * wave + r] = k + L.bqkv[rk * 16 + r];
        vv[16 * wave + r] = v + L.bqkv[rv * 16 + r];
      }
      __syncthreads();
      if (h == 0) prof_mark(a, s, l * 16 + 5);
      // RoPE (kernels.c:340-344): threads 0..31 rotate q pairs, 32..63 k pairs
      if (tid < 64) {
        const int i = tid & 31;
        float* x = tid < 32 ? qv : kv;
        const float c = a.rope[(size_t)pos * kHD + 2 * i], sn = a.rope[(size_t)pos * kHD + 2 * i + 1];
        const float x0 = x[i], x1 = x[i + 32];
        x[i] = x0 * c - x1 * sn;
        x[i + 32] = x1 * c + x0 * sn;
      }
      __syncthreads();
      if (writer && tid < 64) {
        st_coherent(a.kc + cbase + (size_t)pos * kHD + tid, kv[tid]);
        st_coherent(a.vc + cbase + (size_t)pos * kHD + tid, vv[tid]);
      }
      // scores: four lane sums over i = j mod 4, hsum, scale (kernels.c:362-366)
      const int T = pos + 1;
      const float scale = 1.0f / __builtin_sqrtf((float)kHD);
      float lmax = -1e30f;
      for (int t = tid; t < T; t += kPThreads) {
        float4 kk[kHD / 4];
        if (t == pos) {
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) kk[i] = reinterpret_cast<const float4*>(kv)[i];
        } else if (t < nt) {
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) kk[i] = reinterpret_cast<const float4*>(kt + t * kKVRow)[i];
        } else {
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) kk[i] = gld4f(a.kc + cbase + (size_t)t * kHD + 4 * i);
        }
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i = 0; i < kHD / 4; i++) {
          const float4 q4 = reinterpret_cast<const float4*>(qv)[i];
          s0 = s0 + q4.x * kk[i].x;
          s1 = s1 + q4.y * kk[i].y;
          s2 = s2 + q4.z * kk[i].z;
          s3 = s3 + q4.w * kk[i].w;
        }
        const float sv = (s0 + s1 + s2 + s3) * scale;
        sc[t] = sv;
        lmax = __builtin_fmaxf(lmax, sv);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) lmax = __builtin_fmaxf(lmax, __shfl_xor(lmax, o));
      if (lane == 0) m.red[wave] = lmax;
      __syncthreads();
      const float mx = __builtin_fmaxf(__builtin_fmaxf(m.red[0], m.red[1]), __builtin_fmaxf(m.red[2], m.red[3]));
      for (int t = tid; t < T; t += kPThreads) sc[t] = fast_exp(sc[t] - mx);
      __syncthreads();
      if (tid == 0) {
        const int T4 = T & ~3;
        float sum = serial_sum_vec(sc, T4);
        for (int t = T4; t < T; t++) sum = sum + sc[t];
        m.red[8] = sum;
      }
      __syncthreads();
      const float sum = m.red[8];
      for (int t = tid; t < T; t += kPThreads) sc[t] = sc[t] / sum;
      __syncthreads();
      // out_i = sum over t in order of p_t * v_t[i] (kernels.c:372-375)
      if (tid < kHD) {
        float accv = 0.0f;
        int t = 0;
        for (; t + 8 <= nt; t += 8) {
          float vx[8];
#pragma unroll
          for (int u = 0; u < 8; u++) vx[u] = vt[(t + u) * kKVRow + tid];
#pragma unroll
          for (int u = 0; u < 8; u++) accv = accv + sc[t + u] * vx[u];
        }
        for (; t < nt; t++) accv = accv + sc[t] * vt[t * kKVRow + tid];
        constexpr int TB = 32;     // positions past the staged tile: streamed, 32 loads ahead
        for (; t < pos; t += TB) {
          float vx[TB];
#pragma unroll
          for (int u = 0; u < TB; u++) vx[u] = t + u < pos ? gldf(a.vc + cbase + (size_t)(t + u) * kHD + tid) : 0.0f;
#pragma unroll
          for (int u = 0; u < TB; u++)
            if (t + u < pos) accv = accv + sc[t + u] * vx[u];
        }
        accv = accv + sc[pos] * vv[tid];
        ll_put(LATT + h * kHD + tid, __float_as_uint(accv), phase_epoch(ep0, s, E, 4 * l + 0));
      }
      if (h == 0) prof_mark(a, s, l * 16 + 6);
      __syncthreads();
    }
    tok = head_phase<NGD>(a, m, s, pos, ep0, E, bad);
    if (tok < 0) return;
  }
}

// One 32-value block u of the SwiGLU activation: gate rows 32u.., up rows F+32u.. (one 16-row
// group per wave), then silu(gate)*up and quantize_row of the block (kernels.c:390-397).
template <int NGD>
__device__ __forceinline__ void role_gu(const PArgs a, const PSmem m, uint32_t ep0, int pos, int tok) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int D = a.D, nbD = D / 32, E = 4 * a.NL + 1;
  const int u = blockIdx.x - a.nOD - a.nA;
  const int rg = wave < 2 ? 2 * u + wave : a.F / 16 + 2 * u + (wave - 2);
  uint64_t* LX1 = a.ll;
  uint64_t* LACT = a.ll + 3 * D;
  bool bad = false;
  for (int s = 0; s < a.steps; s++, pos++) {
    for (int l = 0; l < a.NL; l++) {
      const LayerView L = a.layers[l];
      const int ng = L.gu.ng;
      RG<NGD> w[1];
      rg_load<NGD>(L.gu, rg, r, j, 0, ng, w[0]);
      recv_x(LX1, D, phase_epoch(ep0, s, E, 4 * l + 1), a.st, m.xl, bad);
      if (__syncthreads_or(bad)) return;
      if (u == 0) prof_mark(a, s, l * 16 + 7);
      norm_quant(m, D, L.ffn_norm, a.eps);
      float acc[1] = {0.0f};
      rg_dot<NGD, 1>(w, 0, ng, nbD, m.xq, j, acc);
      const float v = hsum4(acc[0]);
      if (j == 0) m.gu[16 * wave + r] = v;
      __syncthreads();
      if (tid < 4) quantize_row_dev<QM_SWIGLU>(m.gu, nullptr, 0, 32, nullptr, 0.0f, m.tq, tid, 4);
      __syncthreads();
      if (tid < 9) {
        const uint32_t pay = tid < 4 ? m.tq[tid].x : tid < 8 ? m.tq[tid - 4].y : m.tq[0].w;
        ll_put(LACT + u * 9 + tid, pay, phase_epoch(ep0, s, E, 4 * l + 2));
      }
      if (u == 0) prof_mark(a, s, l * 16 + 8);
      __syncthreads();
    }
    tok = head_phase<NGD>(a, m, s, pos, ep0, E, bad);
    if (tok < 0) return;
  }
}

template <int NGD>
__device__ __forceinline__ void role_head_only(const PArgs a, const PSmem m, uint32_t ep0, int pos, int tok) {
  const int E = 4 * a.NL + 1;
  bool bad = false;
  for (int s = 0; s < a.steps; s++, pos++) {
    tok = head_phase<NGD>(a, m, s, pos, ep0, E, bad);
    if (tok < 0) return;
  }
}

// NGD: groups of 4 blocks for K = D; NGO/NGDN: per-wave groups of o / down after the 4-way split.
template <int NGD, int NGO, int NGDN>
__global__ __launch_bounds__(kPThreads, 1) void k_decode_persistent(PArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const PSmem m = psmem(smem, a.D, a.F);
  const uint32_t ep0 = a.st->epoch;
  const int pos = a.st->pos0;
  const int tok = a.tokens[pos];
  const int wg = blockIdx.x;
  if (wg == 0) prof_mark(a, 0, a.NL * 16 + 3);
  if (a.prof && wg == 0 && threadIdx.x == 0) a.prof[a.NL * 16 + 4] = clock64();
  if (wg < a.nOD) role_od<NGO, NGDN, NGD>(a, m, ep0, pos, tok);
  else if (wg < a.nOD + a.nA) role_attn<NGD>(a, m, ep0, pos, tok);
  else if (wg < a.nOD + a.nA + a.nGU) role_gu<NGD>(a, m, ep0, pos, tok);
  else role_head_only<NGD>(a, m, ep0, pos, tok);
}

}  // namespace q4
