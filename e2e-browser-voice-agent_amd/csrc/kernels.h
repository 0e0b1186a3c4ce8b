// kernels.h -- device code of the Qwen2 Q4_0 token loop for gfx950 (CDNA4, wave64).
//
// Every kernel here reproduces the per-output floating-point operation order of the
// reference's CPU path (h2-own-inference-engine/engine/kernels.c, plain SIMD128 build), so
// logits agree bit for bit.  That matters more than it seems: activations are quantized to
// int8 per 32-block before every projection, and one rounding flip there moves an output
// by a whole quantization step (~1e-3 in the logits).  Floating-point operations are kept
// separate (the library is compiled with -ffp-contract=off); integer work is free to be
// reassociated because it is exact.
//
// Data layouts in HBM (all chosen for coalesced wave64 loads):
//  * Q4 matrix, N x K, nb = K/32 blocks per row, rows padded to a multiple of 64:
//      qs: u32 [N/64][nb][64 rows][4 words]   word j = GGUF bytes {2j, 2j+1, 8+2j, 9+2j}
//      d : f16 [N/64][nb8][64 rows][8]        nb8 = ceil(nb/8); the GGUF fp16 scale, unchanged
//    Word j holds, in its low nibbles, elements {2j,2j+1,8+2j,9+2j} of the block and, in its
//    high nibbles, elements {16+2j,17+2j,24+2j,25+2j}: exactly lane j of the reference's
//    i32x4 block dot (kernels.c:127-136).  One lane of the GPU owns one (row, j) pair.
//  * Quantized activation block (one per 32 values, 64 bytes): for j = 0..3, 16 bytes
//      { A_j, B_j, c_j, dx }: A_j = int8 x at {2j,2j+1,8+2j,9+2j}, B_j = at {16+2j,...},
//      c_j = -8 * (sum of those 8 int8 values), dx = the block scale (kernels.c:98,112).
//    Then sdot4(lo_nibbles, A_j, c_j) + sdot4(hi_nibbles, B_j) = sum (nib-8)*x over lane j.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace q4 {

constexpr int kRowTile = 64;        // rows per weight tile
constexpr int kMaxChunk = 16;       // the reference's prompt chunk (MT, engine/cpu.js:46): the per-token matvec's tile
constexpr int kMaxPass = 1024;      // tokens per device pass; results do not depend on the chunking

// Device-resident step state: pos0 of the current pass, last sampled token.  Kernels read
// pos0 from here so one captured graph replays every decode step.  The persistent decode kernel
// also keeps its exchange epoch here (so consecutive launches never reuse an epoch) and an abort
// flag that any workgroup raises when a bounded wait runs out.
struct State {
  int pos0;
  int next;
  unsigned epoch;
  int abort;
  int fail_phase;
  int pad[3];
};

// ---------------------------------------------------------------- arithmetic helpers

// e^x of kernels.c:69-78 (Cody-Waite reduction, degree-6 Taylor, exponent add), op for op.  The
// two range tests are selects rather than branches (the value computed for x < -87 is discarded).
__device__ __forceinline__ float fast_exp(float x) {
  const float xc = x > 88.0f ? 88.0f : x;
  float n = __builtin_floorf(xc * 1.44269504f + 0.5f);
  float r = xc - n * 0.693145752f - n * 1.42860677e-6f;
  float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.166666672f + r * (0.0416666679f +
            r * (0.00833333377f + r * 0.00138888892f)))));
  const float e = __uint_as_float(__float_as_uint(p) + ((uint32_t)(int32_t)n << 23));
  return x < -87.0f ? 0.0f : e;
}

// ---------------------------------------------------------------- cross-lane maxima

// Maximum over each quad of lanes (4k .. 4k+3, all active): two DPP quad permutations.
__device__ __forceinline__ float quad_max(float v) {
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));
  return v;
}

// Maximum over each group of 32 lanes (all active): quads, then the mirror within 8 and within 16
// lanes (every lane of a quad, then of an 8-group, holds the same value), then lane ^ 16.
__device__ __forceinline__ float max32(float v) {
  v = quad_max(v);
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  return v;
}

// Maximum over the whole wave (all 64 lanes active), the same in every lane.
__device__ __forceinline__ float max64(float v) {
  v = max32(v);
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return __builtin_fmaxf(lo, hi);
}

// ---------------------------------------------------------------- correctly rounded quotients
//
// The reference divides in IEEE binary32 (f32.div).  These forms give the same quotients from a
// product with a reciprocal and fused residual corrections (Markstein's method: P. Markstein,
// "Computation of elementary functions on the IBM RISC System/6000 processor", IBM J. Res. Dev.
// 34(1), 1990), each on a domain where it equals the IEEE quotient for every input — checked
// exhaustively by q4hip_check_division — and fall back to the IEEE division elsewhere.  The
// fallback sits behind a wave-uniform test, so it costs nothing unless some lane needs it.

// a / 127 for a >= 0 (the block scale d = amax / 127, kernels.c:98): exact for every finite a.
__device__ __forceinline__ float div_127(float a) {
  constexpr float c = 1.0f / 127.0f;
  const float q0 = a * c;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), c, q0);
  return a == __builtin_inff() ? a : q;
}

// d ? 1 / d : 0 for d >= 0 (kernels.c:99): the hardware reciprocal estimate and one correction are
// exact for d in [2^-126, 2^126).
__device__ __forceinline__ float inv_scale(float d) {
  const float y0 = __builtin_amdgcn_rcpf(d);
  const float y = __builtin_fmaf(__builtin_fmaf(-d, y0, 1.0f), y0, y0);
  const bool fast = d >= 0x1p-126f && d < 0x1p126f;
  if (__builtin_amdgcn_ballot_w64(!fast && d != 0.0f) == 0) return fast ? y : 0.0f;
  return fast ? y : (d != 0.0f ? 1.0f / d : 0.0f);
}

// 1 / d: exact for d in [2^-126, 2^126).
__device__ __forceinline__ float recip(float d) {
  const float y0 = __builtin_amdgcn_rcpf(d);
  const float y = __builtin_fmaf(__builtin_fmaf(-d, y0, 1.0f), y0, y0);
  const bool fast = d >= 0x1p-126f && d < 0x1p126f;
  if (__builtin_amdgcn_ballot_w64(!fast) == 0) return y;
  return fast ? y : 1.0f / d;
}

// a / N for a >= 0 and a compile-time N (the mean of squares of RMSNorm, kernels.c:84): a power of
// two is a product; N = 896 takes the corrected product for a in [2^-119, inf), exact there.
template <int N>
__device__ __forceinline__ float div_const(float a) {
  if constexpr ((N & (N - 1)) == 0) {
    return a * (1.0f / (float)N);
  } else if constexpr (N == 896) {
    constexpr float c = 1.0f / (float)N;
    const float q0 = a * c;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, (float)N, a), c, q0);
    const bool fast = a >= 0x1p-119f && a < __builtin_inff();
    if (__builtin_amdgcn_ballot_w64(!fast) == 0) return q;
    return fast ? q : a / (float)N;
  } else {
    return a / (float)N;
  }
}

// g / y for y = 1 + fast_exp(-g) (SiLU, kernels.c:395): the corrected product is exact for finite
// g != 0 with y < 2^126 (silu_fast_ok).
__device__ __forceinline__ float silu_quot(float g, float y) {
  const float y0 = __builtin_amdgcn_rcpf(y);
  const float y1 = __builtin_fmaf(__builtin_fmaf(-y, y0, 1.0f), y0, y0);
  const float q0 = g * y1;
  return __builtin_fmaf(__builtin_fmaf(-q0, y, g), y1, q0);
}

__device__ __forceinline__ bool silu_fast_ok(float g, float y) {
  return y < 0x1p126f && g != 0.0f && __builtin_fabsf(g) < __builtin_inff();
}

__device__ __forceinline__ float div_silu(float g, float y) {
  const float q = silu_quot(g, y);
  const bool fast = silu_fast_ok(g, y);
  if (__builtin_amdgcn_ballot_w64(!fast) == 0) return q;
  return fast ? q : g / y;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
}

// ---- the K/V cache element: fp32 (the reference's cache, kernels.c:347-350) or fp16 (half the
// bytes: values rounded to nearest, ties to even, when appended, and widened exactly when read)
typedef _Float16 kvhalf;
template <class KT>
__device__ __forceinline__ float4 kv_ld4(const KT* p);
template <>
__device__ __forceinline__ float4 kv_ld4<float>(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 kv_ld4<kvhalf>(const kvhalf* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(half_bits_to_float(u.x & 0xffffu), half_bits_to_float(u.x >> 16),
                     half_bits_to_float(u.y & 0xffffu), half_bits_to_float(u.y >> 16));
}

// Four consecutive cache values as loaded (kv_raw4) and widened to fp32 (kv_wide4): a register that
// carries cache values across a loop holds them in the loaded form, so that the loop does not wait
// for the load in flight to widen it before the values are used.
template <class KT> struct KvRaw { typedef float4 T; };
template <> struct KvRaw<kvhalf> { typedef uint2 T; };
template <class KT>
__device__ __forceinline__ typename KvRaw<KT>::T kv_raw4(const KT* p) {
  return *reinterpret_cast<const typename KvRaw<KT>::T*>(p);
}
__device__ __forceinline__ float4 kv_wide4(float4 r) { return r; }
__device__ __forceinline__ float4 kv_wide4(uint2 u) {
  return make_float4(half_bits_to_float(u.x & 0xffffu), half_bits_to_float(u.x >> 16),
                     half_bits_to_float(u.y & 0xffffu), half_bits_to_float(u.y >> 16));
}

// Eight consecutive cache values as two float4 (one 16-byte load for fp16, two for fp32).
template <class KT>
__device__ __forceinline__ void kv_ld8(const KT* p, float4& a, float4& b) {
  a = kv_ld4<KT>(p);
  b = kv_ld4<KT>(p + 4);
}
template <>
__device__ __forceinline__ void kv_ld8<kvhalf>(const kvhalf* p, float4& a, float4& b) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  a = make_float4(half_bits_to_float(u.x & 0xffffu), half_bits_to_float(u.x >> 16),
                  half_bits_to_float(u.y & 0xffffu), half_bits_to_float(u.y >> 16));
  b = make_float4(half_bits_to_float(u.z & 0xffffu), half_bits_to_float(u.z >> 16),
                  half_bits_to_float(u.w & 0xffffu), half_bits_to_float(u.w >> 16));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) |
         ((uint32_t)(d & 255) << 24);
}

// f32x4.nearest (ties to even), trunc_sat, then the two saturating narrows (kernels.c:102-107)
__device__ __forceinline__ int quant_one(float v) {
  float r = __builtin_rintf(v);
  if (r != r) return 0;                      // trunc_sat maps NaN to 0
  r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
  return (int)r;
}

__device__ __forceinline__ uint32_t pack_f16x2(int a, int b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}
// a / 16 and b / 16 as fp16 (exact for |a|, |b| <= 2048)
__device__ __forceinline__ uint32_t pack_f16x2_16th(int a, int b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)a * 0.0625f)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)b * 0.0625f)) << 16);
}

// A row of n floats staged in shared memory "by lane" (sq_stage): value i at xl[(i & 3) * st + (i >> 2)],
// st = n/4 + 1, so reference lane j (the values i = j mod 4, kernels.c:81-82) is one contiguous run
// and the four runs start in different banks.
__device__ __forceinline__ float lane_staged(const float* xl, int st, int i) {
  return xl[(i & 3) * st + (i >> 2)];
}

// ---------------------------------------------------------------- quantization

enum QuantMode { QM_PLAIN = 0, QM_NORM = 1, QM_SWIGLU = 2 };

// v = (g / (1 + fast_exp(-g))) * u for 8 values (kernels.c:395).  All 16 inputs are in hand before
// any test, and one wave-uniform test covers the 8 quotients (the exact fallback division only
// where a quotient leaves the domain of the fast form).
__device__ __forceinline__ void swiglu8(const float (&g)[8], const float (&u)[8], float (&v)[8]) {
  float y[8];
  bool fast = true;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    y[k] = 1.0f + fast_exp(-g[k]);
    v[k] = silu_quot(g[k], y[k]);
    fast = fast && silu_fast_ok(g[k], y[k]);
  }
  if (__builtin_amdgcn_ballot_w64(!fast) != 0) {
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (!silu_fast_ok(g[k], y[k])) v[k] = g[k] / y[k];
  }
#pragma unroll
  for (int k = 0; k < 8; k++) v[k] = v[k] * u[k];
}

// Quantize one token row of n values into n/32 activation blocks (quantize_row, kernels.c:90-114),
// with the value transform of the caller fused in: plain, RMSNorm (x*r)*w (kernels.c:85), or
// SwiGLU g/(1+e^-g)*u (kernels.c:395).  Work item t = (block b, lane j); the four lanes of a
// block sit in consecutive threads of one wave and exchange the block maximum by shuffles.
// QM_NORM reads x from the row staged by lane (xl, st); the others read xr (SwiGLU: gate at xr[i],
// up at xr[n + i]).
// `outh` (optional): the matrix-core operand of the multi-token GEMM, 32 bytes per (block, lane j):
// the 8 int8 values as fp16 (exact) in the order of `out`'s two words, then -sum of the 8 values
// as fp16 (exact, |sum| <= 1016), then 7 zero halves.
// One work item (block b, lane j) of quantize_row from its 8 values (elements 2j, 2j+1, 2j+8, 2j+9,
// 2j+16, 2j+17, 2j+24, 2j+25 of the block): the block maximum over the quad of lanes j = 0..3 (four
// consecutive threads of one wave, all active), the scale, the int8 values and their sum, written as
// out[b*4 + j] and, when given, the matrix-core operand outh[2 (b*4 + j)], outh[2 (b*4 + j) + 1].
// The fp16 matrix-core operands of a token's activation blocks, tiled by 16 tokens: per (tile,
// block) 132 uint4 -- [lane chain 4][quarter 4][token 16][8 bytes] (the 16 fp16 values x_0..x_7,
// -sum x, 0 x 7 of a chain in four 8-byte quarters), then the 16 tokens' block scales dx as fp32 --
// so a group of blocks of 16 tokens is contiguous memory, and 16 tokens' quarter of one chain are
// 128 contiguous bytes (one matrix-core operand read by 16 lanes).
constexpr int kXhBlock = 132;   // uint4 per (tile, block)
__host__ __device__ inline size_t xh_tile(int m, int xstride) { return (size_t)(m >> 4) * xstride * kXhBlock; }
__host__ __device__ inline size_t xh_bytes(int tokens, int xstride) {
  return (size_t)((tokens + 15) >> 4) * xstride * kXhBlock * 16;
}

// Quantize the 8 values of reference lane j of block b (quantize_row, kernels.c:90-114) into
// out[4b + j] = {A_j, B_j, -8 sum q, d}; with outh (the token's tile, xh_tile) also the fp16
// operand of token t = m % 16 and, for j = 0, its block scale.  The operand's four quarters (the
// k = 0..15 of the matrix-core product against the weight encoding of gemm_sk.h): q0..q3;
// q4..q7 / 16; -(q0 + .. + q3), -(q4 + .. + q7), 0, 0; zero.
__device__ __forceinline__ void quantize_item(const float (&v)[8], int b, int j, uint4* __restrict__ out,
                                              uint4* __restrict__ outh, int t = 0) {
  float am = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; k++) am = __builtin_fmaxf(am, __builtin_fabsf(v[k]));
  am = quad_max(am);
  const float dd = div_127(am);
  const float id = inv_scale(dd);
  int q[8];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) { q[k] = quant_one(v[k] * id); sum += q[k]; }
  out[(b << 2) + j] = make_uint4(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]),
                                 (uint32_t)(-8 * sum), __float_as_uint(dd));
  if (outh) {
    uint4* o = outh + (size_t)b * kXhBlock;
    uint2* oq = reinterpret_cast<uint2*>(o) + j * 64 + t;       // quarter q of (chain j, token t): oq[16 q]
    oq[0] = make_uint2(pack_f16x2(q[0], q[1]), pack_f16x2(q[2], q[3]));
    oq[16] = make_uint2(pack_f16x2_16th(q[4], q[5]), pack_f16x2_16th(q[6], q[7]));
    oq[32] = make_uint2(pack_f16x2(-(q[0] + q[1] + q[2] + q[3]), -(q[4] + q[5] + q[6] + q[7])), 0u);
    oq[48] = make_uint2(0u, 0u);
    if (j == 0) reinterpret_cast<float*>(o + 128)[t] = dd;
  }
}

// The norm weights of work item t (block t / 4, lane t % 4: the elements quantize_row_dev reads).
__device__ __forceinline__ void norm_weights_item(const float* __restrict__ w, int t, float (&wv)[8]) {
  const int base = ((t >> 2) << 5) + ((t & 3) << 1);
  const int e[8] = {base, base + 1, base + 8, base + 9, base + 16, base + 17, base + 24, base + 25};
#pragma unroll
  for (int k = 0; k < 8; k++) wv[k] = w[e[k]];
}

// With pre (QM_NORM, at most one work item per thread), wpre holds the item's norm weights, loaded
// by the caller before the row's sum of squares; otherwise they are read here.
template <int MODE>
__device__ __forceinline__ void quantize_row_dev(const float* __restrict__ xr, const float* xl, int st, int n,
                                                 const float* __restrict__ w, float rs,
                                                 uint4* __restrict__ out, int tid, int nthreads,
                                                 uint4* __restrict__ outh, int tok,
                                                 const float (&wpre)[8], bool pre) {
  const int nb = n >> 5;
  for (int t = tid; t < (nb << 2); t += nthreads) {
    const int b = t >> 2, j = t & 3;
    const int base = (b << 5) + (j << 1);
    const int e[8] = {base, base + 1, base + 8, base + 9, base + 16, base + 17, base + 24, base + 25};
    float v[8];
    if (MODE == QM_SWIGLU) {
      float g[8], u[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        g[k] = xr[e[k]];
        u[k] = xr[n + e[k]];
      }
      swiglu8(g, u, v);
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int i = e[k];
        if (MODE == QM_NORM) {
          v[k] = (lane_staged(xl, st, i) * rs) * (pre ? wpre[k] : w[i]);
        } else {
          v[k] = xr[i];
        }
      }
    }
    quantize_item(v, b, j, out, outh, tok);
  }
}

// e[0] + e[1] + ... + e[T - 1] in order (the serial sums of RMSNorm and softmax, kernels.c:81-84,
// 372-375) from shared memory with room for ((T + 31) & ~31) + 32 floats (the values past T are
// read, never added): 32 values are added while the next 32 load, the two register sets
// alternating (no copies between them).
__device__ __forceinline__ float ordered_sum(const float* e, int T) {
  const int T32 = T & ~31;
  float sum = 0.0f;
  float4 a[8], b[8];
  auto load = [&](float4* r, int t) {
#pragma unroll
    for (int u = 0; u < 8; u++) r[u] = *reinterpret_cast<const float4*>(e + t + 4 * u);
  };
  auto add = [&](const float4* r) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      sum = sum + r[u].x;
      sum = sum + r[u].y;
      sum = sum + r[u].z;
      sum = sum + r[u].w;
    }
  };
  load(a, 0);
  int t = 0;
  for (; t + 64 <= T32; t += 64) {        // reads reach t + 95 <= T32 + 31
    load(b, t + 32);
    __builtin_amdgcn_sched_barrier(0);
    add(a);
    __builtin_amdgcn_sched_barrier(0);
    load(a, t + 64);
    __builtin_amdgcn_sched_barrier(0);
    add(b);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (t < T32) {                          // one block of 32 left, loaded already
    add(a);
    t += 32;
  }
  for (; t < T; t++) sum = sum + e[t];
  return sum;
}

// Floats per lane row of the squares staged for RMSNorm's sum (sq_stage): n/4 values and
// ordered_sum's read room.
__host__ __device__ inline int sq_stride(int n) { return (((n >> 2) + 31) & ~31) + 32; }

// The row by reference lane (xl[(i & 3) * st + i / 4], read back by lane_staged) and the squares
// x_i * x_i the same way (sq[(i & 3) * sst + i / 4], sst = sq_stride(n)); every product rounds once, as in the
// reference's sum of v * v.
// The loads of a thread's values are all issued before the first store (eight per pass), so the
// staging waits for one memory round trip per pass, not one per value.
__device__ __forceinline__ void sq_stage(const float* __restrict__ x, int n, float* sq, int sst, float* xl,
                                         int st, int tid, int nthreads) {
  for (int i0 = tid; i0 < n; i0 += 8 * nthreads) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = i0 + k * nthreads;
      v[k] = i < n ? x[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = i0 + k * nthreads;
      if (i < n) {
        sq[(i & 3) * sst + (i >> 2)] = v[k] * v[k];
        xl[(i & 3) * st + (i >> 2)] = v[k];
      }
    }
  }
}

// 1 / sqrt(mean(x^2) + eps) with the reference's four lane sums (lane j adds the squares of i = j
// mod 4 in order) and ((l0+l1)+l2)+l3 (kernels.c:81-84), over the squares staged by sq_stage.
// Threads 0..3 run the four lanes; the result is broadcast through `red` (>= 5 floats).
__device__ __forceinline__ float rms_scale_sq(const float* sq, int n, int sst, float eps, float* red) {
  const int tid = threadIdx.x;
  if (tid < 4) red[tid] = ordered_sum(sq + tid * sst, n >> 2);
  __syncthreads();
  if (tid == 0) {
    const float ss = red[0] + red[1] + red[2] + red[3];
    red[4] = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  return red[4];
}

// ---------------------------------------------------------------- Q4_0 matvec

// Device view of one Q4 matrix in the tiled layout:
//   qs: uint4 [N/64][ng][64 rows][4 lanes j]  -- word j of blocks 4g..4g+3 of that row
//   d : uint4 [N/64][nb8][64 rows]            -- 8 fp16 scales (blocks 8c..8c+7) of that row
// A workgroup barrier for shared memory only: this wave's LDS accesses are done, then the waves
// meet.  Outstanding global loads (a poll in flight, ring slots, weights loaded ahead) are not
// waited for, as the fence of __syncthreads would.  The "memory" clobber keeps loads and stores on
// their side.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct Q4Mat {
  const uint4* qs;
  const uint4* d;
  int N, nb, ng, nb8, Np;
};

// Accumulate, for the 16 rows of one wave, lane (r, j)'s partial sums of MT tokens in the
// reference's block order: acc[m] = acc[m] + f32(p_j) * (dw * dx) for b = 0 .. nb-1
// (kernels.c:137, 217-218).  Weights are read 16 bytes per lane (4 blocks of word j), a chunk of
// 32 blocks ahead of the arithmetic.  Activation blocks come from `xs` (shared or global memory),
// token m at xs + m * xstride4 (uint4 units), block b lane j at [b*4 + j].
template <int MT>
__device__ __forceinline__ void matvec_rows16(const Q4Mat& W, int tile, int rr, int j,
                                              const uint4* __restrict__ xs, int xstride4, int M,
                                              float (&acc)[MT]) {
  constexpr int CG = 8;    // groups of 4 blocks per chunk
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
  const int nch = (W.ng + CG - 1) / CG;
  uint4 w[CG], sc[CG / 2];
#pragma unroll
  for (int g = 0; g < CG; g++) w[g] = g < W.ng ? wq[(size_t)g * 256] : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int c = 0; c < CG / 2; c++) sc[c] = c < W.nb8 ? wd[(size_t)c * 64] : make_uint4(0, 0, 0, 0);
  for (int ch = 0; ch < nch; ch++) {
    uint4 wn[CG], sn[CG / 2];
    const int g0 = (ch + 1) * CG;
    if (ch + 1 < nch) {
#pragma unroll
      for (int g = 0; g < CG; g++) wn[g] = g0 + g < W.ng ? wq[(size_t)(g0 + g) * 256] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int c = 0; c < CG / 2; c++) {
        const int c8 = g0 / 2 + c;
        sn[c] = c8 < W.nb8 ? wd[(size_t)c8 * 64] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < CG; g++) {
      const uint32_t ww[4] = {w[g].x, w[g].y, w[g].z, w[g].w};
      const uint4 sv = sc[g >> 1];
      const uint32_t sh[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int b = (ch * CG + g) * 4 + k;
        if (b < W.nb) {
          const int hb = ((g & 1) << 2) + k;            // half index within the 8 scales
          const uint32_t hbits = (hb & 1) ? (sh[hb >> 1] >> 16) : (sh[hb >> 1] & 0xffffu);
          const float dw = half_bits_to_float(hbits);
          const uint32_t lo = ww[k] & 0x0F0F0F0Fu, hi = (ww[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < M) {
              const uint4 xv = xs[(size_t)m * xstride4 + b * 4 + j];
              int p = sdot4(lo, xv.x, (int)xv.z);
              p = sdot4(hi, xv.y, p);
              acc[m] = acc[m] + (float)p * (dw * __uint_as_float(xv.w));
            }
          }
        }
      }
    }
    if (ch + 1 < nch) {
#pragma unroll
      for (int g = 0; g < CG; g++) w[g] = wn[g];
#pragma unroll
      for (int c = 0; c < CG / 2; c++) sc[c] = sn[c];
    }
  }
}

// ((acc_0 + acc_1) + acc_2) + acc_3 over the four lanes of a row (hsum, kernels.c:116-118);
// valid in lane j == 0.
// Lane k (0..3) of this lane's quad, by a DPP quad broadcast (no shared-memory round trip).  Every
// source lane is valid, so bound_ctrl changes nothing; it lets the compiler fold the broadcast into
// the instruction that uses it (v_add_f32_dpp).
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), K * 0x55, 0xF, 0xF, true));
}

// ((l0 + l1) + l2) + l3 over the four lanes of a quad (hsum, kernels.c:116-118), in every lane.
__device__ __forceinline__ float hsum4(float v) {
  const float a0 = quad_lane<0>(v), a1 = quad_lane<1>(v), a2 = quad_lane<2>(v), a3 = quad_lane<3>(v);
  return ((a0 + a1) + a2) + a3;
}

}  // namespace q4
