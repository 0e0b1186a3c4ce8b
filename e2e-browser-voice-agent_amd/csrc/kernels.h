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
constexpr int kMaxChunk = 16;       // tokens per prefill pass (the reference's MT default, engine/cpu.js:228)

// Device-resident step state: pos0 of the current pass, last sampled token.  Kernels read
// pos0 from here so one captured graph replays every decode step.
struct State {
  int pos0;
  int next;
  int pad[2];
};

// ---------------------------------------------------------------- arithmetic helpers

// e^x of kernels.c:69-78 (Cody-Waite reduction, degree-6 Taylor, exponent add), op for op.
__device__ __forceinline__ float fast_exp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  float n = __builtin_floorf(x * 1.44269504f + 0.5f);
  float r = x - n * 0.693145752f - n * 1.42860677e-6f;
  float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.166666672f + r * (0.0416666679f +
            r * (0.00833333377f + r * 0.00138888892f)))));
  return __uint_as_float(__float_as_uint(p) + ((uint32_t)(int32_t)n << 23));
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
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

// ---------------------------------------------------------------- quantization

enum QuantMode { QM_PLAIN = 0, QM_NORM = 1, QM_SWIGLU = 2 };

// Quantize one token row of n values into n/32 activation blocks (quantize_row, kernels.c:90-114),
// with the value transform of the caller fused in: plain, RMSNorm (x*r)*w (kernels.c:85), or
// SwiGLU g/(1+e^-g)*u (kernels.c:395).  Work item t = (block b, lane j); the four lanes of a
// block sit in consecutive threads of one wave and exchange the block maximum by shuffles.
template <int MODE>
__device__ __forceinline__ void quantize_row_dev(const float* __restrict__ xr, int n,
                                                 const float* __restrict__ w, float rs,
                                                 uint4* __restrict__ out, int tid, int nthreads) {
  const int nb = n >> 5;
  for (int t = tid; t < (nb << 2); t += nthreads) {
    const int b = t >> 2, j = t & 3;
    const int base = (b << 5) + (j << 1);
    const int e[8] = {base, base + 1, base + 8, base + 9, base + 16, base + 17, base + 24, base + 25};
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = e[k];
      if (MODE == QM_NORM) {
        v[k] = (xr[i] * rs) * w[i];
      } else if (MODE == QM_SWIGLU) {
        const float g = xr[i];
        v[k] = g / (1.0f + fast_exp(-g)) * xr[n + i];
      } else {
        v[k] = xr[i];
      }
    }
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) am = __builtin_fmaxf(am, __builtin_fabsf(v[k]));
    am = __builtin_fmaxf(am, __shfl_xor(am, 1, 4));
    am = __builtin_fmaxf(am, __shfl_xor(am, 2, 4));
    const float dd = am / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int q[8];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) { q[k] = quant_one(v[k] * id); sum += q[k]; }
    out[(b << 2) + j] = make_uint4(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]),
                                   (uint32_t)(-8 * sum), __float_as_uint(dd));
  }
}

// 1 / sqrt(mean(x^2) + eps) with the reference's four lane sums (lane j takes i = j mod 4, in
// order) and ((l0+l1)+l2)+l3 (kernels.c:81-84).  Threads 0..3 of the block run the lanes;
// the result is broadcast through `red` (>= 5 floats of shared memory).
__device__ __forceinline__ float rms_scale(const float* __restrict__ x, int n, float eps, float* red) {
  const int tid = threadIdx.x;
  if (tid < 4) {
    float s = 0.0f;
    for (int i = tid; i < n; i += 4) { const float v = x[i]; s = s + v * v; }
    red[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    const float ss = red[0] + red[1] + red[2] + red[3];
    red[4] = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  return red[4];
}

}  // namespace q4
