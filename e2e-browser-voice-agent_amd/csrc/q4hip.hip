// q4hip.hip -- HIP kernels and the C ABI (include/q4hip.h) of the Qwen2 Q4_0 token loop.
//
// One pass over M tokens (decode: M = 1) is the reference's forward_pass
// (h2-own-inference-engine/engine/kernels.c:306-415) as a sequence of kernels on the
// context's stream; its barriers become kernel boundaries.  The M = 1 step is captured once
// into a hipGraph that reads the position from device memory, so decode replays it with no
// host work per token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "gemm_sk.h"
#include "kernels.h"
#include "persistent.h"
#include "q4hip.h"

using namespace q4;

// ================================================================ kernels

// GGUF Q4_0 rows [rows][nb][18 B] -> tiled layout (kernels.h, Q4Mat), rows row0.. of the matrix.
// Word j of a block = its value bytes {2j, 2j+1, 8+2j, 9+2j}: the elements of reference lane j.
__global__ void k_repack_q4(const uint8_t* __restrict__ raw, int64_t rows, int nb, int ng, int nb8, int row0,
                            uint32_t* __restrict__ qs, uint16_t* __restrict__ dsc) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * nb) return;
  const int64_t r = idx / nb;
  const int b = (int)(idx - r * nb);
  const int64_t R = row0 + r;
  const int64_t tile = R >> 6;
  const int rr = (int)(R & 63);
  const uint8_t* s = raw + idx * 18;
  dsc[((tile * nb8 + (b >> 3)) * 64 + rr) * 8 + (b & 7)] = (uint16_t)(s[0] | (s[1] << 8));
  const uint8_t* q = s + 2;
  uint32_t* o = qs + (((tile * ng + (b >> 2)) * 64 + rr) * 4) * 4 + (b & 3);
#pragma unroll
  for (int j = 0; j < 4; j++)
    o[j * 4] = (uint32_t)q[2 * j] | ((uint32_t)q[2 * j + 1] << 8) | ((uint32_t)q[8 + 2 * j] << 16) |
               ((uint32_t)q[9 + 2 * j] << 24);
}

// GGUF Q8_0 rows [rows][nb][34 B] -> the Q8 tiled layout: qs uint4 [N/64][ceil(nb/2)][64 rows][4 lanes j],
// the uint4 of lane j and group g = {A_j, B_j} of block 2g then of block 2g+1, where A_j = int8 values
// {2j, 2j+1, 8+2j, 9+2j} and B_j = {16+2j, 17+2j, 24+2j, 25+2j} (the elements of reference lane j,
// kernels.c:157-170); d: the fp16 scales as for Q4_0.
__global__ void k_repack_q8(const uint8_t* __restrict__ raw, int64_t rows, int nb, int ng, int nb8, int row0,
                            uint32_t* __restrict__ qs, uint16_t* __restrict__ dsc) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * nb) return;
  const int64_t r = idx / nb;
  const int b = (int)(idx - r * nb);
  const int64_t R = row0 + r;
  const int64_t tile = R >> 6;
  const int rr = (int)(R & 63);
  const uint8_t* s = raw + idx * 34;
  dsc[((tile * nb8 + (b >> 3)) * 64 + rr) * 8 + (b & 7)] = (uint16_t)(s[0] | (s[1] << 8));
  const uint8_t* q = s + 2;
  uint32_t* o = qs + (((tile * ng + (b >> 1)) * 64 + rr) * 4) * 4 + (b & 1) * 2;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    o[j * 4] = (uint32_t)q[2 * j] | ((uint32_t)q[2 * j + 1] << 8) | ((uint32_t)q[8 + 2 * j] << 16) |
               ((uint32_t)q[9 + 2 * j] << 24);
    o[j * 4 + 1] = (uint32_t)q[16 + 2 * j] | ((uint32_t)q[17 + 2 * j] << 8) | ((uint32_t)q[24 + 2 * j] << 16) |
                   ((uint32_t)q[25 + 2 * j] << 24);
  }
}

// Embedding rows (kernels.c:312-322): x[m][32b+j] = ((q&15)-8)*d, x[m][32b+16+j] = ((q>>4)-8)*d.
// The table stays in GGUF layout [vocab][D/32][18 B]; one token reads 18*D/32 bytes.
__global__ void k_embed(const uint8_t* __restrict__ emb, int D, const int* __restrict__ tokens,
                        const State* __restrict__ st, float* __restrict__ x) {
  const int m = blockIdx.x;
  const int t = tokens[st->pos0 + m];
  const uint8_t* row = emb + (size_t)t * (D / 32) * 18;
  float* xr = x + (size_t)m * D;
  for (int idx = threadIdx.x; idx < D / 2; idx += blockDim.x) {
    const int blk = idx >> 4, j = idx & 15;
    const uint8_t* bp = row + blk * 18;
    const float d = half_bits_to_float((uint32_t)bp[0] | ((uint32_t)bp[1] << 8));
    const int q = bp[2 + j];
    xr[32 * blk + j] = (float)((q & 15) - 8) * d;
    xr[32 * blk + 16 + j] = (float)((q >> 4) - 8) * d;
  }
}

// Quantize rows m_first .. m_first+gridDim.x-1 of `in` into xq rows 0.. (kernels.c:328-331,
// 379, 385-388, 393-397, 405-407).  QM_NORM stages the row's squares for the serial sums and the
// row itself by lane in shared memory (quant_lds: 4 sq_stride(n) + 4 (n/4 + 1) floats).
// With xh and at least 128 rows, workgroup w takes row (w % 8) * ceil(rows / 8) + w / 8 (none past
// rows): workgroup w runs on XCD w % 8, so the 16 rows of an operand tile are quantized on one or
// two XCDs and the tile's lines, 8 bytes of each from every row, are completed in their L2 instead
// of being written back in pieces from all eight (a 1024-token prompt pass: 8.98 -> 8.87 ms; with
// 32 rows the spread over four XCDs instead of eight measured slower, so fewer rows keep row w).
template <int MODE>
__global__ __launch_bounds__(256) void k_quant(const float* __restrict__ in, int ld_in, int n,
                                               const float* __restrict__ w, float eps,
                                               uint4* __restrict__ xq, int xstride, int m_first,
                                               uint4* __restrict__ xh, int rows) {
  extern __shared__ float xl[];
  __shared__ float red[8];
  int row = blockIdx.x;
  if (xh && rows >= 128) {
    row = (int)(blockIdx.x & 7) * ((rows + 7) >> 3) + (int)(blockIdx.x >> 3);
    if (row >= rows) return;
  }
  const float* xr = in + (size_t)(m_first + row) * ld_in;
  const int st = (n >> 2) + 1;
  float rs = 0.0f;
  const int sst = sq_stride(n);
  float* const xs = xl + 4 * sst;         // the row by lane, after the squares
  // with one work item per thread, its norm weights load with the row, ahead of the sum
  const bool one = MODE == QM_NORM && (n >> 3) <= (int)blockDim.x;
  float wv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (one && (int)threadIdx.x < (n >> 3)) norm_weights_item(w, threadIdx.x, wv);
  if (MODE == QM_NORM) {
    sq_stage(xr, n, xl, sst, xs, st, threadIdx.x, blockDim.x);
    __syncthreads();
    rs = rms_scale_sq(xl, n, sst, eps, red);
  }
  quantize_row_dev<MODE>(xr, xs, st, n, w, rs, xq + (size_t)row * xstride * 4, threadIdx.x, blockDim.x,
                         xh ? xh + xh_tile(row, xstride) : nullptr, row & 15, wv, one);
}

enum { OP_STORE = 0, OP_BIAS = 1, OP_ADD = 2 };   // put() of kernels.c:190-194

// y[m][n] (op)= W[n] . x[m] for M tokens (matmul_q4, kernels.c:200-273).  One wave = 16 rows;
// lane (r, j) owns accumulator j of row r (matvec_rows16), then hsum4 and the epilogue of
// put() (kernels.c:190-194).  For one token the activation blocks are staged in shared memory
// (nb*64 bytes of dynamic shared memory); for a prefill chunk they are read from global memory.
template <int MT, int OP>
__global__ __launch_bounds__(64) void k_matvec(Q4Mat W, const uint4* __restrict__ xq, int xstride, int M,
                                               float* __restrict__ y, int ldy, const float* __restrict__ bias) {
  extern __shared__ uint4 xs[];
  const int lane = threadIdx.x, r = lane >> 2, j = lane & 3;
  const int wv = blockIdx.x, tile = wv >> 2, rr = ((wv & 3) << 4) + r;
  const int row = (tile << 6) + rr;
  const uint4* src = xq;
  if (MT == 1) {
    for (int i = lane; i < W.nb * 4; i += 64) xs[i] = xq[i];
    __syncthreads();
    src = xs;
  }
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;
  matvec_rows16<MT>(W, tile, rr, j, src, xstride * 4, M, acc);
#pragma unroll
  for (int m = 0; m < MT; m++) {
    if (m < M) {
      const float v = hsum4(acc[m]);
      if (j == 0 && row < W.N) {
        float* o = y + (size_t)m * ldy + row;
        if (OP == OP_ADD) *o = *o + v;
        else if (OP == OP_BIAS) *o = v + bias[row];
        else *o = v;
      }
    }
  }
}

// y = W x for one token and rows of NB blocks (the 896- and 1536-wide projections and output
// heads): a grid-stride stream over 16-row groups.  Wave w of workgroup b takes groups 4b + w,
// 4b + w + 4G, ... (G workgroups).  Each group's weights are loaded while the previous group's sums
// run, and a wave's first loads are issued before the activation blocks are staged in shared memory
// (once per workgroup), so the two latencies overlap.  The sums are those of k_matvec<1>: lane
// (r, j) adds its terms acc = acc + f32(p) * (dw * dx) in block order (kernels.c:200-229), then
// hsum4 across the row's four lanes.
template <int NB>
struct StreamRegs {
  static constexpr int NG = (NB + 3) / 4, NS = (NB + 7) / 8;
  uint4 w[NG], s[NS];
};

template <int NB>
__device__ __forceinline__ void stream_issue(const Q4Mat& W, int g16, int r, int j, StreamRegs<NB>& R) {
  const int tile = g16 >> 2, rr = ((g16 & 3) << 4) + r;
  const uint4* wq = W.qs + ((size_t)tile * StreamRegs<NB>::NG * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * StreamRegs<NB>::NS * 64 + rr;
#pragma unroll
  for (int g = 0; g < StreamRegs<NB>::NG; g++) R.w[g] = wq[(size_t)g * 256];
#pragma unroll
  for (int c = 0; c < StreamRegs<NB>::NS; c++) R.s[c] = wd[(size_t)c * 64];
}

template <int NB, int OP>
__device__ __forceinline__ void stream_rows(const Q4Mat& W, int g16, int r, int j, const uint4* xs,
                                            const StreamRegs<NB>& R, float* __restrict__ y,
                                            const float* __restrict__ bias) {
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < StreamRegs<NB>::NG; g++) {
    const uint32_t ww[4] = {R.w[g].x, R.w[g].y, R.w[g].z, R.w[g].w};
    const uint4 sv = R.s[g >> 1];
    const uint32_t sh[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int b = g * 4 + k;
      if (b < NB) {
        const int hb = ((g & 1) << 2) + k;
        const uint32_t hbits = (hb & 1) ? (sh[hb >> 1] >> 16) : (sh[hb >> 1] & 0xffffu);
        const float dw = half_bits_to_float(hbits);
        const uint32_t lo = ww[k] & 0x0F0F0F0Fu, hi = (ww[k] >> 4) & 0x0F0F0F0Fu;
        const uint4 xv = xs[b * 4 + j];
        int p = sdot4(lo, xv.x, (int)xv.z);
        p = sdot4(hi, xv.y, p);
        acc = acc + (float)p * (dw * __uint_as_float(xv.w));
      }
    }
  }
  const float v = hsum4(acc);
  const int row = ((g16 >> 2) << 6) + ((g16 & 3) << 4) + r;
  if (j == 0 && row < W.N) {
    float* o = y + row;
    if (OP == OP_ADD) *o = *o + v;
    else if (OP == OP_BIAS) *o = v + bias[row];
    else *o = v;
  }
}

template <int NB, int OP>
__global__ __launch_bounds__(256) void k_matvec_stream(Q4Mat W, const uint4* __restrict__ xq, float* __restrict__ y,
                                                      const float* __restrict__ bias) {
  __shared__ uint4 xs[NB * 4];
  const int tid = threadIdx.x, lane = tid & 63, r = lane >> 2, j = lane & 3;
  const int groups = W.Np >> 4, step = (int)gridDim.x * 4;
  int g16 = (int)blockIdx.x * 4 + (tid >> 6);
  StreamRegs<NB> ra, rb;
  if (g16 < groups) stream_issue<NB>(W, g16, r, j, ra);
  for (int i = tid; i < NB * 4; i += 256) xs[i] = xq[i];
  lds_barrier();
  // two register sets, alternating, so that neither is indexed at run time
  while (g16 < groups) {
    const int g1 = g16 + step;
    if (g1 < groups) stream_issue<NB>(W, g1, r, j, rb);
    stream_rows<NB, OP>(W, g16, r, j, xs, ra, y, bias);
    if (g1 >= groups) break;
    const int g2 = g1 + step;
    if (g2 < groups) stream_issue<NB>(W, g2, r, j, ra);
    stream_rows<NB, OP>(W, g1, r, j, xs, rb, y, bias);
    g16 = g2;
  }
}

// Workgroups of a k_matvec_stream<NB> launch over `groups` 16-row groups: every wave takes the same
// number of groups (the last waves one fewer), at most stream_waves(NB) waves in all -- as many as
// are resident at once (two per SIMD for 28-block rows, one for the wider register sets of 48).
constexpr int stream_waves(int nb) { return nb <= 32 ? 2048 : 1024; }
inline unsigned stream_grid(int groups, int max_waves) {
  const int per = (groups + max_waves - 1) / max_waves;
  const int waves = (groups + per - 1) / per;
  return (unsigned)((waves + 3) / 4);
}

// One token, matrices with many blocks per row (down: 896 x 4864): the same sums as k_matvec<1>,
// with the blocks of a 16-row group spread over four waves.  Wave w forms the terms
// f32(p_j) * (dw * dx) of block groups w, w + 4, ... (every term is independent of the others) into
// shared memory; then wave 0 adds each lane's terms in block order, acc = acc + t, as
// matvec_rows16 does (kernels.c:200-229), and the four lanes of a row combine in hsum order.
// Dynamic shared memory: nb * 64 bytes of activation blocks, then nb * 256 bytes of terms.
constexpr int kSplitWaves = 8, kSplitThreads = 64 * kSplitWaves;
template <int OP>
__global__ __launch_bounds__(kSplitThreads) void k_matvec_split(Q4Mat W, const uint4* __restrict__ xq, float* __restrict__ y,
                                                     const float* __restrict__ bias) {
  extern __shared__ uint4 xs[];
  float* tm = reinterpret_cast<float*>(xs + W.nb * 4);     // [block][lane (r, j)]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int wv = blockIdx.x, tile = wv >> 2, rr = ((wv & 3) << 4) + r;
  const int row = (tile << 6) + rr;
  for (int i = tid; i < W.nb * 4; i += kSplitThreads) xs[i] = xq[i];
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
  constexpr int CG = 8;                                     // this wave's groups in flight
  const int mine = (W.ng - wave + kSplitWaves - 1) / kSplitWaves;   // groups wave, wave + waves, ...
  uint4 w[CG], sc[CG];
#pragma unroll
  for (int c = 0; c < CG; c++) {
    const int g = wave + kSplitWaves * c;
    w[c] = c < mine ? wq[(size_t)g * 256] : make_uint4(0, 0, 0, 0);
    sc[c] = c < mine ? wd[(size_t)(g >> 1) * 64] : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  for (int c0 = 0; c0 < mine; c0 += CG) {
    uint4 wn[CG], sn[CG];
    const bool more = c0 + CG < mine;
    if (more) {
#pragma unroll
      for (int c = 0; c < CG; c++) {
        const int cc = c0 + CG + c, g = wave + kSplitWaves * cc;
        wn[c] = cc < mine ? wq[(size_t)g * 256] : make_uint4(0, 0, 0, 0);
        sn[c] = cc < mine ? wd[(size_t)(g >> 1) * 64] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int c = 0; c < CG; c++) {
      if (c0 + c < mine) {
        const int g = wave + kSplitWaves * (c0 + c);
        const uint32_t ww[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
        const uint32_t sh[4] = {sc[c].x, sc[c].y, sc[c].z, sc[c].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int b = 4 * g + k;
          if (b < W.nb) {
            const int hb = ((g & 1) << 2) + k;                  // half index within the 8 scales
            const uint32_t hbits = (hb & 1) ? (sh[hb >> 1] >> 16) : (sh[hb >> 1] & 0xffffu);
            const float dw = half_bits_to_float(hbits);
            const uint32_t lo = ww[k] & 0x0F0F0F0Fu, hi = (ww[k] >> 4) & 0x0F0F0F0Fu;
            const uint4 xv = xs[b * 4 + j];
            int p = sdot4(lo, xv.x, (int)xv.z);
            p = sdot4(hi, xv.y, p);
            tm[b * 64 + lane] = (float)p * (dw * __uint_as_float(xv.w));
          }
        }
      }
    }
    if (more) {
#pragma unroll
      for (int c = 0; c < CG; c++) { w[c] = wn[c]; sc[c] = sn[c]; }
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // this lane's chain in block order; the next 8 terms are read while the current 8 are added
  float acc = 0.0f;
  int b = 0;
  if (W.nb >= 16) {
    float a[8];
#pragma unroll
    for (int u = 0; u < 8; u++) a[u] = tm[u * 64 + lane];
    for (; b + 16 <= W.nb; b += 8) {
      float n8[8];
#pragma unroll
      for (int u = 0; u < 8; u++) n8[u] = tm[(b + 8 + u) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; u++) acc = acc + a[u];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; u++) a[u] = n8[u];
    }
#pragma unroll
    for (int u = 0; u < 8; u++) acc = acc + a[u];
    b += 8;
  }
  for (; b < W.nb; b++) acc = acc + tm[b * 64 + lane];
  const float v = hsum4(acc);
  if (j == 0 && row < W.N) {
    float* o = y + row;
    if (OP == OP_ADD) *o = *o + v;
    else if (OP == OP_BIAS) *o = v + bias[row];
    else *o = v;
  }
}

// Blocks per row from which one-token projections use k_matvec_split.
constexpr int kSplitMinBlocks = 64;
// The widest row it takes: activation blocks and terms in shared memory.
constexpr int kSplitMaxBlocks = 480;
inline size_t split_lds(int nb) { return (size_t)nb * 320; }

// The widest row of a one-token projection on k_matvec<1> (rows wider than k_matvec_split takes):
// 2048 blocks (K = 65536, the no-allocation matvec's limit), 64 bytes of activation block each in
// shared memory.
constexpr int kMatvec1MaxBlocks = 2048;

// Raise the shared-memory limits of k_matvec_split and k_matvec<1> once per device, with that device
// current (before any graph capture: the handle and matvec constructors call it).
void matvec_split_setup(int device) {
  static std::mutex mu;
  static uint64_t done = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (device < 0 || device >= 64 || (done >> device) & 1) return;
  const int lds = (int)split_lds(kSplitMaxBlocks), lds1 = kMatvec1MaxBlocks * 64;
  (void)hipFuncSetAttribute((const void*)k_matvec_split<0>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)hipFuncSetAttribute((const void*)k_matvec_split<1>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)hipFuncSetAttribute((const void*)k_matvec_split<2>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)hipFuncSetAttribute((const void*)k_matvec<1, 0>, hipFuncAttributeMaxDynamicSharedMemorySize, lds1);
  (void)hipFuncSetAttribute((const void*)k_matvec<1, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, lds1);
  (void)hipFuncSetAttribute((const void*)k_matvec<1, 2>, hipFuncAttributeMaxDynamicSharedMemorySize, lds1);
  (void)hipGetLastError();
  done |= (uint64_t)1 << device;
}

// y[m][n] (op)= W[n] . x[m] for a pass of M tokens (matmul_q4, kernels.c:200-273): the prefill
// projections.  A workgroup computes 16 rows x 32 tokens: lane (r, j) of wave w owns reference lane
// j of row r for tokens 8w..8w+7 of the tile, so every output is acc_j = acc_j + f32(p_j) * (dw * dx)
// over the blocks in order and then ((acc_0 + acc_1) + acc_2) + acc_3 across the four lanes, exactly
// as for one token.  A block's nibbles are split once and used for 8 tokens; the activation blocks
// of the tile's tokens are staged in shared memory one group of 4 blocks at a time
// (double-buffered).  16-row tiles keep narrow matrices (o, down: 896 rows) on many CUs.
constexpr int kGemmRows = 16, kGemmTokens = 32;

template <int OP>
__global__ __launch_bounds__(256) void k_gemm_q4(Q4Mat W, const uint4* __restrict__ xq, int xstride, int M,
                                                float* __restrict__ y, int ldy, const float* __restrict__ bias) {
  __shared__ uint4 xs[2][kGemmTokens][16];   // [buffer][token][block of the group * 4 + j]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int m0 = blockIdx.y * kGemmTokens, row = blockIdx.x * kGemmRows + r;
  const int tile = row >> 6, rr = row & 63;
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
  const bool active = m0 + wave * 8 < M;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; t++) acc[t] = 0.0f;
  auto stage = [&](int g, int buf) {
    for (int i = tid; i < kGemmTokens * 16; i += 256) {
      const int t = i >> 4, k = i & 15, m = m0 + t, b = g * 4 + (k >> 2);
      xs[buf][t][k] = (m < M && b < W.nb) ? xq[(size_t)m * xstride * 4 + b * 4 + (k & 3)] : make_uint4(0, 0, 0, 0);
    }
  };
  stage(0, 0);
  uint4 w = wq[0], sc = wd[0];
  __syncthreads();
  for (int g = 0; g < W.ng; g++) {
    const int buf = g & 1;
    uint4 wn = w, scn = sc;
    if (g + 1 < W.ng) {
      stage(g + 1, buf ^ 1);
      wn = wq[(size_t)(g + 1) * 256];
      if (((g + 1) & 1) == 0) scn = wd[(size_t)((g + 1) >> 1) * 64];
    }
    if (active) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int b = g * 4 + k;
        if (b < W.nb) {
          const int hb = ((g & 1) << 2) + k;
          const uint32_t sw = (hb >> 1) == 0 ? sc.x : (hb >> 1) == 1 ? sc.y : (hb >> 1) == 2 ? sc.z : sc.w;
          const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
          const uint32_t wv = k == 0 ? w.x : k == 1 ? w.y : k == 2 ? w.z : w.w;
          const uint32_t lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
          int p[8];
#pragma unroll
          for (int t = 0; t < 8; t++) {
            const uint4 xv = xs[buf][wave * 8 + t][k * 4 + j];
            p[t] = sdot4(lo, xv.x, (int)xv.z);
            p[t] = sdot4(hi, xv.y, p[t]);
          }
#pragma unroll
          for (int t = 0; t < 8; t++) {
            const float dx = __uint_as_float(xs[buf][wave * 8 + t][k * 4 + j].w);
            acc[t] = acc[t] + (float)p[t] * (dw * dx);
          }
        }
      }
    }
    __syncthreads();
    w = wn;
    sc = scn;
  }
#pragma unroll
  for (int t = 0; t < 8; t++) {
    const float v = hsum4(acc[t]);
    const int m = m0 + wave * 8 + t;
    if (j == 0 && m < M && row < W.N) {
      float* o = y + (size_t)m * ldy + row;
      if (OP == OP_ADD) *o = *o + v;
      else if (OP == OP_BIAS) *o = v + bias[row];
      else *o = v;
    }
  }
}

// logits[n] = dot_q8_q8(W[n], x) for one token (kernels.c:157-170, 412): the Q8_0 output head.  One wave
// = 16 rows, lane (r, j) owns accumulator j of row r; per block p = A_j . xA_j + B_j . xB_j, then
// acc = acc + f32(p) * (dw * dx); activation blocks staged in shared memory (nb * 64 bytes).
__global__ __launch_bounds__(64) void k_matvec_q8(Q4Mat W, const uint4* __restrict__ xq, float* __restrict__ y) {
  extern __shared__ uint4 xs[];
  const int lane = threadIdx.x, r = lane >> 2, j = lane & 3;
  const int wv = blockIdx.x, tile = wv >> 2, rr = ((wv & 3) << 4) + r;
  const int row = (tile << 6) + rr;
  for (int i = lane; i < W.nb * 4; i += 64) xs[i] = xq[i];
  __syncthreads();
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
  float acc = 0.0f;
  uint4 sc = make_uint4(0, 0, 0, 0);
  uint4 wn = wq[0];
  for (int g = 0; g < W.ng; g++) {
    const uint4 w = wn;
    if (g + 1 < W.ng) wn = wq[(size_t)(g + 1) * 256];
    if ((g & 3) == 0) sc = wd[(size_t)(g >> 2) * 64];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int b = 2 * g + h;
      if (b < W.nb) {
        const int hb = b & 7;
        const uint32_t sw = (hb >> 1) == 0 ? sc.x : (hb >> 1) == 1 ? sc.y : (hb >> 1) == 2 ? sc.z : sc.w;
        const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
        const uint4 xv = xs[b * 4 + j];
        int p = sdot4(h ? w.z : w.x, xv.x, 0);
        p = sdot4(h ? w.w : w.y, xv.y, p);
        acc = acc + (float)p * (dw * __uint_as_float(xv.w));
      }
    }
  }
  const float v = hsum4(acc);
  if (j == 0 && row < W.N) y[row] = v;
}

// RoPE on the q and k heads, then K (roped) and V appended to the cache at pos (kernels.c:337-352;
// fp32, or rounded to fp16).  Grid (heads + kv_heads, M), HD/2 threads: thread i owns pair (i, i+HD/2).
template <class KT>
__global__ void k_rope_kv(float* __restrict__ qkv, int QKV, int D, int H, int KVH, int HD,
                          const float* __restrict__ rope, KT* __restrict__ kc, KT* __restrict__ vc,
                          int ctx, int layer, const State* __restrict__ st) {
  const int h = blockIdx.x, m = blockIdx.y, i = threadIdx.x, half = HD / 2;
  const int pos = st->pos0 + m;
  float* v = qkv + (size_t)m * QKV + h * HD;
  const float* cs = rope + (size_t)pos * HD;
  const float c = cs[2 * i], s = cs[2 * i + 1], x0 = v[i], x1 = v[i + half];
  const float y0 = x0 * c - x1 * s, y1 = x1 * c + x0 * s;
  v[i] = y0;
  v[i + half] = y1;
  if (h >= H) {
    const int kh = h - H;
    const size_t off = (((size_t)layer * KVH + kh) * ctx + pos) * HD;
    const float* vs = qkv + (size_t)m * QKV + D + KVH * HD + kh * HD;
    kc[off + i] = (KT)y0;
    kc[off + i + half] = (KT)y1;
    vc[off + i] = (KT)vs[i];
    vc[off + i + half] = (KT)vs[i + half];
  }
}

// Attention for a block of 32 query tokens of one head in a multi-token pass (kernels.c:355-377), in
// the reference's per-(token, head) order: scores as four lane sums over i = j mod 4 times the scale,
// the maximum, e_t = fast_exp(s_t - max) summed in t order, then out_i = sum over t in order of
// (e_t / sum) * v_t[i].  Thread (token mi = tid/8, sub = tid%8) scores positions t = sub (mod 8) and
// accumulates output elements [sub*HD/8, (sub+1)*HD/8) of its token.  K and V come in chunks of 32
// positions staged in shared memory and used by all 32 tokens; scores and e_t go to a global scratch
// row per (token, head) of ctx floats.  Grid (H, ceil(M/32)).
constexpr int kAttnTokens = 32, kAttnChunk = 32;

template <int HD, class KT>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ qkv, int QKV, int H, int KVH,
                                                      const KT* __restrict__ kc, const KT* __restrict__ vc,
                                                      int ctx, int layer, float* __restrict__ att, int D,
                                                      const State* __restrict__ st, int M, float* __restrict__ scr) {
  constexpr int RS = HD + 4, DPT = HD / 8;
  __shared__ __attribute__((aligned(16))) float qs[kAttnTokens][RS];
  __shared__ __attribute__((aligned(16))) float cs[kAttnChunk][RS];     // a K chunk, then V chunks
  __shared__ float ps[kAttnTokens][kAttnChunk + 1];
  __shared__ float rsum[kAttnTokens];
  const int h = blockIdx.x, mb = blockIdx.y * kAttnTokens, tid = threadIdx.x, mi = tid >> 3, sub = tid & 7;
  const int pos0 = st->pos0, kh = h / (H / KVH);
  const int m = mb + mi;
  const int Tm = m < M ? pos0 + m + 1 : 0;
  const int Tb = pos0 + (mb + kAttnTokens < M ? mb + kAttnTokens : M);
  const KT* kb = kc + ((size_t)layer * KVH + kh) * ctx * HD;
  const KT* vb = vc + ((size_t)layer * KVH + kh) * ctx * HD;
  float* srow = scr + ((size_t)(m < M ? m : 0) * H + h) * ctx;
  for (int i = tid; i < kAttnTokens * HD; i += 256) {
    const int r = i / HD, c = i - r * HD;
    qs[r][c] = mb + r < M ? qkv[(size_t)(mb + r) * QKV + h * HD + c] : 0.0f;
  }
  const float scale = 1.0f / __builtin_sqrtf((float)HD);
  float lmax = -1e30f;
  for (int t0 = 0; t0 < Tb; t0 += kAttnChunk) {
    __syncthreads();
    for (int i = tid; i < kAttnChunk * HD / 4; i += 256) {
      const int r = i / (HD / 4), c4 = i - r * (HD / 4), t = t0 + r;
      const float4 v = t < Tb ? kv_ld4<KT>(kb + (size_t)t * HD + 4 * c4) : make_float4(0, 0, 0, 0);
      *reinterpret_cast<float4*>(&cs[r][4 * c4]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kAttnChunk / 8; k++) {
      const int r = sub + 8 * k, t = t0 + r;
      if (t < Tm) {
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < HD / 4; i4++) {
          const float4 q4 = *reinterpret_cast<const float4*>(&qs[mi][4 * i4]);
          const float4 k4 = *reinterpret_cast<const float4*>(&cs[r][4 * i4]);
          s0 = s0 + q4.x * k4.x;
          s1 = s1 + q4.y * k4.y;
          s2 = s2 + q4.z * k4.z;
          s3 = s3 + q4.w * k4.w;
        }
        const float v = (s0 + s1 + s2 + s3) * scale;
        srow[t] = v;
        lmax = __builtin_fmaxf(lmax, v);
      }
    }
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) lmax = __builtin_fmaxf(lmax, __shfl_xor(lmax, o));
  __syncthreads();
  for (int t = sub; t < Tm; t += 8) srow[t] = fast_exp(srow[t] - lmax);
  __syncthreads();
  if (sub == 0 && Tm > 0) {
    float sum = 0.0f;
    int t = 0;
    for (; t + 8 <= Tm; t += 8) {
      float e[8];
#pragma unroll
      for (int u = 0; u < 8; u++) e[u] = srow[t + u];
#pragma unroll
      for (int u = 0; u < 8; u++) sum = sum + e[u];
    }
    for (; t < Tm; t++) sum = sum + srow[t];
    rsum[mi] = sum;
  }
  float acc[DPT];
#pragma unroll
  for (int d = 0; d < DPT; d++) acc[d] = 0.0f;
  for (int t0 = 0; t0 < Tb; t0 += kAttnChunk) {
    __syncthreads();
    for (int i = tid; i < kAttnChunk * HD / 4; i += 256) {
      const int r = i / (HD / 4), c4 = i - r * (HD / 4), t = t0 + r;
      const float4 v = t < Tb ? kv_ld4<KT>(vb + (size_t)t * HD + 4 * c4) : make_float4(0, 0, 0, 0);
      *reinterpret_cast<float4*>(&cs[r][4 * c4]) = v;
    }
    for (int i = tid; i < kAttnTokens * kAttnChunk; i += 256) {
      const int r = i / kAttnChunk, c = i - r * kAttnChunk, mm = mb + r, t = t0 + c;
      ps[r][c] = (mm < M && t < pos0 + mm + 1) ? scr[((size_t)mm * H + h) * ctx + t] / rsum[r] : 0.0f;
    }
    __syncthreads();
    const int n = Tm - t0 < kAttnChunk ? Tm - t0 : kAttnChunk;
    for (int c = 0; c < n; c++) {
      const float p = ps[mi][c];
#pragma unroll
      for (int d4 = 0; d4 < DPT / 4; d4++) {
        const float4 v4 = *reinterpret_cast<const float4*>(&cs[c][sub * DPT + 4 * d4]);
        acc[4 * d4 + 0] = acc[4 * d4 + 0] + p * v4.x;
        acc[4 * d4 + 1] = acc[4 * d4 + 1] + p * v4.y;
        acc[4 * d4 + 2] = acc[4 * d4 + 2] + p * v4.z;
        acc[4 * d4 + 3] = acc[4 * d4 + 3] + p * v4.w;
      }
    }
  }
  if (m < M) {
#pragma unroll
    for (int d = 0; d < DPT; d++) att[(size_t)m * D + h * HD + sub * DPT + d] = acc[d];
  }
}

// Attention for one (head, token) over T = pos0+m+1 cached positions (kernels.c:355-377), in the
// reference's order: scores as four lane sums over i = j mod 4, max, fast_exp and a running sum in
// t order, then out_i = sum over t in order of (e_t/sum)*v_t[i].  Grid (H, M), one wave; thread t
// scores position t (its K row loaded whole), thread i accumulates output element(s) i over t with
// V loaded 32 positions ahead.  Shared: HD + T floats.
template <int HD, class KT>
__global__ __launch_bounds__(64) void k_attn(const float* __restrict__ qkv, int QKV, int D, int H, int KVH,
                                             const KT* __restrict__ kc, const KT* __restrict__ vc,
                                             int ctx, int layer, float* __restrict__ att,
                                             const State* __restrict__ st) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  __shared__ float red[2];
  const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  const int T = st->pos0 + m + 1, kh = h / (H / KVH);
  const float* q = qkv + (size_t)m * QKV + h * HD;
  const KT* kb = kc + ((size_t)layer * KVH + kh) * ctx * HD;
  const KT* vb = vc + ((size_t)layer * KVH + kh) * ctx * HD;
  float* sq = sm;
  float* sc = sm + HD;
  for (int i = tid; i < HD; i += 64) sq[i] = q[i];
  __syncthreads();
  const float scale = 1.0f / __builtin_sqrtf((float)HD);
  float lmax = -1e30f;
  const float4* qr = reinterpret_cast<const float4*>(sq);
  for (int t = tid; t < T; t += 64) {
    const KT* kr = kb + (size_t)t * HD;
    float4 kv[HD / 4];
#pragma unroll
    for (int i4 = 0; i4 < HD / 4; i4++) kv[i4] = kv_ld4<KT>(kr + 4 * i4);
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int i4 = 0; i4 < HD / 4; i4++) {
      const float4 qv = qr[i4];
      s0 = s0 + qv.x * kv[i4].x;
      s1 = s1 + qv.y * kv[i4].y;
      s2 = s2 + qv.z * kv[i4].z;
      s3 = s3 + qv.w * kv[i4].w;
    }
    const float v = (s0 + s1 + s2 + s3) * scale;
    sc[t] = v;
    lmax = __builtin_fmaxf(lmax, v);
  }
  lmax = max64(lmax);
  __syncthreads();
  for (int t = tid; t < T; t += 64) sc[t] = fast_exp(sc[t] - lmax);
  __syncthreads();
  if (tid == 0) {
    float sum = 0.0f;
    int t = 0;
    for (; t + 8 <= T; t += 8) {
      float e[8];
#pragma unroll
      for (int u = 0; u < 8; u++) e[u] = sc[t + u];
#pragma unroll
      for (int u = 0; u < 8; u++) sum = sum + e[u];
    }
    for (; t < T; t++) sum = sum + sc[t];
    red[0] = sum;
  }
  __syncthreads();
  const float sum = red[0];
  for (int t = tid; t < T; t += 64) sc[t] = sc[t] / sum;
  __syncthreads();
  constexpr int E = HD / 64;     // output elements per thread
  constexpr int TB = 32;         // positions per V batch
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; e++) acc[e] = 0.0f;
  float vcur[TB][E];
#pragma unroll
  for (int u = 0; u < TB; u++)
#pragma unroll
    for (int e = 0; e < E; e++) vcur[u][e] = u < T ? (float)vb[(size_t)u * HD + tid + 64 * e] : 0.0f;
  for (int t0 = 0; t0 < T; t0 += TB) {
    float vnext[TB][E];
    const int t1 = t0 + TB;
    if (t1 < T) {
#pragma unroll
      for (int u = 0; u < TB; u++)
#pragma unroll
        for (int e = 0; e < E; e++) vnext[u][e] = t1 + u < T ? (float)vb[(size_t)(t1 + u) * HD + tid + 64 * e] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < TB; u++) {
      if (t0 + u < T) {
        const float p = sc[t0 + u];
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] = acc[e] + p * vcur[u][e];
      }
    }
    if (t1 < T) {
#pragma unroll
      for (int u = 0; u < TB; u++)
#pragma unroll
        for (int e = 0; e < E; e++) vcur[u][e] = vnext[u][e];
    }
  }
#pragma unroll
  for (int e = 0; e < E; e++) att[(size_t)m * D + h * HD + tid + 64 * e] = acc[e];
}

// Greedy sample, stage 1: (max, first index) per 4096-entry slice (cpu-worker.js:156-157).
__device__ __forceinline__ void amax_merge(float& bv, int& bi, float v, int i) {
  if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
}

// This thread's (max, first index) over entries lo + tid + 256 k < hi of a 4096-entry slice: the
// 16 values load together, then merge in index order.
__device__ __forceinline__ void slice_amax(const float* __restrict__ row, int lo, int hi, int tid, float& bv, int& bi) {
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const int i = lo + tid + 256 * k;
    v[k] = i < hi ? row[i] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const int i = lo + tid + 256 * k;
    if (i < hi) amax_merge(bv, bi, v[k], i);
  }
}

__global__ __launch_bounds__(256) void k_argmax1(const float* __restrict__ lg, int V, float* __restrict__ pv,
                                                 int* __restrict__ pi) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int tid = threadIdx.x;
  const int lo = blockIdx.x * 4096, hi = min(V, lo + 4096);
  float bv = 0.0f;
  int bi = -1;
  slice_amax(lg, lo, hi, tid, bv, bi);
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      float v = sv[tid];
      int i = si[tid];
      amax_merge(v, i, sv[tid + s], si[tid + s]);
      sv[tid] = v;
      si[tid] = i;
    }
    __syncthreads();
  }
  if (tid == 0) { pv[blockIdx.x] = sv[0]; pi[blockIdx.x] = si[0]; }
}

// Stage 2: reduce the slices, write tokens[pos0+M] = next and advance pos0 by M, so the next
// replay of the decode graph runs the sampled token.
__global__ __launch_bounds__(256) void k_argmax2(const float* __restrict__ pv, const int* __restrict__ pi, int P,
                                                 int* __restrict__ tokens, State* __restrict__ st, int M) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int tid = threadIdx.x;
  float bv = 0.0f;
  int bi = -1;
  for (int i = tid; i < P; i += 256) amax_merge(bv, bi, pv[i], pi[i]);
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      float v = sv[tid];
      int i = si[tid];
      amax_merge(v, i, sv[tid + s], si[tid + s]);
      sv[tid] = v;
      si[tid] = i;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const int next = si[0] < 0 ? 0 : si[0];
    const int p = st->pos0 + M;
    tokens[p] = next;
    st->next = next;
    st->pos0 = p;
  }
}

// Positions of the M tokens of a pass (pos0 + m), the per-token positions the list attention reads.
__global__ void k_pass_pos(const State* __restrict__ st, int M, int* __restrict__ pos) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m < M) pos[m] = st->pos0 + m;
}

__global__ void k_set_pos(State* st, int pos0) {
  if (threadIdx.x == 0) st->pos0 = pos0;
}

// Raises the abort flag (what a timed-out bounded wait does), for the test of the rerun path.
__global__ void k_raise_abort(State* st) {
  if (threadIdx.x == 0) st->abort = 1;
}

// Q4_0 GEMM for few tokens: y[m][n] (+)= W[n] . x[m] for M <= a few dozen tokens, with every
// output accumulated exactly as matmul_q4 does (four lane chains over the blocks in order, then
// the lane sum; kernels.c:200-229), so results equal k_matvec's and k_gemm_q4's bit for bit.
// Workgroup: 4 waves x 16 rows (lane = row r, chain j) = 64 rows, TPW tokens shared by the waves.
// The activations of a chunk of 8 groups (32 blocks) are staged in shared memory, double
// buffered (the next chunk's loads are in flight during the current chunk); each lane keeps its
// weights 8 groups ahead in registers.  Grid (Np / 64, ceil(M / TPW)).
constexpr int kRowsChunk = 8;   // groups per activation chunk = weight groups in flight

template <int OP, int TPW>
__global__ __launch_bounds__(256) void k_gemm_rows(Q4Mat W, const uint4* __restrict__ xq, int xstride, int M,
                                                  float* __restrict__ y, int ldy, const float* __restrict__ bias) {
  constexpr int PD = kRowsChunk, CU = PD * 16;              // uint4 per token per chunk
  constexpr int NX = (TPW * CU + 255) / 256;                // staged uint4 per thread
  __shared__ uint4 xs[2][TPW][CU];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane >> 2, j = lane & 3;
  const int m0 = blockIdx.y * TPW;
  const int row = blockIdx.x * 64 + wave * 16 + r;
  const int tile = row >> 6, rr = row & 63;
  const uint4* wq = W.qs + ((size_t)tile * W.ng * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * W.nb8 * 64 + rr;
  const int ng = W.ng, nb = W.nb;
  auto xload = [&](int c, uint4* v) {
#pragma unroll
    for (int u = 0; u < NX; u++) {
      const int i = tid + 256 * u, t = i / CU, k = i - t * CU, m = m0 + t, blk = c * PD * 4 + (k >> 2);
      v[u] = (i < TPW * CU && m < M && blk < nb) ? xq[(size_t)m * xstride * 4 + blk * 4 + (k & 3)] : make_uint4(0, 0, 0, 0);
    }
  };
  auto xstore = [&](int buf, const uint4* v) {
#pragma unroll
    for (int u = 0; u < NX; u++) {
      const int i = tid + 256 * u, t = i / CU, k = i - t * CU;
      if (i < TPW * CU) xs[buf][t][k] = v[u];
    }
  };
  uint4 wr[PD], sr[PD / 2];
#pragma unroll
  for (int u = 0; u < PD; u++) wr[u] = wq[(size_t)u * 256];        // past the end: the zeroed tail
#pragma unroll
  for (int u = 0; u < PD / 2; u++) sr[u] = wd[(size_t)u * 64];
  {
    uint4 v[NX];
    xload(0, v);
    xstore(0, v);
  }
  __syncthreads();
  float acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; t++) acc[t] = 0.0f;
  const int nchunks = (ng + PD - 1) / PD;
  for (int c = 0; c < nchunks; c++) {
    const int buf = c & 1;
    uint4 xn[NX];
    if (c + 1 < nchunks) xload(c + 1, xn);
#pragma unroll
    for (int u = 0; u < PD; u++) {
      const int g = c * PD + u;
      if (g < ng) {
        const uint4 w = wr[u], sc = sr[u >> 1];
        wr[u] = wq[(size_t)(g + PD) * 256];
        if (u & 1) sr[u >> 1] = wd[(size_t)((g + PD) >> 1) * 64];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int b = g * 4 + k;
          if (b < nb) {
            const int hb = ((u & 1) << 2) + k;
            const uint32_t sw = (hb >> 1) == 0 ? sc.x : (hb >> 1) == 1 ? sc.y : (hb >> 1) == 2 ? sc.z : sc.w;
            const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
            const uint32_t wv = k == 0 ? w.x : k == 1 ? w.y : k == 2 ? w.z : w.w;
            const uint32_t lo = wv & 0x0F0F0F0Fu, hi = (wv >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int t = 0; t < TPW; t++) {
              const uint4 xv = xs[buf][t][u * 16 + k * 4 + j];
              int p = sdot4(lo, xv.x, (int)xv.z);
              p = sdot4(hi, xv.y, p);
              acc[t] = acc[t] + (float)p * (dw * __uint_as_float(xv.w));
            }
          }
        }
      }
    }
    if (c + 1 < nchunks) xstore(buf ^ 1, xn);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < TPW; t++) {
    const float v = hsum4(acc[t]);
    const int m = m0 + t;
    if (j == 0 && m < M && row < W.N) {
      float* o = y + (size_t)m * ldy + row;
      if (OP == OP_ADD) *o = *o + v;
      else if (OP == OP_BIAS) *o = v + bias[row];
      else *o = v;
    }
  }
}

// ================================================================ batched decode kernels
//
// B independent sequences decode one token each per step.  Sequence b has its own fp32 cache
// [layer][kv_head][ctx][head_dim] at kc + b * seq_stride and its own position pos[b]; projections run
// as one pass of B tokens (k_gemm_q4), so every per-output operation order is the one-token one.

// Embedding rows of tokens tok[0..B) (kernels.c:312-322).
__global__ void k_embed_list(const uint8_t* __restrict__ emb, int D, const int* __restrict__ tok,
                             float* __restrict__ x) {
  const int m = blockIdx.x;
  const uint8_t* row = emb + (size_t)tok[m] * (D / 32) * 18;
  float* xr = x + (size_t)m * D;
  // four byte pairs per thread load together, then dequantize
  for (int i0 = threadIdx.x; i0 < D / 2; i0 += 4 * blockDim.x) {
    uint32_t dh[4], q[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int idx = i0 + k * blockDim.x;
      const uint8_t* bp = row + (idx >> 4) * 18;
      dh[k] = idx < D / 2 ? (uint32_t)bp[0] | ((uint32_t)bp[1] << 8) : 0u;
      q[k] = idx < D / 2 ? bp[2 + (idx & 15)] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int idx = i0 + k * blockDim.x, blk = idx >> 4, j = idx & 15;
      if (idx < D / 2) {
        const float d = half_bits_to_float(dh[k]);
        xr[32 * blk + j] = (float)((int)(q[k] & 15) - 8) * d;
        xr[32 * blk + 16 + j] = (float)((int)(q[k] >> 4) - 8) * d;
      }
    }
  }
}

// RoPE of token b's q and k heads at position pos[b], then K and V appended to sequence b's cache
// (kernels.c:337-352).  Grid (H + KVH, B), HD/2 threads.
template <class KT>
__global__ void k_rope_kv_list(float* __restrict__ qkv, int QKV, int D, int H, int KVH, int HD,
                               const float* __restrict__ rope, KT* __restrict__ kc, KT* __restrict__ vc,
                               int ctx, int layer, const int* __restrict__ pos, size_t seq_stride) {
  const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x, half = HD / 2;
  const int p = pos[b];
  float* v = qkv + (size_t)b * QKV + h * HD;
  const float* cs = rope + (size_t)p * HD;
  const float c = cs[2 * i], s = cs[2 * i + 1], x0 = v[i], x1 = v[i + half];
  const float y0 = x0 * c - x1 * s, y1 = x1 * c + x0 * s;
  v[i] = y0;
  v[i + half] = y1;
  if (h >= H) {
    const int kh = h - H;
    const size_t off = (size_t)b * seq_stride + (((size_t)layer * KVH + kh) * ctx + p) * HD;
    const float* vs = qkv + (size_t)b * QKV + D + KVH * HD + kh * HD;
    kc[off + i] = (KT)y0;
    kc[off + i + half] = (KT)y1;
    vc[off + i] = (KT)vs[i];
    vc[off + i + half] = (KT)vs[i + half];
  }
}

// Attention of token b over positions [0, pos[b]] of sequence b's cache (kernels.c:355-377), in
// two launches that keep the reference's per-head operation order:
//   k_attn_scores_list  scores s_t = (q . k_t) * 1/sqrt(head_dim) of the G = H/KVH heads of kv
//                       head g, 64 positions per workgroup, each thread one position and all G
//                       heads (its K row in registers): grid (ctx/64, KVH, B).
//   k_attn_pv_list      per (column slice, kv head, sequence): max, e_t = fast_exp(s_t - max), the
//                       sum in position order, p_t = e_t / sum, then out[c] = sum_t p_t * v_t[c] in
//                       position order, one thread per (head, column).  Every workgroup of a
//                       (sequence, kv head) recomputes the same softmax from the scores.
// Scores live in sc [B][H][ctx].
constexpr int kScoreRows = 64;
constexpr int kPvCols = 32;
constexpr int kMaxGroup = 8;    // query heads per kv head


// Floats per head row of the softmax array: room for every position plus the sum's read-ahead.
__host__ __device__ inline int pv_row_stride(int ctx) { return ((ctx + 31) & ~31) + 64; }
// Floats per head row of the scores array (rows start 16-byte aligned).
__host__ __device__ inline int score_stride(int ctx) { return (ctx + 3) & ~3; }

// P.V products with p_t taken from a neighbouring lane: within each 16-lane row of a wave, lane K
// holds p of position t0 + K and `row_newbcast:K` (DPP) hands it to every lane of the row as the
// first operand of the product.  pv_step adds one product to the column's sum and then forms the
// next one, so that the product issues while the add's result is pending.  (The product is inline
// assembly and the add plain code: an add in assembly gets a wait state before it from the
// compiler's hazard check, which takes any assembly statement for a possible DPP read of the sum
// written just before.)
template <int K>
__device__ __forceinline__ float pv_mul(float p, float v) {
  float n;
  if constexpr (K == 0)   // the first broadcast of a fresh p register: two wait states after any write
    asm volatile("s_nop 1\n\tv_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "=v"(n) : "v"(p), "v"(v), "n"(K));
  else
    asm volatile("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "=v"(n) : "v"(p), "v"(v), "n"(K));
  return n;
}
template <int K>
__device__ __forceinline__ void pv_step(float& acc, float d, float p, float v, float& n) {
  acc = acc + d;
  n = pv_mul<K>(p, v);
}
template <int K>
__device__ __forceinline__ float f4_at(const float4& v) {
  return (K & 3) == 0 ? v.x : (K & 3) == 1 ? v.y : (K & 3) == 2 ? v.z : v.w;
}
// One batch of 16 positions: the products of the batch (pv_row::mul) or the previous batch's
// products d added while this batch's are formed (pv_row::step); v holds the column's 16 values.
template <int K>
struct pv_row {
  static __device__ __forceinline__ void mul(float p, const float4* v, float* n) {
    pv_row<K - 1>::mul(p, v, n);
    n[K - 1] = pv_mul<(K - 1) & 15>(p, f4_at<K - 1>(v[(K - 1) >> 2]));
  }
  static __device__ __forceinline__ void step(float& acc, const float* d, float p, const float4* v, float* n) {
    pv_row<K - 1>::step(acc, d, p, v, n);
    pv_step<K - 1>(acc, d[K - 1], p, f4_at<K - 1>(v[(K - 1) >> 2]), n[K - 1]);
  }
};
template <>
struct pv_row<0> {
  static __device__ __forceinline__ void mul(float, const float4*, float*) {}
  static __device__ __forceinline__ void step(float&, const float*, float, const float4*, float*) {}
};


template <int HD, class KT>
__global__ __launch_bounds__(64) void k_attn_scores_list(const float* __restrict__ qkv, int QKV, int H, int KVH,
                                                         const KT* __restrict__ kc, int ctx, int layer,
                                                         float* __restrict__ sc, const int* __restrict__ pos,
                                                         size_t seq_stride) {
  __shared__ __attribute__((aligned(16))) float qs[kMaxGroup * HD];
  const int g = blockIdx.y, b = blockIdx.z, t0 = blockIdx.x * kScoreRows, tid = threadIdx.x, G = H / KVH;
  const int T = pos[b] + 1;
  if (t0 >= T) return;
  {
    float4 qv[kMaxGroup * HD / 256];
    const float4* qg = reinterpret_cast<const float4*>(qkv + (size_t)b * QKV + g * G * HD);
#pragma unroll
    for (int u = 0; u < kMaxGroup * HD / 256; u++) {
      const int i = tid + 64 * u;
      qv[u] = i < G * HD / 4 ? qg[i] : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kMaxGroup * HD / 256; u++) reinterpret_cast<float4*>(qs)[tid + 64 * u] = qv[u];
  }
  __syncthreads();
  const int t = t0 + tid;
  if (t >= T) return;
  const KT* kr = kc + (size_t)b * seq_stride + (((size_t)layer * KVH + g) * ctx + t) * HD;
  float4 kv[HD / 4];                     // the whole K row: one round trip to memory, 16-byte loads
#pragma unroll
  for (int u = 0; u < HD / 8; u++) kv_ld8<KT>(kr + 8 * u, kv[2 * u], kv[2 * u + 1]);
  float s[kMaxGroup][4];
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) {
    s[gh][0] = s[gh][1] = s[gh][2] = s[gh][3] = 0.0f;
    if (gh < G) {
#pragma unroll
      for (int u = 0; u < HD / 4; u++) {
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[gh * HD + 4 * u]);
        s[gh][0] = s[gh][0] + q4.x * kv[u].x;
        s[gh][1] = s[gh][1] + q4.y * kv[u].y;
        s[gh][2] = s[gh][2] + q4.z * kv[u].z;
        s[gh][3] = s[gh][3] + q4.w * kv[u].w;
      }
    }
  }
  const float scale = 1.0f / __builtin_sqrtf((float)HD);
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++)
    if (gh < G) sc[((size_t)b * H + g * G + gh) * score_stride(ctx) + t] = (s[gh][0] + s[gh][1] + s[gh][2] + s[gh][3]) * scale;
}

template <int HD, int CR, class KT>
__global__ __launch_bounds__(256) void k_attn_pv_list(const float* __restrict__ sc, int H, int KVH,
                                                      const KT* __restrict__ vc, int ctx, int layer,
                                                      float* __restrict__ att, int D, const int* __restrict__ pos,
                                                      size_t seq_stride, uint4* __restrict__ xq, int xstride,
                                                      uint4* __restrict__ xh, bool xcd_group) {
  extern __shared__ __attribute__((aligned(16))) float lsm[];
  constexpr int CRS = CR + 4, NV = CR * kPvCols / 4 / 256;      // chunk rows (LDS stride), float4 per thread
  constexpr int PB = 2;                   // score float4 per thread and head in one pass (2048 positions)
  constexpr int S = HD / kPvCols;         // column slices of a (sequence, kv head)
  // Workgroup L runs on XCD L mod 8.  With xcd_group the S slices of one (sequence, kv head) get
  // ids of one residue, so they share that XCD's L2: a V row's cache lines are fetched once, not
  // once per slice that touches them (fp16 slices are half a line).
  const int L = blockIdx.x;
  int slice, unit;
  if (xcd_group) {
    const int x = L % kXcds, k = L / kXcds;
    unit = (k / S) * kXcds + x;
    slice = k % S;
  } else {
    unit = L / S;
    slice = L % S;
  }
  const int c0 = slice * kPvCols, g = unit % KVH, b = unit / KVH, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, G = H / KVH;
  const int T = pos[b] + 1, TS = pv_row_stride(ctx), nch = (T + CR - 1) / CR, CS = score_stride(ctx);
  const int T4 = (T + 3) >> 2;
  float* vs = lsm;                        // [2][kPvCols][CRS]: V chunks, column-major, double buffered
  float* p = vs + 2 * kPvCols * CRS;      // [G][TS]
  float* red = p + G * TS;                // [4 waves][kMaxGroup] maxima, [kMaxGroup] max, [kMaxGroup] sum
  float* rmax = red + 4 * kMaxGroup;
  float* rsum = rmax + kMaxGroup;
  const float* sb = sc + ((size_t)b * H + g * G) * CS;
  const KT* vb = vc + (size_t)b * seq_stride + ((size_t)layer * KVH + g) * ctx * HD + c0;
  // V chunks reach shared memory through registers: register set k holds the chunks ch = k mod 3;
  // chunk ch + 1 is stored at the end of chunk ch, and its set then loads chunk ch + 4 (the last
  // chunk again near the end, so that loads and stores stay unconditional)
  // the register sets hold V as loaded (fp16 stays fp16 until it is stored to shared memory)
  typedef typename KvRaw<KT>::T VRaw;
  auto vload = [&](int ch, VRaw* r) {
#pragma unroll
    for (int u = 0; u < NV; u++) {
      // rows from T on are never read: they repeat row T - 1, so the loads carry no condition
      const int i = tid + 256 * u, row = i / (kPvCols / 4), c4 = i - row * (kPvCols / 4);
      const int t = min(ch * CR + row, T - 1);
      r[u] = kv_raw4<KT>(vb + (size_t)t * HD + 4 * c4);
    }
  };
  auto vstore = [&](int buf, const VRaw* r) {
#pragma unroll
    for (int u = 0; u < NV; u++) {
      const int i = tid + 256 * u, row = i / (kPvCols / 4), c4 = i - row * (kPvCols / 4);
      float* d = vs + (buf * kPvCols + 4 * c4) * CRS + row;
      const float4 w = kv_wide4(r[u]);
      d[0] = w.x;
      d[CRS] = w.y;
      d[2 * CRS] = w.z;
      d[3 * CRS] = w.w;
    }
  };
  auto head_max = [&](float* mxh) {       // block-wide maximum of each head (order-free)
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++) {
      const float m = max64(mxh[gh]);   // DPP and one swizzle, not six shared-memory shuffles
      if (lane == 0) red[wave * kMaxGroup + gh] = m;
    }
    __syncthreads();
    if (tid < G)
      rmax[tid] = __builtin_fmaxf(__builtin_fmaxf(red[tid], red[kMaxGroup + tid]),
                                  __builtin_fmaxf(red[2 * kMaxGroup + tid], red[3 * kMaxGroup + tid]));
    __syncthreads();
  };
  // float4 k of head gh in a pass from q0: thread tid takes q0 + tid for k = 0; for k >= 1 the
  // threads are rotated by 64 (gh mod 4), so that the float4s past the first 256 of each head (a
  // context just past a multiple of 1024 leaves one per head) fall to different waves instead of
  // all to wave 0, whose exponentials and divisions the whole workgroup waits for
  auto qof = [&](int q0, int gh, int k) { return q0 + 256 * k + (k == 0 ? tid : ((tid - 64 * (gh & 3)) & 255)); };
  auto load_scores = [&](int q0, float4 (*v)[PB]) {
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++)
#pragma unroll
      for (int k = 0; k < PB; k++) {
        const int q = qof(q0, gh, k);
        v[gh][k] = (gh < G && q < T4) ? *reinterpret_cast<const float4*>(sb + (size_t)gh * CS + 4 * q)
                                      : make_float4(-1e30f, -1e30f, -1e30f, -1e30f);
      }
  };
  auto fold_max = [&](int q0, float4 (*v)[PB], float* mxh) {
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++)
#pragma unroll
      for (int k = 0; k < PB; k++) {
        const int t = 4 * qof(q0, gh, k);
        float m = mxh[gh];
        m = __builtin_fmaxf(m, t < T ? v[gh][k].x : -1e30f);
        m = __builtin_fmaxf(m, t + 1 < T ? v[gh][k].y : -1e30f);
        m = __builtin_fmaxf(m, t + 2 < T ? v[gh][k].z : -1e30f);
        m = __builtin_fmaxf(m, t + 3 < T ? v[gh][k].w : -1e30f);
        mxh[gh] = m;
      }
  };
  auto store_exp = [&](int q0, float4 (*v)[PB]) {   // e_t = fast_exp(s_t - max), kept in v too
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++)
#pragma unroll
      for (int k = 0; k < PB; k++) {
        const int q = qof(q0, gh, k);
        if (gh < G && q < T4) {
          const float mx = rmax[gh];
          float4 e;
          e.x = fast_exp(v[gh][k].x - mx);
          e.y = fast_exp(v[gh][k].y - mx);
          e.z = fast_exp(v[gh][k].z - mx);
          e.w = fast_exp(v[gh][k].w - mx);
          v[gh][k] = e;
          *reinterpret_cast<float4*>(&p[gh * TS + 4 * q]) = e;
        }
      }
  };
  // the first V chunk loads while the softmax runs (the score registers leave no room for more)
  VRaw vr[3][NV];
  vload(0, vr[0]);
  float mxh[kMaxGroup];
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) mxh[gh] = -1e30f;
  float4 v[kMaxGroup][PB];
  const bool one_pass = T4 <= 256 * PB;   // the scores stay in registers from load to division
  if (one_pass) {
    load_scores(0, v);
    fold_max(0, v, mxh);
    head_max(mxh);
    store_exp(0, v);
  } else {
    for (int q0 = 0; q0 < T4; q0 += 256 * PB) {
      load_scores(q0, v);
      fold_max(q0, v, mxh);
    }
    head_max(mxh);
    for (int q0 = 0; q0 < T4; q0 += 256 * PB) {
      load_scores(q0, v);
      store_exp(q0, v);
    }
  }
  __syncthreads();
  if (tid < G) rsum[tid] = ordered_sum(p + tid * TS, T);   // the sum in position order
  __syncthreads();
  if (one_pass) {
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++)
#pragma unroll
      for (int k = 0; k < PB; k++) {
        const int q = qof(0, gh, k);
        if (gh < G && q < T4) {
          const float sum = rsum[gh];
          float4 e = v[gh][k];
          e.x = e.x / sum;
          e.y = e.y / sum;
          e.z = e.z / sum;
          e.w = e.w / sum;
          *reinterpret_cast<float4*>(&p[gh * TS + 4 * q]) = e;
        }
      }
  } else {
    for (int q = tid; q < T4; q += 256) {
#pragma unroll
      for (int gh = 0; gh < kMaxGroup; gh++) {
        if (gh < G) {
          const float sum = rsum[gh];
          float4 e = *reinterpret_cast<const float4*>(&p[gh * TS + 4 * q]);
          e.x = e.x / sum;
          e.y = e.y / sum;
          e.z = e.z / sum;
          e.w = e.w / sum;
          *reinterpret_cast<float4*>(&p[gh * TS + 4 * q]) = e;
        }
      }
    }
  }
  vstore(0, vr[0]);
#pragma unroll
  for (int k = 1; k < 4; k++) vload(min(k, nch - 1), vr[k % 3]);
  // P.V: thread (head, column); positions in order
  const int gh = tid / kPvCols, c = tid - gh * kPvCols;
  const bool active = gh < G;
  const float* pr = p + (active ? gh : 0) * TS;
  float acc = 0.0f;
  // Products of the last batch of a whole chunk are added at the start of the next chunk (while its
  // first shared-memory reads are in flight) or after the last one.
  float pc[16];
  bool carry = false;
  const int rl = tid & 15;                // this lane's position in a batch (its 16-lane row)
  auto add_carry = [&]() {
#pragma unroll
    for (int k = 0; k < 16; k++) acc = acc + pc[k];
    carry = false;
  };
  auto pv_chunk = [&](int ch) {           // acc += p[t] * V[t][c] over chunk ch, positions in order
    const int t0 = ch * CR, m = min(CR, T - t0);
    const float* vcol = vs + ((ch & 1) * kPvCols + c) * CRS;            // vcol[r]: row r, column c
    if (!active) return;
    if (m == CR) {
      // batch j: positions t0 + 16 j .. t0 + 16 j + 15; register set j & 1 holds its p (one per
      // lane: position rl) and the column's 16 V values; the reads run two batches ahead of the adds
      float pb[2];
      float4 va[2][4];
      auto load = [&](int j, int st) {
        pb[st] = pr[t0 + 16 * j + rl];
#pragma unroll
        for (int u = 0; u < 4; u++) va[st][u] = *reinterpret_cast<const float4*>(vcol + 16 * j + 4 * u);
      };
      load(0, 0);
      load(1, 1);
      if (carry) add_carry();
      float d[16];
      pv_row<16>::mul(pb[0], va[0], d);
#pragma unroll
      for (int j = 0; j + 1 < CR / 16; j++) {
        if (j + 2 < CR / 16) load(j + 2, j & 1);
        float n[16];
        pv_row<16>::step(acc, d, pb[(j + 1) & 1], va[(j + 1) & 1], n);
#pragma unroll
        for (int k = 0; k < 16; k++) d[k] = n[k];
      }
#pragma unroll
      for (int k = 0; k < 16; k++) pc[k] = d[k];
      carry = true;
    } else {
      if (carry) add_carry();
      for (int r = 0; r < m; r++) acc = acc + pr[t0 + r] * vcol[r];
    }
  };
  // Full triples: after chunk ch, chunk ch + 1 goes into the other buffer (read last in chunk ch - 1,
  // before the barrier) and its register set loads chunk ch + 4.  The loop has no exit but its
  // head, so the loads in flight are the same on every entry to it.
  int c3 = 0;
  for (; c3 + 3 < nch; c3 += 3)
#pragma unroll
    for (int k = 0; k < 3; k++) {
      __syncthreads();
      pv_chunk(c3 + k);
      vstore((c3 + k + 1) & 1, vr[(k + 1) % 3]);
      vload(min(c3 + k + 4, nch - 1), vr[(k + 1) % 3]);
    }
  // the last one to three chunks, all loaded already
#pragma unroll
  for (int k = 0; k < 3; k++) {
    if (c3 + k < nch) {
      __syncthreads();
      pv_chunk(c3 + k);
      if (c3 + k + 1 < nch) vstore((c3 + k + 1) & 1, vr[(k + 1) % 3]);
    }
  }
  if (active && carry) add_carry();
  if (active) att[(size_t)b * D + (g * G + gh) * HD + c0 + c] = acc;
  if (xq) {
    // the o projection's activation: each head's 32 outputs are one quantize_row block of row b
    // (what k_quant<QM_PLAIN> would compute from att), quantized here by lanes (head, j) of wave 0
    __syncthreads();
    if (active) vs[gh * kPvCols + c] = acc;
    __syncthreads();
    if (tid < 4 * G) {
      const int hh = tid >> 2, j = tid & 3, base = hh * kPvCols + 2 * j;
      const float v[8] = {vs[base], vs[base + 1], vs[base + 8], vs[base + 9],
                          vs[base + 16], vs[base + 17], vs[base + 24], vs[base + 25]};
      const int blk = ((g * G + hh) * HD + c0) >> 5;
      quantize_item(v, blk, j, xq + (size_t)b * xstride * 4, xh ? xh + xh_tile(b, xstride) : nullptr, b & 15);
    }
  }
}

// Greedy token of every row of logits [B][V] (first maximum, cpu-worker.js:157): partial maxima
// over 4096-entry slices, grid (slices, B).
__global__ __launch_bounds__(256) void k_argmax_rows1(const float* __restrict__ lg, int V, float* __restrict__ pv,
                                                      int* __restrict__ pi, int P) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int tid = threadIdx.x, b = blockIdx.y;
  const float* row = lg + (size_t)b * V;
  const int lo = blockIdx.x * 4096, hi = min(V, lo + 4096);
  float bv = 0.0f;
  int bi = -1;
  slice_amax(row, lo, hi, tid, bv, bi);
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      float v = sv[tid];
      int i = si[tid];
      amax_merge(v, i, sv[tid + s], si[tid + s]);
      sv[tid] = v;
      si[tid] = i;
    }
    __syncthreads();
  }
  if (tid == 0) { pv[b * P + blockIdx.x] = sv[0]; pi[b * P + blockIdx.x] = si[0]; }
}

// Reduce the slices of row b: next token into tok[b] (the next step's input) and out[b], pos[b] + 1.
__global__ __launch_bounds__(256) void k_argmax_rows2(const float* __restrict__ pv, const int* __restrict__ pi, int P,
                                                      int* __restrict__ tok, int* __restrict__ pos,
                                                      int* __restrict__ out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int tid = threadIdx.x, b = blockIdx.x;
  float bv = 0.0f;
  int bi = -1;
  for (int i = tid; i < P; i += 256) amax_merge(bv, bi, pv[b * P + i], pi[b * P + i]);
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      float v = sv[tid];
      int i = si[tid];
      amax_merge(v, i, sv[tid + s], si[tid + s]);
      sv[tid] = v;
      si[tid] = i;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const int next = si[0] < 0 ? 0 : si[0];
    tok[b] = next;
    pos[b] = pos[b] + 1;
    if (out) out[b] = next;
  }
}

// ================================================================ host side

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(call)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess) return fail(Q4HIP_EHIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

constexpr size_t kWeightPadQ = 32768, kWeightPadD = 8192;

struct Mat {
  uint32_t* qs = nullptr;
  uint16_t* d = nullptr;
  int fmt = Q4HIP_TYPE_Q4_0;   // Q4HIP_TYPE_Q4_0 or Q4HIP_TYPE_Q8_0 (the output head only)
  int N = 0, K = 0, nb = 0, ng = 0, nb8 = 0, Np = 0;
  int64_t loaded = 0;
  Q4Mat view() const { return Q4Mat{(const uint4*)qs, (const uint4*)d, N, nb, ng, nb8, Np}; }
};

// The zeroing is ordered on stream s, the stream every later upload and kernel of m runs on (a
// non-blocking stream is not ordered after work on the legacy default stream).
int mat_alloc(Mat& m, int N, int K, hipStream_t s, int fmt = Q4HIP_TYPE_Q4_0) {
  m.fmt = fmt;
  m.N = N;
  m.K = K;
  m.nb = K / 32;
  m.ng = fmt == Q4HIP_TYPE_Q8_0 ? (m.nb + 1) / 2 : (m.nb + 3) / 4;
  m.loaded = 0;
  m.nb8 = (m.nb + 7) / 8;
  m.Np = (N + kRowTile - 1) / kRowTile * kRowTile;
  // zeroed tail: the GEMMs' weight prefetch reads up to 8 groups past the last one unconditionally
  const size_t qbytes = (size_t)m.Np * m.ng * 64 + kWeightPadQ, dbytes = (size_t)m.Np * m.nb8 * 16 + kWeightPadD;
  HIPCHK(hipMalloc(&m.qs, qbytes));
  HIPCHK(hipMalloc(&m.d, dbytes));
  HIPCHK(hipMemsetAsync(m.qs, 0, qbytes, s));
  HIPCHK(hipMemsetAsync(m.d, 0, dbytes, s));
  return Q4HIP_OK;
}

void mat_free(Mat& m) {
  if (m.qs) (void)hipFree(m.qs);
  if (m.d) (void)hipFree(m.d);
  m.qs = nullptr;
  m.d = nullptr;
}

// Upload GGUF Q4_0 (or, for a Q8 matrix, Q8_0) rows [row0, row0+rows) of m through a device
// staging buffer.
int mat_upload(Mat& m, int row0, int64_t rows, const void* data, hipStream_t s) {
  if (row0 < 0 || rows <= 0 || row0 + rows > m.N) return fail(Q4HIP_EINVAL, "rows %d..%lld outside 0..%d", row0, (long long)(row0 + rows), m.N);
  const bool q8 = m.fmt == Q4HIP_TYPE_Q8_0;
  const size_t bytes = (size_t)rows * m.nb * (q8 ? 34 : 18);
  uint8_t* raw = nullptr;
  HIPCHK(hipMalloc(&raw, bytes));
  hipError_t e = hipMemcpyAsync(raw, data, bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    const int64_t n = rows * m.nb;
    if (q8)
      k_repack_q8<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(raw, rows, m.nb, m.ng, m.nb8, row0, m.qs, m.d);
    else
      k_repack_q4<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(raw, rows, m.nb, m.ng, m.nb8, row0, m.qs, m.d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(raw);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "%s upload: %s", q8 ? "Q8_0" : "Q4_0", hipGetErrorString(e));
  m.loaded += rows;
  return Q4HIP_OK;
}

struct Layer {
  Mat qkv, o, gu, down;
  float *attn_norm = nullptr, *ffn_norm = nullptr, *bqkv = nullptr;
  int64_t n_attn_norm = 0, n_ffn_norm = 0, n_bqkv = 0;
};

}  // namespace

struct q4hip {
  int D, NL, F, H, KVH, HD, QKV, V, ctx, MT, device;
  float eps;
  hipStream_t stream = nullptr;
  std::vector<Layer> L;
  Mat head;
  uint8_t* embd = nullptr;
  int64_t embd_loaded = 0;
  float* out_norm = nullptr;
  int64_t n_out_norm = 0;
  float* rope = nullptr;
  bool rope_set = false;
  float *x = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr, *logits = nullptr;
  void *kc = nullptr, *vc = nullptr;   // K/V cache [layer][kv_head][ctx][head_dim]: fp32, or fp16 when kv16
  bool kv16 = false;
  int kvb = 4;                         // bytes per cache element
  uint4* xq = nullptr;
  uint4* xh = nullptr;     // the same activations as fp16 matrix-core operands (multi-token passes)
  uint4* xh2 = nullptr;    // the SwiGLU activation's operands when written by the gate|up projection
                           // itself (that kernel still reads xh)
  int xstride = 0;   // activation blocks per token row of xq
  float* ascr = nullptr;   // attention scores of multi-token passes: [MT][H][score_stride(ctx)], allocated on first use
  int* tpos = nullptr;     // positions of the tokens of a pass
  int list_attn = -1;      // multi-token passes use the list attention kernels (1), k_attn_prefill (0), unknown (-1)
  float* am_v = nullptr;
  int* am_i = nullptr;
  int am_parts = 0;
  int* tokens = nullptr;
  State* st = nullptr;
  int* pin_ids = nullptr;     // pinned staging: token ids in, ids out
  int* pin_next = nullptr;
  hipGraphExec_t graph = nullptr;
  bool graph_failed = false;
  int last_mode = 0;
  // persistent decode (one launch per forward/generate call)
  int mode = Q4HIP_DECODE_AUTO;
  bool pers_ok = false;        // shape and device admit the persistent kernel
  bool pers_broken = false;    // a launch failed or timed out: use the graph from then on
  LayerView* d_layers = nullptr;
  uint64_t* ll = nullptr;
  int pers_grid = 0;
  int* pers_wgmap[2] = {nullptr, nullptr};   // physical -> logical workgroup, one attention workgroup per head or two
  const char* pers_why = "";
  int pers_kv_tile = 0;
  size_t pers_lds = 0;
  size_t pers_hc_off = 0, pers_hc_rg = 0;   // resident head row groups: shared-memory offset, bytes each
  bool pers_head_cache = true;              // Q4HIP_HEAD_CACHE=0: stream the whole head every step
  int pers_ring = 0;
  int pers_test_abort = 0;   // persistent launches still to start with the abort flag raised
  int pers_last_steps = 0;   // steps of the last persistent launch (the epochs it may have used)
  int pers_pf[4] = {4, 4, 4, 8};   // weight prefetch delays of the roles (PArgs::pf), measured best
  int pers_nap = 1;
  const void* pers_fn = nullptr;
  uint64_t* lsc = nullptr;     // score exchange of the split attention ([H][ctx] entries)
  int pers_split_from = 512;   // launches starting at this position or later split each head over two workgroups
  bool pers_split_ok = false;  // the roles fit the device with two attention workgroups per head
  // profiling: events recorded around each launch of an eager step
  std::vector<std::pair<int, hipEvent_t>>* prof = nullptr;
};

namespace {

void prof_mark(q4hip* h, int cls) {
  if (!h->prof) return;
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return;
  (void)hipEventRecord(e, h->stream);
  h->prof->push_back({cls, e});
}

int check_ready(q4hip* h) {
  for (int l = 0; l < h->NL; l++) {
    const Layer& y = h->L[l];
    if (y.qkv.loaded < y.qkv.N || y.o.loaded < y.o.N || y.gu.loaded < y.gu.N || y.down.loaded < y.down.N)
      return fail(Q4HIP_ESTATE, "layer %d: weights not fully loaded", l);
    if (y.n_attn_norm < h->D || y.n_ffn_norm < h->D || y.n_bqkv < h->QKV)
      return fail(Q4HIP_ESTATE, "layer %d: norms or bias not loaded", l);
  }
  if (h->embd_loaded < h->V) return fail(Q4HIP_ESTATE, "token embedding not loaded");
  if (h->head.loaded < h->head.N) return fail(Q4HIP_ESTATE, "output head not loaded");
  if (h->n_out_norm < h->D) return fail(Q4HIP_ESTATE, "output norm not loaded");
  if (!h->rope_set) return fail(Q4HIP_ESTATE, "RoPE table not set");
  return Q4HIP_OK;
}

// Kernel choice for passes of M > 8 tokens (every candidate gives the same bits):
//   k_gemm_sk (matrix cores, operands streamed through a shared-memory ring), one lane chain per
//   wave (JS 4) when the matrix has too few rows to give 512 workgroups of 64 rows, else all four
//   chains per wave (JS 1).  Measured on MI355X against the earlier matrix-core GEMM with register
//   prefetch: 1024-token prefill 15.0 -> 10.5 ms, 32-sequence batched step 4.3 -> 3.7 ms.
// Q4HIP_GEMM=valu keeps the matrix cores out (k_gemm_rows up to 64 tokens, else k_gemm_q4).
enum { GK_ROWS2, GK_ROWS1, GK_TILED, GK_SK4, GK_SK1 };

constexpr int kSkR4 = 4, kSkR1 = 4;    // ring slots of k_gemm_sk (JS 4: 43 KB, JS 1: 52.2 KB; 6 or 8 were slower)

// Whether multi-token projections use the matrix cores (not under Q4HIP_GEMM=valu).
bool sk_enabled() {
  static const bool on = [] { const char* e = getenv("Q4HIP_GEMM"); return !(e && strcmp(e, "valu") == 0); }();
  return on;
}

int pick_gemm(const Mat& W, int M, bool have_xh) {
  if (have_xh && sk_enabled() && W.nb % 4 == 0)            // k_gemm_sk takes whole groups of 4 blocks
    return (W.Np / 64) * ((M + 15) / 16) >= 512 ? GK_SK1 : GK_SK4;
  if (M <= 64) return M >= 16 ? GK_ROWS2 : GK_ROWS1;
  return GK_TILED;
}

// Token-tile-major placement of k_gemm_sk's workgroups (sk_place) for passes of a multiple of 8
// token tiles over weights that fit one XCD's 4 MB L2 (the prefill's qkv, o and down).  Otherwise
// row groups run fastest: with few tiles, the workgroups of one row group then meet on one XCD
// whenever the row-group count is a multiple of 8, and the weights are fetched once (measured on
// the 32-sequence step: tile-major placement raised gate/up fetch 0.49 -> 0.90 GB per step).
bool sk_by_tile(const Mat& W, int ntiles) {
  const size_t wbytes = (size_t)W.Np * W.nb * 18;
  return ntiles % kXcds == 0 && wbytes <= ((size_t)3 << 20);
}

template <int OP, int JS, int R>
void launch_sk(hipStream_t s, const Mat& W, const uint4* xh, int xstride, int M, float* y, int ldy, const float* bias) {
  const int nt = (M + 15) / 16;
  const bool by_tile = sk_by_tile(W, nt);
  k_gemm_sk<OP, JS, R><<<(unsigned)sk_grid(W.Np / (JS == 4 ? 16 : 64), nt, by_tile), 256, 0, s>>>(
      W.view(), xh, xstride, M, y, ldy, bias, by_tile);
}

// gate|up projection with the SwiGLU + quantize of its output fused (k_gemm_sk, EPI 1): act of the M
// tokens into xq and xh_out, exactly what the projection followed by k_quant<QM_SWIGLU> writes.
// xh_out must not be xh_in (other workgroups still read their input blocks).  False (nothing
// launched) where that path does not apply; the caller then runs the two launches.
bool launch_gu_swiglu(hipStream_t s, const Mat& W, const uint4* xh_in, int xstride, int M, uint4* xq_out,
                      uint4* xh_out, int F) {
  if (!xh_in || F % 32 || !sk_enabled() || W.nb % 4) return false;
  const int nt = (M + 15) / 16;
  const bool by_tile = sk_by_tile(W, nt);
  k_gemm_sk<OP_STORE, 1, kSkR1, 1><<<(unsigned)sk_grid(F / 32, nt, by_tile), 256, 0, s>>>(
      W.view(), xh_in, xstride, M, nullptr, 0, nullptr, by_tile, xq_out, xh_out, F);
  return true;
}

// q|k|v projection of a batch step with RoPE and the cache append fused (k_gemm_sk, EPI 2): q of the
// B tokens into qkv, k and v into each sequence's cache at its position -- what the bias projection
// followed by k_rope_kv_list writes.  False (nothing launched) where that path does not apply.
bool launch_qkv_rope(hipStream_t s, const Mat& W, const uint4* xh, int xstride, int M, float* qkv, int QKV,
                     const float* bias, const SkRope& rp) {
  if (!xh || rp.hd % 16 || pick_gemm(W, M, true) != GK_SK4) return false;
  const int nt = (M + 15) / 16;
  const bool by_tile = sk_by_tile(W, nt);
  k_gemm_sk<OP_BIAS, 4, kSkR4, 2><<<(unsigned)sk_grid(W.Np / 16, nt, by_tile), 256, 0, s>>>(
      W.view(), xh, xstride, M, qkv, QKV, bias, by_tile, nullptr, nullptr, 0, rp);
  return true;
}

template <int OP, int TPW>
void launch_rows(hipStream_t s, const Mat& W, const uint4* xq, int xstride, int M, float* y, int ldy, const float* bias) {
  k_gemm_rows<OP, TPW><<<dim3((unsigned)(W.Np / 64), (unsigned)((M + TPW - 1) / TPW)), 256, 0, s>>>(
      W.view(), xq, xstride, M, y, ldy, bias);
}

template <int OP>
void launch_matvec(hipStream_t s, const Mat& W, const uint4* xq, int xstride, int M, float* y, int ldy,
                   const float* bias, const uint4* xh = nullptr) {
  const unsigned grid = (unsigned)(W.Np / 16);
  if (M == 1) {
    if (W.nb == 28)
      k_matvec_stream<28, OP><<<stream_grid(W.Np / 16, stream_waves(28)), 256, 0, s>>>(W.view(), xq, y, bias);
    else if (W.nb == 48)
      k_matvec_stream<48, OP><<<stream_grid(W.Np / 16, stream_waves(48)), 256, 0, s>>>(W.view(), xq, y, bias);
    else if (W.nb >= kSplitMinBlocks && W.nb <= kSplitMaxBlocks)
      k_matvec_split<OP><<<grid, kSplitThreads, split_lds(W.nb), s>>>(W.view(), xq, y, bias);
    else
      k_matvec<1, OP><<<grid, 64, (size_t)W.nb * 64, s>>>(W.view(), xq, xstride, 1, y, ldy, bias);
    return;
  }
  if (M <= 8) {
    k_matvec<kMaxChunk, OP><<<grid, 64, 0, s>>>(W.view(), xq, xstride, M, y, ldy, bias);
    return;
  }
  switch (pick_gemm(W, M, xh != nullptr)) {
    case GK_ROWS2: launch_rows<OP, 2>(s, W, xq, xstride, M, y, ldy, bias); break;
    case GK_ROWS1: launch_rows<OP, 1>(s, W, xq, xstride, M, y, ldy, bias); break;
    case GK_SK4: launch_sk<OP, 4, kSkR4>(s, W, xh, xstride, M, y, ldy, bias); break;
    case GK_SK1: launch_sk<OP, 1, kSkR1>(s, W, xh, xstride, M, y, ldy, bias); break;
    default:
      k_gemm_q4<OP><<<dim3((unsigned)(W.Np / kGemmRows), (unsigned)((M + kGemmTokens - 1) / kGemmTokens)), 256, 0, s>>>(
          W.view(), xq, xstride, M, y, ldy, bias);
  }
}

// logits = head . x for one token: Q4_0 (the synthetic configurations) or Q8_0 (real files).
void launch_head(hipStream_t s, const Mat& W, const uint4* xq, float* logits) {
  if (W.fmt == Q4HIP_TYPE_Q8_0)
    k_matvec_q8<<<(unsigned)(W.Np / 16), 64, (size_t)W.nb * 64, s>>>(W.view(), xq, logits);
  else
    launch_matvec<OP_STORE>(s, W, xq, 0, 1, logits, W.N, nullptr);
}

// Attention of a prompt pass (every row reads one shared cache), in three launches: the scores as
// above; k_softmax_rows turns each (row, head)'s scores into p_t = e_t / sum in place (the
// reference's max, e_t = fast_exp(s_t - max), sum in position order, division; kernels.c:367-371);
// k_pv_tiles forms out[c] = sum_t p_t * v_t[c] in position order (kernels.c:372-375) for QT
// consecutive rows at once, so each V chunk staged in shared memory serves QT rows.
// k_softmax_rows: grid (KVH, rows), 256 threads, dynamic shared memory softmax_lds(H, KVH, ctx).
__global__ __launch_bounds__(256) void k_softmax_rows(float* __restrict__ sc, int H, int KVH, int ctx,
                                                      const int* __restrict__ pos) {
  extern __shared__ __attribute__((aligned(16))) float lsm[];
  const int g = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, G = H / KVH;
  const int T = pos[b] + 1, TS = pv_row_stride(ctx), CS = score_stride(ctx), T4 = (T + 3) >> 2;
  float* e = lsm;                         // [G][TS] exponentials
  float* red = e + G * TS;                // [4 waves][kMaxGroup], then max [kMaxGroup], sum [kMaxGroup]
  float* rmax = red + 4 * kMaxGroup;
  float* rsum = rmax + kMaxGroup;
  float* sb = sc + ((size_t)b * H + g * G) * CS;
  float mxh[kMaxGroup];
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) mxh[gh] = -1e30f;
  for (int q = tid; q < T4; q += 256) {                    // maxima (order-free)
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++) {
      if (gh < G) {
        const float4 v = *reinterpret_cast<const float4*>(sb + (size_t)gh * CS + 4 * q);
        const int t = 4 * q;
        float m = mxh[gh];
        m = __builtin_fmaxf(m, v.x);
        m = __builtin_fmaxf(m, t + 1 < T ? v.y : -1e30f);
        m = __builtin_fmaxf(m, t + 2 < T ? v.z : -1e30f);
        m = __builtin_fmaxf(m, t + 3 < T ? v.w : -1e30f);
        mxh[gh] = m;
      }
    }
  }
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) {
    const float m = max64(mxh[gh]);
    if (lane == 0) red[wave * kMaxGroup + gh] = m;
  }
  __syncthreads();
  if (tid < G)
    rmax[tid] = __builtin_fmaxf(__builtin_fmaxf(red[tid], red[kMaxGroup + tid]),
                                __builtin_fmaxf(red[2 * kMaxGroup + tid], red[3 * kMaxGroup + tid]));
  __syncthreads();
  for (int q = tid; q < T4; q += 256) {                    // e_t = fast_exp(s_t - max)
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++) {
      if (gh < G) {
        const float4 v = *reinterpret_cast<const float4*>(sb + (size_t)gh * CS + 4 * q);
        const float mx = rmax[gh];
        float4 x;
        x.x = fast_exp(v.x - mx);
        x.y = fast_exp(v.y - mx);
        x.z = fast_exp(v.z - mx);
        x.w = fast_exp(v.w - mx);
        *reinterpret_cast<float4*>(&e[gh * TS + 4 * q]) = x;
      }
    }
  }
  __syncthreads();
  if (tid < G) rsum[tid] = ordered_sum(e + tid * TS, T);   // the sum in position order
  __syncthreads();
  for (int q = tid; q < T4; q += 256) {                    // p_t = e_t / sum, over the scores
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++) {
      if (gh < G) {
        const float sum = rsum[gh];
        float4 x = *reinterpret_cast<const float4*>(&e[gh * TS + 4 * q]);
        x.x = x.x / sum;
        x.y = x.y / sum;
        x.z = x.z / sum;
        x.w = x.w / sum;
        *reinterpret_cast<float4*>(sb + (size_t)gh * CS + 4 * q) = x;
      }
    }
  }
}

// Q4HIP_PV_TILES=0 keeps prompt passes on k_attn_pv_list (same bits; for comparison).
bool pv_tiles_off() {
  static const bool off = [] { const char* e = getenv("Q4HIP_PV_TILES"); return e && e[0] == '0'; }();
  return off;
}

// Q4HIP_ATTN_ROWS=0 keeps prompt passes on the three-launch path (scores, softmax, P.V tiles; same
// bits): also the path where k_attn_rows does not apply (head_dim 128, or a context whose scores do
// not fit shared memory).
bool attn_rows_off() {
  static const bool off = [] { const char* e = getenv("Q4HIP_ATTN_ROWS"); return e && e[0] == '0'; }();
  return off;
}

size_t softmax_lds(int H, int KVH, int ctx) {
  return (size_t)((H / KVH) * pv_row_stride(ctx) + 6 * kMaxGroup) * sizeof(float);
}

// k_pv_tiles: grid (HD / 32, KVH, ceil(B / QT)), QT * G * 32 threads: thread (row q of the tile, head
// h of the kv group, column c of the slice) runs its own chain over positions 0 .. pos[b] in order,
// p and V read in chunks of 64 positions staged in shared memory (V column-major, 68 floats per
// column: a 16-byte read of 16 columns hits distinct banks).  With xq, each (row, head)'s 32 outputs
// are quantized as one quantize_row block, as in k_attn_pv_list.
constexpr int kPvTileRows = 4;          // QT
constexpr int kPvChunk = 64;
template <int HD, class KT, int NVT>
__global__ __launch_bounds__(1024) void k_pv_tiles(const float* __restrict__ sc, int H, int KVH,
                                                   const KT* __restrict__ vc, int ctx, int layer,
                                                   float* __restrict__ att, int D, const int* __restrict__ pos, int B,
                                                   uint4* __restrict__ xq, int xstride, uint4* __restrict__ xh) {
  constexpr int CHS = kPvChunk + 4;
  __shared__ __attribute__((aligned(16))) float vs[kPvCols * CHS];
  __shared__ __attribute__((aligned(16))) float ps[kPvTileRows * kMaxGroup * CHS];
  const int c0 = blockIdx.x * kPvCols, g = blockIdx.y, b0 = blockIdx.z * kPvTileRows, tid = threadIdx.x;
  const int G = H / KVH, nthr = kPvTileRows * G * kPvCols, CS = score_stride(ctx);
  const int q = tid / (G * kPvCols), h = (tid / kPvCols) % G, c = tid % kPvCols;
  const int b = b0 + q;
  const bool active = tid < nthr && b < B;
  const int T = active ? pos[b] + 1 : 0;
  int tmax = 0;                                            // the tile's longest row
  for (int k = 0; k < kPvTileRows; k++)
    if (b0 + k < B) tmax = max(tmax, pos[b0 + k] + 1);
  const KT* vb = vc + ((size_t)layer * KVH + g) * ctx * HD + c0;
  // staging: V float4 i (row i / 8, columns 4 (i % 8) ..) for i = tid + k blockDim (k < NVT, with
  // NVT blockDim >= 512: blockDim = 128 G) and p float4 tid (row r = tid / 16 of the tile's (q, h) rows,
  // positions 4 (tid % 16) ..; 64 G of them).  A chunk's values come through one of two register
  // sets, loaded two chunks ahead (V as loaded: fp16 stays fp16 until it is stored), so the loads
  // of the next chunks are in flight while one is added; the loop runs in whole pairs, the sets'
  // roles fixed in each pass.
  typedef typename KvRaw<KT>::T VRaw;
  constexpr int NVI = kPvChunk * kPvCols / 4;              // V float4 per chunk
  const bool pth = tid < kPvTileRows * G * (kPvChunk / 4);
  const int pr_ = tid / (kPvChunk / 4), pu4 = (tid % (kPvChunk / 4)) * 4;
  const int pq = pr_ / G, ph = pr_ - pq * G, pb = b0 + pq;
  const int nch = (tmax + kPvChunk - 1) / kPvChunk;
  struct Set {
    VRaw v[NVT];
    float4 p;
  };
  auto load = [&](int ch, Set& st) {
    const int t0 = min(ch, nch - 1) * kPvChunk;
#pragma unroll
    for (int k = 0; k < NVT; k++) {
      const int i = tid + k * (int)blockDim.x;
      if (i < NVI) st.v[k] = kv_raw4<KT>(vb + (size_t)min(t0 + (i >> 3), tmax - 1) * HD + (i & 7) * 4);   // rows from tmax on are never used
    }
    st.p = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (pth && pb < B && t0 + pu4 < tmax)
      st.p = *reinterpret_cast<const float4*>(sc + ((size_t)pb * H + g * G + ph) * CS + t0 + pu4);
  };
  auto store = [&](const Set& st) {
#pragma unroll
    for (int k = 0; k < NVT; k++) {
      const int i = tid + k * (int)blockDim.x, row = i >> 3, c4 = (i & 7) * 4;
      if (i < NVI) {
        const float4 w = kv_wide4(st.v[k]);
        vs[(c4 + 0) * CHS + row] = w.x;
        vs[(c4 + 1) * CHS + row] = w.y;
        vs[(c4 + 2) * CHS + row] = w.z;
        vs[(c4 + 3) * CHS + row] = w.w;
      }
    }
    if (pth) *reinterpret_cast<float4*>(&ps[pr_ * CHS + pu4]) = st.p;
  };
  const float* pr = ps + (q * G + h) * CHS;
  const float* vr = vs + c * CHS;
  float acc = 0.0f;
  auto chunk = [&](int t0) {
    if (active) {
      if (t0 + kPvChunk <= T) {                            // a whole chunk: no select on the chain
#pragma unroll
        for (int u = 0; u < kPvChunk; u += 4) {
          const float4 p4 = *reinterpret_cast<const float4*>(pr + u);
          const float4 v4 = *reinterpret_cast<const float4*>(vr + u);
          acc = acc + p4.x * v4.x;
          acc = acc + p4.y * v4.y;
          acc = acc + p4.z * v4.z;
          acc = acc + p4.w * v4.w;
        }
      } else if (t0 < T) {
        const int n = T - t0;
        for (int u = 0; u < kPvChunk; u++) {
          const float x = acc + pr[u] * vr[u];
          acc = u < n ? x : acc;
        }
      }
    }
  };
  constexpr int NS = 2;                                    // register sets
  Set sets[NS];
#pragma unroll
  for (int k = 0; k < NS; k++) load(k, sets[k]);
  int cs = 0;
  for (; cs + NS < nch; cs += NS)
#pragma unroll
    for (int k = 0; k < NS; k++) {
      __syncthreads();                                     // the previous chunk is read
      store(sets[k]);
      load(cs + k + NS, sets[k]);
      __syncthreads();
      chunk((cs + k) * kPvChunk);
    }
#pragma unroll
  for (int k = 0; k < NS; k++) {                           // the last chunks, loaded already
    if (cs + k < nch) {
      __syncthreads();
      store(sets[k]);
      __syncthreads();
      chunk((cs + k) * kPvChunk);
    }
  }
  if (active) att[(size_t)b * D + (g * G + h) * HD + c0 + c] = acc;
  if (xq) {
    __syncthreads();
    float* o = vs;                                          // [q][h][32] outputs of this slice
    if (active) o[(q * G + h) * kPvCols + c] = acc;
    __syncthreads();
    if (tid < 4 * G * kPvTileRows) {
      const int qq = tid / (4 * G), hh = (tid / 4) % G, j = tid & 3, bb = b0 + qq;
      if (bb < B) {
        const int base = (qq * G + hh) * kPvCols + 2 * j;
        const float v[8] = {o[base], o[base + 1], o[base + 8], o[base + 9],
                            o[base + 16], o[base + 17], o[base + 24], o[base + 25]};
        const int blk = ((g * G + hh) * HD + c0) >> 5;
        quantize_item(v, blk, j, xq + (size_t)bb * xstride * 4, xh ? xh + xh_tile(bb, xstride) : nullptr, bb & 15);
      }
    }
  }
}

// Attention of a prompt pass in one launch (head_dim 64, kernels.c:355-377): workgroup (kv group g,
// row b) keeps the G heads' scores over positions [0, pos[b]] in shared memory and runs there the
// reference's steps in its order -- scores as k_attn_scores_list forms them, the maximum,
// e_t = fast_exp(s_t - max), the sum in position order, p_t = e_t / sum, and out[c] = sum_t p_t *
// v_t[c] in position order (one thread per head and column) -- then writes att and its quantized
// blocks as k_pv_tiles does.  Scores and probabilities never go to memory: the three-launch path
// writes and reads them back twice.  Rows run longest first (row B - 1 - blockIdx.y).
// Grid (KVH, B), kAttnRowsThreads threads, dynamic shared memory attn_rows_lds(G, ctx).
constexpr int kAttnRowsThreads = 512;       // 8 waves: one per head of a group of up to 8
constexpr int kAttnRowsChunk = 64;          // V rows staged per step
__host__ __device__ inline int attn_rows_vstride() { return kAttnRowsChunk + 4; }
inline size_t attn_rows_lds(int G, int ctx) {
  return (size_t)(G * pv_row_stride(ctx) + 2 * 64 * attn_rows_vstride() + 3 * kMaxGroup * 8) * sizeof(float);
}

template <class KT>
__global__ __launch_bounds__(kAttnRowsThreads) void k_attn_rows(const float* __restrict__ qkv, int QKV, int H, int KVH,
                                                               const KT* __restrict__ kc, const KT* __restrict__ vc,
                                                               int ctx, int layer, const int* __restrict__ pos, int B,
                                                               float* __restrict__ att, int D, uint4* __restrict__ xq,
                                                               int xstride, uint4* __restrict__ xh) {
  constexpr int HD = 64, CH = kAttnRowsChunk, NW = kAttnRowsThreads / 64;
  const int CHS = attn_rows_vstride();
  extern __shared__ __attribute__((aligned(16))) float lsm[];
  const int g = blockIdx.x, b = B - 1 - (int)blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = H / KVH, T = pos[b] + 1, TS = pv_row_stride(ctx);
  float* e = lsm;                           // [G][TS] scores, then exponentials, then probabilities
  float* vs = e + G * TS;                   // [2][64 columns][CHS] V chunks, column-major, double-buffered
  float* red = vs + 2 * HD * CHS;           // [NW][kMaxGroup] maxima, [kMaxGroup] max, [kMaxGroup] sum
  float* rmax = red + NW * kMaxGroup;
  float* rsum = rmax + kMaxGroup;
  const size_t cb = ((size_t)layer * KVH + g) * ctx * HD;
  // V: a chunk's 64 rows come through one of NS register sets, loaded NS chunks ahead; the first NS
  // load while the scores and the softmax run (rows from T on repeat row T - 1, never added)
  typedef typename KvRaw<KT>::T VRaw;
  constexpr int NV = CH * HD / 4 / kAttnRowsThreads, NS = 4;  // float4 of a chunk per thread, sets
  const int nch = (T + CH - 1) / CH;
  // lane l of a wave loads row l of the chunk (4 columns), so that its column-major stores below
  // fall on distinct banks
  auto load = [&](int ch, VRaw* r) {
    const int t0 = min(ch, nch - 1) * CH;
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int i = tid + k * kAttnRowsThreads, row = i & 63, c4 = (i >> 6) * 4;
      r[k] = kv_raw4<KT>(vc + cb + (size_t)min(t0 + row, T - 1) * HD + c4);
    }
  };
  VRaw vset[NS][NV];
#pragma unroll
  for (int k = 0; k < NS; k++) load(k, vset[k]);
  // scores (k_attn_scores_list's order): four lane sums over i = j mod 4, summed, scaled; q is read
  // at workgroup-uniform addresses (scalar loads), not through shared memory
  const float* qg = qkv + (size_t)b * QKV + g * G * HD;
  const float scale = 1.0f / __builtin_sqrtf((float)HD);
  float mxh[kMaxGroup];
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) mxh[gh] = -1e30f;
  for (int t = tid; t < T; t += kAttnRowsThreads) {
    const KT* kr = kc + cb + (size_t)t * HD;
    float4 kv[HD / 4];
#pragma unroll
    for (int u = 0; u < HD / 8; u++) kv_ld8<KT>(kr + 8 * u, kv[2 * u], kv[2 * u + 1]);
#pragma unroll
    for (int gh = 0; gh < kMaxGroup; gh++) {
      if (gh < G) {
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int u = 0; u < HD / 4; u++) {
          const float4 q4 = *reinterpret_cast<const float4*>(qg + gh * HD + 4 * u);
          s0 = s0 + q4.x * kv[u].x;
          s1 = s1 + q4.y * kv[u].y;
          s2 = s2 + q4.z * kv[u].z;
          s3 = s3 + q4.w * kv[u].w;
        }
        const float sv = (s0 + s1 + s2 + s3) * scale;
        e[gh * TS + t] = sv;
        mxh[gh] = __builtin_fmaxf(mxh[gh], sv);
      }
    }
  }
  // the maximum of each head (order-free)
#pragma unroll
  for (int gh = 0; gh < kMaxGroup; gh++) {
    const float m = max64(mxh[gh]);
    if (lane == 0) red[wave * kMaxGroup + gh] = m;
  }
  lds_barrier();
  if (tid < G) {
    float m = red[tid];
    for (int w = 1; w < NW; w++) m = __builtin_fmaxf(m, red[w * kMaxGroup + tid]);
    rmax[tid] = m;
  }
  lds_barrier();
  for (int gh = 0; gh < G; gh++) {
    const float mx = rmax[gh];
    for (int t = tid; t < T; t += kAttnRowsThreads) e[gh * TS + t] = fast_exp(e[gh * TS + t] - mx);
  }
  lds_barrier();
  if (tid < G) rsum[tid] = ordered_sum(e + tid * TS, T);   // the sum in position order
  lds_barrier();
  for (int gh = 0; gh < G; gh++) {
    const float sum = rsum[gh];
    for (int t = tid; t < T; t += kAttnRowsThreads) e[gh * TS + t] = e[gh * TS + t] / sum;
  }
  // P.V: thread (head = wave, column = lane) adds p_t * v_t[c] over the chunks in order (each
  // product rounded, then added).  In a batch of 16 positions lane K of every 16-lane row holds p of
  // position K and a DPP broadcast hands it to the whole row as the product's first operand
  // (pv_row), so a wave reads its head's probabilities with one 4-byte read per batch; the
  // products of a batch are formed while the previous batch's are added, and a whole chunk's last
  // batch is added at the start of the next chunk.
  auto store = [&](int buf, const VRaw* r) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int i = tid + k * kAttnRowsThreads, row = i & 63, c4 = (i >> 6) * 4;
      float* d = vs + (buf * HD + c4) * CHS + row;
      const float4 w = kv_wide4(r[k]);
      d[0] = w.x;
      d[CHS] = w.y;
      d[2 * CHS] = w.z;
      d[3 * CHS] = w.w;
    }
  };
  const bool active = wave < G;
  const float* pr = e + (active ? wave : 0) * TS;
  const int rl = lane & 15;
  float acc = 0.0f;
  float pc[16];
  bool carry = false;
  auto add_carry = [&]() {
#pragma unroll
    for (int k = 0; k < 16; k++) acc = acc + pc[k];
    carry = false;
  };
  auto chunk = [&](int ch) {
    const int t0 = ch * CH, m = min(CH, T - t0);
    const float* vcol = vs + ((ch & 1) * HD + lane) * CHS;
    if (!active) return;
    if (m == CH) {
      float pb[2];
      float4 va[2][4];
      auto rd = [&](int j, int st) {
        pb[st] = pr[t0 + 16 * j + rl];
#pragma unroll
        for (int u = 0; u < 4; u++) va[st][u] = *reinterpret_cast<const float4*>(vcol + 16 * j + 4 * u);
      };
      rd(0, 0);
      rd(1, 1);
      if (carry) add_carry();
      float d[16];
      pv_row<16>::mul(pb[0], va[0], d);
#pragma unroll
      for (int j = 0; j + 1 < CH / 16; j++) {
        if (j + 2 < CH / 16) rd(j + 2, j & 1);
        float n[16];
        pv_row<16>::step(acc, d, pb[(j + 1) & 1], va[(j + 1) & 1], n);
#pragma unroll
        for (int k = 0; k < 16; k++) d[k] = n[k];
      }
#pragma unroll
      for (int k = 0; k < 16; k++) pc[k] = d[k];
      carry = true;
    } else {
      if (carry) add_carry();
      for (int r = 0; r < m; r++) acc = acc + pr[t0 + r] * vcol[r];
    }
  };
  // chunk ch sits in buffer ch & 1; after the barrier that opens chunk ch, chunk ch + 1 goes into
  // the other buffer (its last reader, chunk ch - 1, is done) and its register set loads chunk
  // ch + 1 + NS
  store(0, vset[0]);
  load(NS, vset[0]);
  for (int c = 0; c < nch; c += NS) {
#pragma unroll
    for (int k = 0; k < NS; k++) {
      if (c + k < nch) {
        lds_barrier();
        if (c + k + 1 < nch) {
          store((k + 1) & 1, vset[(k + 1) % NS]);
          load(c + k + 1 + NS, vset[(k + 1) % NS]);
        }
        chunk(c + k);
      }
    }
  }
  if (active && carry) add_carry();
  if (active) att[(size_t)b * D + (g * G + wave) * HD + lane] = acc;
  if (xq) {
    // each head's 64 outputs as two quantize_row blocks
    lds_barrier();
    float* o = vs;                                         // [head][64]
    if (active) o[wave * HD + lane] = acc;
    lds_barrier();
    if (tid < 8 * G) {
      const int hh = tid >> 3, blk = (tid >> 2) & 1, j = tid & 3;
      const int base = hh * HD + 32 * blk + 2 * j;
      const float v[8] = {o[base], o[base + 1], o[base + 8], o[base + 9],
                          o[base + 16], o[base + 17], o[base + 24], o[base + 25]};
      const int bi = (((g * G + hh) * HD) >> 5) + blk;
      quantize_item(v, bi, j, xq + (size_t)b * xstride * 4, xh ? xh + xh_tile(b, xstride) : nullptr, b & 15);
    }
  }
}

// Raise k_attn_rows' shared-memory limit to the whole 160 KB once per device, with that device
// current (before any graph capture; attn_list_ok calls it).
constexpr int kAttnRowsMaxLds = 160 * 1024;
bool attn_rows_setup(int device) {
  static std::mutex mu;
  static uint64_t done = 0, ok = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (device < 0 || device >= 64) return false;
  if (!((done >> device) & 1)) {
    const bool a = hipFuncSetAttribute((const void*)k_attn_rows<float>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kAttnRowsMaxLds) == hipSuccess;
    const bool b = hipFuncSetAttribute((const void*)k_attn_rows<kvhalf>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kAttnRowsMaxLds) == hipSuccess;
    (void)hipGetLastError();
    done |= (uint64_t)1 << device;
    if (a && b) ok |= (uint64_t)1 << device;
  }
  return (ok >> device) & 1;
}

template <int MODE>
void launch_quant(hipStream_t s, int rows, const float* in, int ld_in, int n, const float* w, float eps,
                  uint4* xq, int xstride, int m_first, uint4* xh = nullptr) {
  const size_t lds = MODE == QM_NORM ? (size_t)(sq_stride(n) + (n >> 2) + 1) * 4 * sizeof(float) : 0;
  k_quant<MODE><<<xh && rows >= 128 ? 8 * ((rows + 7) / 8) : rows, 256, lds, s>>>(in, ld_in, n, w, eps, xq, xstride, m_first, xh, rows);
}

// V rows per chunk of k_attn_pv_list: 128 (34 KB of LDS for the two chunk buffers) halves the
// chunk steps of 64 rows; 256 was slower again.
constexpr int kPvRows = 128;

size_t attn_pv_lds(int H, int KVH, int ctx) {
  const int G = H / KVH;
  return (size_t)(2 * kPvCols * (kPvRows + 4) + G * pv_row_stride(ctx) + 6 * kMaxGroup) * sizeof(float);
}

// With xq, the P.V kernel also writes the quantized activation of att (k_quant<QM_PLAIN>'s output).
template <class KT>
void launch_attn_list_t(hipStream_t s, int HD, int B, int H, int KVH, const float* qkv, int QKV, const KT* kc,
                        const KT* vc, int ctx, int layer, float* sc, float* att, int D, const int* pos,
                        size_t seq_stride, uint4* xq, int xstride, uint4* xh) {
  const dim3 sg((unsigned)((ctx + kScoreRows - 1) / kScoreRows), (unsigned)KVH, (unsigned)B);
  const unsigned units = (unsigned)KVH * (unsigned)B, pg = units * (unsigned)(HD / kPvCols);
  const bool xcd_group = units % kXcds == 0;
  const size_t lds = attn_pv_lds(H, KVH, ctx);
  const int Gq = H / KVH;
  int dev = 0;
  if (seq_stride == 0 && B > 1 && !pv_tiles_off() && !attn_rows_off() && HD == 64 && Gq <= kMaxGroup &&
      attn_rows_lds(Gq, ctx) <= (size_t)kAttnRowsMaxLds &&
      (attn_rows_lds(Gq, ctx) <= 64 * 1024 || (hipGetDevice(&dev) == hipSuccess && attn_rows_setup(dev)))) {
    // a prompt pass in one launch: scores and probabilities stay in shared memory
    k_attn_rows<KT><<<dim3((unsigned)KVH, (unsigned)B), kAttnRowsThreads, attn_rows_lds(Gq, ctx), s>>>(
        qkv, QKV, H, KVH, kc, vc, ctx, layer, pos, B, att, D, xq, xstride, xh);
    return;
  }
  if (seq_stride == 0 && B > 1 && !pv_tiles_off()) {   // a prompt pass: rows share one cache
    const dim3 tg((unsigned)(HD / kPvCols), (unsigned)KVH, (unsigned)((B + kPvTileRows - 1) / kPvTileRows));
    const int G = H / KVH;
    const unsigned nthr = (unsigned)(kPvTileRows * G * kPvCols);
    // V float4 per thread and chunk: 512 over 128 G threads
    auto tiles = [&](auto hd, auto nvt) {
      k_pv_tiles<decltype(hd)::value, KT, decltype(nvt)::value><<<tg, nthr, 0, s>>>(sc, H, KVH, vc, ctx, layer, att, D,
                                                                                    pos, B, xq, xstride, xh);
    };
    if (HD == 64) k_attn_scores_list<64, KT><<<sg, 64, 0, s>>>(qkv, QKV, H, KVH, kc, ctx, layer, sc, pos, 0);
    else k_attn_scores_list<128, KT><<<sg, 64, 0, s>>>(qkv, QKV, H, KVH, kc, ctx, layer, sc, pos, 0);
    k_softmax_rows<<<dim3((unsigned)KVH, (unsigned)B), 256, softmax_lds(H, KVH, ctx), s>>>(sc, H, KVH, ctx, pos);
    using I64 = std::integral_constant<int, 64>;
    using I128 = std::integral_constant<int, 128>;
    using N1 = std::integral_constant<int, 1>;
    using N2 = std::integral_constant<int, 2>;
    using N4 = std::integral_constant<int, 4>;
    if (HD == 64) {
      if (G >= 4) tiles(I64(), N1()); else if (G >= 2) tiles(I64(), N2()); else tiles(I64(), N4());
    } else {
      if (G >= 4) tiles(I128(), N1()); else if (G >= 2) tiles(I128(), N2()); else tiles(I128(), N4());
    }
    return;
  }
  if (HD == 64) {
    k_attn_scores_list<64, KT><<<sg, 64, 0, s>>>(qkv, QKV, H, KVH, kc, ctx, layer, sc, pos, seq_stride);
    k_attn_pv_list<64, kPvRows, KT><<<pg, 256, lds, s>>>(sc, H, KVH, vc, ctx, layer, att, D, pos, seq_stride, xq, xstride, xh,
                                                         xcd_group);
  } else {
    k_attn_scores_list<128, KT><<<sg, 64, 0, s>>>(qkv, QKV, H, KVH, kc, ctx, layer, sc, pos, seq_stride);
    k_attn_pv_list<128, kPvRows, KT><<<pg, 256, lds, s>>>(sc, H, KVH, vc, ctx, layer, att, D, pos, seq_stride, xq, xstride, xh,
                                                          xcd_group);
  }
}

// kc, vc: fp32 caches, or fp16 ones when kv16.
void launch_attn_list(hipStream_t s, int HD, int B, int H, int KVH, const float* qkv, int QKV, const void* kc,
                      const void* vc, bool kv16, int ctx, int layer, float* sc, float* att, int D, const int* pos,
                      size_t seq_stride, uint4* xq = nullptr, int xstride = 0, uint4* xh = nullptr) {
  if (kv16)
    launch_attn_list_t<kvhalf>(s, HD, B, H, KVH, qkv, QKV, (const kvhalf*)kc, (const kvhalf*)vc, ctx, layer, sc, att,
                               D, pos, seq_stride, xq, xstride, xh);
  else
    launch_attn_list_t<float>(s, HD, B, H, KVH, qkv, QKV, (const float*)kc, (const float*)vc, ctx, layer, sc, att, D,
                              pos, seq_stride, xq, xstride, xh);
}

// Whether the list attention kernels take this shape (query heads per kv head, LDS), and their LDS
// limit raised where needed.  Checked once per shape.
bool attn_list_ok(int H, int KVH, int HD, int ctx) {
  if (H / KVH > kMaxGroup) return false;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) (void)attn_rows_setup(dev);
  const size_t lds = attn_pv_lds(H, KVH, ctx), slds = softmax_lds(H, KVH, ctx);
  if (lds > 160 * 1024) return false;
  if (slds > 64 * 1024 &&
      hipFuncSetAttribute((const void*)k_softmax_rows, hipFuncAttributeMaxDynamicSharedMemorySize, (int)slds) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (lds > 64 * 1024) {
    const void* fns[2] = {HD == 64 ? (const void*)k_attn_pv_list<64, kPvRows, float> : (const void*)k_attn_pv_list<128, kPvRows, float>,
                          HD == 64 ? (const void*)k_attn_pv_list<64, kPvRows, kvhalf> : (const void*)k_attn_pv_list<128, kPvRows, kvhalf>};
    for (const void* fn : fns)
      if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return false;
      }
  }
  return true;
}

// One pass over M <= MT tokens at device position st->pos0 (forward_pass, kernels.c:306-415).
void enqueue_pass(q4hip* h, int M, bool want_logits) {
  const int D = h->D, F = h->F, HD = h->HD, QKV = h->QKV;
  hipStream_t s = h->stream;
  uint4* xh = M > 8 ? h->xh : nullptr;
  prof_mark(h, Q4HIP_PROF_EMBED);
  k_embed<<<M, 256, 0, s>>>(h->embd, D, h->tokens, h->st, h->x);
  if (M > 1 && h->list_attn == 1) k_pass_pos<<<(M + 255) / 256, 256, 0, s>>>(h->st, M, h->tpos);
  const size_t attn_lds = (size_t)(HD + h->ctx) * sizeof(float);
  for (int l = 0; l < h->NL; l++) {
    Layer& y = h->L[l];
    prof_mark(h, Q4HIP_PROF_NORM_Q);
    launch_quant<QM_NORM>(s, M, h->x, D, D, y.attn_norm, h->eps, h->xq, h->xstride, 0, xh);
    prof_mark(h, Q4HIP_PROF_QKV);
    launch_matvec<OP_BIAS>(s, y.qkv, h->xq, h->xstride, M, h->qkv, QKV, y.bqkv, xh);
    prof_mark(h, Q4HIP_PROF_ROPE);
    if (h->kv16)
      k_rope_kv<kvhalf><<<dim3(h->H + h->KVH, M), HD / 2, 0, s>>>(h->qkv, QKV, D, h->H, h->KVH, HD, h->rope, (kvhalf*)h->kc,
                                                                  (kvhalf*)h->vc, h->ctx, l, h->st);
    else
      k_rope_kv<float><<<dim3(h->H + h->KVH, M), HD / 2, 0, s>>>(h->qkv, QKV, D, h->H, h->KVH, HD, h->rope, (float*)h->kc,
                                                                 (float*)h->vc, h->ctx, l, h->st);
    prof_mark(h, Q4HIP_PROF_ATTN);
    bool quantized = false;                 // the list P.V kernel wrote xq (and xh) itself
    if (M > 1 && h->ascr && h->list_attn == 1) {
      launch_attn_list(s, HD, M, h->H, h->KVH, h->qkv, QKV, h->kc, h->vc, h->kv16, h->ctx, l, h->ascr, h->att, D, h->tpos, 0,
                       h->xq, h->xstride, xh);
      quantized = true;
    } else if (M > 1 && h->ascr) {
      const dim3 ag(h->H, (M + kAttnTokens - 1) / kAttnTokens);
      if (HD == 64 && h->kv16)
        k_attn_prefill<64, kvhalf><<<ag, 256, 0, s>>>(h->qkv, QKV, h->H, h->KVH, (const kvhalf*)h->kc, (const kvhalf*)h->vc, h->ctx, l,
                                                      h->att, D, h->st, M, h->ascr);
      else if (HD == 64)
        k_attn_prefill<64, float><<<ag, 256, 0, s>>>(h->qkv, QKV, h->H, h->KVH, (const float*)h->kc, (const float*)h->vc, h->ctx, l,
                                                     h->att, D, h->st, M, h->ascr);
      else if (h->kv16)
        k_attn_prefill<128, kvhalf><<<ag, 256, 0, s>>>(h->qkv, QKV, h->H, h->KVH, (const kvhalf*)h->kc, (const kvhalf*)h->vc, h->ctx,
                                                       l, h->att, D, h->st, M, h->ascr);
      else
        k_attn_prefill<128, float><<<ag, 256, 0, s>>>(h->qkv, QKV, h->H, h->KVH, (const float*)h->kc, (const float*)h->vc, h->ctx, l,
                                                      h->att, D, h->st, M, h->ascr);
    } else if (M == 1 && h->ascr && h->list_attn == 1) {
      launch_attn_list(s, HD, 1, h->H, h->KVH, h->qkv, QKV, h->kc, h->vc, h->kv16, h->ctx, l, h->ascr, h->att, D, &h->st->pos0, 0,
                       h->xq, h->xstride, xh);
      quantized = true;
    } else if (HD == 64 && h->kv16) {
      k_attn<64, kvhalf><<<dim3(h->H, M), 64, attn_lds, s>>>(h->qkv, QKV, D, h->H, h->KVH, (const kvhalf*)h->kc,
                                                             (const kvhalf*)h->vc, h->ctx, l, h->att, h->st);
    } else if (HD == 64) {
      k_attn<64, float><<<dim3(h->H, M), 64, attn_lds, s>>>(h->qkv, QKV, D, h->H, h->KVH, (const float*)h->kc,
                                                            (const float*)h->vc, h->ctx, l, h->att, h->st);
    } else if (h->kv16) {
      k_attn<128, kvhalf><<<dim3(h->H, M), 64, attn_lds, s>>>(h->qkv, QKV, D, h->H, h->KVH, (const kvhalf*)h->kc,
                                                              (const kvhalf*)h->vc, h->ctx, l, h->att, h->st);
    } else {
      k_attn<128, float><<<dim3(h->H, M), 64, attn_lds, s>>>(h->qkv, QKV, D, h->H, h->KVH, (const float*)h->kc,
                                                             (const float*)h->vc, h->ctx, l, h->att, h->st);
    }
    prof_mark(h, Q4HIP_PROF_QUANT);
    if (!quantized) launch_quant<QM_PLAIN>(s, M, h->att, D, D, nullptr, 0.0f, h->xq, h->xstride, 0, xh);
    prof_mark(h, Q4HIP_PROF_O);
    launch_matvec<OP_ADD>(s, y.o, h->xq, h->xstride, M, h->x, D, nullptr, xh);
    prof_mark(h, Q4HIP_PROF_NORM_Q);
    launch_quant<QM_NORM>(s, M, h->x, D, D, y.ffn_norm, h->eps, h->xq, h->xstride, 0, xh);
    prof_mark(h, Q4HIP_PROF_GU);
    uint4* xh_act = xh;      // where the down projection finds the activation's fp16 operands
    if (launch_gu_swiglu(s, y.gu, xh, h->xstride, M, h->xq, h->xh2, F)) {
      xh_act = h->xh2;
    } else {
      launch_matvec<OP_STORE>(s, y.gu, h->xq, h->xstride, M, h->gu, 2 * F, nullptr, xh);
      prof_mark(h, Q4HIP_PROF_SWIGLU);
      launch_quant<QM_SWIGLU>(s, M, h->gu, 2 * F, F, nullptr, 0.0f, h->xq, h->xstride, 0, xh);
    }
    prof_mark(h, Q4HIP_PROF_DOWN);
    launch_matvec<OP_ADD>(s, y.down, h->xq, h->xstride, M, h->x, D, nullptr, xh_act);
  }
  if (want_logits) {
    prof_mark(h, Q4HIP_PROF_NORM_Q);
    launch_quant<QM_NORM>(s, 1, h->x, D, D, h->out_norm, h->eps, h->xq, h->xstride, M - 1);
    prof_mark(h, Q4HIP_PROF_OUT);
    launch_head(s, h->head, h->xq, h->logits);
    prof_mark(h, Q4HIP_PROF_SAMPLE);
    k_argmax1<<<h->am_parts, 256, 0, s>>>(h->logits, h->V, h->am_v, h->am_i);
    k_argmax2<<<1, 256, 0, s>>>(h->am_v, h->am_i, h->am_parts, h->tokens, h->st, M);
  }
  prof_mark(h, -1);
}

// The model shapes the persistent decode kernel is compiled for: Qwen2.5-0.5B and the two small
// shapes of the parity tests.  Any other shape decodes through the graph path.
struct PersInstance {
  int D, F, H, KVH;
  const void* fn;       // fp32 cache
  const void* fn16;     // fp16 cache
  size_t lds_base;
  size_t (*attn_bytes)(int ctx, int ring_slots, int kv_tile);
  size_t (*ll_entries)(int);
  int nRoles, nbm;
  size_t head_cache_off, head_rg_bytes;
};

template <class S>
PersInstance pers_instance() {
  return PersInstance{S::D, S::F, S::H, S::KVH, (const void*)k_decode_persistent<S, float>,
                      (const void*)k_decode_persistent<S, kvhalf>, psmem_base_bytes<S>(), &psmem_attn_bytes<S>,
                      &S::ll_entries, S::nRoles, S::NBM, head_cache_offset<S>(), head_rg_bytes<S>()};
}

const PersInstance* find_pers_instance(int D, int F, int H, int KVH) {
  static const PersInstance table[] = {
      pers_instance<PShape<896, 4864, 14, 2>>(),   // Qwen2.5-0.5B
      pers_instance<PShape<128, 256, 2, 1>>(),
      pers_instance<PShape<256, 512, 4, 1>>(),
  };
  for (const PersInstance& p : table)
    if (p.D == D && p.F == F && p.H == H && p.KVH == KVH) return &p;
  return nullptr;
}

// Placement of the persistent kernel's workgroups: physical workgroup p runs on XCD p mod 8, and
// the logical index (the role order: o/down, attention, K/V, gate/up, head only) comes from this
// map.  The attention workgroups of kv group g take physical slots on XCD g mod 8, so the past K/V
// rows they all stage each layer come from one L2; every other role keeps its order in the
// remaining slots.  Empty when the slots do not suffice (identity placement).
std::vector<int> persistent_wgmap(int G, int nOD, int H, int KVH, int asplit) {
  std::vector<int> map(G, -1);
  std::vector<char> used(G, 0);
  const int grp = H / KVH, nA = H * asplit;
  for (int aidx = 0; aidx < nA; aidx++) {
    int p = (aidx % H) / grp % 8;
    while (p < G && used[p]) p += 8;
    if (p >= G) return {};
    used[p] = 1;
    map[p] = nOD + aidx;
  }
  int p = 0;
  for (int lid = 0; lid < G; lid++) {
    if (lid >= nOD && lid < nOD + nA) continue;
    while (p < G && used[p]) p++;
    if (p >= G) return {};
    used[p] = 1;
    map[p] = lid;
  }
  return map;
}

// Decide once whether this model and device admit the persistent decode kernel, and set it up.
// On refusal h->pers_why says which requirement failed.
void setup_persistent(q4hip* h) {
  if (h->pers_ok || h->pers_broken || h->mode == Q4HIP_DECODE_GRAPH) return;
  h->pers_broken = true;   // until proven otherwise
  auto no = [h](const char* why) { h->pers_why = why; };
  if (h->HD != kHD) return no("head_dim is not 64");
  const PersInstance* pi = find_pers_instance(h->D, h->F, h->H, h->KVH);
  if (!pi) return no("no kernel instance for this model shape");
  h->pers_fn = h->kv16 ? pi->fn16 : pi->fn;
  int lds_max = 0;
  if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, h->device) != hipSuccess)
    return no("cannot query shared memory size");
  const size_t base = pi->lds_base, budget = (size_t)lds_max > 4096 ? (size_t)lds_max - 4096 : 0;
  if (base > budget) return no("shared memory too small");
  // past K/V rows the attention role stages in shared memory; the rest are streamed
  // past K/V rows: staged whole in shared memory when the context fits (no ring), else the first
  // kv_tile positions staged and the rest streamed through a ring of 3 (ctx <= 1024) or 7 slots
  int cap = 192;
  if (const char* e = getenv("Q4HIP_KV_TILE")) cap = std::max(0, std::min(cap, atoi(e)));
  int kv_tile = std::min(h->ctx, cap), ring = 0;
  auto need = [&](int r, int t) { return std::max(base, pi->attn_bytes(h->ctx, r, t)); };
  while (kv_tile > 0 && need(0, kv_tile) > budget) kv_tile--;
  if (kv_tile < h->ctx) {
    ring = h->ctx <= 1024 ? 3 : 7;
    if (need(ring, 0) > budget) ring = 3;
    if (need(ring, 0) > budget) return no("shared memory too small for the K/V ring");
    while (kv_tile > 0 && need(ring, kv_tile) > budget) kv_tile--;
  }
  h->pers_kv_tile = kv_tile;
  h->pers_ring = ring;
  h->pers_lds = need(ring, kv_tile);
  if (hipFuncSetAttribute(h->pers_fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)h->pers_lds) != hipSuccess) {
    (void)hipGetLastError();
    return no("cannot raise the kernel's shared memory limit");
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, h->device) != hipSuccess)
    return no("cannot query CU count");
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, h->pers_fn, kPThreads, h->pers_lds) != hipSuccess || per_cu < 1) {
    (void)hipGetLastError();
    return no("the kernel does not fit on a CU");
  }
  // One workgroup per CU: all of them fit on the device at once, which the waits between them
  // rely on (a workgroup that could not start would only make the others time out and abort).
  const int G = cus;
  if (pi->nRoles > G || G > 256) return no("more roles than CUs");   // the argmax exchange gives one entry per thread
  std::vector<LayerView> lv(h->NL);
  for (int l = 0; l < h->NL; l++) {
    const Layer& y = h->L[l];
    lv[l] = LayerView{y.qkv.view(), y.o.view(), y.gu.view(), y.down.view(), y.attn_norm, y.ffn_norm, y.bqkv};
  }
  const size_t ll_entries = pi->ll_entries(G);
  if (hipMalloc(&h->d_layers, lv.size() * sizeof(LayerView)) != hipSuccess ||
      hipMemcpy(h->d_layers, lv.data(), lv.size() * sizeof(LayerView), hipMemcpyHostToDevice) != hipSuccess ||
      hipMalloc(&h->ll, ll_entries * 8) != hipSuccess || hipMemsetAsync(h->ll, 0, ll_entries * 8, h->stream) != hipSuccess) {
    (void)hipGetLastError();
    return no("device allocation failed");
  }
  h->pers_grid = G;
  h->pers_hc_off = pi->head_cache_off;
  h->pers_hc_rg = pi->head_rg_bytes;
  if (const char* e = getenv("Q4HIP_HEAD_CACHE")) h->pers_head_cache = atoi(e) != 0;
  for (int sp = 1; sp <= 2; sp++) {
    const std::vector<int> map = persistent_wgmap(G, h->D / 16, h->H, h->KVH, sp);
    if (map.empty()) continue;
    if (hipMalloc(&h->pers_wgmap[sp - 1], (size_t)G * sizeof(int)) != hipSuccess ||
        hipMemcpy(h->pers_wgmap[sp - 1], map.data(), (size_t)G * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) {
      (void)hipGetLastError();
      if (h->pers_wgmap[sp - 1]) (void)hipFree(h->pers_wgmap[sp - 1]);
      h->pers_wgmap[sp - 1] = nullptr;       // identity placement
    }
  }
  if (const char* e = getenv("Q4HIP_POLL_SLEEP")) h->pers_nap = std::max(0, std::min(64, atoi(e)));
  // long contexts: two attention workgroups per head when the roles still fit one per CU
  if (pi->nRoles + h->H <= G && h->pers_ring > 0) {
    const size_t lbytes = (size_t)h->H * h->ctx * 8;
    if (hipMalloc(&h->lsc, lbytes) == hipSuccess && hipMemsetAsync(h->lsc, 0, lbytes, h->stream) == hipSuccess) {
      h->pers_split_ok = true;
    } else {
      (void)hipGetLastError();
      if (h->lsc) (void)hipFree(h->lsc);
      h->lsc = nullptr;
    }
  }
  if (const char* e = getenv("Q4HIP_SPLIT_FROM")) h->pers_split_from = std::max(0, atoi(e));
  if (const char* e = getenv("Q4HIP_TEST_ABORT")) h->pers_test_abort = std::max(0, atoi(e));
  if (const char* e = getenv("Q4HIP_PF")) {   // "o,down,attn,gu" in units of 512 cycles (tuning)
    int v[4] = {0, 0, 0, 0};
    if (sscanf(e, "%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3]) == 4)
      for (int i = 0; i < 4; i++) h->pers_pf[i] = std::max(0, std::min(64, v[i]));
  }

  h->pers_ok = true;
  h->pers_broken = false;
}

bool use_persistent(q4hip* h) {
  if (h->mode == Q4HIP_DECODE_GRAPH) return false;
  setup_persistent(h);
  return h->pers_ok && !h->pers_broken;
}

// Attention of the multi-kernel path: the list kernels (scores over 64-position workgroups, softmax
// and P.V per 32-column slice) when the shape admits them, with the [MT][H][ctx] score buffer.
void prepare_attention(q4hip* h) {
  if (h->list_attn < 0) h->list_attn = attn_list_ok(h->H, h->KVH, h->HD, h->ctx) ? 1 : 0;
  if (!h->ascr && (h->list_attn == 1 || h->MT > 1)) {
    if (hipMalloc(&h->ascr, (size_t)h->MT * h->H * score_stride(h->ctx) * sizeof(float)) != hipSuccess) {
      h->ascr = nullptr;
      (void)hipGetLastError();
    }
  }
}

// In AUTO mode, when the persistent kernel cannot split attention over two workgroups per head (too
// few CUs), decode steps whose context reaches this many positions run on the multi-kernel path: its
// attention spreads the scores over many workgroups and reads each kv head's K once, where the
// persistent kernel streams a kv head's K and V through one workgroup per query head.
constexpr int kLongDecodePositions = 3072;

bool long_decode(const q4hip* h, int64_t last_pos) {
  return h->mode == Q4HIP_DECODE_AUTO && !h->pers_split_ok && h->list_attn == 1 && h->ascr &&
         last_pos >= kLongDecodePositions;
}

hipError_t launch_persistent(q4hip* h, int pos0, int steps, unsigned long long* prof = nullptr) {
  PArgs a;
  a.asplit = h->pers_split_ok && pos0 >= h->pers_split_from ? 2 : 1;
  a.lsc = h->lsc;
  a.V = h->V; a.NL = h->NL; a.ctx = h->ctx;
  a.eps = h->eps;
  a.embd = h->embd;
  a.out_norm = h->out_norm;
  a.head = h->head.view();
  a.head_q8 = h->head.fmt == Q4HIP_TYPE_Q8_0;
  a.layers = h->d_layers;
  a.rope = h->rope;
  a.kc = h->kc;
  a.vc = h->vc;
  a.logits = h->logits;
  a.tokens = h->tokens;
  a.st = h->st;
  a.ll = h->ll;
  a.steps = steps;
  a.kv_tile = h->pers_kv_tile;
  a.ring = h->pers_ring;
  a.nap = h->pers_nap;
  a.prof = prof;
  a.wgmap = h->pers_wgmap[a.asplit - 1];
  for (int i = 0; i < 4; i++) a.pf[i] = h->pers_pf[i];
  // Q4_0 head row groups per wave kept in the shared memory the roles outside attention leave
  // free (fp32-cache kernel): as many as fit, while the resident ones stay within the head
  a.hres = 0;
  if (!a.head_q8 && !h->kv16 && h->pers_head_cache && h->pers_lds > h->pers_hc_off) {
    const int ranks = h->pers_grid - h->H * a.asplit, nrg = a.head.Np / 16;
    int n = (int)std::min<size_t>(8, (h->pers_lds - h->pers_hc_off) / (4 * h->pers_hc_rg));
    while (n > 0 && (long)ranks * 4 * n > nrg) n--;
    a.hres = n;
  }
  h->pers_last_steps = steps;
  if (h->pers_test_abort > 0) {          // Q4HIP_TEST_ABORT: the launch finds the flag raised
    h->pers_test_abort--;
    k_raise_abort<<<1, 64, 0, h->stream>>>(h->st);
  }
  void* args[] = {&a};
  return hipLaunchKernel(h->pers_fn, dim3(h->pers_grid), dim3(kPThreads), args, h->pers_lds, h->stream);
}

// After a synchronised persistent launch: a raised abort flag means a bounded wait ran out (for
// example because another process held CUs so not every workgroup could start).  Clears the flag,
// switches this context to the graph path and returns true: the caller reruns the call, which
// overwrites everything the aborted launch wrote (K/V from pos on, tokens after pos).
// An aborted launch returns before it advances the epoch, and some of its roles have already
// posted exchange entries tagged with epochs of that launch (the KV role posts layer 0's rows
// without waiting for anything).  The epoch is moved past every epoch the launch could use, so a
// later persistent launch (after q4hip_set_decode_mode re-enables the path) never takes those
// entries for its own.
bool aborted(q4hip* h) {
  State hs;
  if (hipMemcpy(&hs, h->st, sizeof(State), hipMemcpyDeviceToHost) != hipSuccess) return false;
  if (!hs.abort) return false;
  h->pers_broken = true;
  hs.abort = 0;
  hs.epoch += (uint32_t)h->pers_last_steps * (uint32_t)(4 * h->NL + 1) + 2u;
  (void)hipMemcpy(h->st, &hs, sizeof(State), hipMemcpyHostToDevice);
  return true;
}

int build_graph(q4hip* h) {
  if (h->graph || h->graph_failed) return Q4HIP_OK;
  const char* env = getenv("Q4HIP_GRAPH");
  if (env && env[0] == '0') {   // eager launches, e.g. under a tracer that cannot follow graphs
    h->graph_failed = true;
    return Q4HIP_OK;
  }
  hipGraph_t g = nullptr;
  if (hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    h->graph_failed = true;
    (void)hipGetLastError();
    return Q4HIP_OK;
  }
  enqueue_pass(h, 1, true);
  hipError_t e = hipStreamEndCapture(h->stream, &g);
  if (e == hipSuccess) e = hipGraphInstantiate(&h->graph, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    h->graph = nullptr;
    h->graph_failed = true;
    (void)hipGetLastError();
  }
  return Q4HIP_OK;
}

void decode_step(q4hip* h) {
  if (h->graph) (void)hipGraphLaunch(h->graph, h->stream);
  else enqueue_pass(h, 1, true);
}

}  // namespace

// ================================================================ C ABI

extern "C" {

const char* q4hip_last_error(void) { return g_err.c_str(); }

int q4hip_device_count(int* count) {
  if (!count) return fail(Q4HIP_EINVAL, "null argument");
  HIPCHK(hipGetDeviceCount(count));
  return Q4HIP_OK;
}

void q4hip_destroy(q4hip* h) {
  if (!h) return;
  (void)hipSetDevice(h->device);
  if (h->stream) (void)hipStreamSynchronize(h->stream);
  if (h->graph) (void)hipGraphExecDestroy(h->graph);
  for (Layer& y : h->L) {
    mat_free(y.qkv); mat_free(y.o); mat_free(y.gu); mat_free(y.down);
    if (y.attn_norm) (void)hipFree(y.attn_norm);
    if (y.ffn_norm) (void)hipFree(y.ffn_norm);
    if (y.bqkv) (void)hipFree(y.bqkv);
  }
  mat_free(h->head);
  void* bufs[] = {h->embd, h->out_norm, h->rope, h->x, h->qkv, h->att, h->gu, h->logits, h->kc, h->vc,
                  h->xq, h->am_v, h->am_i, h->tokens, h->st, h->d_layers, h->ll, h->ascr, h->xh, h->xh2, h->tpos,
                  h->lsc, h->pers_wgmap[0], h->pers_wgmap[1]};
  for (void* p : bufs) if (p) (void)hipFree(p);
  if (h->pin_ids) (void)hipHostFree(h->pin_ids);
  if (h->pin_next) (void)hipHostFree(h->pin_next);
  if (h->stream) (void)hipStreamDestroy(h->stream);
  delete h;
}

int q4hip_create(q4hip** out, int dim, int layers, int ffn, int heads, int kv_heads, int vocab, int ctx,
                 int mt, float eps, int device, int kv_type) {
  if (!out) return fail(Q4HIP_EINVAL, "null argument");
  *out = nullptr;
  if (kv_type != Q4HIP_KV_F32 && kv_type != Q4HIP_KV_F16) return fail(Q4HIP_EINVAL, "unknown K/V cache type %d", kv_type);
  if (dim <= 0 || layers <= 0 || ffn <= 0 || heads <= 0 || kv_heads <= 0 || vocab <= 0 || ctx <= 1)
    return fail(Q4HIP_EINVAL, "bad configuration");
  if (dim % 32 || ffn % 32 || dim % heads || heads % kv_heads)
    return fail(Q4HIP_EINVAL, "dim and ffn must be multiples of 32, heads a multiple of kv_heads");
  const int HD = dim / heads;
  if (HD != 64 && HD != 128) return fail(Q4HIP_EINVAL, "head_dim %d unsupported (64 or 128)", HD);
  if ((size_t)(HD + ctx) * 4 > 65536) return fail(Q4HIP_EINVAL, "ctx %d too large for the attention kernel", ctx);
  if (mt <= 0 || mt > kMaxPass) mt = kMaxPass;
  mt = std::min(mt, ctx);
  int ndev = 0;
  HIPCHK(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return fail(Q4HIP_EINVAL, "device %d of %d", device, ndev);
  HIPCHK(hipSetDevice(device));
  matvec_split_setup(device);

  q4hip* h = new q4hip();
  h->D = dim; h->NL = layers; h->F = ffn; h->H = heads; h->KVH = kv_heads; h->HD = HD;
  h->QKV = dim + 2 * kv_heads * HD; h->V = vocab; h->ctx = ctx; h->MT = mt; h->device = device; h->eps = eps;
  h->kv16 = kv_type == Q4HIP_KV_F16;
  h->kvb = h->kv16 ? 2 : 4;
  int rc = Q4HIP_OK;
#define TRY(x) do { rc = (x); if (rc != Q4HIP_OK) { q4hip_destroy(h); return rc; } } while (0)
#define TRYHIP(call) do { hipError_t e_ = (call); if (e_ != hipSuccess) { rc = fail(Q4HIP_EHIP, "%s: %s", #call, hipGetErrorString(e_)); q4hip_destroy(h); return rc; } } while (0)
  TRYHIP(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
  h->L.resize(layers);
  for (int l = 0; l < layers; l++) {
    Layer& y = h->L[l];
    TRY(mat_alloc(y.qkv, h->QKV, dim, h->stream));
    TRY(mat_alloc(y.o, dim, dim, h->stream));
    TRY(mat_alloc(y.gu, 2 * ffn, dim, h->stream));
    TRY(mat_alloc(y.down, dim, ffn, h->stream));
    TRYHIP(hipMalloc(&y.attn_norm, (size_t)dim * 4));
    TRYHIP(hipMalloc(&y.ffn_norm, (size_t)dim * 4));
    TRYHIP(hipMalloc(&y.bqkv, (size_t)h->QKV * 4));
  }
  TRY(mat_alloc(h->head, vocab, dim, h->stream));
  TRYHIP(hipMalloc(&h->embd, (size_t)vocab * (dim / 32) * 18));
  TRYHIP(hipMalloc(&h->out_norm, (size_t)dim * 4));
  TRYHIP(hipMalloc(&h->rope, (size_t)ctx * HD * 4));
  const int M = mt;
  h->xstride = std::max(dim, ffn) / 32;
  TRYHIP(hipMalloc(&h->x, (size_t)M * dim * 4));
  TRYHIP(hipMalloc(&h->qkv, (size_t)M * h->QKV * 4));
  TRYHIP(hipMalloc(&h->att, (size_t)M * dim * 4));
  TRYHIP(hipMalloc(&h->gu, (size_t)M * 2 * ffn * 4));
  TRYHIP(hipMalloc(&h->logits, (size_t)vocab * 4));
  const size_t kvbytes = (size_t)layers * kv_heads * ctx * HD * h->kvb;
  TRYHIP(hipMalloc(&h->kc, kvbytes));
  TRYHIP(hipMalloc(&h->vc, kvbytes));
  TRYHIP(hipMemsetAsync(h->kc, 0, kvbytes, h->stream));
  TRYHIP(hipMemsetAsync(h->vc, 0, kvbytes, h->stream));
  TRYHIP(hipMalloc(&h->xq, (size_t)M * h->xstride * 64));
  TRYHIP(hipMalloc(&h->xh, xh_bytes(M, h->xstride)));
  TRYHIP(hipMemsetAsync(h->xh, 0, xh_bytes(M, h->xstride), h->stream));
  TRYHIP(hipMalloc(&h->xh2, xh_bytes(M, h->xstride)));
  TRYHIP(hipMemsetAsync(h->xh2, 0, xh_bytes(M, h->xstride), h->stream));
  TRYHIP(hipMalloc(&h->tpos, (size_t)M * sizeof(int)));
  h->am_parts = (vocab + 4095) / 4096;
  TRYHIP(hipMalloc(&h->am_v, (size_t)h->am_parts * 4));
  TRYHIP(hipMalloc(&h->am_i, (size_t)h->am_parts * 4));
  TRYHIP(hipMalloc(&h->tokens, (size_t)(ctx + 1) * 4));
  TRYHIP(hipMemsetAsync(h->tokens, 0, (size_t)(ctx + 1) * 4, h->stream));
  TRYHIP(hipMalloc(&h->st, sizeof(State)));
  TRYHIP(hipMemsetAsync(h->st, 0, sizeof(State), h->stream));
  TRYHIP(hipHostMalloc(&h->pin_ids, (size_t)(ctx + 1) * 4, hipHostMallocDefault));
  TRYHIP(hipHostMalloc(&h->pin_next, 64, hipHostMallocDefault));
  // the zeroing above is complete before any later call, whatever stream that call uses
  TRYHIP(hipStreamSynchronize(h->stream));
#undef TRY
#undef TRYHIP
  *out = h;
  return Q4HIP_OK;
}

int q4hip_set_tensor(q4hip* h, int kind, int layer, int row0, int type, const void* data, int64_t rows,
                     size_t nbytes) {
  if (!h || !data) return fail(Q4HIP_EINVAL, "null argument");
  if (rows <= 0) return fail(Q4HIP_EINVAL, "no rows");
  {
    // bytes per row of this kind and type
    const int64_t K = (kind == 3) ? h->F : h->D;
    int64_t per = 0;
    if (type == Q4HIP_TYPE_F32) per = 4;
    else if (type == Q4HIP_TYPE_Q4_0) per = K / 32 * 18;
    else if (type == Q4HIP_TYPE_Q8_0) per = K / 32 * 34;
    if (per > 0 && (uint64_t)rows * (uint64_t)per > (uint64_t)nbytes)
      return fail(Q4HIP_EINVAL, "kind %d: %zu bytes given, %lld rows need %lld", kind, nbytes, (long long)rows,
                  (long long)(rows * per));
  }
  HIPCHK(hipSetDevice(h->device));
  const bool per_layer = kind >= 0 && kind <= 6;
  if (per_layer && (layer < 0 || layer >= h->NL)) return fail(Q4HIP_EINVAL, "layer %d of %d", layer, h->NL);
  if (kind >= 0 && kind <= 3) {
    if (type != Q4HIP_TYPE_Q4_0) return fail(Q4HIP_ETYPE, "kind %d: expected Q4_0", kind);
    Layer& y = h->L[layer];
    Mat* m = kind == 0 ? &y.qkv : kind == 1 ? &y.o : kind == 2 ? &y.gu : &y.down;
    return mat_upload(*m, row0, rows, data, h->stream);
  }
  if (kind == 4 || kind == 5 || kind == 6 || kind == 9) {
    if (type != Q4HIP_TYPE_F32) return fail(Q4HIP_ETYPE, "kind %d: expected F32", kind);
    float* dst;
    int64_t cap, *cnt;
    if (kind == 4) { dst = h->L[layer].attn_norm; cap = h->D; cnt = &h->L[layer].n_attn_norm; }
    else if (kind == 5) { dst = h->L[layer].ffn_norm; cap = h->D; cnt = &h->L[layer].n_ffn_norm; }
    else if (kind == 6) { dst = h->L[layer].bqkv; cap = h->QKV; cnt = &h->L[layer].n_bqkv; }
    else { dst = h->out_norm; cap = h->D; cnt = &h->n_out_norm; }
    if (row0 < 0 || rows <= 0 || row0 + rows > cap) return fail(Q4HIP_EINVAL, "kind %d: values %d..%lld outside 0..%lld", kind, row0, (long long)(row0 + rows), (long long)cap);
    HIPCHK(hipMemcpy(dst + row0, data, (size_t)rows * 4, hipMemcpyHostToDevice));
    *cnt += rows;
    return Q4HIP_OK;
  }
  if (kind == 7) {
    if (type != Q4HIP_TYPE_Q4_0) return fail(Q4HIP_ETYPE, "kind 7: expected Q4_0");
    if (row0 < 0 || rows <= 0 || row0 + rows > h->V) return fail(Q4HIP_EINVAL, "embedding rows outside 0..%d", h->V);
    const size_t rb = (size_t)(h->D / 32) * 18;
    HIPCHK(hipMemcpy(h->embd + (size_t)row0 * rb, data, (size_t)rows * rb, hipMemcpyHostToDevice));
    h->embd_loaded += rows;
    return Q4HIP_OK;
  }
  if (kind == 8) {
    if (type != Q4HIP_TYPE_Q4_0 && type != Q4HIP_TYPE_Q8_0) return fail(Q4HIP_ETYPE, "kind 8: expected Q4_0 or Q8_0");
    if (type != h->head.fmt) {
      if (h->head.loaded > 0) return fail(Q4HIP_ETYPE, "kind 8: rows of Q4_0 and Q8_0 mixed");
      if (h->graph) {   // the captured pass holds the old head's addresses
        (void)hipGraphExecDestroy(h->graph);
        h->graph = nullptr;
      }
      mat_free(h->head);
      const int rc = mat_alloc(h->head, h->V, h->D, h->stream, type);
      if (rc != Q4HIP_OK) return rc;
    }
    return mat_upload(h->head, row0, rows, data, h->stream);
  }
  return fail(Q4HIP_EINVAL, "unknown tensor kind %d", kind);
}

int q4hip_set_rope(q4hip* h, const float* table, int64_t n_floats) {
  if (!h || !table) return fail(Q4HIP_EINVAL, "null argument");
  const int64_t need = (int64_t)h->ctx * h->HD;
  if (n_floats < need)
    return fail(Q4HIP_EINVAL, "RoPE table has %lld floats, ctx %d x head_dim %d needs %lld", (long long)n_floats,
                h->ctx, h->HD, (long long)need);
  HIPCHK(hipSetDevice(h->device));
  HIPCHK(hipMemcpy(h->rope, table, (size_t)h->ctx * h->HD * 4, hipMemcpyHostToDevice));
  h->rope_set = true;
  return Q4HIP_OK;
}

static int check_ids(q4hip* h, const int* ids, int n) {
  for (int i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= h->V) return fail(Q4HIP_EINVAL, "token id %d out of range 0..%d", ids[i], h->V - 1);
  return Q4HIP_OK;
}

int q4hip_forward(q4hip* h, const int* ids, int n, int pos, int* next) {
  if (!h || !ids || !next) return fail(Q4HIP_EINVAL, "null argument");
  if (n <= 0) return fail(Q4HIP_EINVAL, "no tokens");
  if (pos < 0 || (int64_t)pos + n >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full");
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, ids, n);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  prepare_attention(h);
  const bool pers = n == 1 && use_persistent(h) && !long_decode(h, pos);
  if (n == 1 && !pers) build_graph(h);
  memcpy(h->pin_ids, ids, (size_t)n * 4);
  HIPCHK(hipMemcpyAsync(h->tokens + pos, h->pin_ids, (size_t)n * 4, hipMemcpyHostToDevice, h->stream));
  for (int c = 0; c < n; c += h->MT) {
    const int k = std::min(h->MT, n - c);
    const bool last = c + k >= n;
    k_set_pos<<<1, 64, 0, h->stream>>>(h->st, pos + c);
    if (k == 1 && last && pers) {
      HIPCHK(launch_persistent(h, pos + c, 1));
      h->last_mode = Q4HIP_DECODE_PERSISTENT;
    } else if (k == 1 && last && h->graph) {
      HIPCHK(hipGraphLaunch(h->graph, h->stream));
      h->last_mode = Q4HIP_DECODE_GRAPH;
    } else {
      enqueue_pass(h, k, last);
      if (k == 1) h->last_mode = Q4HIP_DECODE_GRAPH;
    }
  }
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(h->pin_next, &h->st->next, 4, hipMemcpyDeviceToHost, h->stream));
  HIPCHK(hipStreamSynchronize(h->stream));
  if (pers && aborted(h)) return q4hip_forward(h, ids, n, pos, next);
  *next = h->pin_next[0];
  return Q4HIP_OK;
}

// Copy n fp32 values of K and of V from the host into the cache at dk, dv: as they are, or rounded to
// fp16 (nearest, ties to even: the conversion of the append kernels) for an fp16 cache.
static int upload_kv(q4hip* h, void* dk, void* dv, const float* k, const float* v, size_t n) {
  if (!h->kv16) {
    HIPCHK(hipMemcpy(dk, k, n * 4, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(dv, v, n * 4, hipMemcpyHostToDevice));
    return Q4HIP_OK;
  }
  std::vector<_Float16> t(n);
  for (size_t i = 0; i < n; i++) t[i] = (_Float16)k[i];
  HIPCHK(hipMemcpy(dk, t.data(), n * 2, hipMemcpyHostToDevice));
  for (size_t i = 0; i < n; i++) t[i] = (_Float16)v[i];
  HIPCHK(hipMemcpy(dv, t.data(), n * 2, hipMemcpyHostToDevice));
  return Q4HIP_OK;
}

int q4hip_set_kv(q4hip* h, int layer, int kv_head, int pos0, int n, const float* k, const float* v) {
  if (!h || !k || !v) return fail(Q4HIP_EINVAL, "null argument");
  if (layer < 0 || layer >= h->NL) return fail(Q4HIP_EINVAL, "layer %d of %d", layer, h->NL);
  if (kv_head < 0 || kv_head >= h->KVH) return fail(Q4HIP_EINVAL, "kv head %d of %d", kv_head, h->KVH);
  if (n <= 0 || pos0 < 0 || (int64_t)pos0 + n > h->ctx) return fail(Q4HIP_ECONTEXT, "positions %d..%lld outside 0..%d", pos0, (long long)pos0 + n, h->ctx);
  HIPCHK(hipSetDevice(h->device));
  HIPCHK(hipStreamSynchronize(h->stream));
  const size_t off = (((size_t)layer * h->KVH + kv_head) * h->ctx + pos0) * h->HD;
  return upload_kv(h, (char*)h->kc + off * h->kvb, (char*)h->vc + off * h->kvb, k, v, (size_t)n * h->HD);
}

int q4hip_set_decode_mode(q4hip* h, int mode) {
  if (!h) return fail(Q4HIP_EINVAL, "null argument");
  if (mode != Q4HIP_DECODE_AUTO && mode != Q4HIP_DECODE_GRAPH && mode != Q4HIP_DECODE_PERSISTENT)
    return fail(Q4HIP_EINVAL, "unknown decode mode %d", mode);
  HIPCHK(hipSetDevice(h->device));
  h->mode = mode;
  if (mode == Q4HIP_DECODE_PERSISTENT) {
    int rc = check_ready(h);
    if (rc) return rc;
    h->pers_broken = false;
    setup_persistent(h);
    if (!h->pers_ok || h->pers_broken) {
      h->mode = Q4HIP_DECODE_AUTO;
      return fail(Q4HIP_EINVAL, "the persistent decode kernel does not support this model or device: %s", h->pers_why);
    }
  }
  return Q4HIP_OK;
}

int q4hip_decode_mode_used(q4hip* h, int* mode) {
  if (!h || !mode) return fail(Q4HIP_EINVAL, "null argument");
  *mode = h->last_mode;
  return Q4HIP_OK;
}

int q4hip_read_logits(q4hip* h, float* out, int n) {
  if (!h || !out) return fail(Q4HIP_EINVAL, "null argument");
  if (n < h->V) return fail(Q4HIP_EINVAL, "buffer of %d floats, vocab is %d", n, h->V);
  HIPCHK(hipSetDevice(h->device));
  HIPCHK(hipStreamSynchronize(h->stream));
  HIPCHK(hipMemcpy(out, h->logits, (size_t)h->V * 4, hipMemcpyDeviceToHost));
  return Q4HIP_OK;
}

static int run_generate(q4hip* h, int first, int pos, int steps, int* out, float* ms) {
  if (!h || (steps > 0 && !out)) return fail(Q4HIP_EINVAL, "null argument");
  if (steps <= 0) return fail(Q4HIP_EINVAL, "steps must be positive");
  if (pos < 0 || (int64_t)pos + steps >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full");
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, &first, 1);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  prepare_attention(h);
  const bool pers = use_persistent(h) && !long_decode(h, (int64_t)pos + steps - 1);
  if (!pers) build_graph(h);
  h->pin_ids[0] = first;
  HIPCHK(hipMemcpyAsync(h->tokens + pos, h->pin_ids, 4, hipMemcpyHostToDevice, h->stream));
  k_set_pos<<<1, 64, 0, h->stream>>>(h->st, pos);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (ms) {
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipEventRecord(e0, h->stream));
  }
  if (pers) {
    HIPCHK(launch_persistent(h, pos, steps));
    h->last_mode = Q4HIP_DECODE_PERSISTENT;
  } else {
    for (int i = 0; i < steps; i++) decode_step(h);
    h->last_mode = Q4HIP_DECODE_GRAPH;
  }
  if (ms) HIPCHK(hipEventRecord(e1, h->stream));
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(h->pin_ids, h->tokens + pos + 1, (size_t)steps * 4, hipMemcpyDeviceToHost, h->stream));
  HIPCHK(hipStreamSynchronize(h->stream));
  const hipError_t te = ms ? hipEventElapsedTime(ms, e0, e1) : hipSuccess;
  if (ms) {
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  if (pers && aborted(h)) return run_generate(h, first, pos, steps, out, ms);
  HIPCHK(te);
  memcpy(out, h->pin_ids, (size_t)steps * 4);
  return Q4HIP_OK;
}

int q4hip_generate(q4hip* h, int first, int pos, int steps, int* out) {
  return run_generate(h, first, pos, steps, out, nullptr);
}

int q4hip_time_generate(q4hip* h, int first, int pos, int steps, int* out, float* ms) {
  if (!ms) return fail(Q4HIP_EINVAL, "null argument");
  return run_generate(h, first, pos, steps, out, ms);
}

int q4hip_profile_pass(q4hip* h, const int* ids, int ntok, int pos, float* us, int n) {
  if (!h || !us || !ids) return fail(Q4HIP_EINVAL, "null argument");
  if (n < Q4HIP_PROF_N) return fail(Q4HIP_EINVAL, "need %d entries", Q4HIP_PROF_N);
  if (ntok <= 0 || ntok > h->MT) return fail(Q4HIP_EINVAL, "%d tokens: one pass takes 1..%d", ntok, h->MT);
  if (pos < 0 || (int64_t)pos + ntok >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full");
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, ids, ntok);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  prepare_attention(h);
  memcpy(h->pin_ids, ids, (size_t)ntok * 4);
  HIPCHK(hipMemcpyAsync(h->tokens + pos, h->pin_ids, (size_t)ntok * 4, hipMemcpyHostToDevice, h->stream));
  k_set_pos<<<1, 64, 0, h->stream>>>(h->st, pos);
  std::vector<std::pair<int, hipEvent_t>> marks;
  h->prof = &marks;
  enqueue_pass(h, ntok, true);
  h->prof = nullptr;
  hipError_t e = hipStreamSynchronize(h->stream);
  for (int i = 0; i < Q4HIP_PROF_N; i++) us[i] = 0.0f;
  for (size_t i = 0; i + 1 < marks.size(); i++) {
    float ms = 0.0f;
    if (e == hipSuccess && hipEventElapsedTime(&ms, marks[i].second, marks[i + 1].second) == hipSuccess &&
        marks[i].first >= 0)
      us[marks[i].first] += ms * 1000.0f;
  }
  for (auto& p : marks) (void)hipEventDestroy(p.second);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "profile: %s", hipGetErrorString(e));
  return Q4HIP_OK;
}

int q4hip_profile(q4hip* h, int token, int pos, float* us, int n) {
  return q4hip_profile_pass(h, &token, 1, pos, us, n);
}

int q4hip_profile_persistent(q4hip* h, int token, int pos, float* us, int n) {
  if (!h || !us) return fail(Q4HIP_EINVAL, "null argument");
  if (n < (h->NL + 1) * 16) return fail(Q4HIP_EINVAL, "need %d entries", (h->NL + 1) * 16);
  if (pos < 0 || pos + 1 >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full");
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, &token, 1);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  if (!use_persistent(h)) return fail(Q4HIP_EINVAL, "the persistent decode kernel is not in use");
  const int G = h->pers_grid;
  const int cnt = (h->NL + 1) * 16 + kProfWG * h->NL * G;
  unsigned long long* d = nullptr;
  HIPCHK(hipMalloc(&d, (size_t)cnt * 8));
  std::vector<unsigned long long> t(cnt, 0);
  hipError_t e = hipMemsetAsync(d, 0, (size_t)cnt * 8, h->stream);
  h->pin_ids[0] = token;
  if (e == hipSuccess) e = hipMemcpyAsync(h->tokens + pos, h->pin_ids, 4, hipMemcpyHostToDevice, h->stream);
  if (e == hipSuccess) {
    k_set_pos<<<1, 64, 0, h->stream>>>(h->st, pos);
    e = launch_persistent(h, pos, 1, d);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
  if (e == hipSuccess) e = hipMemcpy(t.data(), d, (size_t)cnt * 8, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "persistent profile: %s", hipGetErrorString(e));
  if (aborted(h)) return fail(Q4HIP_EHIP, "persistent profile: a bounded wait timed out");
  const unsigned long long t0 = t[h->NL * 16 + 3];
  const int out = std::min(n, cnt);
  for (int i = 0; i < out; i++) us[i] = t[i] ? (float)((double)(long long)(t[i] - t0) * 0.01) : -1.0f;
  // slots 16L+4/5 hold the shader clock counter at kernel start / step end: report its MHz
  const double wall_us = (double)(long long)(t[h->NL * 16 + 2] - t0) * 0.01;
  const double cycles = (double)(long long)(t[h->NL * 16 + 5] - t[h->NL * 16 + 4]);
  us[h->NL * 16 + 4] = wall_us > 0 ? (float)(cycles / wall_us) : -1.0f;
  us[h->NL * 16 + 5] = (float)G;
  return Q4HIP_OK;
}

int q4hip_time_head(q4hip* h, int iters, float* us_per_launch) {
  if (!h || !us_per_launch || iters <= 0) return fail(Q4HIP_EINVAL, "bad argument");
  int rc = check_ready(h);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  HIPCHK(hipEventRecord(e0, h->stream));
  for (int i = 0; i < iters; i++) launch_head(h->stream, h->head, h->xq, h->logits);
  HIPCHK(hipEventRecord(e1, h->stream));
  HIPCHK(hipGetLastError());
  HIPCHK(hipEventSynchronize(e1));
  float ms = 0.0f;
  HIPCHK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *us_per_launch = ms * 1000.0f / iters;
  return Q4HIP_OK;
}

// ---------------------------------------------------------------- batched decode

struct q4hip_batch {
  q4hip* h = nullptr;
  int B = 0, P = 0;
  size_t seq_stride = 0;     // floats of one sequence's K (or V) cache: layers * kv_heads * ctx * head_dim
  size_t attn_lds = 0;
  void *kc = nullptr, *vc = nullptr;   // the sequences' caches, elements of the context's type
  float *logits = nullptr, *am_v = nullptr;
  float* sc = nullptr;       // attention scores [B][heads][ctx]
  int *am_i = nullptr, *tok = nullptr, *pos = nullptr, *out = nullptr;
  int out_cap = 0;           // ints of `out`
  int* pin = nullptr;        // pinned staging: B tokens, B positions
};

namespace {

// One decode step of all B sequences: tokens bt->tok at positions bt->pos; the greedy tokens go to
// bt->tok (and out[0..B) when given) and every position advances by one.
void enqueue_batch_step(q4hip_batch* bt, int* out) {
  q4hip* h = bt->h;
  const int B = bt->B, D = h->D, F = h->F, HD = h->HD, QKV = h->QKV;
  hipStream_t s = h->stream;
  uint4* xh = B > 8 ? h->xh : nullptr;
  k_embed_list<<<B, 256, 0, s>>>(h->embd, D, bt->tok, h->x);
  for (int l = 0; l < h->NL; l++) {
    Layer& y = h->L[l];
    launch_quant<QM_NORM>(s, B, h->x, D, D, y.attn_norm, h->eps, h->xq, h->xstride, 0, xh);
    SkRope rp;
    rp.rope = h->rope; rp.kc = bt->kc; rp.vc = bt->vc; rp.pos = bt->pos; rp.seq_stride = bt->seq_stride;
    rp.ctx = h->ctx; rp.layer = l; rp.H = h->H; rp.KVH = h->KVH; rp.hd = HD; rp.kv16 = h->kv16;
    if (!launch_qkv_rope(s, y.qkv, xh, h->xstride, B, h->qkv, QKV, y.bqkv, rp)) {
      launch_matvec<OP_BIAS>(s, y.qkv, h->xq, h->xstride, B, h->qkv, QKV, y.bqkv, xh);
      if (h->kv16)
        k_rope_kv_list<kvhalf><<<dim3(h->H + h->KVH, B), HD / 2, 0, s>>>(h->qkv, QKV, D, h->H, h->KVH, HD, h->rope,
                                                                         (kvhalf*)bt->kc, (kvhalf*)bt->vc, h->ctx, l,
                                                                         bt->pos, bt->seq_stride);
      else
        k_rope_kv_list<float><<<dim3(h->H + h->KVH, B), HD / 2, 0, s>>>(h->qkv, QKV, D, h->H, h->KVH, HD, h->rope,
                                                                        (float*)bt->kc, (float*)bt->vc, h->ctx, l,
                                                                        bt->pos, bt->seq_stride);
    }
    launch_attn_list(s, HD, B, h->H, h->KVH, h->qkv, QKV, bt->kc, bt->vc, h->kv16, h->ctx, l, bt->sc, h->att, D, bt->pos,
                     bt->seq_stride, h->xq, h->xstride, xh);
    launch_matvec<OP_ADD>(s, y.o, h->xq, h->xstride, B, h->x, D, nullptr, xh);
    launch_quant<QM_NORM>(s, B, h->x, D, D, y.ffn_norm, h->eps, h->xq, h->xstride, 0, xh);
    uint4* xh_act = xh;
    if (launch_gu_swiglu(s, y.gu, xh, h->xstride, B, h->xq, h->xh2, F)) {
      xh_act = h->xh2;
    } else {
      launch_matvec<OP_STORE>(s, y.gu, h->xq, h->xstride, B, h->gu, 2 * F, nullptr, xh);
      launch_quant<QM_SWIGLU>(s, B, h->gu, 2 * F, F, nullptr, 0.0f, h->xq, h->xstride, 0, xh);
    }
    launch_matvec<OP_ADD>(s, y.down, h->xq, h->xstride, B, h->x, D, nullptr, xh_act);
  }
  launch_quant<QM_NORM>(s, B, h->x, D, D, h->out_norm, h->eps, h->xq, h->xstride, 0, xh);
  if (h->head.fmt == Q4HIP_TYPE_Q8_0) {
    for (int b = 0; b < B; b++)
      k_matvec_q8<<<(unsigned)(h->head.Np / 16), 64, (size_t)h->head.nb * 64, s>>>(
          h->head.view(), h->xq + (size_t)b * h->xstride * 4, bt->logits + (size_t)b * h->V);
  } else {
    launch_matvec<OP_STORE>(s, h->head, h->xq, h->xstride, B, bt->logits, h->V, nullptr, xh);
  }
  k_argmax_rows1<<<dim3(bt->P, B), 256, 0, s>>>(bt->logits, h->V, bt->am_v, bt->am_i, bt->P);
  k_argmax_rows2<<<B, 256, 0, s>>>(bt->am_v, bt->am_i, bt->P, bt->tok, bt->pos, out);
}

}  // namespace

void q4hip_batch_destroy(q4hip_batch* bt) {
  if (!bt) return;
  (void)hipSetDevice(bt->h->device);
  (void)hipStreamSynchronize(bt->h->stream);
  void* bufs[] = {bt->kc, bt->vc, bt->logits, bt->am_v, bt->am_i, bt->tok, bt->pos, bt->out, bt->sc};
  for (void* p : bufs) if (p) (void)hipFree(p);
  if (bt->pin) (void)hipHostFree(bt->pin);
  delete bt;
}

int q4hip_batch_create(q4hip_batch** out, q4hip* h, int B) {
  if (!out || !h) return fail(Q4HIP_EINVAL, "null argument");
  *out = nullptr;
  if (B <= 0 || B > h->MT) return fail(Q4HIP_EINVAL, "%d sequences: a batch holds 1..%d (the context's pass size)", B, h->MT);
  if (h->H / h->KVH > kMaxGroup) return fail(Q4HIP_EINVAL, "more than %d query heads per kv head", kMaxGroup);
  HIPCHK(hipSetDevice(h->device));
  const size_t lds = attn_pv_lds(h->H, h->KVH, h->ctx);
  if (!attn_list_ok(h->H, h->KVH, h->HD, h->ctx))
    return fail(Q4HIP_EINVAL, "ctx %d: batched attention needs %zu bytes of shared memory", h->ctx, lds);
  q4hip_batch* bt = new q4hip_batch();
  bt->h = h;
  bt->B = B;
  bt->P = (h->V + 4095) / 4096;
  bt->seq_stride = (size_t)h->NL * h->KVH * h->ctx * h->HD;
  bt->attn_lds = lds;
  const size_t kvbytes = (size_t)B * bt->seq_stride * h->kvb;
  hipError_t e = hipSuccess;
  auto al = [&](void** p, size_t bytes) { if (e == hipSuccess) e = hipMalloc(p, bytes); };
  al((void**)&bt->kc, kvbytes);
  al((void**)&bt->vc, kvbytes);
  al((void**)&bt->logits, (size_t)B * h->V * 4);
  al((void**)&bt->am_v, (size_t)B * bt->P * 4);
  al((void**)&bt->am_i, (size_t)B * bt->P * 4);
  al((void**)&bt->tok, (size_t)B * 4);
  al((void**)&bt->pos, (size_t)B * 4);
  al((void**)&bt->sc, (size_t)B * h->H * score_stride(h->ctx) * 4);
  if (e == hipSuccess) e = hipMemsetAsync(bt->kc, 0, kvbytes, h->stream);
  if (e == hipSuccess) e = hipMemsetAsync(bt->vc, 0, kvbytes, h->stream);
  if (e == hipSuccess) e = hipHostMalloc((void**)&bt->pin, (size_t)2 * B * 4, hipHostMallocDefault);
  if (e == hipSuccess) e = hipStreamSynchronize(h->stream);   // caches zeroed before q4hip_batch_set_kv
  if (e != hipSuccess) {
    const int rc = fail(Q4HIP_EHIP, "batch of %d: %s", B, hipGetErrorString(e));
    q4hip_batch_destroy(bt);
    return rc;
  }
  *out = bt;
  return Q4HIP_OK;
}

int q4hip_batch_set_kv(q4hip_batch* bt, int seq, int layer, int kv_head, int pos0, int n, const float* k,
                       const float* v) {
  if (!bt || !k || !v) return fail(Q4HIP_EINVAL, "null argument");
  q4hip* h = bt->h;
  if (seq < 0 || seq >= bt->B) return fail(Q4HIP_EINVAL, "sequence %d of %d", seq, bt->B);
  if (layer < 0 || layer >= h->NL) return fail(Q4HIP_EINVAL, "layer %d of %d", layer, h->NL);
  if (kv_head < 0 || kv_head >= h->KVH) return fail(Q4HIP_EINVAL, "kv head %d of %d", kv_head, h->KVH);
  if (n <= 0 || pos0 < 0 || (int64_t)pos0 + n > h->ctx) return fail(Q4HIP_ECONTEXT, "positions %d..%lld outside 0..%d", pos0, (long long)pos0 + n, h->ctx);
  HIPCHK(hipSetDevice(h->device));
  HIPCHK(hipStreamSynchronize(h->stream));
  const size_t off = (size_t)seq * bt->seq_stride + (((size_t)layer * h->KVH + kv_head) * h->ctx + pos0) * h->HD;
  return upload_kv(h, (char*)bt->kc + off * h->kvb, (char*)bt->vc + off * h->kvb, k, v, (size_t)n * h->HD);
}

int q4hip_batch_prefill(q4hip_batch* bt, int seq, const int* ids, int n, int pos, int* next) {
  if (!bt || !ids || !next) return fail(Q4HIP_EINVAL, "null argument");
  q4hip* h = bt->h;
  if (seq < 0 || seq >= bt->B) return fail(Q4HIP_EINVAL, "sequence %d of %d", seq, bt->B);
  if (n <= 0) return fail(Q4HIP_EINVAL, "no tokens");
  if (pos < 0 || (int64_t)pos + n >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full");
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, ids, n);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  prepare_attention(h);
  // the passes run eagerly against this sequence's cache; the context's own cache is untouched
  void* kc = h->kc;
  void* vc = h->vc;
  h->kc = (char*)bt->kc + (size_t)seq * bt->seq_stride * h->kvb;
  h->vc = (char*)bt->vc + (size_t)seq * bt->seq_stride * h->kvb;
  memcpy(h->pin_ids, ids, (size_t)n * 4);
  hipError_t e = hipMemcpyAsync(h->tokens + pos, h->pin_ids, (size_t)n * 4, hipMemcpyHostToDevice, h->stream);
  for (int c = 0; e == hipSuccess && c < n; c += h->MT) {
    const int k = std::min(h->MT, n - c);
    k_set_pos<<<1, 64, 0, h->stream>>>(h->st, pos + c);
    enqueue_pass(h, k, c + k >= n);
  }
  h->kc = kc;
  h->vc = vc;
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(h->pin_next, &h->st->next, 4, hipMemcpyDeviceToHost, h->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "batch prefill: %s", hipGetErrorString(e));
  *next = h->pin_next[0];
  return Q4HIP_OK;
}

static int run_batch(q4hip_batch* bt, const int* first, const int* pos, int steps, int* out, float* ms) {
  if (!bt || !first || !pos || !out) return fail(Q4HIP_EINVAL, "null argument");
  q4hip* h = bt->h;
  const int B = bt->B;
  if (steps <= 0) return fail(Q4HIP_EINVAL, "steps must be positive");
  for (int b = 0; b < B; b++)
    if (pos[b] < 0 || (int64_t)pos[b] + steps >= h->ctx) return fail(Q4HIP_ECONTEXT, "context full (sequence %d)", b);
  int rc = check_ready(h);
  if (rc) return rc;
  rc = check_ids(h, first, B);
  if (rc) return rc;
  HIPCHK(hipSetDevice(h->device));
  if ((int64_t)steps * B > bt->out_cap) {
    if (bt->out) HIPCHK(hipFree(bt->out));
    bt->out = nullptr;
    bt->out_cap = 0;
    HIPCHK(hipMalloc(&bt->out, (size_t)steps * B * 4));
    bt->out_cap = steps * B;
  }
  memcpy(bt->pin, first, (size_t)B * 4);
  memcpy(bt->pin + B, pos, (size_t)B * 4);
  HIPCHK(hipMemcpyAsync(bt->tok, bt->pin, (size_t)B * 4, hipMemcpyHostToDevice, h->stream));
  HIPCHK(hipMemcpyAsync(bt->pos, bt->pin + B, (size_t)B * 4, hipMemcpyHostToDevice, h->stream));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (ms) {
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipEventRecord(e0, h->stream));
  }
  for (int i = 0; i < steps; i++) enqueue_batch_step(bt, bt->out + (size_t)i * B);
  if (ms) HIPCHK(hipEventRecord(e1, h->stream));
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(h->stream));
  if (ms) {
    HIPCHK(hipEventElapsedTime(ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  HIPCHK(hipMemcpy(out, bt->out, (size_t)steps * B * 4, hipMemcpyDeviceToHost));
  return Q4HIP_OK;
}

int q4hip_batch_generate(q4hip_batch* bt, const int* first, const int* pos, int steps, int* out) {
  return run_batch(bt, first, pos, steps, out, nullptr);
}

int q4hip_batch_time_generate(q4hip_batch* bt, const int* first, const int* pos, int steps, int* out, float* ms) {
  if (!ms) return fail(Q4HIP_EINVAL, "null argument");
  return run_batch(bt, first, pos, steps, out, ms);
}

int q4hip_batch_read_logits(q4hip_batch* bt, float* out, int64_t n) {
  if (!bt || !out) return fail(Q4HIP_EINVAL, "null argument");
  q4hip* h = bt->h;
  if (n < (int64_t)bt->B * h->V) return fail(Q4HIP_EINVAL, "buffer of %lld floats, batch logits are %lld", (long long)n, (long long)bt->B * h->V);
  HIPCHK(hipSetDevice(h->device));
  HIPCHK(hipStreamSynchronize(h->stream));
  HIPCHK(hipMemcpy(out, bt->logits, (size_t)bt->B * h->V * 4, hipMemcpyDeviceToHost));
  return Q4HIP_OK;
}

// ---------------------------------------------------------------- isolated matvec

struct q4hip_mv {
  int device;
  hipStream_t stream;
  Mat W;
  float *x, *y;
  uint4* xq;
};

void q4hip_mv_destroy(q4hip_mv* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  mat_free(m->W);
  if (m->x) (void)hipFree(m->x);
  if (m->y) (void)hipFree(m->y);
  if (m->xq) (void)hipFree(m->xq);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int q4hip_mv_create(q4hip_mv** out, int N, int K, const void* w, int device) {
  if (!out || !w) return fail(Q4HIP_EINVAL, "null argument");
  *out = nullptr;
  if (N <= 0 || K <= 0 || K % 32) return fail(Q4HIP_EINVAL, "bad shape %d x %d", N, K);
  int ndev = 0;
  HIPCHK(hipGetDeviceCount(&ndev));
  if (device < 0 || device >= ndev) return fail(Q4HIP_EINVAL, "device %d of %d", device, ndev);
  HIPCHK(hipSetDevice(device));
  q4hip_mv* m = new q4hip_mv();
  m->device = device;
  m->stream = nullptr; m->x = nullptr; m->y = nullptr; m->xq = nullptr;
  int rc = Q4HIP_OK;
  hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&m->x, (size_t)K * 4);
  if (e == hipSuccess) e = hipMalloc(&m->y, (size_t)N * 4);
  if (e == hipSuccess) e = hipMalloc(&m->xq, (size_t)(K / 32) * 64);
  if (e != hipSuccess) { rc = fail(Q4HIP_EHIP, "matvec alloc: %s", hipGetErrorString(e)); q4hip_mv_destroy(m); return rc; }
  rc = mat_alloc(m->W, N, K, m->stream);
  if (rc == Q4HIP_OK) rc = mat_upload(m->W, 0, N, w, m->stream);
  if (rc != Q4HIP_OK) { q4hip_mv_destroy(m); return rc; }
  matvec_split_setup(device);
  *out = m;
  return Q4HIP_OK;
}

static void mv_launch(q4hip_mv* m) {
  launch_matvec<OP_STORE>(m->stream, m->W, m->xq, m->W.nb, 1, m->y, m->W.N, nullptr);
}

int q4hip_mv_run(q4hip_mv* m, const float* x, float* y) {
  if (!m || !x || !y) return fail(Q4HIP_EINVAL, "null argument");
  HIPCHK(hipSetDevice(m->device));
  const int K = m->W.K;
  HIPCHK(hipMemcpyAsync(m->x, x, (size_t)K * 4, hipMemcpyHostToDevice, m->stream));
  launch_quant<QM_PLAIN>(m->stream, 1, m->x, K, K, nullptr, 0.0f, m->xq, K / 32, 0);
  mv_launch(m);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(y, m->y, (size_t)m->W.N * 4, hipMemcpyDeviceToHost, m->stream));
  HIPCHK(hipStreamSynchronize(m->stream));
  return Q4HIP_OK;
}

int q4hip_mv_time(q4hip_mv* m, int iters, float* us) {
  if (!m || !us || iters <= 0) return fail(Q4HIP_EINVAL, "bad argument");
  HIPCHK(hipSetDevice(m->device));
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  HIPCHK(hipEventRecord(e0, m->stream));
  for (int i = 0; i < iters; i++) mv_launch(m);
  HIPCHK(hipEventRecord(e1, m->stream));
  HIPCHK(hipGetLastError());
  HIPCHK(hipEventSynchronize(e1));
  float ms = 0.0f;
  HIPCHK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *us = ms * 1000.0f / iters;
  return Q4HIP_OK;
}

int q4hip_mv_time_cold(q4hip_mv* m, int64_t rotate_bytes, int iters, float* us, int* copies_used) {
  if (!m || !us || iters <= 0 || rotate_bytes < 0) return fail(Q4HIP_EINVAL, "bad argument");
  HIPCHK(hipSetDevice(m->device));
  const Mat& W = m->W;
  const size_t qb = (size_t)W.Np * W.ng * 64 + kWeightPadQ, db = (size_t)W.Np * W.nb8 * 16 + kWeightPadD;
  const size_t qa = (qb + 255) / 256 * 256, per = qa + (db + 255) / 256 * 256;
  const int copies = (int)std::max<int64_t>(2, (rotate_bytes + (int64_t)per - 1) / (int64_t)per);
  uint8_t* buf = nullptr;
  HIPCHK(hipMalloc(&buf, per * copies));
  hipError_t e = hipSuccess;
  std::vector<Mat> views(copies, W);
  for (int c = 0; c < copies && e == hipSuccess; c++) {
    uint8_t* base = buf + per * c;
    views[c].qs = (uint32_t*)base;
    views[c].d = (uint16_t*)(base + qa);
    e = hipMemcpyAsync(views[c].qs, W.qs, qb, hipMemcpyDeviceToDevice, m->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(views[c].d, W.d, db, hipMemcpyDeviceToDevice, m->stream);
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) {
    for (int i = 0; i < copies; i++)   // one pass over every copy before timing
      launch_matvec<OP_STORE>(m->stream, views[i], m->xq, W.nb, 1, m->y, W.N, nullptr);
    e = hipEventRecord(e0, m->stream);
  }
  if (e == hipSuccess) {
    for (int i = 0; i < iters; i++)
      launch_matvec<OP_STORE>(m->stream, views[i % copies], m->xq, W.nb, 1, m->y, W.N, nullptr);
    e = hipEventRecord(e1, m->stream);
  }
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipStreamSynchronize(m->stream);
  (void)hipFree(buf);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "cold matvec timing: %s", hipGetErrorString(e));
  *us = ms * 1000.0f / iters;
  if (copies_used) *copies_used = copies;
  return Q4HIP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- matvec without allocation

// The int8 activation blocks of q4hip_mv_run_noalloc (64 bytes per 32 values, the layout
// k_quant writes): one copy per device, held until the process ends and shared by every call on
// that device.  Each call quantizes its whole input into it before the matvec reads it, so
// nothing in it has to start at zero.
constexpr int kNoAllocBlocks = Q4HIP_NOALLOC_MAX_K / 32;
static __device__ __align__(256) uint4 scratch[kNoAllocBlocks * 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint4* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on `device` (current), looked up once per device.  In host code the
// array's name is only a stand-in: kernels get this address.
int scratch_on(int device, uint4** out) {
  if (device < 0 || device >= kMaxDevices) return fail(Q4HIP_EINVAL, "device %d beyond %d", device, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(Q4HIP_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_dev[device] = (uint4*)p;
  }
  *out = g_scratch_dev[device];
  return Q4HIP_OK;
}

// `bytes` of device memory of `device` start at p (checked before any launch, so a host pointer or
// a short buffer is an error, not a memory fault).
int check_device_span(const void* p, size_t bytes, int device, const char* what) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return fail(Q4HIP_EINVAL, "%s: not device memory", what);
  }
  if (a.type != hipMemoryTypeDevice || a.device != device)
    return fail(Q4HIP_EINVAL, "%s: not device memory of device %d", what, device);
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
    (void)hipGetLastError();
    return fail(Q4HIP_EINVAL, "%s: no device allocation holds it", what);
  }
  if ((const char*)p + bytes > (const char*)base + size)
    return fail(Q4HIP_EINVAL, "%s: %zu bytes needed, the allocation ends %zu bytes after it", what, bytes,
                (size_t)((const char*)base + size - (const char*)p));
  return Q4HIP_OK;
}

}  // namespace

extern "C" {

int q4hip_mv_run_noalloc(q4hip_mv* m, const float* x, float* y, void* stream) {
  if (!m || !x || !y) return fail(Q4HIP_EINVAL, "null argument");
  const int K = m->W.K, N = m->W.N;
  if (K > Q4HIP_NOALLOC_MAX_K)
    return fail(Q4HIP_EINVAL, "K = %d exceeds the no-allocation limit of %d", K, Q4HIP_NOALLOC_MAX_K);
  HIPCHK(hipSetDevice(m->device));
  uint4* xq = nullptr;
  int rc = scratch_on(m->device, &xq);
  if (rc == Q4HIP_OK) rc = check_device_span(x, (size_t)K * 4, m->device, "x");
  if (rc == Q4HIP_OK) rc = check_device_span(y, (size_t)N * 4, m->device, "y");
  if (rc != Q4HIP_OK) return rc;
  hipStream_t s = stream ? (hipStream_t)stream : m->stream;
  launch_quant<QM_PLAIN>(s, 1, x, K, K, nullptr, 0.0f, xq, K / 32, 0);
  launch_matvec<OP_STORE>(s, m->W, xq, m->W.nb, 1, y, N, nullptr);
  HIPCHK(hipGetLastError());
  if (!stream) HIPCHK(hipStreamSynchronize(s));
  return Q4HIP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- quotient self-check

namespace {

// Form `mode` over input bit patterns [lo, hi] against the IEEE division (grid-stride, bounded).
__global__ __launch_bounds__(256) void k_check_division(int mode, uint32_t lo, uint32_t hi,
                                                        unsigned long long* bad) {
  unsigned long long n = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)lo + blockIdx.x * blockDim.x + threadIdx.x; i <= hi; i += stride) {
    const float a = __uint_as_float((uint32_t)i);
    float want, got;
    if (mode == 0) {
      want = a / 127.0f;
      got = div_127(a);
    } else if (mode == 1) {
      want = a != 0.0f ? 1.0f / a : 0.0f;
      got = inv_scale(a);
    } else if (mode == 2) {
      const float y = 1.0f + fast_exp(-a);
      want = a / y;
      got = div_silu(a, y);
    } else if (mode == 3) {
      want = a / 896.0f;
      got = div_const<896>(a);
    } else {
      want = 1.0f / a;
      got = recip(a);
    }
    n += __float_as_uint(want) != __float_as_uint(got) && !(want != want && got != got);
  }
  if (n) atomicAdd(bad + mode, n);
}

}  // namespace

extern "C" {

int q4hip_check_division(int device, unsigned long long* mismatches, int n) {
  if (!mismatches || n < 1 || n > 5) return fail(Q4HIP_EINVAL, "need 1..5 counters");
  HIPCHK(hipSetDevice(device));
  unsigned long long* d = nullptr;
  HIPCHK(hipMalloc(&d, 5 * sizeof(unsigned long long)));
  hipError_t e = hipMemset(d, 0, 5 * sizeof(unsigned long long));
  const uint32_t top = 0x7F800000u;   // +inf: every non-negative value
  for (int mode = 0; mode < n && e == hipSuccess; mode++) {
    if (mode == 2) {
      k_check_division<<<8192, 256>>>(mode, 0u, 0x7FFFFFFFu, d);
      k_check_division<<<8192, 256>>>(mode, 0x80000000u, 0xFFFFFFFFu, d);
    } else {
      k_check_division<<<8192, 256>>>(mode, 0u, top, d);
    }
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(mismatches, d, (size_t)n * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(Q4HIP_EHIP, "division check: %s", hipGetErrorString(e));
  return Q4HIP_OK;
}

int q4hip_attn_ring_rows(int pos, int kv_tile, int ring_slots, int split, int half, int kv_f16, int* lo, int* hi,
                         int* loads) {
  if (!lo || !hi || !loads) return fail(Q4HIP_EINVAL, "null argument");
  if (pos < 0 || kv_tile < 0 || (ring_slots != 3 && ring_slots != 7) || (half != 0 && half != 1))
    return fail(Q4HIP_EINVAL, "bad argument");
  // the issues of attn_step, with the kernel's own row arithmetic (attn_ring, kchunk_t0, vslot_t0,
  // vpslot_t0, ring_row): each issue reads `span` rows from its first row on
  const AttnRing r = attn_ring(pos, kv_tile, split != 0, half, kv_f16 != 0);
  const int cs = kchunk_slots(ring_slots);
  int mn = INT_MAX, mx = -1, cnt = 0;
  auto take = [&](int t0, int span, int limit) {
    for (int i = 0; i < span; i++) {
      const int row = ring_row(t0 + i, limit);
      mn = std::min(mn, row);
      mx = std::max(mx, row);
    }
    cnt++;
  };
  for (int wave = 0; wave < 4; wave++) {           // K chunks: cs - 1 ahead, then one per chunk
    const int nloc = attn_nloc(r.nkc, wave);
    if (nloc > 0)
      for (int j = 0; j < nloc + cs - 1; j++) take(kchunk_t0(r.kbeg, j, nloc, wave), 16, r.kend);
  }
  if (!split) {                                    // P.V slots: ring - 1 ahead, then one per slot
    if (r.nck > 0)
      for (int c = 0; c < r.nck + ring_slots - 1; c++) take(vslot_t0(r.nt, c, r.nck, r.vr), r.vr, pos);
  } else {                                         // split: ring - 2 ahead, then one per slot
    if (r.nckv > 0)
      for (int c = 0; c < r.nckv + ring_slots - 2; c++) take(vpslot_t0(c, r.nckv), kVRows, pos);
  }
  *lo = cnt ? mn : 0;
  *hi = cnt ? mx : -1;
  *loads = cnt;
  return Q4HIP_OK;
}

}  // extern "C"
