// gemm_sk.h -- the Q4_0 projection of a few tokens (batched decode) on the matrix cores.
//
// y[m][n] (op)= W[n] . x[m] for up to a few dozen tokens, every output accumulated exactly as
// matmul_q4 does (engine/kernels.c:200-229): four lane chains acc_j += f32(p_j) * (dw * dx) over
// the blocks in order, then ((a0 + a1) + a2) + a3.  p_j, the integer dot of reference lane j's 8
// nibbles (as n - 8) with its 8 int8 activations, is one v_mfma_f32_16x16x16_f16 per 16 rows x 16
// tokens: k = 0..3 carry x_k * (1024 + n_k) (a low nibble becomes fp16 0x6400 | n by a byte
// permute), k = 4..7 carry (x_k / 16) * (1024 + 16 n_k) (a high nibble masked in place, 0x6400 |
// n << 4) = 64 x_k + n_k x_k, k = 8 carries (-sum of x_0..3) * 1032 and k = 9 (-sum of x_4..7) * 72,
// k = 10..15 are zero; every product and partial sum is an integer below 2^21, so the fp32 result
// is exactly p_j.  The chain updates stay on the vector ALUs in block order.
//
// Layout of a workgroup (16 tokens, 256 threads):
//   JS = 4  16 weight rows; wave w runs lane chain w of all 16 rows (for matrices with few rows:
//           four times the workgroups); the chains are added in the reference's order at the end
//   JS = 1  64 weight rows; wave w runs rows 16w .. 16w + 15 with all four chains
// What one group of 4 blocks needs -- the 16 tokens' fp16 operands (8 KB, contiguous in the
// tiled operand layout), their block scales dx, the weight words and the fp16 weight scales of the
// workgroup's rows -- streams through an R-slot ring in shared memory by asynchronous
// global -> LDS loads, R - 1 groups ahead of the group being computed.  Every wave issues the same
// five load instructions per group, so the wait for the oldest slot is a single vmcnt.  JS = 1
// shares each slot among the waves (one barrier per group); with JS = 4 the waves share nothing but
// the scales, so each wave streams its own chain's operands, the dx and the scales through a ring
// of its own and runs without barriers.  Loads past the last group or block are clamped to it
// (valid memory, never used).
#pragma once
#include "kernels.h"

namespace q4 {

typedef __attribute__((address_space(3))) void SkLds;
typedef _Float16 sk_h4 __attribute__((ext_vector_type(4)));
typedef float sk_f4 __attribute__((ext_vector_type(4)));

// Bytes of one ring slot: JS = 1 one shared part; JS = 4 one part (WAVE bytes) per wave, holding
// that wave's chain only.
template <int JS>
struct SkSlot {
  static constexpr int ACT = JS == 4 ? 2048 : 8192; // [block 4]([chain 4] for JS 1)[quarter 4][token 16][8 B]
  static constexpr int DX = 256;                    // [block 4][token 16] f32
  static constexpr int QS = JS == 4 ? 256 : 4096;   // JS 4: [row 16] uint4; JS 1: [chain 4][row 64] uint4
  static constexpr int SC = JS == 4 ? 128 : 512;    // [row][2 dwords]: the 4 fp16 scales of the group
  static constexpr int oDX = ACT, oQS = ACT + DX, oSC = ACT + DX + QS, WAVE = ACT + DX + QS + SC;
  static constexpr int BYTES = JS == 4 ? 4 * WAVE : WAVE;
};

// Wait until at most n of this wave's load instructions are outstanding, and this wave's LDS
// accesses are done, then meet the other waves.  (Not __syncthreads: its workgroup fence would wait
// for every outstanding load into LDS.)
template <int N>
__device__ __forceinline__ void sk_sync() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The same wait without meeting the other waves (a ring of the wave's own).
template <int N>
__device__ __forceinline__ void sk_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}

// Asynchronous global -> LDS loads (global_load_lds): lane l's 16 (or 4) bytes from `src` land at
// LDS address lds + 16 l (4 l); `lds` is wave-uniform and goes to M0.  Written as inline assembly so
// that the compiler does not treat every later shared-memory read as dependent on every load in
// flight (it would wait for all of them): the ring's own vmcnt waits order the reads.  The s_nop
// covers the wait state the hardware needs between writing M0 and the load that reads it.
__device__ __forceinline__ void sk_dma16(const void* src, const void* lds) {
  const uint32_t a = (uint32_t)(uintptr_t)(SkLds*)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(a) : "memory");
}
__device__ __forceinline__ void sk_dma4(const void* src, const void* lds) {
  const uint32_t a = (uint32_t)(uintptr_t)(SkLds*)lds;
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(a) : "memory");
}

// Per-lane sources of a workgroup's loads, computed once; group g adds g times a stride.
//   act  JS 1: this wave's block (4g + wave) of the 16-token tile, 2 KB, two instructions of 1 KB;
//        JS 4: chain `wave` of the group's 4 blocks (512 bytes each), two blocks per instruction
//   dx   JS 1: the same block's 16 block scales (lanes 0..15); JS 4: the 4 blocks' (all lanes)
//   qs   JS 4: row lane (0..15) of the workgroup, chain `wave`; JS 1: row lane (0..63), chain `wave`
//   sc   the 8 bytes of the group's 4 fp16 scales of one row, as two dwords (JS 4: lanes 0..31 take
//        the 16 rows; JS 1: lanes 0..31 take rows 16 wave .. 16 wave + 15)
// Blocks past nb and groups past ng are clamped to the last ones.
template <int JS>
struct SkSrc {
  const uint4* act;      // JS 1: block `wave` of group 0 of the tile; JS 4: the lane's uint4 of chain `wave` of block 0
  const float* dx;       // JS 4: the lane's token scale in block 0
  const uint4* qs;       // group 0
  const uint32_t* sc;    // group 0 (dword 0 of the row's 4-scale half of a uint4)
  int nb, ng, wave, lane;
  // JS 1 local row l (0..63) of the workgroup -> matrix row: R0 + l, or with ffn > 0 (the fused
  // gate|up matrix, R0 = 32 b) gate rows 32 b + l for l < 32 and up rows ffn + 32 b + l - 32.
  static __device__ __forceinline__ int row_of(int R0, int ffn, int l) {
    return ffn > 0 ? (l < 32 ? R0 + l : ffn + R0 + l - 32) : R0 + l;
  }
  // JS 4 with RoPE pairs (hd > 0, the fused qkv projection): row group rg of a head of hd rows
  // holds rows 8p .. 8p + 7 of the head's first half (local rows 0..7) and the matching rows of its
  // second half (local rows 8..15), so each RoPE pair (i, i + hd/2) meets in one workgroup.
  static __device__ __forceinline__ int rope_row(int rg, int hd, int l) {
    const int gpr = hd >> 4, head = rg / gpr, p = rg - head * gpr;
    return head * hd + (l < 8 ? 8 * p + l : (hd >> 1) + 8 * p + l - 8);
  }
  __device__ __forceinline__ SkSrc(const Q4Mat& W, const uint4* xt, int xstride, int T, int R0, int ffn = 0,
                                   int hd = 0) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    nb = W.nb;
    ng = W.ng;
    act = xt + (size_t)T * xstride * kXhBlock;
    dx = reinterpret_cast<const float*>(act + 128) + (lane & 15);
    const int tile = R0 >> 6, rr0 = R0 & 63;
    if (JS == 4) act += wave * 32 + (lane & 31);
    if (JS == 4 && hd > 0) {
      const int rq = rope_row(R0 >> 4, hd, lane & 15), rs = rope_row(R0 >> 4, hd, (lane >> 1) & 15);
      qs = W.qs + ((size_t)(rq >> 6) * ng * 64 + (rq & 63)) * 4 + wave;
      sc = reinterpret_cast<const uint32_t*>(W.d + (size_t)(rs >> 6) * W.nb8 * 64 + (rs & 63)) + (lane & 1);
    } else if (JS == 4) {
      qs = W.qs + ((size_t)tile * ng * 64 + rr0 + (lane & 15)) * 4 + wave;
      sc = reinterpret_cast<const uint32_t*>(W.d + (size_t)tile * W.nb8 * 64 + rr0 + ((lane >> 1) & 15)) +
           (lane & 1);
    } else {
      const int rq = row_of(R0, ffn, lane), rs = row_of(R0, ffn, 16 * wave + ((lane >> 1) & 15));
      qs = W.qs + ((size_t)(rq >> 6) * ng * 64 + (rq & 63)) * 4 + wave;
      sc = reinterpret_cast<const uint32_t*>(W.d + (size_t)(rs >> 6) * W.nb8 * 64 + (rs & 63)) + (lane & 1);
    }
  }
};

// Issue the loads of group g into ring slot `slot`: five instructions per wave, whatever g.
template <int JS>
__device__ __forceinline__ void sk_issue(const unsigned char* slot, const SkSrc<JS>& src, int g) {
  using S = SkSlot<JS>;
  const int lane = src.lane, wave = src.wave;
  g = g < src.ng ? g : src.ng - 1;
  const uint32_t* scg = src.sc + (size_t)(g >> 1) * 256 + ((g & 1) << 1);   // 64 rows x 4 dwords per uint4 group
  if (JS == 4) {
    // this wave's part of the slot: blocks 4g .. 4g + 3 of chain `wave` (lanes 0..31 and 32..63
    // take one block each per instruction), the 4 blocks' dx, the rows' words and scales
    unsigned char* const w = const_cast<unsigned char*>(slot) + wave * S::WAVE;
    const int last = src.nb - 1;
    const int b0 = min(4 * g + (lane >> 5), last), b1 = min(4 * g + 2 + (lane >> 5), last);
    const int bd = min(4 * g + (lane >> 4), last);
    sk_dma16(src.act + (size_t)b0 * kXhBlock, w);
    sk_dma16(src.act + (size_t)b1 * kXhBlock, w + 1024);
    sk_dma4(src.dx + (size_t)bd * kXhBlock * 4, w + S::oDX);
    if (lane < 16) sk_dma16(src.qs + (size_t)g * 256, w + S::oQS);
    if (lane < 32) sk_dma4(scg, w + S::oSC);
    return;
  }
  int b = 4 * g + wave;
  b = b < src.nb ? b : src.nb - 1;
  const uint4* a = src.act + (size_t)b * kXhBlock;
  sk_dma16(a + lane, slot + wave * 2048);
  sk_dma16(a + 64 + lane, slot + wave * 2048 + 1024);
  if (lane < 16) sk_dma4(reinterpret_cast<const float*>(a + 128) + lane, slot + S::oDX + wave * 64);
  {
    sk_dma16(src.qs + (size_t)g * 256, slot + S::oQS + wave * 1024);
    if (lane < 32) sk_dma4(scg, slot + S::oSC + wave * 128);
  }
}

// The B operand of lane quarter kg for one weight word (4 nibble pairs of one block and chain):
// kg 0 the low nibbles as fp16 1024 + n, kg 1 the high nibbles masked in place (no shift) as
// 1024 + 16 n, kg 2 (1032, 72, 0, 0), kg 3 zero: one and-or and two byte permutes per operand.
struct SkB {
  uint32_t mask, orv, sel0, sel1;
  __device__ __forceinline__ explicit SkB(int kg) {
    mask = kg == 0 ? 0x0F0F0F0Fu : kg == 1 ? 0xF0F0F0F0u : 0u;
    orv = kg == 2 ? 0x54800008u : 0u;                        // bytes of fp16 1032 (0x6408) and 72 (0x5480)
    sel0 = kg < 2 ? 0x04010400u : kg == 2 ? 0x03020400u : 0x0C0C0C0Cu;
    sel1 = kg < 2 ? 0x04030402u : 0x0C0C0C0Cu;
  }
  __device__ __forceinline__ sk_h4 operator()(uint32_t wv) const {
    const uint32_t v = (wv & mask) | orv;
    return __builtin_bit_cast(sk_h4, make_uint2(__builtin_amdgcn_perm(0x64646464u, v, sel0),
                                                __builtin_amdgcn_perm(0x64646464u, v, sel1)));
  }
};

// Workgroups are dispatched to the 8 XCDs (each with its own L2) round robin: workgroup L runs on
// XCD L % 8.  The grid is one-dimensional.  With `by_tile` it maps L to (row group, token tile) so
// that the workgroups sharing a token tile -- and so its activation stream -- run on as few XCDs
// as the balance allows: with a multiple of 8 tiles each tile on one XCD, with 1, 2 or 4 tiles
// each on 8 / tiles XCDs; otherwise row groups run fastest (consecutive workgroups on one tile,
// spread over the XCDs), which keeps a weight matrix larger than an L2 shared by the tiles in
// flight.  Measured on the 1024-token prefill: o/down fetch 5.5 -> 1.4 GB per pass with it, but
// gate/up (4.9 MB of weights) 0.85 -> 7.5 GB, at unchanged kernel times; the host chooses per
// matrix.  A batch step of 2 .. kSkPairTiles token tiles (without by_tile) runs the tiles of one row
// group on one XCD, dispatched 8 workgroups apart: they read the group's weights at the same time
// and the XCD's L2 serves the second reader, where row-group-fastest order with a row-group count
// that is not a multiple of 8 (the output head: 2374 groups of 64 rows) put them on different XCDs
// a whole pass apart.  Returns false for padding workgroups (row group past the last).
constexpr int kXcds = 8;
constexpr int kSkPairTiles = 4;

__host__ __device__ inline bool sk_paired(int ntiles, bool by_tile) {
  return !by_tile && ntiles > 1 && ntiles <= kSkPairTiles;
}

__host__ __device__ inline int sk_grid(int nrg, int ntiles, bool by_tile) {
  if (sk_paired(ntiles, by_tile)) return (nrg + kXcds - 1) / kXcds * kXcds * ntiles;
  if (!by_tile || ntiles % kXcds == 0) return nrg * ntiles;
  if (kXcds % ntiles == 0) {
    const int per = kXcds / ntiles;                 // XCDs per tile
    return (nrg + per - 1) / per * kXcds;
  }
  return nrg * ntiles;
}

__device__ __forceinline__ bool sk_place(int L, int nrg, int ntiles, bool by_tile, int& rg, int& T) {
  const int x = L % kXcds, q = L / kXcds;
  if (sk_paired(ntiles, by_tile)) {
    T = q % ntiles;
    rg = (q / ntiles) * kXcds + x;
    return rg < nrg;
  }
  if (!by_tile) {
    rg = L % nrg;
    T = L / nrg;
    return true;
  }
  if (ntiles % kXcds == 0) {
    T = x + kXcds * (q / nrg);
    rg = q % nrg;
    return true;
  }
  if (kXcds % ntiles == 0) {
    const int per = kXcds / ntiles;
    T = x % ntiles;
    rg = q * per + x / ntiles;
    return rg < nrg;
  }
  rg = L % nrg;
  T = L / nrg;
  return true;
}

template <int OP>
__device__ __forceinline__ void sk_put(float* y, int ldy, const float* bias, int M, int N, int m, int n, float v) {
  if (m < M && n < N) {
    float* o = y + (size_t)m * ldy + n;
    if (OP == 2) *o = *o + v;          // OP_ADD
    else if (OP == 1) *o = v + bias[n];   // OP_BIAS
    else *o = v;                        // OP_STORE
  }
}

// What the fused qkv epilogue (EPI 2) needs besides the projection: RoPE table, the caches and the
// per-token positions of a batch of sequences (token m is sequence m).
struct SkRope {
  const float* rope = nullptr;   // [ctx][hd / 2][2] cos, sin
  void* kc = nullptr;            // sequence m's cache at m * seq_stride: [layer][kv head][ctx][hd]
  void* vc = nullptr;
  const int* pos = nullptr;      // position of token m
  size_t seq_stride = 0;
  int ctx = 0, layer = 0, H = 0, KVH = 0, hd = 0;
  bool kv16 = false;             // fp16 caches (else fp32)
};

// Grid sk_grid(row groups, ceil(M / 16)) (one-dimensional); R * SkSlot<JS>::BYTES of static shared memory.
// xt: the fp16 operands and block scales in the 16-token tiles of quantize_item (kXhBlock).
// The ring slots are R distinct shared arrays and the group loop is unrolled by R, so every slot
// address is a constant.
// EPI = 1 (with JS 1): W is the fused gate|up matrix of ffn rows each, row group = block b of the
// SwiGLU activation; the workgroup's waves 0, 1 take gate rows 32 b .. 32 b + 31 and waves 2, 3 the
// matching up rows, and the epilogue writes act = SwiGLU(gate, up) quantized (block b of xq_out
// and xh_out, what k_quant<QM_SWIGLU> writes) instead of y.
// EPI = 2 (with JS 4): W is the q|k|v matrix of a batch step (OP_BIAS); row groups hold RoPE pairs
// (SkSrc::rope_row) and the epilogue applies RoPE to the q and k heads at each token's position,
// writes q to y and appends k and v to the token's sequence cache (what the bias projection
// followed by k_rope_kv_list writes).
template <int OP, int JS, int R, int EPI = 0>
__global__ __launch_bounds__(256) void k_gemm_sk(Q4Mat W, const uint4* __restrict__ xt, int xstride, int M,
                                                float* __restrict__ y, int ldy, const float* __restrict__ bias,
                                                bool by_tile, uint4* __restrict__ xq_out = nullptr,
                                                uint4* __restrict__ xh_out = nullptr, int ffn = 0,
                                                SkRope rp = SkRope()) {
  static_assert(EPI != 1 || JS == 1, "the SwiGLU epilogue needs the 64-row layout");
  static_assert(EPI != 2 || (JS == 4 && OP == 1), "the RoPE epilogue is the 16-row bias projection");
  using S = SkSlot<JS>;
  static_assert(R >= 3 && R <= 8, "ring depth");
  __shared__ __align__(16) unsigned char q0[S::BYTES], q1[S::BYTES], q2[S::BYTES], q3[S::BYTES], q4[S::BYTES],
      q5[S::BYTES], q6[S::BYTES], q7[S::BYTES];
  unsigned char* const ring[8] = {q0, q1, q2, q3, q4, q5, q6, q7};
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, kg = lane >> 4;
  // nrg row groups (16 rows for JS 4, 64 for JS 1, one 32-value block of gate and up for EPI 1)
  // times ceil(M / 16) token tiles, placed by sk_place
  const int nrg = EPI == 1 ? ffn / 32 : JS == 4 ? W.Np / 16 : W.Np / 64;
  int rgi, T;
  if (!sk_place(blockIdx.x, nrg, (M + 15) / 16, by_tile, rgi, T)) return;
  const int R0 = EPI == 1 ? rgi * 32 : JS == 4 ? rgi * 16 : rgi * 64;
  const int ng = W.ng;
  const SkB bop(kg);
  const SkSrc<JS> src(W, xt, xstride, T, R0, EPI == 1 ? ffn : 0, EPI == 2 ? rp.hd : 0);
  constexpr int NJ = JS == 4 ? 1 : 4;
  const int wrow = JS == 4 ? li : 16 * wave + li;            // this lane's weight row in the workgroup
  float acc[NJ][4];
#pragma unroll
  for (int c = 0; c < NJ; c++) acc[c][0] = acc[c][1] = acc[c][2] = acc[c][3] = 0.0f;

  // What one group needs from its ring slot, in registers.
  struct Regs {
    uint2 sc;              // the 4 fp16 weight scales of this lane's row
    uint4 wq[NJ];          // weight words of the 4 blocks, per chain
    uint2 aw[4][NJ];       // fp16 operands, per block and chain
    float4 dx[4];          // the 4 tokens' block scales, per block
  };
  auto read = [&](const unsigned char* slot, Regs& G) {
    if (JS == 4) slot += wave * S::WAVE;                     // this wave's own part
    const uint2* acts = reinterpret_cast<const uint2*>(slot);
    const float4* dxs = reinterpret_cast<const float4*>(slot + S::oDX);
    const uint4* qss = reinterpret_cast<const uint4*>(slot + S::oQS);
    const uint2* scs = reinterpret_cast<const uint2*>(slot + S::oSC);
    G.sc = scs[wrow];
    if (JS == 4) G.wq[0] = qss[li];
    else {
#pragma unroll
      for (int c = 0; c < 4; c++) G.wq[c] = qss[c * 64 + wrow];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      G.dx[k] = dxs[k * 4 + kg];
#pragma unroll
      for (int c = 0; c < NJ; c++)
        G.aw[k][c] = acts[JS == 4 ? (k * 4 + kg) * 16 + li : ((k * 4 + c) * 4 + kg) * 16 + li];
    }
  };
  // The 4 NJ matrix-core products of group g, then the chain updates in block order.
  auto compute = [&](const Regs& G, int g) {
    auto update = [&](int k, const sk_f4 (&d)[NJ]) {
      const uint32_t sw = (k >> 1) == 0 ? G.sc.x : G.sc.y;
      const float dw = half_bits_to_float((k & 1) ? (sw >> 16) : (sw & 0xffffu));
      const float s0 = dw * G.dx[k].x, s1 = dw * G.dx[k].y, s2 = dw * G.dx[k].z, s3 = dw * G.dx[k].w;
#pragma unroll
      for (int c = 0; c < NJ; c++) {
        acc[c][0] = acc[c][0] + d[c][0] * s0;
        acc[c][1] = acc[c][1] + d[c][1] * s1;
        acc[c][2] = acc[c][2] + d[c][2] * s2;
        acc[c][3] = acc[c][3] + d[c][3] * s3;
      }
    };
    auto product = [&](int k, sk_f4 (&d)[NJ]) {
#pragma unroll
      for (int c = 0; c < NJ; c++) {
        const uint32_t wv = k == 0 ? G.wq[c].x : k == 1 ? G.wq[c].y : k == 2 ? G.wq[c].z : G.wq[c].w;
        d[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(sk_h4, G.aw[k][c]), bop(wv),
                                                     (sk_f4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      }
    };
    // every group is whole (the host takes this kernel only for rows of a multiple of 4 blocks),
    // so the loop is straight-line code with no branch the accumulators would be copied around
    (void)g;
    sk_f4 d[4][NJ];
#pragma unroll
    for (int k = 0; k < 4; k++) product(k, d[k]);
#pragma unroll
    for (int k = 0; k < 4; k++) update(k, d[k]);
  };

#pragma unroll
  for (int p = 0; p < R - 1; p++) sk_issue<JS>(ring[p], src, p);
  if (JS == 4) {
    // Software pipeline over groups (JS 4; the 64-row layout has no registers to spare for it):
    // once group g's slot is free (its reads done), a wave reads group g + 1's operands from
    // shared memory, then computes group g from registers read one step earlier.  R is even, so
    // group g uses register set g & 1 in every pass of the unrolled loop.  The ring is the wave's
    // own: its waits cover its own loads and reads, with no barrier.
    static_assert(R % 2 == 0, "register sets alternate with the group parity");
    Regs G[2];
    sk_wait<5 * (R - 2)>();                                  // group 0 has landed
    sk_issue<JS>(ring[R - 1], src, R - 1);
    read(ring[0], G[0]);
    for (int g0 = 0; g0 < ng; g0 += R) {
#pragma unroll
      for (int u = 0; u < R; u++) {
        const int g = g0 + u;
        if (g < ng) {
          // groups g + 1 .. g + R - 1 are in flight: wait for g + 1; group g's slot has been read
          // (into registers, one step earlier) and takes group g + R
          sk_wait<5 * (R - 2)>();
          // the same wait in a form the compiler's wait tracking sees: the registers read in the
          // previous step are ready, so computing from them does not wait for the reads below
          __builtin_amdgcn_s_waitcnt(0xC07F);                // lgkmcnt(0)
          sk_issue<JS>(ring[u], src, g + R);
          read(ring[(u + 1) % R], G[(u + 1) & 1]);
          compute(G[u & 1], g);
        }
      }
    }
  } else {
    for (int g0 = 0; g0 < ng; g0 += R) {
#pragma unroll
      for (int u = 0; u < R; u++) {
        const int g = g0 + u;
        if (g < ng) {
          // group g's loads were followed by those of R - 2 groups
          sk_sync<5 * (R - 2)>();
          // the slot of group g - 1 is free: every wave has passed the barrier after computing it
          sk_issue<JS>(ring[(u + R - 1) % R], src, g + R - 1);
          Regs G;
          read(ring[u], G);
          compute(G, g);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");          // no load into shared memory outlives the loop
  // lane (li, kg) holds tokens 16 T + 4 kg + r of weight row R0 + wrow
  const int m0 = T * 16 + 4 * kg;
  if (EPI == 1) {
    __syncthreads();
    float* gus = reinterpret_cast<float*>(q0);               // [token 16][local row 64]: gate 0..31, up 32..63
#pragma unroll
    for (int r = 0; r < 4; r++)
      gus[(4 * kg + r) * 64 + 16 * wave + li] = ((acc[0][r] + acc[1][r]) + acc[2][r]) + acc[3][r];
    __syncthreads();
    if (tid < 64) {                                          // wave 0: lane (token t, reference lane j)
      const int t = tid >> 2, j = tid & 3, m = T * 16 + t;
      const int e[8] = {2 * j, 2 * j + 1, 8 + 2 * j, 9 + 2 * j, 16 + 2 * j, 17 + 2 * j, 24 + 2 * j, 25 + 2 * j};
      float g[8], u[8], v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        g[k] = gus[t * 64 + e[k]];
        u[k] = gus[t * 64 + 32 + e[k]];
      }
      swiglu8(g, u, v);
      if (m < M) quantize_item(v, rgi, j, xq_out + (size_t)m * xstride * 4, xh_out + xh_tile(m, xstride), m & 15);
    }
  } else if (JS == 1) {
#pragma unroll
    for (int r = 0; r < 4; r++)
      sk_put<OP>(y, ldy, bias, M, W.N, m0 + r, R0 + 16 * wave + li,
                 ((acc[0][r] + acc[1][r]) + acc[2][r]) + acc[3][r]);
  } else {
    __syncthreads();
    float* red = reinterpret_cast<float*>(q0);               // [chain][token][row] (S::BYTES >= 4 KB)
#pragma unroll
    for (int r = 0; r < 4; r++) red[(wave * 16 + 4 * kg + r) * 16 + li] = acc[0][r];
    __syncthreads();
    const float v = ((red[tid] + red[256 + tid]) + red[512 + tid]) + red[768 + tid];
    if (EPI == 2) {
      // thread tid: token m = 16 T + tid / 16, local row l = tid % 16; rows l and l ^ 8 are a RoPE
      // pair (kernels.c:337-352)
      const int l = tid & 15, m = T * 16 + (tid >> 4), hd = rp.hd, half = hd >> 1;
      const int row = SkSrc<4>::rope_row(rgi, hd, l);
      const float x = v + (row < W.N ? bias[row] : 0.0f);
      const float xo = __shfl_xor(x, 8);                     // the pair's other value, same token
      if (m < M && row < W.N) {
        const int head = row / hd, e = row - head * hd, i = e < half ? e : e - half;
        const int p = rp.pos[m];
        float out = x;
        if (head < rp.H + rp.KVH) {
          const float c = rp.rope[(size_t)p * hd + 2 * i], sn = rp.rope[(size_t)p * hd + 2 * i + 1];
          out = e < half ? x * c - xo * sn : x * c + xo * sn;
        }
        if (head < rp.H) {
          y[(size_t)m * ldy + row] = out;
        } else {
          const bool isv = head >= rp.H + rp.KVH;
          const int kh = head - rp.H - (isv ? rp.KVH : 0);
          const size_t off = (size_t)m * rp.seq_stride + (((size_t)rp.layer * rp.KVH + kh) * rp.ctx + p) * hd + e;
          void* cache = isv ? rp.vc : rp.kc;
          if (rp.kv16) reinterpret_cast<_Float16*>(cache)[off] = (_Float16)out;
          else reinterpret_cast<float*>(cache)[off] = out;
        }
      }
    } else {
      sk_put<OP>(y, ldy, bias, M, W.N, T * 16 + (tid >> 4), R0 + (tid & 15), v);
    }
  }
}

}  // namespace q4
