// persistent.h -- the decode step as one persistent launch (one or many greedy steps per launch).
//
// A kernel-per-operation step is ~245 dependent launches of 2.5-20 us each.  Here every workgroup
// (one per CU) stays resident and takes one role for the whole launch:
//   OD  (D/16 WGs)   rows 16w..16w+15 of o and down; owns those rows of the residual x
//   A   (H WGs)      one attention head: its q rows, RoPE, the scores over past positions, then
//                    the current position's from the new K row, softmax and P.V
//   KV  (2 KVH WGs)  the new K (with RoPE) or V row of one kv group: its 64 qkv rows, the cache
//                    store, and the row handed to the group's A workgroups, which meanwhile score
//                    the past positions
//   GU  (F/32 WGs)   gate and up rows of one 32-value block of the SwiGLU activation, quantized
//   all              the output head (row groups round-robin), then the greedy argmax
// Five exchanges per layer (x after down -> A and KV, new K/V -> A, att -> OD, x after o -> GU,
// act -> OD) and one per step (argmax).  Each exchanged value is stored together with the epoch of
// the phase that wrote it in one 8-byte agent-scope store ("LL" store): a reader polls the data
// itself, so a hand-off is one hop, and a thread's entries are all in flight at once.  Every role issues the loads of its
// next weights, norm weights and biases (and the attention role its past K/V rows) before it
// waits, so that traffic overlaps the waits.  Waits are bounded: a timeout raises State::abort and
// every workgroup exits.
//
// The kernel is compiled for one model shape (PShape): every loop over blocks, groups and rows has
// a constant trip count and is unrolled into straight-line code with no per-term branches, and the
// split of o and down over the four waves is fixed per wave.
//
// Arithmetic per output is the one of kernels.h (the reference's lane order), so results are
// bit-identical to the kernel-per-operation path.
#pragma once
#include "gemm_sk.h"
#include "kernels.h"

namespace q4 {

struct LayerView {
  Q4Mat qkv, o, gu, down;
  const float* attn_norm;
  const float* ffn_norm;
  const float* bqkv;
};

struct PArgs {
  int V, NL, ctx;
  float eps;
  const uint8_t* embd;
  const float* out_norm;
  Q4Mat head;       // Q4_0 layout, or the Q8_0 layout of k_repack_q8 when head_q8
  int head_q8;
  const LayerView* layers;
  const float* rope;
  void* kc;        // the K/V cache: fp32, or fp16 in the kernels instantiated for it
  void* vc;
  float* logits;
  int* tokens;
  State* st;
  uint64_t* ll;   // exchange area, offsets in PShape
  int steps;
  int kv_tile;    // past positions of K and V the attention role stages in shared memory
  int ring;       // slots (kRingRows positions each) of the ring that streams the rest: 3 or 7
  int nap;        // sleep between polls of a wait, in units of 64 cycles
  int asplit;     // attention workgroups per head: 1, or 2 for long contexts -- the pair splits the
                  // past positions for the scores (exchanged through lsc) and the 64 output
                  // columns for P.V, so each streams half of K and half of V
  uint64_t* lsc;  // [H][ctx] score entries of the pair exchange (asplit 2)
  unsigned long long* prof;   // optional: phase timestamps of step 0, [(NL + 1) * 16]
  // Delay, in units of 512 cycles, between a role's hand-off and the loads of its next phase's
  // weights: [0] o/down role before the o weights, [1] before the down weights, [2] attention and
  // K/V roles, [3] gate/up role.  The weight bursts then stay out of the memory system while the
  // hand-off they follow is polled for.
  int pf[4];
  const int* wgmap;   // physical workgroup -> logical one (the role order below); identity when null
  int hres;           // row groups of the Q4_0 head each wave outside the attention role keeps in
                      // shared memory for the whole launch (0: the head is streamed whole every step)
};

// This workgroup's logical index.  The host places the attention workgroups of one kv group on one
// XCD (workgroup L runs on XCD L mod 8), so the past K/V rows they all stage come from that XCD's L2
// after the first of them has fetched them.
__device__ __forceinline__ int lwg(const PArgs& a) {
  return a.wgmap ? __builtin_amdgcn_readfirstlane(a.wgmap[blockIdx.x]) : (int)blockIdx.x;
}

__device__ __forceinline__ void pf_delay(int n) {
  for (int i = 0; i < n; i++) __builtin_amdgcn_s_sleep(8);
}

constexpr int kPThreads = 256;
constexpr int kSpinLimit = 1 << 21;
constexpr int kHD = 64;           // head_dim of the persistent path
constexpr int kKVRow = 68;        // floats per staged K/V row (64 + 4: conflict-free row-per-thread reads)

// Even-aligned split of ng groups of 4 blocks over the four waves: wave w takes
// [split_g0, split_g0 + split_cnt).  Even starts keep a wave's fp16 scales in whole uint4 words.
constexpr int split_per(int ng) { return (((ng + 3) >> 2) + 1) & ~1; }
constexpr int split_g0(int ng, int w) { return w * split_per(ng); }
constexpr int split_cnt(int ng, int w) {
  return ng - split_g0(ng, w) <= 0 ? 0 : (ng - split_g0(ng, w) < split_per(ng) ? ng - split_g0(ng, w) : split_per(ng));
}

constexpr int kActStride = 16;    // exchange entries per GU workgroup's 9 activation entries

// Activation entry i (block i / 9, word i % 9) in the exchange area.
struct ActEntry {
  __device__ int operator()(int i) const { return (i / 9) * kActStride + i % 9; }
};
constexpr int kArgStride = 16;    // exchange entries per workgroup's (max, index) pair: a line each

// Entry i of the argmax exchange (workgroup i / 2, word i % 2).
struct ArgEntry {
  __device__ int operator()(int i) const { return (i >> 1) * kArgStride + (i & 1); }
};

struct SameEntry {
  __device__ int operator()(int i) const { return i; }
};

// The model shape a persistent kernel is compiled for (head_dim 64).
template <int D_, int F_, int H_, int KVH_>
struct PShape {
  static constexpr int D = D_, F = F_, H = H_, KVH = KVH_;
  static constexpr int NBD = D / 32, NBF = F / 32, NBM = NBD > NBF ? NBD : NBF;
  static constexpr int NGD = (NBD + 3) / 4, NGF = (NBF + 3) / 4;      // groups of 4 blocks
  static constexpr int NB8D = (NBD + 7) / 8, NB8F = (NBF + 7) / 8;    // uint4 words of 8 scales
  static constexpr int nOD = D / 16, nA = H, nKV = 8 * KVH, nGU = F / 32, nRoles = nOD + nA + nKV + nGU;
  static constexpr int KD = (D + kPThreads - 1) / kPThreads;           // x entries per thread
  static constexpr int NACT = 9 * nGU;                                 // act entries
  static constexpr int KACT = (NACT + kPThreads - 1) / kPThreads;
  static constexpr int STV = D / 4 + 4;                                // stride of the lane runs
  // exchange area, in 8-byte entries: x after o, x after down, x into the head, attention
  // output, quantized activation, the new K and V rows of each kv group ([group][k, v][64]), then
  // two (value, index) argmax buffers used by step parity.
  // Every producer writes whole 128-byte lines (16 entries), each with one store instruction: a
  // line written piecewise (by several waves or workgroups) reaches its readers ~0.3-0.7 us later.
  // The 9 activation entries of a GU workgroup fill a line with padding (kActStride entries), and
  // each K/V workgroup's 16 rows form one line.
  static constexpr int oX1 = 0, oX2 = D, oXH = 2 * D, oATT = 3 * D, oACT = 4 * D;
  static constexpr int oKV = oACT + kActStride * nGU, oARG = oKV + 2 * KVH * kHD;
  static constexpr size_t ll_entries(int G) { return (size_t)oARG + 2 * (size_t)kArgStride * G; }
  static constexpr int RAW = NACT > 2 * kPThreads ? NACT : 2 * kPThreads;   // raw entry words
  static_assert(D % 64 == 0 && F % 32 == 0 && D == H * kHD && H % KVH == 0, "unsupported shape");
  static_assert(D <= 4 * kPThreads, "norm_quant gives half a block lane per thread");
};

// ---------------------------------------------------------------- memory helpers

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) const u32x4 GlobalU32x4;
typedef __attribute__((address_space(1))) const f32x4 GlobalF32x4;
typedef __attribute__((address_space(1))) const f32x2 GlobalF32x2;
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
__device__ __forceinline__ float2 gld2f(const float* p) {
  const f32x2 v = *(GlobalF32x2*)(const void*)p;
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ float gldf(const float* p) { return *(GlobalF32*)(const void*)p; }

__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(kvhalf* p, float v) {
  const kvhalf hv = (kvhalf)v;
  __hip_atomic_store((unsigned short*)p, __builtin_bit_cast(unsigned short, hv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four consecutive K/V cache elements, widened to fp32.
__device__ __forceinline__ float4 kv_gld4(const float* p) { return gld4f(p); }
__device__ __forceinline__ float4 kv_gld4(const kvhalf* p) {
  typedef __attribute__((address_space(1))) const unsigned int GlobalU32;
  const unsigned int a = ((GlobalU32*)(const void*)p)[0], b = ((GlobalU32*)(const void*)p)[1];
  return make_float4(half_bits_to_float(a & 0xffffu), half_bits_to_float(a >> 16), half_bits_to_float(b & 0xffffu),
                     half_bits_to_float(b >> 16));
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// ---------------------------------------------------------------- LL exchange

__device__ __forceinline__ void ll_put(uint64_t* p, uint32_t payload, uint32_t ep) {
  __hip_atomic_store(p, ((uint64_t)ep << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ll_peek(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait for entries base[at(tid + 256k)] (k < K, tid + 256k < n) to carry epoch ep.  All K loads are in
// flight together and only the entries still missing are polled again, so a hand-off costs one
// memory round trip however many entries a thread receives; between polls the wave sleeps
// `nap` x 64 cycles (polls of every waiting workgroup share the memory system with the weight
// stream).  Bounded: after kSpinLimit polls the thread raises st->abort; a raised flag makes
// every waiter give up (`bad`).
template <int K, class At = SameEntry>
__device__ __forceinline__ void ll_recv(const uint64_t* base, int n, uint32_t ep, State* st, bool& bad,
                                        uint32_t (&out)[K], int nap, At at = At()) {
  uint64_t w[K];
#pragma unroll
  for (int k = 0; k < K; k++) {
    const int i = (int)threadIdx.x + kPThreads * k;
    w[k] = i < n ? ll_peek(base + at(i)) : ((uint64_t)ep << 32);
  }
  int spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < K; k++) ok = ok && (uint32_t)(w[k] >> 32) == ep;
    if (ok || bad) break;
    for (int z = 0; z < nap; z++) __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < K; k++) {
      const int i = (int)threadIdx.x + kPThreads * k;
      if (i < n && (uint32_t)(w[k] >> 32) != ep) w[k] = ll_peek(base + at(i));
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

// Complete a wait for one entry whose first poll `w` was issued earlier (ll_recv's loop for K = 1).
__device__ __forceinline__ void ll_wait1(const uint64_t* p, uint64_t& w, uint32_t ep, State* st, bool& bad, int nap) {
  int spins = 0;
  while ((uint32_t)(w >> 32) != ep && !bad) {
    for (int z = 0; z < nap; z++) __builtin_amdgcn_s_sleep(1);
    w = ll_peek(p);
    if (++spins > kSpinLimit) {
      bad = true;
      __hip_atomic_store(&st->abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if ((spins & 255) == 0 && __hip_atomic_load(&st->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      bad = true;
    }
  }
}

// The workgroup-uniform "give up" decision after a wait: a thread whose wait gave up raises the
// shared flag before the barrier, every thread reads it after.  One barrier and one shared-memory
// read, where __syncthreads_or takes three of each.  The flag is cleared once per launch and never
// lowered: a raised flag ends the launch.
__device__ __forceinline__ bool wg_bad(int* flag, bool bad) {
  if (bad) *(volatile int*)flag = 1;
  lds_barrier();
  return *(volatile int*)flag != 0;
}

// ---------------------------------------------------------------- register-resident weights

// CNT groups of one 16-row group, lane (r = lane/4, j = lane%4): word j of 4 blocks per group and
// the fp16 scales of 8 blocks per uint4.
template <int CNT>
struct WR {
  uint4 w[CNT > 0 ? CNT : 1];
  uint4 s[CNT > 0 ? (CNT + 1) / 2 : 1];
};

// Groups [G0, G0 + CNT) (G0 even) of row group rg16 of a matrix with NG groups and NB8 scale words
// per row.
template <int NG, int NB8, int G0, int CNT>
__device__ __forceinline__ void wr_load(const Q4Mat& W, int rg16, int lane, WR<CNT>& R) {
  if constexpr (CNT > 0) {
    const int row = rg16 * 16 + (lane >> 2), j = lane & 3;
    const int tile = row >> 6, rr = row & 63;
    const uint4* wq = W.qs + ((size_t)tile * NG * 64 + rr) * 4 + j + (size_t)G0 * 256;
    const uint4* wd = W.d + ((size_t)tile * NB8 + G0 / 2) * 64 + rr;
#pragma unroll
    for (int g = 0; g < CNT; g++) R.w[g] = gld(wq + (size_t)g * 256);
#pragma unroll
    for (int c = 0; c < (CNT + 1) / 2; c++) R.s[c] = gld(wd + (size_t)c * 64);
  }
}

// The same for the row `row` of this lane (lane j = lane % 4 of it), any row of a 64-row tile.
template <int NG, int NB8, int G0, int CNT>
__device__ __forceinline__ void wr_load_row(const Q4Mat& W, int row, int lane, WR<CNT>& R) {
  if constexpr (CNT > 0) {
    const int j = lane & 3, tile = row >> 6, rr = row & 63;
    const uint4* wq = W.qs + ((size_t)tile * NG * 64 + rr) * 4 + j + (size_t)G0 * 256;
    const uint4* wd = W.d + ((size_t)tile * NB8 + G0 / 2) * 64 + rr;
#pragma unroll
    for (int g = 0; g < CNT; g++) R.w[g] = gld(wq + (size_t)g * 256);
#pragma unroll
    for (int c = 0; c < (CNT + 1) / 2; c++) R.s[c] = gld(wd + (size_t)c * 64);
  }
}

// Terms f32(p_j) * (dw * dx) (kernels.c:137) of the 4 blocks of local group g for N row groups,
// xv[k] = {A_j, B_j, c_j, dx} of block k.  Computed stage by stage (all low-nibble dots, all
// high-nibble dots, then the products) so that the independent blocks and rows interleave; each
// term's own operation order is unchanged.  Blocks past NB (b >= NB) are skipped.
template <int NB, int G0, int CNT, int N>
__device__ __forceinline__ void wr_group_terms(const WR<CNT> (&R)[N], int g, const uint4 (&xv)[4],
                                               float (&t)[N][4]) {
  int p[N][4];
#pragma unroll
  for (int n = 0; n < N; n++)
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if ((G0 + g) * 4 + k < NB) {
        const uint32_t wv = k == 0 ? R[n].w[g].x : k == 1 ? R[n].w[g].y : k == 2 ? R[n].w[g].z : R[n].w[g].w;
        p[n][k] = sdot4(wv & 0x0F0F0F0Fu, xv[k].x, (int)xv[k].z);
      }
    }
#pragma unroll
  for (int n = 0; n < N; n++)
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if ((G0 + g) * 4 + k < NB) {
        const uint32_t wv = k == 0 ? R[n].w[g].x : k == 1 ? R[n].w[g].y : k == 2 ? R[n].w[g].z : R[n].w[g].w;
        p[n][k] = sdot4((wv >> 4) & 0x0F0F0F0Fu, xv[k].y, p[n][k]);
      }
    }
#pragma unroll
  for (int n = 0; n < N; n++)
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if ((G0 + g) * 4 + k < NB) {
        const uint4 sv = R[n].s[g >> 1];
        const int hb = ((g & 1) << 2) + k;
        const uint32_t sw = (hb >> 1) == 0 ? sv.x : (hb >> 1) == 1 ? sv.y : (hb >> 1) == 2 ? sv.z : sv.w;
        const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
        t[n][k] = (float)p[n][k] * (dw * __uint_as_float(xv[k].w));
      }
    }
}

// Mark a value as used here: the loads that produced it complete before this point, and code after
// it stays after it.  Used to software-pipeline shared-memory reads: the next chunk's loads are
// issued, then the current chunk is pinned, then computed, so the compiler can neither wait for
// the newer loads early nor issue them late.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
__device__ __forceinline__ void pin(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }

// Activation blocks of local group g (xq[b * 4 + j]); zero past NB.
template <int NB, int G0>
__device__ __forceinline__ void xg_load(const uint4* xq, int g, int j, uint4 (&xv)[4]) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int b = (G0 + g) * 4 + k;
    xv[k] = b < NB ? xq[b * 4 + j] : make_uint4(0, 0, 0, 0);
  }
}

// The term f32(p_j) * (dw * dx) (kernels.c:137) of block k (0..3) of local group g of one 16-row
// group, xv = {A_j, B_j, c_j, dx} of the block: the arithmetic of wr_group_terms for one block.
template <int CNT>
__device__ __forceinline__ float wr_term(const WR<CNT>& R, int g, int k, const uint4& xv) {
  const uint4 w = R.w[g];
  const uint32_t wv = k == 0 ? w.x : k == 1 ? w.y : k == 2 ? w.z : w.w;
  const uint4 sv = R.s[g >> 1];
  const int hb = ((g & 1) << 2) + k;
  const uint32_t sw = (hb >> 1) == 0 ? sv.x : (hb >> 1) == 1 ? sv.y : (hb >> 1) == 2 ? sv.z : sv.w;
  int p = sdot4(wv & 0x0F0F0F0Fu, xv.x, (int)xv.z);
  p = sdot4((wv >> 4) & 0x0F0F0F0Fu, xv.y, p);
  const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
  return (float)p * (dw * __uint_as_float(xv.w));
}

// acc = acc + term over blocks [4 G0, min(NB, 4 (G0 + CNT))) in order (kernels.c:217-218) for one
// 16-row group, software pipelined by hand: the activation reads run two groups ahead, and each
// addition of group g alternates with one block's term of group g + 1 (the pins fix that order;
// the scheduler would otherwise put a group's dependent additions after the next group's terms).
template <int NB, int G0, int CNT, int N>
__device__ __forceinline__ void wr_dot(const WR<CNT> (&R)[N], const uint4* xq, int j, float (&acc)[N]) {
  static_assert(N == 1, "one row group");
  if constexpr (CNT > 0) {
    uint4 xb[2][4];
    float t[2][4];
    xg_load<NB, G0>(xq, 0, j, xb[0]);
    if (CNT > 1) xg_load<NB, G0>(xq, 1, j, xb[1]);
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (G0 * 4 + k < NB) {
        t[0][k] = wr_term<CNT>(R[0], 0, k, xb[0][k]);
        pin(t[0][k]);
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < CNT; g++) {
      if (g + 2 < CNT) xg_load<NB, G0>(xq, g + 2, j, xb[g & 1]);
      const int n = (g + 1) & 1;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if ((G0 + g) * 4 + k < NB) {
          acc[0] = acc[0] + t[g & 1][k];
          pin(acc[0]);
        }
        if (g + 1 < CNT && (G0 + g + 1) * 4 + k < NB) {
          t[n][k] = wr_term<CNT>(R[0], g + 1, k, xb[n][k]);
          pin(t[n][k]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The same terms written to shared memory, terms[b * 64 + lane], for a serial pass by one wave.
template <int NB, int G0, int CNT>
__device__ __forceinline__ void wr_terms(const WR<CNT>& R, const uint4* xq, int lane, float* terms) {
  if constexpr (CNT > 0) {
    const WR<CNT> RR[1] = {R};
    uint4 xb[2][4];
    xg_load<NB, G0>(xq, 0, lane & 3, xb[0]);
#pragma unroll
    for (int g = 0; g < CNT; g++) {
      if (g + 1 < CNT) xg_load<NB, G0>(xq, g + 1, lane & 3, xb[(g + 1) & 1]);
#pragma unroll
      for (int k = 0; k < 4; k++) pin(xb[g & 1][k]);
      float t[1][4];
      wr_group_terms<NB, G0, CNT, 1>(RR, g, xb[g & 1], t);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int b = (G0 + g) * 4 + k;
        if (b < NB) terms[b * 64 + lane] = t[0][k];
      }
    }
  }
}

// ((0 + t_0) + t_1) + ... + t_{NB-1}: the accumulation order of one reference lane, reading
// terms[b * 64 + lane] 8 blocks ahead of the additions.
template <int NB>
__device__ __forceinline__ float serial_sum(const float* terms, int lane) {
  constexpr int C = 8, NC = (NB + C - 1) / C;
  float buf[2][C];
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < C; u++)
    if (u < NB) buf[0][u] = terms[u * 64 + lane];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    if (c + 1 < NC) {
#pragma unroll
      for (int u = 0; u < C; u++)
        if ((c + 1) * C + u < NB) buf[(c + 1) & 1][u] = terms[((c + 1) * C + u) * 64 + lane];
    }
#pragma unroll
    for (int u = 0; u < C; u++)
      if (c * C + u < NB) pin(buf[c & 1][u]);
#pragma unroll
    for (int u = 0; u < C; u++)
      if (c * C + u < NB) acc = acc + buf[c & 1][u];
  }
  return acc;
}

// ((0 + x_0) + x_1) + ... over a contiguous run of N floats (N a multiple of 16, 16-byte
// aligned), 16 values read ahead of the additions.
template <int N>
__device__ __forceinline__ float run_sum(const float* run) {
  static_assert(N % 16 == 0, "run length");
  constexpr int NC = N / 16;
  const float4* p = reinterpret_cast<const float4*>(run);
  // chunks stream through three register sets, two chunks ahead of the additions; the scheduling
  // fences keep each chunk's reads in place (issued all at once, the reads of the whole run would
  // delay the first addition by ~0.4 us), and pinning s keeps each chunk's additions in place
  float4 buf[3][4];
#pragma unroll
  for (int c = 0; c < 2 && c < NC; c++) {
#pragma unroll
    for (int u = 0; u < 4; u++) buf[c][u] = p[c * 4 + u];
    __builtin_amdgcn_sched_barrier(0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    if (c + 2 < NC) {
#pragma unroll
      for (int u = 0; u < 4; u++) buf[(c + 2) % 3][u] = p[(c + 2) * 4 + u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      s = s + buf[c % 3][u].x;
      s = s + buf[c % 3][u].y;
      s = s + buf[c % 3][u].z;
      s = s + buf[c % 3][u].w;
    }
    pin(s);
    __builtin_amdgcn_sched_barrier(0);
  }
  return s;
}

// Serial sums over values in shared memory, in index order.  Each loop iteration reads two chunks
// of 16 values (the second chunk's reads kept after the first's, so the first can be used while
// the second is in flight) and adds them; nothing is carried across the loop's back edge, so the
// compiler's waits stay exact.  The last partial chunk is added under selects.

// ((0 + x_0) + x_1) + ... + x_{n-1}, x 16-byte aligned and readable up to the next multiple of 16
// past n.
__device__ __forceinline__ float seq_sum(const float* x, int n) {
  const float4* p = reinterpret_cast<const float4*>(x);
  const int nc = n >> 4;
  float s = 0.0f;
  int c = 0;
  for (; c + 2 <= nc; c += 2) {
    float4 A[4], B[4];
#pragma unroll
    for (int u = 0; u < 4; u++) A[u] = p[c * 4 + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) B[u] = p[c * 4 + 4 + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) { s = s + A[u].x; s = s + A[u].y; s = s + A[u].z; s = s + A[u].w; }
#pragma unroll
    for (int u = 0; u < 4; u++) { s = s + B[u].x; s = s + B[u].y; s = s + B[u].z; s = s + B[u].w; }
  }
  float4 A[4], B[4];
  const int ca = c < nc ? c : nc;
#pragma unroll
  for (int u = 0; u < 4; u++) A[u] = p[ca * 4 + u];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < 4; u++) B[u] = p[nc * 4 + u];
  __builtin_amdgcn_sched_barrier(0);
  if (c < nc) {
#pragma unroll
    for (int u = 0; u < 4; u++) { s = s + A[u].x; s = s + A[u].y; s = s + A[u].z; s = s + A[u].w; }
  }
  const int r = n - (nc << 4);
#pragma unroll
  for (int u = 0; u < 4; u++) {
    float t;
    t = s + B[u].x; s = 4 * u + 0 < r ? t : s;
    t = s + B[u].y; s = 4 * u + 1 < r ? t : s;
    t = s + B[u].z; s = 4 * u + 2 < r ? t : s;
    t = s + B[u].w; s = 4 * u + 3 < r ? t : s;
  }
  return s;
}

// acc = ((acc + p_0 * v_0) + p_1 * v_1) + ... over t in [0, n), p and v contiguous in shared
// memory, 16-byte aligned, readable up to the next multiple of 16 past n.
__device__ __forceinline__ float seq_dot4(float acc, const float* p, const float* v, int n) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const int nc = n >> 4;
  int c = 0;
  for (; c + 2 <= nc; c += 2) {
    float4 pa[4], va[4], pb[4], vb[4];
#pragma unroll
    for (int u = 0; u < 4; u++) { pa[u] = p4[c * 4 + u]; va[u] = v4[c * 4 + u]; }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) { pb[u] = p4[c * 4 + 4 + u]; vb[u] = v4[c * 4 + 4 + u]; }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      acc = acc + pa[u].x * va[u].x;
      acc = acc + pa[u].y * va[u].y;
      acc = acc + pa[u].z * va[u].z;
      acc = acc + pa[u].w * va[u].w;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      acc = acc + pb[u].x * vb[u].x;
      acc = acc + pb[u].y * vb[u].y;
      acc = acc + pb[u].z * vb[u].z;
      acc = acc + pb[u].w * vb[u].w;
    }
  }
  float4 pa[4], va[4], pb[4], vb[4];
  const int ca = c < nc ? c : nc;
#pragma unroll
  for (int u = 0; u < 4; u++) { pa[u] = p4[ca * 4 + u]; va[u] = v4[ca * 4 + u]; }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < 4; u++) { pb[u] = p4[nc * 4 + u]; vb[u] = v4[nc * 4 + u]; }
  __builtin_amdgcn_sched_barrier(0);
  if (c < nc) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      acc = acc + pa[u].x * va[u].x;
      acc = acc + pa[u].y * va[u].y;
      acc = acc + pa[u].z * va[u].z;
      acc = acc + pa[u].w * va[u].w;
    }
  }
  const int r = n - (nc << 4);
#pragma unroll
  for (int u = 0; u < 4; u++) {
    float t;
    t = acc + pb[u].x * vb[u].x; acc = 4 * u + 0 < r ? t : acc;
    t = acc + pb[u].y * vb[u].y; acc = 4 * u + 1 < r ? t : acc;
    t = acc + pb[u].z * vb[u].z; acc = 4 * u + 2 < r ? t : acc;
    t = acc + pb[u].w * vb[u].w; acc = 4 * u + 3 < r ? t : acc;
  }
  return acc;
}

// Running sums over values in shared memory with the reads of the next 32 values in flight while
// the current 32 are added (two register batches; the loop carries one batch of reads across its
// back edge).  The values past n up to the next multiple of 32 must be +0: the running sums start
// at +0 and round to nearest, so they never become -0, and adding +0 (or a -0 product) leaves them
// unchanged -- the result is the reference's n-term sum exactly.

// ((0 + x_0) + x_1) + ... + x_{n-1}, x 16-byte aligned.
__device__ __forceinline__ float chain_sum(const float* x, int n) {
  const float4* p = reinterpret_cast<const float4*>(x);
  const int nb = (n + 31) >> 5;
  float s = 0.0f;
  if (nb == 0) return s;
  float4 A[8], B[8];
#pragma unroll
  for (int u = 0; u < 8; u++) A[u] = p[u];
  for (int c = 0;; c += 2) {
    const int c1 = c + 1 < nb ? c + 1 : c;
#pragma unroll
    for (int u = 0; u < 8; u++) B[u] = p[c1 * 8 + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; u++) { s = s + A[u].x; s = s + A[u].y; s = s + A[u].z; s = s + A[u].w; }
    if (c + 1 >= nb) break;
    const int c2 = c + 2 < nb ? c + 2 : c + 1;
#pragma unroll
    for (int u = 0; u < 8; u++) A[u] = p[c2 * 8 + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; u++) { s = s + B[u].x; s = s + B[u].y; s = s + B[u].z; s = s + B[u].w; }
    if (c + 2 >= nb) break;
  }
  return s;
}

// ((0 + p_0 * v_0) + p_1 * v_1) + ... over t < n (each product rounded, then added), p and v
// 16-byte aligned; p (and v) zero past n up to the next multiple of 32.
__device__ __forceinline__ float chain_dot(const float* pp, const float* vv, int n) {
  const float4* p = reinterpret_cast<const float4*>(pp);
  const float4* v = reinterpret_cast<const float4*>(vv);
  const int nb = (n + 31) >> 5;
  float s = 0.0f;
  if (nb == 0) return s;
  float4 PA[8], VA[8], PB[8], VB[8];
#pragma unroll
  for (int u = 0; u < 8; u++) { PA[u] = p[u]; VA[u] = v[u]; }
  for (int c = 0;; c += 2) {
    const int c1 = c + 1 < nb ? c + 1 : c;
#pragma unroll
    for (int u = 0; u < 8; u++) { PB[u] = p[c1 * 8 + u]; VB[u] = v[c1 * 8 + u]; }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; u++) {
      s = s + PA[u].x * VA[u].x; s = s + PA[u].y * VA[u].y; s = s + PA[u].z * VA[u].z; s = s + PA[u].w * VA[u].w;
    }
    if (c + 1 >= nb) break;
    const int c2 = c + 2 < nb ? c + 2 : c + 1;
#pragma unroll
    for (int u = 0; u < 8; u++) { PA[u] = p[c2 * 8 + u]; VA[u] = v[c2 * 8 + u]; }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; u++) {
      s = s + PB[u].x * VB[u].x; s = s + PB[u].y * VB[u].y; s = s + PB[u].z * VB[u].z; s = s + PB[u].w * VB[u].w;
    }
    if (c + 2 >= nb) break;
  }
  return s;
}

__device__ __forceinline__ float embed_value(const uint8_t* emb, int D, int t, int i) {
  const uint8_t* bp = emb + ((size_t)t * (D / 32) + (i >> 5)) * 18;
  const float d = half_bits_to_float((uint32_t)bp[0] | ((uint32_t)bp[1] << 8));
  const int e = i & 31;
  const int q = bp[2 + (e & 15)];
  return (float)((e < 16 ? (q & 15) : (q >> 4)) - 8) * d;
}

// Quantize one 32-block (quantize_row, kernels.c:90-114) by half block lanes: block lane j of
// block b owns elements {2j, 2j+1, 8+2j, 9+2j} (word 0) and {16+2j, 17+2j, 24+2j, 25+2j} (word 1);
// thread 2l + h holds the four values of word h of block lane l = 4b + j, so the eight threads of
// a block are consecutive.  The block maximum is an 8-lane reduction, and the pair combines its
// words and sums by a lane swap.  The h = 0 thread gets block lane l's activation entry:
// {word 0, word 1, -8 * (sum of its 8 values), d}.
__device__ __forceinline__ uint4 quant_half(const float (&v)[4]) {
  float am = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) am = __builtin_fmaxf(am, __builtin_fabsf(v[k]));
  am = quad_max(am);
  am = __builtin_fmaxf(am, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(am), 0x141, 0xF, 0xF, true)));
  const float dd = div_127(am);
  const float id = inv_scale(dd);
  int q[4];
#pragma unroll
  for (int k = 0; k < 4; k++) q[k] = quant_one(v[k] * id);
  const uint32_t w = pack4(q[0], q[1], q[2], q[3]);
  const int sum = (q[0] + q[1]) + (q[2] + q[3]);
  const uint32_t wo = (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xB1, 0xF, 0xF, true);
  const int so = __builtin_amdgcn_mov_dpp(sum, 0xB1, 0xF, 0xF, true);
  return make_uint4(w, wo, (uint32_t)(-8 * (sum + so)), __float_as_uint(dd));
}

// Element k (0..7) of block lane t = (block t/4, lane t%4).
__device__ __forceinline__ int lane_elem(int t, int k) {
  return ((t >> 2) << 5) + ((t & 3) << 1) + ((k >> 1) << 3) + (k & 1);
}

// ---------------------------------------------------------------- shared memory plan

struct PSmem {
  float* xl;      // 4 * STV floats: x by lane runs (value i at (i & 3) * STV + (i >> 2)), or plain
  float* sq;      // 4 * STV floats: x*x in the same layout
  uint4* xq;      // NBM * 4 activation block lanes
  uint4* tq;      // 4
  float* red;     // 16
  float* qv;      // 3 * 64: q, k, v of one head
  float* own;     // 16 residual rows (OD)
  float* gu;      // 64: gate, up (GU)
  float* argv;    // 8
  int* argi;      // 8
  uint32_t* raw;  // RAW words: exchange entries
  int* flag;      // the give-up flag of wg_bad (word 7 of red)
  float* terms;   // last: 64 * NBM per-block terms (OD); for the attention role its ctx + 2 kRingRows
                  // scores, then its K/V ring and staged tile
  uint4* hcache;  // the resident head row groups (every role but attention), inside terms' space
};

// Staged K/V of the attention role: K as rows [kv_tile][kKVRow], V transposed [64][kv_vstride]
// (a lane reads its dimension of 4 positions at once; the stride is 4 mod 64 floats, so the 16
// lanes of a 16-byte read hit distinct banks), K readable 16 positions past the tile, V rows
// 32 positions past it.
__host__ __device__ constexpr int kv_vstride(int kv_tile) { return ((kv_tile + 32 + 63) & ~63) + 4; }
__host__ __device__ constexpr size_t kv_lds_bytes(int kv_tile) {
  return kv_tile == 0 ? 0 : ((size_t)(kv_tile + 16) * kKVRow + (size_t)kHD * kv_vstride(kv_tile)) * 4;
}

// Past K/V rows beyond the staged tile are streamed from HBM through a ring of slots of kRingRows
// rows in shared memory, filled by asynchronous global-to-LDS loads (each wave instruction moves
// 4 rows = 1 KB; a slot is 12 instructions).  V slots hold plain rows.  For the scores the same
// memory is split into per-wave rings of 16-row K chunks, each 4-row group in kGrpFloats (16
// floats of padding, see ring_issue_kc): a wave streams and scores its own chunks.
constexpr int kRingRows = 48;
constexpr int kGrpFloats = 4 * kHD + 16;
constexpr int kSlotFloats = kRingRows / 4 * kGrpFloats;
constexpr int kChunkFloats = 4 * kGrpFloats;
// K chunk slots per wave in a ring of `slots` slots (5 of 7, 2 of 3)
__host__ __device__ constexpr int kchunk_slots(int slots) { return 3 * slots / 4; }
static_assert(4 * kchunk_slots(7) * kChunkFloats <= 7 * kSlotFloats, "per-wave K rings exceed the ring");
static_assert(4 * kchunk_slots(3) * kChunkFloats <= 3 * kSlotFloats, "per-wave K rings exceed the ring");
__host__ __device__ constexpr size_t ring_lds_bytes(int slots) { return (size_t)slots * kSlotFloats * 4; }

template <class S>
constexpr size_t psmem_terms_offset() {
  return (size_t)8 * S::STV * 4 + (size_t)S::NBM * 64 + (size_t)(16 + 16 + 192 + 16 + 64 + 8 + 8) * 4 +
         (size_t)S::RAW * 4;
}

template <class S>
constexpr size_t psmem_base_bytes() {
  return psmem_terms_offset<S>() + (size_t)64 * S::NBM * 4;
}

// What the attention role uses: its scores and their exponentials (ctx + 2 kRingRows floats each,
// 16-byte aligned), then the ring and the staged tile.  They overlap the other roles' term buffer, not anything it shares.
__host__ __device__ constexpr size_t attn_scores_floats(int ctx) { return (size_t)((ctx + 2 * kRingRows + 32 + 3) & ~3); }

template <class S>
constexpr size_t psmem_attn_bytes(int ctx, int ring_slots, int kv_tile) {
  return psmem_terms_offset<S>() + 2 * attn_scores_floats(ctx) * 4 + ring_lds_bytes(ring_slots) +
         kv_lds_bytes(kv_tile);
}

// Resident row groups of the output head, after the K/V role's term buffer (the last shared-memory
// use of the roles outside attention).  One row group holds a wave's WR<NGD> registers: word j of
// the 4 blocks of group g for lane l at uint4 g * 64 + l, then scale word c of row r at uint4
// NGD * 64 + c * 16 + r (64 uint4, one load instruction's worth).  Wave w's k-th row group is
// slot w * hres + k.
template <class S>
constexpr size_t head_cache_offset() {
  return (psmem_terms_offset<S>() + (size_t)64 * S::NBD * 4 + 15) & ~(size_t)15;
}
template <class S>
constexpr size_t head_rg_bytes() { return ((size_t)S::NGD * 64 + 64) * 16; }

template <class S>
__device__ __forceinline__ PSmem psmem(unsigned char* base) {
  PSmem m;
  size_t off = 0;
  m.xl = (float*)(base + off);      off += (size_t)4 * S::STV * 4;
  m.sq = (float*)(base + off);      off += (size_t)4 * S::STV * 4;
  m.xq = (uint4*)(base + off);      off += (size_t)S::NBM * 64;
  m.tq = (uint4*)(base + off);      off += 16 * 4;
  m.red = (float*)(base + off);     off += 16 * 4;
  m.qv = (float*)(base + off);      off += 192 * 4;
  m.own = (float*)(base + off);     off += 16 * 4;
  m.gu = (float*)(base + off);      off += 64 * 4;
  m.argv = (float*)(base + off);    off += 8 * 4;
  m.argi = (int*)(base + off);      off += 8 * 4;
  m.raw = (uint32_t*)(base + off);  off += (size_t)S::RAW * 4;
  m.flag = (int*)(m.red + 7);
  m.terms = (float*)(base + off);
  m.hcache = (uint4*)(base + head_cache_offset<S>());
  return m;
}

__device__ __forceinline__ uint32_t phase_epoch(uint32_t ep0, int s, int E, int code) {
  return ep0 + (uint32_t)(s * E + code) + 1u;
}

__device__ __forceinline__ void prof_mark(const PArgs& a, int s, int slot) {
  if (a.prof && s == 0 && threadIdx.x == 0) a.prof[slot] = wall_clock64();
}

// Per-workgroup timestamps of step 0, after the (NL + 1) * 16 phase slots: [layer][workgroup][8].
constexpr int kProfWG = 8;
__device__ __forceinline__ unsigned long long* prof_slot(const PArgs& a, int s, int l, int k) {
  return a.prof && s == 0 ? a.prof + (size_t)(a.NL + 1) * 16 + ((size_t)l * gridDim.x + lwg(a)) * kProfWG + k
                          : nullptr;
}
// The per-workgroup timestamp k once `v` has been computed (the empty asm consumes v and the
// timestamp is read after it); outstanding memory operations are not waited for.
__device__ __forceinline__ void prof_after(const PArgs& a, int s, int l, int k, float v) {
  if (a.prof && s == 0) {
    asm volatile("" ::"v"(v));
    *prof_slot(a, s, l, k) = wall_clock64();
  }
}
__device__ __forceinline__ void prof_wg(const PArgs& a, int s, int l, int k) {
  if (a.prof && s == 0 && threadIdx.x == 0)
    a.prof[(size_t)(a.NL + 1) * 16 + ((size_t)l * gridDim.x + lwg(a)) * kProfWG + k] = wall_clock64();
}

// ---------------------------------------------------------------- RMSNorm + quantize

template <class S>
__device__ __forceinline__ void stage_x(const PSmem& m, int i, float x) {
  const int o = (i & 3) * S::STV + (i >> 2);
  m.xl[o] = x;
  m.sq[o] = x * x;
}

// Wait for the D-vector at src (epoch ep) and stage it by lane runs, with its squares.
template <class S>
__device__ __forceinline__ void recv_x(const uint64_t* src, uint32_t ep, State* st, const PSmem& m, bool& bad,
                                       int nap) {
  uint32_t v[S::KD];
  ll_recv<S::KD>(src, S::D, ep, st, bad, v, nap);
#pragma unroll
  for (int k = 0; k < S::KD; k++) {
    const int i = (int)threadIdx.x + kPThreads * k;
    if (i < S::D) stage_x<S>(m, i, __uint_as_float(v[k]));
  }
}

// The 4 norm weights of this thread's half block lane (thread 2l + h: word h of block lane l),
// loaded ahead of the wait.
template <class S>
__device__ __forceinline__ void normw_load(const float* w, float (&nw)[4]) {
  const int t = threadIdx.x;
  if (t < S::NBD * 8) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const float2 p = gld2f(w + lane_elem(t >> 1, 4 * (t & 1) + 2 * u));
      nw[2 * u] = p.x;
      nw[2 * u + 1] = p.y;
    }
  }
}

// RMSNorm + quantize of the staged x into m.xq (kernels.c:80-86, 328-331): lanes 0..3 of every
// wave run the four lane sums of x*x in order and the wave forms the scale from them itself (the
// same operations on the same values in every wave, so the same bits), then thread t < NBD*8
// quantizes half a block lane.  No shared-memory round trip and no barrier between the sums and
// the quantize; the values a thread quantizes are read before the sums.  The caller has
// synchronised after staging; returns after a barrier.
template <class S, bool kLdsOnly = false>
__device__ __forceinline__ void norm_quant(const PSmem& m, const float (&nw)[4], float eps, unsigned long long* mark = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63;
  float xv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (tid < S::NBD * 8) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = lane_elem(tid >> 1, 4 * (tid & 1) + k);
      xv[k] = m.xl[(i & 3) * S::STV + (i >> 2)];
    }
  }
  float s = 0.0f;
  if (lane < 4) s = run_sum<S::D / 4>(m.sq + lane * S::STV);
  if (mark && tid == 0) {
    asm volatile("" ::"v"(s));
    *mark = wall_clock64();
  }
  const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 1));
  const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 2));
  const float s3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 3));
  const float rs = recip(__builtin_sqrtf(div_const<S::D>(((s0 + s1) + s2) + s3) + eps));
  if (tid < S::NBD * 8) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = (xv[k] * rs) * nw[k];
    const uint4 q = quant_half(v);
    if ((tid & 1) == 0) m.xq[tid >> 1] = q;
  }
  if constexpr (kLdsOnly) {
    // shared memory only: row groups still loading are waited for where their registers are
    // first used, not here
    lds_barrier();
  } else {
    __syncthreads();
  }
}

// (value, index) merge with the first-maximum rule of cpu-worker.js:157.
__device__ __forceinline__ void arg_merge(float& bv, int& bi, float v, int i) {
  if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
}

// The merge over the whole wave (all lanes active), the result in every lane.  The merge is a
// maximum under a total order (value, then the lower index), so any pairing gives the same result:
// quad permutations and the mirrors within 8 and 16 lanes by DPP, lane ^ 16 by swizzle, then lanes
// 0 and 32 (as max64), with no shared-memory round trip.
template <int C>
__device__ __forceinline__ void arg_dpp(float& bv, int& bi) {
  const float ov = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(bv), C, 0xF, 0xF, true));
  const int oi = __builtin_amdgcn_mov_dpp(bi, C, 0xF, 0xF, true);
  arg_merge(bv, bi, ov, oi);
}
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
  arg_dpp<0xB1>(bv, bi);
  arg_dpp<0x4E>(bv, bi);
  arg_dpp<0x141>(bv, bi);
  arg_dpp<0x140>(bv, bi);
  {
    const float ov = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(bv), 0x401F));
    const int oi = __builtin_amdgcn_ds_swizzle(bi, 0x401F);
    arg_merge(bv, bi, ov, oi);
  }
  const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
  const int i0 = __builtin_amdgcn_readlane(bi, 0);
  const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 32));
  const int i1 = __builtin_amdgcn_readlane(bi, 32);
  bv = v0;
  bi = i0;
  arg_merge(bv, bi, v1, i1);
}

// ---------------------------------------------------------------- the output head + argmax

template <class S>
__device__ __forceinline__ void head_rows(const PArgs& a, const PSmem& m, const WR<S::NGD> (&R)[1], int rg,
                                          int lane, float& bv, int& bi) {
  float acc[1] = {0.0f};
  wr_dot<S::NBD, 0, S::NGD, 1>(R, m.xq, lane & 3, acc);
  const float v = hsum4(acc[0]);
  const int row = rg * 16 + (lane >> 2);
  if ((lane & 3) == 0 && row < a.V) {
    a.logits[row] = v;
    arg_merge(bv, bi, v, row);
  }
}

// This workgroup's rank among the ones that keep head row groups in shared memory (every role
// but attention), or -1.
template <class S>
__device__ __forceinline__ int head_cache_rank(const PArgs& a, int wg) {
  if (wg < S::nOD) return wg;
  if (wg < S::nOD + S::H * a.asplit) return -1;
  return wg - S::H * a.asplit;
}

// Row group k (k < hres) kept by wave `wave` of the workgroup of rank `rank`: row groups
// [0, ranks * 4 * hres) are the resident ones, the rest are streamed.
__device__ __forceinline__ int head_cache_rg(int hres, int rank, int wave, int k) {
  return (rank * 4 + wave) * hres + k;
}

// Issue the asynchronous loads of this wave's resident row groups into `cache` (in the first step's
// head phase, before its wait for x, which drains them).
template <class S>
__device__ __forceinline__ void head_cache_fill(const PArgs& a, uint4* cache, int rank, int hres) {
  const int lane = threadIdx.x & 63, wave = wave_id(), j = lane & 3;
  for (int k = 0; k < hres; k++) {
    const int rg = head_cache_rg(hres, rank, wave, k);
    uint4* dst = cache + (size_t)(wave * hres + k) * (head_rg_bytes<S>() / 16);
    const int rr = (rg & 3) * 16 + (lane >> 2);            // row of lane l within its 64-row tile
    const uint4* wq = a.head.qs + ((size_t)(rg >> 2) * S::NGD * 64 + rr) * 4 + j;
#pragma unroll
    for (int g = 0; g < S::NGD; g++) sk_dma16(wq + (size_t)g * 256, dst + g * 64);
    // lane l: scale word c = l >> 4 of row r = l & 15 (words past NB8D repeat the last one, unused)
    const int c = (lane >> 4) < S::NB8D ? (lane >> 4) : S::NB8D - 1;
    const uint4* wd = a.head.d + ((size_t)(rg >> 2) * S::NB8D + c) * 64 + (rg & 3) * 16 + (lane & 15);
    sk_dma16(wd, dst + S::NGD * 64);
  }
}

// A resident row group into the registers wr_load would have filled.
template <class S>
__device__ __forceinline__ void head_cache_read(const uint4* src, int lane, WR<S::NGD>& R) {
#pragma unroll
  for (int g = 0; g < S::NGD; g++) R.w[g] = src[g * 64 + lane];
#pragma unroll
  for (int c = 0; c < (S::NGD + 1) / 2; c++) R.s[c] = src[S::NGD * 64 + c * 16 + (lane >> 2)];
}

// Logits of this workgroup's Q4_0 row groups (five rotating register buffers: four row groups in
// flight while one is computed; with two, the head streamed ~5 us slower per step); x is received
// and normalised after the first four are issued.
template <class S>
__device__ __forceinline__ bool head_scan_q4(const PArgs& a, const PSmem& m, uint32_t epx, int s, bool& bad,
                                             float& bv, int& bi) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int G = gridDim.x, wg = lwg(a), nRG = a.head.Np / 16, stride = 4 * G;
  float nw[4];
  normw_load<S>(a.out_norm, nw);
  // row groups round-robin over the waves, the o/down workgroups last: they come to the head
  // last (their final down stores end the layers), so they take the fewest row groups
  int rgi = (G - 1 - wg) + G * wave;
  constexpr int NBUF = 5;
  WR<S::NGD> R[NBUF][1];
#pragma unroll
  for (int k = 0; k < NBUF - 1; k++)
    if (rgi + k * stride < nRG) wr_load<S::NGD, S::NB8D, 0, S::NGD>(a.head, rgi + k * stride, lane, R[k][0]);
  recv_x<S>(a.ll + S::oXH, epx, a.st, m, bad, a.nap);
  if (wg_bad(m.flag, bad)) return false;
  prof_mark(a, s, a.NL * 16 + 0);
  norm_quant<S>(m, nw, a.eps);
  for (;;) {
#pragma unroll
    for (int i = 0; i < NBUF; i++) {
      if (rgi + (NBUF - 1) * stride < nRG)
        wr_load<S::NGD, S::NB8D, 0, S::NGD>(a.head, rgi + (NBUF - 1) * stride, lane, R[(i + NBUF - 1) % NBUF][0]);
      head_rows<S>(a, m, R[i], rgi, lane, bv, bi);
      rgi += stride;
      if (rgi >= nRG) return true;
    }
  }
  return true;
}

// The same with resident row groups: the resident ones from shared memory, then the streamed
// ones through the five rotating register buffers.  Workgroups that finish their last
// layer early issue the first four streamed row groups before they wait for x; the o/down
// workgroups, whose down stores end the layers, wait for x first (loads issued before a wait
// delay it: the wait's memory counter covers every earlier load) and work on their resident row
// groups while the streamed ones arrive.
template <class S>
__device__ __forceinline__ bool head_scan_q4_cached(const PArgs& a, const PSmem& m, uint32_t epx, int s, bool& bad,
                                                    float& bv, int& bi) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int G = gridDim.x, wg = lwg(a), nRG = a.head.Np / 16, stride = 4 * G;
  const int rank = head_cache_rank<S>(a, wg), hres = a.hres;
  const int nres = rank >= 0 ? hres : 0;
  float nw[4];
  normw_load<S>(a.out_norm, nw);
  // streamed row groups round-robin over the waves, the o/down workgroups' waves last in each
  // round: they come to the head last, so the last, partial round leaves them out
  const int ord = wg < S::nOD ? 4 * (G - S::nOD) + (S::nOD - 1 - wg) + S::nOD * wave
                              : (G - 1 - wg) + (G - S::nOD) * wave;
  int rgi = (G - S::H * a.asplit) * 4 * hres + ord;
  const bool early = wg >= S::nOD || nres == 0;
  if (s == 0 && nres > 0) head_cache_fill<S>(a, m.hcache, rank, nres);
  constexpr int NBUF = 5;
  WR<S::NGD> R[NBUF][1];
  if (early) {
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++)
      if (rgi + k * stride < nRG) wr_load<S::NGD, S::NB8D, 0, S::NGD>(a.head, rgi + k * stride, lane, R[k][0]);
  }
  recv_x<S>(a.ll + S::oXH, epx, a.st, m, bad, a.nap);
  // every earlier load has completed, the resident row groups' included
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (wg_bad(m.flag, bad)) return false;
  prof_mark(a, s, a.NL * 16 + 0);
  if (!early) {
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++)
      if (rgi + k * stride < nRG) wr_load<S::NGD, S::NB8D, 0, S::NGD>(a.head, rgi + k * stride, lane, R[k][0]);
  }
  // the o/down workgroups' first row groups load while x is normalised and the resident rows run
  norm_quant<S, true>(m, nw, a.eps);
  for (int k = 0; k < nres; k++) {
    WR<S::NGD> C[1];
    head_cache_read<S>(m.hcache + (size_t)(wave * nres + k) * (head_rg_bytes<S>() / 16), lane, C[0]);
    head_rows<S>(a, m, C, head_cache_rg(hres, rank, wave, k), lane, bv, bi);
  }
  if (rgi >= nRG) return true;
  for (;;) {
#pragma unroll
    for (int i = 0; i < NBUF; i++) {
      if (rgi + (NBUF - 1) * stride < nRG)
        wr_load<S::NGD, S::NB8D, 0, S::NGD>(a.head, rgi + (NBUF - 1) * stride, lane, R[(i + NBUF - 1) % NBUF][0]);
      head_rows<S>(a, m, R[i], rgi, lane, bv, bi);
      rgi += stride;
      if (rgi >= nRG) return true;
    }
  }
  return true;
}

// Q8_0 head rows (k_repack_q8 layout): lane (r, j) holds {A_j, B_j} of two blocks per uint4.
template <int NG8, int NB8>
struct WR8 {
  uint4 w[NG8];
  uint4 s[NB8];
};

template <int NG8, int NB8>
__device__ __forceinline__ void wr8_load(const Q4Mat& W, int rg16, int lane, WR8<NG8, NB8>& R) {
  const int row = rg16 * 16 + (lane >> 2), j = lane & 3;
  const int tile = row >> 6, rr = row & 63;
  const uint4* wq = W.qs + ((size_t)tile * NG8 * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * NB8 * 64 + rr;
#pragma unroll
  for (int g = 0; g < NG8; g++) R.w[g] = gld(wq + (size_t)g * 256);
#pragma unroll
  for (int c = 0; c < NB8; c++) R.s[c] = gld(wd + (size_t)c * 64);
}

// dot_q8_q8 of one lane (kernels.c:157-170): per block p = A_j . xA_j + B_j . xB_j, then
// acc = acc + f32(p) * (dw * dx), blocks in order; four blocks per stage, next four read ahead.
template <int NB, int NG8, int NB8>
__device__ __forceinline__ float wr8_dot(const WR8<NG8, NB8>& R, const uint4* xq, int j) {
  constexpr int NQ = (NB + 3) / 4;
  float acc = 0.0f;
  uint4 xb[2][4];
  xg_load<NB, 0>(xq, 0, j, xb[0]);
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    if (q + 1 < NQ) xg_load<NB, 0>(xq, q + 1, j, xb[(q + 1) & 1]);
#pragma unroll
    for (int k = 0; k < 4; k++) pin(xb[q & 1][k]);
    int p[4];
    float t[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int b = 4 * q + k;
      if (b < NB) p[k] = sdot4((b & 1) ? R.w[b >> 1].z : R.w[b >> 1].x, xb[q & 1][k].x, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int b = 4 * q + k;
      if (b < NB) p[k] = sdot4((b & 1) ? R.w[b >> 1].w : R.w[b >> 1].y, xb[q & 1][k].y, p[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int b = 4 * q + k;
      if (b < NB) {
        const uint4 sv = R.s[b >> 3];
        const int hb = b & 7;
        const uint32_t sw = (hb >> 1) == 0 ? sv.x : (hb >> 1) == 1 ? sv.y : (hb >> 1) == 2 ? sv.z : sv.w;
        const float dw = half_bits_to_float((hb & 1) ? (sw >> 16) : (sw & 0xffffu));
        t[k] = (float)p[k] * (dw * __uint_as_float(xb[q & 1][k].w));
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (4 * q + k < NB) acc = acc + t[k];
  }
  return acc;
}

template <class S>
__device__ __forceinline__ void head_rows8(const PArgs& a, const PSmem& m,
                                           const WR8<(S::NBD + 1) / 2, S::NB8D>& R, int rg, int lane,
                                           float& bv, int& bi) {
  const float v = hsum4(wr8_dot<S::NBD, (S::NBD + 1) / 2, S::NB8D>(R, m.xq, lane & 3));
  const int row = rg * 16 + (lane >> 2);
  if ((lane & 3) == 0 && row < a.V) {
    a.logits[row] = v;
    arg_merge(bv, bi, v, row);
  }
}

// Logits of this workgroup's Q8_0 row groups (two rotating register buffers).
template <class S>
__device__ __forceinline__ bool head_scan_q8(const PArgs& a, const PSmem& m, uint32_t epx, int s, bool& bad,
                                             float& bv, int& bi) {
  constexpr int NG8 = (S::NBD + 1) / 2;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int G = gridDim.x, wg = lwg(a), nRG = a.head.Np / 16, stride = 4 * G;
  float nw[4];
  normw_load<S>(a.out_norm, nw);
  int rgi = wg + G * wave;
  WR8<NG8, S::NB8D> R0, R1;
  if (rgi < nRG) wr8_load<NG8, S::NB8D>(a.head, rgi, lane, R0);
  recv_x<S>(a.ll + S::oXH, epx, a.st, m, bad, a.nap);
  if (wg_bad(m.flag, bad)) return false;
  prof_mark(a, s, a.NL * 16 + 0);
  norm_quant<S>(m, nw, a.eps);
  while (rgi < nRG) {
    if (rgi + stride < nRG) wr8_load<NG8, S::NB8D>(a.head, rgi + stride, lane, R1);
    head_rows8<S>(a, m, R0, rgi, lane, bv, bi);
    rgi += stride;
    if (rgi >= nRG) break;
    if (rgi + stride < nRG) wr8_load<NG8, S::NB8D>(a.head, rgi + stride, lane, R0);
    head_rows8<S>(a, m, R1, rgi, lane, bv, bi);
    rgi += stride;
  }
  return true;
}

// Final RMSNorm, logits of this workgroup's row groups, then every workgroup reduces every
// workgroup's (value, index): the same token everywhere.  Returns the token, or -1 on abort.
// HC: this kernel keeps head row groups in shared memory (PArgs::hres).
template <class S, bool HC>
__device__ __forceinline__ int head_phase(const PArgs& a, const PSmem& m, uint32_t ep0, int s, int pos, bool& bad) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int G = gridDim.x, wg = lwg(a), E = 4 * a.NL + 1;
  uint64_t* LARG = a.ll + S::oARG + (size_t)(s & 1) * kArgStride * G;
  const uint32_t epx = phase_epoch(ep0, s, E, 4 * (a.NL - 1) + 3);
  const uint32_t eph = phase_epoch(ep0, s, E, 4 * a.NL);

  float bv = 0.0f;
  int bi = -1;
  const bool ok = a.head_q8 ? head_scan_q8<S>(a, m, epx, s, bad, bv, bi)
                            : HC ? head_scan_q4_cached<S>(a, m, epx, s, bad, bv, bi)
                                 : head_scan_q4<S>(a, m, epx, s, bad, bv, bi);
  if (!ok) return -1;
  wave_argmax(bv, bi);
  if (lane == 0) { m.argv[wave] = bv; m.argi[wave] = bi; }
  __syncthreads();
  if (tid < kArgStride) {
    // every lane of the line merges the four waves' pairs; one store writes the whole line
    bv = m.argv[0];
    bi = m.argi[0];
    for (int w = 1; w < 4; w++) arg_merge(bv, bi, m.argv[w], m.argi[w]);
    ll_put(LARG + kArgStride * wg + tid, tid == 0 ? __float_as_uint(bv) : (uint32_t)bi, eph);
  }
  prof_mark(a, s, a.NL * 16 + 1);
  {
    uint32_t v[2];
    ll_recv<2>(LARG, 2 * G, eph, a.st, bad, v, a.nap, ArgEntry());
    m.raw[tid] = v[0];
    if (tid + kPThreads < 2 * G) m.raw[tid + kPThreads] = v[1];
  }
  if (wg_bad(m.flag, bad)) return -1;
  bv = 0.0f;
  bi = -1;
  for (int g = tid; g < G; g += kPThreads) arg_merge(bv, bi, __uint_as_float(m.raw[2 * g]), (int)m.raw[2 * g + 1]);
  wave_argmax(bv, bi);
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

// ---------------------------------------------------------------- the K/V ring of the attention role

// The rows the attention role's ring loads read (host and device code: q4hip_attn_ring_rows runs the
// same arithmetic on the host so a CPU test can check it).  The role streams the past positions of
// its (layer, kv head) through the ring: rows [kbeg, kend) for its scores in 16-row chunks and, for
// P.V, rows [nt, pos) in slots of vr rows (or, split, rows [0, pos) in half-width slots).  A load of
// a row at or past the end of its stream reads the stream's last row instead, so no load touches the
// current position or a later one: those rows are written during this step by the K/V role, possibly
// on another XCD, and a stale copy could stay in this XCD's L2.
__host__ __device__ constexpr int ring_row(int t, int limit) { return t < limit ? t : limit - 1; }
constexpr int kVRows = 96;   // rows of a half-width P.V slot (split attention)
struct AttnRing {
  int nt;            // staged past positions [0, nt)
  int kbeg, kend;    // K rows scored from the ring
  int obeg, oend;    // split: the pair's other half, whose scores arrive through the exchange
  int vr;            // rows of an unsplit P.V slot
  int nstream, nck, nkc, nckv;
};
__host__ __device__ inline AttnRing attn_ring(int pos, int kv_tile, bool split, int half, bool f16) {
  AttnRing r;
  r.nt = split ? 0 : (pos < kv_tile ? pos : kv_tile);
  const int nall = (pos + kRingRows - 1) / kRingRows;
  r.kbeg = split ? (half == 0 ? 0 : (nall / 2) * kRingRows) : r.nt;
  r.kend = split ? (half == 0 ? (nall / 2) * kRingRows : pos) : pos;
  r.obeg = split ? (half == 0 ? (nall / 2) * kRingRows : 0) : 0;
  r.oend = split ? (half == 0 ? pos : (nall / 2) * kRingRows) : 0;
  r.vr = f16 ? 2 * kRingRows : kRingRows;
  r.nstream = r.kend - r.kbeg;
  r.nck = (r.nstream + r.vr - 1) / r.vr;
  r.nkc = (r.nstream + 15) / 16;
  r.nckv = split ? (pos + kVRows - 1) / kVRows : 0;
  return r;
}
// K chunks of wave w: chunks w, w + 4, ... of the stream; issue j loads chunk min(j, nloc - 1).
__host__ __device__ constexpr int attn_nloc(int nkc, int wave) { return nkc > wave ? (nkc - wave + 3) / 4 : 0; }
__host__ __device__ constexpr int kchunk_t0(int kbeg, int j, int nloc, int wave) {
  return kbeg + 16 * (4 * (j < nloc ? j : nloc - 1) + wave);
}
// First row of P.V slot c (issues past the last slot repeat it): unsplit and split.
__host__ __device__ constexpr int vslot_t0(int nt, int c, int nck, int vr) { return nt + (c < nck ? c : nck - 1) * vr; }
__host__ __device__ constexpr int vpslot_t0(int c, int nckv) { return (c < nckv ? c : nckv - 1) * kVRows; }


typedef __attribute__((address_space(3))) void LdsVoid;
typedef __attribute__((address_space(1))) const void GlobalVoid;

// Issue the asynchronous loads of rows [t0, t0 + kRingRows) of one (layer, kv head) V block into
// `slot` as plain rows: wave w issues instructions w, w+4, w+8, each moving rows t0+4i .. t0+4i+3.
// Rows at or past `limit` (the end of the streamed past positions) are read from row limit - 1
// (ring_row; their values are never used).
__device__ __forceinline__ void ring_issue(const float* src, int t0, int limit, float* slot) {
  const int lane = threadIdx.x & 63, wave = wave_id();
#pragma unroll
  for (int k = 0; k < 3; k++) {
    const int i = wave + 4 * k;
    const int t = t0 + 4 * i + (lane >> 4);
    const float* g = src + (size_t)ring_row(t, limit) * kHD + 4 * (lane & 15);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)g, (LdsVoid*)(slot + i * 256), 16, 0, 0);
  }
}
// fp16 rows: a slot holds 2 kRingRows rows (the same 12 instructions, 8 rows each), row r at
// half 64 r of the slot.
__device__ __forceinline__ void ring_issue(const kvhalf* src, int t0, int limit, float* slot) {
  const int lane = threadIdx.x & 63, wave = wave_id();
#pragma unroll
  for (int k = 0; k < 3; k++) {
    const int i = wave + 4 * k;
    const int t = t0 + 8 * i + (lane >> 3);
    const kvhalf* g = src + (size_t)ring_row(t, limit) * kHD + 8 * (lane & 7);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)g, (LdsVoid*)(slot + i * 256), 16, 0, 0);
  }
}
// Rows of a P.V ring slot: kRingRows fp32 rows or twice as many fp16 rows in the same bytes.
template <class KT>
__host__ __device__ constexpr int vslot_rows() { return sizeof(KT) == 4 ? kRingRows : 2 * kRingRows; }

// One wave's loads of K rows [t0, t0 + 16) into a chunk slot, one 4-row group per instruction at
// slot + g * kGrpFloats.  An instruction places lane l's 16 bytes at float 4 l of its group, and
// lane l fetches elements 4c .. 4c+3 (c = l >> 2) of row l & 3: element 4c + e of group row r
// lands at float 16 c + 4 r + e.  Four lanes per row then read elements 4i + j of their row at
// immediate offsets 16 i, and with the 16-float padding the 16 rows of the wave cover all 64 banks.
// Rows at or past `limit` are read from row limit - 1 (ring_row; their values are never used).
__device__ __forceinline__ void ring_issue_kc(const float* src, int t0, int limit, float* slot) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int t = t0 + 4 * g + (lane & 3);
    const float* p = src + (size_t)ring_row(t, limit) * kHD + 4 * (lane >> 2);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)p, (LdsVoid*)(slot + g * kGrpFloats), 16, 0, 0);
  }
}

// The same for an fp16 cache: 16 rows of 128 bytes in two instructions of 8 rows.  Lane l of
// instruction h fetches bytes 16 c .. 16 c + 15 (c = l >> 3) of row 8 h + (l & 7); instruction h
// lands at byte 1152 h of the chunk (a 128-byte pad between the two), lane l at 16 l.  Row r's
// piece c then sits at byte 1152 (r >> 3) + 128 c + 16 (r & 7): for one c the 16 rows start in 16
// distinct 16-byte bank groups, so the reads below (element 4i + j of a row by lane j) are free of
// conflicts.  2304 bytes of the chunk's kChunkFloats.
constexpr int kChunk16Bytes = 2304;
static_assert(kChunk16Bytes <= kChunkFloats * 4, "fp16 chunk exceeds the chunk slot");
__device__ __forceinline__ void ring_issue_kc(const kvhalf* src, int t0, int limit, float* slot) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int t = t0 + 8 * h + (lane & 7);
    const kvhalf* p = src + (size_t)ring_row(t, limit) * kHD + 8 * (lane >> 3);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)p, (LdsVoid*)((char*)slot + 1152 * h), 16, 0, 0);
  }
}

// Element 4i + pj (i = 0..15) of row pr of a chunk, as fp32: fp32 chunks in ring_issue_kc's group
// layout, fp16 chunks in the layout above.
__device__ __forceinline__ void kchunk_row(const float* chunk, int pr, int pj, float (&kr)[kHD / 4]) {
  const float* row = chunk + (pr >> 2) * kGrpFloats + 4 * (pr & 3) + pj;
#pragma unroll
  for (int i = 0; i < kHD / 4; i++) kr[i] = row[16 * i];
}
__device__ __forceinline__ void kchunk_row16(const float* chunk, int pr, int pj, float (&kr)[kHD / 4]) {
  const unsigned short* hb = reinterpret_cast<const unsigned short*>(
      reinterpret_cast<const char*>(chunk) + 1152 * (pr >> 3) + 16 * (pr & 7) + 2 * pj);
#pragma unroll
  for (int i = 0; i < kHD / 4; i++) kr[i] = half_bits_to_float(hb[64 * (i >> 1) + 4 * (i & 1)]);
}

// Wait until this wave's loads of its oldest K chunk in flight have landed (`cs` - 2 newer chunks
// of N instructions -- 4 for fp32 rows, 2 for fp16 -- may still be outstanding).  Only the
// issuing wave reads a chunk: no barrier.
// Wide K chunks for fp16 caches: 32 rows of 8 pieces (16 bytes each), one row per pair of lanes
// of the scoring wave.  Instruction g (0..3) loads rows 8g .. 8g+7 whole (8 full 128-byte lines):
// lane l fetches piece (l + rot(r)) & 7 of row r = 8g + (l >> 3), rot(r) = (r >> 1) & 7, and it
// lands at byte 1024 g + 16 l, so piece p of row r sits at byte 128 r + 16 ((p - rot(r)) & 7).
// Both lanes of row t read piece p there: over 16 consecutive lanes (8 rows) the 16-byte bank
// groups 8 (t & 1) + ((p - rot(t)) & 7) are distinct, so the reads are free of bank conflicts.
// Rows at or past `limit` are read from row limit - 1 (ring_row; their scores are never stored).
constexpr int kWideRows = 32;
constexpr int kWideFloats = kWideRows * kHD / 2;     // 4 KB of fp16 rows
constexpr int kWideIssue = kWideRows / 8;            // load instructions per chunk
__device__ __forceinline__ int kwide_rot(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ void ring_issue_kw(const kvhalf* src, int t0, int limit, float* slot) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int g = 0; g < kWideIssue; g++) {
    const int r = 8 * g + (lane >> 3);
    const int pc = ((lane & 7) + kwide_rot(r)) & 7;
    const kvhalf* p = src + (size_t)ring_row(t0 + r, limit) * kHD + 8 * pc;
    __builtin_amdgcn_global_load_lds((GlobalVoid*)p, (LdsVoid*)(slot + g * 256), 16, 0, 0);
  }
}
// First row of wide chunk j of wave w (chunks w, w + 4, ... of the stream; j clamped to the last).
__host__ __device__ constexpr int kwide_t0(int kbeg, int j, int nloc, int wave) {
  return kbeg + kWideRows * (4 * (j < nloc ? j : nloc - 1) + wave);
}
// Wide chunk slots in a wave's share of the ring: 5 (7-slot ring) or 2 (3-slot ring).
__host__ __device__ constexpr int kwide_slots(int cs) {
  return cs * kChunkFloats / kWideFloats < 5 ? cs * kChunkFloats / kWideFloats : 5;
}
static_assert(kwide_slots(kchunk_slots(7)) == 5 && kwide_slots(kchunk_slots(3)) == 2, "wide chunk slots");
// Wait for the oldest of the wave's wide chunks in flight (ws - 1 newer ones may stay in flight).
__device__ __forceinline__ void kwide_wait(int ws) {
  if (ws == 5) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kWideIssue) : "memory");
  else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kWideIssue) : "memory");
}

template <int N>
__device__ __forceinline__ void kchunk_wait(int cs) {
  if (cs == 5) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * N) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Wait until this wave's loads of the oldest slot in flight have landed (R - 2 newer slots of 3
// instructions each may still be outstanding: vmcnt(3 (R - 2))) and its LDS accesses are done,
// then meet the other waves.  Not __syncthreads: its workgroup fence waits for every outstanding
// load into LDS (vmcnt(0)), which would leave a single slot in flight.  The "memory" clobber keeps
// the compiler from moving loads or stores across the barrier.
__device__ __forceinline__ void ring_sync(int slots) {
  if (slots == 7) asm volatile("s_waitcnt vmcnt(15) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void ring_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)

// Half-width slots for the split attention's P.V: kVRows rows x 32 of the 64 columns (from c0) as
// plain rows of 32 floats, the footprint of a full slot.  Producer wave pw (waves 1..3) loads rows
// 32 pw .. 32 pw + 31 of a slot with 4 instructions of 8 rows each and forms their products.
__device__ __forceinline__ void ring_issue_vp(const float* src, int t0, int limit, int c0, int pw, float* slot) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = 4 * pw + k;
    const int t = t0 + 8 * i + (lane >> 3);
    const float* g = src + (size_t)ring_row(t, limit) * kHD + c0 + 4 * (lane & 7);
    __builtin_amdgcn_global_load_lds((GlobalVoid*)g, (LdsVoid*)(slot + i * 256), 16, 0, 0);
  }
}

// fp16 rows: producer pw's 32 rows x 32 halves (2 KB) in 2 instructions of 16 rows, landing in
// the upper half of its 4 KB part (byte 2048 + 64 r + 2 col); it reads them all before it writes
// the fp32 products over the part.  Issued as inline assembly (sk_dma16): with the builtin the
// compiler made the producer's every shared-memory read wait for all of its loads in flight;
// vpart_wait orders the reads instead.
__device__ __forceinline__ void ring_issue_vp(const kvhalf* src, int t0, int limit, int c0, int pw, float* slot) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int t = t0 + 32 * pw + 16 * k + (lane >> 2);
    const kvhalf* g = src + (size_t)ring_row(t, limit) * kHD + c0 + 8 * (lane & 3);
    sk_dma16(g, slot + pw * 1024 + 512 + k * 256);
  }
}

// A producer wave's wait for its own rows of the oldest slot in flight (d - 1 newer slots of N
// instructions -- 4 for fp32 rows, 2 for fp16 -- may still be outstanding).
template <int N>
__device__ __forceinline__ void vpart_wait(int d) {
  if (d == 5) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * N) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Hand-off counters of the split P.V in this workgroup's shared memory.  Bounded waits: false
// after kLdsSpinLimit polls (the caller gives up the step like any other timed-out wait).
typedef __attribute__((address_space(3))) int LdsInt;
constexpr int kLdsSpinLimit = 1 << 20;
__device__ __forceinline__ bool lds_wait_ge(volatile LdsInt* c, int v) {
  for (int spin = 0; spin < kLdsSpinLimit; spin++) {
    if (*c >= v) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}
__device__ __forceinline__ bool lds_wait_ge3(volatile LdsInt* c, int v) {
  for (int spin = 0; spin < kLdsSpinLimit; spin++) {
    const int a0 = c[0], a1 = c[1], a2 = c[2];
    if (a0 >= v && a1 >= v && a2 >= v) return true;
  }
  return false;
}


// ---------------------------------------------------------------- roles (one step each)

// Quad-chain rows (o and down of the OD role).  Wave w owns rows 4w..4w+3 of the workgroup's 16;
// lane l is (row l >> 4, reference lane j = (l >> 2) & 3, phase p = l & 3).  Phase p holds the
// groups g = 4k + p of four blocks and forms their terms f32(p_j) * (dw * dx) (kernels.c:137); the
// four lanes of the quad all run the same chain acc = acc + term over the blocks in order
// (kernels.c:217-218), taking each term from the lane that formed it by a DPP quad broadcast.  The
// chain runs while the terms of later groups are formed, with no shared-memory terms and no barrier
// between the waves.
template <int NG>
struct QR {
  static constexpr int NK = (NG + 3) / 4;   // groups per phase
  uint4 w[NK];                              // word j of the group's 4 blocks
  uint2 s[NK];                              // the group's 4 fp16 scales
};

__device__ __forceinline__ uint2 gld2u(const void* p) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(1))) const u32x2 GU2;
  const u32x2 v = *(GU2*)p;
  return make_uint2(v.x, v.y);
}

// Groups 4k + p (the last group where 4k + p is past NG: never used) of row `row`.
template <int NG, int NB8>
__device__ __forceinline__ void qr_load(const Q4Mat& W, int row, int lane, QR<NG>& R) {
  const int j = (lane >> 2) & 3, p = lane & 3, tile = row >> 6, rr = row & 63;
  const uint4* wq = W.qs + ((size_t)tile * NG * 64 + rr) * 4 + j;
  const uint4* wd = W.d + (size_t)tile * NB8 * 64 + rr;
#pragma unroll
  for (int k = 0; k < QR<NG>::NK; k++) {
    const int g = 4 * k + p < NG ? 4 * k + p : NG - 1;
    R.w[k] = gld(wq + (size_t)g * 256);
    R.s[k] = gld2u(reinterpret_cast<const uint2*>(wd + (size_t)(g >> 1) * 64) + (g & 1));
  }
}

// Activation blocks 4g .. 4g+3 of lane j (g clamped like the weights).
template <int NG>
__device__ __forceinline__ void qr_xload(const uint4* xq, int k, int p, int j, uint4 (&xv)[4]) {
  const int g = 4 * k + p < NG ? 4 * k + p : NG - 1;
#pragma unroll
  for (int i = 0; i < 4; i++) xv[i] = xq[(4 * g + i) * 4 + j];
}

template <int Q>
__device__ __forceinline__ float quad_add(float acc, float t) {
  return acc + quad_lane<Q>(t);
}

// The term of block i (0..3) of this lane's group of round k.
template <int NG>
__device__ __forceinline__ float qr_term(const QR<NG>& R, int k, int i, const uint4& xv) {
  const uint4 w = R.w[k];
  const uint32_t wv = i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
  const uint32_t sw = i < 2 ? R.s[k].x : R.s[k].y;
  int pp = sdot4(wv & 0x0F0F0F0Fu, xv.x, (int)xv.z);
  pp = sdot4((wv >> 4) & 0x0F0F0F0Fu, xv.y, pp);
  const float dw = half_bits_to_float((i & 1) ? (sw >> 16) : (sw & 0xffffu));
  return (float)pp * (dw * __uint_as_float(xv.w));
}

// The chain steps of phase q of round k: the terms of group 4k + q in order, from that phase's lane.
template <int NB, int NG, int Q>
__device__ __forceinline__ float qr_phase(float acc, int k, const float (&t)[4]) {
  if (4 * k + Q < NG) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (4 * (4 * k + Q) + i < NB) acc = quad_add<Q>(acc, t[i]);
  }
  return acc;
}

// The chain ((0 + t_0) + t_1) + ... + t_{NB-1} of reference lane j of this lane's row, software
// pipelined by hand: in round k the four phases' chain steps (dependent adds) alternate with the
// terms of round k + 1, one block after each phase, and the activation reads run two rounds
// ahead.  The pins fix that order (the scheduler would otherwise place every add after the terms).
template <int NB, int NG>
__device__ __forceinline__ float qr_chain(const QR<NG>& R, const uint4* xq, int lane) {
  constexpr int NK = QR<NG>::NK;
  const int j = (lane >> 2) & 3, p = lane & 3;
  float acc = 0.0f;
  float t[2][4];
  uint4 xv[2][4];
  qr_xload<NG>(xq, 0, p, j, xv[0]);
  if (NK > 1) qr_xload<NG>(xq, 1, p, j, xv[1]);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    t[0][i] = qr_term<NG>(R, 0, i, xv[0][i]);
    pin(t[0][i]);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < NK; k++) {
    // xv[(k + 1) & 1] holds round k + 1's activations; round k + 2's go into xv[k & 1]
    if (k + 2 < NK) qr_xload<NG>(xq, k + 2, p, j, xv[k & 1]);
    const int n = (k + 1) & 1;
#define Q4_PHASE(Q)                                                          \
    acc = qr_phase<NB, NG, Q>(acc, k, t[k & 1]);                             \
    pin(acc);                                                                \
    if (k + 1 < NK) {                                                        \
      t[n][Q] = qr_term<NG>(R, k + 1, Q, xv[n][Q]);                          \
      pin(t[n][Q]);                                                          \
    }
    Q4_PHASE(0)
    Q4_PHASE(1)
    Q4_PHASE(2)
    Q4_PHASE(3)
#undef Q4_PHASE
    __builtin_amdgcn_sched_barrier(0);
  }
  return acc;
}

// ((a_0 + a_1) + a_2) + a_3 over the reference lanes of this lane's row: lane 4j of the 16-lane row
// holds chain j (DPP row broadcasts), in every lane of the row.
template <int K>
__device__ __forceinline__ float row_lane(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + K, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_hsum(float acc) {
  const float a0 = row_lane<0>(acc), a1 = row_lane<4>(acc), a2 = row_lane<8>(acc), a3 = row_lane<12>(acc);
  return ((a0 + a1) + a2) + a3;
}

// o and down rows 16w..16w+15: wave v takes rows 16w + 4v .. 16w + 4v + 3 as quad chains; every lane
// of a row keeps that row's residual x in a register.  The 16 results meet in shared memory and
// wave 0 stores them as one line.
template <class S>
__device__ __forceinline__ bool od_step(const PArgs& a, const PSmem& m, uint32_t ep0, int s, int tok, bool& bad) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wg = lwg(a), row = wg * 16 + 4 * wave + (lane >> 4), E = 4 * a.NL + 1;
  const bool writer = (lane & 15) == 0;
  float own = embed_value(a.embd, S::D, tok, row);   // the residual x of this lane's row
  for (int l = 0; l < a.NL; l++) {
    const LayerView& L = a.layers[l];
    // ---- o: x1 = x + W_o . quantize(att)
    if (l > 0) pf_delay(a.pf[0]);
    QR<S::NGD> ro;
    qr_load<S::NGD, S::NB8D>(L.o, row, lane, ro);
    {
      uint32_t v[S::KD];
      ll_recv<S::KD>(a.ll + S::oATT, S::D, phase_epoch(ep0, s, E, 4 * l + 0), a.st, bad, v, a.nap);
#pragma unroll
      for (int k = 0; k < S::KD; k++)
        if (tid + kPThreads * k < S::D) m.xl[tid + kPThreads * k] = __uint_as_float(v[k]);
    }
    if (wg_bad(m.flag, bad)) return false;
    if (wg == 0) prof_mark(a, s, l * 16 + 0);
    prof_wg(a, s, l, 0);
    if (tid < S::NBD * 8) {
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; k++) v[k] = m.xl[lane_elem(tid >> 1, 4 * (tid & 1) + k)];
      const uint4 q = quant_half(v);
      if ((tid & 1) == 0) m.xq[tid >> 1] = q;
    }
    __syncthreads();
    {
      const float v = row_hsum(qr_chain<S::NBD, S::NGD>(ro, m.xq, lane));
      own = own + v;
      if (writer) m.own[row - wg * 16] = own;
      lds_barrier();
      // the workgroup's 16 rows as one 128-byte line (lines written piecewise reach readers later)
      if (tid < 16) ll_put(a.ll + S::oX1 + wg * 16 + tid, __float_as_uint(m.own[tid]), phase_epoch(ep0, s, E, 4 * l + 1));
    }
    if (wg == 0) prof_mark(a, s, l * 16 + 1);
    prof_wg(a, s, l, 1);
    // ---- down: x2 = x1 + W_down . act (act arrives quantized)
    pf_delay(a.pf[1]);
    QR<S::NGF> rd;
    qr_load<S::NGF, S::NB8F>(L.down, row, lane, rd);
    {
      uint32_t v[S::KACT];
      ll_recv<S::KACT>(a.ll + S::oACT, S::NACT, phase_epoch(ep0, s, E, 4 * l + 2), a.st, bad, v, a.nap, ActEntry());
#pragma unroll
      for (int k = 0; k < S::KACT; k++)
        if (tid + kPThreads * k < S::NACT) m.raw[tid + kPThreads * k] = v[k];
    }
    if (wg_bad(m.flag, bad)) return false;
    for (int b = tid; b < S::NBF; b += kPThreads) {
      uint32_t e[9];
#pragma unroll
      for (int k = 0; k < 9; k++) e[k] = m.raw[b * 9 + k];
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        const int c = -8 * (sdot4(e[jj], 0x01010101u, 0) + sdot4(e[4 + jj], 0x01010101u, 0));
        m.xq[b * 4 + jj] = make_uint4(e[jj], e[4 + jj], (uint32_t)c, e[8]);
      }
    }
    __syncthreads();
    if (wg == 0) prof_mark(a, s, l * 16 + 2);
    prof_wg(a, s, l, 2);
    {
      const float v = row_hsum(qr_chain<S::NBF, S::NGF>(rd, m.xq, lane));
      own = own + v;
      if (writer) m.own[row - wg * 16] = own;
      lds_barrier();
      if (tid < 16)
        ll_put(a.ll + (l == a.NL - 1 ? S::oXH : S::oX2) + wg * 16 + tid, __float_as_uint(m.own[tid]),
               phase_epoch(ep0, s, E, 4 * l + 3));
    }
    if (wg == 0) prof_mark(a, s, l * 16 + 3);
    prof_wg(a, s, l, 3);
  }
  return true;
}

// One attention head h: q rows of h and k, v rows of its kv group, RoPE, K/V append (first head of
// the group), attention over the cache (kernels.c:333-377).  Past K/V rows (up to kv_tile of them)
// are staged in shared memory while the role waits for x.
//
// K/V of a position are written once per launch (agent-scope stores), by the first head of the
// group, and are first read by the other heads at least one step later: each position is read only
// once pos has moved past it.
template <class S, class KT>
__device__ __forceinline__ bool attn_step(const PArgs& a, const PSmem& m, uint32_t ep0, int s, int pos, int tok,
                                          bool& bad) {
  constexpr bool kF16 = sizeof(KT) == 2;   // fp16 rows stream in half the bytes (same ring memory)
  constexpr int VR = vslot_rows<KT>();       // rows of a P.V ring slot
  constexpr int NKC = kF16 ? 2 : 4;          // load instructions per K chunk
  constexpr int NVP = kF16 ? 2 : 4;          // per producer and half-width V slot
  constexpr int GRP = S::H / S::KVH;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), r = lane >> 2, j = lane & 3;
  const int E = 4 * a.NL + 1;
  const int aidx = lwg(a) - S::nOD, h = aidx % S::H, half = aidx / S::H, kh = h / GRP;
  const bool split = a.asplit > 1;
  const bool mark = aidx == 0;
  const int rq = (h * kHD) / 16 + wave;
  float* qv = m.qv;
  float* kv = m.qv + 64;
  float* vv = m.qv + 128;
  float* sc = m.terms;                                     // ctx + 2 kRingRows scores
  float* ee = sc + attn_scores_floats(a.ctx);              // their exponentials
  float* ring = ee + attn_scores_floats(a.ctx);            // a.ring slots of kRingRows rows
  const int vstride = kv_vstride(a.kv_tile);
  float* kt = ring + (size_t)a.ring * kSlotFloats;        // [kv_tile][kKVRow] K
  float* vT = kt + (size_t)(a.kv_tile + 16) * kKVRow;      // [64][vstride] V transposed
  // K rows streamed for the scores: [kbeg, kend) in chunks of kRingRows -- positions [nt, pos), or
  // in split mode this workgroup's half of the chunks of [0, pos) (the other half: [obeg, oend))
  const AttnRing ar = attn_ring(pos, a.kv_tile, split, half, kF16);
  const int nt = ar.nt, kbeg = ar.kbeg, kend = ar.kend, obeg = ar.obeg, oend = ar.oend;
  for (int l = 0; l < a.NL; l++) {
    const LayerView& L = a.layers[l];
    if (l > 0) pf_delay(a.pf[2]);
    WR<S::NGD> wq[1];
    wr_load<S::NGD, S::NB8D, 0, S::NGD>(L.qkv, rq, lane, wq[0]);
    float nw[4];
    normw_load<S>(L.attn_norm, nw);
    float bq = 0.0f;
    if (j == 0) bq = gldf(L.bqkv + rq * 16 + r);
    float rc = 0.0f, rsn = 0.0f;
    if (tid < 32) {
      const float2 cs = gld2f(a.rope + (size_t)pos * kHD + 2 * tid);
      rc = cs.x;
      rsn = cs.y;
    }
    const size_t cbase = ((size_t)l * S::KVH + kh) * a.ctx * kHD;
    // stage K and V of positions [0, nt), four 16-byte loads in flight per thread
    for (int i0 = 0; i0 < nt * 32; i0 += 4 * kPThreads) {
      float4 v4[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int idx = i0 + u * kPThreads + tid;
        if (idx < nt * 32) {
          const int which = idx >= nt * 16, rem = idx - which * nt * 16, t = rem >> 4, c4 = (rem & 15) * 4;
          v4[u] = kv_gld4((const KT*)(which ? a.vc : a.kc) + cbase + (size_t)t * kHD + c4);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int idx = i0 + u * kPThreads + tid;
        if (idx < nt * 32) {
          const int which = idx >= nt * 16, rem = idx - which * nt * 16, t = rem >> 4, c4 = (rem & 15) * 4;
          if (which) {
            vT[(c4 + 0) * vstride + t] = v4[u].x;
            vT[(c4 + 1) * vstride + t] = v4[u].y;
            vT[(c4 + 2) * vstride + t] = v4[u].z;
            vT[(c4 + 3) * vstride + t] = v4[u].w;
          } else {
            *reinterpret_cast<float4*>(kt + t * kKVRow + c4) = v4[u];
          }
        }
      }
    }
    // past positions [kbeg, kend) stream through the ring: for the scores in 16-row chunks, wave w
    // taking chunks w, w + 4, ... through its own ring of cs slots (the first ones load during the
    // wait for x); for P.V in slots of kRingRows (or kVRows) rows
    const int nstream = ar.nstream, nck = ar.nck;
    const int nkc = ar.nkc, nloc = attn_nloc(nkc, wave);
    const int cs = kchunk_slots(a.ring);
    float* wring = ring + (size_t)wave * cs * kChunkFloats;
    const KT* kgl = (const KT*)a.kc + cbase;
    const KT* vgl = (const KT*)a.vc + cbase;
    // fp16 K: wide chunks, one row per pair of lanes
    const bool wide = kF16;
    const int ws = kwide_slots(cs), nlw = attn_nloc((nstream + kWideRows - 1) / kWideRows, wave);
    if (wide) {
      if constexpr (kF16)
        if (nlw > 0)
          for (int j = 0; j < ws - 1; j++)
            ring_issue_kw(kgl, kwide_t0(kbeg, j, nlw, wave), kend, wring + (size_t)j * kWideFloats);
    } else if (nloc > 0) {
      for (int j = 0; j < cs - 1; j++)
        ring_issue_kc(kgl, kchunk_t0(kbeg, j, nloc, wave), kend, wring + (size_t)j * kChunkFloats);
    }
    if (l == 0) {
      for (int i = tid; i < S::D; i += kPThreads) stage_x<S>(m, i, embed_value(a.embd, S::D, tok, i));
    } else {
      recv_x<S>(a.ll + S::oX2, phase_epoch(ep0, s, E, 4 * (l - 1) + 3), a.st, m, bad, a.nap);
    }
    if (wg_bad(m.flag, bad)) return false;
    if (mark) prof_mark(a, s, l * 16 + 4);
    prof_wg(a, s, l, 0);
    norm_quant<S>(m, nw, a.eps);
    if (mark) prof_mark(a, s, l * 16 + 9);
    float acc[1] = {0.0f};
    wr_dot<S::NBD, 0, S::NGD, 1>(wq, m.xq, j, acc);
    const float q = hsum4(acc[0]);
    if (j == 0) qv[16 * wave + r] = q + bq;
    __syncthreads();
    if (mark) prof_mark(a, s, l * 16 + 5);
    // RoPE (kernels.c:340-344) of the q pairs
    if (tid < 32) {
      const float x0 = qv[tid], x1 = qv[tid + 32];
      qv[tid] = x0 * rc - x1 * rsn;
      qv[tid + 32] = x1 * rc + x0 * rsn;
    }
    __syncthreads();
    if (mark) prof_mark(a, s, l * 16 + 11);
    // scores: four lane sums over i = j mod 4, hsum, scale (kernels.c:362-366)
    const int T = pos + 1;
    const float scale = 1.0f / __builtin_sqrtf((float)kHD);
    float lmax = -1e30f;
    // staged positions [0, nt): one thread per position
    if (tid < nt) {
      float4 qr[kHD / 4];
#pragma unroll
      for (int i = 0; i < kHD / 4; i++) qr[i] = reinterpret_cast<const float4*>(qv)[i];
#pragma unroll
      for (int i = 0; i < kHD / 4; i++) pin(qr[i]);
      for (int t = tid; t < nt; t += kPThreads) {
        {
          float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
          const float4* kr = reinterpret_cast<const float4*>(kt + t * kKVRow);
          float4 ka[8], kb[8];
#pragma unroll
          for (int i = 0; i < 8; i++) ka[i] = kr[i];
#pragma unroll
          for (int i = 0; i < 8; i++) kb[i] = kr[8 + i];
#pragma unroll
          for (int i = 0; i < 8; i++) pin(ka[i]);
#pragma unroll
          for (int i = 0; i < 8; i++) {
            s0 = s0 + qr[i].x * ka[i].x;
            s1 = s1 + qr[i].y * ka[i].y;
            s2 = s2 + qr[i].z * ka[i].z;
            s3 = s3 + qr[i].w * ka[i].w;
          }
#pragma unroll
          for (int i = 0; i < 8; i++) pin(kb[i]);
#pragma unroll
          for (int i = 0; i < 8; i++) {
            s0 = s0 + qr[8 + i].x * kb[i].x;
            s1 = s1 + qr[8 + i].y * kb[i].y;
            s2 = s2 + qr[8 + i].z * kb[i].z;
            s3 = s3 + qr[8 + i].w * kb[i].w;
          }
          const float sv = (s0 + s1 + s2 + s3) * scale;
          sc[t] = sv;
          lmax = __builtin_fmaxf(lmax, sv);
        }
      }
    }
    // positions [nt, pos) streamed through the ring: 4 threads per position, thread j runs the
    // reference's lane j (i = j mod 4), the lanes are combined in hsum order
    if (nck > 0) {
      const int R = a.ring;
      const int pj = lane & 3, pr = lane >> 2;   // lane pj of row pr of the wave's chunk
      if constexpr (kF16) {
        if (wide && nlw > 0) {
          // lane pair (row t = lane >> 1, h = lane & 1): lane h runs the reference lanes 2h and
          // 2h + 1 of row t's score (elements 4i + 2h and 4i + 2h + 1, each product rounded, then
          // added, i in order); the pair's four lane sums then combine in hsum order
          const int h = lane & 1, tr = lane >> 1;
          float2 qh[kHD / 4];
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) qh[i] = *reinterpret_cast<const float2*>(qv + 4 * i + 2 * h);
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) asm volatile("" : "+v"(qh[i].x), "+v"(qh[i].y));
          const int rot = kwide_rot(tr);
          for (int j = 0; j < nlw; j++) {
            // the chunk ws - 1 ahead into the slot read in the previous iteration, then wait for
            // this one (loads complete in order)
            const int jn = j + ws - 1;
            ring_issue_kw(kgl, kwide_t0(kbeg, jn, nlw, wave), kend, wring + (size_t)(jn % ws) * kWideFloats);
            kwide_wait(ws);
            // dwords h and h + 2 of each piece: elements 8p + 2h, +1 and 8p + 4 + 2h, +1
            const uint32_t* row = reinterpret_cast<const uint32_t*>(wring + (size_t)(j % ws) * kWideFloats) + 32 * tr + h;
            uint32_t dl[8], dh[8];
#pragma unroll
            for (int p = 0; p < 8; p++) {
              const int o = 4 * ((p - rot) & 7);
              dl[p] = row[o];
              dh[p] = row[o + 2];
            }
            float ca = 0.0f, cb = 0.0f;
#pragma unroll
            for (int i = 0; i < kHD / 4; i++) {
              const uint32_t d = (i & 1) ? dh[i >> 1] : dl[i >> 1];
              ca = ca + qh[i].x * half_bits_to_float(d & 0xffffu);
              cb = cb + qh[i].y * half_bits_to_float(d >> 16);
            }
            // lane 2t gets lane 2t + 1's sums (quad_perm [1, 1, 3, 3])
            const float c2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(ca), 0xF5, 0xF, 0xF, true));
            const float c3 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(cb), 0xF5, 0xF, 0xF, true));
            const float sv = (((ca + cb) + c2) + c3) * scale;
            const int t = kwide_t0(kbeg, j, nlw, wave) + tr;
            if (h == 0 && t < kend) {
              sc[t] = sv;
              lmax = __builtin_fmaxf(lmax, sv);
            }
          }
        }
      }
      if (!wide && nloc > 0) {
        float qj[kHD / 4];                        // this lane's reference lane of q
#pragma unroll
        for (int i = 0; i < kHD / 4; i++) qj[i] = qv[4 * i + pj];
        for (int j = 0; j < nloc; j++) {
          kchunk_wait<NKC>(cs);
          // element 4i + pj of chunk row pr
          const float* chunk = wring + (size_t)(j % cs) * kChunkFloats;
          float kr[kHD / 4];
          if (kF16) kchunk_row16(chunk, pr, pj, kr);
          else kchunk_row(chunk, pr, pj, kr);
          // all 16 reads in flight before the first use (else one LDS round trip per step)
          asm volatile("" : "+v"(kr[0]), "+v"(kr[1]), "+v"(kr[2]), "+v"(kr[3]), "+v"(kr[4]), "+v"(kr[5]),
                       "+v"(kr[6]), "+v"(kr[7]), "+v"(kr[8]), "+v"(kr[9]), "+v"(kr[10]), "+v"(kr[11]),
                       "+v"(kr[12]), "+v"(kr[13]), "+v"(kr[14]), "+v"(kr[15]));
          float sj = 0.0f;
#pragma unroll
          for (int i = 0; i < kHD / 4; i++) sj = sj + qj[i] * kr[i];
          // lanes pj = 1, 2, 3 of the quad into lane 0 (DPP quad_perm)
          const float s1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(sj), 0xF9, 0xF, 0xF, true));
          const float s2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(sj), 0xFE, 0xF, 0xF, true));
          const float s3 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(sj), 0xFF, 0xF, 0xF, true));
          const int t = kbeg + 16 * (4 * j + wave) + pr;
          if (pj == 0 && t < kend) {
            const float sv = (((sj + s1) + s2) + s3) * scale;
            sc[t] = sv;
            lmax = __builtin_fmaxf(lmax, sv);
          }
          const int jn = j + cs - 1;
          ring_issue_kc(kgl, kchunk_t0(kbeg, jn, nloc, wave), kend, wring + (size_t)(jn % cs) * kChunkFloats);
        }
      }
      ring_drain();
      __syncthreads();
      prof_wg(a, s, l, 2);
      // the ring is free: the first V slots stream in while exp, sum and division run
      if (!split)
        for (int c = 0; c < R - 1; c++)
          ring_issue(vgl, vslot_t0(nt, c, nck, VR), pos, ring + (size_t)c * kSlotFloats);
    }
    const int nckv = ar.nckv;     // split P.V: half-width V slots
    if (split) {
      // the pair exchanges its scores: publish [kbeg, kend), receive [obeg, oend) (8 entries in
      // flight per thread, missing ones polled again; bounded like every wait)
      const uint32_t eps = phase_epoch(ep0, s, E, 4 * l + 0);
      uint64_t* ex = a.lsc + (size_t)h * a.ctx;
      for (int t = kbeg + tid; t < kend; t += kPThreads) ll_put(ex + t, __float_as_uint(sc[t]), eps);
      if (nckv > 0 && wave != 0)
        for (int c = 0; c < a.ring - 2; c++)
          ring_issue_vp(vgl, vpslot_t0(c, nckv), pos, 32 * half, wave - 1, ring + (size_t)c * kSlotFloats);
      for (int b0 = obeg; b0 < oend; b0 += 8 * kPThreads) {
        uint64_t w[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const int t = b0 + kPThreads * k + tid;
          w[k] = t < oend ? ll_peek(ex + t) : ((uint64_t)eps << 32);
        }
        int spins = 0;
        for (;;) {
          bool ok = true;
#pragma unroll
          for (int k = 0; k < 8; k++) ok = ok && (uint32_t)(w[k] >> 32) == eps;
          if (ok || bad) break;
          for (int z = 0; z < a.nap; z++) __builtin_amdgcn_s_sleep(1);
#pragma unroll
          for (int k = 0; k < 8; k++) {
            const int t = b0 + kPThreads * k + tid;
            if (t < oend && (uint32_t)(w[k] >> 32) != eps) w[k] = ll_peek(ex + t);
          }
          if (++spins > kSpinLimit) {
            bad = true;
            __hip_atomic_store(&a.st->abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else if ((spins & 255) == 0 && __hip_atomic_load(&a.st->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            bad = true;
          }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const int t = b0 + kPThreads * k + tid;
          if (t < oend) sc[t] = __uint_as_float((uint32_t)w[k]);
        }
      }
      if (wg_bad(m.flag, bad)) return false;
      prof_wg(a, s, l, 3);
      for (int t = obeg + tid; t < oend; t += kPThreads) lmax = __builtin_fmaxf(lmax, sc[t]);
    }
    // The softmax over the past positions, while the new K row is on its way.  The new position
    // comes last in the reference's running maximum and sum (kernels.c:362-369), so with the past
    // maximum M the exponentials e_t = fast_exp(s_t - M) and their running sum over t < pos are
    // already the reference's unless the new score exceeds M; then everything is redone with it.
    // Waves 1 and 2 poll for the group's new K and V rows (issued first, so the loads are in
    // flight during the softmax); the barriers in between wait for shared memory only.
    const bool kpoll = tid >= 64 && tid < 64 + 2 * kHD;
    // entry of row li of k (or v): the K/V role's workgroup p = (li & 31) >> 3 writes its 16 rows
    // {8p..8p+7, 32+8p..32+8p+7} as one line, slot (li >> 5) * 8 + (li & 7)
    const int kvt = (tid - 64) & 127, kvli = kvt & 63;
    const uint64_t* ksrc = a.ll + S::oKV + 2 * kh * kHD + (kvt >> 6) * kHD + ((kvli & 31) >> 3) * 16 +
                           (kvli >> 5) * 8 + (kvli & 7);
    const uint32_t ekv = phase_epoch(ep0, s, E, 4 * l + 0);
    uint64_t kw = (uint64_t)ekv << 32;
    if (kpoll) kw = ll_peek(ksrc);
    lmax = max64(lmax);
    if (lane == 0) m.red[wave] = lmax;
    lds_barrier();
    const float mpast = __builtin_fmaxf(__builtin_fmaxf(m.red[0], m.red[1]), __builtin_fmaxf(m.red[2], m.red[3]));
    for (int t = tid; t < ((pos + 31) & ~31); t += kPThreads) ee[t] = t < pos ? fast_exp(sc[t] - mpast) : 0.0f;
    lds_barrier();
    if (tid == 0) {
      m.red[8] = chain_sum(ee, pos);
      prof_after(a, s, l, 6, m.red[8]);
    } else if (kpoll) {
      ll_wait1(ksrc, kw, ekv, a.st, bad, a.nap);
      const float kval = __uint_as_float((uint32_t)kw);
      kv[tid - 64] = kval;    // kv and vv are adjacent: 0..63 K, 64..127 V
      if (wave == 1 && !bad) {
        // wave 1 holds the new K row: the current position's score while wave 0 sums the past
        // ones.  Lane i forms q_i * k_i; lane j < 4 adds the products j, j+4, ... in order, and the
        // four lane sums combine in hsum order (kernels.c:362-366).
        float* pq = m.gu;
        pq[lane] = qv[lane] * kval;
        float pj[kHD / 4];
#pragma unroll
        for (int i = 0; i < kHD / 4; i++) pj[i] = pq[4 * i + (lane & 3)];
        float sj = 0.0f;
#pragma unroll
        for (int i = 0; i < kHD / 4; i++) sj = sj + pj[i];
        const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), 0));
        const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), 1));
        const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), 2));
        const float s3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), 3));
        if (lane == 0) {
          const float sv = (s0 + s1 + s2 + s3) * scale;
          sc[pos] = sv;
          if (sv > mpast) {
            m.red[9] = 1.0f;               // the new score is the maximum: redo below
          } else {
            // e_pos stays out of ee[] until the barrier: wave 0's chain reads the zero padding
            // past pos in whole 32-value chunks
            m.red[10] = fast_exp(sv - mpast);
            m.red[9] = 0.0f;
          }
        }
      }
    }
    if (wg_bad(m.flag, bad)) return false;
    if (mark) prof_mark(a, s, l * 16 + 15);
    prof_wg(a, s, l, 4);
    if (mark) prof_mark(a, s, l * 16 + 12);
    const bool redo = m.red[9] != 0.0f;
    if (redo) {
      const float mx = sc[pos];
      for (int t = tid; t < ((T + 31) & ~31); t += kPThreads) ee[t] = t < T ? fast_exp(sc[t] - mx) : 0.0f;
      __syncthreads();
      if (tid == 0) m.red[8] = chain_sum(ee, T);
      __syncthreads();
    }
    if (mark) prof_mark(a, s, l * 16 + 13);
    // the running sum over every position: the past positions' chain, then the new one's term last
    const float sum = redo ? m.red[8] : m.red[8] + m.red[10];
    for (int t = tid; t < T; t += kPThreads) sc[t] = (t == pos && !redo ? m.red[10] : ee[t]) / sum;
    volatile LdsInt* cnt = (volatile LdsInt*)(m.red + 12);   // split P.V hand-offs (below)
    if (tid < 4) cnt[tid] = 0;
    __syncthreads();
    if (mark) prof_mark(a, s, l * 16 + 14);
    prof_wg(a, s, l, 5);
    // out_i = sum over t in order of p_t * v_t[i] (kernels.c:372-375): staged positions, then the
    // streamed ones slot by slot (wave 0 adds while every wave keeps the ring filled), then pos
    float accv = 0.0f;
    if (split) {
      // this workgroup's 32 output columns over [0, pos) in half-width slots of kVRows rows.  Each
      // producer wave (1..3) streams its 32 rows of every slot, turns them into the products
      // p_t * v_t[i] in place and counts the slot in cnt[pw]; wave 0 waits for all three counts,
      // reads the slot, counts it in cnt[3] and adds the products in position order (each product
      // rounded, then added, as acc + p * v).  Slot c + D reuses the buffer of slot c + D - R
      // once wave 0 has read that; no barrier between the waves.
      const int R = a.ring, D = R - 2;
      if (wave != 0) {
        const int pw = wave - 1;
        for (int c = 0; c < nckv; c++) {
          vpart_wait<NVP>(D);
          float* part = ring + (size_t)(c % R) * kSlotFloats + pw * 1024;
          const float* pc = sc + c * kVRows + 32 * pw;
          if constexpr (kF16) {
            // lane (column pair cp = lane & 15, row group rg = lane >> 4): rows 8 rg .. 8 rg + 7 of the
            // part, columns 2 cp and 2 cp + 1 -- p of its 8 rows in two 16-byte reads, one 4-byte read
            // of V per row, the row's two products in one 8-byte store: 10 reads in flight together
            const int cp = lane & 15, rg = lane >> 4;
            const float4 pa = *reinterpret_cast<const float4*>(pc + 8 * rg);
            const float4 pb = *reinterpret_cast<const float4*>(pc + 8 * rg + 4);
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(part + 512) + 8 * rg * 16 + cp;   // fp16 rows
            uint32_t vv[8];
#pragma unroll
            for (int r = 0; r < 8; r++) vv[r] = vw[r * 16];
            asm volatile("" ::: "memory");   // every read of the part (fp16 rows included) before any write
            const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
            float2* out = reinterpret_cast<float2*>(part) + 8 * rg * 16 + cp;
#pragma unroll
            for (int r = 0; r < 8; r++)
              out[r * 16] = make_float2(pr[r] * half_bits_to_float(vv[r] & 0xffffu), pr[r] * half_bits_to_float(vv[r] >> 16));
          } else {
            float pv[16], vx[16];
#pragma unroll
            for (int k = 0; k < 16; k++) {
              pv[k] = pc[(lane + 64 * k) >> 5];
              vx[k] = part[lane + 64 * k];
            }
            asm volatile("" ::: "memory");   // every read of the part before any write
#pragma unroll
            for (int k = 0; k < 16; k++) part[lane + 64 * k] = pv[k] * vx[k];
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (lane == 0) cnt[pw] = c + 1;
          const int cn = c + D;
          if (!lds_wait_ge(cnt + 3, cn - R + 1)) {
            bad = true;
            break;
          }
          asm volatile("" ::: "memory");
          ring_issue_vp(vgl, vpslot_t0(cn, nckv), pos, 32 * half, pw, ring + (size_t)(cn % R) * kSlotFloats);
        }
      } else {
        for (int c = 0; c < nckv; c++) {
          if (!lds_wait_ge3(cnt, c + 1)) {
            bad = true;
            break;
          }
          asm volatile("" ::: "memory");
          // lanes 0..31 hold this workgroup's columns (lanes 32..63 read the next row, unused)
          const float* slot = ring + (size_t)(c % R) * kSlotFloats + lane;
          const int n = pos - c * kVRows;
          float pr[kVRows];
          if (n >= kVRows) {
            // a full slot, no select on the chain, read in quarters of 24 positions: two quarters
            // ahead at first, then each quarter's reads issued before the one before it is added
            // (12 reads in flight, so every wait is exact)
            constexpr int Q = kVRows / 4;
#pragma unroll
            for (int u = 0; u < 2 * Q; u++) pr[u] = slot[u * 32];
#pragma unroll
            for (int q = 0; q < 4; q++) {
#pragma unroll
              for (int u = q * Q; u < (q + 1) * Q; u++) pin(pr[u]);
              if (q + 2 < 4) {
#pragma unroll
                for (int u = (q + 2) * Q; u < (q + 3) * Q; u++) pr[u] = slot[u * 32];
              }
              if (q == 3) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                // every lane stores the same count: a store under lane == 0 would end the basic
                // block here, and the compiler then sinks all four quarters' additions after it
                cnt[3] = c + 1;
                __builtin_amdgcn_sched_barrier(0);
              }
#pragma unroll
              for (int u = q * Q; u < (q + 1) * Q; u++) accv = accv + pr[u];
              __builtin_amdgcn_sched_barrier(0);
            }
          } else {
#pragma unroll
            for (int u = 0; u < kVRows; u++) pr[u] = slot[u * 32];
#pragma unroll
            for (int u = 0; u < kVRows; u++) pin(pr[u]);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane == 0) cnt[3] = c + 1;
#pragma unroll
            for (int u = 0; u < kVRows; u++) {
              const float t = accv + pr[u];
              accv = u < n ? t : accv;
            }
          }
        }
      }
      ring_drain();
      if (wg_bad(m.flag, bad)) {
        if (tid == 0) __hip_atomic_store(&a.st->abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
      if (tid < 32) {
        const int d = 32 * half + tid;
        accv = accv + sc[pos] * vv[d];
        ll_put(a.ll + S::oATT + h * kHD + d, __float_as_uint(accv), phase_epoch(ep0, s, E, 4 * l + 0));
      }
      if (mark) prof_mark(a, s, l * 16 + 6);
      prof_wg(a, s, l, 1);
      __syncthreads();
      continue;
    }
    if (tid < kHD && nt > 0) accv = seq_dot4(0.0f, sc, vT + tid * vstride, nt);
    if (nck > 0) {
      const int R = a.ring;
      for (int c = 0; c < nck; c++) {
        ring_sync(R);
        if (tid < kHD) {
          const float* slot = ring + (size_t)(c % R) * kSlotFloats + tid;
          const unsigned short* slot16 = reinterpret_cast<const unsigned short*>(ring + (size_t)(c % R) * kSlotFloats) + tid;
#pragma unroll
          for (int hf = 0; hf < VR / kRingRows; hf++) {    // kRingRows rows at a time
            const int r0 = hf * kRingRows;
            const float* pc = sc + nt + c * VR + r0;
            const int n = nstream - c * VR - r0;
            float pv[kRingRows], vx[kRingRows];
#pragma unroll
            for (int u = 0; u < kRingRows; u++) {
              pv[u] = pc[u];
              vx[u] = kF16 ? half_bits_to_float(slot16[(r0 + u) * kHD]) : slot[(r0 + u) * kHD];
            }
            if (n >= kRingRows) {                // full rows: no select on the chain
#pragma unroll
              for (int u = 0; u < kRingRows; u++) accv = accv + pv[u] * vx[u];
            } else {
#pragma unroll
              for (int u = 0; u < kRingRows; u++) {
                const float t = accv + pv[u] * vx[u];
                accv = u < n ? t : accv;
              }
            }
          }
        }
        const int cn = c + R - 1;
        ring_issue(vgl, vslot_t0(nt, cn, nck, VR), pos, ring + (size_t)(cn % R) * kSlotFloats);
      }
      ring_drain();
    }
    if (tid < kHD) {
      accv = accv + sc[pos] * vv[tid];
      ll_put(a.ll + S::oATT + h * kHD + tid, __float_as_uint(accv), phase_epoch(ep0, s, E, 4 * l + 0));
    }
    if (mark) prof_mark(a, s, l * 16 + 6);
    prof_wg(a, s, l, 1);
    __syncthreads();
  }
  return true;
}

// One 32-value block u of the SwiGLU activation: gate rows 32u.., up rows F+32u.. (one 16-row
// group per wave), then silu(gate)*up and quantize_row of the block (kernels.c:390-397).
// The new K (with RoPE) or V rows of one kv group per layer (kernels.c:333-353), 16 rows per
// workgroup: workgroup 8g + 4c + p of the role takes rows {8p .. 8p+7} and {32+8p .. 32+8p+7} of
// group g's 64 k (c = 0) or v (c = 1) rows, so the RoPE pairs (i, i+32) stay together.  RMSNorm +
// quantize of x; each wave forms the terms of its share of the blocks for the 16 rows, wave 0 adds
// them in the reference's order, adds the bias, applies RoPE to k, stores the rows at pos and hands
// them to the group's attention workgroups.
template <class S, int W, class KT>
__device__ __forceinline__ bool kv_step(const PArgs& a, const PSmem& m, uint32_t ep0, int s, int pos, int tok,
                                        bool& bad) {
  constexpr int G0 = split_g0(S::NGD, W), C = split_cnt(S::NGD, W);
  const int tid = threadIdx.x, lane = tid & 63, r = lane >> 2, j = lane & 3;
  const int E = 4 * a.NL + 1;
  const int kidx = lwg(a) - S::nOD - S::H * a.asplit;
  const int kh = kidx >> 3, isv = (kidx >> 2) & 1, p = kidx & 3;
  const int pi = 8 * p + (r & 7);                       // RoPE pair index of this lane's row
  const int li = r < 8 ? pi : 32 + pi;                  // the row within the group's 64
  const int row = S::D + isv * S::KVH * kHD + kh * kHD + li;
  for (int l = 0; l < a.NL; l++) {
    const LayerView& L = a.layers[l];
    if (l > 0) pf_delay(a.pf[2]);
    WR<C> w;
    wr_load_row<S::NGD, S::NB8D, G0, C>(L.qkv, row, lane, w);
    float nw[4];
    normw_load<S>(L.attn_norm, nw);
    float b = 0.0f, rc = 0.0f, rsn = 0.0f;
    if (W == 0 && j == 0) {
      b = gldf(L.bqkv + row);
      if (!isv) {
        const float2 cs = gld2f(a.rope + (size_t)pos * kHD + 2 * pi);
        rc = cs.x;
        rsn = cs.y;
      }
    }
    if (l == 0) {
      for (int i = tid; i < S::D; i += kPThreads) stage_x<S>(m, i, embed_value(a.embd, S::D, tok, i));
    } else {
      recv_x<S>(a.ll + S::oX2, phase_epoch(ep0, s, E, 4 * (l - 1) + 3), a.st, m, bad, a.nap);
    }
    if (wg_bad(m.flag, bad)) return false;
    prof_wg(a, s, l, 0);
    norm_quant<S>(m, nw, a.eps, prof_slot(a, s, l, 7));
    prof_wg(a, s, l, 2);
    wr_terms<S::NBD, G0, C>(w, m.xq, lane, m.terms);
    __syncthreads();
    if constexpr (W == 0) {
      const float v = hsum4(serial_sum<S::NBD>(m.terms, lane)) + b;
      prof_wg(a, s, l, 3);
      // RoPE (kernels.c:340-344): lane 4r holds row i = 8p + r (r < 8) or i + 32 (r >= 8); the
      // partner of the pair sits 32 lanes away
      const float o = __shfl_xor(v, 32);
      float y = v;
      if (!isv) y = r < 8 ? v * rc - o * rsn : v * rc + o * rsn;
      y = (float)(KT)y;    // the value the cache holds (fp16 caches: rounded), also the one handed over
      if (j == 0) {
        const size_t cbase = ((size_t)l * S::KVH + kh) * a.ctx * kHD;
        st_coherent((KT*)(isv ? a.vc : a.kc) + cbase + (size_t)pos * kHD + li, y);
        // the workgroup's 16 rows as one line (slot r: row li), written by one instruction
        ll_put(a.ll + S::oKV + (2 * kh + isv) * kHD + p * 16 + r, __float_as_uint(y), phase_epoch(ep0, s, E, 4 * l + 0));
      }
      prof_wg(a, s, l, 1);
    }
  }
  return true;
}

template <class S>
__device__ __forceinline__ bool gu_step(const PArgs& a, const PSmem& m, uint32_t ep0, int s, bool& bad) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), r = lane >> 2, j = lane & 3;
  const int E = 4 * a.NL + 1;
  const int u = lwg(a) - S::nOD - S::H * a.asplit - S::nKV;
  const int rg = wave < 2 ? 2 * u + wave : S::F / 16 + 2 * u + (wave - 2);
  for (int l = 0; l < a.NL; l++) {
    const LayerView& L = a.layers[l];
    if (l > 0) pf_delay(a.pf[3]);
    WR<S::NGD> w[1];
    wr_load<S::NGD, S::NB8D, 0, S::NGD>(L.gu, rg, lane, w[0]);
    float nw[4];
    normw_load<S>(L.ffn_norm, nw);
    recv_x<S>(a.ll + S::oX1, phase_epoch(ep0, s, E, 4 * l + 1), a.st, m, bad, a.nap);
    if (wg_bad(m.flag, bad)) return false;
    if (u == 0) prof_mark(a, s, l * 16 + 7);
    prof_wg(a, s, l, 0);
    norm_quant<S>(m, nw, a.eps, prof_slot(a, s, l, 7));
    if (u == 0) prof_mark(a, s, l * 16 + 10);
    prof_wg(a, s, l, 2);
    float acc[1] = {0.0f};
    wr_dot<S::NBD, 0, S::NGD, 1>(w, m.xq, j, acc);
    const float v = hsum4(acc[0]);
    if (j == 0) m.gu[16 * wave + r] = v;
    prof_wg(a, s, l, 3);
    __syncthreads();
    // silu(gate) * up, one value per lane of wave 0, then quantize_row of the block; word w of the
    // block (A_j for w = j, B_j for w = 4 + j, kernels.h layout) gathers its four int8 by shuffles
    if (tid < 64) {
      const int i = tid & 31;
      const float g = m.gu[i];
      const float x = div_silu(g, 1.0f + fast_exp(-g)) * m.gu[32 + i];
      const float am = max32(__builtin_fabsf(x));
      const float dd = div_127(am);
      const float id = inv_scale(dd);
      const int q = quant_one(x * id);
      const int w = tid & 7, e0 = ((w >> 2) << 4) + ((w & 3) << 1);
      const int q0 = __shfl(q, e0), q1 = __shfl(q, e0 + 1), q2 = __shfl(q, e0 + 8), q3 = __shfl(q, e0 + 9);
      const uint32_t ep = phase_epoch(ep0, s, E, 4 * l + 2);
      // the whole 16-entry line (entries 9..15 are padding), written by one instruction
      if (tid < 8) ll_put(a.ll + S::oACT + u * kActStride + tid, pack4(q0, q1, q2, q3), ep);
      else if (tid < kActStride) ll_put(a.ll + S::oACT + u * kActStride + tid, __float_as_uint(dd), ep);
    }
    if (u == 0) prof_mark(a, s, l * 16 + 8);
    prof_wg(a, s, l, 1);
  }
  return true;
}

template <class S, class KT>
__global__ __launch_bounds__(kPThreads, 1) void k_decode_persistent(PArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const PSmem m = psmem<S>(smem);
  const uint32_t ep0 = a.st->epoch;
  int pos = a.st->pos0;
  int tok = a.tokens[pos];
  const int wg = lwg(a), wave = wave_id();
  if (threadIdx.x == 0) *m.flag = 0;
  __syncthreads();
  if (wg == 0) prof_mark(a, 0, a.NL * 16 + 3);
  if (a.prof && wg == 0 && threadIdx.x == 0) a.prof[a.NL * 16 + 4] = clock64();
  bool bad = false;
  for (int s = 0; s < a.steps; s++, pos++) {
    bool ok = true;
    if (wg < S::nOD) {
      ok = od_step<S>(a, m, ep0, s, tok, bad);
    } else if (wg < S::nOD + S::H * a.asplit) {
      ok = attn_step<S, KT>(a, m, ep0, s, pos, tok, bad);
    } else if (wg < S::nOD + S::H * a.asplit + S::nKV) {
      switch (wave) {
        case 0: ok = kv_step<S, 0, KT>(a, m, ep0, s, pos, tok, bad); break;
        case 1: ok = kv_step<S, 1, KT>(a, m, ep0, s, pos, tok, bad); break;
        case 2: ok = kv_step<S, 2, KT>(a, m, ep0, s, pos, tok, bad); break;
        default: ok = kv_step<S, 3, KT>(a, m, ep0, s, pos, tok, bad); break;
      }
    } else if (wg < S::nOD + S::H * a.asplit + S::nKV + S::nGU) {
      ok = gu_step<S>(a, m, ep0, s, bad);
    }
    if (!ok) return;
    // resident head row groups in the fp32-cache kernel only: in the fp16-cache kernel the added
    // code slowed the long-context attention loops by 1.5% (code placement), for no gain there
    tok = head_phase<S, sizeof(KT) == 4>(a, m, ep0, s, pos, bad);
    if (tok < 0) return;
  }
  if (wg == 0 && threadIdx.x == 0) {
    const int E = 4 * a.NL + 1;
    a.st->pos0 = pos;
    a.st->next = tok;
    a.st->epoch = ep0 + (uint32_t)(a.steps * E) + 1u;
  }
}

}  // namespace q4
