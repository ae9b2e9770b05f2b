// W4A16 group-128 linear for gfx950: y[M, N] = x[M, K] . W^T (M = 1: GEMV;
// M <= 64: batched decode; more rows: a prompt batch, 16-row tiles in grid.z).
//
// Weights stay in the AutoGPTQ layout.  One int32 word of qweight holds the
// 8 consecutive k of one column, which is exactly the 8 bf16 values one lane
// feeds to v_mfma_f32_16x16x32_bf16 as its B operand, so weights go from a
// global load straight into registers with no LDS staging:
//
//   * lane (c = lane % 16, r = lane / 16) loads, for qweight row 4*kstep + r,
//     LW consecutive words at columns ncol .. ncol+LW-1 (ncol = n0 + LW*c);
//     word t feeds n-tile t, whose MFMA column c is output column ncol + t;
//   * a nibble becomes bf16 (128 + q) with one AND-OR against 0x43004300
//     (bf16 128.0 has a unit of least precision of exactly 1): four AND-ORs
//     and three shifts per word, giving k order (0,4,1,5,2,6,3,7);
//   * the activation operand is permuted into the same k order (the
//     contraction only needs A and B to agree on it);
//   * per chunk of k-steps inside one group the MFMA sums acc = sum x*(128+q)
//     and, against an all-ones B, xs = sum x; the chunk's exact contribution
//     is s * (acc - (128 + z) * xs), accumulated in fp32 (scale after dot).
//
// A workgroup of W waves owns one column block of 16*LW columns and one tile
// of 16 rows (more rows go to grid.z and share the weights through L2; an
// output with few column blocks takes shorter row tiles, so that it still gets
// up to 256 workgroups); its waves split the K range
// (double-buffered chunks of CK k-steps) and their fp32 sums meet in LDS in a
// fixed order, so results do not depend on timing.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "t2i_common.h"
#include "w4a16_tile.h"
#include "qk_prep.h"

namespace t2i {

// XROWS: the activation rows are read whole (see load_chunk); the host picks it for
// row tiles of 8 or 16 rows.  TILED: qweight in the tile layout of
// t2i_w4a16_tile_qweight.
template <int MT, int LW, int W, int CK, bool NORM, bool XROWS, bool TILED, int PRE = 0, bool NXT = false>
__global__ __launch_bounds__(64 * W) void w4a16_mfma_kernel(const uint16_t* x_, const uint32_t* qw_, const uint16_t* sc_,
                                                             const uint32_t* qz_, const uint16_t* aux_, int N_, int M_,
                                                             int K_, int G_, const LinearParams p_) {
  LinearParams p = p_;
  p.x = x_; p.qw = qw_; p.sc = sc_; p.qz = qz_; p.N = N_; p.K = K_; p.ldx = K_; p.chunks = K_ / (32 * CK);
  p.M = M_ & 0xFFFFFF;
  p.rt = 1 << (M_ >> 24);
  if constexpr (NORM) p.gamma = aux_; else p.residual = aux_;
  linear_tile<MT, LW, W, CK, NORM, XROWS, TILED, PRE, NXT>(p, G_, blockIdx.x, blockIdx.z);
}

// qweight [K/8, N] (AutoGPTQ: word row k/8, column n) into the tile layout the
// decode linear reads whole lines of: one 256-word tile per (16-column block cb,
// 128-deep group g), tile cb * (K/128) + g, and in it word row 4 j + r of the
// group, column c at (16 r + c) * 4 + j.  A lane (c, r) of the kernel then finds
// its words of one chunk's k-steps j side by side (16 bytes for 4 k-steps), and a
// workgroup's weights of one column block are one contiguous range.
__global__ void tile_qweight_kernel(const uint32_t* __restrict__ qw, int K, int N, uint32_t* __restrict__ tiles) {
  const int groups = K / GS;
  const size_t total = (size_t)(K / 8) * N;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (size_t)gridDim.x * blockDim.x) {
    const size_t tile = o >> 8;
    const int w = (int)(o & 255);
    const int cb = (int)(tile / groups), g = (int)(tile - (size_t)cb * groups);
    const int j = w & 3, c = (w >> 2) & 15, r = w >> 6;
    tiles[o] = qw[(size_t)(g * 16 + 4 * j + r) * N + cb * 16 + c];
  }
}

// ============================================================================
// Prompt-sized GEMM (hundreds of rows and more): a 64 x 128 output tile per
// 256-thread workgroup, 4 waves of 64 x 32 (1 along M x 4 along N), one 128-k
// tile (= one quantisation group) per step.  Each wave rebuilds the bf16 operand
// of its own 32 columns only, and the weights are unpacked in k order
// (b_operand_kord), so the activation fragments go to the MFMA as they lie in
// LDS: 158 VALU instructions a wave per k-tile against 238 for 2 x 2 waves of
// 32 x 64 (which rebuilt each column's operand in both wave rows and permuted
// every activation fragment), for 48 MFMAs against 40 (each wave sums all 64
// rows).  Measured at 8192 rows: qkv 117 -> 107 us, gate_up with SwiGLU 184 ->
// 170 us, down with the residual 90 -> 79-82 us, o_proj unchanged at ~60 us;
// the outputs are bit-identical.  51 KB of LDS and at most 168
// registers a lane (launch bounds) let three workgroups share a CU, so the
// others' k-loops cover one's barriers, prologue and epilogue, and the VALU and
// MFMA work of three waves a SIMD interleave (measured against two workgroups a
// CU with three stage buffers, for this tile too: qkv 107 -> 117 us, o_proj 62
// -> 70 us; and against one 128 x 128 workgroup of 8 waves a CU before that).
//   * Every operand of a k-tile (activations, packed weights, the group's scale
//     and zero words) is loaded straight into LDS (global_load_lds, no
//     registers); two stage buffers: k-tile kt + 1 loads while kt is computed.
//   * The pipeline's waits are all explicit: a wave waits (vmcnt) until its own
//     loads of the k-tile it is about to compute have landed, the workgroup meets
//     at a barrier (then everyone's have), and LDS is read with ds_read in inline
//     asm followed by explicit lgkmcnt waits.  The compiler's own waits for loads
//     into LDS cover every load in flight (no per-buffer tracking across a loop),
//     which would serialise the pipeline, and __syncthreads would do the same.
//   * LDS holds each A fragment as 64 lanes x 16 bytes (row c, k 8 r .. 8 r + 7
//     of lane 16 r + c, in memory order: one contiguous read, no bank conflicts);
//     the packed weights as the k-tile's 16 qweight rows in pairs (one 1 KB load
//     per pair, 128 bytes of padding between pairs: the four rows of a fragment
//     read meet two-way bank conflicts at most).
//   * Arithmetic as the decode kernel: MFMA over bf16(128 + q), per group and
//     column total += scale * (dot + zb * rowsum).  The row sums come either from
//     an all-ones MFMA per row fragment (XSP = 0: a third of the matrix-core work,
//     since every wave sums all 64 rows), or precomputed by the kernel that wrote
//     x (XSP = 1: one fp32 sum a row and group; XSP = 2: two half-group sums),
//     loaded into LDS with the k-tile (16 of 48 MFMAs a wave per k-tile go): at
//     8192 rows qkv 110 -> 104 us, o_proj 55.7 -> 53.1 us, gate_up with SwiGLU
//     152 -> 144 us, down 77.4 -> 76.8 us (same box, interleaved rounds).
// ============================================================================
constexpr int GM_BM = 64, GM_BN = 128;
constexpr int GM_WAVES = 4;
constexpr int GM_THREADS = 64 * GM_WAVES;
constexpr int GM_WCOLS = 32;                             // columns per wave
constexpr int GM_WN = GM_BN / GM_WCOLS;                  // waves along N (4)
constexpr int GM_NJ = GM_WCOLS / 16;                     // 16-column n-tiles per wave (2)
constexpr int GM_MF = GM_BM / (GM_WAVES / GM_WN) / 16;   // 16-row fragments per wave (4)
constexpr int GM_AF = GM_BM / 16 * KSG;       // A fragments per k-tile (1 KB each)
constexpr int GM_AF_W = GM_AF / GM_WAVES;     // issued per wave
constexpr int GM_BPAIR = GS / 8 / 2;          // qweight row pairs per k-tile (1 KB each with GM_BN = 128)
constexpr int GM_BROW = GM_BN;                // words per qweight row of the tile
constexpr int GM_BPAIR_W = 2 * GM_BROW + 32;  // words per padded row pair
constexpr int GM_BPAIR_PW = GM_BPAIR / GM_WAVES;   // weight row pairs loaded per wave
static_assert(GM_BPAIR % GM_WAVES == 0 && GM_BN == 128, "whole weight row pairs per wave, 1 KB loads");
constexpr int GM_STAGES = 2;
// epilogue: each wave parks its 64 x 32 results as bf16 in LDS (rows padded to
// 40 values) and stores them back as 16-byte row pieces
constexpr int GM_EP_LD = GM_WCOLS + 8;
constexpr int GM_EP_WAVE = 2 * GM_BM * GM_EP_LD;   // two regions (paired: gate and up outputs)

struct GemmStage {
  u32x4 a[GM_AF * 64];
  uint32_t b[GM_BPAIR * GM_BPAIR_W];
  uint32_t qs[64];          // fp16 scales of the tile's 128 columns, two per word
  uint32_t qz[64];          // qzeros words of the tile's columns (16 used)
  float xs[2 * GM_BM];      // precomputed row sums of the k-tile (XSP > 0): part u of row i at 64 u + i
};
static_assert(GM_WAVES * GM_EP_WAVE * 2 <= (int)sizeof(GemmStage) * GM_STAGES, "epilogue fits in the stages");

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)lds, 4, 0, 0);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// LDS reads at addr + OFF, OFF in the instruction's 16-bit offset field (no
// address arithmetic per read).
template <int OFF = 0>
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t lds_read4(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// Workgroup barrier that orders memory accesses for the compiler without the
// hardware waits of __syncthreads (loads it must cover are waited for first).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// k-tile kt into stage st (rows past M reload row M - 1; their outputs are never
// stored).  Each wave loads its A fragments and weight row pairs; wave 0 also the
// scale and zero words, wave 1 the precomputed row sums (XSP > 0).
template <int XSP>
__device__ __forceinline__ void gemm_issue(const LinearParams& p, int m0, int n0, int kt, int wave, int lane,
                                           GemmStage& st) {
  if constexpr (XSP > 0) {
    if (wave == 1) {
      // group-major sums: the k-tile's 64 rows are 256 contiguous bytes a part
      const float* src = p.xs + (size_t)(kt * XSP) * p.ldxs + min(m0 + lane, p.M - 1);
#pragma unroll
      for (int u = 0; u < XSP; ++u) lds_dma4(src + (size_t)u * p.ldxs, &st.xs[GM_BM * u]);
    }
  }
  const int c = lane & 15, r = lane >> 4;
#pragma unroll
  for (int i = 0; i < GM_AF_W; ++i) {
    const int f = wave * GM_AF_W + i, mi = f / KSG, ks = f % KSG;
    const int m = min(m0 + 16 * mi + c, p.M - 1);
    lds_dma16(p.x + (size_t)m * p.ldx + kt * GS + 32 * ks + 8 * r, &st.a[f * 64]);
  }
  // qweight row pair q = rows 2 q, 2 q + 1 of the k-tile: lane l takes words 4 (l % 32) .. + 3 of row 2 q + l / 32
#pragma unroll
  for (int i = 0; i < GM_BPAIR_PW; ++i) {
    const int q = wave * GM_BPAIR_PW + i;
    lds_dma16(p.qw + (size_t)(kt * (GS / 8) + 2 * q + (lane >> 5)) * p.N + n0 + 4 * (lane & 31),
              &st.b[q * GM_BPAIR_W]);
  }
  if (wave == 0) {
    lds_dma4(p.sc + (size_t)kt * p.N + n0 + 2 * lane, &st.qs[0]);
    lds_dma4(p.qz + (size_t)kt * (p.N >> 3) + (n0 >> 3) + min(lane, GM_BN / 8 - 1), &st.qz[0]);
  }
}


// Fragments of k-step ks: A of this wave's rows, B of its columns.
struct GemmFrags {
  u32x4 a[GM_MF];
  uint32_t b[GM_NJ];
};

// abase: this lane's slot of the first A fragment; bbase: this lane's word of
// k-step 0, fragment 0 (qweight row r = lane / 16, column 32 wn + c).  Every
// other read is a constant offset from these.
template <int KS, int I = 0>
__device__ __forceinline__ void gemm_read(uint32_t abase, uint32_t bbase, GemmFrags& f) {
  if constexpr (I < GM_MF) {
    f.a[I] = lds_read16<(I * KSG + KS) * 1024>(abase);
    gemm_read<KS, I + 1>(abase, bbase, f);
  } else if constexpr (I < GM_MF + GM_NJ) {
    constexpr int j = I - GM_MF;   // qweight row 4 KS + r, column 32 wn + 16 j + c
    f.b[j] = lds_read4<4 * (2 * KS * GM_BPAIR_W + 16 * j)>(bbase);
    gemm_read<KS, I + 1>(abase, bbase, f);
  }
}

// Waits for the LDS reads in flight except the most recent N (register ties keep
// the uses of the waited fragments after the wait).
template <int N>
__device__ __forceinline__ void wait_lds(GemmFrags& f) {
  static_assert(GM_MF == 4 && GM_NJ == 2, "the waits tie four A fragments and two B words");
  static_assert(N == 0 || N == GM_MF + GM_NJ, "one k-step of fragments or none");
  if constexpr (N == 0)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f.a[0]), "+v"(f.a[1]), "+v"(f.a[2]), "+v"(f.a[3]), "+v"(f.b[0]),
                 "+v"(f.b[1]));
  else
    asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(f.a[0]), "+v"(f.a[1]), "+v"(f.a[2]), "+v"(f.a[3]), "+v"(f.b[0]),
                 "+v"(f.b[1]));
}

// k-step KS of a k-tile: read k-step KS + 1's fragments into nxt, then compute
// KS from cur (read one k-step earlier).  OWN: the row sums by all-ones MFMAs.
template <int KS, bool OWN>
__device__ __forceinline__ void gemm_kstep(uint32_t abase, uint32_t bbase, GemmFrags& cur, GemmFrags& nxt,
                                           uint32_t magic, f32x4 (&P)[GM_MF][GM_NJ], f32x4 (&xs)[GM_MF]) {
  if constexpr (KS + 1 < KSG) {
    gemm_read<KS + 1>(abase, bbase, nxt);
    wait_lds<GM_MF + GM_NJ>(cur);
  } else {
    wait_lds<0>(cur);
  }
  const bf16x8 ones = ones_operand();
  bf16x8 b[GM_NJ];
#pragma unroll
  for (int j = 0; j < GM_NJ; ++j) b[j] = b_operand_kord(cur.b[j], magic);
#pragma unroll
  for (int mi = 0; mi < GM_MF; ++mi) {
    const bf16x8 a = __builtin_bit_cast(bf16x8, cur.a[mi]);
    if constexpr (OWN) xs[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, xs[mi], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < GM_NJ; ++j) P[mi][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[j], P[mi][j], 0, 0, 0);
  }
  if constexpr (KS + 1 < KSG) gemm_kstep<KS + 1, OWN>(abase, bbase, nxt, cur, magic, P, xs);
}

template <int XSP>
__device__ __forceinline__ void gemm_compute(const GemmStage& st, int wn, int lane, int ncol0,
                                             f32x4 (&total)[GM_MF][GM_NJ]) {
  const uint32_t abase = lds_addr(&st.a[0]) + 16 * lane;
  // lane (r, c): qweight row 4 ks + r = pair 2 ks + r / 2, row r % 2 of the pair; column 32 wn + c
  const int rr = lane >> 4, cc = lane & 15;
  const uint32_t bbase =
      lds_addr(&st.b[0]) + 4 * ((rr >> 1) * GM_BPAIR_W + (rr & 1) * GM_BROW + GM_WCOLS * wn + cc);
  // this lane's columns: ncol0 + 16 j, tile-local lc + 16 j; their scales are words
  // (lc >> 1) + 8 j, their zero words (lc >> 3) + 2 j
  const int lc = ncol0 & (GM_BN - 1);
  const uint32_t sbase = lds_addr(&st.qs[0]) + 4 * (lc >> 1);
  const uint32_t zbase = lds_addr(&st.qz[0]) + 4 * (lc >> 3);
  static_assert(GM_NJ == 2, "two scale and zero words a lane");
  uint32_t sw[GM_NJ], zw[GM_NJ];
  sw[0] = lds_read4<0>(sbase);  zw[0] = lds_read4<0>(zbase);
  sw[1] = lds_read4<32>(sbase); zw[1] = lds_read4<8>(zbase);
  // precomputed row sums: rows 16 mi + 4 r .. + 3 of part u lie together at 64 u + 16 mi + 4 r
  f32x4 xs[GM_MF], xs2[GM_MF];
  if constexpr (XSP > 0) {
    const uint32_t xbase = lds_addr(&st.xs[0]) + 16 * (lane >> 4);
    xs[0] = __builtin_bit_cast(f32x4, lds_read16<0>(xbase));
    xs[1] = __builtin_bit_cast(f32x4, lds_read16<64>(xbase));
    xs[2] = __builtin_bit_cast(f32x4, lds_read16<128>(xbase));
    xs[3] = __builtin_bit_cast(f32x4, lds_read16<192>(xbase));
    if constexpr (XSP == 2) {
      xs2[0] = __builtin_bit_cast(f32x4, lds_read16<256>(xbase));
      xs2[1] = __builtin_bit_cast(f32x4, lds_read16<320>(xbase));
      xs2[2] = __builtin_bit_cast(f32x4, lds_read16<384>(xbase));
      xs2[3] = __builtin_bit_cast(f32x4, lds_read16<448>(xbase));
    }
  }
  static_assert(GM_MF == 4, "four row fragments of precomputed sums");
  const uint32_t magic = magic_vgpr();
  f32x4 P[GM_MF][GM_NJ];
#pragma unroll
  for (int mi = 0; mi < GM_MF; ++mi) {
    if constexpr (XSP == 0) xs[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < GM_NJ; ++j) P[mi][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  GemmFrags f0, f1;
  gemm_read<0>(abase, bbase, f0);
  gemm_kstep<0, XSP == 0>(abase, bbase, f0, f1, magic, P, xs);
  // The scale, zero and row-sum reads were issued first: done with the last wait,
  // which the empty asm orders before their uses.
  asm volatile("" : "+v"(sw[0]), "+v"(sw[1]), "+v"(zw[0]), "+v"(zw[1]));
  if constexpr (XSP > 0) {
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi) asm volatile("" : "+v"(xs[mi]));
  }
  if constexpr (XSP == 2) {
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi) {
      asm volatile("" : "+v"(xs2[mi]));
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[mi][i] += xs2[mi][i];
    }
  }
  const int zshift = (ncol0 & 7) * 4;   // the same for every fragment (16 j keeps the low bits)
  const bool odd = ncol0 & 1;
#pragma unroll
  for (int j = 0; j < GM_NJ; ++j) {
    const float zb = -(float)(128 + 1 + ((zw[j] >> zshift) & 0xFu));
    const float sc = f16_to_f32(odd ? (sw[j] >> 16) : (sw[j] & 0xFFFFu));
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) total[mi][j][i] = fmaf(sc, fmaf(zb, xs[mi][i], P[mi][j][i]), total[mi][j][i]);
  }
}

template <int XSP>
__global__ __launch_bounds__(GM_THREADS, 3) void w4a16_gemm_kernel(const LinearParams p, const QkvPrepParams pp) {
  __shared__ GemmStage stg[GM_STAGES];
  const int lane = threadIdx.x & 63;
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // the wave's 32-column slice
  const int c = lane & 15, r = lane >> 4;
  // tiles in row-major order (row tile major), each XCD taking one contiguous
  // range of them so that the row tiles it works on stay in its L2
  const int MT = (p.M + GM_BM - 1) / GM_BM, NT = p.N / GM_BN;
  const int T = MT * NT, id = blockIdx.x;
  const int tile = (T & 7) ? id : (id & 7) * (T >> 3) + (id >> 3);
  const int m0 = (tile / NT) * GM_BM, n0 = (tile % NT) * GM_BN;
  const int ncol0 = n0 + GM_WCOLS * wn + c;   // this lane's column in n-tile 0
  const int KT = p.K / GS;

  f32x4 total[GM_MF][GM_NJ];
#pragma unroll
  for (int mi = 0; mi < GM_MF; ++mi)
#pragma unroll
    for (int j = 0; j < GM_NJ; ++j) total[mi][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step kt: load k-tile kt + 1 into the other stage (its last reader, k-tile
  // kt - 1, is done: every wave met the barrier after it), compute k-tile kt, then
  // wait until this wave's loads of kt + 1 have landed and meet the other waves
  // (then everyone's have).  The last step issues no loads, so nothing is in
  // flight when the epilogue starts.
  gemm_issue<XSP>(p, m0, n0, 0, wn, lane, stg[0]);
  wait_vm<0>();
  lds_barrier();
  int kt = 0;
  for (; kt + 1 < KT; ++kt) {
    gemm_issue<XSP>(p, m0, n0, kt + 1, wn, lane, stg[(kt + 1) & 1]);
    gemm_compute<XSP>(stg[kt & 1], wn, lane, ncol0, total);
    wait_vm<0>();
    lds_barrier();
  }
  gemm_compute<XSP>(stg[kt & 1], wn, lane, ncol0, total);
  lds_barrier();   // every wave is done reading the stages: they become the epilogue's tiles

  // ---- epilogue: total[mi][j][i] is row 16 mi + 4 r + i, column 32 wn + 16 j + c
  // of the tile.  Each wave parks its bf16 results in its own LDS region,
  // row-major, then stores them as 16-byte row pieces (a lane's MFMA outputs are
  // one column of four rows, which would take 2-byte stores).
  uint16_t* ep = reinterpret_cast<uint16_t*>(&stg[0]) + wn * GM_EP_WAVE;
  const int ncolw = n0 + GM_WCOLS * wn;        // the wave's first column
  if (p.epi == EPI_QKV_PREP) {
    // The 64 x 128 tile is one head of rows m0 .. m0 + 63: every wave parks its 32
    // columns, then each 16-lane row g = 4 wn + r takes tile rows g, g + 16, g + 32,
    // g + 48 through prep_vector, as prefill_prep_kernel does for the same rows.
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < GM_NJ; ++j)
          ep[(16 * mi + 4 * r + i) * GM_EP_LD + 16 * j + c] = (uint16_t)f32_to_bf16(total[mi][j][i]);
    const int head = n0 / ATT_D;   // uniform: q heads, then k, then v
    const bool isq = head < pp.Hq;
    const bool normed = head < pp.Hq + pp.Hkv;
    const u32x4 gv = prep_load(isq ? pp.qn : pp.kn, c, pp.style);   // loaded (unused) for v too
    __syncthreads();   // the other waves' columns are in LDS (waits for the stores, unlike lds_barrier)
    const uint16_t* tile = reinterpret_cast<const uint16_t*>(&stg[0]);
    const int g = 4 * wn + r;
#pragma unroll
    for (int rr = 0; rr < GM_BM / 16; ++rr) {
      const int row = g + 16 * rr;
      const int m = m0 + row;
      if (m >= p.M) continue;   // uniform over the 16-lane row
      const int b = m / pp.T, t = m - b * pp.T, pos = pp.p0 + t;
      // the lane's piece (prep_load's layout): column col of the tile lies in wave
      // col / 32's region at col % 32
      u32x4 raw;
      if (pp.style == 0) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(tile + (c >> 3) * GM_EP_WAVE + row * GM_EP_LD + 4 * (c & 7));
        const u32x2 hi =
            *reinterpret_cast<const u32x2*>(tile + (2 + (c >> 3)) * GM_EP_WAVE + row * GM_EP_LD + 4 * (c & 7));
        raw = u32x4{lo.x, lo.y, hi.x, hi.y};
      } else {
        raw = *reinterpret_cast<const u32x4*>(tile + (c >> 2) * GM_EP_WAVE + row * GM_EP_LD + 8 * (c & 3));
      }
      // v heads pass through (the branch is uniform over the workgroup)
      u32x4 y = raw;
      if (normed) {
        const u32x4 rp = *reinterpret_cast<const u32x4*>(pp.rope + (size_t)pos * ATT_D + 8 * c);
        y = prep_vector(raw, rp, gv, true, pp.style, pp.eps);
      }
      uint16_t* dst;
      if (isq) dst = pp.q + (((size_t)b * pp.Hq + head) * pp.T + t) * ATT_D;
      else if (normed) dst = pp.kc + (((size_t)b * pp.Hkv + (head - pp.Hq)) * pp.cap + pos) * ATT_D;
      else dst = pp.vc + (((size_t)b * pp.Hkv + (head - pp.Hq - pp.Hkv)) * pp.cap + pos) * ATT_D;
      prep_store(dst, c, pp.style, y);
    }
  } else if (p.epi == EPI_STORE || p.epi == EPI_RESIDUAL) {
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < GM_NJ; ++j)
          ep[(16 * mi + 4 * r + i) * GM_EP_LD + 16 * j + c] = (uint16_t)f32_to_bf16(total[mi][j][i]);
    __builtin_amdgcn_wave_barrier();
    // 64 rows x 32 columns = 256 pieces of 8 values, 4 a lane
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = lane + 64 * u, row = q >> 2, ch = q & 3;
      const int m = m0 + row;
      const size_t off = (size_t)min(m, p.M - 1) * p.ldy + ncolw + 8 * ch;
      u32x4 v = *reinterpret_cast<const u32x4*>(ep + row * GM_EP_LD + 8 * ch);
      if (p.epi == EPI_RESIDUAL) {
        const u32x4 rv = *reinterpret_cast<const u32x4*>(p.residual + off);
        v.x = pack_bf16x2(bf16_lo(v.x) + bf16_lo(rv.x), bf16_hi(v.x) + bf16_hi(rv.x));
        v.y = pack_bf16x2(bf16_lo(v.y) + bf16_lo(rv.y), bf16_hi(v.y) + bf16_hi(rv.y));
        v.z = pack_bf16x2(bf16_lo(v.z) + bf16_lo(rv.z), bf16_hi(v.z) + bf16_hi(rv.z));
        v.w = pack_bf16x2(bf16_lo(v.w) + bf16_lo(rv.w), bf16_hi(v.w) + bf16_hi(rv.w));
      }
      if (m < p.M) *reinterpret_cast<u32x4*>(p.y0 + off) = v;
    }
  } else {
    // interleaved pairs: gate in the even column, up in the odd one; output column
    // (32 wn + 16 j + c) / 2 of the tile's 64.  SwiGLU: of MFMA rows i0, i0 + 1 the
    // even lane computes row i0 and the odd lane row i0 + 1 (one exchange gives
    // each its other operand), so every lane evaluates SiLU 16 times, not 32;
    // results go to region 0.  Paired: gate to region 0, up to region 1.
    const bool odd = c & 1;
#pragma unroll
    for (int mi = 0; mi < GM_MF; ++mi)
#pragma unroll
      for (int j = 0; j < GM_NJ; ++j) {
        if (p.epi == EPI_SWIGLU) {
#pragma unroll
          for (int i0 = 0; i0 < 4; i0 += 2) {
            const float send = odd ? total[mi][j][i0] : total[mi][j][i0 + 1];
            const float recv = __shfl_xor(send, 1, 64);
            const float g = round_bf16(odd ? recv : total[mi][j][i0]);
            const float u = round_bf16(odd ? total[mi][j][i0 + 1] : recv);
            const int row = 16 * mi + 4 * r + i0 + (odd ? 1 : 0);
            ep[row * GM_EP_LD + 8 * j + (c >> 1)] = (uint16_t)f32_to_bf16(round_bf16(silu_fast(g)) * u);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            ep[(16 * mi + 4 * r + i) * GM_EP_LD + 8 * j + (c >> 1) + (odd ? GM_BM * GM_EP_LD : 0)] =
                (uint16_t)f32_to_bf16(total[mi][j][i]);
        }
      }
    __builtin_amdgcn_wave_barrier();
    // 64 rows x 16 output columns per region = 128 pieces of 8 values, 2 a lane
    const int regions = p.epi == EPI_SWIGLU ? 1 : 2;
    for (int reg = 0; reg < regions; ++reg) {
      uint16_t* dst = reg ? p.y1 : p.y0;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = lane + 64 * u, row = q >> 1, ch = q & 1;
        const int m = m0 + row;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ep + reg * GM_BM * GM_EP_LD + row * GM_EP_LD + 8 * ch);
        if (m < p.M) *reinterpret_cast<u32x4*>(dst + (size_t)m * p.ldy + (ncolw >> 1) + 8 * ch) = v;
      }
    }
    if (p.epi == EPI_SWIGLU && p.ys) {
      // The tile's 64 output columns are one half group of the next product's k:
      // wave 0 sums each row (lane = row) over the four waves' regions in a fixed
      // order, for that product's row sums.
      __syncthreads();   // every wave's region is written
      if (wn == 0) {
        const uint16_t* base = reinterpret_cast<const uint16_t*>(&stg[0]) + lane * GM_EP_LD;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < GM_WAVES; ++w) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(base + w * GM_EP_WAVE + 8 * h);
            s += (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) + (bf16_lo(v.z) + bf16_hi(v.z)) +
                 (bf16_lo(v.w) + bf16_hi(v.w));
          }
        }
        const int m = m0 + lane;
        if (m < p.M) p.ys[(size_t)(n0 >> 7) * p.ldys + m] = s;
      }
    }
  }
}

__global__ void dequant_f32_kernel(const uint32_t* __restrict__ qw, const uint32_t* __restrict__ qz,
                                   const uint16_t* __restrict__ sc, int K, int N, float* __restrict__ W) {
  const int n = blockIdx.x;
  const int row = blockIdx.y * blockDim.x + threadIdx.x;   // qweight row = k / 8
  if (row >= K / 8) return;
  const uint32_t w = qw[(size_t)row * N + n];
  const int g = row / (GS / 8);
  const float s = f16_to_f32(sc[(size_t)g * N + n]);
  const int z = (int)((qz[(size_t)g * (N >> 3) + (n >> 3)] >> (4 * (n & 7))) & 0xFu) + 1;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = (float)((int)((w >> (4 * j)) & 0xFu) - z) * s;
  float* dst = W + (size_t)n * K + row * 8;
  *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
  *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
}

}  // namespace t2i

// ============================================================================
// host side
// ============================================================================
namespace t2i_host {

using namespace t2i;

// Compiled tile configurations: (MT m-tiles, LW words per lane, W waves, CK k-steps per chunk).
// Row tiles beyond 16 rows go to grid.z, except for the 64-column outputs that
// two m-tiles bring from one-to-two rounds of the CUs to one (plan_linear).
#define T2I_LINEAR_CONFIGS(X) \
  X(2, 4, 8, 4)               \
  X(1, 1, 8, 2)               \
  X(1, 1, 8, 4)               \
  X(1, 1, 16, 4)              \
  X(1, 1, 16, 2)              \
  X(1, 2, 16, 4)              \
  X(1, 2, 16, 2)              \
  X(1, 2, 8, 4)               \
  X(1, 4, 8, 4)               \
  X(1, 4, 4, 4)               \
  X(1, 8, 4, 4)

bool config_exists(int MT, int LW, int W, int CK) {
#define T2I_MATCH(a, b, c, d) if (MT == a && LW == b && W == c && CK == d) return true;
  T2I_LINEAR_CONFIGS(T2I_MATCH)
#undef T2I_MATCH
  return false;
}

void finish_plan(LinearPlan& pl, int M, int K, int N) {
  pl.cbs = N / (16 * pl.LW);
  pl.chunks = K / (32 * pl.CK);
  // Row tiles shorter than 16 rows when the column blocks alone leave CUs idle:
  // every workgroup reads all K of its rows, so at 64 column blocks and 16 rows a
  // workgroup reads 4x more activation than weight bytes; 4 tiles of 4 rows give
  // 256 workgroups of a quarter of that (the tiles of a column block share its
  // weights in one L2, see xcd_block).  Measured on the Qwen3-0.6B o_proj / down
  // (64 column blocks): 4.6 -> 3.8 and 5.9 -> 4.7 us at M = 16, 5.0 -> 4.5 us
  // (down, M = 8).  More than 256 workgroups (two a CU) measured slower at every
  // point, and so did narrower column blocks at M = 1 (4 or 8 columns of the 16
  // MFMA columns: no faster, or 3 % slower).
  pl.rt = 16 * pl.MT;
  while (pl.MT == 1 && pl.rt > 1 && pl.cbs * ((M + pl.rt / 2 - 1) / (pl.rt / 2)) <= 256) pl.rt /= 2;
#ifdef T2I_TUNING
  if (const char* env = getenv("T2I_RT")) {
    const int rt = atoi(env);
    if (pl.MT == 1 && rt >= 1 && rt <= 16 && (rt & (rt - 1)) == 0) pl.rt = rt;
  }
#endif
  pl.mz = (M + pl.rt - 1) / pl.rt;
}

// Tile choice, from an HBM-cold sweep (graph-launched, 42-300 weight copies)
// of every Qwen3-0.6B / 1.7B linear shape at M in {1, 8, 16, 32, 64} over all
// compiled plans: one 16-row tile per workgroup (more rows go to grid.z and
// share the weights in their XCD's L2), and the narrowest column block that
// keeps the column-block x row-tile count at 256 or less: 16 columns (1 word
// per lane, 16 waves, chunks of 2 k-steps; 8 waves up to 16 rows, see the end),
// else 32 (2 words, 8 waves), else 64 (4 words, 8 waves).  The rule picks the
// measured optimum, or a plan within 4 % of it, at 38 of the 40 shape/M points,
// and is within 9 % at all.  Splitting K across workgroups was measured slower:
// the fp32 partials and an arrival counter add memory round trips that cost
// more than the parallelism they add at these sizes, so K is only split
// between the waves of a workgroup.
LinearPlan plan_linear(int M, int K, int N, bool paired, bool norm, bool wide) {
  LinearPlan pl{};
  pl.MT = 1;
  pl.CK = 4;
  const int mz = (M + 15) / 16;
  if (((N / 16) * mz <= 256 || N % 32) && !paired) {
    // (N not a multiple of 32: 16-column blocks are the only whole ones)
    pl.LW = 1; pl.W = 16; pl.CK = 2;
  } else if ((N / 32) * mz <= 256 || N % 64) {
    // The fused-norm paired (RMSNorm + gate/up) output takes 8 waves of 4-step
    // chunks like the plain one (0.12-0.18 us faster than 16 waves of 2-step
    // chunks on the Qwen3-0.6B gate_up at M <= 16, at 148 registers a lane);
    // 16-wave workgroups (wide) take 16 waves of 2-step chunks.
    pl.LW = 2;
    pl.W = paired && norm && wide ? 16 : 8;
    pl.CK = paired && norm && wide ? 2 : 4;
  } else {
    pl.LW = 4; pl.W = 8;
    // Two 16-row m-tiles a workgroup (each weight dequantised once for 32 rows)
    // when the one-tile plan would need between one and two rounds of the 256
    // CUs: then one round.  Measured HBM-cold (us a launch, one tile -> two):
    // Qwen3-0.6B gate_up at M = 64 6.56 -> 5.79, Qwen3-1.7B gate_up at M = 32
    // 9.72 -> 9.09; at 2 or more rounds (Qwen3-1.7B gate_up, M = 64) and at
    // every other plan, one tile is faster.  Outputs carry the one-tile plan's
    // bits (the rows of an MFMA tile are independent).
    const int groups = (N / 64) * mz;
    if (!norm && !wide && groups > 256 && groups <= 512) pl.MT = 2;
  }
  bool chosen = false;   // tuning builds: a plan given in T2I_PLAN is kept as given
#ifdef T2I_TUNING
  // tuning builds only: T2I_PLAN="MT,LW,W,CK" overrides the choice
  if (const char* env = getenv("T2I_PLAN")) {
    LinearPlan o = pl;
    if (sscanf(env, "%d,%d,%d,%d", &o.MT, &o.LW, &o.W, &o.CK) == 4 && config_exists(o.MT, o.LW, o.W, o.CK) &&
        N % (16 * o.LW) == 0 && (!paired || o.LW >= 2)) {
      pl = o;
      chosen = true;
    }
  }
#endif
  finish_plan(pl, M, K, N);
  // 16-column blocks: 8 waves of 4-step chunks when each wave holds at most 3
  // chunks (K <= 3072: the straight schedules): half the partial sums to reduce
  // and half the waves to meet at the barrier, the same loads in flight.  The K
  // split then depends on the shape alone, so a row's outputs do not depend on
  // how many rows share the launch.  Measured HBM-cold with the chunk loads in use
  // order (us a launch, the previous plan -> this one): Qwen3-0.6B qkv 2.92 -> 2.88
  // (M = 1), 3.09 -> 2.92 (M = 8), 3.23 -> 3.14 (M = 16), with the fused norm 3.86
  // -> 3.69 (M = 16); o_proj 3.68 -> 3.46 (M = 32), 4.05 -> 3.88 (M = 64);
  // Qwen3-1.7B qkv 3.91 -> 3.82 (M = 1), 4.68 -> 4.52 (M = 16), o_proj 3.78 -> 3.70
  // (M = 1), 4.07 -> 3.91 (M = 16); with the tiled weights the Qwen3-0.6B down (K =
  // 3072) 4.32 -> 3.92 (M = 32), 4.76 -> 4.56 (M = 64).  Six 4-step chunks a wave
  // (Qwen3-1.7B down, K = 6144) lose to 16 waves of 2-step chunks (6.20 -> 6.87 us
  // at M = 1).
  if (!wide && !chosen && pl.LW == 1 && K / (32 * 4 * 8) <= 3) {
    pl.W = 8;
    pl.CK = 4;
    pl.chunks = K / (32 * 4);
  }
  return pl;
}

}  // namespace t2i_host

namespace {

using namespace t2i;
using t2i_host::aligned16;
using t2i_host::fail;
using t2i_host::LinearPlan;
using t2i_host::plan_linear;

template <int MT, int LW, int W, int CK, bool NORM, bool XROWS, bool TILED, int PRE = 0, bool NXT = false>
hipError_t launch_t(const LinearParams& p, dim3 grid, hipStream_t s) {
  // the kernel takes x rows of K values (ldx = K) and K / (32 CK) chunks, as every plan here sets them
  if (p.ldx != p.K || p.chunks != p.K / (32 * CK)) return hipErrorInvalidValue;
  if (p.M >= (1 << 24) || p.rt < 1 || p.rt > 16 * MT || (p.rt & (p.rt - 1))) return hipErrorInvalidValue;
  const int m_rt = p.M | (__builtin_ctz((unsigned)p.rt) << 24);   // M and log2 of the row-tile height
  hipLaunchKernelGGL((w4a16_mfma_kernel<MT, LW, W, CK, NORM, XROWS, TILED, PRE, NXT>), grid, dim3(64 * W), 0, s, p.x, p.qw, p.sc,
                     p.qz, NORM ? p.gamma : p.residual, p.N, m_rt, p.K, (int)grid.x, p);
  return hipGetLastError();
}

// Whole-row activation loads, from row tiles of 4 rows up: measured over the
// HBM-cold sweep, 0.05-0.7 us less per launch with tiles of 8 or 16 rows (qkv and
// gate_up at M = 16: -0.22 us; down at M = 64: -0.7 us) and ~0.04 us less with
// tiles of 4 (o_proj and down at M = 16, a tile loading only the instructions that
// hold its rows); tiles of 1 or 2 rows gain nothing, within +-0.07 us.  Not compiled
// for 16 waves of 4-step chunks, whose registers are already at the limit.
// chain: 0 none, 1 the chained norm's consumer (PRE), 2 its producer (NXT); compiled
// for the decode plans of 8 waves of 4-step chunks at 16 (both) or 32 columns (PRE).
template <int MT, int LW, int W, int CK, bool TILED>
hipError_t launch_cfg(const LinearParams& p, dim3 grid, hipStream_t s, bool norm, int chain) {
  constexpr bool XOK = MT == 1 && (CK == 2 || (CK == 4 && W < 16));
  if (chain) {
    constexpr bool CH = MT == 1 && W == 8 && CK == 4 && XOK;
    if constexpr (CH && LW <= 2) {
      const bool xr = p.rt >= 4;
      if (chain == 1 && p.K == 1024)
        return xr ? launch_t<MT, LW, W, CK, false, true, TILED, 1, false>(p, grid, s)
                  : launch_t<MT, LW, W, CK, false, false, TILED, 1, false>(p, grid, s);
      if (chain == 1 && p.K == 2048)
        return xr ? launch_t<MT, LW, W, CK, false, true, TILED, 2, false>(p, grid, s)
                  : launch_t<MT, LW, W, CK, false, false, TILED, 2, false>(p, grid, s);
      if constexpr (LW == 1) {
        if (chain == 2)
          return xr ? launch_t<MT, LW, W, CK, false, true, TILED, 0, true>(p, grid, s)
                    : launch_t<MT, LW, W, CK, false, false, TILED, 0, true>(p, grid, s);
      }
    }
    return hipErrorInvalidValue;
  }
  int min_rt = 4;
#ifdef T2I_TUNING
  // tuning builds only: T2I_XROWS_MIN_RT = smallest row tile given whole-row loads (17: never)
  if (const char* env = getenv("T2I_XROWS_MIN_RT")) min_rt = atoi(env);
#endif
  if constexpr (MT > 1) {   // the fused norm and whole-row loads work on one 16-row tile
    (void)min_rt;
    return norm ? hipErrorInvalidValue : launch_t<MT, LW, W, CK, false, false, TILED>(p, grid, s);
  } else {
    if constexpr (XOK) {
      if (p.rt >= min_rt)
        return norm ? launch_t<MT, LW, W, CK, true, true, TILED>(p, grid, s)
                    : launch_t<MT, LW, W, CK, false, true, TILED>(p, grid, s);
    }
    return norm ? launch_t<MT, LW, W, CK, true, false, TILED>(p, grid, s)
                : launch_t<MT, LW, W, CK, false, false, TILED>(p, grid, s);
  }
}

hipError_t launch_plan(const LinearPlan& pl, const LinearParams& p, bool norm, bool tiled, hipStream_t s,
                       int chain = 0) {
  const dim3 grid(pl.cbs, 1, pl.mz);
#define T2I_LAUNCH(a, b, c, d)                                                                 \
  if (pl.MT == a && pl.LW == b && pl.W == c && pl.CK == d)                                     \
    return tiled ? launch_cfg<a, b, c, d, true>(p, grid, s, norm, chain)                       \
                 : launch_cfg<a, b, c, d, false>(p, grid, s, norm, chain);
  T2I_LINEAR_CONFIGS(T2I_LAUNCH)
#undef T2I_LAUNCH
  return hipErrorInvalidValue;
}

// The prompt GEMM over p's rows, with its own row sums or p.xs in p.xs_parts parts.
hipError_t launch_gemm(const LinearParams& p, const QkvPrepParams& pp, hipStream_t s) {
  const unsigned tiles = (unsigned)((p.M + GM_BM - 1) / GM_BM) * (unsigned)(p.N / GM_BN);
  if (!p.xs) hipLaunchKernelGGL(w4a16_gemm_kernel<0>, dim3(tiles), dim3(GM_THREADS), 0, s, p, pp);
  else if (p.xs_parts == 1) hipLaunchKernelGGL(w4a16_gemm_kernel<1>, dim3(tiles), dim3(GM_THREADS), 0, s, p, pp);
  else hipLaunchKernelGGL(w4a16_gemm_kernel<2>, dim3(tiles), dim3(GM_THREADS), 0, s, p, pp);
  return hipGetLastError();
}

// Rows from which the LDS-tiled GEMM replaces the 16-row-tile kernel.
int gemm_min_rows() {
#ifdef T2I_TUNING
  if (const char* env = getenv("T2I_GEMM_MIN_M")) return atoi(env);
#endif
  return 512;
}

int check_weights(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  int K, int N, int group_size) {
  if (!qweight || !qzeros || !scales) return fail(T2I_ERR_NULL, "qweight/qzeros/scales must not be NULL");
  if (group_size != GS) return fail(T2I_ERR_GROUP, "group_size %d unsupported (only 128)", group_size);
  if (K <= 0 || K % GS) return fail(T2I_ERR_SHAPE, "K=%d must be a positive multiple of 128", K);
  if (N <= 0 || N % 16) return fail(T2I_ERR_SHAPE, "N=%d must be a positive multiple of 16", N);
  if (!aligned16(qweight) || !aligned16(scales)) return fail(T2I_ERR_ALIGN, "qweight/scales must be 16-byte aligned");
  if (((uintptr_t)qzeros & 3u) != 0) return fail(T2I_ERR_ALIGN, "qzeros must be 4-byte aligned");
  return T2I_OK;
}

// gamma != NULL: the fused-norm variant (x is normalised with gamma, eps first).
// xs / xs_parts: x's precomputed row sums (may be NULL: the prompt GEMM forms its
// own; other kernels never need them); ys: the SwiGLU output's half-group sums
// (prompt GEMM only; may be NULL).
// Plans that read the AutoGPTQ words faster than the tiles, when a call has both:
// 64-column blocks of one m-tile, whose lanes' 64 tiled bytes per chunk leave each
// load instruction with 16-byte pieces 64 bytes apart (measured HBM-cold, us a
// launch, AutoGPTQ -> tiles: Qwen3-0.6B gate_up-shaped N = 6144 at M = 32 4.04 ->
// 4.16, qkv at M = 64 4.03 -> 4.10), and the fused-norm paired gate_up at
// 32-column blocks (4.00 -> 4.03 at M = 16).  Every other decode plan reads the
// tiles faster (down at M = 16 4.12 -> 3.68, o_proj 3.30 -> 3.19, qkv at M = 32
// 3.45 -> 3.21).
bool autogptq_reads_faster(const LinearPlan& pl, bool paired, bool norm) {
  return (pl.LW == 4 && pl.MT == 1) || (paired && norm && pl.LW == 2);
}

// tiles (may be NULL): qweight's words in the tile layout of t2i_w4a16_tile_qweight,
// read by the 16-row-tile kernel; qweight may then be NULL (no prompt-GEMM rows).
int run_linear(int epi, const uint16_t* x, int M, const uint16_t* gamma, float eps, const int32_t* qweight,
               const int32_t* qzeros, const uint16_t* scales, int K, int N, int group_size,
               const uint16_t* residual, uint16_t* y0, uint16_t* y1, void* stream, const float* xs = nullptr,
               int xs_parts = 1, float* ys = nullptr, const int32_t* tiles = nullptr, const float* ss_in = nullptr,
               const uint16_t* g_next = nullptr, uint16_t* xg = nullptr, float* ss_out = nullptr) {
  int rc = check_weights(qweight ? qweight : tiles, qzeros, scales, K, N, group_size);
  if (rc) return rc;
  if (qweight && tiles && !aligned16(tiles)) return fail(T2I_ERR_ALIGN, "tiles must be 16-byte aligned");
  if (xs_parts != 1 && xs_parts != 2) return fail(T2I_ERR_VALUE, "sum_parts must be 1 or 2");
  if (ys && epi != EPI_SWIGLU) return fail(T2I_ERR_VALUE, "y_sums is only written with swiglu");
  if ((xs && ((uintptr_t)xs & 3u)) || (ys && ((uintptr_t)ys & 3u)))
    return fail(T2I_ERR_ALIGN, "row sums must be 4-byte aligned");
  if (!x || !y0) return fail(T2I_ERR_NULL, "x and y must not be NULL");
  if (epi == EPI_PAIRED && !y1) return fail(T2I_ERR_NULL, "y1 must not be NULL when swiglu == 0");
  if (epi == EPI_RESIDUAL && !residual) return fail(T2I_ERR_NULL, "residual must not be NULL");
  if (M < 1 || M > T2I_MAX_ROWS) return fail(T2I_ERR_SHAPE, "M=%d must be in [1, %d]", M, T2I_MAX_ROWS);
  if (!aligned16(x) || !aligned16(y0) || (y1 && !aligned16(y1)) || (residual && !aligned16(residual)))
    return fail(T2I_ERR_ALIGN, "activation pointers must be 16-byte aligned");
  if (gamma) {
    if (!aligned16(gamma)) return fail(T2I_ERR_ALIGN, "norm_weight must be 16-byte aligned");
    if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  }
  const bool paired = epi == EPI_SWIGLU || epi == EPI_PAIRED;
  if (paired && N % 32) return fail(T2I_ERR_SHAPE, "paired N=%d must be a multiple of 32", N);
  const int chain = ss_in ? 1 : (g_next ? 2 : 0);
  if (chain) {
    if (gamma || xs || ys) return fail(T2I_ERR_VALUE, "the chained norm takes no norm_weight and no row sums");
    if (chain == 1 && (epi == EPI_RESIDUAL || g_next))
      return fail(T2I_ERR_VALUE, "the chained norm's consumer has no residual and no next norm");
    if (chain == 1 && K != 1024 && K != 2048) return fail(T2I_ERR_SHAPE, "K=%d: the chained norm's consumer takes K = 1024 or 2048", K);
    if (chain == 1 && !(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
    if (chain == 2 && (epi != EPI_RESIDUAL || !xg || !ss_out))
      return fail(T2I_ERR_VALUE, "the chained norm's producer needs the residual epilogue, xg and ss_out");
    if ((ss_in && !aligned16(ss_in)) || (g_next && !aligned16(g_next)) || (xg && !aligned16(xg)) ||
        (ss_out && ((uintptr_t)ss_out & 3u)))
      return fail(T2I_ERR_ALIGN, "chained-norm buffers: 16-byte aligned (ss_out 4-byte)");
    if (M >= gemm_min_rows()) return fail(T2I_ERR_SHAPE, "M=%d: the chained norm serves fewer than %d rows", M, gemm_min_rows());
  }
  if (!gamma && M >= gemm_min_rows() && N % GM_BN == 0) {
    // prompt-sized: the LDS-tiled GEMM, over the AutoGPTQ words
    if (!qweight)
      return fail(T2I_ERR_SHAPE, "M=%d: prompt rows (>= %d) read qweight, which is NULL", M, gemm_min_rows());
    LinearParams p{};
    p.x = x;
    p.qw = reinterpret_cast<const uint32_t*>(qweight);
    p.qz = reinterpret_cast<const uint32_t*>(qzeros);
    p.sc = scales;
    p.residual = residual;
    p.y0 = y0;
    p.y1 = y1;
    p.M = M; p.K = K; p.N = N;
    p.ldx = K;
    p.ldy = paired ? N / 2 : N;
    p.epi = epi;
    p.xs = xs;
    p.xs_parts = xs_parts;
    p.ldxs = M;
    p.ys = ys;
    p.ldys = M;
    return t2i_host::hip_status(launch_gemm(p, QkvPrepParams{}, reinterpret_cast<hipStream_t>(stream)),
                                "w4a16 gemm launch");
  }
  if (ys) return fail(T2I_ERR_SHAPE, "y_sums needs the prompt GEMM (M >= %d, N a multiple of %d)", gemm_min_rows(), GM_BN);
  const LinearPlan pl = plan_linear(M, K, N, paired, gamma != nullptr, false);
  if (chain && !(pl.MT == 1 && pl.W == 8 && pl.CK == 4 && pl.LW <= (chain == 2 ? 1 : 2)))
    return fail(T2I_ERR_SHAPE, "M=%d K=%d N=%d: no chained-norm form of this plan", M, K, N);
  const bool tiled = tiles && !(qweight && autogptq_reads_faster(pl, paired, gamma != nullptr));
  LinearParams p{};
  p.x = x;
  p.qw = reinterpret_cast<const uint32_t*>(tiled ? tiles : qweight);
  p.qz = reinterpret_cast<const uint32_t*>(qzeros);
  p.sc = scales;
  p.residual = residual;
  p.y0 = y0;
  p.y1 = y1;
  p.gamma = gamma;
  p.eps = eps;
  p.M = M; p.K = K; p.N = N;
  p.ldx = K;
  p.ldy = paired ? N / 2 : N;
  p.chunks = pl.chunks;
  p.epi = epi;
  p.rt = pl.rt;
  p.ss_in = ss_in;
  p.g_next = g_next;
  p.xg = xg;
  p.ss_out = ss_out;
  return t2i_host::hip_status(
      launch_plan(pl, p, gamma != nullptr, tiled, reinterpret_cast<hipStream_t>(stream), chain), "w4a16 linear launch");
}

}  // namespace

namespace {
int run_prefill_qkv(const uint16_t* x, const float* x_sums, int32_t B, int32_t T, int32_t p0, const int32_t* qweight,
                    const int32_t* qzeros, const uint16_t* scales, int32_t K, int32_t group_size, int32_t Hq,
                    int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                    const uint16_t* rope, int32_t rope_style, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                    int32_t ctx_cap, void* stream) {
  if (!x || !q_norm || !k_norm || !rope || !q_out || !k_cache || !v_cache)
    return fail(T2I_ERR_NULL, "prefill projection pointers must not be NULL");
  if (x_sums && ((uintptr_t)x_sums & 3u)) return fail(T2I_ERR_ALIGN, "x_sums must be 4-byte aligned");
  if (D != ATT_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (B < 1 || T < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv || Hq + 2 * Hkv > 0x3FFF)
    return fail(T2I_ERR_SHAPE, "B=%d T=%d Hq=%d Hkv=%d invalid", B, T, Hq, Hkv);
  const long long M = (long long)B * T;
  if (M < gemm_min_rows() || M > T2I_MAX_ROWS)
    return fail(T2I_ERR_SHAPE, "B*T=%lld must be in [%d, %d] (the prompt GEMM)", M, gemm_min_rows(), T2I_MAX_ROWS);
  if (p0 < 0 || ctx_cap < 1 || p0 + T > ctx_cap)
    return fail(T2I_ERR_SHAPE, "positions %d..%d exceed the cache (%d)", p0, p0 + T - 1, ctx_cap);
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  const int N = (Hq + 2 * Hkv) * ATT_D;
  int rc = check_weights(qweight, qzeros, scales, K, N, group_size);
  if (rc) return rc;
  if (!aligned16(x) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(rope) ||
      !aligned16(q_norm) || !aligned16(k_norm))
    return fail(T2I_ERR_ALIGN, "prefill projection tensors must be 16-byte aligned");
  LinearParams p{};
  p.x = x;
  p.qw = reinterpret_cast<const uint32_t*>(qweight);
  p.qz = reinterpret_cast<const uint32_t*>(qzeros);
  p.sc = scales;
  p.M = (int)M; p.K = K; p.N = N;
  p.ldx = K;
  p.ldy = N;
  p.epi = EPI_QKV_PREP;
  QkvPrepParams pp{};
  pp.qn = q_norm; pp.kn = k_norm; pp.rope = rope; pp.q = q_out; pp.kc = k_cache; pp.vc = v_cache;
  pp.T = T; pp.Hq = Hq; pp.Hkv = Hkv; pp.cap = ctx_cap; pp.p0 = p0; pp.style = rope_style; pp.eps = eps;
  static_assert(GM_BN == ATT_D, "one prompt-GEMM column tile is one head");
  p.xs = x_sums;
  p.xs_parts = 1;
  p.ldxs = p.M;
  return t2i_host::hip_status(launch_gemm(p, pp, reinterpret_cast<hipStream_t>(stream)), "prefill projection launch");
}
}  // namespace

extern "C" int t2i_prefill_qkv_rope_kv(const uint16_t* x, int32_t B, int32_t T, int32_t p0, const int32_t* qweight,
                                       const int32_t* qzeros, const uint16_t* scales, int32_t K, int32_t group_size,
                                       int32_t Hq, int32_t Hkv, int32_t D, const uint16_t* q_norm,
                                       const uint16_t* k_norm, float eps, const uint16_t* rope, int32_t rope_style,
                                       uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap,
                                       void* stream) {
  return run_prefill_qkv(x, nullptr, B, T, p0, qweight, qzeros, scales, K, group_size, Hq, Hkv, D, q_norm, k_norm,
                         eps, rope, rope_style, q_out, k_cache, v_cache, ctx_cap, stream);
}

extern "C" int t2i_prefill_qkv_rope_kv_sums(const uint16_t* x, const float* x_sums, int32_t B, int32_t T, int32_t p0,
                                            const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                            int32_t K, int32_t group_size, int32_t Hq, int32_t Hkv, int32_t D,
                                            const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                            const uint16_t* rope, int32_t rope_style, uint16_t* q_out,
                                            uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, void* stream) {
  if (!x_sums) return fail(T2I_ERR_NULL, "x_sums must not be NULL");
  return run_prefill_qkv(x, x_sums, B, T, p0, qweight, qzeros, scales, K, group_size, Hq, Hkv, D, q_norm, k_norm,
                         eps, rope, rope_style, q_out, k_cache, v_cache, ctx_cap, stream);
}

extern "C" int t2i_w4a16_linear(const uint16_t* x, int32_t M, const int32_t* qweight,
                                const int32_t* qzeros, const uint16_t* scales, int32_t K,
                                int32_t N, int32_t group_size, const uint16_t* residual,
                                uint16_t* y, void* stream) {
  return run_linear(residual ? EPI_RESIDUAL : EPI_STORE, x, M, nullptr, 0.0f, qweight, qzeros, scales, K, N,
                    group_size, residual, y, nullptr, stream);
}

extern "C" int t2i_w4a16_gate_up(const uint16_t* x, int32_t M, const int32_t* qweight,
                                 const int32_t* qzeros, const uint16_t* scales, int32_t K,
                                 int32_t N, int32_t group_size, int32_t swiglu, uint16_t* y0,
                                 uint16_t* y1, void* stream) {
  return run_linear(swiglu ? EPI_SWIGLU : EPI_PAIRED, x, M, nullptr, 0.0f, qweight, qzeros, scales, K, N,
                    group_size, nullptr, y0, y1, stream);
}

extern "C" int t2i_w4a16_linear_sums(const uint16_t* x, const float* x_sums, int32_t sum_parts, int32_t M,
                                     const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                     int32_t K, int32_t N, int32_t group_size, const uint16_t* residual, uint16_t* y,
                                     void* stream) {
  if (!x_sums) return fail(T2I_ERR_NULL, "x_sums must not be NULL");
  return run_linear(residual ? EPI_RESIDUAL : EPI_STORE, x, M, nullptr, 0.0f, qweight, qzeros, scales, K, N,
                    group_size, residual, y, nullptr, stream, x_sums, sum_parts);
}

extern "C" int t2i_w4a16_gate_up_sums(const uint16_t* x, const float* x_sums, int32_t sum_parts, int32_t M,
                                      const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                      int32_t K, int32_t N, int32_t group_size, int32_t swiglu, uint16_t* y0,
                                      uint16_t* y1, float* y_sums, void* stream) {
  return run_linear(swiglu ? EPI_SWIGLU : EPI_PAIRED, x, M, nullptr, 0.0f, qweight, qzeros, scales, K, N,
                    group_size, nullptr, y0, y1, stream, x_sums, sum_parts, y_sums);
}

extern "C" int t2i_w4a16_rmsnorm_linear(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                                        const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                        int32_t K, int32_t N, int32_t group_size, uint16_t* y, void* stream) {
  if (!norm_weight) return fail(T2I_ERR_NULL, "norm_weight must not be NULL");
  return run_linear(EPI_STORE, x, M, norm_weight, eps, qweight, qzeros, scales, K, N, group_size, nullptr, y,
                    nullptr, stream);
}

extern "C" int t2i_w4a16_rmsnorm_gate_up(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                                         const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                                         int32_t K, int32_t N, int32_t group_size, int32_t swiglu, uint16_t* y0,
                                         uint16_t* y1, void* stream) {
  if (!norm_weight) return fail(T2I_ERR_NULL, "norm_weight must not be NULL");
  return run_linear(swiglu ? EPI_SWIGLU : EPI_PAIRED, x, M, norm_weight, eps, qweight, qzeros, scales, K, N,
                    group_size, nullptr, y0, y1, stream);
}

extern "C" int t2i_w4a16_tile_qweight(const int32_t* qweight, int32_t K, int32_t N, int32_t* tiles, void* stream) {
  if (!qweight || !tiles) return fail(T2I_ERR_NULL, "qweight and tiles must not be NULL");
  if (K <= 0 || K % GS) return fail(T2I_ERR_SHAPE, "K=%d must be a positive multiple of 128", K);
  if (N <= 0 || N % 16) return fail(T2I_ERR_SHAPE, "N=%d must be a positive multiple of 16", N);
  if (!aligned16(qweight) || !aligned16(tiles)) return fail(T2I_ERR_ALIGN, "qweight and tiles must be 16-byte aligned");
  const size_t total = (size_t)(K / 8) * N;
  const uintptr_t a = (uintptr_t)qweight, b = (uintptr_t)tiles, bytes = total * 4;
  if (a < b + bytes && b < a + bytes) return fail(T2I_ERR_VALUE, "tiles must not overlap qweight");
  const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(t2i::tile_qweight_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(qweight), K, N, reinterpret_cast<uint32_t*>(tiles));
  return t2i_host::hip_status(hipGetLastError(), "tile_qweight launch");
}

extern "C" int t2i_w4a16_linear_tiles(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                                      const int32_t* qweight, const int32_t* tiles, const int32_t* qzeros,
                                      const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                                      int32_t epilogue, const uint16_t* residual, uint16_t* y0, uint16_t* y1,
                                      void* stream) {
  if (!tiles) return fail(T2I_ERR_NULL, "tiles must not be NULL");
  int epi;
  switch (epilogue) {
    case T2I_TILES_STORE: epi = residual ? EPI_RESIDUAL : EPI_STORE; break;
    case T2I_TILES_SWIGLU: epi = EPI_SWIGLU; break;
    case T2I_TILES_PAIRED: epi = EPI_PAIRED; break;
    default: return fail(T2I_ERR_VALUE, "epilogue %d unknown", epilogue);
  }
  if (epilogue != T2I_TILES_STORE && residual) return fail(T2I_ERR_VALUE, "a residual goes with the plain store only");
  if (norm_weight && residual) return fail(T2I_ERR_VALUE, "the fused-norm form takes no residual");
  return run_linear(epi, x, M, norm_weight, eps, qweight, qzeros, scales, K, N, group_size, residual, y0, y1, stream,
                    nullptr, 1, nullptr, tiles);
}

extern "C" int t2i_w4a16_linear_tiles_chain(const uint16_t* x, int32_t M, const float* x_sumsq, float eps,
                                            const int32_t* qweight, const int32_t* tiles, const int32_t* qzeros,
                                            const uint16_t* scales, int32_t K, int32_t N, int32_t group_size,
                                            int32_t epilogue, const uint16_t* residual, uint16_t* y0, uint16_t* y1,
                                            const uint16_t* next_norm_weight, uint16_t* xg_out, float* sumsq_out,
                                            void* stream) {
  if (!tiles) return fail(T2I_ERR_NULL, "tiles must not be NULL");
  if (!x_sumsq && !next_norm_weight) return fail(T2I_ERR_NULL, "x_sumsq or next_norm_weight must be given");
  int epi;
  switch (epilogue) {
    case T2I_TILES_STORE: epi = residual ? EPI_RESIDUAL : EPI_STORE; break;
    case T2I_TILES_SWIGLU: epi = EPI_SWIGLU; break;
    case T2I_TILES_PAIRED: epi = EPI_PAIRED; break;
    default: return fail(T2I_ERR_VALUE, "epilogue %d unknown", epilogue);
  }
  if (epilogue != T2I_TILES_STORE && residual) return fail(T2I_ERR_VALUE, "a residual goes with the plain store only");
  return run_linear(epi, x, M, nullptr, eps, qweight, qzeros, scales, K, N, group_size, residual, y0, y1, stream,
                    nullptr, 1, nullptr, tiles, x_sumsq, next_norm_weight, xg_out, sumsq_out);
}

extern "C" int t2i_w4a16_chain_supported(int32_t M, int32_t K, int32_t N, int32_t role) {
  if (M < 1 || M >= gemm_min_rows() || K <= 0 || K % GS || N <= 0 || N % 16) return 0;
  const bool paired = role == 2;
  if (role < 0 || role > 2 || (paired && N % 32)) return 0;
  if (role >= 1 && K != 1024 && K != 2048) return 0;
  const LinearPlan pl = plan_linear(M, K, N, paired, false, false);
  return pl.MT == 1 && pl.W == 8 && pl.CK == 4 && pl.LW <= (role == 0 ? 1 : 2);
}

extern "C" int t2i_w4a16_dequant_f32(const int32_t* qweight, const int32_t* qzeros,
                                     const uint16_t* scales, int32_t K, int32_t N,
                                     int32_t group_size, float* W_nk, void* stream) {
  int rc = check_weights(qweight, qzeros, scales, K, N, group_size);
  if (rc) return rc;
  if (!W_nk) return fail(T2I_ERR_NULL, "W_nk must not be NULL");
  if (!aligned16(W_nk)) return fail(T2I_ERR_ALIGN, "W_nk must be 16-byte aligned");
  const int rows = K / 8;
  dim3 grid(N, (rows + 255) / 256);
  hipLaunchKernelGGL(t2i::dequant_f32_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint32_t*>(qweight), reinterpret_cast<const uint32_t*>(qzeros),
                     scales, K, N, W_nk);
  return t2i_host::hip_status(hipGetLastError(), "dequant launch");
}
