// Device-side building blocks of the W4A16 decode linear (gfx950), shared by
// the standalone linear kernel and the fused kernels that run a linear phase.
#pragma once

#include "t2i_common.h"

namespace t2i {

constexpr int GS = 128;             // quantisation group along K
constexpr int KSG = GS / 32;        // MFMA k-steps per group
constexpr uint32_t MAGIC = 0x43004300u;  // two bf16 128.0
constexpr uint32_t NIB2 = 0x000F000Fu;

// EPI_LL: each output value goes out as one 64-bit word, the bf16 bits in the
// low half and the launch's tag in the high half, stored agent-coherently
// (written through to the device-coherent level), so a consumer in the same
// launch on any XCD can poll the word itself until the tag shows it is this
// launch's value (one word per lane and column: one-word-per-lane tiles only).
// EPI_QKV_PREP (the prompt GEMM only): the tile is one q, k or v head of the
// fused projection; it gets the q/k RMSNorm + RoPE of qk_prep.h and goes to the
// q rows and the KV cache (QkvPrepParams) instead of y0.
enum : int { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_PAIRED = 3, EPI_LL = 4, EPI_QKV_PREP = 5 };

// Destinations and norm/RoPE inputs of EPI_QKV_PREP (row m = b * T + t, position
// p0 + t): q heads to q [B, Hq, T, 128], k and v heads to the caches
// [B, Hkv, cap, 128] at that position.
struct QkvPrepParams {
  const uint16_t* qn;     // [128] q norm weight
  const uint16_t* kn;     // [128] k norm weight
  const uint16_t* rope;   // [>= p0 + T, 128] cos even / sin odd
  uint16_t* q;
  uint16_t* kc;
  uint16_t* vc;
  int T, Hq, Hkv, cap, p0, style;
  float eps;
};

struct LinearParams {
  const uint16_t* x;
  const uint32_t* qw;
  const uint32_t* qz;
  const uint16_t* sc;
  const uint16_t* residual;
  uint16_t* y0;
  uint16_t* y1;
  const uint16_t* gamma;   // RMSNorm weight [K] of the fused-norm variant
  float eps;
  int M, K, N;
  int ldx, ldy;
  int chunks;           // K / (32 * CK)
  int epi;
  int rt;               // rows per row tile: 16, or fewer to give a narrow output more workgroups
  unsigned long long* ll;   // EPI_LL: [M][ldy] tagged words
  uint32_t tag;             // EPI_LL: this launch's tag; yll: its low 16 bits
  // Phases of one launch (linear_phase) hand rows over as tagged 32-bit words,
  // bf16 bits | tag << 16: input (xll, in place of x), residual (rll, in place of
  // residual) and output (yll, in place of y0), each used when not NULL; the
  // input and residual words are awaited until they carry xtag / rtag.
  const uint32_t* xll;
  const uint32_t* rll;
  uint32_t* yll;
  uint32_t xtag, rtag;
  unsigned* ctl;            // ctl[2]: the launch's error word (bounded waits)
  // Prompt GEMM only.  xs: fp32 sums of each row of x over each 128-wide k group,
  // group-major: the sums of group g for rows 0 .. M - 1 at xs + g * ldxs
  // (xs_parts = 1), or over each 64-wide half group, halves 2 g and 2 g + 1
  // (xs_parts = 2), taken in place of the kernel's own row-sum products.  ys
  // (EPI_SWIGLU, may be NULL): the sums of each output row's bf16 values over each
  // 64-wide column half group, half h of row m at ys[h * ldys + m].
  const float* xs;
  float* ys;
  int ldxs, xs_parts, ldys;
  // Chained RMSNorm between decode linears.  ss_in (consumer, PRE): x holds
  // bf16(x_raw * gamma) and ss_in [M][K/16] the sums of x_raw^2 over each 16-wide
  // block of k; the product's fp32 sums are scaled by the row's 1 / rms.  g_next,
  // xg, ss_out (producer, NXT, residual epilogue): besides y, the next norm's
  // input bf16(y * g_next) [M][ldy] and the sums of y^2 over each 16-column block
  // [M][N/16].
  const float* ss_in;
  const uint16_t* g_next;
  uint16_t* xg;
  float* ss_out;
};

// MAGIC in a VGPR.  A VALU instruction reads at most one scalar operand (SGPR or
// literal) on gfx9, so with the nibble mask as that operand the AND-OR takes
// MAGIC from a VGPR and stays one v_and_or_b32; with both as constants the
// compiler splits it into an AND and an OR.
__device__ __forceinline__ uint32_t magic_vgpr() {
  uint32_t m = MAGIC;
  asm volatile("" : "+v"(m));
  return m;
}

// magic: MAGIC, held in a VGPR (magic_vgpr).
__device__ __forceinline__ bf16x8 b_operand(uint32_t w, uint32_t magic) {
  u32x4 d;
  d.x = (w & NIB2) | magic;           // (k0, k4)
  d.y = ((w >> 4) & NIB2) | magic;    // (k1, k5)
  d.z = ((w >> 8) & NIB2) | magic;    // (k2, k6)
  d.w = ((w >> 12) & NIB2) | magic;   // (k3, k7)
  return __builtin_bit_cast(bf16x8, d);
}

// The same eight values in k order, to meet an activation fragment as it lies in
// memory: word j is (k 2j, k 2j + 1), byte j of w (nibbles 2j, 2j + 1) put in
// the low half and byte j of w >> 4 (nibble 2j + 1 at its bottom) in the high
// half by one byte permute, then the AND-OR.  One shift and two instructions a
// pair: nine a word against b_operand's seven, and the activations need no
// reordering.
__device__ __forceinline__ bf16x8 b_operand_kord(uint32_t w, uint32_t magic) {
  const uint32_t w4 = w >> 4;
  u32x4 d;
  // selector bytes 0-3 take bytes of w, 4-7 bytes of w4, 0x0C gives a zero byte
  d.x = (__builtin_amdgcn_perm(w4, w, 0x0C040C00u) & NIB2) | magic;   // (k0, k1)
  d.y = (__builtin_amdgcn_perm(w4, w, 0x0C050C01u) & NIB2) | magic;   // (k2, k3)
  d.z = (__builtin_amdgcn_perm(w4, w, 0x0C060C02u) & NIB2) | magic;   // (k4, k5)
  d.w = (__builtin_amdgcn_perm(w4, w, 0x0C070C03u) & NIB2) | magic;   // (k6, k7)
  return __builtin_bit_cast(bf16x8, d);
}

// v holds bf16 pairs (k0,k1) (k2,k3) (k4,k5) (k6,k7); reorder to match b_operand,
// one byte permute (v_perm_b32) per output word.
__device__ __forceinline__ bf16x8 a_operand(u32x4 v) {
  u32x4 d;
  d.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);   // (lo x, lo z)
  d.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);   // (hi x, hi z)
  d.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  d.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return __builtin_bit_cast(bf16x8, d);
}

__device__ __forceinline__ bf16x8 ones_operand() {
  u32x4 d = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  return __builtin_bit_cast(bf16x8, d);
}

// g * sigmoid(g) on v_exp_f32 and v_rcp_f32: a few ulp of fp32 from silu_f32 (the
// result is rounded to bf16 right after).  For the prompt GEMM's epilogue, where
// the libm exponential and the IEEE division cost more than its k-loop's last steps.
__device__ __forceinline__ float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

template <int LW>
__device__ __forceinline__ void load_words(const uint32_t* src, uint32_t (&w)[LW]) {
  if constexpr (LW == 8) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(src);
    const u32x4 b = *reinterpret_cast<const u32x4*>(src + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (LW == 4) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(src);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (LW == 2) {
    const u32x2 a = *reinterpret_cast<const u32x2*>(src);
    w[0] = a.x; w[1] = a.y;
  } else {
    w[0] = *src;
  }
}

// Raw fp16 scales of LW consecutive columns, two per word (converted only when
// the chunk is computed, so issuing a chunk's loads never waits for them).
// LW 16-bit values from src (fp16 scales or bf16 residuals) as 32-bit words.  One
// value (odd: at an odd index) comes as the aligned word holding it (half_of picks
// it): a 16-bit load would be widened right after the load, which makes the
// compiler wait for it there.
template <int LW>
__device__ __forceinline__ void load_scales(const uint16_t* src, uint32_t (&s)[(LW + 1) / 2], int odd = 0) {
  if constexpr (LW == 8) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(src);
    s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w;
  } else if constexpr (LW == 4) {
    const u32x2 a = *reinterpret_cast<const u32x2*>(src);
    s[0] = a.x; s[1] = a.y;
  } else if constexpr (LW == 2) {
    s[0] = *reinterpret_cast<const uint32_t*>(src);
  } else {
    s[0] = *reinterpret_cast<const uint32_t*>(src - odd);
  }
}

// Bits of value t of this lane's columns; odd: the lane's first column is odd (LW == 1).
template <int LW>
__device__ __forceinline__ uint32_t half_of(const uint32_t (&s)[(LW + 1) / 2], int t, bool odd) {
  const bool hi = LW == 1 ? odd : (t & 1) != 0;
  return hi ? (s[t >> 1] >> 16) : (s[t >> 1] & 0xFFFFu);
}

// Operands of one chunk (CK k-steps, all inside one quantisation group), as loaded.
template <int MT, int LW, int CK>
struct Chunk {
  uint32_t w[CK][LW];
  u32x4 x[MT][CK];
  u32x4 g[CK];                // fused-norm variant: norm weight of k 8 r .. 8 r + 7 of each k-step
  u32x4 gp;                   // fused-norm variant (load_chunk): 8-value piece lane % (4 CK) of the
                              // chunk's norm weight, spread to g through LDS (norm_pieces)
  uint32_t s[(LW + 1) / 2];   // fp16 scales of this lane's LW columns
  uint32_t zw;                // qzeros word holding this lane's columns
};

// Activation row held by A-operand row `local` of the row tile at mbase.  A tile
// of p.rt rows repeats its last row in the MFMA rows past p.rt, and rows past M
// repeat row M - 1: the loads stay unconditional, an MFMA output row depends on
// its own A row only, and the repeats are never stored.
__device__ __forceinline__ int tile_row(const LinearParams& p, int mbase, int local) {
  return min(mbase + min(local, p.rt - 1), p.M - 1);
}

// Activation rows read whole (XROWS, one 16-row tile): load instruction i of a
// chunk covers tile rows (16 / CK) i .. (16 / CK) (i + 1) - 1, lane l row
// (16 / CK) i + l / (4 CK) and k-block l % (4 CK) (8 bf16 values) of the chunk, so
// an instruction reads 16 / CK pieces of CK * 64 contiguous bytes instead of 16
// pieces of 64 bytes.  Every workgroup reads the tile's activation rows through
// its XCD's L2, and the fewer, longer pieces cost fewer L2 requests (a read-only
// probe of the qkv loads at M = 16: 0.4 us less per launch).  x_fragments then
// moves the values into the MFMA layout through LDS.
template <int CK>
__device__ __forceinline__ int xrow_of(int lane, int i) { return (16 / CK) * i + lane / (4 * CK); }

// 16-byte LDS unit of (tile row, k-block) in a wave's chunk region: k-block
// major, the row XOR-swizzled with the k-block so that the stores of one load
// instruction and the reads of one k-step each meet 16 distinct bank groups per
// 16 lanes.
template <int CK>
__device__ __forceinline__ int xunit(int row, int kb) { return 16 * kb + (row ^ ((kb * 4 / CK) & 15)); }

// A chunk's loads go out in the order their values are used: the activations
// (moved through LDS first), the norm weight, the packed weights (the MFMAs),
// then the scales and zeros (the step after the MFMAs, which waits for them
// only then).  Loads retire in issue order, so each wait also covers every load
// issued before it.  Measured over the decode sweep against weights first:
// activations first 0.584 -> 0.600 TB/s, the scales and zeros awaited after the
// MFMAs 0.600 -> 0.609.
template <int MT, int LW, int CK, bool NORM, bool XROWS = false, bool TILED = false>
__device__ __forceinline__ void load_chunk(const LinearParams& p, int ch, int ncol, int c, int r, int mbase,
                                           Chunk<MT, LW, CK>& b) {
  const int ks0 = ch * CK;
  if constexpr (XROWS) {
    static_assert(MT == 1 && (CK == 2 || CK == 4), "whole-row loads of one 16-row tile");
    const int lane = 16 * r + c;
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      // only the loads that hold real rows of the tile (workgroup-uniform)
      if (i == 0 || xrow_of<CK>(0, i) < p.rt) {
        const int m = tile_row(p, mbase, xrow_of<CK>(lane, i));
        b.x[0][i] = *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.ldx + ks0 * 32 + 8 * (lane % (4 * CK)));
      }
    }
  } else {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      const int m = tile_row(p, mbase, mi * 16 + c);
#pragma unroll
      for (int j = 0; j < CK; ++j)
        b.x[mi][j] = *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.ldx + (ks0 + j) * 32 + r * 8);
    }
  }
  if constexpr (NORM)   // one load a lane: piece lane % (4 CK) of the chunk's norm weight (norm_pieces)
    b.gp = *reinterpret_cast<const u32x4*>(p.gamma + ks0 * 32 + 8 * ((16 * r + c) % (4 * CK)));
  if constexpr (TILED) {
    // qweight as 16-column tiles (t2i_w4a16_tile_qweight): the lane's LW columns
    // lie in one tile, their words for this chunk's k-steps contiguous
    static_assert(CK == 2 || CK == 4, "chunks of 2 or 4 k-steps: within one group");
    const uint32_t* src = p.qw + (size_t)((ncol >> 4) * (p.K / GS) + ks0 / KSG) * 256 + (r * 16 + (ncol & 15)) * 4 +
                          ks0 % KSG;
#pragma unroll
    for (int t = 0; t < LW; ++t) {
      if constexpr (CK == 4) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(src + 4 * t);
        b.w[0][t] = a.x; b.w[1][t] = a.y; b.w[2][t] = a.z; b.w[3][t] = a.w;
      } else {
        const u32x2 a = *reinterpret_cast<const u32x2*>(src + 4 * t);
        b.w[0][t] = a.x; b.w[1][t] = a.y;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < CK; ++j)
      load_words<LW>(p.qw + (size_t)((ks0 + j) * 4 + r) * p.N + ncol, b.w[j]);
  }
  const int g = ks0 / KSG;
  load_scales<LW>(p.sc + (size_t)g * p.N + ncol, b.s, ncol & 1);
  b.zw = p.qz[(size_t)g * (p.N >> 3) + (ncol >> 3)];
}

// The weight half of load_chunk (packed words, norm weight, scales, zeros):
// nothing here depends on the activations.
template <int MT, int LW, int CK, bool NORM>
__device__ __forceinline__ void load_chunk_w(const LinearParams& p, int ch, int ncol, int r, Chunk<MT, LW, CK>& b) {
  const int ks0 = ch * CK;
#pragma unroll
  for (int j = 0; j < CK; ++j)
    load_words<LW>(p.qw + (size_t)((ks0 + j) * 4 + r) * p.N + ncol, b.w[j]);
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < CK; ++j) b.g[j] = *reinterpret_cast<const u32x4*>(p.gamma + (ks0 + j) * 32 + r * 8);
  }
  const int g = ks0 / KSG;
  load_scales<LW>(p.sc + (size_t)g * p.N + ncol, b.s, ncol & 1);
  b.zw = p.qz[(size_t)g * (p.N >> 3) + (ncol >> 3)];
}

// 8 consecutive bf16 values held as tagged 32-bit words (word i = bf16 bits |
// tag << 16), read as four agent-coherent 64-bit loads.
struct Tagged8 {
  unsigned long long w[4];
};
__device__ __forceinline__ void tagged_issue(const uint32_t* src, Tagged8& t) {
#pragma unroll
  for (int q = 0; q < 4; ++q) t.w[q] = ld_coh64(src + 2 * q);
}
__device__ __forceinline__ bool tagged_ready(const Tagged8& t, uint32_t tag) {
  bool ok = true;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    ok = ok && (uint32_t)((t.w[q] >> 16) & 0xFFFFu) == tag && (uint32_t)(t.w[q] >> 48) == tag;
  return ok;
}
// Wait (bounded) until all 8 words carry tag, then the values as 4 bf16 pairs.
__device__ __forceinline__ u32x4 tagged_wait8(const uint32_t* src, Tagged8 t, uint32_t tag, unsigned* ctl) {
  int spins = 0;
  while (!tagged_ready(t, tag)) {
    if (wait_gives_up(spins, ctl)) break;
    tagged_issue(src, t);
  }
  uint32_t v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = (uint32_t)(t.w[q] & 0xFFFFu) | (uint32_t)((t.w[q] >> 16) & 0xFFFF0000u);
  return u32x4{v[0], v[1], v[2], v[3]};
}
// One tagged word, awaited (bounded); its bf16 bits in both halves of the result.
__device__ __forceinline__ uint32_t tagged_wait1(const uint32_t* src, uint32_t tag, unsigned* ctl) {
  uint32_t w = ld_coh32(src);
  int spins = 0;
  while ((w >> 16) != tag) {
    if (wait_gives_up(spins, ctl)) break;
    w = ld_coh32(src);
  }
  return (w & 0xFFFFu) | (w << 16);
}

// The activation half, agent-coherent (the rows were written in the same launch).
template <int MT, int LW, int CK>
__device__ __forceinline__ void load_chunk_x_coh(const LinearParams& p, int ch, int c, int r, int mbase,
                                                 Chunk<MT, LW, CK>& b) {
  const int ks0 = ch * CK;
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int m = tile_row(p, mbase, mi * 16 + c);
#pragma unroll
    for (int j = 0; j < CK; ++j) b.x[mi][j] = ld_coh128(p.x + (size_t)m * p.ldx + (ks0 + j) * 32 + r * 8);
  }
}

// Pins a loaded value at this point: code that uses it cannot be moved above the
// pin (say, to a point shared by the chunk schedules, where it would wait for the
// chunk's loads before the other chunks' loads are issued).
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(u32x4& v) { asm volatile("" : "+v"(v)); }

// The activation rows of a chunk loaded whole (load_chunk with XROWS) into the MFMA
// layout (lane (c, r), k-step j: tile row c, k 32 j + 8 r .. + 7 of the chunk),
// through this wave's CK * 1 KB region of LDS.  One wave writes and reads its own
// region, so no barrier is needed.
// A tile of rt < 16 rows loads only the instructions that hold its real rows, and
// every MFMA row past rt reads the tile's last row.
template <int LW, int CK>
__device__ __forceinline__ void x_fragments(Chunk<1, LW, CK>& b, u32x4* region, int lane, int rt) {
#pragma unroll
  for (int i = 0; i < CK; ++i) {
    if (i == 0 || xrow_of<CK>(0, i) < rt) {
      pin(b.x[0][i]);
      region[xunit<CK>(xrow_of<CK>(lane, i), lane % (4 * CK))] = b.x[0][i];
    }
  }
  const int c = lane & 15, r = lane >> 4;
  const int row = min(c, rt - 1);
#pragma unroll
  for (int j = 0; j < CK; ++j) b.x[0][j] = region[xunit<CK>(row, 4 * j + r)];
}

// NORM (fused-norm variant, MT = 1): the A operand is bf16(x * gamma), and the
// lane's share of its row's sum of squares accumulates in ss; the row's 1 / rms
// multiplies the finished sums (see the kernel).
template <int MT, int LW, int CK, bool NORM>
__device__ __forceinline__ void compute_chunk(Chunk<MT, LW, CK>& b, float (&total)[MT][LW][4], float& ss,
                                              int zshift) {
#pragma unroll
  for (int j = 0; j < CK; ++j) {
#pragma unroll
    for (int t = 0; t < LW; ++t) pin(b.w[j][t]);
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) pin(b.x[mi][j]);
    if constexpr (NORM) pin(b.g[j]);
  }
  const bf16x8 ones = ones_operand();
  const uint32_t magic = magic_vgpr();
  f32x4 acc[MT][LW];
  f32x4 xs[MT];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    xs[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < LW; ++t) acc[mi][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int j = 0; j < CK; ++j) {
    bf16x8 bop[LW];
#pragma unroll
    for (int t = 0; t < LW; ++t) bop[t] = b_operand(b.w[j][t], magic);
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      u32x4 xv = b.x[mi][j];
      if constexpr (NORM) {
        const uint32_t xa[4] = {xv.x, xv.y, xv.z, xv.w};
        const uint32_t ga[4] = {b.g[j].x, b.g[j].y, b.g[j].z, b.g[j].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16_lo(xa[e]), hi = bf16_hi(xa[e]);
          ss = fmaf(lo, lo, ss);
          ss = fmaf(hi, hi, ss);
          o[e] = pack_bf16x2(lo * bf16_lo(ga[e]), hi * bf16_hi(ga[e]));
        }
        xv = u32x4{o[0], o[1], o[2], o[3]};
      }
      const bf16x8 a = a_operand(xv);
      xs[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, xs[mi], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < LW; ++t)
        acc[mi][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bop[t], acc[mi][t], 0, 0, 0);
    }
  }
  // the scales and zeros, loaded after the weights, are waited for only now
#pragma unroll
  for (int i = 0; i < (LW + 1) / 2; ++i) pin(b.s[i]);
  pin(b.zw);
  const uint32_t zw = b.zw >> zshift;   // zero nibble of column ncol + t at bits 4t
#pragma unroll
  for (int t = 0; t < LW; ++t) {
    const float zb = -(float)(128 + 1 + ((zw >> (4 * t)) & 0xFu));
    const float sc = f16_to_f32(half_of<LW>(b.s, t, (zshift & 4) != 0));
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        total[mi][t][i] = fmaf(sc, fmaf(zb, xs[mi][i], acc[mi][t][i]), total[mi][t][i]);
  }
}

// NC chunks of a wave in a straight line: every chunk's loads are in flight
// before the first is computed (the first, A, was issued by the caller), and
// each computation waits for its own chunk only: one memory round trip for the
// whole K slice of the wave.  Up to 6 chunks of 2 k-steps without the fused
// norm (12 registers a chunk at one word per lane), 3 otherwise.
// A chunk from load_chunk, computed: its activation rows first into the MFMA
// layout when they were loaded whole (XROWS; xreg is the wave's LDS region).
// The chunk's norm weight in the operand layout (lane (c, r), k-step j: piece
// 4 j + r) from the one piece each lane loaded, through the wave's 4 CK units of
// LDS (greg): one load a lane instead of CK (RMSNorm + gate_up + SwiGLU at batch
// 16: 4.09 -> 4.00 us, same bits).  One wave writes and reads its own region, in order.
template <int LW, int CK>
__device__ __forceinline__ void norm_pieces(Chunk<1, LW, CK>& b, u32x4* greg, int lane) {
  pin(b.gp);
  if (lane < 4 * CK) greg[lane] = b.gp;
#pragma unroll
  for (int j = 0; j < CK; ++j) b.g[j] = greg[4 * j + (lane >> 4)];
}

template <int MT, int LW, int CK, bool NORM, bool XROWS>
__device__ __forceinline__ void compute_loaded(Chunk<MT, LW, CK>& b, float (&total)[MT][LW][4], float& ss,
                                               int zshift, u32x4* xreg, int lane, int rt, u32x4* greg) {
  if constexpr (XROWS) x_fragments<LW, CK>(b, xreg, lane, rt);
  if constexpr (NORM) norm_pieces<LW, CK>(b, greg, lane);
  compute_chunk<MT, LW, CK, NORM>(b, total, ss, zshift);
}

// issue() runs once every chunk's loads are issued (the epilogue's own loads,
// which then retire after the chunks').
template <int MT, int LW, int CK, bool NORM, bool XROWS, bool TILED, int NC, class Issue>
__device__ __forceinline__ void straight_chunks(const LinearParams& p, int c_begin, int ncol, int c, int r, int mbase,
                                                Chunk<MT, LW, CK>& A, float (&total)[MT][LW][4], float& ss,
                                                int zshift, u32x4* xreg, u32x4* greg, const Issue& issue) {
  const int lane = 16 * r + c;
  if constexpr (NC == 1) {
    issue();
    compute_loaded<MT, LW, CK, NORM, XROWS>(A, total, ss, zshift, xreg, lane, p.rt, greg);
  } else {
    Chunk<MT, LW, CK> rest[NC - 1];
#pragma unroll
    for (int i = 1; i < NC; ++i)
      load_chunk<MT, LW, CK, NORM, XROWS, TILED>(p, c_begin + i, ncol, c, r, mbase, rest[i - 1]);
    issue();
    compute_loaded<MT, LW, CK, NORM, XROWS>(A, total, ss, zshift, xreg, lane, p.rt, greg);
#pragma unroll
    for (int i = 1; i < NC; ++i)
      compute_loaded<MT, LW, CK, NORM, XROWS>(rest[i - 1], total, ss, zshift, xreg, lane, p.rt, greg);
  }
}

// One output value of a phase: a tagged word when the phase hands its rows over
// (yll), else an agent-coherent bf16 store.
__device__ __forceinline__ void emit_coh(const LinearParams& p, size_t idx, uint16_t v) {
  if (p.yll) st_coh32(p.yll + idx, (uint32_t)v | (p.tag << 16));
  else st_coh16(p.y0 + idx, v);
}

// Output row m of this lane's LW columns (ncol .. ncol + LW - 1) from the fp32
// sums v; res holds the row's residual values (bf16 pairs), fetched at the start.
// COH: agent-coherent stores (one 16-bit store a value; one or two words a lane).
// NXT (one column a lane, residual epilogue): also the next norm's input and the
// row's sum of squares over the 16 columns of the lane's 16-lane row (gword: the
// aligned word of g_next holding this column's weight).
template <int LW, bool COH = false, bool NXT = false>
__device__ __forceinline__ void store_row(const LinearParams& p, int ncol, int m, const float (&v_in)[LW],
                                          const uint32_t (&res)[(LW + 1) / 2], uint32_t gword = 0) {
  static_assert(!COH || LW <= 2, "coherent stores: one or two words a lane");
  static_assert(!NXT || (LW == 1 && !COH), "the chained norm's producer: one column a lane");
  if (m >= p.M) return;   // uniform over the 16 lanes of a row
  if constexpr (LW == 1) {
    if (p.epi == EPI_LL) {
      const unsigned long long w = (unsigned long long)f32_to_bf16(v_in[0]) | ((unsigned long long)p.tag << 32);
      __hip_atomic_store(p.ll + (size_t)m * p.ldy + ncol, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
  if (p.epi == EPI_STORE || p.epi == EPI_RESIDUAL) {
    float v[LW];
#pragma unroll
    for (int t = 0; t < LW; ++t) v[t] = v_in[t];
    if (p.epi == EPI_RESIDUAL) {
#pragma unroll
      for (int t = 0; t < LW; ++t) v[t] = round_bf16(v[t]) + bf16_to_f32((uint16_t)half_of<LW>(res, t, ncol & 1));
    }
    uint16_t* dst = p.y0 + (size_t)m * p.ldy + ncol;
    if constexpr (COH) {
#pragma unroll
      for (int t = 0; t < LW; ++t) emit_coh(p, (size_t)m * p.ldy + ncol + t, (uint16_t)f32_to_bf16(v[t]));
    } else if constexpr (LW == 1) {
      const uint16_t yb = (uint16_t)f32_to_bf16(v[0]);
      dst[0] = yb;
      if constexpr (NXT) {
        const float y = bf16_to_f32(yb);
        const float g = bf16_to_f32((uint16_t)(gword >> (16 * (ncol & 1))));
        p.xg[(size_t)m * p.ldy + ncol] = (uint16_t)f32_to_bf16(y * g);
        const float sq = row_sum16(y * y);
        if ((ncol & 15) == 0) p.ss_out[(size_t)m * (p.N >> 4) + (ncol >> 4)] = sq;
      }
    } else {
      uint32_t packed[LW / 2];
#pragma unroll
      for (int j = 0; j < LW / 2; ++j) packed[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
      if constexpr (LW == 8) *reinterpret_cast<u32x4*>(dst) = u32x4{packed[0], packed[1], packed[2], packed[3]};
      else if constexpr (LW == 4) *reinterpret_cast<u32x2*>(dst) = u32x2{packed[0], packed[1]};
      else *reinterpret_cast<uint32_t*>(dst) = packed[0];
    }
  } else if constexpr (LW >= 2) {
    // fused column 2q = gate q, 2q + 1 = up q
    float o0[LW / 2], o1[LW / 2];
#pragma unroll
    for (int q = 0; q < LW / 2; ++q) {
      const float g = round_bf16(v_in[2 * q]);
      const float u = round_bf16(v_in[2 * q + 1]);
      if (p.epi == EPI_SWIGLU) {
        o0[q] = round_bf16(silu_f32(g)) * u;
        o1[q] = 0.0f;
      } else {
        o0[q] = g;
        o1[q] = u;
      }
    }
    const size_t off = (size_t)m * p.ldy + (ncol >> 1);
    if constexpr (LW == 8) {
      *reinterpret_cast<u32x2*>(p.y0 + off) = u32x2{pack_bf16x2(o0[0], o0[1]), pack_bf16x2(o0[2], o0[3])};
      if (p.epi == EPI_PAIRED)
        *reinterpret_cast<u32x2*>(p.y1 + off) = u32x2{pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3])};
    } else if constexpr (LW == 4) {
      *reinterpret_cast<uint32_t*>(p.y0 + off) = pack_bf16x2(o0[0], o0[1]);
      if (p.epi == EPI_PAIRED) *reinterpret_cast<uint32_t*>(p.y1 + off) = pack_bf16x2(o1[0], o1[1]);
    } else if constexpr (COH) {
      emit_coh(p, off, (uint16_t)f32_to_bf16(o0[0]));   // SwiGLU output (paired outputs are not handed over)
    } else {
      p.y0[off] = (uint16_t)f32_to_bf16(o0[0]);
      if (p.epi == EPI_PAIRED) p.y1[off] = (uint16_t)f32_to_bf16(o1[0]);
    }
  }
}

// Reduce the waves' sums of one tile in LDS (one barrier, fixed order) and store:
// every wave that had chunks (wave < nw) parks its sums (and, fused norm, its
// rows' sums of squares) in red ([W][E][64]) and s_ss ([W][16]); then wave
// 4 mi + i adds row i of m-tile mi over the waves in wave order and stores it.
// PRE (chained norm, consumer; PRE 4-wide pieces a lane): ssq holds this lane's share
// of its row's block sums of squares (ss_in); the row's 16 lanes add theirs.  NXT:
// gword goes to store_row.
template <int MT, int LW, int W, bool NORM, bool COH, int PRE = 0, bool NXT = false>
__device__ __forceinline__ void reduce_store(const LinearParams& p, int ncol, int nw, int st_mi, int st_i,
                                             int st_local, int st_m, const float (&total)[MT][LW][4], float ss,
                                             const uint32_t (&resv)[(LW + 1) / 2], float* red, float* s_ss,
                                             const f32x4* ssq = nullptr, uint32_t gword = 0) {
  constexpr int E = MT * LW * 4;
  static_assert(W >= 4 * MT, "one reducing wave per (m-tile, row of the lane)");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if constexpr (NORM) {
    ss += __shfl_xor(ss, 16, 64);   // the four k sub-blocks of A row c
    ss += __shfl_xor(ss, 32, 64);
  }
  if (wave < nw) {
    float* dst = red + wave * E * 64 + lane;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int t = 0; t < LW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[((mi * LW + t) * 4 + i) * 64] = total[mi][t][i];
    if constexpr (NORM) {
      if (lane < 16) s_ss[wave * 16 + lane] = ss;
    }
  }
  __syncthreads();
  if (wave >= 4 * MT) return;
  float v[LW];
#pragma unroll
  for (int t = 0; t < LW; ++t) v[t] = 0.0f;
  float t_ss = 0.0f;   // fused norm: output row st_local of the tile is A row st_local (MT = 1)
  for (int w = 0; w < nw; ++w) {
    const float* src = red + w * E * 64 + lane;
#pragma unroll
    for (int t = 0; t < LW; ++t) v[t] += src[((st_mi * LW + t) * 4 + st_i) * 64];
    if constexpr (NORM) t_ss += s_ss[w * 16 + st_local];
  }
  if constexpr (PRE > 0) {
    float part = 0.0f;
#pragma unroll
    for (int q = 0; q < PRE; ++q) part += ((ssq[q][0] + ssq[q][1]) + ssq[q][2]) + ssq[q][3];
    t_ss = row_sum16(part);   // the row's 16 lanes: every block of K
  }
  if constexpr (NORM || PRE > 0) {
    const float inv = round_bf16(1.0f / sqrtf(t_ss / (float)p.K + p.eps));
#pragma unroll
    for (int t = 0; t < LW; ++t) v[t] *= inv;
  }
  store_row<LW, COH, NXT>(p, ncol, st_m, v, resv, gword);
}

// Workgroups are dealt to the 8 XCDs round robin by linear id, and each XCD has
// its own L2.  Neighbouring column blocks share 128-byte lines of qweight,
// scales and qzeros, so the blocks are renumbered to give each XCD one
// contiguous range of them: a shared line is then fetched from HBM once, not
// once per XCD.  (With G a multiple of 8 the row-tile index in grid.z keeps
// the XCD, so the row tiles of a column block share its weights in one L2.)
__device__ __forceinline__ int xcd_block(int b, int G) {
  return (G & 7) ? b : (b & 7) * (G >> 3) + (b >> 3);
}

// NORM: the fused-RMSNorm variant.  RMSNorm(x) W = (1 / rms) (x * gamma) W for
// each row, so the waves multiply bf16(x * gamma) by the weights as soon as
// their own loads land, summing each row's squares alongside, and the row's
// 1 / rms, bf16(1 / sqrt(mean(x^2) + eps)) as the standalone RMSNorm rounds it,
// multiplies the finished sums.  Normalising before the product needs every
// row's full sum of squares first, that is two workgroup barriers ahead of the
// MFMAs (measured 0.92 against 0.86 ms per decode step); the only change is
// where the products are rounded to bf16.
// Everything the first loads' addresses need comes as leading scalar arguments
// (x, qweight, scales, qzeros, the residual or norm weight, N, M, K and the
// column-block count G = gridDim.x), which the library is built to preload into
// SGPRs at wave launch: the first loads are issued without waiting for a load of
// the kernel arguments (measured 4.8 -> 4.4 us per launch over the decode shapes).
// The other fields come from p_ (the epilogue's, needed once the data is in).
// M_ carries log2 of the row-tile height in bits 24 and up (M < 2^24).
// One workgroup's tile of the decode linear: column block bx (of G) and row tile bz.
// after_loads() runs once the first chunk's loads are issued and before any of
// them is waited for (a fused kernel issues its own loads there).
struct NoHook {
  __device__ __forceinline__ void operator()() const {}
};
// XROWS: activation rows read whole (load_chunk), through a per-wave LDS region.
// TILED: qweight in the 16-column tile layout (t2i_w4a16_tile_qweight).
// RES: the launch may have a residual (residual epilogue); the fused-norm variant
// has none and issues no residual load (an unused load still costs: RMSNorm +
// gate_up + SwiGLU at batch 16 4.18 -> 4.08 us without it).
// PRE / NXT: the chained norm's consumer (x pre-multiplied by the norm weight, the
// rows' sums of squares in ss_in) and producer (residual epilogue that also writes
// the next norm's input and block sums of squares); see LinearParams.
template <int MT, int LW, int W, int CK, bool NORM, bool XROWS = false, bool TILED = false, int PRE = 0,
          bool NXT = false, bool RES = !NORM && PRE == 0, class Hook = NoHook>
__device__ __forceinline__ void linear_tile(const LinearParams& p, int G, int bx, int bz,
                                            const Hook& after_loads = Hook()) {
  static_assert(!(NORM && RES), "the fused-norm variant has no residual");
  static_assert(!NORM || MT == 1, "the fused-norm variant works on one 16-row tile");
  static_assert(PRE == 0 || (!NORM && !RES && MT == 1), "the chained norm's consumer: one tile, no residual");
  static_assert(!NXT || (RES && LW == 1 && MT == 1), "the chained norm's producer: residual, one column a lane");
  constexpr int E = MT * LW * 4;      // fp32 results per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar control flow
  const int c = lane & 15;
  const int r = lane >> 4;
  const int ncol = xcd_block(bx, G) * (16 * LW) + LW * c;
  const int zshift = (ncol & 7) * 4;
  const int mbase = bz * p.rt;   // row tile of this workgroup

  // this wave's chunks: a contiguous slice of K
  const int per_wave = (p.chunks + W - 1) / W;
  const int c_begin = wave * per_wave;
  const int c_end = min(c_begin + per_wave, p.chunks);

  float total[MT][LW][4];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int t = 0; t < LW; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) total[mi][t][i] = 0.0f;
  float ss = 0.0f;   // fused norm: this lane's share of its A row's sum of squares

  // every wave loads a first chunk (a wave without chunks reloads the last and computes nothing)
  Chunk<MT, LW, CK> A, B;
  __shared__ u32x4 xsh[XROWS ? W * CK * 64 : 1];   // each wave's chunk region (XROWS)
  u32x4* const xreg = &xsh[XROWS ? wave * CK * 64 : 0];
  __shared__ u32x4 gsh[NORM ? W * 4 * CK : 1];     // each wave's norm-weight pieces (NORM)
  u32x4* const greg = &gsh[NORM ? wave * 4 * CK : 0];
  load_chunk<MT, LW, CK, NORM, XROWS, TILED>(p, min(c_begin, p.chunks - 1), ncol, c, r, mbase, A);
  // The residual values this wave stores (residual epilogue) are fetched with
  // the chunks, so the epilogue waits for nothing: after every chunk's loads in
  // the straight schedules (they retire last; ahead of the later chunks the sweep
  // measured 0.5 % slower), before the loop otherwise.  The load is
  // unconditional: waves that store nothing fetch a clamped row and drop it.
  const int st_mi = min(wave >> 2, MT - 1), st_i = wave & 3;
  const int st_local = st_mi * 16 + r * 4 + st_i;
  const int st_m = st_local < p.rt ? mbase + st_local : p.M;   // the row this lane stores (M: none)
  uint32_t resv[(LW + 1) / 2] = {};
  f32x4 ssq[PRE > 0 ? PRE : 1] = {};   // PRE: this lane's pieces of its row's block sums of squares (K = 1024 PRE)
  uint32_t gword[1] = {};              // NXT: the word of g_next holding this lane's column
  const auto load_res = [&]() {
    if constexpr (RES)   // (a launch without one reads the scales row instead: in bounds, unused)
      load_scales<LW>(p.residual ? p.residual + (size_t)min(st_m, p.M - 1) * p.ldy + ncol : p.sc + ncol, resv,
                      ncol & 1);
    if constexpr (NXT) load_scales<1>(p.g_next + ncol, gword, ncol & 1);
    if constexpr (PRE > 0) {
      const float* src = p.ss_in + (size_t)min(st_m, p.M - 1) * (64 * PRE) + 4 * c;
#pragma unroll
      for (int q = 0; q < PRE; ++q) ssq[q] = *reinterpret_cast<const f32x4*>(src + 64 * q);
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  after_loads();
  __builtin_amdgcn_sched_barrier(0);
  // One word per lane: straight-line schedules for up to 6 chunks per wave (3
  // with the fused norm), else a double-buffered loop.
  // Wider tiles use the loop alone, which keeps their registers (occupancy) as
  // they were; their decode plans have one chunk per wave.
  const int n = c_end - c_begin;   // wave-uniform
  bool looped = true;
  if constexpr (LW == 1) {
    constexpr bool DEEP = !NORM && CK == 2;   // 4..6 chunks in registers: 12 a chunk
    looped = false;
    if (n == 1) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 1>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else if (n == 2) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 2>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else if (n == 3) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 3>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else if (DEEP && n == 4) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 4>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else if (DEEP && n == 5) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 5>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else if (DEEP && n == 6) {
      straight_chunks<MT, LW, CK, NORM, XROWS, TILED, 6>(p, c_begin, ncol, c, r, mbase, A, total, ss, zshift, xreg, greg,
                                                            load_res);
    } else {
      looped = true;
    }
  }
  if (looped) {
    load_res();
    for (int ch = c_begin; ch < c_end; ch += 2) {
      if (ch + 1 < c_end) load_chunk<MT, LW, CK, NORM, XROWS, TILED>(p, ch + 1, ncol, c, r, mbase, B);
      compute_loaded<MT, LW, CK, NORM, XROWS>(A, total, ss, zshift, xreg, lane, p.rt, greg);
      if (ch + 1 >= c_end) break;
      if (ch + 2 < c_end) load_chunk<MT, LW, CK, NORM, XROWS, TILED>(p, ch + 2, ncol, c, r, mbase, A);
      compute_loaded<MT, LW, CK, NORM, XROWS>(B, total, ss, zshift, xreg, lane, p.rt, greg);
    }
  }

  // ---- reduce the waves of this workgroup in LDS: one barrier, fixed order ----
  const int nw = (p.chunks + per_wave - 1) / per_wave;   // waves that had chunks
  __shared__ float red[W * E * 64];
  __shared__ float s_ss[NORM ? W : 1][16];
  reduce_store<MT, LW, W, NORM, false, PRE, NXT>(p, ncol, nw, st_mi, st_i, st_local, st_m, total, ss, resv, red,
                                                 &s_ss[0][0], ssq, gword[0]);
}

// One workgroup's tile of a linear phase inside a launch that runs dependent
// phases (the one-launch decode step): each wave requests the weights of all its
// chunks, then wait() runs (workgroup-uniform; whatever the caller issues
// there), then the activation rows and the residual come in with agent-coherent
// loads, as tagged words awaited until they carry this launch's tag (xll / rll)
// or as bf16 rows a previous launch wrote.  Chunk
// ranges, arithmetic and reduction order are linear_tile's, so a plan gives the
// same bits as the standalone kernel.  Straight schedules only, of at most NMAX
// chunks a wave (3 with the fused norm, 6 without at CK = 2); returns false (and
// computes nothing) for a plan beyond that, which the host rejects up front.
// The output goes out as tagged words (yll) or agent-coherent bf16 stores; the
// stores are not waited for (a consumer awaits the tags, or the launch's end).
template <int MT, int LW, int CK, bool NORM, int NC, int NMAX>
__device__ __forceinline__ void phase_weights(const LinearParams& p, int c_begin, int ncol, int r,
                                              Chunk<MT, LW, CK> (&ch)[NMAX]) {
#pragma unroll
  for (int i = 0; i < NC; ++i) load_chunk_w<MT, LW, CK, NORM>(p, c_begin + i, ncol, r, ch[i]);
}
template <int MT, int LW, int CK, bool NORM, int NC, int NMAX>
__device__ __forceinline__ void phase_compute(const LinearParams& p, int c_begin, int c, int r, int mbase,
                                              Chunk<MT, LW, CK> (&ch)[NMAX], float (&total)[MT][LW][4],
                                              float& ss, int zshift) {
  if (p.xll) {
    // tagged input words: all requested, then each group awaited in order
    Tagged8 raw[NC][MT][CK];
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int j = 0; j < CK; ++j)
          tagged_issue(p.xll + (size_t)tile_row(p, mbase, mi * 16 + c) * p.ldx + ((c_begin + i) * CK + j) * 32 + r * 8,
                       raw[i][mi][j]);
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int j = 0; j < CK; ++j)
          ch[i].x[mi][j] = tagged_wait8(
              p.xll + (size_t)tile_row(p, mbase, mi * 16 + c) * p.ldx + ((c_begin + i) * CK + j) * 32 + r * 8,
              raw[i][mi][j], p.xtag, p.ctl);
  } else {
#pragma unroll
    for (int i = 0; i < NC; ++i) load_chunk_x_coh<MT, LW, CK>(p, c_begin + i, c, r, mbase, ch[i]);
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) compute_chunk<MT, LW, CK, NORM>(ch[i], total, ss, zshift);
}

template <int MT, int LW, int W, int CK, bool NORM, int NMAX, class Wait>
__device__ __forceinline__ bool linear_phase(const LinearParams& p, int G, int bx, int bz, float* red, float* s_ss,
                                             const Wait& wait) {
  static_assert(NMAX >= 1 && NMAX <= (NORM ? 3 : 6), "straight schedules of up to 3 chunks (fused norm) or 6");
  static_assert(NMAX <= 3 || CK == 2, "more than three chunks in registers only at two k-steps a chunk");
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int r = lane >> 4;
  const int ncol = xcd_block(bx, G) * (16 * LW) + LW * c;
  const int zshift = (ncol & 7) * 4;
  const int mbase = bz * p.rt;
  const int per_wave = (p.chunks + W - 1) / W;
  const int c_begin = wave * per_wave;
  const int n = min(c_begin + per_wave, p.chunks) - c_begin;   // wave-uniform; <= 0: no chunks
  const bool fits = per_wave <= NMAX;

  float total[MT][LW][4];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int t = 0; t < LW; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) total[mi][t][i] = 0.0f;
  float ss = 0.0f;
  Chunk<MT, LW, CK> ch[NMAX];
  if (fits) {
    if (n == 1) phase_weights<MT, LW, CK, NORM, 1, NMAX>(p, c_begin, ncol, r, ch);
    if constexpr (NMAX >= 2) if (n == 2) phase_weights<MT, LW, CK, NORM, 2, NMAX>(p, c_begin, ncol, r, ch);
    if constexpr (NMAX >= 3) if (n == 3) phase_weights<MT, LW, CK, NORM, 3, NMAX>(p, c_begin, ncol, r, ch);
    if constexpr (NMAX >= 4) if (n == 4) phase_weights<MT, LW, CK, NORM, 4, NMAX>(p, c_begin, ncol, r, ch);
    if constexpr (NMAX >= 5) if (n == 5) phase_weights<MT, LW, CK, NORM, 5, NMAX>(p, c_begin, ncol, r, ch);
    if constexpr (NMAX >= 6) if (n == 6) phase_weights<MT, LW, CK, NORM, 6, NMAX>(p, c_begin, ncol, r, ch);
  }
  wait();
  // the row this lane stores and, with a residual, its values
  const int st_mi = min(wave >> 2, MT - 1), st_i = wave & 3;
  const int st_local = st_mi * 16 + r * 4 + st_i;
  const int st_m = st_local < p.rt ? mbase + st_local : p.M;   // M: none
  uint32_t resv[(LW + 1) / 2];
#pragma unroll
  for (int i = 0; i < (LW + 1) / 2; ++i) resv[i] = 0u;
  if constexpr (!NORM && LW == 1) {
    const size_t ridx = (size_t)min(st_m, p.M - 1) * p.ldy + ncol;
    if (p.rll) resv[0] = tagged_wait1(p.rll + ridx, p.rtag, p.ctl);
    else if (p.residual) resv[0] = ld_coh32(reinterpret_cast<const uint32_t*>(p.residual + ridx - (ncol & 1)));
  }
  if (!fits) return false;
  if (n == 1) phase_compute<MT, LW, CK, NORM, 1, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  if constexpr (NMAX >= 2) if (n == 2) phase_compute<MT, LW, CK, NORM, 2, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  if constexpr (NMAX >= 3) if (n == 3) phase_compute<MT, LW, CK, NORM, 3, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  if constexpr (NMAX >= 4) if (n == 4) phase_compute<MT, LW, CK, NORM, 4, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  if constexpr (NMAX >= 5) if (n == 5) phase_compute<MT, LW, CK, NORM, 5, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  if constexpr (NMAX >= 6) if (n == 6) phase_compute<MT, LW, CK, NORM, 6, NMAX>(p, c_begin, c, r, mbase, ch, total, ss, zshift);
  const int nw = (p.chunks + per_wave - 1) / per_wave;
  reduce_store<MT, LW, W, NORM, true>(p, ncol, nw, st_mi, st_i, st_local, st_m, total, ss, resv, red, s_ss);
  return true;
}

}  // namespace t2i

namespace t2i_host {
// The decode linear's tile plan for an M x K x N product (defined with the
// standalone kernel, which launches it; the one-launch decode step runs the same
// plans so that both give the same bits).
struct LinearPlan {
  int MT, LW, W, CK;
  int rt;       // rows per row tile (16 * MT, or fewer)
  int mz;       // row tiles (grid.z)
  int cbs;      // column blocks (grid.x)
  int chunks;   // K / (32 * CK)
};
// wide: the plan for 16-wave workgroups (the one-launch decode step's).
LinearPlan plan_linear(int M, int K, int N, bool paired, bool norm, bool wide);
}  // namespace t2i_host
