// q/k RMSNorm + RoPE of one head vector (D = 128), shared by the prompt pass's
// prep kernel and the prompt GEMM's fused q|k|v epilogue so that both give the
// same bits.  A head vector is held by a 16-lane row of a wave: lane c holds the
// 4 rotation pairs p = 4c .. 4c + 3, elements (i0, i1) = (p, p + 64) (two halves)
// or (2p, 2p + 1) (interleaved), that is two 8-byte pieces or one 16-byte piece of
// the vector, and the 4 (cos, sin) pairs of the RoPE row as one 16-byte piece.
// Rounding follows the decode path and the reference runtime in bf16 compute
// (quantized_qwen3/model.py:246-253): x * inv, then * gamma, then the rotation,
// each rounded to bf16.
#pragma once

#include "t2i_common.h"

namespace t2i {

// Lane c's piece of a head vector: style 0 the i0 values of pairs 4c .. 4c + 3
// then their i1 values (two 8-byte pieces), style 1 the four pairs interleaved.
__device__ __forceinline__ u32x4 prep_load(const uint16_t* vec, int c, int style) {
  if (style == 0) {
    const u32x2 a = *reinterpret_cast<const u32x2*>(vec + 4 * c);
    const u32x2 b = *reinterpret_cast<const u32x2*>(vec + 64 + 4 * c);
    return u32x4{a.x, a.y, b.x, b.y};
  }
  return *reinterpret_cast<const u32x4*>(vec + 8 * c);
}

__device__ __forceinline__ void prep_unpack(u32x4 v, int style, float (&x0)[4], float (&x1)[4]) {
  if (style == 0) {
    x0[0] = bf16_lo(v.x); x0[1] = bf16_hi(v.x); x0[2] = bf16_lo(v.y); x0[3] = bf16_hi(v.y);
    x1[0] = bf16_lo(v.z); x1[1] = bf16_hi(v.z); x1[2] = bf16_lo(v.w); x1[3] = bf16_hi(v.w);
  } else {
    x0[0] = bf16_lo(v.x); x1[0] = bf16_hi(v.x); x0[1] = bf16_lo(v.y); x1[1] = bf16_hi(v.y);
    x0[2] = bf16_lo(v.z); x1[2] = bf16_hi(v.z); x0[3] = bf16_lo(v.w); x1[3] = bf16_hi(v.w);
  }
}

__device__ __forceinline__ u32x4 prep_pack(const float (&y0)[4], const float (&y1)[4], int style) {
  if (style == 0)
    return u32x4{pack_bf16x2(y0[0], y0[1]), pack_bf16x2(y0[2], y0[3]), pack_bf16x2(y1[0], y1[1]),
                 pack_bf16x2(y1[2], y1[3])};
  return u32x4{pack_bf16x2(y0[0], y1[0]), pack_bf16x2(y0[1], y1[1]), pack_bf16x2(y0[2], y1[2]),
               pack_bf16x2(y0[3], y1[3])};
}

__device__ __forceinline__ void prep_store(uint16_t* vec, int c, int style, u32x4 v) {
  if (style == 0) {
    *reinterpret_cast<u32x2*>(vec + 4 * c) = u32x2{v.x, v.y};
    *reinterpret_cast<u32x2*>(vec + 64 + 4 * c) = u32x2{v.z, v.w};
  } else {
    *reinterpret_cast<u32x4*>(vec + 8 * c) = v;
  }
}

// Two values rounded to bf16 by one v_cvt_pk_bf16_f32 (the same bits as two
// round_bf16 calls).
__device__ __forceinline__ void round_pair(float& a, float& b) {
  const uint32_t p = pack_bf16x2(a, b);
  a = bf16_lo(p);
  b = bf16_hi(p);
}

// The lane's piece of the normalised and rotated vector (normed: q or k; a v
// vector passes through).  raw: the lane's piece (prep_load's layout), rp: its
// RoPE pairs, gv: its piece of the norm weight.  The sum of squares is a 16-lane
// DPP sum, so the 16 lanes of the row call it together.  The roundings of the
// two elements of a pair go together, and the rotation's sums are rounded by the
// final packing.
__device__ __forceinline__ u32x4 prep_vector(u32x4 raw, u32x4 rp, u32x4 gv, bool normed, int style, float eps) {
  constexpr int D = ATT_D;
  const float cs[4] = {bf16_lo(rp.x), bf16_lo(rp.y), bf16_lo(rp.z), bf16_lo(rp.w)};
  const float sn[4] = {bf16_hi(rp.x), bf16_hi(rp.y), bf16_hi(rp.z), bf16_hi(rp.w)};
  float g0[4], g1[4], x0[4], x1[4];
  prep_unpack(gv, style, g0, g1);
  prep_unpack(raw, style, x0, x1);
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss += x0[e] * x0[e] + x1[e] * x1[e];
  ss = row_sum16(ss);
  const float inv = round_bf16(1.0f / sqrtf(ss / (float)D + eps));
  float y0[4], y1[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float n0 = x0[e] * inv, n1 = x1[e] * inv;
    round_pair(n0, n1);
    n0 *= g0[e];
    n1 *= g1[e];
    round_pair(n0, n1);
    float c0 = n0 * cs[e], c1 = n1 * cs[e];
    float s0 = -n1 * sn[e], s1 = n0 * sn[e];
    round_pair(c0, c1);
    round_pair(s0, s1);
    y0[e] = normed ? c0 + s0 : x0[e];
    y1[e] = normed ? c1 + s1 : x1[e];
  }
  return prep_pack(y0, y1, style);
}

}  // namespace t2i
