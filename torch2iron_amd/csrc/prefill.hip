// Prompt (prefill) kernels for gfx950: every prompt row of a batch at once.
//
//   * t2i_prefill_qk_rope_kv: per-head q/k RMSNorm + RoPE of every prompt row,
//     q stored per (sequence, head) for the attention, k and v written into the
//     contiguous KV cache at their positions;
//   * t2i_prefill_attention: causal GQA attention of the prompt rows over the
//     cache on MFMA (flash-attention style: 64-key blocks through LDS, an online
//     softmax per query row, P . V on MFMA), bf16 context out.
//
// Rounding follows the decode path (and the reference runtime in bf16
// compute, quantized_qwen3/model.py:246-253, 268-280): q/k norm and RoPE round
// at the same points; scores and softmax are fp32; the softmax weights enter
// the P . V product as bf16 (model.py:277 casts them to the compute dtype
// before that product), and each row's normaliser sums those bf16 weights.
#include <math.h>

#include "t2i_common.h"
#include "qk_prep.h"

namespace t2i {

constexpr int PF_D = 128;

// ============================================================================
// q/k RMSNorm + RoPE + KV-cache write for every prompt row
// ============================================================================
struct PrefillPrepParams {
  const uint16_t* qkv;    // [B*T, (Hq + 2 Hkv) * D] raw projection, row b*T + t
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* rope;   // [>= p0 + T, D] cos even / sin odd
  uint16_t* q;            // [B, Hq, T, D]
  uint16_t* kc;           // [B, Hkv, cap, D]
  uint16_t* vc;
  int B, T, Hq, Hkv, cap, p0, style;
  float eps;
};

// One workgroup (4 waves) per prompt row.  A head vector is held by a 16-lane
// row of a wave (the lane layout of qk_prep.h).  A wave covers 4 vectors, the
// workgroup 16 at a time; every load of PREP_NB such batches (and the norm
// weights and the RoPE row) is issued before the first vector is normalised.
// Loads are unconditional (vectors past the last reload it; nothing is stored
// for them).
constexpr int PREP_NB = 2;

__global__ __launch_bounds__(256) void prefill_prep_kernel(const PrefillPrepParams p) {
  constexpr int D = PF_D;
  const int row = blockIdx.x;
  const int b = row / p.T;
  const int t = row - b * p.T;
  const int pos = p.p0 + t;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 4 + (lane >> 4);   // 0 .. 15
  const int nvec = p.Hq + 2 * p.Hkv;
  const uint16_t* src_row = p.qkv + (size_t)row * nvec * D;
  for (int base = 0; base < nvec; base += 16 * PREP_NB) {
    u32x4 raw[PREP_NB];
#pragma unroll
    for (int j = 0; j < PREP_NB; ++j)
      raw[j] = prep_load(src_row + (size_t)min(base + 16 * j + slot, nvec - 1) * D, c, p.style);
    const u32x4 rp = *reinterpret_cast<const u32x4*>(p.rope + (size_t)pos * D + 8 * c);   // (cos, sin) x 4
    const u32x4 gqv = prep_load(p.qn, c, p.style);
    const u32x4 gkv = prep_load(p.kn, c, p.style);
    // all of the batch's loads before the first use (the compiler would sink a
    // vector's loads behind the previous vector's normalisation)
#pragma unroll
    for (int j = 0; j < PREP_NB; ++j) asm volatile("" : "+v"(raw[j]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < PREP_NB; ++j) {
      const int vi = base + 16 * j + slot;   // uniform over the 16-lane row
      const bool isq = vi < p.Hq;
      const bool normed = vi < p.Hq + p.Hkv;   // q and k: RMSNorm + RoPE; v as is
      const u32x4 y = prep_vector(raw[j], rp, isq ? gqv : gkv, normed, p.style, p.eps);
      if (vi >= nvec) continue;
      uint16_t* dst;
      if (isq) dst = p.q + (((size_t)b * p.Hq + vi) * p.T + t) * D;
      else if (normed) dst = p.kc + (((size_t)b * p.Hkv + (vi - p.Hq)) * p.cap + pos) * D;
      else dst = p.vc + (((size_t)b * p.Hkv + (vi - p.Hq - p.Hkv)) * p.cap + pos) * D;
      prep_store(dst, c, p.style, y);
    }
  }
}

// ============================================================================
// causal GQA flash attention over the cache
// ============================================================================
constexpr int PF_ROWS = 64;                 // query rows per workgroup (over the kv head's q heads)
constexpr int PF_KEYS = 64;                 // keys per block
constexpr int PF_KLD = PF_D + 8;            // K tile row stride (bf16): 272 bytes
// Transposed V tile row stride: 136 bytes = 34 banks, so the 16 rows (dims) of an
// 8-byte A-operand read fall on 16 distinct bank pairs (a 144-byte stride put dims
// c and c + 8 on one pair, and the staging stores of 16 dims 8 apart on one bank:
// 69 against 62 us a layer, with 5x the LDS bank conflicts).
constexpr int PF_VLD = PF_KEYS + 4;

struct PrefillAttnParams {
  const uint16_t* q;      // [B, Hq, T, D]
  const uint16_t* kc;     // [B, Hkv, cap, D]
  const uint16_t* vc;
  uint16_t* out;          // [B*T, Hq * D]
  float* out_sums;        // NULL, or [Hq, B*T]: each head's sum of its bf16 context values
  int B, T, Hq, Hkv, cap, p0;
  float scale_log2;       // D^-1/2 * log2(e)
};

// One workgroup per (sequence b, kv head h, query block); 4 waves of 16 query
// rows.  Row j of the PF_ROWS is q head h * Q + j / BQ at prompt row
// t0 + j % BQ (BQ = PF_ROWS / Q), so the q heads sharing kv head h share every
// K / V block.  Everything runs transposed, so that a lane holds one query row:
//   S^T = K Q^T: A = K from LDS (lane (c, r): key c, dims 8 r ..), B = the
//     wave's q rows (registers); the output gives lane (c, r) row 16 w + c's
//     scores for keys 4 r .. 4 r + 3 of each 16-key tile;
//   online softmax per lane (the row's max and sum over the four lanes of the
//     row with two exchanges), rescaling the lane's own outputs;
//   O^T += V^T P^T: B = P^T straight from the softmax registers (a k-step's 32
//     keys in the order tile 2 ks keys 4 r ..+3, tile 2 ks + 1 keys 4 r ..+3 --
//     any order works as long as A uses the same), A = V^T from LDS read in that
//     order; the output gives lane (c, r) row c's dims 16 n + 4 r .. + 3.
// V is transposed in registers on its way into LDS (four keys x eight dims a
// thread, byte permutes, 8-byte stores).  Against the untransposed form (S = Q K^T
// with rows spread over lanes, P through a per-wave LDS tile, V stored as 2-byte
// pieces): 66.0 -> 47.7 us a layer at 16 sequences x 512 rows (same box).
template <int Q>
__global__ __launch_bounds__(256, 3) void prefill_attention_kernel(const PrefillAttnParams p) {
  constexpr int D = PF_D;
  constexpr int BQ = PF_ROWS / Q;           // prompt rows per q head in the tile
  // Query blocks are dealt last block first (grid.y counts down): the causal
  // work of a block grows with its position, so the longest go out first and
  // the short ones fill the tail.
  const int t0 = (gridDim.y - 1 - blockIdx.y) * BQ;
  const int h = blockIdx.x % p.Hkv;
  const int b = blockIdx.x / p.Hkv;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int r = lane >> 4;

  __shared__ __align__(16) uint16_t s_k[PF_KEYS * PF_KLD];     // [key][dim]
  __shared__ __align__(16) uint16_t s_vt[D * PF_VLD];          // [dim][key]

  // ---- this lane's query row j = 16 wave + c, as the B operand (dims 32 ks + 8 r ..) ----
  const int jrow = wave * 16 + c;
  const int t_row = t0 + jrow % BQ;
  const int head = h * Q + jrow / BQ;
  const int qpos = p.p0 + t_row;             // keys beyond it are masked
  u32x4 qb[4];
  {
    const uint16_t* src = p.q + (((size_t)b * p.Hq + head) * p.T + min(t_row, p.T - 1)) * D + 8 * r;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = *reinterpret_cast<const u32x4*>(src + ks * 32);
  }
  // the smallest query position of the wave's rows (wave-uniform): rows j0 ..
  // j0 + 15 of the tile are prompt rows t0 + j % BQ
  const int j0 = wave * 16;
  const int qmin = p.p0 + t0 + ((j0 % BQ) + 16 <= BQ ? j0 % BQ : 0);
  const int last_t = min(t0 + BQ, p.T) - 1;
  const int kend = p.p0 + last_t + 1;        // keys [0, kend) can be attended
  const size_t cache_base = ((size_t)b * p.Hkv + h) * (size_t)p.cap * D;

  float m = -INFINITY, l = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K / V block staging: 64 keys x 128 dims each = 1024 chunks of 16 bytes; 4 per
  // thread.  K chunk q: key q / 16, dims 8 (q % 16), stored as loaded.  V: thread
  // (key group g = tid % 16, octet o = tid / 16) loads keys 4 g .. 4 g + 3 of dims
  // 8 o .. 8 o + 7 and stores each dim's four keys as one 8-byte piece of s_vt (16
  // lanes of a store cover one dim's 64 keys: no bank conflicts).  Loads are
  // unconditional (keys past kend reload key kend - 1: finite values whose
  // softmax weights are zero).
  const int vgrp = tid & 15, voct = tid >> 4;
  auto load_block = [&](int kb, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q16 = tid + 256 * u;
      const int kkey = min(kb * PF_KEYS + (q16 >> 4), kend - 1);
      const int vkey = min(kb * PF_KEYS + 4 * vgrp + u, kend - 1);
      kr[u] = *reinterpret_cast<const u32x4*>(p.kc + cache_base + (size_t)kkey * D + 8 * (q16 & 15));
      vr[u] = *reinterpret_cast<const u32x4*>(p.vc + cache_base + (size_t)vkey * D + 8 * voct);
    }
  };
  auto store_block = [&](u32x4 (&kr)[4], u32x4 (&vr)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q16 = tid + 256 * u;
      *reinterpret_cast<u32x4*>(s_k + (q16 >> 4) * PF_KLD + 8 * (q16 & 15)) = kr[u];
    }
    const uint32_t w0[4] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w};
    const uint32_t w1[4] = {vr[1].x, vr[1].y, vr[1].z, vr[1].w};
    const uint32_t w2[4] = {vr[2].x, vr[2].y, vr[2].z, vr[2].w};
    const uint32_t w3[4] = {vr[3].x, vr[3].y, vr[3].z, vr[3].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // dims 2 e (low halves) and 2 e + 1 (high halves) of keys 4 g .. 4 g + 3
      const u32x2 lo = u32x2{__builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u), __builtin_amdgcn_perm(w3[e], w2[e], 0x05040100u)};
      const u32x2 hi = u32x2{__builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u), __builtin_amdgcn_perm(w3[e], w2[e], 0x07060302u)};
      *reinterpret_cast<u32x2*>(s_vt + (8 * voct + 2 * e) * PF_VLD + 4 * vgrp) = lo;
      *reinterpret_cast<u32x2*>(s_vt + (8 * voct + 2 * e + 1) * PF_VLD + 4 * vgrp) = hi;
    }
  };

  const int nblocks = (kend + PF_KEYS - 1) / PF_KEYS;
  u32x4 kr[4], vr[4];
  load_block(0, kr, vr);
  for (int kb = 0; kb < nblocks; ++kb) {
    __syncthreads();                          // the previous block's tiles are consumed
    store_block(kr, vr);
    __syncthreads();
    if (kb + 1 < nblocks) load_block(kb + 1, kr, vr);
    // ---- S^T = K Q^T: 4 key tiles of 16 ----
    f32x4 s[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(s_k + (n * 16 + c) * PF_KLD + ks * 32 + 8 * r);
        s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka),
                                                       __builtin_bit_cast(bf16x8, qb[ks]), s[n], 0, 0, 0);
      }
    }
    // ---- online softmax of the lane's row (log2 domain), causal mask ----
    // Blocks that every row of the wave sees whole skip the mask.  The scale goes
    // into the exponent's FMA (the max of the scaled scores is the scaled max); a
    // masked score is -inf, whose weight 2^-inf is 0.
    if (kb * PF_KEYS + PF_KEYS - 1 > qmin) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kb * PF_KEYS + n * 16 + 4 * r + i > qpos) s[n][i] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
#pragma unroll
    for (int n = 1; n < 4; ++n) mx = fmaxf(mx, fmaxf(fmaxf(s[n][0], s[n][1]), fmaxf(s[n][2], s[n][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx * p.scale_log2);   // finite: every row attends key 0
    const float f = __builtin_amdgcn_exp2f(m - mn);  // 0 while m is -inf
    float sum = 0.0f;
    uint32_t pw[4][2];                        // bf16 weights, two keys a word
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const uint32_t w = pack_bf16x2(__builtin_amdgcn_exp2f(fmaf(s[n][i], p.scale_log2, -mn)),
                                       __builtin_amdgcn_exp2f(fmaf(s[n][i + 1], p.scale_log2, -mn)));
        pw[n][i / 2] = w;
        sum += __uint_as_float(w << 16) + __uint_as_float(w & 0xFFFF0000u);   // the rounded weights
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    l = l * f + sum;
    m = mn;
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[n][i] *= f;
    // ---- O^T += V^T P^T: 2 k-steps of 32 keys, 8 dim tiles ----
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 pb = u32x4{pw[2 * ks][0], pw[2 * ks][1], pw[2 * ks + 1][0], pw[2 * ks + 1][1]};
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const uint16_t* vrow = s_vt + (n * 16 + c) * PF_VLD + ks * 32 + 4 * r;
        const u32x2 v0 = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 v1 = *reinterpret_cast<const u32x2*>(vrow + 16);
        const u32x4 va = u32x4{v0.x, v0.y, v1.x, v1.y};
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, va),
                                                       __builtin_bit_cast(bf16x8, pb), o[n], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: the lane holds row jrow's dims 16 n + 4 r .. + 3 ----
  if (t_row < p.T) {
    uint16_t* dst = p.out + ((size_t)b * p.T + t_row) * p.Hq * D + (size_t)head * D + 4 * r;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float hs = 0.0f;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const float y0 = round_bf16(o[n][0] * inv), y1 = round_bf16(o[n][1] * inv);
      const float y2 = round_bf16(o[n][2] * inv), y3 = round_bf16(o[n][3] * inv);
      *reinterpret_cast<u32x2*>(dst + n * 16) = u32x2{pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
      hs += ((y0 + y1) + (y2 + y3));
    }
    if (p.out_sums) {
      // the head's 128 values are one quantisation group of the next product's k
      hs += __shfl_xor(hs, 16, 64);
      hs += __shfl_xor(hs, 32, 64);
      if (r == 0) p.out_sums[(size_t)head * p.B * p.T + (size_t)b * p.T + t_row] = hs;
    }
  }
}

}  // namespace t2i

// ============================================================================
// host side
// ============================================================================
using t2i_host::aligned16;
using t2i_host::fail;

extern "C" int t2i_prefill_qk_rope_kv(const uint16_t* qkv, int32_t B, int32_t T, int32_t p0, int32_t Hq,
                                      int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm,
                                      float eps, const uint16_t* rope, int32_t rope_style, uint16_t* q_out,
                                      uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, void* stream) {
  if (!qkv || !q_norm || !k_norm || !rope || !q_out || !k_cache || !v_cache)
    return fail(T2I_ERR_NULL, "prefill prep pointers must not be NULL");
  if (D != t2i::PF_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (B < 1 || T < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv) return fail(T2I_ERR_SHAPE, "B=%d T=%d Hq=%d Hkv=%d invalid", B, T, Hq, Hkv);
  if (p0 < 0 || ctx_cap < 1 || p0 + T > ctx_cap) return fail(T2I_ERR_SHAPE, "positions %d..%d exceed the cache (%d)", p0, p0 + T - 1, ctx_cap);
  if ((long long)B * T > 0x7FFFFFFF / 2) return fail(T2I_ERR_SHAPE, "B*T too large");
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  t2i::PrefillPrepParams p{};
  p.qkv = qkv; p.qn = q_norm; p.kn = k_norm; p.rope = rope; p.q = q_out; p.kc = k_cache; p.vc = v_cache;
  p.B = B; p.T = T; p.Hq = Hq; p.Hkv = Hkv; p.cap = ctx_cap; p.p0 = p0; p.style = rope_style; p.eps = eps;
  hipLaunchKernelGGL(t2i::prefill_prep_kernel, dim3(B * T), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
  return t2i_host::hip_status(hipGetLastError(), "prefill prep launch");
}

namespace {
int run_prefill_attention(const uint16_t* q, int32_t B, int32_t T, int32_t p0, int32_t Hq, int32_t Hkv, int32_t D,
                          const uint16_t* k_cache, const uint16_t* v_cache, int32_t ctx_cap, uint16_t* out,
                          float* out_sums, void* stream) {
  if (!q || !k_cache || !v_cache || !out) return fail(T2I_ERR_NULL, "prefill attention pointers must not be NULL");
  if (out_sums && ((uintptr_t)out_sums & 3u)) return fail(T2I_ERR_ALIGN, "out_sums must be 4-byte aligned");
  if (D != t2i::PF_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (B < 1 || T < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv) return fail(T2I_ERR_SHAPE, "B=%d T=%d Hq=%d Hkv=%d invalid", B, T, Hq, Hkv);
  const int Q = Hq / Hkv;
  if (Q != 1 && Q != 2 && Q != 4 && Q != 8) return fail(T2I_ERR_SHAPE, "Hq/Hkv=%d must be 1, 2, 4 or 8", Q);
  if (p0 < 0 || ctx_cap < 1 || p0 + T > ctx_cap) return fail(T2I_ERR_SHAPE, "positions %d..%d exceed the cache (%d)", p0, p0 + T - 1, ctx_cap);
  if ((long long)B * Hkv > 0x7FFFFFFF || (T + t2i::PF_ROWS / (Hq / Hkv) - 1) / (t2i::PF_ROWS / (Hq / Hkv)) > 65535)
    return fail(T2I_ERR_SHAPE, "B=%d Hkv=%d T=%d exceed the grid", B, Hkv, T);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return fail(T2I_ERR_ALIGN, "prefill attention tensors must be 16-byte aligned");
  t2i::PrefillAttnParams p{};
  p.q = q; p.kc = k_cache; p.vc = v_cache; p.out = out; p.out_sums = out_sums;
  p.B = B; p.T = T; p.Hq = Hq; p.Hkv = Hkv; p.cap = ctx_cap; p.p0 = p0;
  p.scale_log2 = (float)(1.4426950408889634 / sqrt((double)D));
  const int bq = t2i::PF_ROWS / Q;
  const dim3 grid(B * Hkv, (T + bq - 1) / bq);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (Q) {
    case 1: hipLaunchKernelGGL((t2i::prefill_attention_kernel<1>), grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL((t2i::prefill_attention_kernel<2>), grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((t2i::prefill_attention_kernel<4>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((t2i::prefill_attention_kernel<8>), grid, dim3(256), 0, s, p); break;
  }
  return t2i_host::hip_status(hipGetLastError(), "prefill attention launch");
}
}  // namespace

extern "C" int t2i_prefill_attention(const uint16_t* q, int32_t B, int32_t T, int32_t p0, int32_t Hq, int32_t Hkv,
                                     int32_t D, const uint16_t* k_cache, const uint16_t* v_cache, int32_t ctx_cap,
                                     uint16_t* out, void* stream) {
  return run_prefill_attention(q, B, T, p0, Hq, Hkv, D, k_cache, v_cache, ctx_cap, out, nullptr, stream);
}

extern "C" int t2i_prefill_attention_sums(const uint16_t* q, int32_t B, int32_t T, int32_t p0, int32_t Hq,
                                          int32_t Hkv, int32_t D, const uint16_t* k_cache, const uint16_t* v_cache,
                                          int32_t ctx_cap, uint16_t* out, float* out_sums, void* stream) {
  if (!out_sums) return fail(T2I_ERR_NULL, "out_sums must not be NULL");
  return run_prefill_attention(q, B, T, p0, Hq, Hkv, D, k_cache, v_cache, ctx_cap, out, out_sums, stream);
}
