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

#include <type_traits>

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
constexpr int PF_MF = 1;                    // 16-row fragments per wave (4 waves x 16 rows)
constexpr int PF_KEYS = 64;                 // keys per block
constexpr int PF_KLD = PF_D + 8;            // K tile row stride (bf16): 272 bytes
constexpr int PF_VLD = PF_KEYS + 8;         // transposed V tile row stride: 144 bytes
constexpr int PF_PLD = PF_KEYS + 8;         // P tile row stride

struct PrefillAttnParams {
  const uint16_t* q;      // [B, Hq, T, D]
  const uint16_t* kc;     // [B, Hkv, cap, D]
  const uint16_t* vc;
  uint16_t* out;          // [B*T, Hq * D]
  float* out_sums;        // NULL, or [B*T, Hq]: each head's sum of its bf16 context values
  int B, T, Hq, Hkv, cap, p0;
  float scale_log2;       // D^-1/2 * log2(e)
};

// One workgroup per (sequence b, kv head h, query block); 4 waves of PF_MF
// 16-row MFMA fragments.  Row j of the PF_ROWS is q head h * Q + j / BQ at
// prompt row t0 + j % BQ (BQ = PF_ROWS / Q), so the q heads sharing kv head h
// share every K / V block.  Measured slower at 16 sequences x 512 rows: two
// fragments a wave (128 rows a workgroup: 141 against 121 us a layer), and P
// written as 32-bit words of key pairs swapped between neighbouring lanes.
//   S = Q K^T: A = q rows (registers, 4 k-steps of 32 dims), B = K from LDS;
//   online softmax per row in fp32 (rows 4r + i of the lane's MFMA output);
//   O += P V: P goes to A layout through a per-wave LDS tile, B = V^T from LDS.
template <int Q>
__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(const PrefillAttnParams p) {
  constexpr int D = PF_D;
  constexpr int MF = PF_MF;
  constexpr int BQ = PF_ROWS / Q;           // prompt rows per q head in the tile
  // Query blocks are dealt last block first (grid.y counts down): the causal
  // work of a block grows with its position, so the longest go out first and
  // the short ones fill the tail.
  const int t0 = (gridDim.y - 1 - blockIdx.y) * BQ;
  const int h = blockIdx.x % p.Hkv;
  const int b = blockIdx.x / p.Hkv;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int r = lane >> 4;

  __shared__ __align__(16) uint16_t s_k[PF_KEYS * PF_KLD];     // [key][dim]
  __shared__ __align__(16) uint16_t s_vt[D * PF_VLD];          // [dim][key]
  __shared__ __align__(16) uint16_t s_p[4][MF * 16 * PF_PLD];  // per wave [row][key]

  // ---- the wave's query rows as A operands (fragment mi: row c) ----
  u32x4 qa[MF][4];
#pragma unroll
  for (int mi = 0; mi < MF; ++mi) {
    const int jrow = wave * 16 * MF + mi * 16 + c;
    const int t_a = t0 + jrow % BQ;
    const int head_a = h * Q + jrow / BQ;
    const uint16_t* src = p.q + (((size_t)b * p.Hq + head_a) * p.T + min(t_a, p.T - 1)) * D + 8 * r;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qa[mi][ks] = *reinterpret_cast<const u32x4*>(src + ks * 32);
  }
  // the rows this lane holds in MFMA outputs: 4r + i of each fragment
  int qpos[MF][4];
#pragma unroll
  for (int mi = 0; mi < MF; ++mi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = wave * 16 * MF + mi * 16 + 4 * r + i;
      qpos[mi][i] = p.p0 + t0 + j % BQ;        // absolute query position (masks keys beyond it)
    }
  // the smallest query position of the wave's rows (wave-uniform): rows j0 ..
  // j0 + 16 MF - 1 of the tile are prompt rows t0 + j % BQ
  const int j0 = __builtin_amdgcn_readfirstlane(wave) * 16 * MF;
  const int qmin = p.p0 + t0 + ((j0 % BQ) + 16 * MF <= BQ ? j0 % BQ : 0);
  const int last_t = min(t0 + BQ, p.T) - 1;
  const int kend = p.p0 + last_t + 1;        // keys [0, kend) can be attended
  const size_t cache_base = ((size_t)b * p.Hkv + h) * (size_t)p.cap * D;

  float m[MF][4], l[MF][4];
  f32x4 o[MF][8];
#pragma unroll
  for (int mi = 0; mi < MF; ++mi) {
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[mi][i] = -INFINITY; l[mi][i] = 0.0f; }
#pragma unroll
    for (int n = 0; n < 8; ++n) o[mi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // K / V block staging: 64 keys x 128 dims each = 1024 chunks of 16 bytes; 4 per thread.
  // K chunk q: key q / 16, dims 8 (q % 16) (a wave stores 4 whole rows, 16 bytes a
  // lane).  V chunk q: key q % 64, dims 8 (q / 64): the transposed store then
  // writes 64 consecutive keys of one dim per instruction (conflict-free), where
  // the K mapping would put the 16 lanes of a key row 8 rows of s_vt apart, all in
  // one bank.  Loads are unconditional (keys past kend reload key kend - 1), and
  // those keys are zeroed when the block is staged, not right after the load: a
  // select there would make the compiler wait for the load at once, leaving
  // nothing in flight behind the compute.
  auto load_block = [&](int kb, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q16 = tid + 256 * u;
      const int kkey = kb * PF_KEYS + (q16 >> 4);
      const int vkey = kb * PF_KEYS + (q16 & 63);
      kr[u] = *reinterpret_cast<const u32x4*>(p.kc + cache_base + (size_t)min(kkey, kend - 1) * D + 8 * (q16 & 15));
      vr[u] = *reinterpret_cast<const u32x4*>(p.vc + cache_base + (size_t)min(vkey, kend - 1) * D + 8 * (q16 >> 6));
    }
  };
  auto store_block = [&](int kb, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      asm volatile("" : "+v"(kr[u]), "+v"(vr[u]));   // the loads are waited for here, not earlier
      const int q16 = tid + 256 * u;
      const int kkey = kb * PF_KEYS + (q16 >> 4);
      const int key = q16 & 63, d0 = 8 * (q16 >> 6);
      const u32x4 zero4 = u32x4{0u, 0u, 0u, 0u};
      const u32x4 kv = kkey < kend ? kr[u] : zero4;
      const u32x4 vv = kb * PF_KEYS + key < kend ? vr[u] : zero4;
      *reinterpret_cast<u32x4*>(s_k + (q16 >> 4) * PF_KLD + 8 * (q16 & 15)) = kv;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_vt[(d0 + 2 * e) * PF_VLD + key] = (uint16_t)(w[e] & 0xFFFFu);
        s_vt[(d0 + 2 * e + 1) * PF_VLD + key] = (uint16_t)(w[e] >> 16);
      }
    }
  };

  const int nblocks = (kend + PF_KEYS - 1) / PF_KEYS;
  uint16_t* pt = s_p[wave];
  // Block kb: stage its K / V (loaded two blocks earlier) in LDS, refill the
  // register set with block kb + 2, then compute.  Two sets in flight hide the
  // load latency behind two blocks of compute.  Every load is issued, also past
  // the last block (clamped: all lanes read key kend - 1), so that the compiler
  // knows that the other set's loads are in flight behind this set's and waits
  // for this set only; with the loads under a condition it waits for all.
  auto step = [&](const int kb, u32x4 (&kr)[4], u32x4 (&vr)[4]) {
    __syncthreads();                          // the previous block's tiles are consumed
    store_block(kb, kr, vr);
    __syncthreads();
    load_block(kb + 2, kr, vr);
    // ---- S = Q K^T for 4 key tiles of 16; each K fragment feeds every row fragment ----
    f32x4 s[MF][4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int mi = 0; mi < MF; ++mi) s[mi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 kb16 = *reinterpret_cast<const u32x4*>(s_k + (n * 16 + c) * PF_KLD + ks * 32 + 8 * r);
#pragma unroll
        for (int mi = 0; mi < MF; ++mi)
          s[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qa[mi][ks]),
                                                             __builtin_bit_cast(bf16x8, kb16), s[mi][n], 0, 0, 0);
      }
    }
    // ---- online softmax (log2 domain), causal mask; P into the wave's LDS tile ----
    // Blocks that every row of the wave sees whole skip the mask and its guards.
    auto softmax = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
      for (int mi = 0; mi < MF; ++mi) {
        float pv[4][4];   // [i][n]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float mx = -INFINITY;
#pragma unroll
          for (int n = 0; n < 4; ++n) {
            const int key = kb * PF_KEYS + n * 16 + c;
            const float v = (!MASK || key <= qpos[mi][i]) ? s[mi][n][i] * p.scale_log2 : -INFINITY;
            pv[i][n] = v;
            mx = fmaxf(mx, v);
          }
          mx = row_max16(mx);
          const float mn = fmaxf(m[mi][i], mx);
          const float f = m[mi][i] > -INFINITY ? __builtin_amdgcn_exp2f(m[mi][i] - mn) : 0.0f;
          float sum = 0.0f;
#pragma unroll
          for (int n = 0; n < 4; ++n) {
            const float x = round_bf16(__builtin_amdgcn_exp2f(pv[i][n] - mn));
            const float e = (!MASK || pv[i][n] > -INFINITY) ? x : 0.0f;
            pv[i][n] = e;
            sum += e;
          }
          sum = row_sum16(sum);
          l[mi][i] = l[mi][i] * f + sum;
          m[mi][i] = mn;
#pragma unroll
          for (int n = 0; n < 8; ++n) o[mi][n][i] *= f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int n = 0; n < 4; ++n)
            pt[(mi * 16 + 4 * r + i) * PF_PLD + n * 16 + c] = (uint16_t)f32_to_bf16(pv[i][n]);
      }
    };
    if (kb * PF_KEYS + PF_KEYS - 1 <= qmin) softmax(std::false_type{});
    else softmax(std::true_type{});
    __builtin_amdgcn_s_waitcnt(0xc07f);       // lgkmcnt(0): the wave's P writes are done
    __builtin_amdgcn_wave_barrier();
    // ---- O += P V: 2 k-steps of 32 keys, 8 dim tiles; each V fragment feeds every row fragment ----
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 pa[MF];
#pragma unroll
      for (int mi = 0; mi < MF; ++mi)
        pa[mi] = *reinterpret_cast<const u32x4*>(pt + (mi * 16 + c) * PF_PLD + ks * 32 + 8 * r);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const u32x4 vb = *reinterpret_cast<const u32x4*>(s_vt + (n * 16 + c) * PF_VLD + ks * 32 + 8 * r);
#pragma unroll
        for (int mi = 0; mi < MF; ++mi)
          o[mi][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, pa[mi]),
                                                             __builtin_bit_cast(bf16x8, vb), o[mi][n], 0, 0, 0);
      }
    }
  };
  u32x4 kr0[4], vr0[4], kr1[4], vr1[4];
  load_block(0, kr0, vr0);
  load_block(1, kr1, vr1);
  int kb = 0;
  for (; kb + 1 < nblocks; kb += 2) {
    step(kb, kr0, vr0);
    step(kb + 1, kr1, vr1);
  }
  if (kb < nblocks) step(kb, kr0, vr0);

  // ---- normalise and store: lane holds rows 4r + i, dims n * 16 + c ----
#pragma unroll
  for (int mi = 0; mi < MF; ++mi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = wave * 16 * MF + mi * 16 + 4 * r + i;
      const int t = t0 + j % BQ;
      if (t >= p.T) continue;
      const int head = h * Q + j / BQ;
      uint16_t* dst = p.out + ((size_t)b * p.T + t) * p.Hq * D + (size_t)head * D;
      const float inv = l[mi][i] > 0.0f ? 1.0f / l[mi][i] : 0.0f;
      float hs = 0.0f;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const uint32_t v = f32_to_bf16(o[mi][n][i] * inv);
        dst[n * 16 + c] = (uint16_t)v;
        hs += __uint_as_float(v << 16);
      }
      if (p.out_sums) {
        // the head's 128 values are one quantisation group of the next product's k
        hs = row_sum16(hs);
        if (c == 0) p.out_sums[((size_t)b * p.T + t) * p.Hq + head] = hs;
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
