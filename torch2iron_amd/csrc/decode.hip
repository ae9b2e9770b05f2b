// Decode-layer kernels around the W4A16 linears, for gfx950:
//   * weighted RMSNorm (optionally gathering rows from the embedding table);
//   * GQA decode attention with q/k RMSNorm, RoPE and the KV-cache write of the
//     current token folded into its prologue (split over the context; the last
//     chunk of each sequence and kv head to finish merges the chunks);
//   * the tied bf16 lm_head on MFMA with a fused greedy argmax;
//   * device-side greedy / prompt bookkeeping so a decode step can be replayed
//     from a captured graph without host work.
//
// Elementwise rounding follows the reference runtime in bf16 compute
// (quantized_qwen3/model.py:172-196, 215-216, 322-327): every product and sum
// that the reference rounds to bf16 is rounded here at the same point.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "t2i_common.h"

namespace t2i {

// ============================================================================
// RMSNorm
// ============================================================================
constexpr int NORM_THREADS = 256;
constexpr int NORM_MAX_CHUNKS = 4;   // 16-byte chunks per thread: H <= 8192

// One workgroup of T threads a row; thread t holds the 16-byte chunks t, t + T, ...
// (at most MC).  The sum of squares: each thread's chunks in order, a wave sum,
// then the waves' sums in wave order.  Rows of at most 128 chunks run with T = 128
// (one chunk a thread), wider rows with T = 256: the same chunk per thread and so
// the same sums as 256 threads with half of them idle (128 threads: 10.2 -> 7.6 us
// for 8192 rows of 1024).
// gsum (may be NULL): fp32 sums of each output row's bf16 values over each
// 128-wide group, group-major [H / 128][rows] (H a multiple of 128): sixteen
// lanes hold one group, each sums its 8 values in order, then a 16-lane DPP sum.
template <int T, int MC>
__global__ __launch_bounds__(T) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ tokens, int V, int H,
    const uint16_t* __restrict__ w, float eps, uint16_t* __restrict__ x_out,
    uint16_t* __restrict__ y, unsigned long long* __restrict__ keys, float* __restrict__ gsum) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  int src_row = row;
  bool zero_row = false;
  if (tokens) {
    src_row = tokens[row];
    if (src_row < 0 || src_row >= V) { src_row = 0; zero_row = true; }   // out-of-range id: zero row
  }
  const uint16_t* src = x + (size_t)src_row * H;
  const int chunks = H / 8;
  u32x4 v[MC];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < MC; ++i) {
    const int ch = tid + i * T;
    if (ch < chunks) {
      v[i] = zero_row ? u32x4{0u, 0u, 0u, 0u} : *reinterpret_cast<const u32x4*>(src + ch * 8);
      const uint32_t a[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_lo(a[j]), hi = bf16_hi(a[j]);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
      }
    }
  }
  __shared__ float part[T / 64];
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < T / 64; ++i) total += part[i];
  const float inv = round_bf16(1.0f / sqrtf(total / (float)H + eps));
#pragma unroll
  for (int i = 0; i < MC; ++i) {
    const int ch = tid + i * T;
    if (ch < chunks) {
      const u32x4 g = *reinterpret_cast<const u32x4*>(w + ch * 8);
      const uint32_t a[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      const uint32_t b[4] = {g.x, g.y, g.z, g.w};
      uint32_t o[4];
      float gs = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = round_bf16(round_bf16(bf16_lo(a[j]) * inv) * bf16_lo(b[j]));
        const float hi = round_bf16(round_bf16(bf16_hi(a[j]) * inv) * bf16_hi(b[j]));
        o[j] = pack_bf16x2(lo, hi);
        gs += lo;
        gs += hi;
      }
      *reinterpret_cast<u32x4*>(y + (size_t)row * H + ch * 8) = u32x4{o[0], o[1], o[2], o[3]};
      if (x_out) *reinterpret_cast<u32x4*>(x_out + (size_t)row * H + ch * 8) = v[i];
      if (gsum) {
        gs = row_sum16(gs);
        if ((ch & 15) == 0) gsum[(size_t)(ch >> 4) * gridDim.x + row] = gs;
      }
    }
  }
  if (keys && tid == 0) keys[row] = 0ull;
}

// ============================================================================
// GQA decode attention
// ============================================================================
constexpr int ATT_THREADS = 256;

// Context slots per lane: a workgroup covers 16 * rows slots (16 groups of 16
// lanes, one slot per group and pass).  Fewer rows for more q heads per kv
// head keeps the per-lane score and accumulator registers bounded.
constexpr int att_rows(int q) { return q <= 2 ? 8 : (q == 4 ? 4 : 2); }

// Chunk-state scratch of t2i_decode_attention_noalloc: one copy per device,
// zero-initialised at load (16 MiB).  Host code never passes this name to a
// kernel; it takes the copy's device address from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[(size_t)16 << 20] = {};

struct AttnParams {
  const uint16_t* qkv;
  const int32_t* pos;
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* rope;
  uint16_t* kc;
  uint16_t* vc;
  uint16_t* out;
  float* part_o;        // [B*Hkv][S][Q][D]  unnormalised context of each split
  float* part_ml;       // [B*Hkv][S][Q][2]  (max score, sum of exponentials) of each split
  unsigned* arrivals;   // [B*Hkv]           splits finished; zero between launches
  int Hq, Hkv, ctx_cap, splits, style;
  int chunk;            // context slots per split (at most 16 * ROWS)
  float eps, scale;
};


// One workgroup per (sequence b, kv head h, chunk of 16 * ROWS context slots).
// A single workgroup per (b, h) streaming the whole context was measured 2-4x
// slower at every decode shape: one CU keeps about 64 KB of loads in flight,
// which at HBM latency is some 30 GB/s, so the context must be spread over
// enough workgroups to occupy every CU, and the chunks' states merged.
//   1. prologue inputs: the raw q/k/v rows of this kv head and the norm gammas are
//      loaded alongside the position, the RoPE row and then the chunk's K and V rows
//      once it is known: loads retire in issue order, so the q/k RMSNorm + RoPE below
//      waits only for its own inputs while K/V are in flight;
//   2. every 16-lane group scores its slots (8 dims per lane, a dot2 chain and a
//      16-lane DPP sum); each wave keeps one softmax state (max, sum over its four
//      groups) and forms its unnormalised context on the MFMA from the fp32
//      weights (as three bf16 parts) and the V rows as they lie in registers; the
//      waves' states meet in LDS, in a fixed order;
//   3. with several chunks per (b, h), each chunk stores its state agent-coherently and
//      the last chunk to arrive merges all of them in chunk order (deterministic) and
//      writes the bf16 context; it also resets the arrival counter for the next launch.
// Everything the loads issued before the position need (pos, the qkv rows, the
// caches, the norm weights and the shape) leads the argument list as scalars,
// which the library is built to preload into SGPRs at wave launch (14 SGPRs:
// six pointers and two packed words); the rest come from p_, whose loads then
// run alongside the position's.
//   heads_     = Hq | Hkv << 15 | rope_style << 30
//   cap_chunk_ = ctx_cap | chunk << 23   (chunk <= 256)
//   PREP = false (t2i_decode_attention_prepared): q, k and v come normalised and
//   rotated already, as three row arrays: qkv_ = q [B, Hq*D], qn_ = k [B, Hkv*D],
//   kn_ = v [B, Hkv*D]; no norm weights and no RoPE table are read.
template <int Q, int ROWS, bool PREP = true>
__global__ __launch_bounds__(ATT_THREADS) void decode_attention_kernel(const int32_t* pos_, const uint16_t* qkv_,
                                                                       uint16_t* kc_, uint16_t* vc_,
                                                                       const uint16_t* qn_, const uint16_t* kn_,
                                                                       int heads_, int cap_chunk_, const AttnParams p_) {
  AttnParams p = p_;
  p.pos = pos_; p.qkv = qkv_; p.kc = kc_; p.vc = vc_; p.qn = qn_; p.kn = kn_;
  p.Hq = heads_ & 0x7FFF; p.Hkv = (heads_ >> 15) & 0x7FFF; p.style = heads_ >> 30;
  p.ctx_cap = cap_chunk_ & 0x7FFFFF; p.chunk = (int)((unsigned)cap_chunk_ >> 23);
  constexpr int D = ATT_D;
  constexpr int NV = (Q + 2 + 3) / 4;   // prologue vectors (q heads, k, v) per wave
  const int bh = blockIdx.x;
  const int b = bh / p.Hkv;
  const int h = bh - b * p.Hkv;
  const int split = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;              // dims 8c .. 8c+7 of a slot
  const int rg = lane >> 4;
  const int grp = wave * 4 + rg;        // slot group 0..15

  __shared__ __align__(16) uint16_t s_q[Q][D];    // q heads after norm + RoPE (bf16)
  __shared__ __align__(16) uint16_t s_kv[2][D];   // current k (after norm + RoPE) and v
  __shared__ float s_wm[4][Q], s_wl[4][Q];
  __shared__ __align__(16) float s_wacc[4][Q][D];
  __shared__ int s_last;

  // ---- 1. loads that do not need the position go out with it ----
  // The raw q/k/v rows of this kv head and the norm weights are loaded while
  // the position is (a scalar load, waited for on its own counter), and so are
  // the chunk's first two passes of K / V rows (below).  The RoPE row through
  // scalar loads, so that its wait does not cover the K / V rows, measured
  // slower (10.5 -> 11.0 us a call, 0.848 -> 0.864 ms a step).  Every load is
  // unconditional (clamped indices, results selected after the load): a load
  // under a lane-divergent condition whose other side writes the same registers
  // makes the compiler wait for all loads in flight there.
  const int pos_raw = p.pos[b];
  const size_t qkv_row = (size_t)b * (p.Hq + 2 * p.Hkv) * D;
  const size_t cache_base = ((size_t)b * p.Hkv + h) * (size_t)p.ctx_cap * D;
  const int t0 = split * p.chunk;
  const int i0 = p.style == 0 ? lane : 2 * lane;        // pair (i0, i1) rotates together
  const int i1 = p.style == 0 ? lane + D / 2 : 2 * lane + 1;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  float px0[NV], px1[NV], pg0[NV], pg1[NV];
#pragma unroll
  for (int n = 0; n < NV; ++n) {
    const int vi = min(wv + 4 * n, Q + 1);   // waves past the last vector reload it; unused
    const uint16_t* src;
    if constexpr (PREP) {
      const int hrow = vi < Q ? h * Q + vi : (vi == Q ? p.Hq + h : p.Hq + p.Hkv + h);
      src = p.qkv + qkv_row + (size_t)hrow * D;
    } else {
      src = vi < Q ? p.qkv + ((size_t)b * p.Hq + h * Q + vi) * D
                   : (vi == Q ? p.qn : p.kn) + ((size_t)b * p.Hkv + h) * D;
    }
    px0[n] = bf16_to_f32(src[i0]);
    px1[n] = bf16_to_f32(src[i1]);
    if constexpr (PREP) {
      const uint16_t* gamma = vi < Q ? p.qn : p.kn;   // v takes no gamma; loaded, unused
      pg0[n] = bf16_to_f32(gamma[i0]);
      pg1[n] = bf16_to_f32(gamma[i1]);
    } else {
      pg0[n] = pg1[n] = 1.0f;
    }
  }
  // The chunk's first two passes of K / V rows (slots t0 + grp and t0 + 16 + grp,
  // clamped into the cache) go out before the position is known: every chunk that
  // holds a valid slot starts at a valid slot, so they are wasted only for chunks
  // wholly past the position (32 slots each).  Measured at batch 16, 577 of 640
  // slots, HBM-cold: 11.50 -> 11.08 us a call (one pass: 11.30; three: 11.31; four:
  // 11.48; all eight, reading past the chunk's end: 12.44), decode step 0.829 ->
  // 0.813 ms.  Scoring masks every slot at or past the chunk's end, and the current
  // slot's row is patched from LDS below, so these rows are used as loaded.
  u32x4 kreg[ROWS], vreg[ROWS];
  constexpr int SPEC = ROWS < 2 ? ROWS : 2;
#pragma unroll
  for (int it = 0; it < SPEC; ++it) {
    const int ts = min(t0 + it * 16 + grp, p.ctx_cap - 1);
    kreg[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.kc + cache_base + (size_t)ts * D + 8 * c));
    vreg[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.vc + cache_base + (size_t)ts * D + 8 * c));
  }
  __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of everything that needs pos

  // a position outside the cache attends to nothing and writes nothing (zero output)
  const bool valid = pos_raw >= 0 && pos_raw < p.ctx_cap;
  const int pos = valid ? pos_raw : 0;
  const int L = valid ? pos + 1 : 0;
  const int t1 = min(t0 + p.chunk, L);
  const size_t part = (size_t)bh * p.splits + split;

  if (t0 < t1) {
    // ---- the RoPE row, then the chunk's K / V rows ----
    const float cs = PREP ? bf16_to_f32(p.rope[(size_t)pos * D + 2 * lane]) : 1.0f;
    const float sn = PREP ? bf16_to_f32(p.rope[(size_t)pos * D + 2 * lane + 1]) : 0.0f;
    __builtin_amdgcn_sched_barrier(0);   // the RoPE row ahead of the K / V rows
    // the remaining passes: slots past the chunk's end reload its first slot; masked
    // when scored.  The K/V stream is read once per step: non-temporal loads
    // (measured 12.8 -> 12.1 us per call at batch 16, context 577, decode step 889 ->
    // 870 us with the lm_head's)
#pragma unroll
    for (int it = SPEC; it < ROWS; ++it) {
      const int t = t0 + it * 16 + grp;
      const int tl = t < t1 ? t : t0;
      kreg[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.kc + cache_base + (size_t)tl * D + 8 * c));
      vreg[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.vc + cache_base + (size_t)tl * D + 8 * c));
    }

    // ---- q heads and the current k: per-head RMSNorm then RoPE; v as is ----
    // computed by every wave and selected (no branch that the loads above could
    // be moved into, behind the K / V loads)
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int vi = wv + 4 * n;
      float x0 = px0[n], x1 = px1[n];
      if constexpr (PREP) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = round_bf16(1.0f / sqrtf(ss / (float)D + p.eps));
        const float n0 = round_bf16(round_bf16(x0 * inv) * pg0[n]);
        const float n1 = round_bf16(round_bf16(x1 * inv) * pg1[n]);
        const float y0 = round_bf16(round_bf16(n0 * cs) + round_bf16(-n1 * sn));
        const float y1 = round_bf16(round_bf16(n1 * cs) + round_bf16(n0 * sn));
        x0 = vi <= Q ? y0 : x0;
        x1 = vi <= Q ? y1 : x1;
      }
      if (vi >= Q + 2) continue;
      if (vi < Q) {
        s_q[vi][i0] = (uint16_t)f32_to_bf16(x0);
        s_q[vi][i1] = (uint16_t)f32_to_bf16(x1);
      } else {
        const int which = vi - Q;   // 0 = k, 1 = v
        const uint16_t b0 = (uint16_t)f32_to_bf16(x0), b1 = (uint16_t)f32_to_bf16(x1);
        s_kv[which][i0] = b0;
        s_kv[which][i1] = b1;
        if (pos < t1) {   // this workgroup owns the current slot: persist it
          uint16_t* dst = (which == 0 ? p.kc : p.vc) + cache_base + (size_t)pos * D;
          dst[i0] = b0;
          dst[i1] = b1;
        }
      }
    }
    __syncthreads();

    // ---- 2. scores on the VALU, the wave's softmax state, the context on the MFMA ----
    // The chunk that owns the current slot loaded its cache rows before writing
    // them: the lanes that hold that slot take k and v from LDS instead (a
    // divergent patch in one wave; the other lanes never hold it).
    if (t0 <= pos && pos < t1) {   // workgroup-uniform
      const int rel = pos - t0;
      if (grp == (rel & 15)) {
        const u32x4 kcur = reinterpret_cast<const u32x4*>(&s_kv[0][0])[c];
        const u32x4 vcur = reinterpret_cast<const u32x4*>(&s_kv[1][0])[c];
        const int itp = rel >> 4;
#pragma unroll
        for (int it = 0; it < ROWS; ++it) {
          if (it == itp) {
            kreg[it] = kcur;
            vreg[it] = vcur;
          }
        }
      }
    }
    u32x4 qv[Q];   // dims 8c .. 8c+7 of each q head, bf16 pairs
#pragma unroll
    for (int j = 0; j < Q; ++j) qv[j] = reinterpret_cast<const u32x4*>(&s_q[j][0])[c];
    const float sl2 = p.scale * 1.4426950408889634f;   // log2 units
    // every lane of a 16-lane group ends with its slot's full score (row_sum16)
    float sc[ROWS][Q];
#pragma unroll
    for (int it = 0; it < ROWS; ++it) {
      const int t = t0 + it * 16 + grp;
      const u32x4 kk = kreg[it];
#pragma unroll
      for (int j = 0; j < Q; ++j) {
        float d = dot2_bf16(qv[j].x, kk.x, 0.0f);   // bf16 products are exact in fp32
        d = dot2_bf16(qv[j].y, kk.y, d);
        d = dot2_bf16(qv[j].z, kk.z, d);
        d = dot2_bf16(qv[j].w, kk.w, d);
        d = row_sum16(d);
        sc[it][j] = t < t1 ? d * sl2 : -INFINITY;   // a slot past the chunk's end weighs nothing
      }
    }
    // one softmax state per wave: the max and the sum over its four groups' slots
    float m[Q], mz[Q], l[Q];
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      m[j] = sc[0][j];
#pragma unroll
      for (int it = 1; it < ROWS; ++it) m[j] = fmaxf(m[j], sc[it][j]);
      m[j] = fmaxf(m[j], __shfl_xor(m[j], 16, 64));
      m[j] = fmaxf(m[j], __shfl_xor(m[j], 32, 64));
      mz[j] = m[j] > -INFINITY ? m[j] : 0.0f;   // a wave with no slot: 2^-inf = 0 below
      l[j] = 0.0f;
    }
    float pe[ROWS][Q];
#pragma unroll
    for (int it = 0; it < ROWS; ++it)
#pragma unroll
      for (int j = 0; j < Q; ++j) {
        pe[it][j] = exp2_fast(sc[it][j] - mz[j]);
        l[j] += pe[it][j];
      }
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      l[j] += __shfl_xor(l[j], 16, 64);
      l[j] += __shfl_xor(l[j], 32, 64);
    }
    // Context O[h][d] = sum over the wave's slots of P[h][slot] V[slot][d] on
    // v_mfma_f32_16x16x32_bf16: the 32 k values are the 8 rows (it) of each of the
    // four groups, which is how the slots already lie (lane (c, rg) holds rows it
    // of slot group rg).  A = P: lane (c, rg) row h = c (zero past Q), k = its rows,
    // as three bf16 parts, p = p0 + p1 + p2 (p0 = bf16(p), p1 = bf16(p - p0),
    // p2 = p - p0 - p1, each difference exact in fp32), which carry all 24 bits of
    // the fp32 weight: products with bf16 V are exact and the MFMA sums in fp32.
    // (With bf16 weights, or two parts, more outputs miss the correctly rounded
    // bf16 value and greedy decode drifts at near-ties.)  B = V for dim 8 c + e: lane
    // (c, rg) column c, k = its rows, one byte permute per pair of rows.  So lane
    // (c, r) ends with O[4 r + i][8 c + e] in acc[e][i], and the MFMA has summed the
    // four groups.
    constexpr int NB = (ROWS + 7) / 8;   // k-blocks of 8 rows
    f32x4 acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float pw[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int it = 8 * b + u;
        float v = 0.0f;
        if (it < ROWS) {
          v = pe[it][0];
#pragma unroll
          for (int j = 1; j < Q; ++j) v = c == j ? pe[it][j] : v;
          v = c < Q ? v : 0.0f;
        }
        pw[u] = v;
      }
      float p1[8], p2[8];   // what bf16 leaves of each weight, in two parts
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        p1[u] = pw[u] - round_bf16(pw[u]);
        p2[u] = p1[u] - round_bf16(p1[u]);
      }
      const bf16x8 a[3] = {
          __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(pw[0], pw[1]), pack_bf16x2(pw[2], pw[3]),
                                           pack_bf16x2(pw[4], pw[5]), pack_bf16x2(pw[6], pw[7])}),
          __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(p1[0], p1[1]), pack_bf16x2(p1[2], p1[3]),
                                           pack_bf16x2(p1[4], p1[5]), pack_bf16x2(p1[6], p1[7])}),
          __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(p2[0], p2[1]), pack_bf16x2(p2[2], p2[3]),
                                           pack_bf16x2(p2[4], p2[5]), pack_bf16x2(p2[6], p2[7])})};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t wv[8];   // bf16 bits of dim 8 c + e, rows 8 b .. 8 b + 7
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int it = 8 * b + u;
          const uint32_t w = it < ROWS ? (e < 2 ? vreg[it].x : e < 4 ? vreg[it].y : e < 6 ? vreg[it].z : vreg[it].w) : 0u;
          wv[u] = w;
        }
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;   // high or low halves of the pair
        const u32x4 vb = u32x4{__builtin_amdgcn_perm(wv[1], wv[0], sel), __builtin_amdgcn_perm(wv[3], wv[2], sel),
                               __builtin_amdgcn_perm(wv[5], wv[4], sel), __builtin_amdgcn_perm(wv[7], wv[6], sel)};
        // smallest part first, so each sum adds the larger terms last
#pragma unroll
        for (int k = 2; k >= 0; --k)
          acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[k], __builtin_bit_cast(bf16x8, vb), acc[e], 0, 0, 0);
      }
    }
    // the wave's state: heads 4 r + i < Q of this lane, dims 8 c .. 8 c + 7
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * rg + i;
      if (h < Q) {
        float* dst = &s_wacc[wave][h][8 * c];
        *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]};
      }
    }
    if (lane < Q) {
      float mw = m[0], lw = l[0];
#pragma unroll
      for (int j = 1; j < Q; ++j) {
        mw = lane == j ? m[j] : mw;
        lw = lane == j ? l[j] : lw;
      }
      s_wm[wave][lane] = mw;
      s_wl[wave][lane] = lw;
    }
    __syncthreads();

    // ---- merge the four waves; one chunk: write the context, else store the state ----
    for (int idx = tid; idx < Q * D; idx += ATT_THREADS) {
      const int j = idx / D, d = idx - j * D;
      float M = s_wm[0][j];
#pragma unroll
      for (int w = 1; w < 4; ++w) M = fmaxf(M, s_wm[w][j]);
      float lsum = 0.0f, o = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = state_weight(s_wm[w][j], M);
        lsum = fmaf(s_wl[w][j], f, lsum);
        o = fmaf(s_wacc[w][j][d], f, o);
      }
      if (p.splits == 1) {
        p.out[(size_t)b * p.Hq * D + (size_t)(h * Q + j) * D + d] = (uint16_t)f32_to_bf16(o / lsum);
      } else {
        st_agent(p.part_o + (part * Q + j) * D + d, o);
        if (d == 0) {
          st_agent(p.part_ml + (part * Q + j) * 2, M);
          st_agent(p.part_ml + (part * Q + j) * 2 + 1, lsum);
        }
      }
    }
  } else if (p.splits > 1) {
    if (tid < Q) {   // an empty chunk: a state that weighs nothing
      st_agent(p.part_ml + (part * Q + tid) * 2, -INFINITY);
      st_agent(p.part_ml + (part * Q + tid) * 2 + 1, 0.0f);
    }
  } else {
    for (int idx = tid; idx < Q * D; idx += ATT_THREADS)
      p.out[(size_t)b * p.Hq * D + (size_t)h * Q * D + idx] = 0;
  }
  if (p.splits == 1) return;

  // ---- 3. the last chunk of (b, h) to arrive merges every chunk's state, in chunk order ----
  // Hand-off between workgroups on different XCDs (each XCD has its own L2), at the
  // level of the gfx950 memory system rather than through release/acquire fences:
  //   producer: the state stores are agent-scope atomic stores (global_store sc1:
  //             written through to the device-coherent level); every wave waits
  //             for its stores to complete (s_waitcnt vmcnt(0)), the workgroup
  //             barrier orders that before thread 0's agent-scope fetch_add;
  //   consumer: the merger's loads are agent-scope atomic loads (global_load sc1:
  //             no stale L2 copy), issued only after thread 0's fetch_add has
  //             returned the count that makes it last (its value goes through LDS
  //             and a barrier); the compiler-only fence keeps them there.
  // A release fetch_add and an acquire fence give the same order through the
  // memory model, but their L2 write-back and invalidate (buffer_wbl2 / buffer_inv
  // at agent scope) cost 12.5 us and 3.1 us per call at batch 16, context 577
  // (25.2 and 15.8 us against 12.7 us), measured.  Counting the arrival without
  // waiting for the stores, with the states as flagged 64-bit words that the
  // merger polls, measured slower too (13.4 against 11.8 us per call: the merger
  // then meets the last chunk's words still in flight and polls again), and so did
  // merging in a second kernel after this one, with the launch boundary as the
  // hand-off (0.897 against 0.874 ms per decode step at batch 16).
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const unsigned before = __hip_atomic_fetch_add(p.arrivals + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = before == (unsigned)(p.splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // The merger's state addresses are computed from the arrival count's outcome
  // (dep is 1 here, through an asm the compiler cannot see into), so neither the
  // compiler nor the hardware can issue a state load before thread 0's fetch_add
  // has returned and the barrier has passed its result on: the order holds by data
  // dependence, whatever a compiler does with relaxed loads and fences.
  int dep = s_last;
  asm volatile("" : "+v"(dep));
  const float* part_ml = p.part_ml + (dep - 1);
  const float* part_o = p.part_o + (dep - 1);
  for (int idx = tid; idx < Q * D; idx += ATT_THREADS) {
    const int j = idx / D, d = idx - j * D;
    float M = -INFINITY, lsum = 0.0f, o = 0.0f;
    // chunk states in groups of 8: the loads of a group are issued back to back
    for (int s0 = 0; s0 < p.splits; s0 += 8) {
      float ms[8], ls[8], os[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {   // unconditional loads (clamped), as above
        const size_t st = (size_t)bh * p.splits + min(s0 + u, p.splits - 1);
        ms[u] = ld_agent(part_ml + (st * Q + j) * 2);
        ls[u] = ld_agent(part_ml + (st * Q + j) * 2 + 1);
        os[u] = ld_agent(part_o + (st * Q + j) * D + d);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (ls[u] > 0.0f && s0 + u < p.splits) {   // an empty chunk stored no context
          const float mn = fmaxf(M, ms[u]);
          const float fa = state_weight(M, mn), fb = exp2_fast(ms[u] - mn);
          lsum = lsum * fa + ls[u] * fb;
          o = o * fa + os[u] * fb;
          M = mn;
        }
      }
    }
    p.out[(size_t)b * p.Hq * D + (size_t)(h * Q + j) * D + d] =
        lsum > 0.0f ? (uint16_t)f32_to_bf16(o / lsum) : (uint16_t)0;
  }
  if (tid == 0) __hip_atomic_store(p.arrivals + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================================
// lm_head (bf16 tied embedding) + greedy argmax
// ============================================================================
// 4 waves of up to 5 16-row tiles of the vocabulary each.  The workgroup count
// is a multiple of 256 (one equal share per CU; Qwen3's 9496 tiles: 512
// workgroups of 18 or 19 tiles, two a CU; a wave's 64-deep slice of its tiles
// is 10 KB, two slices in flight), each workgroup taking a contiguous range.  Measured at batch 16,
// HBM-cold, final norm fused (us a call, same box): 2 tiles a wave (1280
// workgroups, a fifth one on each CU) 56.8; 3 tiles 55.2; 4 tiles 54.3; 5 tiles
// 52.5; 6 tiles 53.0; 8 tiles 65.9; 8 waves of 2 tiles 58.3.  Earlier forms:
// grids whose workgroups are all resident from the start with tiles dealt to the
// waves in a stride were slower (67-69 against 61 us), and loads of 64
// contiguous bytes of each row no faster than 16-byte pieces.
constexpr int LMH_WAVES = 4;
constexpr int LMH_COLS = 80;                // vocab columns per wave
constexpr int LMH_TILES = LMH_COLS / 16;    // MFMA n-tiles per wave
constexpr int LMH_MAX_K = 4096;   // 16 x K bf16 of LDS (plus 8 KB of regions)

__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// One workgroup: LMH_WAVES waves x LMH_COLS vocab rows; the activation rows
// (M <= 16) are staged once in LDS and shared by the waves.
//   * The table is read as 8 rows x 128 bytes per load instruction (lane l: row
//     8 h + l / 8 of the tile, 16 bytes at k-block l % 8 of the 64-deep slice):
//     whole 128-byte lines.  The MFMA operand (lane (c, r): row c, 8 k) would take
//     16 rows x 16 bytes per instruction, 64-byte pieces of each row per
//     instruction pair; a read-only probe of the two patterns streamed the table at
//     7.2 against 5.7 TB/s.  Each tile's slice goes through the wave's 2 KB LDS
//     region into the operand layout: 16-byte units k-block major, the row
//     XOR-swizzled by the k-block, so that the stores of a load and the reads of an
//     MFMA operand each meet 16 distinct bank groups per 16 lanes.
//   * The activation rows sit unpadded, 16-byte unit u of row m at u ^ (m & 15)
//     (m & 7 when K is not a multiple of 128): conflict-free operand reads, and
//     32 KB plus the 8 KB of regions at K = 1024 (room for four workgroups a CU).
//   * The MFMA pairs k-block r of the slice's first half with the activation's
//     k-block r and the second half likewise (lane (c, r) takes k 8 r and 32 + 8 r).
__device__ __forceinline__ int lmh_unit(int row, int kb) { return 16 * kb + (row ^ ((2 * kb) & 15)); }

//   * NORM: hin holds the un-normalised rows and the workgroup applies the final
//     RMSNorm (gamma, eps) to its staged copy before the first product, in
//     rmsnorm_kernel's order (thread t sums chunks t, t + 256, ... of each row,
//     then wave_sum and the four wave partials in order; its 128-thread form for
//     rows of at most 128 chunks gives the same sums), so the normalised rows
//     and every logit carry the bits of t2i_rmsnorm followed by t2i_lm_head_argmax.
//     This runs while the first table slice is in flight.  K is a power of two, so
//     each thread's pieces use one or two gamma pieces, loaded with its h.
template <bool NORM>
__global__ __launch_bounds__(64 * LMH_WAVES) void lm_head_kernel(
    const uint16_t* __restrict__ hin, int M, const uint16_t* __restrict__ E, int V, int K,
    float* __restrict__ logits, unsigned long long* __restrict__ keys, const uint16_t* __restrict__ gamma,
    float eps) {
  // this workgroup's tiles [tb, te) of the V / 16 (contiguous, balanced)
  extern __shared__ u32x4 s_dyn[];                  // [16][K / 8] units of h, then the waves' regions
  const int ku = K / 8;                             // 16-byte units per activation row
  const int hmask = (ku & 15) ? 7 : 15;
  u32x4* const s_hu = s_dyn;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int r = lane >> 4;
  u32x4* const region = s_dyn + 16 * ku + wave * 128;
  const int T = V / 16;
  const int tb = (int)((long long)blockIdx.x * T / gridDim.x);
  const int te = (int)((long long)(blockIdx.x + 1) * T / gridDim.x);
  const int tile0 = tb + LMH_TILES * wave;
  const int n0 = tile0 * 16;
  f32x4 acc[LMH_TILES];
#pragma unroll
  for (int t = 0; t < LMH_TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  bool tile_ok[LMH_TILES];
#pragma unroll
  for (int t = 0; t < LMH_TILES; ++t) tile_ok[t] = tile0 + t < te;

  // Double-buffered over 64-deep k slices: the next slice's rows are in flight
  // while the current one is multiplied.  A tile past the workgroup's range
  // reloads the wave's first tile, or the workgroup's, rows that are loaded
  // anyway (an unconditional load; its results are dropped).  The table is read
  // once per step: non-temporal loads.
  const int nfirst = min(n0, (te - 1) * 16);
  auto load_slice = [&](int k0, u32x4 (&bv)[LMH_TILES][2]) {
#pragma unroll
    for (int t = 0; t < LMH_TILES; ++t) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = (tile_ok[t] ? n0 + 16 * t : nfirst) + 8 * h + (lane >> 3);
        bv[t][h] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(E + (size_t)row * K + k0 + 8 * (lane & 7)));
      }
    }
  };
  auto mul_slice = [&](int k0, const u32x4 (&bv)[LMH_TILES][2]) {
    const int u0 = k0 / 8;
    const u32x4* hrow = s_hu + c * ku;
    const bf16x8 a0 = __builtin_bit_cast(bf16x8, hrow[(u0 + r) ^ (c & hmask)]);
    const bf16x8 a1 = __builtin_bit_cast(bf16x8, hrow[(u0 + 4 + r) ^ (c & hmask)]);
#pragma unroll
    for (int t = 0; t < LMH_TILES; ++t) {
      // the wave's region holds one tile's slice at a time (LDS operations of a
      // wave complete in order, so the next tile's stores follow these reads)
      region[lmh_unit(lane >> 3, lane & 7)] = bv[t][0];
      region[lmh_unit(8 + (lane >> 3), lane & 7)] = bv[t][1];
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, region[lmh_unit(c, r)]);
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, region[lmh_unit(c, 4 + r)]);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[t], 0, 0, 0);
    }
  };
  // Stage h (rows >= M are zero) while the first weight slice is in flight: each
  // thread issues its loads of h (8 at a time), then the slice, then stores h to
  // LDS, which waits for the h loads only (loads retire in issue order).  Loads
  // and stores are unconditional (clamped): a load sunk into a branch gets a wait
  // for every load in flight.
  u32x4 b0[LMH_TILES][2], b1[LMH_TILES][2];
  constexpr int NSTEP = 64 * LMH_WAVES;   // threads: the stride of every piece loop below
  u32x4 gv[2];                            // NORM: gamma pieces (tid + j NSTEP) % ku, j = 0, 1
  {
    const int nst = 16 * ku;   // 16-byte pieces of the 16-row tile
    for (int base = 0; base < nst; base += 8 * NSTEP) {
      u32x4 hv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = min(base + u * NSTEP + tid, nst - 1);
        const int m = idx / ku, ch = idx - m * ku;
        hv[u] = *reinterpret_cast<const u32x4*>(hin + (size_t)min(m, M - 1) * K + ch * 8);
      }
      if (base == 0) {
        if constexpr (NORM) {
#pragma unroll
          for (int j = 0; j < 2; ++j) gv[j] = *reinterpret_cast<const u32x4*>(gamma + ((tid + j * NSTEP) & (ku - 1)) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_slice(0, b0);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {   // past the tile: the last piece again (same value)
        const int idx = min(base + u * 64 * LMH_WAVES + tid, nst - 1);
        const int m = idx / ku, ch = idx - m * ku;
        s_hu[m * ku + (ch ^ (m & hmask))] = m < M ? hv[u] : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    // per-row sums of squares in rmsnorm_kernel's order; the partials and the
    // rows' 1 / rms sit in the waves' regions, unused until the first product
    float* const s_part = reinterpret_cast<float*>(s_dyn + 16 * ku);   // [16][LMH_WAVES]
    float* const s_inv = s_part + 16 * LMH_WAVES;                       // [16]
    float ss[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) ss[m] = 0.0f;
    for (int ch = tid; ch < ku; ch += NSTEP) {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const u32x4 v = s_hu[m * ku + (ch ^ (m & hmask))];
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16_lo(a[j]), hi = bf16_hi(a[j]);
          ss[m] = fmaf(lo, lo, ss[m]);
          ss[m] = fmaf(hi, hi, ss[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float w = wave_sum(ss[m]);
      if (lane == 0) s_part[m * LMH_WAVES + wave] = w;
    }
    __syncthreads();
    if (tid < 16) {
      float total = 0.0f;
#pragma unroll
      for (int w = 0; w < LMH_WAVES; ++w) total += s_part[tid * LMH_WAVES + w];
      s_inv[tid] = round_bf16(1.0f / sqrtf(total / (float)K + eps));
    }
    __syncthreads();
    // each thread normalises its pieces tid + j NSTEP (gamma piece j % 2)
    for (int j = 0; j * NSTEP < 16 * ku; ++j) {
      const int idx = tid + j * NSTEP;
      const int m = idx / ku, ch = idx - m * ku;
      if (m < M) {
        u32x4* const dst = &s_hu[m * ku + (ch ^ (m & hmask))];
        const u32x4 v = *dst;
        const u32x4 g = (j & 1) ? gv[1] : gv[0];
        const float inv = s_inv[m];
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
        const uint32_t b[4] = {g.x, g.y, g.z, g.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = round_bf16(round_bf16(bf16_lo(a[q]) * inv) * bf16_lo(b[q]));
          const float hi = round_bf16(round_bf16(bf16_hi(a[q]) * inv) * bf16_hi(b[q]));
          o[q] = pack_bf16x2(lo, hi);
        }
        *dst = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
    __syncthreads();
  }
  // Loads inside the loop are unconditional (a load skipped on one path makes the
  // compiler's wait counts conservative for both); the last one or two slices are
  // peeled.
  // sched_barrier keeps each slice's loads ahead of the previous slice's MFMAs.
  int k0 = 0;
  for (; k0 + 128 < K; k0 += 128) {
    load_slice(k0 + 64, b1);
    __builtin_amdgcn_sched_barrier(0);
    mul_slice(k0, b0);
    __builtin_amdgcn_sched_barrier(0);
    load_slice(k0 + 128, b0);
    __builtin_amdgcn_sched_barrier(0);
    mul_slice(k0 + 64, b1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (k0 + 64 < K) {
    load_slice(k0 + 64, b1);
    __builtin_amdgcn_sched_barrier(0);
    mul_slice(k0, b0);
    mul_slice(k0 + 64, b1);
  } else {
    mul_slice(k0, b0);
  }

  // lane holds logits[m = 4r + i][n = n0 + 16t + c]; each wave's best keys go to
  // the start of its own region (16 words of 8 bytes), read after the barrier
  unsigned long long* s_best = reinterpret_cast<unsigned long long*>(region);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * r + i;
    unsigned long long best = 0ull;
#pragma unroll
    for (int t = 0; t < LMH_TILES; ++t) {
      if (!tile_ok[t]) continue;
      const int n = n0 + 16 * t + c;
      if (logits && m < M) logits[(size_t)m * V + n] = acc[t][i];
      best = umax64(best, argmax_key(acc[t][i], (uint32_t)n));
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const unsigned long long o = __shfl_xor(best, off, 64);
      best = umax64(best, o);
    }
    if (c == 0) s_best[m] = best;
  }
  __syncthreads();
  if (tid < M) {
    const unsigned long long* s0 = reinterpret_cast<const unsigned long long*>(s_dyn + 16 * ku);
    unsigned long long best = s0[tid];
#pragma unroll
    for (int w = 1; w < LMH_WAVES; ++w) best = umax64(best, s0[w * 256 + tid]);   // 128 units = 256 words a region
    if (best) atomicMax(&keys[tid], best);
  }
}

__global__ void greedy_advance_kernel(const unsigned long long* __restrict__ keys, int B, int32_t* tokens,
                                      int32_t* positions, int32_t* history, int hist_cap, int32_t* step) {
  const int s = *step;
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const int32_t tok = (int32_t)(0xFFFFFFFFu - (uint32_t)(keys[b] & 0xFFFFFFFFull));
    tokens[b] = tok;
    if (history && s < hist_cap) history[(size_t)b * hist_cap + s] = tok;
    positions[b] += 1;
  }
  __syncthreads();
  if (threadIdx.x == 0) *step = s + 1;
}

__global__ void prompt_advance_kernel(const int32_t* __restrict__ prompt, int B, int P, int32_t* tokens,
                                      int32_t* positions) {
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const int np = positions[b] + 1;
    positions[b] = np;
    if (np < P) tokens[b] = prompt[(size_t)b * P + np];
  }
}

}  // namespace t2i

// ============================================================================
// host side
// ============================================================================
namespace {
using namespace t2i;
using t2i_host::aligned16;
using t2i_host::fail;

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Attention plan: the context is split into chunks of 16 * rows slots, one
// workgroup each; with more than one chunk, their states meet in a workspace:
// the arrival counters (zero between launches), each chunk's (max, sum) pairs
// and each chunk's context.
struct AttnPlan {
  int rows, chunk, splits;
  size_t off_ml, off_o, bytes;
};

AttnPlan plan_attention(int B, int Hq, int Hkv, int ctx_cap) {
  AttnPlan pl{};
  const int Q = Hq / Hkv;
  pl.rows = att_rows(Q);
  bool tuned = false;   // tuning builds: rows given in T2I_ATTN_ROWS are kept
#ifdef T2I_TUNING
  if (const char* env = getenv("T2I_ATTN_ROWS")) {
    const int r = atoi(env);
    if ((r == 4 || r == 8 || r == 9 || r == 16) && Q <= 2) {
      pl.rows = r;
      tuned = true;
    }
  }
#endif
  pl.chunk = 16 * pl.rows;
  pl.splits = (ctx_cap + pl.chunk - 1) / pl.chunk;
  const size_t units = (size_t)B * Hkv;
  // Workgroups are balanced over the 256 CUs when their count is a multiple of
  // 256: then take the fewest splits (at most a quarter more) that make it so,
  // with correspondingly shorter chunks.  Measured at batch 16, context ~576:
  // 6 splits (768 workgroups) 1.011 ms per decode step against 5 (640) 1.023 ms;
  // at batch 8, context 1088, 12 splits against 9 were no faster.
  if (units * pl.splits >= 256 && (units * pl.splits) % 256) {
    for (int s = pl.splits + 1; 4 * s <= 5 * pl.splits; ++s) {
      if ((units * s) % 256 == 0) {
        pl.splits = s;
        pl.chunk = (ctx_cap + s - 1) / s;
        break;
      }
    }
  }
  // Still unbalanced: fewer, longer chunks of up to 144 slots (9 passes) when their
  // count makes a multiple of 256 (batch 8, 1088 slots: 8 chunks of 136, 512
  // workgroups, two a CU, instead of 9 chunks of 128, 576 workgroups).
  if (!tuned && Q <= 2 && pl.rows == 8 && units * pl.splits >= 256 && (units * pl.splits) % 256) {
    const int s9 = (ctx_cap + 16 * 9 - 1) / (16 * 9);
    if (s9 < pl.splits && (units * s9) % 256 == 0) {
      pl.rows = 9;
      pl.splits = s9;
      pl.chunk = (ctx_cap + s9 - 1) / s9;
    }
  }
  // A balanced chunk that fits in seven passes runs seven (batch 16, 640 slots: 6 chunks
  // of 107): the eighth pass would only reload masked slots.
  if (!tuned && Q <= 2 && pl.rows == 8 && pl.splits > 1 && pl.chunk <= 16 * 7) pl.rows = 7;
  if (pl.splits > 1) {
    pl.off_ml = align256(units * sizeof(unsigned));
    pl.off_o = pl.off_ml + align256(units * pl.splits * Q * 2 * sizeof(float));
    pl.bytes = pl.off_o + units * pl.splits * Q * ATT_D * sizeof(float);
  }
  return pl;
}

template <int Q, int ROWS, bool PREP>
hipError_t launch_attention(const AttnParams& p, dim3 grid, hipStream_t s) {
  const int heads = p.Hq | p.Hkv << 15 | p.style << 30;
  const int cap_chunk = (int)((unsigned)p.ctx_cap | (unsigned)p.chunk << 23);
  hipLaunchKernelGGL((decode_attention_kernel<Q, ROWS, PREP>), grid, dim3(ATT_THREADS), 0, s, p.pos, p.qkv, p.kc,
                     p.vc, p.qn, p.kn, heads, cap_chunk, p);
  return hipGetLastError();
}

template <bool PREP>
hipError_t launch_attention_plan(const AttnParams& p, int Q, int rows, dim3 grid, hipStream_t s) {
  switch (Q * 100 + rows) {
    case 104: return launch_attention<1, 4, PREP>(p, grid, s);
    case 107: return launch_attention<1, 7, PREP>(p, grid, s);
    case 108: return launch_attention<1, 8, PREP>(p, grid, s);
    case 109: return launch_attention<1, 9, PREP>(p, grid, s);
    case 116: return launch_attention<1, 16, PREP>(p, grid, s);
    case 204: return launch_attention<2, 4, PREP>(p, grid, s);
    case 207: return launch_attention<2, 7, PREP>(p, grid, s);
    case 208: return launch_attention<2, 8, PREP>(p, grid, s);
    case 209: return launch_attention<2, 9, PREP>(p, grid, s);
    case 216: return launch_attention<2, 16, PREP>(p, grid, s);
    case 404: return launch_attention<4, 4, PREP>(p, grid, s);
    default: return launch_attention<8, 2, PREP>(p, grid, s);
  }
}

}  // namespace

namespace {
int run_rmsnorm(const uint16_t* x, const int32_t* tokens, int32_t V, int32_t M, int32_t H, const uint16_t* weight,
                float eps, uint16_t* x_out, uint16_t* y, uint64_t* argmax_keys, float* y_sums, void* stream) {
  if (!x || !weight || !y) return fail(T2I_ERR_NULL, "x, weight and y must not be NULL");
  if (y_sums && H % 128) return fail(T2I_ERR_SHAPE, "H=%d must be a multiple of 128 with y_sums", H);
  if (y_sums && ((uintptr_t)y_sums & 3u)) return fail(T2I_ERR_ALIGN, "y_sums must be 4-byte aligned");
  if (tokens && !x_out) return fail(T2I_ERR_NULL, "x_out is required with tokens");
  if (tokens && V < 1) return fail(T2I_ERR_SHAPE, "V=%d must be positive with tokens", V);
  if (M < 1) return fail(T2I_ERR_SHAPE, "M=%d must be positive", M);
  if (H < 8 || H % 8 || H > 8 * NORM_THREADS * NORM_MAX_CHUNKS)
    return fail(T2I_ERR_SHAPE, "H=%d must be a multiple of 8 in [8, %d]", H, 8 * NORM_THREADS * NORM_MAX_CHUNKS);
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(y) || (x_out && !aligned16(x_out)))
    return fail(T2I_ERR_ALIGN, "rmsnorm pointers must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto* keys = reinterpret_cast<unsigned long long*>(argmax_keys);
  // rows of up to 128 chunks: one chunk a thread, 128 threads (the same chunk per
  // thread, so the same sums, as 256 threads with half of them idle)
  if (H <= 8 * 128)
    hipLaunchKernelGGL((t2i::rmsnorm_kernel<128, 1>), dim3(M), dim3(128), 0, st, x, tokens, V, H, weight, eps, x_out,
                       y, keys, y_sums);
  else
    hipLaunchKernelGGL((t2i::rmsnorm_kernel<NORM_THREADS, NORM_MAX_CHUNKS>), dim3(M), dim3(NORM_THREADS), 0, st, x,
                       tokens, V, H, weight, eps, x_out, y, keys, y_sums);
  return t2i_host::hip_status(hipGetLastError(), "rmsnorm launch");
}
}  // namespace

extern "C" int t2i_rmsnorm(const uint16_t* x, const int32_t* tokens, int32_t V, int32_t M, int32_t H,
                           const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y,
                           uint64_t* argmax_keys, void* stream) {
  return run_rmsnorm(x, tokens, V, M, H, weight, eps, x_out, y, argmax_keys, nullptr, stream);
}

extern "C" int t2i_rmsnorm_sums(const uint16_t* x, const int32_t* tokens, int32_t V, int32_t M, int32_t H,
                                const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y, float* y_sums,
                                void* stream) {
  if (!y_sums) return fail(T2I_ERR_NULL, "y_sums must not be NULL");
  return run_rmsnorm(x, tokens, V, M, H, weight, eps, x_out, y, nullptr, y_sums, stream);
}

extern "C" size_t t2i_decode_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t ctx_cap) {
  if (B < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv || ctx_cap < 1) return 0;
  return plan_attention(B, Hq, Hkv, ctx_cap).bytes;
}

namespace {
// Argument checks shared by both attention entry points.
int check_attention(const uint16_t* qkv, const int32_t* positions, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                    const uint16_t* q_norm, const uint16_t* k_norm, float eps, const uint16_t* rope,
                    int32_t rope_style, const uint16_t* k_cache, const uint16_t* v_cache, int32_t ctx_cap,
                    const uint16_t* ctx) {
  if (!qkv || !positions || !q_norm || !k_norm || !rope || !k_cache || !v_cache || !ctx)
    return fail(T2I_ERR_NULL, "attention pointers must not be NULL");
  if (D != ATT_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (B < 1 || Hkv < 1 || Hq < Hkv || Hq % Hkv) return fail(T2I_ERR_SHAPE, "B=%d Hq=%d Hkv=%d invalid", B, Hq, Hkv);
  const int Q = Hq / Hkv;
  if (Q != 1 && Q != 2 && Q != 4 && Q != 8) return fail(T2I_ERR_SHAPE, "Hq/Hkv=%d must be 1, 2, 4 or 8", Q);
  if (ctx_cap < 1) return fail(T2I_ERR_SHAPE, "ctx_cap=%d must be positive", ctx_cap);
  if (Hq > 0x7FFF || ctx_cap > 0x7FFFFF) return fail(T2I_ERR_SHAPE, "Hq=%d or ctx_cap=%d too large", Hq, ctx_cap);
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(ctx))
    return fail(T2I_ERR_ALIGN, "attention tensors must be 16-byte aligned");
  return T2I_OK;
}

// Launch with the chunk states at arrivals / part_ml / part_o (unused when the
// plan has a single chunk).
int run_attention(const AttnPlan& pl, const uint16_t* qkv, const int32_t* positions, int32_t B, int32_t Hq,
                  int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                  const uint16_t* rope, int32_t rope_style, uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap,
                  uint16_t* ctx, unsigned* arrivals, float* part_ml, float* part_o, void* stream) {
  const int Q = Hq / Hkv;
  AttnParams p{};
  p.qkv = qkv; p.pos = positions; p.qn = q_norm; p.kn = k_norm; p.rope = rope;
  p.kc = k_cache; p.vc = v_cache; p.out = ctx;
  p.arrivals = arrivals;
  p.part_ml = part_ml;
  p.part_o = part_o;
  p.Hq = Hq; p.Hkv = Hkv; p.ctx_cap = ctx_cap; p.splits = pl.splits; p.chunk = pl.chunk; p.style = rope_style;
  p.eps = eps;
  p.scale = (float)(1.0 / sqrt((double)D));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(B * Hkv, pl.splits);
  const hipError_t e = rope ? launch_attention_plan<true>(p, Q, pl.rows, grid, s)
                            : launch_attention_plan<false>(p, Q, pl.rows, grid, s);
  return t2i_host::hip_status(e, "attention launch");
}

// ---- library-held chunk-state scratch (the allocation-free entry point) ----
// Fixed layout, whatever the call's shape: the arrival counters of up to
// ATT_SCRATCH_UNITS (sequence, kv head) pairs first, then the chunk states.  The
// array is zero-initialised when the code object is loaded, and every call
// leaves the counters it used at zero again, so the counters start at zero for
// every call; a counter word never holds anything else.
constexpr int ATT_SCRATCH_UNITS = 8192;
constexpr size_t ATT_SCRATCH_COUNTERS = ATT_SCRATCH_UNITS * sizeof(unsigned);
constexpr size_t ATT_SCRATCH_BYTES = (size_t)16 << 20;   // T2I_DECODE_ATTENTION_SCRATCH_BYTES
constexpr int ATT_MAX_DEVICES = 64;
static_assert(ATT_SCRATCH_BYTES == T2I_DECODE_ATTENTION_SCRATCH_BYTES, "header and library agree");

std::mutex g_scratch_mu;
char* g_scratch_ptr[ATT_MAX_DEVICES];   // device address of `scratch` on each device, once known

// The device address of the copy of `scratch` on the device that `stream`
// belongs to (the current device for the null stream), set up on the first call
// on that device with that device current.  Host code uses only this address:
// the array's own name on the host is a stand-in, not a device address.
int scratch_for_stream(hipStream_t stream, char** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return t2i_host::hip_status(e, "hipGetDevice");
  int dev = cur;
  if (stream) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return t2i_host::hip_status(e, "hipStreamGetDevice");
  }
  if (dev < 0 || dev >= ATT_MAX_DEVICES) return fail(T2I_ERR_VALUE, "device %d beyond %d", dev, ATT_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return t2i_host::hip_status(e, "hipSetDevice");
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(t2i::scratch));
    if (dev != cur) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess && r != hipSuccess) return t2i_host::hip_status(r, "hipSetDevice");
    }
    if (e != hipSuccess) return t2i_host::hip_status(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(T2I_ERR_NULL, "scratch has no device address");
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return T2I_OK;
}
}  // namespace

extern "C" int t2i_decode_attention(const uint16_t* qkv, const int32_t* positions, int32_t B, int32_t Hq,
                                    int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm,
                                    float eps, const uint16_t* rope, int32_t rope_style, uint16_t* k_cache,
                                    uint16_t* v_cache, int32_t ctx_cap, uint16_t* ctx, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  int rc = check_attention(qkv, positions, B, Hq, Hkv, D, q_norm, k_norm, eps, rope, rope_style, k_cache, v_cache,
                           ctx_cap, ctx);
  if (rc) return rc;
  const AttnPlan pl = plan_attention(B, Hq, Hkv, ctx_cap);
  if (pl.bytes) {
    if (!workspace) return fail(T2I_ERR_WORKSPACE, "workspace of %zu bytes required", pl.bytes);
    if (workspace_bytes < pl.bytes) return fail(T2I_ERR_WORKSPACE, "workspace %zu < required %zu", workspace_bytes, pl.bytes);
    if (!aligned16(workspace)) return fail(T2I_ERR_ALIGN, "workspace must be 16-byte aligned");
  }
  char* ws = pl.bytes ? reinterpret_cast<char*>(workspace) : nullptr;
  return run_attention(pl, qkv, positions, B, Hq, Hkv, D, q_norm, k_norm, eps, rope, rope_style, k_cache, v_cache,
                       ctx_cap, ctx, ws ? reinterpret_cast<unsigned*>(ws) : nullptr,
                       ws ? reinterpret_cast<float*>(ws + pl.off_ml) : nullptr,
                       ws ? reinterpret_cast<float*>(ws + pl.off_o) : nullptr, stream);
}

extern "C" int t2i_decode_attention_prepared(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                             const int32_t* positions, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                             uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap, uint16_t* ctx,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!k || !v) return fail(T2I_ERR_NULL, "attention pointers must not be NULL");
  if (!aligned16(k) || !aligned16(v)) return fail(T2I_ERR_ALIGN, "attention tensors must be 16-byte aligned");
  // the shared checks, with k and v standing in for the norm weights and q for the table
  int rc = check_attention(q, positions, B, Hq, Hkv, D, k, v, 1e-6f, q, 0, k_cache, v_cache, ctx_cap, ctx);
  if (rc) return rc;
  const AttnPlan pl = plan_attention(B, Hq, Hkv, ctx_cap);
  if (pl.bytes) {
    if (!workspace) return fail(T2I_ERR_WORKSPACE, "workspace of %zu bytes required", pl.bytes);
    if (workspace_bytes < pl.bytes) return fail(T2I_ERR_WORKSPACE, "workspace %zu < required %zu", workspace_bytes, pl.bytes);
    if (!aligned16(workspace)) return fail(T2I_ERR_ALIGN, "workspace must be 16-byte aligned");
  }
  char* ws = pl.bytes ? reinterpret_cast<char*>(workspace) : nullptr;
  // rope == NULL selects the kernel form that takes q / k / v as they are
  return run_attention(pl, q, positions, B, Hq, Hkv, D, k, v, 1e-6f, nullptr, 0, k_cache, v_cache, ctx_cap, ctx,
                       ws ? reinterpret_cast<unsigned*>(ws) : nullptr,
                       ws ? reinterpret_cast<float*>(ws + pl.off_ml) : nullptr,
                       ws ? reinterpret_cast<float*>(ws + pl.off_o) : nullptr, stream);
}

extern "C" int t2i_decode_attention_noalloc(const uint16_t* qkv, const int32_t* positions, int32_t B, int32_t Hq,
                                            int32_t Hkv, int32_t D, const uint16_t* q_norm, const uint16_t* k_norm,
                                            float eps, const uint16_t* rope, int32_t rope_style, uint16_t* k_cache,
                                            uint16_t* v_cache, int32_t ctx_cap, uint16_t* ctx, void* stream) {
  int rc = check_attention(qkv, positions, B, Hq, Hkv, D, q_norm, k_norm, eps, rope, rope_style, k_cache, v_cache,
                           ctx_cap, ctx);
  if (rc) return rc;
  const AttnPlan pl = plan_attention(B, Hq, Hkv, ctx_cap);
  const size_t units = (size_t)B * Hkv;
  const size_t states = pl.bytes ? pl.bytes - pl.off_ml : 0;   // chunk states after the counters
  if (pl.bytes && (units > ATT_SCRATCH_UNITS || states > ATT_SCRATCH_BYTES - ATT_SCRATCH_COUNTERS))
    return fail(T2I_ERR_WORKSPACE, "B*Hkv=%zu (max %d) or %zu bytes of chunk states (max %zu) exceed the "
                "library's scratch", units, ATT_SCRATCH_UNITS, states, ATT_SCRATCH_BYTES - ATT_SCRATCH_COUNTERS);
  char* base = nullptr;
  if (pl.bytes) {
    rc = scratch_for_stream(reinterpret_cast<hipStream_t>(stream), &base);
    if (rc) return rc;
  }
  return run_attention(pl, qkv, positions, B, Hq, Hkv, D, q_norm, k_norm, eps, rope, rope_style, k_cache, v_cache,
                       ctx_cap, ctx, base ? reinterpret_cast<unsigned*>(base) : nullptr,
                       base ? reinterpret_cast<float*>(base + ATT_SCRATCH_COUNTERS) : nullptr,
                       base ? reinterpret_cast<float*>(base + ATT_SCRATCH_COUNTERS + (pl.off_o - pl.off_ml)) : nullptr,
                       stream);
}

namespace {

// Launch the lm_head (NORM: with the final RMSNorm of x applied in the kernel)
// over 16-row slices of the M rows.
template <bool NORM>
int run_lm_head(const uint16_t* h, int32_t M, const uint16_t* gamma, float eps, const uint16_t* E, int32_t V,
                int32_t K, float* logits, uint64_t* argmax_keys, void* stream) {
  if (!h || !E || !argmax_keys) return fail(T2I_ERR_NULL, "h, E and argmax_keys must not be NULL");
  if (M < 1) return fail(T2I_ERR_SHAPE, "M=%d must be positive", M);
  if (V < 16 || V % 16) return fail(T2I_ERR_SHAPE, "V=%d must be a positive multiple of 16", V);
  if (K < 64 || K % 64 || K > LMH_MAX_K) return fail(T2I_ERR_SHAPE, "K=%d must be a multiple of 64 in [64, %d]", K, LMH_MAX_K);
  if (!aligned16(h) || !aligned16(E) || (logits && !aligned16(logits)))
    return fail(T2I_ERR_ALIGN, "lm_head tensors must be 16-byte aligned");
  if (NORM) {
    if (!gamma) return fail(T2I_ERR_NULL, "norm_weight must not be NULL");
    if (K & (K - 1)) return fail(T2I_ERR_SHAPE, "K=%d must be a power of two with the fused norm", K);
    if (!aligned16(gamma)) return fail(T2I_ERR_ALIGN, "norm_weight must be 16-byte aligned");
    if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  }
  // at most LMH_WAVES * LMH_TILES tiles a workgroup; a multiple of 256 workgroups
  // once there are more than 256
  const int tiles = V / 16;
  int wgs = (tiles + LMH_WAVES * LMH_TILES - 1) / (LMH_WAVES * LMH_TILES);
  if (wgs > 256) wgs = (wgs + 255) / 256 * 256;
  dim3 grid(wgs);
  const size_t lds = (size_t)16 * K * sizeof(uint16_t) + (size_t)LMH_WAVES * 128 * 16;   // h + the waves' regions
  if (lds > 65536) {
    // the attribute belongs to the function on the current device: remember the
    // raised limit per device (a larger K raises it again)
    constexpr int kMaxDevices = 64;
    static std::atomic<size_t> raised[kMaxDevices];
    int dev = 0;
    int rc = t2i_host::hip_status(hipGetDevice(&dev), "lm_head device query");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices || lds > raised[dev].load(std::memory_order_relaxed)) {
      rc = t2i_host::hip_status(
          hipFuncSetAttribute(reinterpret_cast<const void*>(t2i::lm_head_kernel<NORM>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "lm_head LDS attribute");
      if (rc) return rc;
      if (dev >= 0 && dev < kMaxDevices) {
        size_t cur = raised[dev].load(std::memory_order_relaxed);
        while (cur < lds && !raised[dev].compare_exchange_weak(cur, lds, std::memory_order_relaxed)) {
        }
      }
    }
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int m0 = 0; m0 < M; m0 += 16) {
    const int mc = (M - m0) < 16 ? (M - m0) : 16;
    hipLaunchKernelGGL(t2i::lm_head_kernel<NORM>, grid, dim3(64 * LMH_WAVES), lds, s, h + (size_t)m0 * K, mc, E, V,
                       K, logits ? logits + (size_t)m0 * V : nullptr,
                       reinterpret_cast<unsigned long long*>(argmax_keys) + m0, gamma, eps);
    int rc = t2i_host::hip_status(hipGetLastError(), "lm_head launch");
    if (rc) return rc;
  }
  return T2I_OK;
}

}  // namespace

extern "C" int t2i_lm_head_argmax(const uint16_t* h, int32_t M, const uint16_t* E, int32_t V, int32_t K,
                                  float* logits, uint64_t* argmax_keys, void* stream) {
  return run_lm_head<false>(h, M, nullptr, 0.0f, E, V, K, logits, argmax_keys, stream);
}

extern "C" int t2i_rmsnorm_lm_head_argmax(const uint16_t* x, int32_t M, const uint16_t* norm_weight, float eps,
                                          const uint16_t* E, int32_t V, int32_t K, float* logits,
                                          uint64_t* argmax_keys, void* stream) {
  return run_lm_head<true>(x, M, norm_weight, eps, E, V, K, logits, argmax_keys, stream);
}

extern "C" int t2i_greedy_advance(const uint64_t* argmax_keys, int32_t B, int32_t* tokens, int32_t* positions,
                                  int32_t* history, int32_t hist_cap, int32_t* step, void* stream) {
  if (!argmax_keys || !tokens || !positions || !step) return fail(T2I_ERR_NULL, "greedy_advance pointers must not be NULL");
  if (B < 1 || B > 1024) return fail(T2I_ERR_SHAPE, "B=%d must be in [1, 1024]", B);
  if (history && hist_cap < 1) return fail(T2I_ERR_VALUE, "hist_cap must be positive");
  hipLaunchKernelGGL(t2i::greedy_advance_kernel, dim3(1), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const unsigned long long*>(argmax_keys), B, tokens, positions, history,
                     hist_cap, step);
  return t2i_host::hip_status(hipGetLastError(), "greedy_advance launch");
}

extern "C" int t2i_prompt_advance(const int32_t* prompt, int32_t B, int32_t P, int32_t* tokens, int32_t* positions,
                                  void* stream) {
  if (!prompt || !tokens || !positions) return fail(T2I_ERR_NULL, "prompt_advance pointers must not be NULL");
  if (B < 1 || B > 1024 || P < 1) return fail(T2I_ERR_SHAPE, "B=%d P=%d invalid", B, P);
  hipLaunchKernelGGL(t2i::prompt_advance_kernel, dim3(1), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     prompt, B, P, tokens, positions);
  return t2i_host::hip_status(hipGetLastError(), "prompt_advance launch");
}
