// One (sequence, kv head, context split) item of GQA decode attention, for
// kernels that produce q / k / v in the same launch as tagged 64-bit words (the
// bf16 bits in the low half, the producing launch's tag in the high half) and
// keep one 16-wave workgroup per CU (gfx950).
//
// The item's first slots of K / V go straight into LDS (attn_prefetch, up to
// 192 slots a workgroup) as soon as the item is known, ahead of the projection
// the launch runs first; attn_run then polls the q, k, v words it needs until
// their tags show this launch's values, applies the per-head q / k RMSNorm and
// RoPE (the rounding chain of t2i_decode_attention), writes the current slot to
// the cache, folds the prefetched slots and streams the rest through registers.
// A split context is merged by split 0, which polls the other splits' tagged
// partial states in split order.  Every wait is bounded (wait_gives_up): a
// wait that gives up raises the error word (ctl[2]) and the workgroup carries
// on, so the launch always ends.
#pragma once

#include "t2i_common.h"

namespace t2i {

constexpr int AI_WAVES = 16;
constexpr int AI_THREADS = 64 * AI_WAVES;
constexpr int AI_GROUPS = 4 * AI_WAVES;          // 64 slot groups of 16 lanes
constexpr int AI_PF = 3;                         // slots per group prefetched into LDS
constexpr int AI_PF_SLOTS = AI_GROUPS * AI_PF;   // 192
constexpr int AI_ROWS = 4;                       // slots per group in each streamed pass
constexpr size_t AI_LDS_KV = (size_t)AI_WAVES * AI_PF * 2 * 64 * 16;   // 96 KiB of prefetched K / V

// Poll one tagged word until it carries `tag` (bounded, see wait_gives_up).
__device__ __forceinline__ unsigned long long ai_poll(const unsigned long long* src, uint32_t tag, unsigned* ctl) {
  unsigned long long w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int spins = 0;
  while ((uint32_t)(w >> 32) != tag) {
    if (wait_gives_up(spins, ctl)) break;
    w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return w;
}

struct AttnArgs {
  const unsigned long long* ll;   // [B][ldll] tagged q | k | v words
  int ldll;
  const int32_t* pos;
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* rope;
  uint16_t* kc;                   // [B][Hkv][ctx_cap][D]
  uint16_t* vc;
  uint16_t* out;                  // [B][Hq * D] bf16, or
  uint32_t* out_ll;               // [B][Hq * D] tagged 32-bit words (bf16 | tag low 16 bits << 16)
  unsigned long long* st;         // [U][S - 1][Q][D + 2] tagged partial states of splits 1 .. S-1
  unsigned* ctl;                  // [2]: the error word
  int B, Hq, Hkv, ctx_cap, style, S;
  float eps, scale;
  uint32_t tag;
};

// Pointers into the workgroup's LDS (the caller owns the arrays).
struct AttnSmem {
  uint16_t* raw;   // [Q + 2][D]
  uint16_t* q;     // [Q][D]
  uint16_t* kv;    // [2][D]
  float* wm;       // [AI_WAVES][Q]
  float* wl;       // [AI_WAVES][Q]
  float* wacc;     // [AI_WAVES][Q][D]
};

struct AttnItem {
  int b, h, s, u;
  bool valid;      // position inside the cache (else: no write, zero output)
  int pos, t0, t1;
  size_t cache_base;
};

__device__ __forceinline__ AttnItem attn_item(const AttnArgs& a, int item) {
  constexpr int D = ATT_D;
  AttnItem it;
  it.u = item / a.S;
  it.s = item - it.u * a.S;
  it.b = it.u / a.Hkv;
  it.h = it.u - it.b * a.Hkv;
  const int pos_raw = a.pos[it.b];
  it.valid = pos_raw >= 0 && pos_raw < a.ctx_cap;
  it.pos = it.valid ? pos_raw : 0;
  const int L = it.valid ? it.pos + 1 : 0;
  const int chunk = (L + a.S - 1) / a.S;
  it.t0 = min(it.s * chunk, L);
  it.t1 = min(it.t0 + chunk, L);
  it.cache_base = ((size_t)it.b * a.Hkv + it.h) * (size_t)a.ctx_cap * D;
  return it;
}

typedef __attribute__((address_space(3))) void ai_lds_t;
typedef __attribute__((address_space(1))) void ai_global_t;

// The item's first AI_PF slots of every group, K and V, straight into LDS
// ([wave][AI_PF][K, V][64 lanes] of 16 bytes; each lane reads back what it loaded).
// Slots past the split read slot 0 (always present) and are masked when scored.
__device__ __forceinline__ void attn_prefetch(const AttnArgs& a, const AttnItem& it, u32x4* kv_lds) {
  constexpr int D = ATT_D;
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int grp = wave * 4 + (lane >> 4);
#pragma unroll
  for (int i = 0; i < AI_PF; ++i) {
    const int t = it.t0 + i * AI_GROUPS + grp;
    const int tl = t < it.t1 ? t : 0;
    u32x4* dst = kv_lds + ((size_t)(wave * AI_PF + i) * 2) * 64;
    __builtin_amdgcn_global_load_lds((ai_global_t*)(a.kc + it.cache_base + (size_t)tl * D + 8 * c), (ai_lds_t*)dst,
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds((ai_global_t*)(a.vc + it.cache_base + (size_t)tl * D + 8 * c),
                                     (ai_lds_t*)(dst + 64), 16, 0, 0);
  }
}

// Scores of RPP slots per group folded into the group's online softmax state.
template <int Q, int RPP>
__device__ __forceinline__ void attn_fold(const int (&t)[RPP], int t1, int pos, const u32x4 (&qv)[Q], u32x4 kcur,
                                          u32x4 vcur, float sl2, const u32x4 (&kr)[RPP], const u32x4 (&vr_in)[RPP],
                                          float (&m)[Q], float (&l)[Q], float (&acc)[Q][8]) {
  const u32x4 zero4 = u32x4{0u, 0u, 0u, 0u};
  float sc[RPP][Q];
  u32x4 vr[RPP];
#pragma unroll
  for (int it = 0; it < RPP; ++it) {
    const u32x4 kk = t[it] == pos ? kcur : kr[it];
    vr[it] = t[it] < t1 ? (t[it] == pos ? vcur : vr_in[it]) : zero4;
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      float d = dot2_bf16(qv[j].x, kk.x, 0.0f);
      d = dot2_bf16(qv[j].y, kk.y, d);
      d = dot2_bf16(qv[j].z, kk.z, d);
      d = dot2_bf16(qv[j].w, kk.w, d);
      d = row_sum16(d);
      sc[it][j] = t[it] < t1 ? d * sl2 : -INFINITY;
    }
  }
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    float mn = m[j];
#pragma unroll
    for (int it = 0; it < RPP; ++it) mn = fmaxf(mn, sc[it][j]);
    const float alpha = state_weight(m[j], mn);
    const float mz = mn > -INFINITY ? mn : 0.0f;
    l[j] *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] *= alpha;
    m[j] = mn;
#pragma unroll
    for (int it = 0; it < RPP; ++it) {
      float vf[8];
      unpack8(vr[it], vf);
      const float pe = exp2_fast(sc[it][j] - mz);
      l[j] += pe;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(pe, vf[e], acc[j][e]);
    }
  }
}

// The item (every thread of the workgroup calls it).  COH: the context goes out
// as tagged 32-bit words (out_ll, read by other workgroups of the same launch).
// Returns whether this workgroup wrote the item's context rows (split 0).
template <int Q, bool COH>
__device__ __forceinline__ bool attn_run(const AttnArgs& a, const AttnItem& it, const u32x4* kv_lds,
                                         const AttnSmem& sm) {
  constexpr int D = ATT_D;
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int grp = wave * 4 + (lane >> 4);
  const int b = it.b, h = it.h, pos = it.pos, t0 = it.t0, t1 = it.t1;

  // ---- the item's q, k and v values (tagged words) ----
  if (tid < (Q + 2) * D) {
    const int vi = tid / D, d = tid - (tid / D) * D;
    const int hrow = vi < Q ? h * Q + vi : (vi == Q ? a.Hq + h : a.Hq + a.Hkv + h);
    const unsigned long long w = ai_poll(a.ll + (size_t)b * a.ldll + (size_t)hrow * D + d, a.tag, a.ctl);
    sm.raw[vi * D + d] = (uint16_t)(w & 0xFFFFu);
  }
  const int i0 = a.style == 0 ? lane : 2 * lane;
  const int i1 = a.style == 0 ? lane + D / 2 : 2 * lane + 1;
  const int vi = min(wave, Q + 1);
  const uint16_t* gamma = vi < Q ? a.qn : a.kn;
  const float g0 = bf16_to_f32(gamma[i0]), g1 = bf16_to_f32(gamma[i1]);
  const float cs = bf16_to_f32(a.rope[(size_t)pos * D + 2 * lane]);
  const float sn = bf16_to_f32(a.rope[(size_t)pos * D + 2 * lane + 1]);
  __syncthreads();
  // q heads and the current k: per-head RMSNorm then RoPE; v as is
  {
    float x0 = bf16_to_f32(sm.raw[vi * D + i0]), x1 = bf16_to_f32(sm.raw[vi * D + i1]);
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float inv = round_bf16(1.0f / sqrtf(ss / (float)D + a.eps));
    const float n0 = round_bf16(round_bf16(x0 * inv) * g0);
    const float n1 = round_bf16(round_bf16(x1 * inv) * g1);
    const float y0 = round_bf16(round_bf16(n0 * cs) + round_bf16(-n1 * sn));
    const float y1 = round_bf16(round_bf16(n1 * cs) + round_bf16(n0 * sn));
    x0 = vi <= Q ? y0 : x0;
    x1 = vi <= Q ? y1 : x1;
    if (wave < Q) {
      sm.q[wave * D + i0] = (uint16_t)f32_to_bf16(x0);
      sm.q[wave * D + i1] = (uint16_t)f32_to_bf16(x1);
    } else if (wave < Q + 2) {
      const int which = wave - Q;   // 0 = k, 1 = v
      const uint16_t b0 = (uint16_t)f32_to_bf16(x0), b1 = (uint16_t)f32_to_bf16(x1);
      sm.kv[which * D + i0] = b0;
      sm.kv[which * D + i1] = b1;
      if (it.valid && pos >= t0 && pos < t1) {   // this split holds the current slot: persist it
        uint16_t* dst = (which == 0 ? a.kc : a.vc) + it.cache_base + (size_t)pos * D;
        dst[i0] = b0;
        dst[i1] = b1;
      }
    }
  }
  __syncthreads();

  // ---- scores and the online softmax of each 16-lane group ----
  u32x4 qv[Q];
#pragma unroll
  for (int j = 0; j < Q; ++j) qv[j] = reinterpret_cast<const u32x4*>(sm.q + j * D)[c];
  const u32x4 kcur = reinterpret_cast<const u32x4*>(sm.kv)[c];
  const u32x4 vcur = reinterpret_cast<const u32x4*>(sm.kv + D)[c];
  const float sl2 = a.scale * 1.4426950408889634f;
  float m[Q], l[Q], acc[Q][8];
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
  }
  // the prefetched slots (each lane reads back what it loaded itself)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  {
    int t[AI_PF];
    u32x4 kr[AI_PF], vr[AI_PF];
#pragma unroll
    for (int i = 0; i < AI_PF; ++i) {
      t[i] = t0 + i * AI_GROUPS + grp;
      const u32x4* src = kv_lds + ((size_t)(wave * AI_PF + i) * 2) * 64;
      kr[i] = src[lane];
      vr[i] = src[64 + lane];
    }
    attn_fold<Q, AI_PF>(t, t1, pos, qv, kcur, vcur, sl2, kr, vr, m, l, acc);
  }
  // the rest of a long split, AI_ROWS slots a group per pass
  for (int base = t0 + AI_PF_SLOTS; base < t1; base += AI_GROUPS * AI_ROWS) {
    int t[AI_ROWS];
    u32x4 kr[AI_ROWS], vr[AI_ROWS];
#pragma unroll
    for (int i = 0; i < AI_ROWS; ++i) {
      t[i] = base + i * AI_GROUPS + grp;
      const int tl = t[i] < t1 ? t[i] : t0;
      kr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.kc + it.cache_base + (size_t)tl * D + 8 * c));
      vr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.vc + it.cache_base + (size_t)tl * D + 8 * c));
    }
    attn_fold<Q, AI_ROWS>(t, t1, pos, qv, kcur, vcur, sl2, kr, vr, m, l, acc);
  }

  // ---- merge the four groups of each wave, then the 16 waves in LDS, in order ----
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const float mo = __shfl_xor(m[j], off, 64);
      const float lo = __shfl_xor(l[j], off, 64);
      const float mn = fmaxf(m[j], mo);
      const float fa = state_weight(m[j], mn), fb = state_weight(mo, mn);
      l[j] = l[j] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = acc[j][e] * fa + __shfl_xor(acc[j][e], off, 64) * fb;
      m[j] = mn;
    }
  }
  if ((lane >> 4) == 0) {
#pragma unroll
    for (int j = 0; j < Q; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.wacc[(wave * Q + j) * D + 8 * c + e] = acc[j][e];
      if (c == 0) {
        sm.wm[wave * Q + j] = m[j];
        sm.wl[wave * Q + j] = l[j];
      }
    }
  }
  __syncthreads();

  // ---- this split's state; split 0 merges the others, in split order ----
  if (tid < Q * D) {
    const int j = tid / D, d = tid - (tid / D) * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AI_WAVES; ++w) M = fmaxf(M, sm.wm[w * Q + j]);
    float lsum = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < AI_WAVES; ++w) {
      const float f = state_weight(sm.wm[w * Q + j], M);
      lsum = fmaf(sm.wl[w * Q + j], f, lsum);
      o = fmaf(sm.wacc[(w * Q + j) * D + d], f, o);
    }
    const size_t row = (size_t)(D + 2);
    if (it.s > 0) {
      unsigned long long* dst = a.st + ((size_t)(it.u * (a.S - 1) + it.s - 1) * Q + j) * row;
      const unsigned long long hi = (unsigned long long)a.tag << 32;
      __hip_atomic_store(dst + d, hi | __float_as_uint(o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(dst + D, hi | __float_as_uint(M), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(dst + D + 1, hi | __float_as_uint(lsum), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      for (int sp = 1; sp < a.S; ++sp) {
        const unsigned long long* src = a.st + ((size_t)(it.u * (a.S - 1) + sp - 1) * Q + j) * row;
        const float op = __uint_as_float((uint32_t)ai_poll(src + d, a.tag, a.ctl));
        const float mp = __uint_as_float((uint32_t)ai_poll(src + D, a.tag, a.ctl));
        const float lp = __uint_as_float((uint32_t)ai_poll(src + D + 1, a.tag, a.ctl));
        if (lp > 0.0f) {   // an empty split weighs nothing
          const float mn = fmaxf(M, mp);
          const float fa = state_weight(M, mn), fb = exp2_fast(mp - mn);
          lsum = lsum * fa + lp * fb;
          o = o * fa + op * fb;
          M = mn;
        }
      }
      const size_t idx = (size_t)b * a.Hq * D + (size_t)(h * Q + j) * D + d;
      const uint16_t v = lsum > 0.0f ? (uint16_t)f32_to_bf16(o / lsum) : (uint16_t)0;
      if constexpr (COH) st_coh32(a.out_ll + idx, (uint32_t)v | (a.tag << 16));
      else a.out[idx] = v;
    }
  }
  return it.s == 0;
}

}  // namespace t2i
