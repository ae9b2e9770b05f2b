// The front of the decode layer in one cooperative launch (gfx950): input
// RMSNorm + fused q|k|v projection, then GQA decode attention with q/k RMSNorm,
// RoPE and the KV-cache write of the current token.
//
// One 16-wave workgroup per CU, all co-resident (cooperative launch).  Every
// workgroup first computes one 16-column block of the qkv projection for all
// rows (the decode linear's tile, bit-identical to t2i_w4a16_rmsnorm_linear)
// and sends each value out as a tagged 64-bit word; it then takes one
// (sequence, kv head, context split) item of the attention, polls the q, k and
// v words it needs until their tags show this launch's values, and attends.
// The item's K / V rows were issued before the projection's first arithmetic,
// straight into LDS (up to 192 slots a workgroup), so the context stream
// overlaps the projection, its hand-off and the prologue; the rest of a long
// context streams through registers.  A context split over several
// workgroups is merged by split 0, which polls the other splits' tagged
// partial states; with one split per item there is no merge.
//
// Tags: the workspace holds a launch counter; a launch's tag is the counter
// value plus one, read by every workgroup at the start, and the last workgroup
// to finish advances the counter.  A word from an earlier launch therefore
// never carries the current tag (the zero-filled workspace carries tag 0).
// Every wait is bounded: a wait that gives up raises the workspace's error
// flag and the workgroup carries on, so the launch always ends.
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "t2i_common.h"
#include "w4a16_tile.h"

namespace t2i {

constexpr int FQ_WAVES = 16;
constexpr int FQ_THREADS = 64 * FQ_WAVES;
constexpr int FQ_GROUPS = 4 * FQ_WAVES;          // 64 slot groups of 16 lanes
constexpr int FQ_PF = 3;                         // slots per group prefetched into LDS
constexpr int FQ_PF_SLOTS = FQ_GROUPS * FQ_PF;   // 192
constexpr int FQ_ROWS = 4;                       // slots per group in each streamed pass
constexpr int FQ_SPIN = 1 << 18;                 // polls before a wait gives up
constexpr size_t FQ_LDS_KV = (size_t)FQ_WAVES * FQ_PF * 2 * 64 * 16;   // 96 KiB of prefetched K / V

struct FqaParams {
  LinearParams lin;             // the qkv projection, EPI_LL into lin.ll [B][N]
  const int32_t* pos;
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* rope;
  uint16_t* kc;
  uint16_t* vc;
  uint16_t* out;                // [B][Hq * D]
  unsigned long long* st;       // [U][S - 1][Q][D + 2] tagged partial states of splits 1 .. S-1
  unsigned* ctl;                // [0] launch counter, [1] finished workgroups, [2] error flag
  int B, Hq, Hkv, ctx_cap, style, S, nb;
  float eps, scale;
};

__device__ __forceinline__ void fq_fail(unsigned* ctl) {
  __hip_atomic_store(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll one tagged word until it carries `tag` (bounded).
__device__ __forceinline__ unsigned long long fq_poll(const unsigned long long* src, uint32_t tag, unsigned* ctl) {
  unsigned long long w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int spins = 0;
  while ((uint32_t)(w >> 32) != tag) {
    if (++spins >= FQ_SPIN) { fq_fail(ctl); break; }
    __builtin_amdgcn_s_sleep(1);
    w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return w;
}

// Scores of RPP slots per group folded into the group's online softmax state.
template <int Q, int RPP>
__device__ __forceinline__ void fq_fold(const int (&t)[RPP], int t1, int pos, const u32x4 (&qv)[Q], u32x4 kcur,
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

typedef __attribute__((address_space(3))) void fq_lds_t;
typedef __attribute__((address_space(1))) void fq_global_t;

template <int Q, bool NORM>
__global__ __launch_bounds__(FQ_THREADS) void fused_qkv_attention_kernel(const FqaParams p) {
  constexpr int D = ATT_D;
  extern __shared__ u32x4 fq_kv[];   // [wave][FQ_PF][K, V][64 lanes]
  __shared__ __align__(16) uint16_t s_raw[Q + 2][D];
  __shared__ __align__(16) uint16_t s_q[Q][D];
  __shared__ __align__(16) uint16_t s_kv[2][D];
  __shared__ float s_wm[FQ_WAVES][Q], s_wl[FQ_WAVES][Q];
  __shared__ float s_wacc[FQ_WAVES][Q][D];

  const int G = gridDim.x;
  const int wg = blockIdx.x;
  const uint32_t tag = __hip_atomic_load(p.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  // this workgroup's attention item: (sequence b, kv head h, split s); past the
  // last item a workgroup only takes part in the projection
  const int U = p.B * p.Hkv;
  const bool has_item = wg < U * p.S;
  const int item = has_item ? wg : 0;
  const int u = item / p.S, s = item - (item / p.S) * p.S;
  const int b = u / p.Hkv, h = u - (u / p.Hkv) * p.Hkv;
  const int pos_raw = p.pos[b];
  const bool valid = pos_raw >= 0 && pos_raw < p.ctx_cap;
  const int pos = valid ? pos_raw : 0;
  const int L = valid ? pos + 1 : 0;
  const int chunk = (L + p.S - 1) / p.S;
  const int t0 = min(s * chunk, L);
  const int t1 = min(t0 + chunk, L);
  const size_t cache_base = ((size_t)b * p.Hkv + h) * (size_t)p.ctx_cap * D;

  // ---- the item's first slots straight into LDS, issued once the projection's
  // first loads are out (loads complete in issue order) ----
  auto prefetch = [&]() {
    if (!has_item) return;   // workgroup-uniform
    // lane indices recomputed here: nothing lane-dependent stays live across the projection
    const int pl_lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = pl_lane & 15;
    const int grp = wave * 4 + (pl_lane >> 4);
#pragma unroll
    for (int it = 0; it < FQ_PF; ++it) {
      const int t = t0 + it * FQ_GROUPS + grp;
      const int tl = t < t1 ? t : 0;   // slot 0 always exists; masked when scored
      u32x4* dst = fq_kv + ((size_t)(wave * FQ_PF + it) * 2) * 64;
      __builtin_amdgcn_global_load_lds((fq_global_t*)(p.kc + cache_base + (size_t)tl * D + 8 * c), (fq_lds_t*)dst,
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((fq_global_t*)(p.vc + cache_base + (size_t)tl * D + 8 * c),
                                       (fq_lds_t*)(dst + 64), 16, 0, 0);
    }
  };

  // ---- phase 1: qkv column blocks (normally one per workgroup) ----
  {
    LinearParams lp = p.lin;
    lp.tag = tag;
    bool first = true;
    for (int blk = wg; blk < p.nb; blk += G) {
      if (first) {
        linear_tile<1, 1, 16, 2, NORM>(lp, p.nb, blk, 0, prefetch);
        first = false;
      } else {
        linear_tile<1, 1, 16, 2, NORM>(lp, p.nb, blk, 0);
      }
      __syncthreads();
    }
    if (first) prefetch();   // no projection block: the prefetch still goes out
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int grp = wave * 4 + (lane >> 4);
  if (has_item) {
    // ---- phase 2a: the item's q, k and v values (tagged words) ----
    if (tid < (Q + 2) * D) {
      const int vi = tid / D, d = tid - (tid / D) * D;
      const int hrow = vi < Q ? h * Q + vi : (vi == Q ? p.Hq + h : p.Hq + p.Hkv + h);
      const unsigned long long w = fq_poll(p.lin.ll + (size_t)b * p.lin.ldy + (size_t)hrow * D + d, tag, p.ctl);
      s_raw[vi][d] = (uint16_t)(w & 0xFFFFu);
    }
    const int i0 = p.style == 0 ? lane : 2 * lane;
    const int i1 = p.style == 0 ? lane + D / 2 : 2 * lane + 1;
    const int vi = min(wave, Q + 1);
    const uint16_t* gamma = vi < Q ? p.qn : p.kn;
    const float g0 = bf16_to_f32(gamma[i0]), g1 = bf16_to_f32(gamma[i1]);
    const float cs = bf16_to_f32(p.rope[(size_t)pos * D + 2 * lane]);
    const float sn = bf16_to_f32(p.rope[(size_t)pos * D + 2 * lane + 1]);
    __syncthreads();
    // q heads and the current k: per-head RMSNorm then RoPE (the rounding chain of
    // t2i_decode_attention); v as is
    {
      float x0 = bf16_to_f32(s_raw[vi][i0]), x1 = bf16_to_f32(s_raw[vi][i1]);
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float inv = round_bf16(1.0f / sqrtf(ss / (float)D + p.eps));
      const float n0 = round_bf16(round_bf16(x0 * inv) * g0);
      const float n1 = round_bf16(round_bf16(x1 * inv) * g1);
      const float y0 = round_bf16(round_bf16(n0 * cs) + round_bf16(-n1 * sn));
      const float y1 = round_bf16(round_bf16(n1 * cs) + round_bf16(n0 * sn));
      x0 = vi <= Q ? y0 : x0;
      x1 = vi <= Q ? y1 : x1;
      if (wave < Q) {
        s_q[wave][i0] = (uint16_t)f32_to_bf16(x0);
        s_q[wave][i1] = (uint16_t)f32_to_bf16(x1);
      } else if (wave < Q + 2) {
        const int which = wave - Q;   // 0 = k, 1 = v
        const uint16_t b0 = (uint16_t)f32_to_bf16(x0), b1 = (uint16_t)f32_to_bf16(x1);
        s_kv[which][i0] = b0;
        s_kv[which][i1] = b1;
        if (valid && pos >= t0 && pos < t1) {   // this split holds the current slot: persist it
          uint16_t* dst = (which == 0 ? p.kc : p.vc) + cache_base + (size_t)pos * D;
          dst[i0] = b0;
          dst[i1] = b1;
        }
      }
    }
    __syncthreads();

    // ---- phase 2b: scores and the online softmax of each 16-lane group ----
    u32x4 qv[Q];
#pragma unroll
    for (int j = 0; j < Q; ++j) qv[j] = reinterpret_cast<const u32x4*>(&s_q[j][0])[c];
    const u32x4 kcur = reinterpret_cast<const u32x4*>(&s_kv[0][0])[c];
    const u32x4 vcur = reinterpret_cast<const u32x4*>(&s_kv[1][0])[c];
    const float sl2 = p.scale * 1.4426950408889634f;
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
      int t[FQ_PF];
      u32x4 kr[FQ_PF], vr[FQ_PF];
#pragma unroll
      for (int it = 0; it < FQ_PF; ++it) {
        t[it] = t0 + it * FQ_GROUPS + grp;
        const u32x4* src = fq_kv + ((size_t)(wave * FQ_PF + it) * 2) * 64;
        kr[it] = src[lane];
        vr[it] = src[64 + lane];
      }
      fq_fold<Q, FQ_PF>(t, t1, pos, qv, kcur, vcur, sl2, kr, vr, m, l, acc);
    }
    // the rest of a long split, FQ_ROWS slots a group per pass
    for (int base = t0 + FQ_PF_SLOTS; base < t1; base += FQ_GROUPS * FQ_ROWS) {
      int t[FQ_ROWS];
      u32x4 kr[FQ_ROWS], vr[FQ_ROWS];
#pragma unroll
      for (int it = 0; it < FQ_ROWS; ++it) {
        t[it] = base + it * FQ_GROUPS + grp;
        const int tl = t[it] < t1 ? t[it] : t0;
        kr[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.kc + cache_base + (size_t)tl * D + 8 * c));
        vr[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.vc + cache_base + (size_t)tl * D + 8 * c));
      }
      fq_fold<Q, FQ_ROWS>(t, t1, pos, qv, kcur, vcur, sl2, kr, vr, m, l, acc);
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
        for (int e = 0; e < 8; ++e) s_wacc[wave][j][8 * c + e] = acc[j][e];
        if (c == 0) { s_wm[wave][j] = m[j]; s_wl[wave][j] = l[j]; }
      }
    }
    __syncthreads();

    // ---- phase 2c: this split's state; split 0 merges the others, in split order ----
    if (tid < Q * D) {
      const int j = tid / D, d = tid - (tid / D) * D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < FQ_WAVES; ++w) M = fmaxf(M, s_wm[w][j]);
      float lsum = 0.0f, o = 0.0f;
#pragma unroll
      for (int w = 0; w < FQ_WAVES; ++w) {
        const float f = state_weight(s_wm[w][j], M);
        lsum = fmaf(s_wl[w][j], f, lsum);
        o = fmaf(s_wacc[w][j][d], f, o);
      }
      const size_t row = (size_t)(D + 2);
      if (s > 0) {
        unsigned long long* dst = p.st + ((size_t)(u * (p.S - 1) + s - 1) * Q + j) * row;
        const unsigned long long hi = (unsigned long long)tag << 32;
        __hip_atomic_store(dst + d, hi | __float_as_uint(o), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
          __hip_atomic_store(dst + D, hi | __float_as_uint(M), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(dst + D + 1, hi | __float_as_uint(lsum), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        for (int sp = 1; sp < p.S; ++sp) {
          const unsigned long long* src = p.st + ((size_t)(u * (p.S - 1) + sp - 1) * Q + j) * row;
          const float op = __uint_as_float((uint32_t)fq_poll(src + d, tag, p.ctl));
          const float mp = __uint_as_float((uint32_t)fq_poll(src + D, tag, p.ctl));
          const float lp = __uint_as_float((uint32_t)fq_poll(src + D + 1, tag, p.ctl));
          if (lp > 0.0f) {   // an empty split weighs nothing
            const float mn = fmaxf(M, mp);
            const float fa = state_weight(M, mn), fb = exp2_fast(mp - mn);
            lsum = lsum * fa + lp * fb;
            o = o * fa + op * fb;
            M = mn;
          }
        }
        p.out[(size_t)b * p.Hq * D + (size_t)(h * Q + j) * D + d] =
            lsum > 0.0f ? (uint16_t)f32_to_bf16(o / lsum) : (uint16_t)0;
      }
    }
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the unused prefetch lands before the end
  }

  // ---- the last workgroup to finish advances the launch counter ----
  __syncthreads();
  if (tid == 0) {
    const unsigned before = __hip_atomic_fetch_add(p.ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before == (unsigned)(G - 1)) {
      __hip_atomic_store(p.ctl + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(p.ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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

constexpr int FQ_MAX_DEVICES = 64;
constexpr int FQ_MAX_ROWS = 16;

size_t fq_align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workgroups of the launch on the current device: one per CU, provided the
// kernel fits one 16-wave workgroup per CU (checked once per device and kernel).
struct FqDevice {
  int cus = 0;
  bool ready[2][2] = {{false, false}, {false, false}};   // [Q == 2][NORM]
  bool ok[2][2] = {{false, false}, {false, false}};
};
std::mutex g_fq_mu;
FqDevice g_fq_dev[FQ_MAX_DEVICES];

template <int Q, bool NORM>
int fq_setup(int dev, FqDevice& d) {
  const int qi = Q == 2, ni = NORM;
  if (d.ready[qi][ni]) return d.ok[qi][ni] ? T2I_OK : fail(T2I_ERR_VALUE, "the fused kernel does not fit one workgroup a CU");
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&fused_qkv_attention_kernel<Q, NORM>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)FQ_LDS_KV);
  if (e != hipSuccess) return t2i_host::hip_status(e, "fused kernel LDS limit");
  int occ = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(
                                                         &fused_qkv_attention_kernel<Q, NORM>),
                                                   FQ_THREADS, FQ_LDS_KV);
  if (e != hipSuccess) return t2i_host::hip_status(e, "fused kernel occupancy");
  d.ready[qi][ni] = true;
  d.ok[qi][ni] = occ >= 1;
  (void)dev;
  return d.ok[qi][ni] ? T2I_OK : fail(T2I_ERR_VALUE, "the fused kernel does not fit one workgroup a CU");
}

struct FqPlan {
  int G, S, U;
  size_t off_st, off_ctl, bytes;
};

FqPlan fq_plan(int cus, int B, int Hq, int Hkv, int N) {
  FqPlan pl{};
  pl.G = cus;
  pl.U = B * Hkv;
  pl.S = 1;
  while (pl.S < 16 && pl.U * pl.S * 2 <= pl.G) pl.S *= 2;
  const int Q = Hq / Hkv;
  const size_t ll = (size_t)B * N * 8;
  pl.off_st = fq_align256(ll);
  pl.off_ctl = pl.off_st + fq_align256((size_t)pl.U * (pl.S - 1) * Q * (ATT_D + 2) * 8);
  pl.bytes = pl.off_ctl + 256;
  return pl;
}

int fq_cus(int* cus, int* dev_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return t2i_host::hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= FQ_MAX_DEVICES) return fail(T2I_ERR_VALUE, "device %d beyond %d", dev, FQ_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_fq_mu);
  if (g_fq_dev[dev].cus == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return t2i_host::hip_status(e, "CU count");
    g_fq_dev[dev].cus = n;
  }
  *cus = g_fq_dev[dev].cus;
  *dev_out = dev;
  return T2I_OK;
}

}  // namespace

extern "C" size_t t2i_qkv_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv) {
  if (B < 1 || B > FQ_MAX_ROWS || Hkv < 1 || Hq % Hkv) return 0;
  int cus = 0, dev = 0;
  if (fq_cus(&cus, &dev)) return 0;
  return fq_plan(cus, B, Hq, Hkv, (Hq + 2 * Hkv) * ATT_D).bytes;
}

extern "C" size_t t2i_qkv_attention_error_offset(int32_t B, int32_t Hq, int32_t Hkv) {
  if (B < 1 || B > FQ_MAX_ROWS || Hkv < 1 || Hq % Hkv) return 0;
  int cus = 0, dev = 0;
  if (fq_cus(&cus, &dev)) return 0;
  return fq_plan(cus, B, Hq, Hkv, (Hq + 2 * Hkv) * ATT_D).off_ctl + 2 * sizeof(unsigned);
}

extern "C" int t2i_qkv_attention(const uint16_t* x, int32_t B, const uint16_t* norm_weight, float eps,
                                 const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, int32_t K,
                                 int32_t group_size, const int32_t* positions, int32_t Hq, int32_t Hkv, int32_t D,
                                 const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* rope,
                                 int32_t rope_style, uint16_t* k_cache, uint16_t* v_cache, int32_t ctx_cap,
                                 uint16_t* ctx, void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !qweight || !qzeros || !scales || !positions || !q_norm || !k_norm || !rope || !k_cache || !v_cache ||
      !ctx)
    return fail(T2I_ERR_NULL, "fused qkv attention pointers must not be NULL");
  if (group_size != 128) return fail(T2I_ERR_GROUP, "group_size %d unsupported (only 128)", group_size);
  if (D != ATT_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (B < 1 || B > FQ_MAX_ROWS) return fail(T2I_ERR_SHAPE, "B=%d must be in [1, %d]", B, FQ_MAX_ROWS);
  if (Hkv < 1 || Hq < Hkv || Hq % Hkv || (Hq / Hkv != 1 && Hq / Hkv != 2))
    return fail(T2I_ERR_SHAPE, "Hq=%d Hkv=%d: 1 or 2 q heads per kv head", Hq, Hkv);
  if (K <= 0 || K % 128) return fail(T2I_ERR_SHAPE, "K=%d must be a positive multiple of 128", K);
  if (ctx_cap < 1) return fail(T2I_ERR_SHAPE, "ctx_cap=%d must be positive", ctx_cap);
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  if (!aligned16(x) || !aligned16(qweight) || !aligned16(scales) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(ctx) || (norm_weight && !aligned16(norm_weight)) || ((uintptr_t)qzeros & 3u))
    return fail(T2I_ERR_ALIGN, "fused qkv attention tensors must be 16-byte aligned");
  int cus = 0, dev = 0;
  int rc = fq_cus(&cus, &dev);
  if (rc) return rc;
  const int N = (Hq + 2 * Hkv) * ATT_D;
  const FqPlan pl = fq_plan(cus, B, Hq, Hkv, N);
  if (pl.U > pl.G) return fail(T2I_ERR_SHAPE, "B*Hkv=%d exceeds the %d workgroups of one launch", pl.U, pl.G);
  if (!workspace || workspace_bytes < pl.bytes)
    return fail(T2I_ERR_WORKSPACE, "workspace of %zu bytes required", pl.bytes);
  if (!aligned16(workspace)) return fail(T2I_ERR_ALIGN, "workspace must be 16-byte aligned");
  const int Q = Hq / Hkv;
  const bool norm = norm_weight != nullptr;
  {
    std::lock_guard<std::mutex> lock(g_fq_mu);
    FqDevice& d = g_fq_dev[dev];
    rc = Q == 2 ? (norm ? fq_setup<2, true>(dev, d) : fq_setup<2, false>(dev, d))
                : (norm ? fq_setup<1, true>(dev, d) : fq_setup<1, false>(dev, d));
    if (rc) return rc;
  }
  char* ws = reinterpret_cast<char*>(workspace);
  FqaParams p{};
  LinearParams& lp = p.lin;
  lp.x = x;
  lp.qw = reinterpret_cast<const uint32_t*>(qweight);
  lp.qz = reinterpret_cast<const uint32_t*>(qzeros);
  lp.sc = scales;
  lp.gamma = norm_weight;
  lp.eps = eps;
  lp.M = B; lp.K = K; lp.N = N;
  lp.ldx = K;
  lp.ldy = N;
  lp.chunks = K / 64;
  lp.epi = EPI_LL;
  lp.rt = 16;
  lp.ll = reinterpret_cast<unsigned long long*>(ws);
  p.pos = positions; p.qn = q_norm; p.kn = k_norm; p.rope = rope;
  p.kc = k_cache; p.vc = v_cache; p.out = ctx;
  p.st = reinterpret_cast<unsigned long long*>(ws + pl.off_st);
  p.ctl = reinterpret_cast<unsigned*>(ws + pl.off_ctl);
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.ctx_cap = ctx_cap; p.style = rope_style; p.S = pl.S; p.nb = N / 16;
  p.eps = eps;
  p.scale = (float)(1.0 / sqrt((double)D));
  void* args[] = {&p};
  const void* fn = Q == 2 ? (norm ? reinterpret_cast<const void*>(&fused_qkv_attention_kernel<2, true>)
                                  : reinterpret_cast<const void*>(&fused_qkv_attention_kernel<2, false>))
                          : (norm ? reinterpret_cast<const void*>(&fused_qkv_attention_kernel<1, true>)
                                  : reinterpret_cast<const void*>(&fused_qkv_attention_kernel<1, false>));
  hipError_t e = hipLaunchCooperativeKernel(fn, dim3(pl.G), dim3(FQ_THREADS), args, (unsigned)FQ_LDS_KV,
                                            reinterpret_cast<hipStream_t>(stream));
  return t2i_host::hip_status(e, "fused qkv attention launch");
}
