// The front of the decode layer in one cooperative launch (gfx950): input
// RMSNorm + fused q|k|v projection, then GQA decode attention with q/k RMSNorm,
// RoPE and the KV-cache write of the current token.
//
// One 16-wave workgroup per CU, all co-resident (cooperative launch).  Every
// workgroup first computes one 16-column block of the qkv projection for all
// rows (the decode linear's 16-wave tile: t2i_w4a16_rmsnorm_linear's arithmetic,
// whose standalone plan may split K over 8 waves instead, so the two agree up to
// the order of the fp32 partial sums) and sends each value out as a tagged
// 64-bit word; it then runs one
// (sequence, kv head, context split) attention item on those words
// (attn_item.h).  The item's first K / V slots are issued into LDS right after
// the projection's first loads, so the context stream overlaps the projection.
//
// Tags: the workspace holds a launch counter; a launch's tag is the counter
// value plus one, read by every workgroup at the start, and the last workgroup
// to finish advances the counter.  A word from an earlier launch therefore
// never carries the current tag (the zero-filled workspace carries tag 0).
// Every wait is bounded: a wait that gives up raises the workspace's error
// word and the workgroup carries on, so the launch always ends.
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "attn_item.h"
#include "t2i_common.h"
#include "w4a16_tile.h"

namespace t2i {

struct FqaParams {
  LinearParams lin;             // the qkv projection, EPI_LL into lin.ll [B][N]
  AttnArgs att;                 // the attention items (att.ll = lin.ll)
  unsigned* ctl;                // [0] launch counter, [1] finished workgroups, [2] error word
  int nb;                       // qkv column blocks
};

template <int Q, bool NORM>
__global__ __launch_bounds__(AI_THREADS) void fused_qkv_attention_kernel(const FqaParams p) {
  constexpr int D = ATT_D;
  extern __shared__ u32x4 fq_kv[];   // prefetched K / V: [wave][AI_PF][K, V][64 lanes]
  __shared__ __align__(16) uint16_t s_raw[(Q + 2) * D];
  __shared__ __align__(16) uint16_t s_q[Q * D];
  __shared__ __align__(16) uint16_t s_kv[2 * D];
  __shared__ float s_wm[AI_WAVES * Q], s_wl[AI_WAVES * Q];
  __shared__ float s_wacc[AI_WAVES * Q * D];

  const int G = gridDim.x;
  const int wg = blockIdx.x;
  const uint32_t tag = __hip_atomic_load(p.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  AttnArgs a = p.att;
  a.tag = tag;

  // this workgroup's attention item: (sequence b, kv head h, split s); past the
  // last item a workgroup only takes part in the projection
  const bool has_item = wg < p.att.B * p.att.Hkv * p.att.S;
  const AttnItem it = attn_item(a, has_item ? wg : 0);
  // the item's first slots go straight into LDS once the projection's first
  // loads are out (loads complete in issue order)
  auto prefetch = [&]() {
    if (has_item) attn_prefetch(a, it, fq_kv);
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

  // ---- phase 2: the attention item ----
  if (has_item) {
    const AttnSmem sm{s_raw, s_q, s_kv, s_wm, s_wl, s_wacc};
    attn_run<Q, false>(a, it, fq_kv, sm);
  }

  // ---- the last workgroup to finish advances the launch counter ----
  __syncthreads();
  if (threadIdx.x == 0) {
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
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)AI_LDS_KV);
  if (e != hipSuccess) return t2i_host::hip_status(e, "fused kernel LDS limit");
  int occ = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(
                                                         &fused_qkv_attention_kernel<Q, NORM>),
                                                   AI_THREADS, AI_LDS_KV);
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
  AttnArgs& a = p.att;
  a.ll = lp.ll;
  a.ldll = N;
  a.pos = positions; a.qn = q_norm; a.kn = k_norm; a.rope = rope;
  a.kc = k_cache; a.vc = v_cache; a.out = ctx;
  a.st = reinterpret_cast<unsigned long long*>(ws + pl.off_st);
  p.ctl = reinterpret_cast<unsigned*>(ws + pl.off_ctl);
  a.ctl = p.ctl;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.ctx_cap = ctx_cap; a.style = rope_style; a.S = pl.S;
  a.eps = eps;
  a.scale = (float)(1.0 / sqrt((double)D));
  p.nb = N / 16;
  void* args[] = {&p};
  const void* fn = Q == 2 ? (norm ? reinterpret_cast<const void*>(&fused_qkv_attention_kernel<2, true>)
                                  : reinterpret_cast<const void*>(&fused_qkv_attention_kernel<2, false>))
                          : (norm ? reinterpret_cast<const void*>(&fused_qkv_attention_kernel<1, true>)
                                  : reinterpret_cast<const void*>(&fused_qkv_attention_kernel<1, false>));
  hipError_t e = hipLaunchCooperativeKernel(fn, dim3(pl.G), dim3(AI_THREADS), args, (unsigned)AI_LDS_KV,
                                            reinterpret_cast<hipStream_t>(stream));
  return t2i_host::hip_status(e, "fused qkv attention launch");
}
