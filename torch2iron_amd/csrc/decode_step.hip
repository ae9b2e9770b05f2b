// The decode step's layers in one cooperative launch (gfx950): for every
// layer, RMSNorm + qkv projection, attention (q/k norm, RoPE, KV write), o_proj
// + residual, RMSNorm + gate/up + SwiGLU and down + residual, for all rows, as
// phases of one persistent grid of 16-wave workgroups, one per CU.
//
// Phases hand over through tagged words in the workspace, with no barrier: the
// qkv projection's values go out as 64-bit words (bf16 | 32-bit tag) that the
// attention items poll (attn_item.h); every other phase writes its rows as
// 32-bit words (bf16 | 16-bit tag), and a consumer reads its input rows, and its
// residual, as agent-coherent loads repeated until every word carries the
// producing layer's tag.  A producer never waits for its stores.  A workgroup
// requests its next tile's weights, which depend on nothing, before it reads
// its input, so the weight stream overlaps the hand-off; the K / V prefetch of
// a layer's attention item goes out before the layer's qkv projection reads
// its input.  No buffer is rewritten within a launch before everything that
// reads it is done.  Two buffers are reused by every layer:
//   * the qkv words: layer l + 1's are written once all of layer l's residual
//     stream exists, which needs every context row of layer l, which needs
//     every read of layer l's qkv words;
//   * the attention split states st ([B*Hkv][S-1][Q][D+2], written by splits
//     1 .. S-1 of each (b, h) item and read by its split 0, the merger): a
//     split of layer l + 1 writes its state only after it has read its q/k/v
//     words of layer l + 1 for row b, which exist only once row b's residual
//     stream of layer l exists, which needs row b's whole context row of layer
//     l (o_proj reads every head), which each merger of (b, h) writes only
//     after it has read every split state of layer l.  The states also carry
//     the layer's tag, so a merger never takes another layer's state: it would
//     wait instead, and a wait that gives up raises the error word.
//
// The linear phases run the decode linear's tiles (linear_phase, with
// linear_tile's chunk ranges, arithmetic and reduction order) on the plans
// plan_linear gives 16-wave workgroups: the standalone kernels take 8 waves
// where that is faster, so a phase's output matches t2i_w4a16_* on the same
// input up to the order of the fp32 partial sums (within one bf16 rounding).  The attention items are those of
// t2i_qkv_attention.  Layer 0 takes its input already normalised (the embedding
// gather fuses that RMSNorm); the residual stream comes in and goes out in x.
//
// Tags: a launch's tag base is the launch counter plus one (read by every
// workgroup at the start), and layer l's words carry base * L + l (its low 16
// bits in a 32-bit word).  The last workgroup to finish advances the launch
// counter.  Every wait is bounded and raises the error word instead of
// hanging, so the launch always ends.
#include <math.h>

#include <mutex>

#include "attn_item.h"
#include "t2i_common.h"
#include "w4a16_tile.h"

namespace t2i {

// Chunks a wave of each linear phase (straight schedules: a wave's chunks and
// their tagged input words all in registers, within the 128 a lane of a 16-wave
// workgroup): 2 (K <= 2048 at 16 waves), and 3 for the down projection (K <=
// 3072: Qwen3-0.6B's 3072).
constexpr int DS_CHUNKS = 2;
constexpr int DS_CHUNKS_DOWN = 3;

struct StepPhase {
  int tiles;   // column blocks x row tiles
  int cbs;     // column blocks
  int rt;      // rows per row tile
};

struct StepParams {
  const t2i_decode_layer* layers;   // [L], device memory
  int L;
  const uint16_t* xn0;              // layer 0's normalised input [B][H]
  uint16_t* x;                      // residual stream [B][H]: in before layer 0, out after the last
  const int32_t* pos;
  const uint16_t* rope;
  unsigned long long* ll;           // [B][Nqkv] tagged qkv words
  unsigned long long* st;           // attention split states
  uint32_t* ctx;                    // [L][B][Hq * D] tagged words
  uint32_t* xmid;                   // [L][B][H]     residual stream after attention, tagged words
  uint32_t* h;                      // [L][B][I]     SwiGLU output, tagged words
  uint32_t* xs;                     // [L - 1][B][H] residual stream between layers, tagged words
  unsigned* ctl;                    // [0] launch counter, [1] finished workgroups, [2] error word
  int B, H, I, Hq, Hkv, ctx_cap, style, S, U, Nqkv;
  float eps, scale;
  StepPhase qkv, o, gu, dn;
};

#ifdef T2I_STEP_TRACE
// Phase timestamps for timeline studies (builds with T2I_STEP_TRACE only):
// [workgroup][layer][8] of the 100 MHz wall clock, written by thread 0.
__device__ unsigned long long* g_step_trace;
#define STEP_TRACE(l, i)                                                                            \
  do {                                                                                              \
    if (threadIdx.x == 0 && g_step_trace)                                                           \
      g_step_trace[((size_t)blockIdx.x * p.L + (l)) * 8 + (i)] = wall_clock64();                    \
  } while (0)
#else
#define STEP_TRACE(l, i) \
  do {                   \
  } while (0)
#endif

template <int Q>
__global__ __launch_bounds__(AI_THREADS) void decode_step_kernel(const StepParams p) {
  constexpr int D = ATT_D;
  extern __shared__ u32x4 st_kv[];                    // prefetched K / V (attn_prefetch layout)
  __shared__ __align__(16) float s_red[16 * 8 * 64];  // the linear phases' reduction; the attention's wave states alias it
  __shared__ float s_ss[16 * 16];
  __shared__ __align__(16) uint16_t s_raw[(Q + 2) * D];
  __shared__ __align__(16) uint16_t s_q[Q * D];
  __shared__ __align__(16) uint16_t s_kv[2 * D];
  __shared__ float s_wm[AI_WAVES * Q], s_wl[AI_WAVES * Q];
  static_assert(AI_WAVES * Q * D <= 16 * 8 * 64, "the attention's wave states fit the reduction buffer");

  const int G = gridDim.x;
  const int wg = blockIdx.x;
  const uint32_t base = __hip_atomic_load(p.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  AttnArgs a{};
  a.ll = p.ll;
  a.ldll = p.Nqkv;
  a.pos = p.pos;
  a.rope = p.rope;
  a.st = p.st;
  a.ctl = p.ctl;
  a.B = p.B; a.Hq = p.Hq; a.Hkv = p.Hkv; a.ctx_cap = p.ctx_cap; a.style = p.style; a.S = p.S;
  a.eps = p.eps;
  a.scale = p.scale;
  const bool has_item = wg < p.U * p.S;
  const AttnItem it = attn_item(a, has_item ? wg : 0);
  const AttnSmem sm{s_raw, s_q, s_kv, s_wm, s_wl, s_red};
  const size_t bh = (size_t)p.B * p.H;

  for (int l = 0; l < p.L; ++l) {
    const t2i_decode_layer& w = p.layers[l];
    const uint32_t tag = base * (uint32_t)p.L + (uint32_t)l;
    const uint32_t tag16 = tag & 0xFFFFu, prev16 = (tag - 1u) & 0xFFFFu;   // this layer's, the last layer's
    const uint32_t* x_in = l == 0 ? nullptr : p.xs + (size_t)(l - 1) * bh;   // layer 0: p.x
    uint32_t* x_out = l == p.L - 1 ? nullptr : p.xs + (size_t)l * bh;        // last layer: p.x
    uint32_t* ctx = p.ctx + (size_t)l * p.B * p.Hq * D;
    uint32_t* xmid = p.xmid + (size_t)l * bh;
    uint32_t* hbuf = p.h + (size_t)l * p.B * p.I;
    a.tag = tag;
    a.kc = w.k_cache;
    a.vc = w.v_cache;
    a.qn = w.q_norm;
    a.kn = w.k_norm;
    a.out_ll = ctx;
    STEP_TRACE(l, 0);

    // ---- RMSNorm + qkv projection (64-bit tagged words) ----
    {
      LinearParams lp{};
      lp.x = p.xn0;           // layer 0
      lp.xll = x_in;          // later layers: the last layer's output words
      lp.xtag = prev16;
      lp.qw = reinterpret_cast<const uint32_t*>(w.qkv_qweight);
      lp.qz = reinterpret_cast<const uint32_t*>(w.qkv_qzeros);
      lp.sc = w.qkv_scales;
      lp.gamma = w.input_norm;
      lp.eps = p.eps;
      lp.M = p.B; lp.K = p.H; lp.N = p.Nqkv;
      lp.ldx = p.H; lp.ldy = p.Nqkv;
      lp.chunks = p.H / 64;
      lp.epi = EPI_LL;
      lp.rt = p.qkv.rt;
      lp.ll = p.ll;
      lp.tag = tag;
      lp.ctl = p.ctl;
      bool issued = false;
      auto prefetch = [&]() {
        if (issued) return;
        issued = true;
        if (has_item) attn_prefetch(a, it, st_kv);
      };
      for (int t = wg; t < p.qkv.tiles; t += G) {
        const int bx = t % p.qkv.cbs, bz = t / p.qkv.cbs;
        if (l == 0) linear_phase<1, 1, 16, 2, false, DS_CHUNKS>(lp, p.qkv.cbs, bx, bz, s_red, s_ss, prefetch);
        else linear_phase<1, 1, 16, 2, true, DS_CHUNKS>(lp, p.qkv.cbs, bx, bz, s_red, s_ss, prefetch);
        __syncthreads();
      }
      prefetch();   // no qkv tile: the prefetch still goes out
    }
    STEP_TRACE(l, 1);

    // ---- attention items (the context as tagged words) ----
    if (has_item) attn_run<Q, true>(a, it, st_kv, sm);
    __syncthreads();   // the wave states (aliasing s_red) are read before the next reduction
    STEP_TRACE(l, 2);

    const auto nothing = []() {};
    // ---- o_proj + residual ----
    {
      LinearParams lp{};
      lp.xll = ctx;
      lp.xtag = tag16;
      lp.residual = p.x;      // layer 0
      lp.rll = x_in;          // later layers
      lp.rtag = prev16;
      lp.yll = xmid;
      lp.tag = tag;
      lp.qw = reinterpret_cast<const uint32_t*>(w.o_qweight);
      lp.qz = reinterpret_cast<const uint32_t*>(w.o_qzeros);
      lp.sc = w.o_scales;
      lp.M = p.B; lp.K = p.Hq * D; lp.N = p.H;
      lp.ldx = p.Hq * D; lp.ldy = p.H;
      lp.chunks = p.Hq * D / 64;
      lp.epi = EPI_RESIDUAL;
      lp.rt = p.o.rt;
      lp.ctl = p.ctl;
      for (int t = wg; t < p.o.tiles; t += G) {
        linear_phase<1, 1, 16, 2, false, DS_CHUNKS>(lp, p.o.cbs, t % p.o.cbs, t / p.o.cbs, s_red, s_ss, nothing);
        __syncthreads();
      }
    }
    STEP_TRACE(l, 3);

    // ---- RMSNorm + gate/up + SwiGLU ----
    {
      LinearParams lp{};
      lp.xll = xmid;
      lp.xtag = tag16;
      lp.yll = hbuf;
      lp.tag = tag;
      lp.qw = reinterpret_cast<const uint32_t*>(w.gate_up_qweight);
      lp.qz = reinterpret_cast<const uint32_t*>(w.gate_up_qzeros);
      lp.sc = w.gate_up_scales;
      lp.gamma = w.post_attention_norm;
      lp.eps = p.eps;
      lp.M = p.B; lp.K = p.H; lp.N = 2 * p.I;
      lp.ldx = p.H; lp.ldy = p.I;
      lp.chunks = p.H / 64;
      lp.epi = EPI_SWIGLU;
      lp.rt = p.gu.rt;
      lp.ctl = p.ctl;
      for (int t = wg; t < p.gu.tiles; t += G) {
        linear_phase<1, 2, 16, 2, true, DS_CHUNKS>(lp, p.gu.cbs, t % p.gu.cbs, t / p.gu.cbs, s_red, s_ss, nothing);
        __syncthreads();
      }
    }
    STEP_TRACE(l, 4);

    // ---- down + residual ----
    {
      LinearParams lp{};
      lp.xll = hbuf;
      lp.xtag = tag16;
      lp.rll = xmid;
      lp.rtag = tag16;
      lp.yll = x_out;         // the last layer: bf16 rows into p.x
      lp.y0 = p.x;
      lp.tag = tag;
      lp.qw = reinterpret_cast<const uint32_t*>(w.down_qweight);
      lp.qz = reinterpret_cast<const uint32_t*>(w.down_qzeros);
      lp.sc = w.down_scales;
      lp.M = p.B; lp.K = p.I; lp.N = p.H;
      lp.ldx = p.I; lp.ldy = p.H;
      lp.chunks = p.I / 64;
      lp.epi = EPI_RESIDUAL;
      lp.rt = p.dn.rt;
      lp.ctl = p.ctl;
      for (int t = wg; t < p.dn.tiles; t += G) {
        linear_phase<1, 1, 16, 2, false, DS_CHUNKS_DOWN>(lp, p.dn.cbs, t % p.dn.cbs, t / p.dn.cbs, s_red, s_ss,
                                                         nothing);
        __syncthreads();
      }
    }
    STEP_TRACE(l, 5);
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
using t2i_host::LinearPlan;
using t2i_host::plan_linear;

constexpr int DS_MAX_DEVICES = 64;
constexpr int DS_MAX_ROWS = 16;

size_t ds_align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct DsDevice {
  int cus = 0;
  bool ready[2] = {false, false};   // [Q == 2]
  bool ok[2] = {false, false};
};
std::mutex g_ds_mu;
DsDevice g_ds_dev[DS_MAX_DEVICES];

int ds_device(int* cus, int* dev_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return t2i_host::hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= DS_MAX_DEVICES) return fail(T2I_ERR_VALUE, "device %d beyond %d", dev, DS_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_ds_mu);
  if (g_ds_dev[dev].cus == 0) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return t2i_host::hip_status(e, "CU count");
    g_ds_dev[dev].cus = n;
  }
  *cus = g_ds_dev[dev].cus;
  *dev_out = dev;
  return T2I_OK;
}

// One 16-wave workgroup must fit a CU (checked once per device and kernel).
template <int Q>
int ds_setup(DsDevice& d) {
  const int qi = Q == 2;
  if (!d.ready[qi]) {
    const void* fn = reinterpret_cast<const void*>(&decode_step_kernel<Q>);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)AI_LDS_KV);
    if (e != hipSuccess) return t2i_host::hip_status(e, "decode step LDS limit");
    int occ = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, AI_THREADS, AI_LDS_KV);
    if (e != hipSuccess) return t2i_host::hip_status(e, "decode step occupancy");
    d.ready[qi] = true;
    d.ok[qi] = occ >= 1;
  }
  return d.ok[qi] ? T2I_OK : fail(T2I_ERR_VALUE, "the decode step kernel does not fit one workgroup a CU");
}

struct DsPlan {
  bool ok;
  int G, S, U;
  StepPhase qkv, o, gu, dn;
  size_t off_st, off_ctx, off_xmid, off_h, off_xs, off_ctl, bytes;
};

// A phase plan the step kernel runs: plan_linear's choice must be one of its
// compiled tiles, with a straight schedule (at most `maxc` chunks a wave).
bool ds_phase(const LinearPlan& lp, int LW, int maxc, StepPhase* out) {
  if (lp.MT != 1 || lp.LW != LW || lp.W != 16 || lp.CK != 2) return false;
  if ((lp.chunks + 15) / 16 > maxc) return false;
  out->cbs = lp.cbs;
  out->rt = lp.rt;
  out->tiles = lp.cbs * lp.mz;
  return true;
}

DsPlan ds_plan(int cus, int B, int L, int H, int I, int Hq, int Hkv) {
  DsPlan pl{};
  pl.ok = false;
  if (B < 1 || B > DS_MAX_ROWS || L < 1 || Hkv < 1 || Hq % Hkv || (Hq / Hkv != 1 && Hq / Hkv != 2)) return pl;
  if (H <= 0 || H % 128 || I <= 0 || I % 128) return pl;
  const int D = ATT_D;
  const int Nqkv = (Hq + 2 * Hkv) * D;
  if (!ds_phase(plan_linear(B, H, Nqkv, false, true, true), 1, DS_CHUNKS, &pl.qkv)) return pl;
  if (!ds_phase(plan_linear(B, Hq * D, H, false, false, true), 1, DS_CHUNKS, &pl.o)) return pl;
  if (!ds_phase(plan_linear(B, H, 2 * I, true, true, true), 2, DS_CHUNKS, &pl.gu)) return pl;
  if (!ds_phase(plan_linear(B, I, H, false, false, true), 1, DS_CHUNKS_DOWN, &pl.dn)) return pl;
  pl.G = cus;
  pl.U = B * Hkv;
  if (pl.U > pl.G) return pl;
  pl.S = 1;
  while (pl.S < 16 && pl.U * pl.S * 2 <= pl.G) pl.S *= 2;
  const int Q = Hq / Hkv;
  size_t off = ds_align256((size_t)B * Nqkv * 8);   // tagged qkv words first
  pl.off_st = off;
  off += ds_align256((size_t)pl.U * (pl.S - 1) * Q * (D + 2) * 8);
  pl.off_ctx = off;
  off += ds_align256((size_t)L * B * Hq * D * 4);
  pl.off_xmid = off;
  off += ds_align256((size_t)L * B * H * 4);
  pl.off_h = off;
  off += ds_align256((size_t)L * B * I * 4);
  pl.off_xs = off;
  off += ds_align256((size_t)(L > 1 ? L - 1 : 1) * B * H * 4);
  pl.off_ctl = off;
  pl.bytes = off + 256;
  pl.ok = true;
  return pl;
}

}  // namespace

#ifdef T2I_STEP_TRACE
extern "C" int t2i_decode_step_trace(void* buf) {
  return t2i_host::hip_status(hipMemcpyToSymbol(HIP_SYMBOL(t2i::g_step_trace), &buf, sizeof(buf)),
                              "decode step trace buffer");
}
#endif

extern "C" size_t t2i_decode_step_workspace_bytes(int32_t B, int32_t n_layers, int32_t hidden, int32_t intermediate,
                                                  int32_t Hq, int32_t Hkv) {
  int cus = 0, dev = 0;
  if (ds_device(&cus, &dev)) return 0;
  const DsPlan pl = ds_plan(cus, B, n_layers, hidden, intermediate, Hq, Hkv);
  return pl.ok ? pl.bytes : 0;
}

extern "C" size_t t2i_decode_step_offset(int32_t B, int32_t n_layers, int32_t hidden, int32_t intermediate,
                                         int32_t Hq, int32_t Hkv, int32_t region) {
  int cus = 0, dev = 0;
  if (ds_device(&cus, &dev)) return 0;
  const DsPlan pl = ds_plan(cus, B, n_layers, hidden, intermediate, Hq, Hkv);
  if (!pl.ok) return 0;
  switch (region) {
    case 0: return pl.off_ctx;
    case 1: return pl.off_xmid;
    case 2: return pl.off_h;
    case 3: return pl.off_xs;
    case 4: return pl.off_ctl + 2 * sizeof(unsigned);
    default: return 0;
  }
}

extern "C" int t2i_decode_step(const t2i_decode_layer* layers, int32_t n_layers, const uint16_t* xn0, uint16_t* x,
                               int32_t B, int32_t hidden, int32_t intermediate, int32_t Hq, int32_t Hkv, int32_t D,
                               int32_t group_size, const int32_t* positions, const uint16_t* rope, int32_t rope_style,
                               int32_t ctx_cap, float eps, void* workspace, size_t workspace_bytes, void* stream) {
  if (!layers || !xn0 || !x || !positions || !rope) return fail(T2I_ERR_NULL, "decode step pointers must not be NULL");
  if (group_size != 128) return fail(T2I_ERR_GROUP, "group_size %d unsupported (only 128)", group_size);
  if (D != ATT_D) return fail(T2I_ERR_SHAPE, "head_dim %d unsupported (only 128)", D);
  if (ctx_cap < 1) return fail(T2I_ERR_SHAPE, "ctx_cap=%d must be positive", ctx_cap);
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  if (!aligned16(xn0) || !aligned16(x) || !aligned16(workspace))
    return fail(T2I_ERR_ALIGN, "decode step activations and workspace must be 16-byte aligned");
  int cus = 0, dev = 0;
  int rc = ds_device(&cus, &dev);
  if (rc) return rc;
  const DsPlan pl = ds_plan(cus, B, n_layers, hidden, intermediate, Hq, Hkv);
  if (!pl.ok)
    return fail(T2I_ERR_SHAPE,
                "decode step: B=%d hidden=%d intermediate=%d Hq=%d Hkv=%d has no one-launch plan (B <= 16, 1 or 2 q "
                "heads per kv head, the decode linear's 16-wave tiles)",
                B, hidden, intermediate, Hq, Hkv);
  if (!workspace || workspace_bytes < pl.bytes)
    return fail(T2I_ERR_WORKSPACE, "workspace of %zu bytes required", pl.bytes);
  const int Q = Hq / Hkv;
  {
    std::lock_guard<std::mutex> lock(g_ds_mu);
    rc = Q == 2 ? ds_setup<2>(g_ds_dev[dev]) : ds_setup<1>(g_ds_dev[dev]);
    if (rc) return rc;
  }
  char* ws = reinterpret_cast<char*>(workspace);
  StepParams p{};
  p.layers = layers;
  p.L = n_layers;
  p.xn0 = xn0;
  p.x = x;
  p.pos = positions;
  p.rope = rope;
  p.ll = reinterpret_cast<unsigned long long*>(ws);
  p.st = reinterpret_cast<unsigned long long*>(ws + pl.off_st);
  p.ctx = reinterpret_cast<uint32_t*>(ws + pl.off_ctx);
  p.xmid = reinterpret_cast<uint32_t*>(ws + pl.off_xmid);
  p.h = reinterpret_cast<uint32_t*>(ws + pl.off_h);
  p.xs = reinterpret_cast<uint32_t*>(ws + pl.off_xs);
  p.ctl = reinterpret_cast<unsigned*>(ws + pl.off_ctl);
  p.B = B; p.H = hidden; p.I = intermediate; p.Hq = Hq; p.Hkv = Hkv; p.ctx_cap = ctx_cap; p.style = rope_style;
  p.S = pl.S; p.U = pl.U; p.Nqkv = (Hq + 2 * Hkv) * D;
  p.eps = eps;
  p.scale = (float)(1.0 / sqrt((double)D));
  p.qkv = pl.qkv; p.o = pl.o; p.gu = pl.gu; p.dn = pl.dn;
  void* args[] = {&p};
  const void* fn = Q == 2 ? reinterpret_cast<const void*>(&decode_step_kernel<2>)
                          : reinterpret_cast<const void*>(&decode_step_kernel<1>);
  hipError_t e = hipLaunchCooperativeKernel(fn, dim3(pl.G), dim3(AI_THREADS), args, (unsigned)AI_LDS_KV,
                                            reinterpret_cast<hipStream_t>(stream));
  return t2i_host::hip_status(e, "decode step launch");
}
