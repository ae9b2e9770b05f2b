// W4A16 group-128 linear for gfx950: y[M, N] = x[M, K] . W^T, 1 <= M <= 64.
//
// Weights stay in the AutoGPTQ layout.  One int32 word of qweight holds the
// 8 consecutive k of one column, which is exactly the 8 bf16 values one lane
// feeds to v_mfma_f32_16x16x32_bf16 as its B operand, so weights go from a
// 128-bit global load straight into registers with no LDS staging:
//
//   * lane (c = lane % 16, r = lane / 16) loads, for qweight row 4*kstep + r,
//     LW consecutive words at columns ncol .. ncol+LW-1 (ncol = n0 + LW*c);
//     word t feeds n-tile t, whose MFMA column c is output column ncol + t;
//   * a nibble becomes bf16 (128 + q) with one AND-OR against 0x43004300
//     (bf16 128.0 has a unit of least precision of exactly 1), four
//     AND-ORs and three shifts per word, in k order (0,4,1,5,2,6,3,7);
//   * the activation operand is permuted into the same k order (the
//     contraction only needs A and B to agree on it);
//   * per group of 128 k the MFMA sums acc = sum x*(128+q) and, with an
//     all-ones B, xs = sum x; the group's exact contribution is then
//     s * (acc - (128 + z) * xs), accumulated in fp32 (scale after dot).
//
// A workgroup of W waves shares one column block and splits the block's K
// range between its waves; their fp32 sums meet in LDS.  When there are too
// few column blocks to fill the GPU, `splits` workgroups share a column block
// and the last one to finish (atomic counter in the workspace) adds the fp32
// partials in split order, so the result does not depend on timing.
#include "t2i_common.h"

namespace t2i {

constexpr int GS = 128;             // quantisation group along K
constexpr int KS = GS / 32;         // MFMA k-steps per group
constexpr int WAVES = 4;            // waves per workgroup
constexpr uint32_t MAGIC = 0x43004300u;  // two bf16 128.0
constexpr uint32_t NIB2 = 0x000F000Fu;

enum : int { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_PAIRED = 3 };

struct LinearParams {
  const uint16_t* x;
  const uint32_t* qw;
  const uint32_t* qz;
  const uint16_t* sc;
  const uint16_t* residual;
  uint16_t* y0;
  uint16_t* y1;
  float* partial;       // [splits][M][N] fp32
  uint32_t* counters;   // one per column block
  int M, K, N;
  int ldx, ldy;
  int n_groups;         // K / GS
  int gpw;              // groups per wave
  int splits;           // workgroups per column block
};

__device__ __forceinline__ bf16x8 b_operand(uint32_t w) {
  u32x4 d;
  d.x = (w & NIB2) | MAGIC;           // (k0, k4)
  d.y = ((w >> 4) & NIB2) | MAGIC;    // (k1, k5)
  d.z = ((w >> 8) & NIB2) | MAGIC;    // (k2, k6)
  d.w = ((w >> 12) & NIB2) | MAGIC;   // (k3, k7)
  return __builtin_bit_cast(bf16x8, d);
}

// v holds bf16 pairs (k0,k1) (k2,k3) (k4,k5) (k6,k7); reorder to match b_operand.
__device__ __forceinline__ bf16x8 a_operand(u32x4 v) {
  u32x4 d;
  d.x = (v.x & 0xFFFFu) | (v.z << 16);
  d.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
  d.z = (v.y & 0xFFFFu) | (v.w << 16);
  d.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
  return __builtin_bit_cast(bf16x8, d);
}

__device__ __forceinline__ bf16x8 ones_operand() {
  u32x4 d = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  return __builtin_bit_cast(bf16x8, d);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

template <int LW>
__device__ __forceinline__ void load_words(const uint32_t* src, uint32_t (&w)[LW]) {
  if constexpr (LW == 8) {
    u32x4 a = *reinterpret_cast<const u32x4*>(src);
    u32x4 b = *reinterpret_cast<const u32x4*>(src + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    u32x4 a = *reinterpret_cast<const u32x4*>(src);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  }
}

template <int LW>
__device__ __forceinline__ void load_scales(const uint16_t* src, float (&s)[LW]) {
  if constexpr (LW == 8) {
    u32x4 a = *reinterpret_cast<const u32x4*>(src);
    uint32_t v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { s[2 * i] = f16_to_f32(v[i] & 0xFFFFu); s[2 * i + 1] = f16_to_f32(v[i] >> 16); }
  } else {
    u32x2 a = *reinterpret_cast<const u32x2*>(src);
    s[0] = f16_to_f32(a.x & 0xFFFFu); s[1] = f16_to_f32(a.x >> 16);
    s[2] = f16_to_f32(a.y & 0xFFFFu); s[3] = f16_to_f32(a.y >> 16);
  }
}

template <int MT, int LW, int EPI>
__global__ __launch_bounds__(64 * WAVES) void w4a16_mfma_kernel(const LinearParams p) {
  constexpr int NT = LW;
  constexpr int E = MT * NT * 4;      // fp32 results per lane
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int r = lane >> 4;
  const int ncol = blockIdx.x * (16 * LW) + LW * c;
  const int g_begin = (blockIdx.y * WAVES + wave) * p.gpw;
  const int g_end = min(g_begin + p.gpw, p.n_groups);

  float total[MT][NT][4];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) total[mi][t][i] = 0.0f;

  const bf16x8 ones = ones_operand();

  for (int g = g_begin; g < g_end; ++g) {
    uint32_t wv[KS][LW];
    u32x4 xv[MT][KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint32_t* src = p.qw + (size_t)(g * (GS / 8) + ks * 4 + r) * p.N + ncol;
      load_words<LW>(src, wv[ks]);
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      const int m = mi * 16 + c;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (m < p.M) {
          xv[mi][ks] = *reinterpret_cast<const u32x4*>(p.x + (size_t)m * p.ldx + g * GS + ks * 32 + r * 8);
        } else {
          xv[mi][ks] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    float s[LW];
    load_scales<LW>(p.sc + (size_t)g * p.N + ncol, s);
    const uint32_t zw = p.qz[(size_t)g * (p.N >> 3) + (ncol >> 3)] >> ((ncol & 7) * 4);

    f32x4 acc[MT][NT];
    f32x4 xs[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
      xs[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mi][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 bop[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) bop[t] = b_operand(wv[ks][t]);
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        const bf16x8 a = a_operand(xv[mi][ks]);
        xs[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, xs[mi], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          acc[mi][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bop[t], acc[mi][t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float zb = -(float)(128 + 1 + ((zw >> (4 * t)) & 0xFu));
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          total[mi][t][i] = fmaf(s[t], fmaf(zb, xs[mi][i], acc[mi][t][i]), total[mi][t][i]);
    }
  }

  // ---- reduce the waves of this workgroup in LDS (fixed order) ----
  __shared__ float red[(WAVES - 1) * E * 64];
  if (wave > 0) {
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[(((wave - 1) * E) + (mi * NT + t) * 4 + i) * 64 + lane] = total[mi][t][i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < WAVES; ++w)
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          total[mi][t][i] += red[(((w - 1) * E) + (mi * NT + t) * 4 + i) * 64 + lane];

  // ---- cross-workgroup split-K: last finisher sums partials in split order ----
  if (p.splits > 1) {
    float* part = p.partial + (size_t)blockIdx.y * p.M * p.N;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mi * 16 + r * 4 + i;
        if (m < p.M) {
          float* dst = part + (size_t)m * p.N + ncol;
#pragma unroll
          for (int t = 0; t < NT; t += 4)
            *reinterpret_cast<f32x4*>(dst + t) =
                f32x4{total[mi][t][i], total[mi][t + 1][i], total[mi][t + 2][i], total[mi][t + 3][i]};
        }
      }
    __threadfence();
    uint32_t prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(&p.counters[blockIdx.x], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev != (uint32_t)(p.splits - 1)) return;
    __threadfence();
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) total[mi][t][i] = 0.0f;
    for (int sp = 0; sp < p.splits; ++sp) {
      const float* src = p.partial + (size_t)sp * p.M * p.N;
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mi * 16 + r * 4 + i;
          if (m < p.M) {
            const float* s4 = src + (size_t)m * p.N + ncol;
#pragma unroll
            for (int t = 0; t < NT; t += 4) {
              f32x4 v = *reinterpret_cast<const f32x4*>(s4 + t);
              total[mi][t][i] += v.x; total[mi][t + 1][i] += v.y;
              total[mi][t + 2][i] += v.z; total[mi][t + 3][i] += v.w;
            }
          }
        }
    }
    if (lane == 0) __hip_atomic_store(&p.counters[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue (C layout: lane holds rows mi*16 + 4r + i, columns ncol .. ncol+LW-1) ----
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = mi * 16 + r * 4 + i;
      if (m >= p.M) continue;
      if constexpr (EPI == EPI_STORE || EPI == EPI_RESIDUAL) {
        uint32_t packed[LW / 2];
        if constexpr (EPI == EPI_RESIDUAL) {
          const uint16_t* res = p.residual + (size_t)m * p.ldy + ncol;
          uint32_t rv[LW / 2];
          if constexpr (LW == 8) {
            u32x4 a = *reinterpret_cast<const u32x4*>(res);
            rv[0] = a.x; rv[1] = a.y; rv[2] = a.z; rv[3] = a.w;
          } else {
            u32x2 a = *reinterpret_cast<const u32x2*>(res);
            rv[0] = a.x; rv[1] = a.y;
          }
#pragma unroll
          for (int j = 0; j < LW / 2; ++j)
            packed[j] = pack_bf16x2(round_bf16(total[mi][2 * j][i]) + bf16_lo(rv[j]),
                                    round_bf16(total[mi][2 * j + 1][i]) + bf16_hi(rv[j]));
        } else {
#pragma unroll
          for (int j = 0; j < LW / 2; ++j)
            packed[j] = pack_bf16x2(total[mi][2 * j][i], total[mi][2 * j + 1][i]);
        }
        uint16_t* dst = p.y0 + (size_t)m * p.ldy + ncol;
        if constexpr (LW == 8) {
          *reinterpret_cast<u32x4*>(dst) = u32x4{packed[0], packed[1], packed[2], packed[3]};
        } else {
          *reinterpret_cast<u32x2*>(dst) = u32x2{packed[0], packed[1]};
        }
      } else {
        // fused columns 4j+e = gate 2j+e, 4j+2+e = up 2j+e
        uint32_t out0[LW / 4], out1[LW / 4];
#pragma unroll
        for (int j = 0; j < LW / 4; ++j) {
          const float g0 = round_bf16(total[mi][4 * j][i]);
          const float g1 = round_bf16(total[mi][4 * j + 1][i]);
          const float u0 = round_bf16(total[mi][4 * j + 2][i]);
          const float u1 = round_bf16(total[mi][4 * j + 3][i]);
          if constexpr (EPI == EPI_SWIGLU) {
            out0[j] = pack_bf16x2(round_bf16(silu_f32(g0)) * u0, round_bf16(silu_f32(g1)) * u1);
          } else {
            out0[j] = pack_bf16x2(g0, g1);
            out1[j] = pack_bf16x2(u0, u1);
          }
        }
        const size_t off = (size_t)m * p.ldy + (ncol >> 1);
        if constexpr (LW == 8) {
          *reinterpret_cast<u32x2*>(p.y0 + off) = u32x2{out0[0], out0[1]};
          if constexpr (EPI == EPI_PAIRED) *reinterpret_cast<u32x2*>(p.y1 + off) = u32x2{out1[0], out1[1]};
        } else {
          *reinterpret_cast<uint32_t*>(p.y0 + off) = out0[0];
          if constexpr (EPI == EPI_PAIRED) *reinterpret_cast<uint32_t*>(p.y1 + off) = out1[0];
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
namespace {

using namespace t2i;
using t2i_host::aligned16;
using t2i_host::fail;

struct Plan {
  int MT, LW, cbs, gpw, splits;
  size_t ws_bytes;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Tile / split choice.  Column blocks of 16*LW columns; each workgroup's four
// waves take consecutive groups of K; `splits` workgroups share a column block
// when there are too few column blocks to give every CU work.
Plan plan_linear(int M, int K, int N, bool need_lw8_or_4) {
  (void)need_lw8_or_4;
  Plan pl{};
  pl.MT = (M + 15) / 16;
  if (pl.MT == 3) pl.MT = 4;
  pl.LW = (pl.MT == 1 && N % 128 == 0) ? 8 : 4;
  pl.cbs = N / (16 * pl.LW);
  const int G = K / GS;
  const int target_wgs = 512;
  int max_splits = (G + WAVES - 1) / WAVES;
  int splits = (target_wgs + pl.cbs - 1) / pl.cbs;
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  int gpw = (G + splits * WAVES - 1) / (splits * WAVES);
  splits = (G + gpw * WAVES - 1) / (gpw * WAVES);
  pl.gpw = gpw;
  pl.splits = splits;
  pl.ws_bytes = splits > 1 ? align256((size_t)pl.cbs * 4) + (size_t)splits * M * N * 4 : 0;
  return pl;
}

template <int MT, int LW, int EPI>
hipError_t launch_t(const LinearParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((w4a16_mfma_kernel<MT, LW, EPI>), grid, dim3(64 * WAVES), 0, s, p);
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_epi(const Plan& pl, const LinearParams& p, hipStream_t s) {
  dim3 grid(pl.cbs, pl.splits);
  if (pl.LW == 8) {
    if (pl.MT == 1) return launch_t<1, 8, EPI>(p, grid, s);
  } else {
    if (pl.MT == 1) return launch_t<1, 4, EPI>(p, grid, s);
    if (pl.MT == 2) return launch_t<2, 4, EPI>(p, grid, s);
    if (pl.MT == 4) return launch_t<4, 4, EPI>(p, grid, s);
  }
  return hipErrorInvalidValue;
}

int check_weights(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  int K, int N, int group_size) {
  if (!qweight || !qzeros || !scales) return fail(T2I_ERR_NULL, "qweight/qzeros/scales must not be NULL");
  if (group_size != GS) return fail(T2I_ERR_GROUP, "group_size %d unsupported (only 128)", group_size);
  if (K <= 0 || K % GS) return fail(T2I_ERR_SHAPE, "K=%d must be a positive multiple of 128", K);
  if (N <= 0 || N % 64) return fail(T2I_ERR_SHAPE, "N=%d must be a positive multiple of 64", N);
  if (!aligned16(qweight) || !aligned16(scales)) return fail(T2I_ERR_ALIGN, "qweight/scales must be 16-byte aligned");
  if (((uintptr_t)qzeros & 3u) != 0) return fail(T2I_ERR_ALIGN, "qzeros must be 4-byte aligned");
  return T2I_OK;
}

int run_linear(int epi, const uint16_t* x, int M, const int32_t* qweight, const int32_t* qzeros,
               const uint16_t* scales, int K, int N, int group_size, const uint16_t* residual,
               uint16_t* y0, uint16_t* y1, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_weights(qweight, qzeros, scales, K, N, group_size);
  if (rc) return rc;
  if (!x || !y0) return fail(T2I_ERR_NULL, "x and y must not be NULL");
  if (epi == EPI_PAIRED && !y1) return fail(T2I_ERR_NULL, "y1 must not be NULL when swiglu == 0");
  if (epi == EPI_RESIDUAL && !residual) return fail(T2I_ERR_NULL, "residual must not be NULL");
  if (M < 1 || M > 64) return fail(T2I_ERR_SHAPE, "M=%d must be in [1, 64]", M);
  if (!aligned16(x) || !aligned16(y0) || (y1 && !aligned16(y1)) || (residual && !aligned16(residual)))
    return fail(T2I_ERR_ALIGN, "activation pointers must be 16-byte aligned");
  if ((epi == EPI_SWIGLU || epi == EPI_PAIRED) && N % 128)
    return fail(T2I_ERR_SHAPE, "gate/up N=%d must be a multiple of 128", N);
  const Plan pl = plan_linear(M, K, N, false);
  if (pl.ws_bytes) {
    if (!ws) return fail(T2I_ERR_WORKSPACE, "workspace of %zu bytes required", pl.ws_bytes);
    if (ws_bytes < pl.ws_bytes) return fail(T2I_ERR_WORKSPACE, "workspace %zu < required %zu", ws_bytes, pl.ws_bytes);
    if (!aligned16(ws)) return fail(T2I_ERR_ALIGN, "workspace must be 16-byte aligned");
  }
  LinearParams p{};
  p.x = x;
  p.qw = reinterpret_cast<const uint32_t*>(qweight);
  p.qz = reinterpret_cast<const uint32_t*>(qzeros);
  p.sc = scales;
  p.residual = residual;
  p.y0 = y0;
  p.y1 = y1;
  p.counters = reinterpret_cast<uint32_t*>(ws);
  p.partial = ws ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + align256((size_t)pl.cbs * 4)) : nullptr;
  p.M = M; p.K = K; p.N = N;
  p.ldx = K;
  p.ldy = (epi == EPI_SWIGLU || epi == EPI_PAIRED) ? N / 2 : N;
  p.n_groups = K / GS;
  p.gpw = pl.gpw;
  p.splits = pl.splits;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (epi) {
    case EPI_STORE: e = launch_epi<EPI_STORE>(pl, p, s); break;
    case EPI_RESIDUAL: e = launch_epi<EPI_RESIDUAL>(pl, p, s); break;
    case EPI_SWIGLU: e = launch_epi<EPI_SWIGLU>(pl, p, s); break;
    default: e = launch_epi<EPI_PAIRED>(pl, p, s); break;
  }
  return t2i_host::hip_status(e, "w4a16 linear launch");
}

}  // namespace

extern "C" size_t t2i_w4a16_linear_workspace_bytes(int32_t M, int32_t K, int32_t N) {
  if (M < 1 || M > 64 || K <= 0 || K % GS || N <= 0 || N % 64) return 0;
  return plan_linear(M, K, N, false).ws_bytes;
}

extern "C" size_t t2i_w4a16_gate_up_workspace_bytes(int32_t M, int32_t K, int32_t N) {
  return t2i_w4a16_linear_workspace_bytes(M, K, N);
}

extern "C" int t2i_w4a16_linear(const uint16_t* x, int32_t M, const int32_t* qweight,
                                const int32_t* qzeros, const uint16_t* scales, int32_t K,
                                int32_t N, int32_t group_size, const uint16_t* residual,
                                uint16_t* y, void* workspace, size_t workspace_bytes,
                                void* stream) {
  return run_linear(residual ? EPI_RESIDUAL : EPI_STORE, x, M, qweight, qzeros, scales, K, N,
                    group_size, residual, y, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int t2i_w4a16_gate_up(const uint16_t* x, int32_t M, const int32_t* qweight,
                                 const int32_t* qzeros, const uint16_t* scales, int32_t K,
                                 int32_t N, int32_t group_size, int32_t swiglu, uint16_t* y0,
                                 uint16_t* y1, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return run_linear(swiglu ? EPI_SWIGLU : EPI_PAIRED, x, M, qweight, qzeros, scales, K, N,
                    group_size, nullptr, y0, y1, workspace, workspace_bytes, stream);
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
