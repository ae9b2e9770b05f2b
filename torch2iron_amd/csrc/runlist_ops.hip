// The standalone elementwise operators of the reference's batch-decode runlist,
// for gfx950:
//   * RMSNormRoPE         per-row weighted RMSNorm then RoPE (q or k heads);
//   * SiLUMul             silu(left) * right;
//   * ResidualAddRMSNorm  x <- x + update, then the weighted RMSNorm of the sum.
// The decode layer of this library folds each of them into the kernel next to
// it (the norms into the linears, the q/k norm and RoPE into the attention
// prologue, SiLU into the gate/up epilogue, the residual add into the o_proj and
// down epilogues).  These kernels let a runlist written for the NPU
// (quantized_qwen3/batch_decode_fused.py:426-539) run entry for entry.
//
// Rounding follows the reference runtime in bf16 compute
// (quantized_qwen3/model.py:172-196, 215-216, 322-327), at the points where the
// fused forms of this library round, so an entry produces the bits of the fused
// step it stands for:
//   RMSNormRoPE: inv = bf16(1/sqrt(mean(x^2) + eps)); n = bf16(bf16(x * inv) * g);
//                y0 = bf16(bf16(n0 * cos) + bf16(-n1 * sin)),
//                y1 = bf16(bf16(n1 * cos) + bf16(n0 * sin))  (the attention prologue's);
//   SiLUMul:     bf16(bf16(silu(g)) * u)                  (the SwiGLU epilogue's);
//   ResidualAddRMSNorm: s = bf16(x + u); y = t2i_rmsnorm(s)  (rmsnorm_kernel's order).
// Every kernel reads an element before any lane writes it and writes only the
// elements it read, so outputs may alias inputs (the runlist updates "x" and
// "queries" in place).
#include <math.h>

#include "t2i_common.h"

namespace t2i {

constexpr int RO_THREADS = 256;   // four waves, one row each (RMSNormRoPE)
constexpr int RA_THREADS = 256;   // one row per workgroup (ResidualAddRMSNorm)
constexpr int RA_MAX_CHUNKS = 4;  // 16-byte chunks per thread: H <= 8192
constexpr int SM_THREADS = 256;   // eight elements per thread (SiLUMul)

// Row r takes angle row r / rows_per_angle (the reference's q rows are
// [batch][head], one angle row per batch row).  style 0 rotates the pair
// (i, i + cols/2), style 1 the pair (2i, 2i + 1); pair i takes cos at angle
// column 2i and sin at 2i + 1.  NP pairs per lane: cols <= 128 NP.
template <int NP>
__global__ __launch_bounds__(RO_THREADS) void rmsnorm_rope_kernel(const uint16_t* x, int rows, int cols,
                                                                  const uint16_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ ang,
                                                                  int rows_per_angle, float eps, int style,
                                                                  uint16_t* y) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (RO_THREADS / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;   // wave-uniform
  const int half = cols >> 1;
  const uint16_t* src = x + (size_t)row * cols;
  const uint16_t* arow = ang + (size_t)(row / rows_per_angle) * cols;
  float a0[NP], a1[NP];
  int i0[NP], i1[NP];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int pi = lane + 64 * k;
    const int pc = pi < half ? pi : 0;   // clamped: every load in range
    i0[k] = style == 0 ? pc : 2 * pc;
    i1[k] = style == 0 ? pc + half : 2 * pc + 1;
    a0[k] = bf16_to_f32(src[i0[k]]);
    a1[k] = bf16_to_f32(src[i1[k]]);
    if (pi >= half) a0[k] = a1[k] = 0.0f;
    ss += a0[k] * a0[k] + a1[k] * a1[k];
  }
  ss = wave_sum(ss);
  const float inv = round_bf16(1.0f / sqrtf(ss / (float)cols + eps));
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int pi = lane + 64 * k;
    if (pi >= half) continue;
    const float n0 = round_bf16(round_bf16(a0[k] * inv) * bf16_to_f32(w[i0[k]]));
    const float n1 = round_bf16(round_bf16(a1[k] * inv) * bf16_to_f32(w[i1[k]]));
    const float cs = bf16_to_f32(arow[2 * pi]);
    const float sn = bf16_to_f32(arow[2 * pi + 1]);
    const float y0 = round_bf16(round_bf16(n0 * cs) + round_bf16(-n1 * sn));
    const float y1 = round_bf16(round_bf16(n1 * cs) + round_bf16(n0 * sn));
    y[(size_t)row * cols + i0[k]] = (uint16_t)f32_to_bf16(y0);
    y[(size_t)row * cols + i1[k]] = (uint16_t)f32_to_bf16(y1);
  }
}

__global__ __launch_bounds__(SM_THREADS) void silu_mul_kernel(const uint16_t* g_, const uint16_t* u_, size_t n8,
                                                            uint16_t* out) {
  const size_t i = (size_t)blockIdx.x * SM_THREADS + threadIdx.x;
  if (i >= n8) return;
  const u32x4 g = reinterpret_cast<const u32x4*>(g_)[i];
  const u32x4 u = reinterpret_cast<const u32x4*>(u_)[i];
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = round_bf16(silu_f32(bf16_lo(gw[j]))) * bf16_lo(uw[j]);
    const float hi = round_bf16(silu_f32(bf16_hi(gw[j]))) * bf16_hi(uw[j]);
    o[j] = pack_bf16x2(lo, hi);
  }
  reinterpret_cast<u32x4*>(out)[i] = u32x4{o[0], o[1], o[2], o[3]};
}

// One workgroup per row.  The sum of squares runs in rmsnorm_kernel's order
// (thread t: chunks t, t + 256, ..; wave_sum; the four wave partials in order),
// so y carries the bits t2i_rmsnorm gives for the summed row.
__global__ __launch_bounds__(RA_THREADS) void residual_add_rmsnorm_kernel(const uint16_t* x, const uint16_t* u,
                                                                        int H, const uint16_t* __restrict__ w,
                                                                        float eps, uint16_t* x_out,
                                                                        uint16_t* y) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int chunks = H / 8;
  u32x4 v[RA_MAX_CHUNKS];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < RA_MAX_CHUNKS; ++i) {
    const int ch = tid + i * RA_THREADS;
    if (ch < chunks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(x + (size_t)row * H + ch * 8);
      const u32x4 b = *reinterpret_cast<const u32x4*>(u + (size_t)row * H + ch * 8);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
      uint32_t s[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[j] = pack_bf16x2(bf16_lo(aw[j]) + bf16_lo(bw[j]), bf16_hi(aw[j]) + bf16_hi(bw[j]));
        const float lo = bf16_lo(s[j]), hi = bf16_hi(s[j]);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
      }
      v[i] = u32x4{s[0], s[1], s[2], s[3]};
    }
  }
  __shared__ float part[RA_THREADS / 64];
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < RA_THREADS / 64; ++i) total += part[i];
  const float inv = round_bf16(1.0f / sqrtf(total / (float)H + eps));
#pragma unroll
  for (int i = 0; i < RA_MAX_CHUNKS; ++i) {
    const int ch = tid + i * RA_THREADS;
    if (ch < chunks) {
      const u32x4 g = *reinterpret_cast<const u32x4*>(w + ch * 8);
      const uint32_t a[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      const uint32_t b[4] = {g.x, g.y, g.z, g.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = round_bf16(round_bf16(bf16_lo(a[j]) * inv) * bf16_lo(b[j]));
        const float hi = round_bf16(round_bf16(bf16_hi(a[j]) * inv) * bf16_hi(b[j]));
        o[j] = pack_bf16x2(lo, hi);
      }
      *reinterpret_cast<u32x4*>(x_out + (size_t)row * H + ch * 8) = v[i];
      *reinterpret_cast<u32x4*>(y + (size_t)row * H + ch * 8) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

}  // namespace t2i

using t2i_host::aligned16;
using t2i_host::fail;

extern "C" int t2i_rmsnorm_rope(const uint16_t* x, int32_t rows, int32_t cols, const uint16_t* weight,
                                const uint16_t* angles, int32_t angle_rows, float eps, int32_t rope_style,
                                uint16_t* y, void* stream) {
  if (!x || !weight || !angles || !y) return fail(T2I_ERR_NULL, "x, weight, angles and y must not be NULL");
  if (rows < 1 || cols < 2 || cols % 2 || cols > 1024)
    return fail(T2I_ERR_SHAPE, "rows=%d must be positive and cols=%d even in [2, 1024]", rows, cols);
  if (angle_rows < 1 || angle_rows > rows || rows % angle_rows)
    return fail(T2I_ERR_SHAPE, "angle_rows=%d must divide rows=%d", angle_rows, rows);
  if (rope_style != 0 && rope_style != 1) return fail(T2I_ERR_VALUE, "rope_style must be 0 or 1");
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  const int np = (cols / 2 + 63) / 64;
  const dim3 grid((rows + t2i::RO_THREADS / 64 - 1) / (t2i::RO_THREADS / 64));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rpa = rows / angle_rows;
  if (np == 1)
    hipLaunchKernelGGL(t2i::rmsnorm_rope_kernel<1>, grid, dim3(t2i::RO_THREADS), 0, s, x, rows, cols, weight, angles,
                       rpa, eps, rope_style, y);
  else if (np == 2)
    hipLaunchKernelGGL(t2i::rmsnorm_rope_kernel<2>, grid, dim3(t2i::RO_THREADS), 0, s, x, rows, cols, weight, angles,
                       rpa, eps, rope_style, y);
  else if (np <= 4)
    hipLaunchKernelGGL(t2i::rmsnorm_rope_kernel<4>, grid, dim3(t2i::RO_THREADS), 0, s, x, rows, cols, weight, angles,
                       rpa, eps, rope_style, y);
  else
    hipLaunchKernelGGL(t2i::rmsnorm_rope_kernel<8>, grid, dim3(t2i::RO_THREADS), 0, s, x, rows, cols, weight, angles,
                       rpa, eps, rope_style, y);
  return t2i_host::hip_status(hipGetLastError(), "rmsnorm_rope launch");
}

extern "C" int t2i_silu_mul(const uint16_t* left, const uint16_t* right, int64_t n, uint16_t* out, void* stream) {
  if (!left || !right || !out) return fail(T2I_ERR_NULL, "left, right and out must not be NULL");
  if (n < 8 || n % 8) return fail(T2I_ERR_SHAPE, "n=%lld must be a positive multiple of 8", (long long)n);
  if (!aligned16(left) || !aligned16(right) || !aligned16(out))
    return fail(T2I_ERR_ALIGN, "silu_mul pointers must be 16-byte aligned");
  const size_t n8 = (size_t)n / 8;
  const size_t blocks = (n8 + t2i::SM_THREADS - 1) / t2i::SM_THREADS;
  if (blocks > 0x7FFFFFFF) return fail(T2I_ERR_SHAPE, "n=%lld too large", (long long)n);
  hipLaunchKernelGGL(t2i::silu_mul_kernel, dim3((unsigned)blocks), dim3(t2i::SM_THREADS), 0,
                     reinterpret_cast<hipStream_t>(stream), left, right, n8, out);
  return t2i_host::hip_status(hipGetLastError(), "silu_mul launch");
}

extern "C" int t2i_residual_add_rmsnorm(const uint16_t* x, const uint16_t* update, int32_t M, int32_t H,
                                        const uint16_t* weight, float eps, uint16_t* x_out, uint16_t* y,
                                        void* stream) {
  if (!x || !update || !weight || !x_out || !y) return fail(T2I_ERR_NULL, "residual_add_rmsnorm pointers must not be NULL");
  if (M < 1) return fail(T2I_ERR_SHAPE, "M=%d must be positive", M);
  if (H < 8 || H % 8 || H > 8 * t2i::RA_THREADS * t2i::RA_MAX_CHUNKS)
    return fail(T2I_ERR_SHAPE, "H=%d must be a multiple of 8 in [8, %d]", H, 8 * t2i::RA_THREADS * t2i::RA_MAX_CHUNKS);
  if (!(eps > 0.0f)) return fail(T2I_ERR_VALUE, "eps must be positive");
  if (!aligned16(x) || !aligned16(update) || !aligned16(weight) || !aligned16(x_out) || !aligned16(y))
    return fail(T2I_ERR_ALIGN, "residual_add_rmsnorm pointers must be 16-byte aligned");
  hipLaunchKernelGGL(t2i::residual_add_rmsnorm_kernel, dim3(M), dim3(t2i::RA_THREADS), 0,
                     reinterpret_cast<hipStream_t>(stream), x, update, H, weight, eps, x_out, y);
  return t2i_host::hip_status(hipGetLastError(), "residual_add_rmsnorm launch");
}
