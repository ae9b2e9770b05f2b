// HBM read ceiling for the linear's roofline: a kernel that only streams bytes.
//
// A W4A16 linear call moves 1-4 MB, so its rate is set by the launch and one
// memory round trip as much as by bandwidth.  This kernel reads the same number of
// bytes the same way (16-byte non-temporal loads, every load of a lane issued
// before any is used, 256-thread workgroups) and does nothing else: timed on the
// same byte counts and the same cold-buffer rotation, it gives what a launch of
// that size can reach on the machine, and on a large buffer the bulk streaming
// rate.  Each wave XORs its words and stores one word, so nothing is optimised
// away and the result can be checked.
#include "t2i_common.h"

namespace t2i {

constexpr int SR_THREADS = 256;

// wave XOR over 64 lanes (DPP within rows of 16, then across the four rows)
__device__ __forceinline__ uint32_t wave_xor(uint32_t v) {
  v ^= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v ^= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v ^= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  v ^= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);  // row_mirror
  v ^= (uint32_t)__shfl_xor((int)v, 16, 64);
  v ^= (uint32_t)__shfl_xor((int)v, 32, 64);
  return v;
}

// Workgroup g reads 16-byte words g * 256 * LPT + i * 256 + tid, i < LPT (a
// coalesced 4 KB per load instruction of the workgroup); words past n read as zero.
template <int LPT>
__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4* __restrict__ src, size_t n,
                                                                 uint32_t* __restrict__ out) {
  const size_t base = (size_t)blockIdx.x * SR_THREADS * LPT + threadIdx.x;
  u32x4 v[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) v[i] = __builtin_nontemporal_load(src + min(base + (size_t)i * SR_THREADS, n - 1));
  __builtin_amdgcn_sched_barrier(0);   // every load in flight before the first is used
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < LPT; ++i)
    if (base + (size_t)i * SR_THREADS < n) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  acc = wave_xor(acc);
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * (SR_THREADS / 64) + (threadIdx.x >> 6)] = acc;
}

}  // namespace t2i

namespace {

size_t sr_blocks(size_t bytes, int lpt) {
  const size_t words = bytes / 16;
  const size_t per = (size_t)t2i::SR_THREADS * lpt;
  return (words + per - 1) / per;
}

bool sr_lpt_ok(int lpt) { return lpt == 1 || lpt == 2 || lpt == 4 || lpt == 8; }

}  // namespace

extern "C" int64_t t2i_stream_read_out_words(size_t bytes, int32_t loads_per_thread) {
  if (!sr_lpt_ok(loads_per_thread) || bytes == 0 || bytes % 16) return 0;
  return (int64_t)(sr_blocks(bytes, loads_per_thread) * (t2i::SR_THREADS / 64));
}

extern "C" int t2i_stream_read(const void* src, size_t bytes, int32_t loads_per_thread, uint32_t* out,
                               void* stream) {
  using namespace t2i_host;
  if (!src || !out) return fail(T2I_ERR_NULL, "t2i_stream_read: src and out are required");
  if (!aligned16(src)) return fail(T2I_ERR_ALIGN, "t2i_stream_read: src must be 16-byte aligned");
  if (bytes == 0 || bytes % 16)
    return fail(T2I_ERR_SHAPE, "t2i_stream_read: bytes (%zu) must be a positive multiple of 16", bytes);
  if (!sr_lpt_ok(loads_per_thread))
    return fail(T2I_ERR_VALUE, "t2i_stream_read: loads_per_thread must be 1, 2, 4 or 8 (got %d)", loads_per_thread);
  const size_t blocks = sr_blocks(bytes, loads_per_thread);
  if (blocks > 0x1FFFFFFFu) return fail(T2I_ERR_SHAPE, "t2i_stream_read: %zu bytes is too many", bytes);
  const auto* s = static_cast<const t2i::u32x4*>(src);
  const size_t n = bytes / 16;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(t2i::SR_THREADS);
  switch (loads_per_thread) {
    case 1: hipLaunchKernelGGL(t2i::stream_read_kernel<1>, grid, block, 0, st, s, n, out); break;
    case 2: hipLaunchKernelGGL(t2i::stream_read_kernel<2>, grid, block, 0, st, s, n, out); break;
    case 4: hipLaunchKernelGGL(t2i::stream_read_kernel<4>, grid, block, 0, st, s, n, out); break;
    default: hipLaunchKernelGGL(t2i::stream_read_kernel<8>, grid, block, 0, st, s, n, out); break;
  }
  return hip_status(hipGetLastError(), "t2i_stream_read launch");
}
