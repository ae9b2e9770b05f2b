// Shared device helpers and host-side error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "t2i_hip.h"

namespace t2i {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// threadIdx.x behind an empty asm: values derived from it are recomputed where a
// phase uses them instead of being hoisted out of a persistent kernel's layer
// loop and held in registers across every other phase.
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// ---- bf16 / fp16 scalar conversions (bit patterns held in uint16/uint32) ----

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// fp32 -> bf16 with round to nearest even: one v_cvt_pk_bf16_f32 per pair of values.
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float(f32_to_bf16(f) << 16); }

// a.lo * b.lo + a.hi * b.hi + c over bf16 pairs (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// silu(g) = g / (1 + e^-g) in fp32 (libm exponential, IEEE division); the decode
// SwiGLU epilogue and the standalone SiLU-multiply round it to bf16 right after.
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// ---- attention helpers ----
constexpr int ATT_D = 128;   // head dimension of the attention kernels

__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

// Scores are kept in log2 units (scaled by log2 e), so every exponential is a
// single v_exp_f32.  2^(m - M) is the weight of a softmax state with running max m
// under a new max M; an empty state (m = -inf) weighs nothing.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float state_weight(float m, float M) { return m > -INFINITY ? exp2_fast(m - M) : 0.0f; }

// ---- 16-lane row reductions with DPP (a wave64 is four rows of 16 lanes) ----

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of each row; every lane of the row receives the sum.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

// ---- agent-coherent exchange between workgroups of one launch ----
// The L2 of each XCD is not coherent with the others.  A relaxed agent-scope
// store is written through to the device-coherent level (sc1) and a relaxed
// agent-scope load bypasses stale cached copies (sc1), so workgroups on
// different XCDs can hand data over without an L2 write-back fence: the
// producer stores with st_agent, waits for its stores (wait_stores) and then
// bumps an agent-scope counter; a consumer that observes the counter reads
// the data with ld_agent.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Agent-coherent activations of a launch that runs several dependent phases:
// the producer writes with st_coh16, waits for its stores and bumps an arrival
// counter; a consumer that has seen the counter reads with ld_coh32 / ld_coh128
// (relaxed agent-scope atomics: never served by a stale copy in its XCD's L2).
__device__ __forceinline__ void st_coh16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coh32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_coh64(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 ld_coh128(const void* p) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// The error word of a launch whose workgroups wait on each other (ctl[2]): a
// bounded wait that gives up raises it, and every other wait then gives up early.
constexpr int WAIT_SPIN = 1 << 18;   // polls before a wait gives up
__device__ __forceinline__ void ctl_fail(unsigned* ctl) {
  __hip_atomic_store(ctl + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ctl_failed(const unsigned* ctl) {
  return __hip_atomic_load(ctl + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
// true when the wait should give up (spin budget spent, or the error word up)
__device__ __forceinline__ bool wait_gives_up(int& spins, unsigned* ctl) {
  if (++spins >= WAIT_SPIN || ((spins & 255) == 0 && ctl_failed(ctl))) {
    ctl_fail(ctl);
    return true;
  }
  __builtin_amdgcn_s_sleep(1);
  return false;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  // combine the four rows: lanes l, l^16, l^32, l^48 hold row sums
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

}  // namespace t2i

// ---- host-side error helpers (defined in abi.hip) ----
namespace t2i_host {
int fail(int code, const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
}  // namespace t2i_host
