// Shared helpers for the gfx950 kernels of mindpipe_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/mindpipe_amd.h"

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef int i4_t __attribute__((ext_vector_type(4)));
typedef int i16_t __attribute__((ext_vector_type(16)));

#define MP_CHECK_LAUNCH()                      \
  do {                                         \
    if (hipGetLastError() != hipSuccess)       \
      return MP_ERR_HIP;                       \
  } while (0)

static inline bool mp_aligned(const void *p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

static inline int64_t mp_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- scalar conversions (round to nearest even everywhere)
__device__ __forceinline__ float mp_h2f(uint16_t b) {
  return __half2float(__ushort_as_half(b));
}
__device__ __forceinline__ uint16_t mp_f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}
// fp32 -> fp16 -> fp32: the value PyTorch keeps after a half op.
__device__ __forceinline__ float mp_rh(float f) { return __half2float(__float2half_rn(f)); }

__device__ __forceinline__ float mp_bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t mp_f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float mp_load_as_f32(const void *p, int64_t i, int dtype) {
  if (dtype == MP_F16) return mp_h2f(static_cast<const uint16_t *>(p)[i]);
  if (dtype == MP_BF16) return mp_bf2f(static_cast<const uint16_t *>(p)[i]);
  return static_cast<const float *>(p)[i];
}

__device__ __forceinline__ void mp_store_from_f32(void *p, int64_t i, int dtype, float v) {
  if (dtype == MP_F16) static_cast<uint16_t *>(p)[i] = mp_f2h(v);
  else if (dtype == MP_BF16) static_cast<uint16_t *>(p)[i] = mp_f2bf(v);
  else static_cast<float *>(p)[i] = v;
}

// 16 bytes of a row as floats: 8 values of a 16-bit dtype or 4 of fp32
template <int DT>
struct MpChunk16 {
  static constexpr int N = DT == MP_F32 ? 4 : 8;
};
template <int DT>
__device__ __forceinline__ void mp_chunk_to_f32(const uint4 v, float (&f)[MpChunk16<DT>::N]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (DT == MP_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xFFFFu), hi = static_cast<uint16_t>(w[i] >> 16);
      f[2 * i] = DT == MP_F16 ? mp_h2f(lo) : mp_bf2f(lo);
      f[2 * i + 1] = DT == MP_F16 ? mp_h2f(hi) : mp_bf2f(hi);
    }
  }
}
// SwiGLU of fp16 values g, u (given as floats): round(round(silu(g)) * u), the
// rounding of PyTorch's half ops (silu in fp32, rounded; the product rounded).
__device__ __forceinline__ uint16_t mp_swiglu_h(float g, float u) {
  const float sg = mp_rh(g / (1.0f + expf(-g)));
  return mp_f2h(sg * u);
}

// ---- wave64 reductions (DPP-backed shuffles)
__device__ __forceinline__ float mp_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float mp_wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

// Uniform-order float multiply/add that the compiler may not contract into an
// FMA: the W8A8 epilogue is specified as (acc * s_tok) * s_ch + bias with
// three separate roundings.
__device__ __forceinline__ float mp_mul(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float mp_add(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// Workgroup barrier that waits only for this wave's LDS traffic (lgkmcnt),
// not for outstanding global loads, so weight prefetches stay in flight
// across it.  The "memory" clobber keeps the compiler from moving LDS
// accesses across the barrier.
__device__ __forceinline__ void mp_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- raw buffer loads
// Buffer resource over [p, p + bytes) (gfx9 descriptor word 3: 32-bit data
// format); a load at an offset past `bytes` returns zeros.  The per-lane part of
// an address goes in voff, a wave-uniform part in soff (a scalar register: the
// caller guarantees uniformity, readfirstlane only tells the compiler).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mp_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 mp_buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  typedef unsigned int u4v __attribute__((ext_vector_type(4)));
  const u4v v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff),
                                                      __builtin_amdgcn_readfirstlane(static_cast<int>(soff)), 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ i4_t mp_buf_load16i(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(i4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                        r, static_cast<int>(voff), __builtin_amdgcn_readfirstlane(static_cast<int>(soff)), 0));
}
// Vector stores through a buffer descriptor: offsets at or past its size are dropped,
// so guarded stores need no branch.
__device__ __forceinline__ void mp_buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint4 v) {
  typedef unsigned int u4v __attribute__((ext_vector_type(4)));
  const u4v w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, static_cast<int>(voff), 0, 0);
}
__device__ __forceinline__ void mp_buf_store4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, static_cast<int>(voff), 0, 0);
}
__device__ __forceinline__ void mp_buf_store2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, static_cast<int>(voff), 0, 0);
}
__device__ __forceinline__ uint32_t mp_buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff),
                                              __builtin_amdgcn_readfirstlane(static_cast<int>(soff)), 0);
}

// LDS budget (bytes) for an activation chunk staged by the decode kernels.
constexpr int kMpXLdsBudget = 60 * 1024;
