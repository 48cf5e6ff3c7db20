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

// Compute units of the current device (cached per device id).
static inline int mp_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = v;
  }
  return cache[dev];
}

// Measurement knobs: the environment variables that steer a kernel choice (MP_W4_*, MP_W8_*) are
// read only by a library compiled with -DMP_MEASUREMENT_KNOBS (python -m mindpipe_amd.build
// --knobs).  The default build ignores the environment, so every call takes the tested default.
static inline const char *mp_knob(const char *name) {
#ifdef MP_MEASUREMENT_KNOBS
  return getenv(name);
#else
  (void)name;
  return nullptr;
#endif
}

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

// fp32 -> bf16 -> fp32: the value PyTorch keeps after a bfloat16 op.
__device__ __forceinline__ float mp_rbf(float f) { return mp_bf2f(mp_f2bf(f)); }

// Rounding of a value to the dtype of the op that produced it (the reference's fake-quant
// path runs every op in the activation dtype).  kRoundNone keeps fp32.
enum mp_round_mode { kRoundNone = 0, kRoundF16 = 1, kRoundBF16 = 2 };
__device__ __forceinline__ float mp_round_mode_apply(float v, int mode) {
  const float h = mp_rh(v), b = mp_rbf(v);
  return mode == kRoundF16 ? h : (mode == kRoundBF16 ? b : v);
}
__host__ __device__ inline int mp_round_mode_of(int dtype) {
  return dtype == MP_F16 ? kRoundF16 : (dtype == MP_BF16 ? kRoundBF16 : kRoundNone);
}

// The fake per-token / per-channel int8 rule (quantize_*_absmax of the reference's
// fake_quant.py:10-31) in the input dtype: s = r(r(max(amax, 1e-5)) / 127), code =
// rint(r(v / s)), every op rounded once (r = mp_round_mode_apply).  In fp16 the codes stay
// within +-127; in bf16 (8-bit significand) r(v / s) can reach +-127.5 and the code +-128.
// int8 holds -128 but not +128, so a row is stored as (q, s) when no code is +128, as
// (-q, -s) when some code is +128 and none is -128 (the products q * s are the same bits),
// and with +128 clamped to 127 when both occur (the one case that departs from the reference
// values; it needs two entries of opposite sign within 0.4% of the row maximum).
__device__ __forceinline__ float mp_fake_scale(float amax, int mode) {
  float a = mp_round_mode_apply(amax, mode);
  if (a < 1e-5f) a = mp_round_mode_apply(1e-5f, mode);
  return mp_round_mode_apply(a / 127.0f, mode);
}
__device__ __forceinline__ float mp_fake_code(float v, float s, int mode) {
  return rintf(mp_round_mode_apply(v / s, mode));
}
// Sign of the stored row (+1 or -1) from the row's largest and smallest values.
__device__ __forceinline__ float mp_fake_row_sign(float vmax, float vmin, float s, int mode) {
  const bool pos128 = mp_fake_code(vmax, s, mode) >= 128.f;
  const bool neg128 = mp_fake_code(vmin, s, mode) <= -128.f;
  return (pos128 && !neg128) ? -1.f : 1.f;
}
// Stored int8 code of v for a row of sign sg (-1: negated row).
__device__ __forceinline__ int mp_fake_store(float v, float s, float sg, int mode) {
  const float q = sg * mp_fake_code(v, s, mode);
  return static_cast<int>(fminf(fmaxf(q, -128.f), 127.f));
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

// The same for bf16 values: round(round(silu(g)) * u) in bf16.
__device__ __forceinline__ uint16_t mp_swiglu_bf(float g, float u) {
  const float sg = mp_rbf(g / (1.0f + expf(-g)));
  return mp_f2bf(sg * u);
}

// SwiGLU of the grouped GEMM1 epilogue, h = silu(g) * u for the fp32 products g, u.  mode
// kRoundNone keeps fp32 (the runtime rule); kRoundF16 / kRoundBF16 round as the reference's
// fake path (fake_quant.py:184-185): gate and up as F.linear's output, silu(gate), and the
// product, each once.  mode is uniform, so the branch costs the runtime path nothing.
__device__ __forceinline__ float mp_swiglu_epi(float g, float u, int mode) {
#pragma clang fp contract(off)
  if (mode != kRoundNone) {
    const float gr = mp_round_mode_apply(g, mode), ur = mp_round_mode_apply(u, mode);
    const float sg = mp_round_mode_apply(__fdiv_rn(gr, 1.0f + expf(-gr)), mode);
    return mp_round_mode_apply(sg * ur, mode);
  }
  return __fdiv_rn(g, 1.0f + expf(-g)) * u;
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

// ---- per-row statistics of the int8 row quantizers (256-thread workgroups)
struct mp_rowstat {
  float amax, vmax, vmin;
  int bad;
};
__device__ __forceinline__ mp_rowstat mp_block_rowstat(mp_rowstat st, float (*red)[4], int *wbad) {
  const int tid = threadIdx.x;
  st.amax = mp_wave_max(st.amax);
  st.vmax = mp_wave_max(st.vmax);
  st.vmin = mp_wave_min(st.vmin);
  const int wb = __any(st.bad);
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = st.amax;
    red[1][tid >> 6] = st.vmax;
    red[2][tid >> 6] = st.vmin;
    wbad[tid >> 6] = wb;
  }
  __syncthreads();
  mp_rowstat o;
  o.amax = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  o.vmax = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  o.vmin = fminf(fminf(red[2][0], red[2][1]), fminf(red[2][2], red[2][3]));
  o.bad = wbad[0] | wbad[1] | wbad[2] | wbad[3];
  return o;
}

// Scale of a row and the sign of its stored codes.
template <int RULE>
__device__ __forceinline__ void mp_row_scale(const mp_rowstat &st, int mode, float min_scale, float &s, float &sg) {
  if (RULE == MP_SCALE_FP32) {
    s = st.amax / 127.0f;
    if (s < min_scale) s = min_scale;
    sg = 1.f;
  } else {
    s = mp_fake_scale(st.amax, mode);
    sg = mp_fake_row_sign(st.vmax, st.vmin, s, mode);
  }
}

template <int RULE>
__device__ __forceinline__ uint32_t mp_row_code(float v, float s, float sg, int mode) {
  if (RULE == MP_SCALE_FP32) {
    float r = (s == 0.f) ? 0.f : rintf(v / s);
    r = fminf(fmaxf(r, -127.f), 127.f);
    return static_cast<uint32_t>(static_cast<int>(r)) & 0xFFu;
  }
  return static_cast<uint32_t>(mp_fake_store(v, s, sg, mode)) & 0xFFu;
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
