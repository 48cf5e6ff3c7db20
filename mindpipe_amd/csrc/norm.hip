// Fused residual add + RMSNorm + per-token dynamic int8 quantisation: the step
// in front of every quantized linear of a decoder layer.
//
//   sum      = float(x) + float(residual)               (fp32)
//   residual_out = round(sum)                            (input dtype)
//   r        = 1 / sqrt(mean(sum^2) + eps)               (fp32)
//   y        = round(round(sum * r) * weight)            (input dtype, two roundings)
//   s        = max|y| / 127,  q = rint(y / s) clamped to +-127 (0 for a zero row)
//
// This is the chain add-RMSNorm -> dynamic per-token quant of the reference
// runtime (vllm_ascend.patch:755-787: npu_add_rms_norm_dynamic_quant, or
// npu_add_rms_norm followed by the linear's npu_dynamic_quant), with the
// RMSNorm arithmetic of vLLM's native RMSNorm (fp32 sum and statistics, output
// rounded to the input dtype before the weight multiply).  The quantisation
// uses the same scale and rounding expressions as mp_quant_per_token_i8, so the
// fused result equals the unfused chain on the same y bit for bit.
//
// One 256-thread workgroup per row.  The vector kernel keeps the row in
// registers (8 elements per 16-byte load, V loads per thread, H <= 16384), so
// every output is written by the thread that read its inputs: in-place calls
// (residual_out == residual, y == x) are safe.
#include "mp_common.h"

namespace {

template <bool BF16>
__device__ __forceinline__ float nq_ld(uint16_t b) {
  return BF16 ? mp_bf2f(b) : mp_h2f(b);
}
template <bool BF16>
__device__ __forceinline__ uint16_t nq_st(float f) {
  return BF16 ? mp_f2bf(f) : mp_f2h(f);
}
template <bool BF16>
__device__ __forceinline__ float nq_round(float f) {
  return nq_ld<BF16>(nq_st<BF16>(f));
}

__device__ __forceinline__ float nq_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// workgroup sum / max of one value per thread, fixed order over the 4 waves (LDS-only
// barriers: the stores already issued need not complete first)
__device__ __forceinline__ float nq_block_sum(float v, float *red) {
  v = nq_wave_sum(v);
  mp_lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  mp_lds_barrier();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float nq_block_max(float v, float *red) {
  v = mp_wave_max(v);
  mp_lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  mp_lds_barrier();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ int8_t nq_code(float v, float s) {
  float r = (s == 0.f) ? 0.f : rintf(v / s);
  r = fminf(fmaxf(r, -127.f), 127.f);
  return static_cast<int8_t>(static_cast<int>(r));
}

template <int V, bool BF16>
__global__ __launch_bounds__(256) void add_rmsnorm_quant_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ res, const uint16_t *__restrict__ w, float eps,
    int h, uint16_t *__restrict__ res_out, uint16_t *__restrict__ y, int8_t *__restrict__ q,
    float *__restrict__ s_out) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * h;
  float v[V][8];
  float ss = 0.f;
  // the norm weights are loaded with the row: a load after the residual stores would wait
  // for them
  uint4 wv[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = (tid + 256 * i) * 8;
    wv[i] = *reinterpret_cast<const uint4 *>(w + (c < h ? c : 0));
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = (tid + 256 * i) * 8;
    const bool ok = c < h;
    const int cc = ok ? c : 0;
    const uint4 a = *reinterpret_cast<const uint4 *>(x + base + cc);
    const uint4 b = res ? *reinterpret_cast<const uint4 *>(res + base + cc) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t ah = static_cast<uint16_t>(aw[e >> 1] >> (16 * (e & 1)));
      const uint16_t bh = static_cast<uint16_t>(bw[e >> 1] >> (16 * (e & 1)));
      float f = nq_ld<BF16>(ah);
      if (res) f = mp_add(f, nq_ld<BF16>(bh));
      f = ok ? f : 0.f;
      v[i][e] = f;
      ss = mp_add(ss, mp_mul(f, f));
    }
  }
  if (res_out) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int c = (tid + 256 * i) * 8;
      if (c < h) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = static_cast<uint32_t>(nq_st<BF16>(v[i][2 * e])) |
                 (static_cast<uint32_t>(nq_st<BF16>(v[i][2 * e + 1])) << 16);
        *reinterpret_cast<uint4 *>(res_out + base + c) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  const float var = nq_block_sum(ss, red) / static_cast<float>(h);
  const float r = 1.0f / sqrtf(var + eps);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = (tid + 256 * i) * 8;
    const bool ok = c < h;
    const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float we = nq_ld<BF16>(static_cast<uint16_t>(ww[e >> 1] >> (16 * (e & 1))));
      const float yn = nq_round<BF16>(mp_mul(v[i][e], r));
      const float yv = ok ? nq_round<BF16>(mp_mul(yn, we)) : 0.f;
      v[i][e] = yv;
      amax = fmaxf(amax, fabsf(yv));
    }
    if (y && ok) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = static_cast<uint32_t>(nq_st<BF16>(v[i][2 * e])) |
               (static_cast<uint32_t>(nq_st<BF16>(v[i][2 * e + 1])) << 16);
      *reinterpret_cast<uint4 *>(y + base + c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  if (!q) return;  // kernel argument: uniform over the workgroup
  const float s = nq_block_max(amax, red) / 127.0f;
  if (tid == 0) s_out[blockIdx.x] = s;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = (tid + 256 * i) * 8;
    if (c < h) {
      uint32_t o[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(nq_code(v[i][e], s))) << (8 * (e & 3));
      *reinterpret_cast<uint2 *>(q + base + c) = make_uint2(o[0], o[1]);
    }
  }
}

// Any H / alignment: three passes over the row (statistics, max, outputs); the
// outputs are written only in the last pass, by the thread that re-reads the
// same element, so in-place calls stay safe.
template <bool BF16>
__global__ __launch_bounds__(256) void add_rmsnorm_quant_scalar_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ res, const uint16_t *__restrict__ w, float eps,
    int64_t h, uint16_t *__restrict__ res_out, uint16_t *__restrict__ y, int8_t *__restrict__ q,
    float *__restrict__ s_out) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * h;
  auto sum_at = [&](int64_t c) {
    float f = nq_ld<BF16>(x[base + c]);
    if (res) f = mp_add(f, nq_ld<BF16>(res[base + c]));
    return f;
  };
  float ss = 0.f;
  for (int64_t c = tid; c < h; c += 256) {
    const float f = sum_at(c);
    ss = mp_add(ss, mp_mul(f, f));
  }
  const float var = nq_block_sum(ss, red) / static_cast<float>(h);
  const float r = 1.0f / sqrtf(var + eps);
  auto y_at = [&](float f, int64_t c) {
    return nq_round<BF16>(mp_mul(nq_round<BF16>(mp_mul(f, r)), nq_ld<BF16>(w[c])));
  };
  float s = 0.f;
  if (q) {
    float amax = 0.f;
    for (int64_t c = tid; c < h; c += 256) amax = fmaxf(amax, fabsf(y_at(sum_at(c), c)));
    s = nq_block_max(amax, red) / 127.0f;
    if (tid == 0) s_out[blockIdx.x] = s;
  }
  for (int64_t c = tid; c < h; c += 256) {
    const float f = sum_at(c);
    const float yv = y_at(f, c);
    if (res_out) res_out[base + c] = nq_st<BF16>(f);
    if (y) y[base + c] = nq_st<BF16>(yv);
    if (q) q[base + c] = nq_code(yv, s);
  }
}

}  // namespace

extern "C" int mp_add_rms_norm_quant(const void *x, const void *residual, const void *weight, float eps, int64_t m,
                                     int64_t h, int dtype, void *residual_out, void *y, int8_t *q, float *scale,
                                     mp_stream_t stream) {
  if (dtype != MP_F16 && dtype != MP_BF16) return MP_ERR_DTYPE;
  if (m < 0 || h <= 0) return MP_ERR_SHAPE;
  if ((q == nullptr) != (scale == nullptr)) return MP_ERR_ARG;
  if (m == 0) return MP_OK;
  if (!x || !weight || (!y && !q && !residual_out)) return MP_ERR_ARG;
  if (m > INT32_MAX || h > INT32_MAX) return MP_ERR_SHAPE;
  if (!(eps >= 0.f)) return MP_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto *xp = static_cast<const uint16_t *>(x);
  const auto *rp = static_cast<const uint16_t *>(residual);
  const auto *wp = static_cast<const uint16_t *>(weight);
  auto *rop = static_cast<uint16_t *>(residual_out);
  auto *yp = static_cast<uint16_t *>(y);
  const bool bf = dtype == MP_BF16;
  const bool vec = h % 8 == 0 && h <= 16384 && mp_aligned(x, 16) && mp_aligned(weight, 16) &&
                   (!residual || mp_aligned(residual, 16)) && (!residual_out || mp_aligned(residual_out, 16)) &&
                   (!y || mp_aligned(y, 16)) && (!q || mp_aligned(q, 8));
  const dim3 grid(static_cast<unsigned>(m));
  const int hi = static_cast<int>(h);
  if (vec) {
    const int v = static_cast<int>(mp_cdiv(h, 2048));
#define MP_NQ(V_)                                                                                            \
  do {                                                                                                       \
    if (bf)                                                                                                  \
      hipLaunchKernelGGL((add_rmsnorm_quant_kernel<V_, true>), grid, dim3(256), 0, s, xp, rp, wp, eps, hi,  \
                         rop, yp, q, scale);                                                                 \
    else                                                                                                     \
      hipLaunchKernelGGL((add_rmsnorm_quant_kernel<V_, false>), grid, dim3(256), 0, s, xp, rp, wp, eps, hi, \
                         rop, yp, q, scale);                                                                 \
  } while (0)
    if (v <= 1) MP_NQ(1);
    else if (v == 2) MP_NQ(2);
    else if (v <= 4) MP_NQ(4);
    else MP_NQ(8);
#undef MP_NQ
  } else if (bf) {
    hipLaunchKernelGGL((add_rmsnorm_quant_scalar_kernel<true>), grid, dim3(256), 0, s, xp, rp, wp, eps, h, rop, yp,
                       q, scale);
  } else {
    hipLaunchKernelGGL((add_rmsnorm_quant_scalar_kernel<false>), grid, dim3(256), 0, s, xp, rp, wp, eps, h, rop, yp,
                       q, scale);
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}
