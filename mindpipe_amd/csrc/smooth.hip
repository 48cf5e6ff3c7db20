// SmoothQuant smoothing on the GPU: column abs-max statistics, the smoothing scales and the
// in-place column scaling of the weights that share a norm.
//
// Reference (restated, not translated):
//   * get_act_scales      smoothquant/calibration.py:27-58   per-input-channel max |x| over tokens
//   * _compute_smooth_scales smoothquant/smooth.py:7-25      s = (a^alpha / w^(1-alpha)).clamp(1e-5)
//   * smooth_ln_fcs_llama_like smoothquant/smooth.py:91-101  ln.weight /= s, fc.weight *= s
//
// Layout: a matrix is [rows, k] row-major (weights [N, K], activations [tokens, K], a 3-D expert
// tensor [E, N, K] as E*N rows).  The column statistics are fp32 (exact: max and abs of a 16-bit
// or fp32 value), kept across calls so that several fcs / calibration batches accumulate into one
// vector.  The scale arithmetic is the reference's in the weight dtype: each op computed in fp32
// and rounded once to the dtype, as PyTorch's half / bf16 ops are.
#include "mp_common.h"

namespace {

constexpr int kColThreads = 64;   // threads along K per workgroup (8 columns each)
constexpr int kRowThreads = 4;    // thread rows per workgroup
constexpr int kColsPerWg = 8 * kColThreads;

__device__ __forceinline__ float mp_round_dt(float v, int dtype) {
  return dtype == MP_F16 ? mp_rh(v) : (dtype == MP_BF16 ? mp_rbf(v) : v);
}

// colmax[j] = max(colmax[j], max_r |x[r, j]|): each thread owns 8 consecutive columns of a
// 512-column strip and strides over rows; the 4 thread rows meet in LDS and the strip's maxima go
// to memory with an atomic max on the float bits (non-negative floats order as their bit patterns).
template <int DT>
__global__ __launch_bounds__(kColThreads *kRowThreads) void colmax_abs_kernel(const void *__restrict__ x, int64_t rows,
                                                                               int64_t k, int64_t rows_per_wg,
                                                                               uint32_t *__restrict__ colmax) {
  constexpr int ES = DT == MP_F32 ? 4 : 2;
  __shared__ float part[kRowThreads][kColsPerWg];
  const int tx = threadIdx.x % kColThreads, ty = threadIdx.x / kColThreads;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kColsPerWg + 8 * tx;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_wg;
  const int64_t r1 = r0 + rows_per_wg < rows ? r0 + rows_per_wg : rows;
  float m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m[i] = 0.f;
  const bool full = c0 + 8 <= k && (k * ES) % 16 == 0;
  for (int64_t r = r0 + ty; r < r1; r += kRowThreads) {
    const char *row = static_cast<const char *>(x) + r * k * ES;
    if (full) {
      if constexpr (DT == MP_F32) {
        const uint4 a = *reinterpret_cast<const uint4 *>(row + c0 * 4);
        const uint4 b = *reinterpret_cast<const uint4 *>(row + c0 * 4 + 16);
        float f[4], g[4];
        mp_chunk_to_f32<MP_F32>(a, f);
        mp_chunk_to_f32<MP_F32>(b, g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          m[i] = fmaxf(m[i], fabsf(f[i]));
          m[4 + i] = fmaxf(m[4 + i], fabsf(g[i]));
        }
      } else {
        float f[8];
        mp_chunk_to_f32<DT>(*reinterpret_cast<const uint4 *>(row + c0 * 2), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) m[i] = fmaxf(m[i], fabsf(f[i]));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < k) m[i] = fmaxf(m[i], fabsf(mp_load_as_f32(row, c0 + i, DT)));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) part[ty][8 * tx + i] = m[i];
  __syncthreads();
  for (int c = threadIdx.x; c < kColsPerWg; c += kColThreads * kRowThreads) {
    float v = part[0][c];
#pragma unroll
    for (int t = 1; t < kRowThreads; ++t) v = fmaxf(v, part[t][c]);
    const int64_t col = static_cast<int64_t>(blockIdx.x) * kColsPerWg + c;
    // NaN inputs: fmaxf keeps the other operand, as torch.max does not; the reference's statistics
    // come from finite calibration activations and weights
    if (col < k && v > 0.f) atomicMax(colmax + col, __float_as_uint(v));
  }
}

__global__ void fill_zero_kernel(uint32_t *__restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// s_j in the weight dtype from the fp32 statistics a_j (activations) and w_j (weights):
//   a = R(a_j); w = max over fcs, clamp(min = 1e-5) -> R(1e-5) where below;
//   s = R(R(a^alpha) / R(w^(1-alpha))), clamp(min = 1e-5).
// The exponents are alpha and 1 - alpha as PyTorch sees them: Python doubles cast to float for a
// half / bf16 tensor (so 1 - alpha is formed in double, then cast).
__global__ void smooth_scales_kernel(const float *__restrict__ act_max, const float *__restrict__ w_colmax, int64_t k,
                                     float e1, float e2, int dtype, void *__restrict__ scales) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= k) return;
  const float floor_dt = mp_round_dt(1e-5f, dtype);
  const float a = mp_round_dt(act_max[j], dtype);
  float w = mp_round_dt(w_colmax[j], dtype);  // exact: a max of dtype values
  w = w < 1e-5f ? floor_dt : w;
  // fp32 powers correctly rounded: a square root at 0.5 (torch's own path), otherwise the double
  // power rounded to float (powf is only faithful, and differs between platforms near fp16 ties)
  const float pa = e1 == 0.5f ? sqrtf(a) : static_cast<float>(pow(static_cast<double>(a), static_cast<double>(e1)));
  const float pw = e2 == 0.5f ? sqrtf(w) : static_cast<float>(pow(static_cast<double>(w), static_cast<double>(e2)));
  float s = mp_round_dt(mp_round_dt(pa, dtype) / mp_round_dt(pw, dtype), dtype);
  s = s < 1e-5f ? floor_dt : s;
  mp_store_from_f32(scales, j, dtype, s);
}

// w[r, j] = R(w[r, j] * s[j]) (or / s[j]) in place, 8 columns per thread (one 16-byte access of a
// 16-bit dtype when VEC: k % 8 == 0 and 16-byte aligned rows and scales).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void scale_columns_kernel(void *__restrict__ w, int64_t rows, int64_t k,
                                                            const void *__restrict__ scales, int divide) {
  const int64_t n8 = (k + 7) / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * n8) return;
  const int64_t r = idx / n8, c0 = 8 * (idx % n8);
  if constexpr (VEC) {
    uint4 *wp = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(w) + r * k + c0);
    float v[8], sc[8];
    mp_chunk_to_f32<DT>(*wp, v);
    mp_chunk_to_f32<DT>(*reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(scales) + c0), sc);
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = divide ? v[2 * i] / sc[2 * i] : v[2 * i] * sc[2 * i];
      const float b = divide ? v[2 * i + 1] / sc[2 * i + 1] : v[2 * i + 1] * sc[2 * i + 1];
      const uint32_t lo = DT == MP_F16 ? mp_f2h(a) : mp_f2bf(a), hi = DT == MP_F16 ? mp_f2h(b) : mp_f2bf(b);
      o[i] = lo | (hi << 16);
    }
    *wp = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t c = c0 + i;
      if (c >= k) break;
      const float sv = mp_load_as_f32(scales, c, DT);
      const float v = mp_load_as_f32(w, r * k + c, DT);
      mp_store_from_f32(w, r * k + c, DT, divide ? v / sv : v * sv);
    }
  }
}

}  // namespace

extern "C" int mp_colmax_abs(const void *x, int dtype, int64_t rows, int64_t k, int accumulate, float *colmax,
                             mp_stream_t stream) {
  if (dtype != MP_F16 && dtype != MP_BF16 && dtype != MP_F32) return MP_ERR_DTYPE;
  if (rows < 0 || k <= 0) return MP_ERR_SHAPE;
  if (!colmax || (rows > 0 && !x)) return MP_ERR_ARG;
  if (!mp_aligned(x, 16) || !mp_aligned(colmax, 4)) return MP_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto *cm = reinterpret_cast<uint32_t *>(colmax);
  if (!accumulate) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(mp_cdiv(k, 256))), dim3(256), 0, s, cm, k);
    MP_CHECK_LAUNCH();
  }
  if (rows == 0) return MP_OK;
  const int64_t strips = mp_cdiv(k, kColsPerWg);
  // about 2048 workgroups in all, at least 16 rows each
  int64_t splits = mp_cdiv(2048, strips);
  int64_t per = mp_cdiv(rows, splits);
  per = per < 16 ? 16 : per;
  splits = mp_cdiv(rows, per);
  if (strips > INT32_MAX || splits > 65535) return MP_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(strips), static_cast<unsigned>(splits));
  const dim3 block(kColThreads * kRowThreads);
  if (dtype == MP_F16) hipLaunchKernelGGL(colmax_abs_kernel<MP_F16>, grid, block, 0, s, x, rows, k, per, cm);
  else if (dtype == MP_BF16) hipLaunchKernelGGL(colmax_abs_kernel<MP_BF16>, grid, block, 0, s, x, rows, k, per, cm);
  else hipLaunchKernelGGL(colmax_abs_kernel<MP_F32>, grid, block, 0, s, x, rows, k, per, cm);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_smooth_scales(const float *act_max, const float *w_colmax, int64_t k, double alpha, int dtype,
                                void *scales, mp_stream_t stream) {
  if (dtype != MP_F16 && dtype != MP_BF16 && dtype != MP_F32) return MP_ERR_DTYPE;
  if (k <= 0) return MP_ERR_SHAPE;
  if (!act_max || !w_colmax || !scales) return MP_ERR_ARG;
  if (!(alpha >= 0.0 && alpha <= 1.0)) return MP_ERR_ARG;
  const float e1 = static_cast<float>(alpha), e2 = static_cast<float>(1.0 - alpha);
  hipLaunchKernelGGL(smooth_scales_kernel, dim3(static_cast<unsigned>(mp_cdiv(k, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), act_max, w_colmax, k, e1, e2, dtype, scales);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_scale_columns(void *w, int dtype, int64_t rows, int64_t k, const void *scales, int divide,
                                mp_stream_t stream) {
  if (dtype != MP_F16 && dtype != MP_BF16 && dtype != MP_F32) return MP_ERR_DTYPE;
  if (rows < 0 || k <= 0) return MP_ERR_SHAPE;
  if (rows == 0) return MP_OK;
  if (!w || !scales) return MP_ERR_ARG;
  const int64_t items = rows * mp_cdiv(k, 8);
  if (mp_cdiv(items, 256) > INT32_MAX) return MP_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(mp_cdiv(items, 256)));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = k % 8 == 0 && mp_aligned(w, 16) && mp_aligned(scales, 16);
#define MP_SCALE_COLS(DT_, V_) \
  hipLaunchKernelGGL((scale_columns_kernel<DT_, V_>), grid, dim3(256), 0, s, w, rows, k, scales, divide)
  if (dtype == MP_F16) {
    if (vec) MP_SCALE_COLS(MP_F16, true);
    else MP_SCALE_COLS(MP_F16, false);
  } else if (dtype == MP_BF16) {
    if (vec) MP_SCALE_COLS(MP_BF16, true);
    else MP_SCALE_COLS(MP_BF16, false);
  } else {
    MP_SCALE_COLS(MP_F32, false);
  }
#undef MP_SCALE_COLS
  MP_CHECK_LAUNCH();
  return MP_OK;
}
