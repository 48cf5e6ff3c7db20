// Dequantising GEMM for gfx950: Y = dq(A) . dq(B)^T in fp16 / bf16 MFMA with fp32 accumulation.
//
// Every element is rounded to the arithmetic dtype exactly as the reference builds the
// tensors it multiplies:
//   - int8 codes with a per-row scale: r(q * s), the value quantize_*_absmax returns
//     (smoothquant/fake_quant.py:10-31);
//   - packed uint4 with group scales / zeros: r((u - z) * s), the weight
//     pseudo_quantize_tensor returns (awq/quantize/quantizer.py:89-96);
//   - plain fp16 / bf16 activations as they are.
// q * s and (u - z) * s are exact in fp32 (at most 8 + 11 significant bits), so one fp32
// product and one conversion give the dtype's rounding of the exact value.  The products of
// the MFMA are exact and summed in fp32 -- the arithmetic of F.linear on those tensors, up to
// the order of the fp32 sum.
//
// Used where the reference's fake-quant / pseudo-quant numerics must be reproduced to a
// fraction of an output ulp: the fake-rule MoE expert chain (a 1-ulp change of a gate / up
// value flips codes of the coarse per-token requant that follows), the bf16 fake-rule W8A8
// linear and the bf16 W4A16 linear (bf16 rounding of each dequantised weight is ~2^-9).
#include "dq_gemm.h"

namespace {

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef _Float16 hf2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));

constexpr int kDBM = 128, kDBN = 128, kDBK = 64, kDLD = kDBK + 8;  // LDS row stride in 16-bit elements
constexpr uint32_t kDOob = 0x80000000u;                             // past every descriptor

// Two fp32 values (exact products) rounded to the dtype, packed.
template <int DT>
__device__ __forceinline__ uint32_t dq_pack2(float a, float b) {
  if constexpr (DT == MP_F16) {
    const hf2_t v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    const bf2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
  }
}

template <int DT>
__device__ __forceinline__ float dq_to_f32(uint16_t b) {
  return DT == MP_F16 ? mp_h2f(b) : mp_bf2f(b);
}

template <int DT>
__device__ __forceinline__ f16_t dq_mfma(uint4 a, uint4 b, f16_t c) {
  if constexpr (DT == MP_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0,
                                                  0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8_t, a), __builtin_bit_cast(bf8_t, b), c, 0,
                                                   0, 0);
}

// 16 int8 codes times the row scale -> 16 dtype values (two 16-byte LDS chunks).
template <int DT>
__device__ __forceinline__ void dq_i8x16(uint4 v, float s, uint4 &lo, uint4 &hi) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f0 = static_cast<float>(static_cast<int8_t>(w[i] & 0xFFu)) * s;
    const float f1 = static_cast<float>(static_cast<int8_t>((w[i] >> 8) & 0xFFu)) * s;
    const float f2 = static_cast<float>(static_cast<int8_t>((w[i] >> 16) & 0xFFu)) * s;
    const float f3 = static_cast<float>(static_cast<int8_t>(w[i] >> 24)) * s;
    o[2 * i] = dq_pack2<DT>(f0, f1);
    o[2 * i + 1] = dq_pack2<DT>(f2, f3);
  }
  lo = make_uint4(o[0], o[1], o[2], o[3]);
  hi = make_uint4(o[4], o[5], o[6], o[7]);
}

// 8 nibbles of one packed word (columns 8q .. 8q+7 in natural order): (u - z) * s.
template <int DT>
__device__ __forceinline__ uint4 dq_u4x8(uint32_t w, float z, float s) {
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = (static_cast<float>((w >> (8 * j)) & 0xFu) - z) * s;
    const float b = (static_cast<float>((w >> (8 * j + 4)) & 0xFu) - z) * s;
    o[j] = dq_pack2<DT>(a, b);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Row range of a workgroup: dense tiles of kDBM rows, or for grouped launches the
// blockIdx.y-th (expert, 128-row chunk) in expert-major order; false past the last chunk.
__device__ __forceinline__ bool dq_rows(const mp_dq_args &p, int64_t &rb, int64_t &re, int &expert) {
  if (!p.offsets) {
    rb = static_cast<int64_t>(blockIdx.y) * kDBM;
    re = rb + kDBM < p.rows ? rb + kDBM : p.rows;
    expert = 0;
    return rb < p.rows;
  }
  int64_t slot = blockIdx.y;
  for (int e = 0; e < p.n_experts; ++e) {
    const int64_t lo = p.offsets[e], hi = p.offsets[e + 1];
    const int64_t nch = (hi - lo + kDBM - 1) / kDBM;
    if (slot < nch) {
      rb = lo + slot * kDBM;
      re = rb + kDBM < hi ? rb + kDBM : hi;
      expert = e;
      return true;
    }
    slot -= nch;
  }
  return false;
}

// 128 x 128 output tile (SWIGLU: 128 rows x 64 h columns from 64 gate + 64 up weight rows)
// per workgroup of 4 waves, each 64 x 64 (2 x 2 MFMA 32x32x16 tiles), BK = 64.  Each thread
// stages its A and B pieces of the next K tile in registers while the current tile is
// multiplied from LDS (double-buffered), dequantising on the way to LDS.
template <int DT, int AF, int BF, int EPI>
__global__ __launch_bounds__(256) void dq_gemm_kernel(mp_dq_args p) {
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][kDBM * kDLD];
  __shared__ __attribute__((aligned(16))) uint16_t sb[2][kDBN * kDLD];
  constexpr bool SWI = EPI == MP_EPI_SWIGLU;
  constexpr int ACH = AF == MP_DQ_DT ? 4 : 2;  // 16-byte A pieces per thread per K tile
  constexpr int BCH = BF == MP_DQ_U4GRP ? 1 : (BF == MP_DQ_DT ? 4 : 2);
  int64_t rb, re;
  int expert;
  if (!dq_rows(p, rb, re, expert)) return;  // workgroup-uniform
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int k = static_cast<int>(p.k);
  const int nkt = k / kDBK;
  const int64_t n_out = p.n;
  const int64_t nb_rows = SWI ? 2 * n_out : n_out;  // weight rows per expert
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * (SWI ? kDBN / 2 : kDBN);

  // ---- A pieces: rows of this tile (rows past the buffer read zeros through the descriptor)
  const uint32_t aesz = AF == MP_DQ_DT ? 2 : 1;
  const auto ar = mp_rsrc(p.a, static_cast<uint32_t>(p.rows * k * aesz));
  uint32_t aoff[ACH];
  float ascale[ACH];
  int arow[ACH], acol[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + i * 256;
    arow[i] = AF == MP_DQ_DT ? (c >> 3) : (c >> 2);
    acol[i] = AF == MP_DQ_DT ? (c & 7) * 8 : (c & 3) * 16;
    const int64_t m = rb + arow[i];
    aoff[i] = m < p.rows ? static_cast<uint32_t>((m * k + acol[i]) * aesz) : kDOob;
    ascale[i] = (AF == MP_DQ_I8ROW && m < p.rows) ? p.a_scale[m] : 0.f;
  }
  // ---- B pieces: weight rows of this tile (clamped into the expert's rows)
  int brow[BCH], bcol[BCH];
  const uint8_t *bptr[BCH];
  float bscale[BCH];
  int64_t bn[BCH];
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int c = tid + i * 256;
    brow[i] = BF == MP_DQ_U4GRP ? (c >> 1) : (BF == MP_DQ_DT ? (c >> 3) : (c >> 2));
    bcol[i] = BF == MP_DQ_U4GRP ? (c & 1) * 32 : (BF == MP_DQ_DT ? (c & 7) * 8 : (c & 3) * 16);
    int64_t n;
    if (SWI) {
      const int64_t cc = col0 + (brow[i] & 63);
      n = (cc < n_out ? cc : n_out - 1) + (brow[i] >= 64 ? n_out : 0);
    } else {
      n = col0 + brow[i] < n_out ? col0 + brow[i] : n_out - 1;
    }
    bn[i] = n;
    if (BF == MP_DQ_U4GRP) {
      bptr[i] = static_cast<const uint8_t *>(p.b) + n * (k / 2) + bcol[i] / 2;
      bscale[i] = 0.f;
    } else if (BF == MP_DQ_DT) {
      const int64_t rowg = static_cast<int64_t>(expert) * nb_rows + n;
      bptr[i] = static_cast<const uint8_t *>(p.b) + (rowg * k + bcol[i]) * 2;
      bscale[i] = 0.f;
    } else {
      const int64_t rowg = static_cast<int64_t>(expert) * nb_rows + n;
      bptr[i] = static_cast<const uint8_t *>(p.b) + rowg * k + bcol[i];
      bscale[i] = p.b_scale[rowg];
    }
  }
  const int ngroups = BF == MP_DQ_U4GRP ? k / p.group : 1;

  uint4 areg[ACH], breg[BCH];
  float bz[BCH], bs[BCH];  // MP_DQ_U4GRP: zero point and scale of the piece's group
  auto load_tile = [&](int kt) {
    kt = kt < nkt ? kt : nkt - 1;
    const uint32_t kb = static_cast<uint32_t>(kt) * kDBK;
#pragma unroll
    for (int i = 0; i < ACH; ++i) areg[i] = mp_buf_load16(ar, aoff[i] + kb * aesz, 0);
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      if (BF == MP_DQ_U4GRP) {
        breg[i] = *reinterpret_cast<const uint4 *>(bptr[i] + kb / 2);
        const int64_t gi = bn[i] * ngroups + (kb + bcol[i]) / p.group;
        bs[i] = dq_to_f32<DT>(p.b_gscale[gi]);
        bz[i] = p.b_gzero ? dq_to_f32<DT>(p.b_gzero[gi]) : 8.0f;
      } else {
        breg[i] = *reinterpret_cast<const uint4 *>(bptr[i] + kb * (BF == MP_DQ_DT ? 2 : 1));
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      uint16_t *dst = &sa[buf][arow[i] * kDLD + acol[i]];
      if (AF == MP_DQ_DT) {
        *reinterpret_cast<uint4 *>(dst) = areg[i];
      } else {
        uint4 lo, hi;
        dq_i8x16<DT>(areg[i], ascale[i], lo, hi);
        *reinterpret_cast<uint4 *>(dst) = lo;
        *reinterpret_cast<uint4 *>(dst + 8) = hi;
      }
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      uint16_t *dst = &sb[buf][brow[i] * kDLD + bcol[i]];
      if (BF == MP_DQ_U4GRP) {
        const uint32_t w[4] = {breg[i].x, breg[i].y, breg[i].z, breg[i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4 *>(dst + 8 * q) = dq_u4x8<DT>(w[q], bz[i], bs[i]);
      } else if (BF == MP_DQ_DT) {
        *reinterpret_cast<uint4 *>(dst) = breg[i];
      } else {
        uint4 lo, hi;
        dq_i8x16<DT>(breg[i], bscale[i], lo, hi);
        *reinterpret_cast<uint4 *>(dst) = lo;
        *reinterpret_cast<uint4 *>(dst + 8) = hi;
      }
    }
  };

  f16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  // B rows of the wave's two 32-row MFMA tiles: dense / F32 the wave's 64 columns; SwiGLU the
  // wave's 32 gate rows and the matching 32 up rows
  const int brow0 = SWI ? wn * 32 : wn * 64;
  const int brow1 = SWI ? 64 + wn * 32 : wn * 64 + 32;
  auto mma = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < kDBK / 16; ++ks) {
      uint4 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const uint4 *>(&sa[cur][(wm * 64 + i * 32 + (lane & 31)) * kDLD + ks * 16 +
                                                          8 * (lane >> 5)]);
      bf[0] = *reinterpret_cast<const uint4 *>(&sb[cur][(brow0 + (lane & 31)) * kDLD + ks * 16 + 8 * (lane >> 5)]);
      bf[1] = *reinterpret_cast<const uint4 *>(&sb[cur][(brow1 + (lane & 31)) * kDLD + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = dq_mfma<DT>(af[i], bf[j], acc[i][j]);
    }
  };

  load_tile(0);
  store_tile(0);
  load_tile(1);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    mma(kt & 1);
    if (kt + 1 < nkt) store_tile((kt + 1) & 1);  // workgroup-uniform
    load_tile(kt + 2);
    __syncthreads();
  }

  // ---- epilogues (accumulator r of MFMA tile (i, j): row 8 (r >> 2) + 4 (lane >> 5) + (r & 3),
  // column lane % 32)
  const int64_t mbase = rb + wm * 64 + 4 * (lane >> 5);
  if constexpr (SWI) {
    const int mode = DT == MP_F16 ? kRoundF16 : kRoundBF16;
    const int64_t col = col0 + wn * 32 + (lane & 31);
    const bool cval = col < n_out;
    float *hbuf = static_cast<float *>(p.y);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = mbase + i * 32 + 8 * (r >> 2) + (r & 3);
        const bool mval = m < re;
        const float h = mp_swiglu_epi(acc[i][0][r], acc[i][1][r], mode);
        if (mval && cval) hbuf[m * p.ldy + col] = h;
        float a = (mval && cval) ? fabsf(h) : 0.f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        if ((lane & 31) == 0 && mval) p.amax_partial[m * p.n_partial + static_cast<int64_t>(blockIdx.x) * 2 + wn] = a;
      }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = col0 + wn * 64 + j * 32 + (lane & 31);
      const bool cval = col < n_out;
      const float bv = (EPI == MP_EPI_DENSE && p.bias) ? mp_load_as_f32(p.bias, cval ? col : 0, p.bias_dtype) : 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = mbase + i * 32 + 8 * (r >> 2) + (r & 3);
          if (m < re && cval) {
            const float v = EPI == MP_EPI_DENSE ? mp_add(acc[i][j][r], bv) : acc[i][j][r];
            mp_store_from_f32(p.y, m * p.ldy + col, EPI == MP_EPI_DENSE ? p.out_dtype : MP_F32, v);
          }
        }
    }
  }
}

// ---------------------------------------------------------------- any-K kernel
// One thread per (row, 32 output columns): the same element rounding and an fp32 sum, for
// K that is not a multiple of 64 (correctness path).
template <int DT, int AF, int BF, int EPI>
__global__ __launch_bounds__(256) void dq_simple_kernel(mp_dq_args p) {
  constexpr bool SWI = EPI == MP_EPI_SWIGLU;
  const int64_t ncg = (p.n + 31) / 32;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= p.rows * ncg) return;
  const int64_t m = tid / ncg, cg = tid % ncg;
  int expert = 0;
  if (p.offsets) {
    for (int e = 0; e < p.n_experts; ++e)
      if (m >= p.offsets[e] && m < p.offsets[e + 1]) expert = e;
    if (m >= p.offsets[p.n_experts]) return;
  }
  const int64_t k = p.k;
  const int64_t nb_rows = SWI ? 2 * p.n : p.n;
  const int ngroups = BF == MP_DQ_U4GRP ? static_cast<int>(k / p.group) : 1;
  const float as = AF == MP_DQ_I8ROW ? p.a_scale[m] : 0.f;
  auto aval = [&](int64_t kk) -> float {
    if (AF == MP_DQ_DT) return dq_to_f32<DT>(static_cast<const uint16_t *>(p.a)[m * k + kk]);
    return mp_round_mode_apply(static_cast<float>(static_cast<const int8_t *>(p.a)[m * k + kk]) * as,
                               DT == MP_F16 ? kRoundF16 : kRoundBF16);
  };
  auto dot = [&](int64_t n) -> float {
    const int64_t rowg = static_cast<int64_t>(expert) * nb_rows + n;
    float acc = 0.f;
    for (int64_t kk = 0; kk < k; ++kk) {
      float w;
      if (BF == MP_DQ_U4GRP) {
        const uint32_t u = (static_cast<const uint32_t *>(p.b)[n * (k / 8) + kk / 8] >> (4 * (kk & 7))) & 0xFu;
        const int64_t gi = n * ngroups + kk / p.group;
        const float s = dq_to_f32<DT>(p.b_gscale[gi]);
        const float z = p.b_gzero ? dq_to_f32<DT>(p.b_gzero[gi]) : 8.0f;
        w = (static_cast<float>(u) - z) * s;
      } else if (BF == MP_DQ_DT) {
        w = dq_to_f32<DT>(static_cast<const uint16_t *>(p.b)[rowg * k + kk]);
      } else {
        w = static_cast<float>(static_cast<const int8_t *>(p.b)[rowg * k + kk]) * p.b_scale[rowg];
      }
      w = mp_round_mode_apply(w, DT == MP_F16 ? kRoundF16 : kRoundBF16);
      acc = fmaf(aval(kk), w, acc);
    }
    return acc;
  };
  float amax = 0.f;
  for (int c = 0; c < 32; ++c) {
    const int64_t col = cg * 32 + c;
    if (col >= p.n) break;
    if (SWI) {
      const float h = mp_swiglu_epi(dot(col), dot(p.n + col), DT == MP_F16 ? kRoundF16 : kRoundBF16);
      static_cast<float *>(p.y)[m * p.ldy + col] = h;
      amax = fmaxf(amax, fabsf(h));
    } else {
      float v = dot(col);
      if (EPI == MP_EPI_DENSE && p.bias) v = mp_add(v, mp_load_as_f32(p.bias, col, p.bias_dtype));
      mp_store_from_f32(p.y, m * p.ldy + col, EPI == MP_EPI_DENSE ? p.out_dtype : MP_F32, v);
    }
  }
  // partial p covers columns [32 p, 32 p + 32) (the tiled kernel's blockIdx.x * 2 + wn)
  if (SWI) p.amax_partial[m * p.n_partial + cg] = amax;
}

template <int DT, int AF, int BF>
int dq_launch_fmt(const mp_dq_args &p, int epi, hipStream_t stream) {
  if (p.k % kDBK == 0 && (BF != MP_DQ_U4GRP || p.group % 32 == 0)) {
    const int64_t ntile = mp_cdiv(p.n, epi == MP_EPI_SWIGLU ? kDBN / 2 : kDBN);
    const int64_t mslots = mp_cdiv(p.rows, kDBM) + (p.offsets ? p.n_experts : 0);
    if (ntile > INT32_MAX || mslots > 65535) return MP_ERR_SHAPE;
    const dim3 grid(static_cast<unsigned>(ntile), static_cast<unsigned>(mslots));
    if (epi == MP_EPI_SWIGLU)
      hipLaunchKernelGGL((dq_gemm_kernel<DT, AF, BF, MP_EPI_SWIGLU>), grid, dim3(256), 0, stream, p);
    else if (epi == MP_EPI_F32)
      hipLaunchKernelGGL((dq_gemm_kernel<DT, AF, BF, MP_EPI_F32>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dq_gemm_kernel<DT, AF, BF, MP_EPI_DENSE>), grid, dim3(256), 0, stream, p);
  } else {
    const int64_t threads = p.rows * mp_cdiv(p.n, 32);
    const dim3 grid(static_cast<unsigned>(mp_cdiv(threads, 256)));
    if (epi == MP_EPI_SWIGLU)
      hipLaunchKernelGGL((dq_simple_kernel<DT, AF, BF, MP_EPI_SWIGLU>), grid, dim3(256), 0, stream, p);
    else if (epi == MP_EPI_F32)
      hipLaunchKernelGGL((dq_simple_kernel<DT, AF, BF, MP_EPI_F32>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dq_simple_kernel<DT, AF, BF, MP_EPI_DENSE>), grid, dim3(256), 0, stream, p);
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}

}  // namespace

int mp_launch_dq_gemm(const mp_dq_args &p, int epi, hipStream_t stream) {
  if (p.dt != MP_F16 && p.dt != MP_BF16) return MP_ERR_DTYPE;
  if (!p.a || !p.b || !p.y) return MP_ERR_ARG;
  if (p.rows < 0 || p.n <= 0 || p.k <= 0) return MP_ERR_SHAPE;
  if (p.rows == 0) return MP_OK;
  const bool u4 = p.b_fmt == MP_DQ_U4GRP;
  if (u4 && (p.offsets || !p.b_gscale || p.group <= 0 || p.k % p.group || p.k % 8)) return MP_ERR_SHAPE;
  if (p.b_fmt == MP_DQ_I8ROW && !p.b_scale) return MP_ERR_ARG;
  if (p.b_fmt != MP_DQ_I8ROW && p.b_fmt != MP_DQ_DT && !u4) return MP_ERR_ARG;
  if (p.a_fmt == MP_DQ_I8ROW && !p.a_scale) return MP_ERR_ARG;
  if (p.a_fmt != MP_DQ_DT && p.a_fmt != MP_DQ_I8ROW) return MP_ERR_ARG;
  if (epi == MP_EPI_SWIGLU && (!p.amax_partial || p.n_partial < 2 * mp_cdiv(p.n, 64))) return MP_ERR_ARG;
  if (p.offsets && (p.n_experts <= 0 || p.n_experts > 1024)) return MP_ERR_SHAPE;
  // 32-bit descriptor offsets over A and 32-bit tile arithmetic
  if (p.rows * p.k * (p.a_fmt == MP_DQ_DT ? 2 : 1) >= (int64_t(1) << 31) || p.k > (1 << 20)) return MP_ERR_SHAPE;
  if (p.k % kDBK == 0 && (!mp_aligned(p.a, 16) || !mp_aligned(p.b, 16))) return MP_ERR_ALIGN;  // tiled loads
  const bool a8 = p.a_fmt == MP_DQ_I8ROW, b8 = p.b_fmt == MP_DQ_I8ROW;
  if (u4 && a8) return MP_ERR_ARG;  // packed weights multiply plain activations only
  if (p.dt == MP_F16) {
    if (u4) return dq_launch_fmt<MP_F16, MP_DQ_DT, MP_DQ_U4GRP>(p, epi, stream);
    if (a8 && b8) return dq_launch_fmt<MP_F16, MP_DQ_I8ROW, MP_DQ_I8ROW>(p, epi, stream);
    if (b8) return dq_launch_fmt<MP_F16, MP_DQ_DT, MP_DQ_I8ROW>(p, epi, stream);
    if (a8) return dq_launch_fmt<MP_F16, MP_DQ_I8ROW, MP_DQ_DT>(p, epi, stream);
    return dq_launch_fmt<MP_F16, MP_DQ_DT, MP_DQ_DT>(p, epi, stream);
  }
  if (u4) return dq_launch_fmt<MP_BF16, MP_DQ_DT, MP_DQ_U4GRP>(p, epi, stream);
  if (a8 && b8) return dq_launch_fmt<MP_BF16, MP_DQ_I8ROW, MP_DQ_I8ROW>(p, epi, stream);
  if (b8) return dq_launch_fmt<MP_BF16, MP_DQ_DT, MP_DQ_I8ROW>(p, epi, stream);
  if (a8) return dq_launch_fmt<MP_BF16, MP_DQ_I8ROW, MP_DQ_DT>(p, epi, stream);
  return dq_launch_fmt<MP_BF16, MP_DQ_DT, MP_DQ_DT>(p, epi, stream);
}

// The fake-quant linear at any operand widths: y = F.linear(dq(a), dq(b), bias) with each operand
// either plain values in the dtype (a width of 16 bits or more: not quantized) or int8 codes with
// a per-row scale, rounded to the dtype as the reference's fake-quant tensors are.
extern "C" int mp_dq_linear(const void *a, const float *a_scale, const void *b, const float *b_scale,
                            const void *bias, int dtype, void *y, int64_t m, int64_t n, int64_t k,
                            mp_stream_t stream) {
  if (!a || !b || !y) return MP_ERR_ARG;
  if (dtype != MP_F16 && dtype != MP_BF16) return MP_ERR_DTYPE;
  mp_dq_args d{};
  d.dt = dtype;
  d.a = a;
  d.a_fmt = a_scale ? MP_DQ_I8ROW : MP_DQ_DT;
  d.a_scale = a_scale;
  d.b = b;
  d.b_fmt = b_scale ? MP_DQ_I8ROW : MP_DQ_DT;
  d.b_scale = b_scale;
  d.bias = bias;
  d.bias_dtype = dtype;
  d.y = y;
  d.out_dtype = dtype;
  d.ldy = n;
  d.rows = m;
  d.n = n;
  d.k = k;
  return mp_launch_dq_gemm(d, MP_EPI_DENSE, reinterpret_cast<hipStream_t>(stream));
}
