// W8A8 MoE chain for gfx950: routing (stable counting sort by expert) fused
// with the per-token int8 quant, GMM1 + SwiGLU + requant, GMM2, and the
// weighted un-permute.  The two grouped GEMMs use the tiled int8 MFMA kernel
// of w8a8.hip with a grouped row schedule.
#include "dq_gemm.h"

#include <mutex>

namespace {

constexpr int kMaxExperts = 1024;

// Single-workgroup stable counting sort of the T*top_k assignments by expert.
// Writes group_offsets [E+1] and row_of_slot [T*top_k].  Assignment a =
// t*top_k + j keeps (t, j) order inside its expert, so the routed layout is
// deterministic.  Wave w owns the w-th quarter of the assignments (whole batches
// of 64): it counts its quarter per expert (LDS atomics; the ids are cached in LDS,
// the first kRouteLds of them), the per-(wave, expert) bases follow from a prefix
// over experts and waves, and each wave then places its quarter 64 at a time,
// ranking a lane among the lower lanes of its expert with one ballot per distinct
// expert of the batch.
constexpr int kRouteLds = 16384;
constexpr int kRouteWaves = 4;

__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_kernel(const int32_t *__restrict__ ids,
                                                                    int64_t n_assign, int n_experts,
                                                                    int64_t *__restrict__ offsets,
                                                                    int32_t *__restrict__ row_of_slot,
                                                                    int32_t *__restrict__ invalid) {
  __shared__ int cnt[kRouteWaves][kMaxExperts];  // per-wave counts, then per-wave cursors
  __shared__ int16_t sid[kRouteLds];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kRouteWaves * n_experts; i += blockDim.x) cnt[i / n_experts][i % n_experts] = 0;
  __syncthreads();
  const int64_t nb = (n_assign + 63) / 64;                         // batches of 64
  const int64_t per = (nb + kRouteWaves - 1) / kRouteWaves;       // batches per wave
  const int64_t lo = wave * per * 64, hi = (wave + 1) * per * 64 < n_assign ? (wave + 1) * per * 64 : n_assign;
  for (int64_t a = lo + lane; a < hi; a += 64) {
    const int e = ids[a];
    const bool ok = e >= 0 && e < n_experts;
    if (a < kRouteLds) sid[a] = static_cast<int16_t>(ok ? e : -1);
    if (ok) atomicAdd(&cnt[wave][e], 1);
    else if (invalid) atomicAdd(invalid, 1);
  }
  __syncthreads();
  if (tid == 0) {
    // offsets[e] = sum of earlier experts; the cursor of (wave w, expert e) starts after the
    // earlier waves' rows of e
    int64_t run = 0;
    offsets[0] = 0;
    for (int e = 0; e < n_experts; ++e) {
      for (int w = 0; w < kRouteWaves; ++w) {
        const int c = cnt[w][e];
        cnt[w][e] = static_cast<int>(run);
        run += c;
      }
      offsets[e + 1] = run;
    }
  }
  __syncthreads();
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int64_t base = lo; base < hi; base += 64) {
    const int64_t a = base + lane;
    const bool valid = a < hi;
    int e = -1;
    if (valid) {
      if (a < kRouteLds) {
        e = sid[a];
      } else {
        const int v = ids[a];
        e = (v >= 0 && v < n_experts) ? v : -1;
      }
    }
    const bool ok = e >= 0;
    int rank = 0, total = 0;
    uint64_t pending = __ballot(ok);
    while (pending) {  // one pass per distinct expert of the batch (wave-uniform)
      const int leader = __ffsll(static_cast<long long>(pending)) - 1;
      const int ee = __builtin_amdgcn_readlane(e, leader);
      const uint64_t m = __ballot(ok && e == ee);
      if (ok && e == ee) {
        rank = __popcll(m & below);
        total = __popcll(m);
      }
      pending &= ~m;
    }
    const int pos = ok ? cnt[wave][e] + rank : -1;
    if (valid) row_of_slot[a] = pos;
    // the last lane of each expert in this batch advances the wave's cursor
    __builtin_amdgcn_wave_barrier();
    if (ok && rank == total - 1) cnt[wave][e] += total;
    __builtin_amdgcn_wave_barrier();
  }
}

// Per-token quant of x[t] for routed row row_of_slot[a], 16-byte loads: the row is
// read once for its statistics and again (from L2) for the codes, stored 4 or 8 at a time.
// Needs h a multiple of the values per 16 bytes and 16-byte aligned rows (host check).
// RULE: MP_SCALE_FP32 (runtime) or MP_SCALE_FAKE in DT's rounding (signed stored scale).
template <int DT, int RULE>
__global__ __launch_bounds__(256) void moe_permute_quant_vec_kernel(const void *__restrict__ x, int64_t h, int top_k,
                                                                   const int32_t *__restrict__ row_of_slot,
                                                                   int8_t *__restrict__ routed,
                                                                   float *__restrict__ routed_scale) {
  constexpr int N = MpChunk16<DT>::N;
  constexpr int ESZ = DT == MP_F32 ? 4 : 2;
  constexpr int MODE = DT == MP_F16 ? kRoundF16 : (DT == MP_BF16 ? kRoundBF16 : kRoundNone);
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t a = blockIdx.x;
  const int64_t t = a / top_k;
  const int r = row_of_slot[a];
  if (r < 0) return;  // workgroup-uniform
  const int tid = threadIdx.x;
  const int64_t nch = h / N;
  const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const char *>(x) + t * h * ESZ);
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  for (int64_t c = tid; c < nch; c += 256) {
    float f[N];
    mp_chunk_to_f32<DT>(src[c], f);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      st.amax = fmaxf(st.amax, fabsf(f[i]));
      if (RULE != MP_SCALE_FP32) {
        st.vmax = fmaxf(st.vmax, f[i]);
        st.vmin = fminf(st.vmin, f[i]);
      }
    }
  }
  st = mp_block_rowstat(st, red, wbad);
  float s, sg;
  mp_row_scale<RULE>(st, MODE, 0.0f, s, sg);
  if (tid == 0) routed_scale[r] = sg * s;
  int8_t *dst = routed + static_cast<int64_t>(r) * h;
  for (int64_t c = tid; c < nch; c += 256) {
    float f[N];
    mp_chunk_to_f32<DT>(src[c], f);
    uint32_t w[N / 4];
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      w[i] = mp_row_code<RULE>(f[4 * i], s, sg, MODE) | (mp_row_code<RULE>(f[4 * i + 1], s, sg, MODE) << 8) |
             (mp_row_code<RULE>(f[4 * i + 2], s, sg, MODE) << 16) |
             (mp_row_code<RULE>(f[4 * i + 3], s, sg, MODE) << 24);
    if constexpr (N == 8) *reinterpret_cast<uint2 *>(dst + c * 8) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t *>(dst + c * 4) = w[0];
  }
}

// Per-token quant of x[t] written to every routed row that copies it.  One
// workgroup per assignment; the activation row is re-read from L2 per copy.
template <int RULE>
__global__ __launch_bounds__(256) void moe_permute_quant_kernel(const void *__restrict__ x, int x_dtype,
                                                               int64_t h, int top_k,
                                                               const int32_t *__restrict__ row_of_slot,
                                                               int8_t *__restrict__ routed,
                                                               float *__restrict__ routed_scale) {
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t a = blockIdx.x;
  const int64_t t = a / top_k;
  const int r = row_of_slot[a];
  if (r < 0) return;
  const int tid = threadIdx.x;
  const int mode = mp_round_mode_of(x_dtype);
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  for (int64_t c = tid; c < h; c += 256) {
    const float v = mp_load_as_f32(x, t * h + c, x_dtype);
    st.amax = fmaxf(st.amax, fabsf(v));
    st.vmax = fmaxf(st.vmax, v);
    st.vmin = fminf(st.vmin, v);
  }
  st = mp_block_rowstat(st, red, wbad);
  float s, sg;
  mp_row_scale<RULE>(st, mode, 0.0f, s, sg);
  if (tid == 0) routed_scale[r] = sg * s;
  for (int64_t c = tid; c < h; c += 256)
    routed[static_cast<int64_t>(r) * h + c] =
        static_cast<int8_t>(mp_row_code<RULE>(mp_load_as_f32(x, t * h + c, x_dtype), s, sg, mode));
}

// Routing of pre-quantized input (int8 rows x_q [T, H] with fp32 scales): routed row
// row_of_slot[a] copies token a / top_k, 16 bytes per thread-step when the rows allow it.
template <bool VEC>
__global__ __launch_bounds__(256) void moe_permute_rows_kernel(const int8_t *__restrict__ xq, const float *__restrict__ xs,
                                                              int64_t h, int top_k,
                                                              const int32_t *__restrict__ row_of_slot,
                                                              int8_t *__restrict__ routed,
                                                              float *__restrict__ routed_scale) {
  const int64_t a = blockIdx.x;
  const int64_t t = a / top_k;
  const int r = row_of_slot[a];
  if (r < 0) return;
  if (threadIdx.x == 0) routed_scale[r] = xs[t];
  if constexpr (VEC) {
    const uint4 *src = reinterpret_cast<const uint4 *>(xq + t * h);
    uint4 *dst = reinterpret_cast<uint4 *>(routed + static_cast<int64_t>(r) * h);
    for (int64_t c = threadIdx.x; c < h / 16; c += 256) dst[c] = src[c];
  } else {
    for (int64_t c = threadIdx.x; c < h; c += 256) routed[static_cast<int64_t>(r) * h + c] = xq[t * h + c];
  }
}

// Requant of the SwiGLU output: per routed row, the abs-max over the GMM1 workgroups'
// partial maxima, then the codes of the row quantizer.  The fake rule in bf16 also needs the
// row's largest and smallest value (mp_fake_row_sign), which the partials do not carry: that
// case reads the row once more for them (SIGNED).  VEC: 16-byte loads of the fp32 row
// (inter % 4 == 0), four codes per store.
template <int RULE, bool SIGNED, bool VEC>
__global__ __launch_bounds__(256) void moe_requant_kernel(const float *__restrict__ hbuf, const float *__restrict__ part,
                                                         int n_partial, int64_t inter, int mode, int8_t *__restrict__ q,
                                                         float *__restrict__ s_out) {
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const float *row = hbuf + r * inter;
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  if (SIGNED) {
    for (int64_t c = tid; c < inter; c += 256) {
      const float v = row[c];
      st.amax = fmaxf(st.amax, fabsf(v));
      st.vmax = fmaxf(st.vmax, v);
      st.vmin = fminf(st.vmin, v);
    }
  } else {
    for (int i = tid; i < n_partial; i += 256) st.amax = fmaxf(st.amax, part[r * n_partial + i]);
  }
  st = mp_block_rowstat(st, red, wbad);
  float s, sg;
  mp_row_scale<RULE>(st, mode, 0.0f, s, sg);
  if (tid == 0) s_out[r] = sg * s;
  if (VEC) {
    const float4 *src = reinterpret_cast<const float4 *>(row);
    uint32_t *dst = reinterpret_cast<uint32_t *>(q + r * inter);
    for (int64_t c = tid; c < inter / 4; c += 256) {
      const float4 v = src[c];
      dst[c] = mp_row_code<RULE>(v.x, s, sg, mode) | (mp_row_code<RULE>(v.y, s, sg, mode) << 8) |
               (mp_row_code<RULE>(v.z, s, sg, mode) << 16) | (mp_row_code<RULE>(v.w, s, sg, mode) << 24);
    }
  } else {
    for (int64_t c = tid; c < inter; c += 256) q[r * inter + c] = static_cast<int8_t>(mp_row_code<RULE>(row[c], s, sg, mode));
  }
}

// Weighted un-permute of a token's assignments, four columns per thread (VEC: h % 4 == 0,
// 16-byte aligned y rows) or one.
//   FAKE = false: out[t, c] = sum_j w[t, j] * y[row_of_slot[t, j], c] in fp32 in slot order,
//                 one rounding to out_dtype.
//   FAKE = true : the reference's index_add_ in out_dtype r: over the assignments in
//                 ascending expert order (= ascending routed row), out = r(out + r(r(y) * w)).
template <bool FAKE, bool VEC>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float *__restrict__ y,
                                                         const int32_t *__restrict__ row_of_slot,
                                                         const float *__restrict__ w, int64_t t_count, int top_k,
                                                         int64_t h, void *__restrict__ out, int out_dtype) {
  constexpr int NC = VEC ? 4 : 1;
  const int64_t per_row = h / NC;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= t_count * per_row) return;
  const int64_t t = tid / per_row, c = (tid % per_row) * NC;
  const int mode = mp_round_mode_of(out_dtype);
  float acc[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) acc[i] = 0.f;
  int prev = -1;  // FAKE: rows are taken in ascending order, the smallest above prev each time
  for (int j = 0; j < top_k; ++j) {
    int r, slot;
    if (FAKE) {
      r = INT32_MAX;
      slot = -1;
      for (int jj = 0; jj < top_k; ++jj) {
        const int rr = row_of_slot[t * top_k + jj];
        if (rr > prev && rr < r) {
          r = rr;
          slot = jj;
        }
      }
      if (slot < 0) break;
      prev = r;
    } else {
      r = row_of_slot[t * top_k + j];
      slot = j;
      if (r < 0) continue;
    }
    const float wj = w[t * top_k + slot];
    float v[NC];
    if constexpr (VEC) {
      const float4 y4 = *reinterpret_cast<const float4 *>(y + static_cast<int64_t>(r) * h + c);
      v[0] = y4.x;
      v[1] = y4.y;
      v[2] = y4.z;
      v[3] = y4.w;
    } else {
      v[0] = y[static_cast<int64_t>(r) * h + c];
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      if (FAKE)
        acc[i] = mp_round_mode_apply(
            mp_add(acc[i], mp_round_mode_apply(mp_mul(mp_round_mode_apply(v[i], mode), wj), mode)), mode);
      else
        acc[i] = mp_add(acc[i], mp_mul(wj, v[i]));
    }
  }
  const int64_t o = t * h + c;
  if constexpr (VEC) {
    if (out_dtype == MP_F32) {
      *reinterpret_cast<float4 *>(static_cast<float *>(out) + o) =
          make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else {
      uint16_t b[NC];
#pragma unroll
      for (int i = 0; i < NC; ++i) b[i] = out_dtype == MP_F16 ? mp_f2h(acc[i]) : mp_f2bf(acc[i]);
      *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + o) =
          make_uint2(b[0] | (static_cast<uint32_t>(b[1]) << 16), b[2] | (static_cast<uint32_t>(b[3]) << 16));
    }
  } else {
    mp_store_from_f32(out, o, out_dtype, acc[0]);
  }
}

}  // namespace

// ====================================================================== C ABI

extern "C" size_t mp_moe_route_workspace_bytes(int64_t t, int64_t h, int n_experts) {
  (void)t;
  (void)h;
  (void)n_experts;
  return 256;  // invalid-id counter (kept for future multi-workgroup routing)
}

extern "C" int mp_moe_permute_quant(const void *x, int x_dtype, const float *x_scale, int64_t t, int64_t h,
                                    const int32_t *topk_ids, int top_k, int n_experts, int scale_rule, int8_t *routed,
                                    float *routed_scale, int32_t *row_of_slot, int64_t *group_offsets, void *workspace,
                                    size_t workspace_bytes, mp_stream_t stream) {
  if (!x || !topk_ids || !routed || !routed_scale || !row_of_slot || !group_offsets) return MP_ERR_ARG;
  if (x_dtype != MP_F16 && x_dtype != MP_BF16 && x_dtype != MP_F32 && x_dtype != MP_I8) return MP_ERR_DTYPE;
  if (x_dtype == MP_I8 && !x_scale) return MP_ERR_ARG;
  if (scale_rule != MP_SCALE_FP32 && scale_rule != MP_SCALE_FAKE) return MP_ERR_ARG;
  if (scale_rule == MP_SCALE_FAKE && x_dtype == MP_F32) return MP_ERR_DTYPE;
  if (t < 0 || h <= 0 || top_k <= 0 || n_experts <= 0 || n_experts > kMaxExperts) return MP_ERR_SHAPE;
  if (t * top_k > INT32_MAX) return MP_ERR_SHAPE;
  if (workspace && workspace_bytes < mp_moe_route_workspace_bytes(t, h, n_experts)) return MP_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t n_assign = t * top_k;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(64 * kRouteWaves), 0, s, topk_ids, n_assign, n_experts, group_offsets,
                     row_of_slot, static_cast<int32_t *>(workspace));
  MP_CHECK_LAUNCH();
  if (n_assign == 0) return MP_OK;
  const dim3 g(static_cast<unsigned>(n_assign));
  if (x_dtype == MP_I8) {  // pre-quantized rows: routing only
    const int8_t *xq = static_cast<const int8_t *>(x);
    if (h % 16 == 0 && mp_aligned(x, 16) && mp_aligned(routed, 16))
      hipLaunchKernelGGL(moe_permute_rows_kernel<true>, g, dim3(256), 0, s, xq, x_scale, h, top_k, row_of_slot, routed,
                         routed_scale);
    else
      hipLaunchKernelGGL(moe_permute_rows_kernel<false>, g, dim3(256), 0, s, xq, x_scale, h, top_k, row_of_slot,
                         routed, routed_scale);
    MP_CHECK_LAUNCH();
    return MP_OK;
  }
  const int per16 = x_dtype == MP_F32 ? 4 : 8;  // values per 16 bytes
  const bool fake = scale_rule == MP_SCALE_FAKE;
  if (h % per16 == 0 && mp_aligned(x, 16) && mp_aligned(routed, 8)) {
#define MP_PQ_VEC(DT_, RULE_) \
  hipLaunchKernelGGL((moe_permute_quant_vec_kernel<DT_, RULE_>), g, dim3(256), 0, s, x, h, top_k, row_of_slot, routed, \
                     routed_scale)
    if (x_dtype == MP_F16) {
      if (fake) MP_PQ_VEC(MP_F16, MP_SCALE_FAKE);
      else MP_PQ_VEC(MP_F16, MP_SCALE_FP32);
    } else if (x_dtype == MP_BF16) {
      if (fake) MP_PQ_VEC(MP_BF16, MP_SCALE_FAKE);
      else MP_PQ_VEC(MP_BF16, MP_SCALE_FP32);
    } else {
      MP_PQ_VEC(MP_F32, MP_SCALE_FP32);
    }
#undef MP_PQ_VEC
  } else if (fake) {
    hipLaunchKernelGGL(moe_permute_quant_kernel<MP_SCALE_FAKE>, g, dim3(256), 0, s, x, x_dtype, h, top_k, row_of_slot,
                       routed, routed_scale);
  } else {
    hipLaunchKernelGGL(moe_permute_quant_kernel<MP_SCALE_FP32>, g, dim3(256), 0, s, x, x_dtype, h, top_k, row_of_slot,
                       routed, routed_scale);
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}

static int64_t gmm1_partials(int64_t inter) { return 2 * mp_cdiv(inter, 64); }

extern "C" size_t mp_moe_gmm1_workspace_bytes(int64_t rows, int64_t inter) {
  const size_t hbytes = static_cast<size_t>(rows) * static_cast<size_t>(inter) * sizeof(float);
  const size_t pbytes = static_cast<size_t>(rows) * static_cast<size_t>(gmm1_partials(inter)) * sizeof(float);
  return ((hbytes + 255) & ~static_cast<size_t>(255)) + pbytes;
}

extern "C" int mp_i8_gemm_swiglu_requant(const int8_t *routed, const float *routed_scale, const int8_t *w13,
                                         const float *s13, const int64_t *group_offsets, int n_experts,
                                         int64_t rows, int64_t h, int64_t inter, int scale_rule, int act_dtype,
                                         int8_t *q_out, float *s_out, void *workspace, size_t workspace_bytes,
                                         mp_stream_t stream) {
  if (!routed || !routed_scale || !w13 || !s13 || !group_offsets || !q_out || !s_out || !workspace)
    return MP_ERR_ARG;
  if (scale_rule != MP_SCALE_FP32 && scale_rule != MP_SCALE_FAKE) return MP_ERR_ARG;
  if (scale_rule == MP_SCALE_FAKE && act_dtype != MP_F16 && act_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (rows < 0 || h <= 0 || inter <= 0 || n_experts <= 0 || n_experts > kMaxExperts) return MP_ERR_SHAPE;
  if (h % 64 != 0 || h > (1 << 17)) return MP_ERR_SHAPE;
  if (workspace_bytes < mp_moe_gmm1_workspace_bytes(rows, inter)) return MP_ERR_WORKSPACE;
  if (rows == 0) return MP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float *hbuf = static_cast<float *>(workspace);
  const size_t hbytes = static_cast<size_t>(rows) * static_cast<size_t>(inter) * sizeof(float);
  float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) + ((hbytes + 255) & ~static_cast<size_t>(255)));
  const int mode = scale_rule == MP_SCALE_FAKE ? mp_round_mode_of(act_dtype) : kRoundNone;
  const int n_partial = static_cast<int>(gmm1_partials(inter));
  int rc;
  if (scale_rule == MP_SCALE_FAKE) {
    // the reference's F.linear on the fake-quant tensors: fp16 / bf16 MFMA on r(q * s) values
    // (the int8 product of the unrounded q * s moves gate / up by an ulp often enough to flip
    // requant codes: ~4e-3 of output error at Mixtral-like shapes)
    mp_dq_args d{};
    d.dt = act_dtype;
    d.a = routed;
    d.a_fmt = MP_DQ_I8ROW;
    d.a_scale = routed_scale;
    d.b = w13;
    d.b_fmt = MP_DQ_I8ROW;
    d.b_scale = s13;
    d.y = hbuf;
    d.out_dtype = MP_F32;
    d.ldy = inter;
    d.amax_partial = part;
    d.n_partial = n_partial;
    d.offsets = group_offsets;
    d.n_experts = n_experts;
    d.rows = rows;
    d.n = inter;
    d.k = h;
    rc = mp_launch_dq_gemm(d, MP_EPI_SWIGLU, s);
  } else {
    mp_i8_args a{};
    a.a = routed;
    a.s_a = routed_scale;
    a.b = w13;
    a.s_b = s13;
    a.y = hbuf;
    a.out_dtype = MP_F32;
    a.amax_partial = part;
    a.n_partial = n_partial;
    a.offsets = group_offsets;
    a.n_experts = n_experts;
    a.rows = rows;
    a.n = inter;
    a.k = h;
    a.ldy = inter;
    a.epi_round = mode;
    rc = mp_launch_i8_gemm(a, MP_EPI_SWIGLU, s);
  }
  if (rc != MP_OK) return rc;
  const bool vec = inter % 4 == 0 && mp_aligned(q_out, 4) && mp_aligned(hbuf, 16);
  const dim3 g(static_cast<unsigned>(rows));
#define MP_RQ(RULE_, SIGNED_, VEC_)                                                                              \
  hipLaunchKernelGGL((moe_requant_kernel<RULE_, SIGNED_, VEC_>), g, dim3(256), 0, s, hbuf, part, n_partial, inter, \
                     mode, q_out, s_out)
  if (scale_rule == MP_SCALE_FP32) {
    if (vec) MP_RQ(MP_SCALE_FP32, false, true);
    else MP_RQ(MP_SCALE_FP32, false, false);
  } else if (mode == kRoundBF16) {  // the bf16 codes reach +-128: the row's sign needs its extremes
    if (vec) MP_RQ(MP_SCALE_FAKE, true, true);
    else MP_RQ(MP_SCALE_FAKE, true, false);
  } else {
    if (vec) MP_RQ(MP_SCALE_FAKE, false, true);
    else MP_RQ(MP_SCALE_FAKE, false, false);
  }
#undef MP_RQ
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_w8a8_grouped_gemm(const int8_t *q, const float *s, const int8_t *w, const float *s_w,
                                    const int64_t *group_offsets, int n_experts, int64_t rows, int64_t n,
                                    int64_t k, int scale_rule, int act_dtype, void *y, int out_dtype,
                                    mp_stream_t stream) {
  if (!q || !s || !w || !s_w || !group_offsets || !y) return MP_ERR_ARG;
  if (out_dtype != MP_F32 && out_dtype != MP_F16 && out_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (scale_rule != MP_SCALE_FP32 && scale_rule != MP_SCALE_FAKE) return MP_ERR_ARG;
  if (rows < 0 || n <= 0 || k <= 0 || n_experts <= 0 || n_experts > kMaxExperts) return MP_ERR_SHAPE;
  if (scale_rule == MP_SCALE_FAKE) {
    if (act_dtype != MP_F16 && act_dtype != MP_BF16) return MP_ERR_DTYPE;
    if (k > (1 << 20)) return MP_ERR_SHAPE;
    if (rows == 0) return MP_OK;
    mp_dq_args d{};
    d.dt = act_dtype;
    d.a = q;
    d.a_fmt = MP_DQ_I8ROW;
    d.a_scale = s;
    d.b = w;
    d.b_fmt = MP_DQ_I8ROW;
    d.b_scale = s_w;
    d.y = y;
    d.out_dtype = out_dtype;
    d.ldy = n;
    d.offsets = group_offsets;
    d.n_experts = n_experts;
    d.rows = rows;
    d.n = n;
    d.k = k;
    return mp_launch_dq_gemm(d, out_dtype == MP_F32 ? MP_EPI_F32 : MP_EPI_DENSE, reinterpret_cast<hipStream_t>(stream));
  }
  if (k % 64 != 0 || k > (1 << 17)) return MP_ERR_SHAPE;
  if (rows == 0) return MP_OK;
  mp_i8_args a{};
  a.a = q;
  a.s_a = s;
  a.b = w;
  a.s_b = s_w;
  a.y = y;
  a.out_dtype = out_dtype;
  a.offsets = group_offsets;
  a.n_experts = n_experts;
  a.rows = rows;
  a.n = n;
  a.k = k;
  a.ldy = n;
  return mp_launch_i8_gemm(a, out_dtype == MP_F32 ? MP_EPI_F32 : MP_EPI_DENSE, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int mp_moe_unpermute_combine(const float *y, const int32_t *row_of_slot, const float *topk_w, int64_t t,
                                        int top_k, int64_t h, int scale_rule, void *out, int out_dtype,
                                        mp_stream_t stream) {
  if (!y || !row_of_slot || !topk_w || !out) return MP_ERR_ARG;
  if (out_dtype != MP_F32 && out_dtype != MP_F16 && out_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (scale_rule != MP_SCALE_FP32 && scale_rule != MP_SCALE_FAKE) return MP_ERR_ARG;
  if (scale_rule == MP_SCALE_FAKE && out_dtype == MP_F32) return MP_ERR_DTYPE;
  if (t < 0 || top_k <= 0 || top_k > 64 || h <= 0) return MP_ERR_SHAPE;
  if (t == 0) return MP_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool vec = h % 4 == 0 && mp_aligned(y, 16) && mp_aligned(out, out_dtype == MP_F32 ? 16 : 8);
  const dim3 g(static_cast<unsigned>(mp_cdiv(vec ? t * (h / 4) : t * h, 256)));
#define MP_CB(FAKE_, VEC_) \
  hipLaunchKernelGGL((moe_combine_kernel<FAKE_, VEC_>), g, dim3(256), 0, st, y, row_of_slot, topk_w, t, top_k, h, out, \
                     out_dtype)
  if (scale_rule == MP_SCALE_FAKE) {
    if (vec) MP_CB(true, true);
    else MP_CB(true, false);
  } else {
    if (vec) MP_CB(false, true);
    else MP_CB(false, false);
  }
#undef MP_CB
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// ---------------------------------------------------------------- allocation-free GMM1
// mp_i8_gemm_swiglu_requant with its scratch (the fp32 SwiGLU rows and the per-row abs-max
// partials) in a library-owned device array instead of a caller workspace, for callers that
// cannot allocate.  Each GPU holds its own copy of `scratch` (64 MiB, until the process ends);
// host code never passes the array's name to a kernel (that is a host-side stand-in): the
// device address comes from hipGetSymbolAddress, once per device, on the first call with that
// device current.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// race.  Nothing in it has to start at zero -- the requant reads only rows and partials the
// GEMM epilogue wrote in the same call.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kNoAllocMaxDevices] = {};

static int mp_scratch_address(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) return MP_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return MP_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MP_OK;
}

extern "C" int mp_i8_gemm_swiglu_requant_noalloc(const int8_t *routed, const float *routed_scale, const int8_t *w13,
                                                 const float *s13, const int64_t *group_offsets, int n_experts,
                                                 int64_t rows, int64_t h, int64_t inter, int scale_rule,
                                                 int act_dtype, int8_t *q_out, float *s_out, mp_stream_t stream) {
  if (rows < 0 || inter <= 0) return MP_ERR_SHAPE;
  if (mp_moe_gmm1_workspace_bytes(rows, inter) > kNoAllocScratchBytes) return MP_ERR_WORKSPACE;
  void *ws = nullptr;
  const int rc = mp_scratch_address(&ws);
  if (rc != MP_OK) return rc;
  return mp_i8_gemm_swiglu_requant(routed, routed_scale, w13, s13, group_offsets, n_experts, rows, h, inter,
                                   scale_rule, act_dtype, q_out, s_out, ws, kNoAllocScratchBytes, stream);
}

// ---------------------------------------------------------------- misc
extern "C" const char *mp_strerror(int status) {
  switch (status) {
    case MP_OK: return "ok";
    case MP_ERR_SHAPE: return "mindpipe_amd: unsupported shape or group size";
    case MP_ERR_DTYPE: return "mindpipe_amd: unsupported dtype";
    case MP_ERR_ALIGN: return "mindpipe_amd: pointer alignment (16 bytes required)";
    case MP_ERR_HIP: return "mindpipe_amd: HIP kernel launch failed";
    case MP_ERR_ARG: return "mindpipe_amd: missing buffer or bad enum argument";
    case MP_ERR_WORKSPACE: return "mindpipe_amd: workspace too small";
    default: return "mindpipe_amd: unknown status";
  }
}

extern "C" int mp_abi_version(void) { return 2; }
