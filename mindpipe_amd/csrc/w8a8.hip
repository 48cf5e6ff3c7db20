// W8A8 for gfx950: per-token / per-channel int8 quantizers and the int8 MFMA
// GEMM with the per-token x per-channel scale epilogue (dense and grouped).
#include "dq_gemm.h"
#include <type_traits>

namespace {

// ------------------------------------------------------------------ row quantizer
// One 256-thread workgroup per row.  Pass 1: abs-max (and, for the fake rule, the largest
// and smallest value: the sign rule of mp_fake_row_sign); pass 2: codes (the row is re-read
// from L2).  RULE selects the scale arithmetic (see mp_scale_rule): MP_SCALE_FP32, or
// MP_SCALE_FAKE in the input dtype (fp16 / bf16) with the stored scale signed like the row.
template <int RULE>
__global__ __launch_bounds__(256) void rowquant_kernel(const void *__restrict__ x, int x_dtype, int64_t k,
                                                       int8_t *__restrict__ q, float *__restrict__ s_f32,
                                                       uint16_t *__restrict__ s_src, int s_src_bf16,
                                                       float min_scale, int32_t *__restrict__ bad) {
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = row * k;
  const int mode = mp_round_mode_of(x_dtype);
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  for (int64_t c = tid; c < k; c += 256) {
    const float v = mp_load_as_f32(x, base + c, x_dtype);
    st.bad |= !isfinite(v);
    st.amax = fmaxf(st.amax, fabsf(v));
    st.vmax = fmaxf(st.vmax, v);
    st.vmin = fminf(st.vmin, v);
  }
  st = mp_block_rowstat(st, red, wbad);
  float s, sg;
  mp_row_scale<RULE>(st, mode, min_scale, s, sg);
  if (tid == 0) {
    if (s_f32) s_f32[row] = sg * s;
    if (s_src) s_src[row] = s_src_bf16 ? mp_f2bf(sg * s) : mp_f2h(sg * s);
    if (bad && st.bad) atomicAdd(bad, 1);
  }
  for (int64_t c = tid; c < k; c += 256) {
    const float v = mp_load_as_f32(x, base + c, x_dtype);
    q[base + c] = static_cast<int8_t>(mp_row_code<RULE>(v, s, sg, mode));
  }
}

// The fake per-row rule at a code width of 2..7 bits (quantize_*_absmax with n_bits < 8,
// fake_quant.py:10-31): q_max = 2^(n-1) - 1, s = r(r(max(amax, 1e-5)) / q_max), code =
// rint(r(v / s)), every op rounded to the input dtype.  |r(v / s)| stays below q_max + 1 (s is
// within half an ulp of amax / q_max), so the codes fit int8 and need no sign rule.
__global__ __launch_bounds__(256) void fake_rows_nbit_kernel(const void *__restrict__ x, int x_dtype, int64_t k,
                                                             float q_max, int8_t *__restrict__ q,
                                                             float *__restrict__ s_out) {
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = row * k;
  const int mode = mp_round_mode_of(x_dtype);
  mp_rowstat st{0.f, 0.f, 0.f, 0};
  for (int64_t c = tid; c < k; c += 256) st.amax = fmaxf(st.amax, fabsf(mp_load_as_f32(x, base + c, x_dtype)));
  st = mp_block_rowstat(st, red, wbad);
  float a = mp_round_mode_apply(st.amax, mode);
  if (a < 1e-5f) a = mp_round_mode_apply(1e-5f, mode);
  const float s = mp_round_mode_apply(a / q_max, mode);
  if (tid == 0) s_out[row] = s;
  for (int64_t c = tid; c < k; c += 256) {
    const float v = mp_load_as_f32(x, base + c, x_dtype);
    const float code = rintf(mp_round_mode_apply(v / s, mode));
    q[base + c] = static_cast<int8_t>(static_cast<int>(fminf(fmaxf(code, -128.f), 127.f)));
  }
}

// The same quantizer with 16-byte loads and 4- or 8-byte code stores (k a multiple of the
// values per 16 bytes, 16-byte aligned rows); the per-element arithmetic is the same.
template <int RULE, int DT>
__global__ __launch_bounds__(256) void rowquant_vec_kernel(const void *__restrict__ x, int64_t k,
                                                           int8_t *__restrict__ q, float *__restrict__ s_f32,
                                                           uint16_t *__restrict__ s_src, int s_src_bf16,
                                                           float min_scale, int32_t *__restrict__ bad) {
  constexpr int N = MpChunk16<DT>::N, ESZ = DT == MP_F32 ? 4 : 2;
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nch = k / N;
  const int mode = DT == MP_F16 ? kRoundF16 : (DT == MP_BF16 ? kRoundBF16 : kRoundNone);
  const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const char *>(x) + row * k * ESZ);
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  for (int64_t c = tid; c < nch; c += 256) {
    float f[N];
    mp_chunk_to_f32<DT>(src[c], f);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      st.bad |= !isfinite(f[i]);
      st.amax = fmaxf(st.amax, fabsf(f[i]));
      if (RULE != MP_SCALE_FP32) {
        st.vmax = fmaxf(st.vmax, f[i]);
        st.vmin = fminf(st.vmin, f[i]);
      }
    }
  }
  st = mp_block_rowstat(st, red, wbad);
  float s, sg;
  mp_row_scale<RULE>(st, mode, min_scale, s, sg);
  if (tid == 0) {
    if (s_f32) s_f32[row] = sg * s;
    if (s_src) s_src[row] = s_src_bf16 ? mp_f2bf(sg * s) : mp_f2h(sg * s);
    if (bad && st.bad) atomicAdd(bad, 1);
  }
  int8_t *dst = q + row * k;
  for (int64_t c = tid; c < nch; c += 256) {
    float f[N];
    mp_chunk_to_f32<DT>(src[c], f);
    uint32_t w[N / 4];
#pragma unroll
    for (int g = 0; g < N / 4; ++g) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) word |= mp_row_code<RULE>(f[4 * g + e], s, sg, mode) << (8 * e);
      w[g] = word;
    }
    if constexpr (N == 8) *reinterpret_cast<uint2 *>(dst + c * 8) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t *>(dst + c * 4) = w[0];
  }
}

// ------------------------------------------------------------------ decode GEMV (M <= 64)
// 16-byte activation pieces a thread of an NT-thread skinny workgroup stages per K chunk; a chunk
// holds at most skinny_pmax(NT) * NT pieces (the launcher sizes chunks to that).
constexpr int skinny_pmax(int nt) { return kMpXLdsBudget / 16 / nt + 1; }

// One workgroup of NW waves per 16 output columns; each wave takes a contiguous
// range of 64-byte K blocks, and the waves are summed exactly (int32) through LDS.  The int8
// activations are staged once per workgroup into LDS (K chunks within the LDS
// budget).  MFMA i32_16x16x64_i8: B = weight rows straight from HBM (16 B per
// lane), A = activations from LDS (row m = lane%16, zero beyond M).  Weight
// loads are double-buffered, U blocks per buffer.
template <int MT, int NW>
__global__ __launch_bounds__(NW * 64) void i8_skinny_kernel(mp_i8_args p, int cb) {
  // Straight-line hot path (clamped loads, masked surplus blocks): control-flow
  // joins make the compiler wait for every outstanding load.
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int U = 4;
  constexpr int NT = NW * 64;
  const int xstride = cb * 64 + 16;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_cols = static_cast<int>(p.n);
  const int k = static_cast<int>(p.k);
  const int m_rows = static_cast<int>(p.rows);
  const int n = blockIdx.x * 16 + (lane & 15);
  const int nn = n < n_cols ? n : n_cols - 1;
  const int kq = lane >> 4;
  const int nblk = k >> 6;
  const int mlast = m_rows - 1;
  uint8_t *dummy = smem + m_rows * xstride;
  const int8_t *wrow = p.b + static_cast<int64_t>(nn) * k + 16 * kq;
  i4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = i4_t{0, 0, 0, 0};
  i4_t wa[U], wb[U];

  for (int c0 = 0; c0 < nblk; c0 += cb) {
    const int cbn = (nblk - c0) < cb ? (nblk - c0) : cb;
    // contiguous block range per wave: consecutive loads of a wave read the two halves
    // of each 128-byte weight line (round-robin blocks would leave every line half used)
    const int per = (cbn + NW - 1) / NW;
    const int jlo = wave * per;
    const int nmine = cbn > jlo ? (cbn - jlo < per ? cbn - jlo : per) : 0;
    const int rmax = nmine > 0 ? nmine - 1 : 0;
    const int bmax = c0 + cbn - 1;
    auto issue = [&](i4_t *w, int r0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = (r0 + u) < rmax ? (r0 + u) : rmax;
        int b = c0 + jlo + r;
        b = b < bmax ? b : bmax;
        w[u] = *reinterpret_cast<const i4_t *>(wrow + b * 64);
      }
    };
    auto compute = [&](const i4_t *w, int r0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u;
        const bool live = r < nmine;
        int jl = jlo + (r < rmax ? r : rmax);
        jl = jl < cbn - 1 ? jl : cbn - 1;
        const i4_t wv = live ? w[u] : i4_t{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int ma = t * 16 + (lane & 15);
          const int mac = ma < mlast ? ma : mlast;
          i4_t a = *reinterpret_cast<const i4_t *>(smem + mac * xstride + jl * 64 + 16 * kq);
          a = ma < m_rows ? a : i4_t{0, 0, 0, 0};
          acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wv, acc[t], 0, 0, 0);
        }
      }
    };
    constexpr int PMAX = skinny_pmax(NT);
    const int pieces = m_rows * cbn * 4;  // <= PMAX * NT: the launcher's chunk rule
    i4_t xv[PMAX];
#pragma unroll
    for (int i = 0; i < PMAX; ++i) {
      int q = tid + i * NT;
      q = q < pieces ? q : pieces - 1;
      const int m = q / (cbn * 4), c16 = q % (cbn * 4);
      xv[i] = *reinterpret_cast<const i4_t *>(p.a + static_cast<int64_t>(m) * k + c0 * 64 + c16 * 16);
    }
    issue(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (c0 > 0) mp_lds_barrier();
#pragma unroll
    for (int i = 0; i < PMAX; ++i) {
      const int q = tid + i * NT;
      const int qc = q < pieces ? q : pieces - 1;
      const int m = qc / (cbn * 4), c16 = qc % (cbn * 4);
      uint8_t *dst = q < pieces ? smem + m * xstride + c16 * 16 : dummy;
      *reinterpret_cast<i4_t *>(dst) = xv[i];
    }
    mp_lds_barrier();
    const int ngrp = (nmine + U - 1) / U;
    for (int g = 0; g < ngrp; g += 2) {
      if (g + 1 < ngrp) issue(wb, (g + 1) * U);
      __builtin_amdgcn_sched_barrier(0);
      compute(wa, g * U);
      if (g + 1 >= ngrp) break;
      if (g + 2 < ngrp) issue(wa, (g + 2) * U);
      __builtin_amdgcn_sched_barrier(0);
      compute(wb, (g + 1) * U);
    }
  }
  mp_lds_barrier();
  int *red = reinterpret_cast<int *>(smem);  // [NW][MT][4][64]
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * MT + t) * 4 + i) * 64 + lane] = acc[t][i];
  mp_lds_barrier();
  for (int o = tid; o < MT * 256; o += NT) {
    const int t = o >> 8, r = o & 255;
    const int l = r & 63, i = r >> 6;
    int v = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[((w * MT + t) * 4 + i) * 64 + l];
    const int m = t * 16 + 4 * (l >> 4) + i;
    const int col = blockIdx.x * 16 + (l & 15);
    if (m < m_rows && col < n_cols) {
      float yv = mp_mul(mp_mul(static_cast<float>(v), p.s_a[m]), p.s_b[col]);
      if (p.bias) yv = mp_add(yv, mp_load_as_f32(p.bias, col, p.bias_dtype));
      mp_store_from_f32(p.y, static_cast<int64_t>(m) * p.ldy + col, p.out_dtype, yv);
    }
  }
}

// 16 bytes per lane from a buffer into LDS (lane l at byte 16 l of the wave-uniform lds address).  The
// cast to an LDS pointer stays in this non-template function: inside a kernel template, with an operand
// that depends on a template parameter, it makes the host pass drop the kernel's launch stub.
__device__ __forceinline__ void mid_lds_load16(__amdgpu_buffer_rsrc_t r, int8_t *lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(lds)), 16, voff, 0, 0,
      0);
}

// Skinny GEMM (M <= 32) with direct global->LDS loads: a workgroup of four waves per 16 NCT output
// columns, each wave a contiguous quarter of K in 128-byte steps, streaming its activation rows (16 MT)
// and the workgroup's weight rows (16 NCT) into a ring of three LDS stages of its own, two steps ahead,
// by `buffer_load_dwordx4 ... lds` (lane l at byte 16 l of 8 rows x 128 B; chunk c of row r at slot
// c ^ ((r >> 1) & 7)).  The rings are wave-private, so a step waits only for the wave's own loads and
// LDS reads (no barrier in the K loop).  MFMA i32_16x16x64_i8 (A: activation row lane % 16, B: weight
// row lane % 16, 16 bytes of a 64-byte K piece per lane).  Rows past M and N sit past their buffer
// descriptors (zeros, no memory access).  The four waves' int32 sums meet in LDS; the epilogue is
// i8_skinny_kernel's, so the outputs are the same bits.
constexpr int kSdStages = 3;
constexpr size_t skdma_smem(int mt, int nct) {
  return static_cast<size_t>(4) * kSdStages * (16 * mt + 16 * nct) * 128;
}

template <int MT, int NCT>
__global__ __launch_bounds__(256) void i8_skinny_dma_kernel(mp_i8_args p) {
  constexpr int S = kSdStages, BK = 128;
  constexpr int AR = 16 * MT, BR = 16 * NCT;                // activation / weight rows per stage
  constexpr int QA = AR / 8, QB = BR / 8, QW = QA + QB;     // load instructions per stage
  constexpr int STAGE = (AR + BR) * BK;
  constexpr uint32_t kOob = 0x80000000u;
  extern __shared__ __attribute__((aligned(16))) int8_t smem_sd[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int8_t *ring = smem_sd + wave * S * STAGE;
  const int64_t k = p.k;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BR;
  const int64_t b_rows = p.n - n0 < BR ? p.n - n0 : BR;
  const __amdgpu_buffer_rsrc_t arsrc = mp_rsrc(p.a, static_cast<uint32_t>(p.rows * k));
  const __amdgpu_buffer_rsrc_t brsrc = mp_rsrc(p.b + n0 * k, static_cast<uint32_t>(b_rows * k));
  // this wave's K steps [s0, s1)
  const int nkt = static_cast<int>(k / BK);
  const int s0 = nkt * wave / 4, s1 = nkt * (wave + 1) / 4;
  uint32_t voff[QW];
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const bool is_a = q < QA;
    const int r = (is_a ? q : q - QA) * 8 + lane / 8;
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    voff[q] = r < (is_a ? p.rows : b_rows) ? static_cast<uint32_t>(r * k + 16 * c) : kOob;
  }
  auto issue = [&](int step, int slot) {
    const bool live = step < s1;
    const uint32_t kb = static_cast<uint32_t>(step) * BK;
#pragma unroll
    for (int q = 0; q < QW; ++q)
      mid_lds_load16(q < QA ? arsrc : brsrc, ring + slot * STAGE + (q < QA ? q * 8 : AR + (q - QA) * 8) * BK,
                     live && voff[q] != kOob ? voff[q] + kb : kOob);
  };
  i4_t acc[NCT][MT];
#pragma unroll
  for (int j = 0; j < NCT; ++j)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[j][t] = i4_t{0, 0, 0, 0};
  const int swz = (lane >> 1) & 7, kq = lane >> 4, row = lane & 15;
  auto compute = [&](int slot) {
    const int8_t *st = ring + slot * STAGE;
    i4_t af[2][MT], bf[2][NCT];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int sl = 16 * ((4 * ks + kq) ^ swz);
#pragma unroll
      for (int t = 0; t < MT; ++t) af[ks][t] = *reinterpret_cast<const i4_t *>(st + (16 * t + row) * BK + sl);
#pragma unroll
      for (int j = 0; j < NCT; ++j) bf[ks][j] = *reinterpret_cast<const i4_t *>(st + (AR + 16 * j + row) * BK + sl);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < NCT; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[j][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[ks][t], bf[ks][j], acc[j][t], 0, 0, 0);
  };
  issue(s0, 0);
  issue(s0 + 1, 1);
  int slot = 0;
  for (int s = s0; s < s1; ++s) {
    // own loads of step s landed (the next step's may remain) and own reads of the slot refilled next
    // are done; the ring is this wave's alone
    if constexpr (QW == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
    else if constexpr (QW == 6) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
    else if constexpr (QW == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    else if constexpr (QW == 10) asm volatile("s_waitcnt vmcnt(10) lgkmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)" ::: "memory");
    static_assert(QW >= 4 && QW <= 12 && QW % 2 == 0, "the wait counts one stage of loads");
    issue(s + 2, slot == 0 ? 2 : slot - 1);
    compute(slot);
    slot = slot == S - 1 ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS DMA outstanding past this point
  mp_lds_barrier();                                 // every ring is done: reuse LDS for the sums
  int *red = reinterpret_cast<int *>(smem_sd);      // [4][NCT * MT][4][64]
#pragma unroll
  for (int j = 0; j < NCT; ++j)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * NCT * MT + j * MT + t) * 4 + i) * 64 + lane] = acc[j][t][i];
  mp_lds_barrier();
  for (int o = tid; o < NCT * MT * 256; o += 256) {
    const int jt = o >> 8, r = o & 255;
    const int j = jt / MT, t = jt % MT;
    const int l = r & 63, i = r >> 6;
    int v = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) v += red[((w * NCT * MT + jt) * 4 + i) * 64 + l];
    const int64_t m = t * 16 + 4 * (l >> 4) + i;
    const int64_t col = n0 + j * 16 + (l & 15);
    if (m < p.rows && col < p.n) {
      float yv = mp_mul(mp_mul(static_cast<float>(v), p.s_a[m]), p.s_b[col]);
      if (p.bias) yv = mp_add(yv, mp_load_as_f32(p.bias, col, p.bias_dtype));
      mp_store_from_f32(p.y, m * p.ldy + col, p.out_dtype, yv);
    }
  }
}

// ------------------------------------------------------------------ GEMV (M <= 2)
// A wave owns R weight rows over all of K.  In chunk j lane l covers K bytes
// [1024 j + 16 l, +16), so each weight load reads 1 KB of one row contiguously
// (a load whose lanes touch 16 rows costs the CU several times the issue slots)
// and the MR activation rows come the same way; v_dot4_i32_i8 multiplies
// exactly.  C chunks are issued before any is used.  Lanes past K, and
// activation rows past M, load beyond their buffer: zeros, no memory access.  A
// wave butterfly sums the int32 partials exactly; the epilogue is the shared
// (acc * s_tok) * s_ch (+ bias) of the other kernels, so the outputs are the same
// bits.
template <int R, int MR, int C>
__global__ __launch_bounds__(256) void i8_gemv_kernel(mp_i8_args p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_cols = static_cast<int>(p.n);
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= n_cols) return;  // wave-uniform; no barrier in the kernel
  const uint32_t k = static_cast<uint32_t>(p.k);
  const int m_rows = static_cast<int>(p.rows);
  const uint32_t wbytes = static_cast<uint32_t>(n_cols) * k;
  const uint32_t xbytes = static_cast<uint32_t>(m_rows) * k;
  const auto wr = mp_rsrc(p.b, wbytes);
  const auto xr = mp_rsrc(p.a, xbytes);
  uint32_t wbase[R], xbase[MR];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = row0 + r < n_cols ? row0 + r : n_cols - 1;
    wbase[r] = static_cast<uint32_t>(n) * k;
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) xbase[m] = m < m_rows ? static_cast<uint32_t>(m) * k : xbytes;
  const int nch = static_cast<int>((k + 1023u) / 1024u);
  int acc[MR][R];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0;
  for (int j0 = 0; j0 < nch; j0 += C) {
    i4_t w[C][R], xv[C][MR];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const uint32_t kx = static_cast<uint32_t>(j0 + c) * 1024u + 16u * lane;
      const bool live = kx < k;  // chunks past nch give kx >= k too
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint4 v = mp_buf_load16(wr, live ? wbase[r] + kx : wbytes, 0);
        w[c][r] = i4_t{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const uint4 v = mp_buf_load16(xr, live ? xbase[m] + kx : xbytes, 0);
        xv[c][m] = i4_t{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[m][r] = __builtin_amdgcn_sdot4(xv[c][m][e], w[c][r][e], acc[m][r], false);
  }
  // exact int32 sums over the 64 lanes
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) acc[m][r] += __shfl_xor(acc[m][r], o, 64);
  // lane m * R + r stores output (m, row0 + r)
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int col = row0 + r;
      if (lane == m * R + r && m < m_rows && col < n_cols) {
        float yv = mp_mul(mp_mul(static_cast<float>(acc[m][r]), p.s_a[m]), p.s_b[col]);
        if (p.bias) yv = mp_add(yv, mp_load_as_f32(p.bias, col, p.bias_dtype));
        mp_store_from_f32(p.y, static_cast<int64_t>(m) * p.ldy + col, p.out_dtype, yv);
      }
    }
}

// ------------------------------------------------------------------ tiled GEMM
// BM x BN output tile per workgroup of 4 waves (2 x 2, each (BM/2) x (BN/2)
// built from MFMA i32_32x32x32_i8 tiles), BK-byte K steps, LDS double buffer
// with a 16-byte row pad (conflict-free ds_read_b128 for the MFMA fragments),
// D + 1 K tiles in flight in registers (a workgroup per CU or fewer: the loads'
// latency must be covered by the workgroup's own MFMA time).
// Grouped mode maps blockIdx.y to (expert, row tile) by walking the
// cumulative row offsets; surplus tiles exit.
template <int BM, int BN, int BK, int EPI, int D = 0>
__global__ __launch_bounds__(256) void i8_tiled_kernel(mp_i8_args p) {
  constexpr int LD = BK + 16;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int CA = BM * BK / 16 / 256;  // 16-byte chunks per thread
  constexpr int CB = BN * BK / 16 / 256;
  constexpr int CPR = BK / 16;            // chunks per row
  static_assert(EPI != MP_EPI_SWIGLU || TN == 2, "SwiGLU pairs gate/up in one wave");
  __shared__ __attribute__((aligned(16))) int8_t sa[2][BM * LD];
  __shared__ __attribute__((aligned(16))) int8_t sb[2][BN * LD];
  // fp32 / 16-bit epilogues: per-token scales of the tile's rows, then the column scales
  // and biases (fp32) of its columns, staged once so the epilogue reads no global memory
  // (a global load there waits for every store issued before it)
  __shared__ __attribute__((aligned(16))) float tscale[BM + 2 * BN];
  static_assert(BM + BN == 256, "one epilogue scale per thread");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int64_t row_begin, row_end;
  int e = 0;
  int tile_n = blockIdx.x;
  if (p.offsets) {
    int64_t slot = blockIdx.y;
    bool found = false;
    for (e = 0; e < p.n_experts; ++e) {
      const int64_t lo = p.offsets[e], hi = p.offsets[e + 1];
      const int64_t tiles = (hi - lo + BM - 1) / BM;
      if (slot < tiles) {
        row_begin = lo + slot * BM;
        row_end = hi < row_begin + BM ? hi : row_begin + BM;
        found = true;
        break;
      }
      slot -= tiles;
    }
    if (!found) return;
  } else if (p.xcd_row_tiles > 0) {
    // 1-D grid: row tile (x / 8) % T of column tile (x / 8T) * 8 + x % 8, so the T row tiles of a
    // column tile run on one XCD at nearly the same time and share its weight rows in L2
    const int tr = p.xcd_row_tiles, bx = blockIdx.x;
    tile_n = (bx / (8 * tr)) * 8 + (bx & 7);
    row_begin = static_cast<int64_t>((bx >> 3) % tr) * BM;
    if (static_cast<int64_t>(tile_n) * BN >= p.n || row_begin >= p.rows) return;  // padding; uniform
    row_end = p.rows < row_begin + BM ? p.rows : row_begin + BM;
  } else {
    row_begin = static_cast<int64_t>(blockIdx.y) * BM;
    row_end = p.rows < row_begin + BM ? p.rows : row_begin + BM;
  }
  const int64_t k = p.k;
  const int64_t n_out = p.n;
  const int64_t nb_rows = (EPI == MP_EPI_SWIGLU) ? 2 * n_out : n_out;  // weight rows per expert
  const int8_t *bexp = p.b + static_cast<int64_t>(e) * nb_rows * k;
  const float *sbexp = p.s_b + static_cast<int64_t>(e) * nb_rows;
  const int64_t col0 = static_cast<int64_t>(tile_n) * ((EPI == MP_EPI_SWIGLU) ? BN / 2 : BN);

  // A chunks through a descriptor over the tile's rows: a chunk of a row past row_end sits
  // past the descriptor and reads zeros, so every thread issues the same loads with no branch
  // (a branch around a load makes the compiler's waits count only the loads every path issues,
  // which drains the register stages early).  The launcher bounds BM * K below 2^31.
  const __amdgpu_buffer_rsrc_t arsrc = mp_rsrc(p.a + row_begin * p.k, static_cast<uint32_t>((row_end - row_begin) * p.k));
  uint32_t aoff[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int c = tid + i * 256;
    const int64_t lr = c / CPR;
    aoff[i] = row_begin + lr < row_end ? static_cast<uint32_t>(lr * p.k + (c % CPR) * 16) : 0x80000000u;
  }
  const int8_t *bsrc[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) {
    const int c = tid + i * 256;
    const int lr = c / CPR;
    int64_t wr;
    if (EPI == MP_EPI_SWIGLU) {
      const int64_t oc = col0 + (lr % (BN / 2));
      const int64_t occ = oc < n_out ? oc : n_out - 1;
      wr = (lr < BN / 2) ? occ : n_out + occ;
    } else {
      const int64_t oc = col0 + lr;
      wr = oc < n_out ? oc : n_out - 1;
    }
    bsrc[i] = bexp + wr * k + (c % CPR) * 16;
  }

  // Epilogue scales, loaded before the tiles (one load of each kind on every thread, past
  // a descriptor or clamped where the thread owns none: the load count is the same on
  // every path, so the waits below stay partial): thread t < BM the per-token scale of
  // row row_begin + t (zero past row_end), t >= BM the scale and bias of column
  // col0 + t - BM (clamped).
  constexpr bool STAGED_SCALES = EPI != MP_EPI_SWIGLU;
  float ts_a = 0.f, ts_b = 0.f, ts_bias = 0.f;
  if constexpr (STAGED_SCALES) {
    ts_a = __uint_as_float(mp_buf_load4(mp_rsrc(p.s_a + row_begin, static_cast<uint32_t>((row_end - row_begin) * 4)),
                                        tid < BM ? static_cast<uint32_t>(tid) * 4 : 0x80000000u, 0));
    int64_t c = col0 + ((tid - BM) & (BN - 1));
    c = c < n_out ? c : n_out - 1;
    ts_b = sbexp[c];
    if (EPI == MP_EPI_DENSE) {
      const bool hb = p.bias != nullptr;
      const float bv = mp_load_as_f32(hb ? p.bias : static_cast<const void *>(sbexp), c, hb ? p.bias_dtype : MP_F32);
      ts_bias = hb ? bv : 0.f;
    }
  }

  // D + 1 register stages of tiles in flight.  Loads are unconditional (clamped to
  // the last tile), so every wait is a partial vmcnt.
  i4_t areg[D + 1][CA], breg[D + 1][CB];
  const int64_t nkt = k / BK;
  auto load_tile = [&](int set, int64_t kt) {
    kt = kt < nkt ? kt : nkt - 1;
    const int64_t off = kt * BK;
#pragma unroll
    for (int i = 0; i < CA; ++i) areg[set][i] = mp_buf_load16i(arsrc, aoff[i], static_cast<uint32_t>(off));
#pragma unroll
    for (int i = 0; i < CB; ++i) breg[set][i] = *reinterpret_cast<const i4_t *>(bsrc[i] + off);
  };
  auto store_tile = [&](int set, int buf) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<i4_t *>(&sa[buf][(c / CPR) * LD + (c % CPR) * 16]) = areg[set][i];
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<i4_t *>(&sb[buf][(c / CPR) * LD + (c % CPR) * 16]) = breg[set][i];
    }
  };

  i16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // LDS rows read by this lane's fragments
  int arow_l[TM], brow_l[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) arow_l[i] = (wm * WM + i * 32 + (lane & 31)) * LD + 16 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int lr = (EPI == MP_EPI_SWIGLU) ? (j * (BN / 2) + wn * 32 + (lane & 31))
                                          : (wn * WN + j * 32 + (lane & 31));
    brow_l[j] = lr * LD + 16 * (lane >> 5);
  }
  auto mma = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      i4_t af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const i4_t *>(&sa[cur][arow_l[i] + ks * 32]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const i4_t *>(&sb[cur][brow_l[j] + ks * 32]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // Register set s holds tile t with t % (D + 1) == s; at step kt tiles kt+1 .. kt+D+1
  // are in flight.  Tile kt+1 goes to LDS after tile kt is multiplied, and its set is
  // refilled with tile kt+D+2.
  // (barriers wait for LDS traffic only: the prefetched global loads stay in flight)
#pragma unroll
  for (int d = 0; d <= D; ++d) load_tile(d, d);
  store_tile(0, 0);
  load_tile(0, D + 1);
  mp_lds_barrier();
  if constexpr (STAGED_SCALES) {  // read in the epilogue, after the K loop's barriers
    tscale[tid] = tid < BM ? ts_a : ts_b;
    if (tid >= BM) tscale[BN + tid] = ts_bias;  // waves 2-3: uniform
  }
  for (int64_t kt0 = 0; kt0 < nkt; kt0 += D + 1) {
#pragma unroll
    for (int d = 0; d <= D; ++d) {
      const int64_t kt = kt0 + d;
      const int nxt = (d + 1) % (D + 1);
      if (kt < nkt) {  // workgroup-uniform
        mma(static_cast<int>(kt & 1));
        if (kt + 1 < nkt) store_tile(nxt, static_cast<int>((kt + 1) & 1));
      }
      load_tile(nxt, kt + D + 2);
      mp_lds_barrier();
    }
  }

  // ---------------------------------------------------------------- epilogues
  if (EPI == MP_EPI_SWIGLU) {
    const int64_t col = col0 + wn * 32 + (lane & 31);
    const bool cval = col < n_out;
    const int64_t colc = cval ? col : n_out - 1;
    const float sg = sbexp[colc], su = sbexp[n_out + colc];
    float *hbuf = static_cast<float *>(p.y);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = row_begin + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const bool mval = m < row_end;
        const float sa_m = mval ? p.s_a[m] : 0.f;
        const float g = mp_mul(mp_mul(static_cast<float>(acc[i][0][r]), sa_m), sg);
        const float u = mp_mul(mp_mul(static_cast<float>(acc[i][1][r]), sa_m), su);
        const float h = mp_swiglu_epi(g, u, p.epi_round);
        if (mval && cval) hbuf[m * p.ldy + col] = h;
        float a = (mval && cval) ? fabsf(h) : 0.f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        if ((lane & 31) == 0 && mval)
          p.amax_partial[m * p.n_partial + static_cast<int64_t>(tile_n) * 2 + wn] = a;
      }
    }
  } else {
    // stores through a descriptor over the tile's rows: rows past row_end and columns past
    // n_out (offset past the descriptor) are dropped without a branch (a branch per store
    // makes the compiler wait for the stores before it)
    const uint32_t esz = (EPI == MP_EPI_F32 || p.out_dtype == MP_F32) ? 4 : 2;
    const bool bf = p.out_dtype == MP_BF16, hb = EPI == MP_EPI_DENSE && p.bias != nullptr;
    const uint32_t ldy = static_cast<uint32_t>(p.ldy);
    const __amdgpu_buffer_rsrc_t yr = mp_rsrc(static_cast<char *>(p.y) + row_begin * p.ldy * esz,
                                              static_cast<uint32_t>(row_end - row_begin) * ldy * esz);
    const int lm0 = wm * WM + 4 * (lane >> 5);
    // a wave's 8 KB region in the A buffers (128-byte K steps; 64-byte steps leave too little room)
    constexpr bool STAGE_FITS = WN * 2 * WM <= 8192 && 4 * 8192 <= 2 * BM * LD;
    if (STAGE_FITS && EPI != MP_EPI_F32 && p.staged_epilogue && esz == 2) {  // workgroup-uniform
      // 16-bit outputs through LDS: the wave converts its WM x WN tile into a private row-major
      // region of the A buffers (free after the K loop's last barrier; lane pairs exchange
      // halves so each lane writes 32-bit words of two adjacent columns), then reads it back
      // as 16-byte chunks: 8 global stores per lane instead of 64 two-byte ones.  The launcher
      // sets staged_epilogue only with N and the row stride multiples of 8 and y 16-byte
      // aligned, so a chunk lies wholly inside or wholly outside the output.
      int8_t *stage = &sa[0][0] + wave * 8192;
      const bool odd = lane & 1;
      const uint32_t sel_lo = odd ? 0x01000504u : 0x05040100u;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int cl = wn * WN + j * 32 + (lane & 31);
        const float sbv = tscale[BM + cl], bv = tscale[BM + BN + cl];
        const int cb = (j * 32 + (lane & 31)) & ~1;  // even column of the lane pair, within the wave tile
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f4_t s4 = *reinterpret_cast<const f4_t *>(tscale + lm0 + i * 32 + 8 * q);
            uint32_t hv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][4 * q + e]), s4[e]), sbv);
              if (hb) v = mp_add(v, bv);
              hv[e] = bf ? mp_f2bf(v) : mp_f2h(v);
            }
            const uint32_t p01 = hv[0] | (hv[1] << 16), p23 = hv[2] | (hv[3] << 16);
            const uint32_t recv = __shfl_xor(odd ? p01 : p23, 1, 64);
            const uint32_t mine = odd ? p23 : p01;
            const int r = i * 32 + 4 * (lane >> 5) + 8 * q + (odd ? 2 : 0);  // row within the wave tile
            *reinterpret_cast<uint32_t *>(stage + r * (2 * WN) + cb * 2) = __builtin_amdgcn_perm(recv, mine, sel_lo);
            *reinterpret_cast<uint32_t *>(stage + (r + 1) * (2 * WN) + cb * 2) =
                __builtin_amdgcn_perm(recv, mine, sel_lo + 0x02020202u);
          }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // wave-private region: own writes first
      constexpr int CPR16 = WN / 8;                         // 16-byte chunks per tile row
#pragma unroll
      for (int t = 0; t < WM * CPR16 / 64; ++t) {
        const int c = t * 64 + lane;
        const int lr = c / CPR16, cc = (c % CPR16) * 8;
        const uint4 v = *reinterpret_cast<const uint4 *>(stage + lr * (2 * WN) + cc * 2);
        const int64_t col = col0 + wn * WN + cc;
        const uint32_t off = col < n_out ? (static_cast<uint32_t>(wm * WM + lr) * ldy + static_cast<uint32_t>(col)) * 2
                                         : 0x80000000u;
        mp_buf_store16(yr, off, v);
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int cl = wn * WN + j * 32 + (lane & 31);
      const int64_t col = col0 + cl;
      const bool cval = col < n_out;
      const float sbv = tscale[BM + cl], bv = tscale[BM + BN + cl];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4_t s4 = *reinterpret_cast<const f4_t *>(tscale + lm0 + i * 32 + 8 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int lm = lm0 + i * 32 + 8 * q + e;
            float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][4 * q + e]), s4[e]), sbv);
            if (hb) v = mp_add(v, bv);
            const uint32_t off = cval ? (static_cast<uint32_t>(lm) * ldy + static_cast<uint32_t>(col)) * esz : 0x80000000u;
            if (esz == 4) mp_buf_store4(yr, off, __float_as_uint(v));
            else mp_buf_store2(yr, off, bf ? mp_f2bf(v) : mp_f2h(v));
          }
        }
    }
  }
}

// ------------------------------------------------------------------ grouped (MoE) GEMM
// Expert-grouped int8 GEMM for experts of up to a few hundred routed rows.  A work
// item is rows [row_begin, row_end) of one expert, at most 256 of them, against 128
// weight rows (fp32 / 16-bit outputs: 128 output columns; SwiGLU: 64 gate rows and
// the 64 matching up rows), so a weight slice streams from HBM once per 256 rows of
// its expert.  Items are numbered expert-major with the row chunk fastest; the
// workgroups the dispatcher places on XCD x (id % 8) walk the x-th eighth of the
// items, so the items an XCD runs together share their expert's activation rows (and
// a slice's row chunks share its weights) in that XCD's L2.  The launch is
// persistent (one workgroup per CU): the next item's first K tiles are loaded before
// the current item's epilogue.
// Eight waves: wave w loads the 32-row A slab w; wave (wr, wn) = (w >> 1, w & 1)
// multiplies the 32-row tiles wr and 4 + wr (rows [32 wr, +32) and [128 + 32 wr, +32))
// and owns the 64 columns wn, so an expert of up to 128 rows keeps all eight waves busy
// (two per SIMD) and one of up to 256 rows gives each wave both tiles.  A slab or tile
// past the expert's rows is inactive: its wave loads no A rows for it and skips its
// MFMAs (the K loop is instantiated for one and for two tiles; every wave runs the same
// barriers).  128-byte K steps (a 64-lane load covers 8 rows x 128 B), D + 1 register
// stages in flight, LDS double buffer of 144-byte rows.
constexpr int kMoeBM = 256, kMoeBN = 128, kMoeBK = 128, kMoeLD = kMoeBK + 16, kMoeThreads = 512;
constexpr int kMoeMaxExperts = 1024;
// LDS: double-buffered A and B tiles; two buffers each of the item's per-token scales and
// column scales; the group offsets
constexpr size_t kMoeSmem = static_cast<size_t>(2) * (kMoeBM + kMoeBN) * kMoeLD +
                            2 * (kMoeBM + kMoeBN) * sizeof(float) + (kMoeMaxExperts + 1) * sizeof(int64_t);

__device__ __forceinline__ int moe_row_chunks(const int64_t *off, int e) {
  const int64_t c = off[e + 1] - off[e];
  return c > 0 ? static_cast<int>((c + kMoeBM - 1) / kMoeBM) : 0;
}

// Item g of the expert-major numbering: expert e, weight slice, 256-row chunk.
// Every lane returns the same values (wave-level scan over the experts).
__device__ __forceinline__ void moe_find_item(const int64_t *off, int ne, int n_slices, int g, int lane, int &e,
                                              int &slice, int64_t &row_begin, int64_t &row_end) {
  int found = -1, rem = 0, chunks = 1, base = 0;
  for (int c0 = 0; c0 < ne && found < 0; c0 += 64) {
    const int ch = c0 + lane < ne ? moe_row_chunks(off, c0 + lane) : 0;
    const int it = ch * n_slices;
    int incl = it;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o, 64);
      incl += lane >= o ? t : 0;
    }
    const bool mine = it > 0 && g >= base + incl - it && g < base + incl;
    const unsigned long long bal = __ballot(mine);
    if (bal) {
      const int src = __ffsll(static_cast<long long>(bal)) - 1;
      found = c0 + src;
      chunks = __shfl(ch, src, 64);
      rem = g - base - (__shfl(incl, src, 64) - __shfl(it, src, 64));
    }
    base += __shfl(incl, 63, 64);
  }
  e = __builtin_amdgcn_readfirstlane(found < 0 ? 0 : found);
  chunks = __builtin_amdgcn_readfirstlane(chunks);
  rem = __builtin_amdgcn_readfirstlane(rem);
  slice = rem / chunks;
  row_begin = off[e] + static_cast<int64_t>(rem % chunks) * kMoeBM;
  row_end = off[e + 1] < row_begin + kMoeBM ? off[e + 1] : row_begin + kMoeBM;
}

// One step of the transposing max butterfly over 2B values per lane: lanes l and l ^ B
// exchange half of their values; the lane with bit B set keeps the upper half.
template <int B>
__device__ __forceinline__ void moe_max_step(float (&v)[32], int lane) {
  const bool hi = (lane & B) != 0;
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const float send = hi ? v[j] : v[j + B];
    const float keep = hi ? v[j + B] : v[j];
    v[j] = fmaxf(keep, __shfl_xor(send, B, 64));
  }
}

template <int EPI, int D>
__global__ __launch_bounds__(kMoeThreads) void i8_moe_kernel(mp_i8_args p, int n_slices) {
  constexpr int BM = kMoeBM, BN = kMoeBN, BK = kMoeBK, LD = kMoeLD, NT = kMoeThreads;
  constexpr int CPR = BK / 16;          // 16-byte chunks per tile row
  constexpr int CA = 4;                 // A loads per lane per K step (its wave's 32 rows)
  constexpr int CB = BN * CPR / NT;     // B loads (2)
  constexpr int TM = 2, TN = 2;         // 32x32 MFMA tiles per wave: rows 32 wr, 128 + 32 wr; 64 columns
  constexpr bool SWI = EPI == MP_EPI_SWIGLU;
  extern __shared__ __attribute__((aligned(16))) int8_t smem_moe[];
  int8_t *sa = smem_moe;                // [2][BM * LD]
  int8_t *sb = smem_moe + 2 * BM * LD;  // [2][BN * LD]
  float *ssa = reinterpret_cast<float *>(smem_moe + 2 * (BM + BN) * LD);  // [2][BM] per-token scales
  float *ssc = ssa + 2 * BM;                                              // [2][BN] column scales
  int64_t *soff = reinterpret_cast<int64_t *>(ssc + 2 * BN);             // [E + 1] group offsets
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wn = wave & 1;

  // ---- this workgroup's items (every wave derives the same ones).  The offsets are read
  // from an LDS copy, so finding the next item never waits on the tile loads in flight.
  const int ne = p.n_experts;
  for (int i = tid; i <= ne; i += NT) soff[i] = p.offsets[i];
  mp_lds_barrier();
  const int64_t *off = soff;
  int total = 0;
  for (int c0 = 0; c0 < ne; c0 += 64) {
    int it = c0 + lane < ne ? moe_row_chunks(off, c0 + lane) * n_slices : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) it += __shfl_xor(it, o, 64);
    total += it;
  }
  // uniform to the compiler too: item state derived from it stays in scalar registers
  // (a buffer descriptor it thinks divergent turns every load into a waterfall loop)
  total = __builtin_amdgcn_readfirstlane(total);
  const int share = (total + 7) / 8;
  const int xcd = static_cast<int>(blockIdx.x) % 8, stride = static_cast<int>(gridDim.x) / 8;
  int idx = static_cast<int>(blockIdx.x) / 8;
  if (idx >= share || xcd * share + idx >= total) return;  // workgroup-uniform, before any barrier

  const int64_t k = p.k;
  const int64_t n_out = p.n;
  const int64_t nb_rows = SWI ? 2 * n_out : n_out;  // weight rows per expert
  const int64_t nkt = k / BK;

  // A: lane's rows 32 wave + 8 i + lane / 8 (i < CA), chunk lane % 8, through a
  // buffer descriptor that ends at row_end (rows past it read as zeros, no traffic)
  const int arow0 = 32 * wave + (lane >> 3);
  const uint32_t aoff0 = static_cast<uint32_t>(arow0 * k + (lane & 7) * 16);
  // B: chunk c = tid + i * NT of the 128 x 128 tile
  int boff_row[CB];
#pragma unroll
  for (int i = 0; i < CB; ++i) boff_row[i] = (tid + i * NT) / CPR;
  const int bchunk = (tid % CPR) * 16;

  int e, slice;
  int64_t row_begin, row_end;
  __amdgpu_buffer_rsrc_t arsrc;
  const int8_t *bsrc[CB];
  bool lact, mact0, mact1;  // the wave's A slab loads; its tiles 0 and 1 multiply
  // next item's scale held by this thread: tid < BM per-token scale of row tid, BM <= tid <
  // BM + BN the scale of weight row tid - BM of the tile
  float scale_a = 0.f, scale_b = 0.f;
  int par = 0;  // scale buffers of the current item
  auto set_item = [&](int g) {
    moe_find_item(off, ne, n_slices, g, lane, e, slice, row_begin, row_end);
    arsrc = mp_rsrc(p.a + row_begin * k, static_cast<uint32_t>((row_end - row_begin) * k));
    lact = row_begin + 32 * wave < row_end;
    mact0 = row_begin + 32 * wr < row_end;
    mact1 = row_begin + 128 + 32 * wr < row_end;
    const int8_t *bexp = p.b + (p.shared_b ? 0 : static_cast<int64_t>(e) * nb_rows * k);
    const int64_t col0 = static_cast<int64_t>(slice) * (SWI ? BN / 2 : BN);
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int lr = boff_row[i];
      int64_t wr;
      if (SWI) {
        const int64_t oc = col0 + (lr % (BN / 2));
        const int64_t occ = oc < n_out ? oc : n_out - 1;
        wr = (lr < BN / 2) ? occ : n_out + occ;
      } else {
        const int64_t oc = col0 + lr;
        wr = oc < n_out ? oc : n_out - 1;
      }
      bsrc[i] = bexp + wr * k + bchunk;
    }
  };
  // Epilogue scales of the item, loaded ahead of the epilogue (whose stores may alias
  // them), one per thread: per-token scales (zeros past row_end) and the scales of the
  // tile's weight rows.  They go to the item's LDS scale buffers after the K loop's first
  // barrier, so the epilogue waits on no global load.
  auto load_scales = [&]() {
    // both loads on every thread (one of them, or both, past its descriptor): no branch
    const __amdgpu_buffer_rsrc_t srsrc = mp_rsrc(p.s_a + row_begin, static_cast<uint32_t>((row_end - row_begin) * 4));
    scale_a = __uint_as_float(mp_buf_load4(srsrc, tid < BM ? static_cast<uint32_t>(tid * 4) : 0x80000000u, 0));
    const __amdgpu_buffer_rsrc_t brsrc =
        mp_rsrc(p.s_b + (p.shared_b ? 0 : static_cast<int64_t>(e) * nb_rows), static_cast<uint32_t>(nb_rows * 4));
    {
      const int lr = (tid - BM) & (BN - 1);
      const int64_t col0 = static_cast<int64_t>(slice) * (SWI ? BN / 2 : BN);
      int64_t wr;
      if (SWI) {
        const int64_t oc = col0 + (lr % (BN / 2));
        const int64_t occ = oc < n_out ? oc : n_out - 1;
        wr = (lr < BN / 2) ? occ : n_out + occ;
      } else {
        const int64_t oc = col0 + lr;
        wr = oc < n_out ? oc : n_out - 1;
      }
      const bool mine = tid >= BM && tid < BM + BN;
      scale_b = __uint_as_float(mp_buf_load4(brsrc, mine ? static_cast<uint32_t>(wr * 4) : 0x80000000u, 0));
    }
  };

  i4_t areg[D + 1][CA], breg[D + 1][CB];
  // Every wave issues the same loads on every path (a uniform count keeps the compiler's
  // load-wait accounting exact across items): idle slabs load A at offsets past the
  // descriptor (zeros, no memory traffic) and skip the LDS stores and MFMAs.
  auto load_tile = [&](int set, int64_t kt) {
    kt = kt < 0 ? 0 : (kt < nkt ? kt : nkt - 1);  // every load stays inside the item's K range
    const uint32_t koff = static_cast<uint32_t>(kt * BK);
    const uint32_t ab = lact ? aoff0 : 0x80000000u;
#pragma unroll
    for (int i = 0; i < CA; ++i) areg[set][i] = mp_buf_load16i(arsrc, ab + static_cast<uint32_t>(8 * i * k), koff);
#pragma unroll
    for (int i = 0; i < CB; ++i) breg[set][i] = *reinterpret_cast<const i4_t *>(bsrc[i] + kt * BK);
  };
  auto store_tile = [&](int set, int buf) {
    if (lact) {  // wave-uniform
#pragma unroll
      for (int i = 0; i < CA; ++i)
        *reinterpret_cast<i4_t *>(sa + buf * BM * LD + (arow0 + 8 * i) * LD + (lane & 7) * 16) = areg[set][i];
    }
#pragma unroll
    for (int i = 0; i < CB; ++i)
      *reinterpret_cast<i4_t *>(sb + buf * BN * LD + boff_row[i] * LD + bchunk) = breg[set][i];
  };

  i16_t acc[TM][TN];
  int arow_l[TM], brow_l[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) arow_l[i] = (32 * wr + 128 * i + (lane & 31)) * LD + 16 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int lr = SWI ? (j * (BN / 2) + wn * 32 + (lane & 31)) : (wn * 64 + j * 32 + (lane & 31));
    brow_l[j] = lr * LD + 16 * (lane >> 5);
  }
  // the wave's active tiles: TA = 1 (tile 0) or 2 (both)
  auto mma = [&](int cur, auto ta_tag) {
    constexpr int TA = decltype(ta_tag)::value;
    const int8_t *ca = sa + cur * BM * LD;
    const int8_t *cb = sb + cur * BN * LD;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      i4_t af[TA], bf[TN];
#pragma unroll
      for (int i = 0; i < TA; ++i) af[i] = *reinterpret_cast<const i4_t *>(ca + arow_l[i] + ks * 32);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const i4_t *>(cb + brow_l[j] + ks * 32);
#pragma unroll
      for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };
  // Register set s holds tile t with t % (D + 1) == s; at step kt tiles kt+1 .. kt+D+1
  // are in flight.  Tile kt+1 goes to LDS after tile kt is multiplied, and its set is
  // refilled with tile kt+D+2 (loads past the last tile are clamped to it, never used).
  // The item's tiles 0 .. D are loaded before the loop.
  auto k_loop = [&]() {
    store_tile(0, 0);
    load_tile(0, D + 1);
    mp_lds_barrier();
    // scale buffers par were last read in the epilogue two items back: every wave has
    // passed at least one barrier since (waves 0-3 and 4-5: wave-uniform branches)
    if (tid < BM) ssa[par * BM + tid] = scale_a;
    else if (tid < BM + BN) ssc[par * BN + tid - BM] = scale_b;
    for (int64_t kt0 = 0; kt0 < nkt; kt0 += D + 1) {
#pragma unroll
      for (int d = 0; d <= D; ++d) {
        const int64_t kt = kt0 + d;
        const int nxt = (d + 1) % (D + 1);
        if (kt < nkt) {  // workgroup-uniform
          if (mact1) mma(static_cast<int>(kt & 1), std::integral_constant<int, 2>{});
          else if (mact0) mma(static_cast<int>(kt & 1), std::integral_constant<int, 1>{});
          if (kt + 1 < nkt) store_tile(nxt, static_cast<int>((kt + 1) & 1));
        }
        load_tile(nxt, kt + D + 2);
        mp_lds_barrier();
      }
    }
  };
  // tiles 0 .. D of the item (first_tile 0), or D + 1 copies of the current item's last
  // tile when there is no next item (L2-resident; keeps the load count of every path equal)
  auto prologue = [&](int64_t first_tile) {
#pragma unroll
    for (int d = 0; d <= D; ++d) load_tile(d, first_tile + d);
  };

  set_item(xcd * share + idx);
  prologue(0);
  load_scales();
  while (true) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    k_loop();

    // the current item's epilogue parameters, then the next item's first tiles (the
    // loop's last barrier has passed: LDS is free, the register stages are consumed)
    const bool cur_act = mact0;
    const int cur_slice = slice;
    const int64_t cur_begin = row_begin, cur_end = row_end;
    idx += stride;
    const bool has_next = idx < share && xcd * share + idx < total;  // workgroup-uniform
    if (has_next) set_item(xcd * share + idx);
    prologue(has_next ? 0 : nkt - 1);

    if (cur_act) {
      // element r of tile (i, j): local row 32 wr + 128 i + 8 (r >> 2) + 4 (lane >> 5) + (r & 3).
      // Stores go through buffer descriptors over the item's rows: rows past cur_end and
      // columns past n_out (offset kOob) are dropped without a branch.  (Guarding each
      // store with a branch makes the compiler wait for every earlier store.)
      constexpr uint32_t kOob = 0x80000000u;
      const uint32_t nrows = static_cast<uint32_t>(cur_end - cur_begin);
      const uint32_t ldy = static_cast<uint32_t>(p.ldy);
      const int lm0 = 32 * wr + 4 * (lane >> 5);
      // the lane's per-token scales: rows lm0 + 128 i + 8 q + (0..3)
      float sa_r[TM][16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f4_t s4 = *reinterpret_cast<const f4_t *>(ssa + par * BM + lm0 + 128 * i + 8 * q);
#pragma unroll
          for (int c = 0; c < 4; ++c) sa_r[i][4 * q + c] = s4[c];
        }
      if (SWI) {
        // h = silu((acc_g * s_tok) * s_g) * ((acc_u * s_tok) * s_u), and the abs-max of
        // each row over the wave's 32 columns: the 32 row values of a lane are reduced
        // across the 32 lanes of its half by a transposing butterfly (31 exchanges; after
        // it lane l holds the maximum of row value l % 32)
        const int64_t col = static_cast<int64_t>(cur_slice) * (BN / 2) + wn * 32 + (lane & 31);
        const bool cval = col < n_out;
        const float sg = ssc[par * BN + wn * 32 + (lane & 31)], su = ssc[par * BN + BN / 2 + wn * 32 + (lane & 31)];
        const __amdgpu_buffer_rsrc_t hr = mp_rsrc(static_cast<float *>(p.y) + cur_begin * p.ldy, nrows * ldy * 4);
        float v[32];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int lm = lm0 + i * 128 + 8 * (r >> 2) + (r & 3);
            const float gv = mp_mul(mp_mul(static_cast<float>(acc[i][0][r]), sa_r[i][r]), sg);
            const float uv = mp_mul(mp_mul(static_cast<float>(acc[i][1][r]), sa_r[i][r]), su);
            const float h = mp_swiglu_epi(gv, uv, p.epi_round);
            mp_buf_store4(hr, cval ? (static_cast<uint32_t>(lm) * ldy + static_cast<uint32_t>(col)) * 4 : kOob,
                          __float_as_uint(h));
            v[i * 16 + r] = (cval && static_cast<uint32_t>(lm) < nrows) ? fabsf(h) : 0.f;
          }
        moe_max_step<16>(v, lane);
        moe_max_step<8>(v, lane);
        moe_max_step<4>(v, lane);
        moe_max_step<2>(v, lane);
        moe_max_step<1>(v, lane);
        const int jv = lane & 31;
        const int lm = lm0 + (jv >> 4) * 128 + 8 * ((jv & 15) >> 2) + (jv & 3);
        const uint32_t np = static_cast<uint32_t>(p.n_partial);
        const __amdgpu_buffer_rsrc_t pr = mp_rsrc(p.amax_partial + cur_begin * p.n_partial, nrows * np * 4);
        mp_buf_store4(pr, (static_cast<uint32_t>(lm) * np + static_cast<uint32_t>(cur_slice * 2 + wn)) * 4,
                      __float_as_uint(v[0]));
      } else if (EPI == MP_EPI_AMAX) {
        // y = (acc * s_tok) * s_ch (+ bias), rounded to the 16-bit output and stored (the
        // arithmetic and order of the dense epilogues), and the abs-max of each row's rounded
        // values over the wave's 64 columns, reduced as in the SwiGLU epilogue, into
        // amax_partial[row][2 * slice + wave column]
        const bool bf = p.out_dtype == MP_BF16, hb = p.bias != nullptr;
        const __amdgpu_buffer_rsrc_t yr =
            mp_rsrc(static_cast<char *>(p.y) + cur_begin * p.ldy * 2, nrows * ldy * 2);
        float v[32];
#pragma unroll
        for (int t = 0; t < 32; ++t) v[t] = 0.f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t col = static_cast<int64_t>(cur_slice) * BN + wn * 64 + j * 32 + (lane & 31);
          const bool cval = col < n_out;
          const float scj = ssc[par * BN + wn * 64 + j * 32 + (lane & 31)];
          const float bj = hb ? mp_load_as_f32(p.bias, cval ? col : n_out - 1, p.bias_dtype) : 0.f;
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int lm = lm0 + i * 128 + 8 * (r >> 2) + (r & 3);
              float yv = mp_mul(mp_mul(static_cast<float>(acc[i][j][r]), sa_r[i][r]), scj);
              yv = hb ? mp_add(yv, bj) : yv;
              const uint16_t hv = bf ? mp_f2bf(yv) : mp_f2h(yv);
              const uint32_t off =
                  cval ? (static_cast<uint32_t>(lm) * ldy + static_cast<uint32_t>(col)) * 2 : kOob;
              mp_buf_store2(yr, off, hv);
              const float rv = bf ? mp_bf2f(hv) : mp_h2f(hv);
              v[i * 16 + r] = fmaxf(v[i * 16 + r], (cval && static_cast<uint32_t>(lm) < nrows) ? fabsf(rv) : 0.f);
            }
        }
        moe_max_step<16>(v, lane);
        moe_max_step<8>(v, lane);
        moe_max_step<4>(v, lane);
        moe_max_step<2>(v, lane);
        moe_max_step<1>(v, lane);
        const int jv = lane & 31;
        const int lm = lm0 + (jv >> 4) * 128 + 8 * ((jv & 15) >> 2) + (jv & 3);
        const uint32_t np = static_cast<uint32_t>(p.n_partial);
        const __amdgpu_buffer_rsrc_t pr = mp_rsrc(p.amax_partial + cur_begin * p.n_partial, nrows * np * 4);
        mp_buf_store4(pr, (static_cast<uint32_t>(lm) * np + static_cast<uint32_t>(cur_slice * 2 + wn)) * 4,
                      __float_as_uint(v[0]));
      } else {
        const uint32_t esz = EPI == MP_EPI_F32 ? 4 : 2;
        const bool bf = p.out_dtype == MP_BF16;
        const __amdgpu_buffer_rsrc_t yr =
            mp_rsrc(static_cast<char *>(p.y) + cur_begin * p.ldy * esz, nrows * ldy * esz);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t col = static_cast<int64_t>(cur_slice) * BN + wn * 64 + j * 32 + (lane & 31);
          const bool cval = col < n_out;
          const float scj = ssc[par * BN + wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int lm = lm0 + i * 128 + 8 * (r >> 2) + (r & 3);
              const float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][r]), sa_r[i][r]), scj);
              const uint32_t off =
                  cval ? (static_cast<uint32_t>(lm) * ldy + static_cast<uint32_t>(col)) * esz : kOob;
              if (EPI == MP_EPI_F32) mp_buf_store4(yr, off, __float_as_uint(v));
              else mp_buf_store2(yr, off, bf ? mp_f2bf(v) : mp_f2h(v));
            }
        }
      }
    }
    load_scales();  // (the next item's, or again the current one's at the end)
    if (!has_next) break;
    par ^= 1;
  }
}

// ------------------------------------------------------------------ large-M dense GEMM
// 256 x 256 output tile per workgroup of 8 waves (2 along M x 4 along N), each
// wave 128 x 64 = 4 x 2 MFMA i32_32x32x32_i8 tiles (128 accumulator registers,
// so two waves fit per SIMD; the 32x32x32 form runs at twice the rate of
// 16x16x64 on gfx950).  BK = 64, LDS double buffer and two register stages: K
// tile kt+2 is in flight while tile kt is multiplied and tile kt+1 is written to
// the other LDS buffer; the LDS-only barrier leaves those loads outstanding.
// Within a step the LDS traffic is interleaved into the MFMA stream (see step()).
// Tiles are assigned XCD-major: the workgroups the dispatcher places on one
// XCD (id % 8) take a contiguous run of tiles, ordered in 4-row-tile bands, so
// concurrent tiles share A and B rows in that XCD's L2.
// LDS tiles: 64-byte rows, the 16-byte chunk c of row r stored at slot
// c ^ ((r >> 2) & 3).  Both access patterns are bank-conflict free: a store
// covers 4 rows x 4 chunks per 16 lanes (rows 4q..4q+3 land on the four 16-bank
// quarters), a fragment read 16 rows of one chunk (16 distinct 4-bank groups).
constexpr int kBigBM = 256, kBigBN = 256, kBigBK = 64, kBigLD = kBigBK, kBigThreads = 512;

__device__ __forceinline__ void big_tile_coords(int id, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  const int per = total / 8, rem = total % 8;
  const int xcd = id % 8, local = id / 8;
  const int t = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int band = t / (4 * tiles_n);
  const int inb = t % (4 * tiles_n);
  const int rows_in_band = (tiles_m - band * 4) < 4 ? (tiles_m - band * 4) : 4;
  tm = band * 4 + inb % rows_in_band;
  tn = inb / rows_in_band;
}

// Epilogue of the large-M kernels for one wave's TM x TN grid of 32x32 int32
// accumulators: element r of tile (i, j) is row mbase + 32 i + 8 (r >> 2) + (r & 3)
// (mbase includes 4 (lane >> 5)), column nbase + 32 j + lane % 32.
// y = (acc * s_tok[m]) * s_ch[n] (+ bias[n]) in OUT_DT.  In a full-row tile the
// lane's per-token scales come in runs of 4 rows and are read once as float4;
// only the column guard (one per j) remains.  A partial tile clamps every row.
template <int OUT_DT, int TM, int TN>
__device__ __forceinline__ void big_epilogue(const mp_i8_args &p, const i16_t (&acc)[TM][TN], int64_t mbase,
                                             int64_t nbase, bool full_rows, int lane) {
  const bool has_bias = p.bias != nullptr;
  float sbv[TN], bv[TN];
  bool cval[TN];
  int64_t colv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = nbase + j * 32 + (lane & 31);
    cval[j] = col < p.n;
    colv[j] = col;
    const int64_t colc = cval[j] ? col : p.n - 1;
    sbv[j] = p.s_b[colc];
    bv[j] = has_bias ? mp_load_as_f32(p.bias, colc, p.bias_dtype) : 0.f;
  }
  auto put = [&](int64_t m, int j, float v) {
    if (OUT_DT == MP_F16) static_cast<uint16_t *>(p.y)[m * p.ldy + colv[j]] = mp_f2h(v);
    else if (OUT_DT == MP_BF16) static_cast<uint16_t *>(p.y)[m * p.ldy + colv[j]] = mp_f2bf(v);
    else static_cast<float *>(p.y)[m * p.ldy + colv[j]] = v;
  };
  const bool vec_sa = (reinterpret_cast<uintptr_t>(p.s_a) & 15) == 0;
  // 16-bit outputs, even N / row stride: lanes (2c, 2c+1) swap halves so each stores
  // two adjacent columns of two rows as 32-bit words (half the store instructions)
  if (OUT_DT != MP_F32 && full_rows && vec_sa && (p.n & 1) == 0 && (p.ldy & 1) == 0 &&
      (reinterpret_cast<uintptr_t>(p.y) & 3) == 0) {
    const bool odd = lane & 1;
    // perm(recv, mine): bytes 0-3 = mine, 4-7 = recv.  Even lane: [own | partner] of
    // rows e0 / e1; odd lane: [partner | own] of rows e2 / e3 (columns 2c, 2c+1)
    const uint32_t sel_lo = odd ? 0x01000504u : 0x05040100u;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float4 s4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) s4[g] = *reinterpret_cast<const float4 *>(p.s_a + mbase + i * 32 + 8 * g);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (!cval[j]) continue;  // the pair partner has the same guard (N even)
        uint32_t *yw = reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(p.y) + (colv[j] & ~int64_t(1)));
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float sv[4] = {s4[g].x, s4[g].y, s4[g].z, s4[g].w};
          uint32_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][4 * g + e]), sv[e]), sbv[j]);
            v = has_bias ? mp_add(v, bv[j]) : v;
            h[e] = OUT_DT == MP_F16 ? mp_f2h(v) : mp_f2bf(v);
          }
          const uint32_t p01 = h[0] | (h[1] << 16), p23 = h[2] | (h[3] << 16);
          // even lane keeps rows e0, e1 and takes the partner's; odd lane rows e2, e3
          const uint32_t recv = __shfl_xor(odd ? p01 : p23, 1, 64);
          const uint32_t mine = odd ? p23 : p01;
          const uint32_t w0 = __builtin_amdgcn_perm(recv, mine, sel_lo);
          const uint32_t w1 = __builtin_amdgcn_perm(recv, mine, sel_lo + 0x02020202u);
          const int64_t m = mbase + i * 32 + 8 * g + (odd ? 2 : 0);
          yw[(m * p.ldy) >> 1] = w0;
          yw[((m + 1) * p.ldy) >> 1] = w1;
        }
      }
    }
    return;
  }
  if (full_rows && vec_sa) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float4 s4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) s4[g] = *reinterpret_cast<const float4 *>(p.s_a + mbase + i * 32 + 8 * g);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (!cval[j]) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float4 q = s4[r >> 2];
          const float sa = (r & 3) == 0 ? q.x : ((r & 3) == 1 ? q.y : ((r & 3) == 2 ? q.z : q.w));
          float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][r]), sa), sbv[j]);
          v = has_bias ? mp_add(v, bv[j]) : v;
          put(mbase + i * 32 + 8 * (r >> 2) + (r & 3), j, v);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = mbase + i * 32 + 8 * (r >> 2) + (r & 3);
        const int64_t mc = m < p.rows ? m : p.rows - 1;
        float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][r]), p.s_a[mc]), sbv[j]);
        v = has_bias ? mp_add(v, bv[j]) : v;
        if (cval[j] && m < p.rows) put(m, j, v);
      }
}

// Epilogues of the grouped (expert) launches of the large-M kernel, for one wave's
// 4 x 2 accumulator tiles at rows mbase + 32 i + 8 (r >> 2) + (r & 3) (< row_end)
// and columns nbase + lane % 32 (+ 32 j for F32).  Arithmetic as in
// i8_tiled_kernel: F32 y = (acc * s_a) * s_b; SWIGLU g / u = (acc * s_a) * s_gate /
// s_up, h = silu(g) * u to the fp32 workspace plus the row's abs-max over the
// wave's 32 columns into amax_partial[m][4 * blockIdx.x + wave column].
template <int EPI, int TM>
__device__ __forceinline__ void grouped_epilogue(const mp_i8_args &p, const i16_t (&acc)[TM][2], int64_t mbase,
                                                 int64_t row_end, int64_t nbase, const float *sbexp, int lane) {
  float *yb = static_cast<float *>(p.y);
  if (EPI == MP_EPI_SWIGLU) {
    const int64_t col = nbase + (lane & 31);
    const bool cval = col < p.n;
    const int64_t colc = cval ? col : p.n - 1;
    const float sg = sbexp[colc], su = sbexp[p.n + colc];
    const int64_t pidx = static_cast<int64_t>(blockIdx.x) * 4 + (nbase % 128) / 32;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = mbase + i * 32 + 8 * (r >> 2) + (r & 3);
        const bool mval = m < row_end;
        const float sa_m = mval ? p.s_a[m] : 0.f;
        const float g = mp_mul(mp_mul(static_cast<float>(acc[i][0][r]), sa_m), sg);
        const float u = mp_mul(mp_mul(static_cast<float>(acc[i][1][r]), sa_m), su);
        const float h = mp_swiglu_epi(g, u, p.epi_round);
        if (mval && cval) yb[m * p.ldy + col] = h;
        float a = (mval && cval) ? fabsf(h) : 0.f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        if ((lane & 31) == 0 && mval) p.amax_partial[m * p.n_partial + pidx] = a;
      }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = nbase + j * 32 + (lane & 31);
      if (col >= p.n) continue;
      const float sb = sbexp[col];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = mbase + i * 32 + 8 * (r >> 2) + (r & 3);
          if (m >= row_end) continue;
          yb[m * p.ldy + col] = mp_mul(mp_mul(static_cast<float>(acc[i][j][r]), p.s_a[m]), sb);
        }
    }
  }
}

// LDS-staged epilogue of one wave's 128 x 64 tile for 16-bit outputs: in two
// passes of 64 rows the wave writes its converted values into a private 8 KB LDS
// region (row-major, 128-byte rows; lane pairs exchange halves so each writes
// 32-bit words) and reads them back as 16-byte chunks, so a lane issues 16
// global_store_dwordx4 instead of 64 narrow stores.  Needs a full-row,
// full-column tile, a row stride that is a multiple of 8 elements, 16-byte
// aligned y and s_tok; the caller checks.  Wave-private: only lgkmcnt waits.
template <int OUT_DT>
__device__ __forceinline__ void big_epilogue_staged(const mp_i8_args &p, const i16_t (&acc)[4][2], int64_t mbase_w,
                                                    int64_t nbase_w, int lane, int8_t *stage) {
  const bool has_bias = p.bias != nullptr;
  const bool odd = lane & 1;
  const uint32_t sel_lo = odd ? 0x01000504u : 0x05040100u;
  float sbv[2], bv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = nbase_w + j * 32 + (lane & 31);
    sbv[j] = p.s_b[col];
    bv[j] = has_bias ? mp_load_as_f32(p.bias, col, p.bias_dtype) : 0.f;
  }
  const int64_t row_l = 4 * (lane >> 5);  // row of element 0 within the 32-row tile
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * h + ii;
      float4 s4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        s4[g] = *reinterpret_cast<const float4 *>(p.s_a + mbase_w + row_l + i * 32 + 8 * g);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float sv[4] = {s4[g].x, s4[g].y, s4[g].z, s4[g].w};
          uint32_t hv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = mp_mul(mp_mul(static_cast<float>(acc[i][j][4 * g + e]), sv[e]), sbv[j]);
            v = has_bias ? mp_add(v, bv[j]) : v;
            hv[e] = OUT_DT == MP_F16 ? mp_f2h(v) : mp_f2bf(v);
          }
          const uint32_t p01 = hv[0] | (hv[1] << 16), p23 = hv[2] | (hv[3] << 16);
          const uint32_t recv = __shfl_xor(odd ? p01 : p23, 1, 64);
          const uint32_t mine = odd ? p23 : p01;
          const uint32_t w0 = __builtin_amdgcn_perm(recv, mine, sel_lo);
          const uint32_t w1 = __builtin_amdgcn_perm(recv, mine, sel_lo + 0x02020202u);
          // local row within the 64-row pass, column pair (2c, 2c+1) of the 64 columns
          const int r = ii * 32 + static_cast<int>(row_l) + 8 * g + (odd ? 2 : 0);
          const int cb = (j * 32 + (lane & 31)) & ~1;
          *reinterpret_cast<uint32_t *>(stage + r * 128 + cb * 2) = w0;
          *reinterpret_cast<uint32_t *>(stage + (r + 1) * 128 + cb * 2) = w1;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = q * 64 + lane;  // 16-byte chunk: row c / 8, columns 8 (c % 8) ..
      const i4_t v = *reinterpret_cast<const i4_t *>(stage + c * 16);
      const int64_t m = mbase_w + h * 64 + c / 8;
      *reinterpret_cast<i4_t *>(static_cast<uint16_t *>(p.y) + m * p.ldy + nbase_w + 8 * (c % 8)) = v;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // region reused by the next pass
  }
}

template <int OUT_DT, int EPI, int TMW = 4>
__global__ __launch_bounds__(kBigThreads, TMW == 2 ? 4 : 2) void i8_gemm_big_kernel(mp_i8_args p, int tiles_m,
                                                                                 int tiles_n) {
  constexpr bool GROUPED = EPI != MP_EPI_DENSE;  // grouped expert GEMM: F32 (GEMM2) or SWIGLU (GEMM1)
  constexpr bool SWI = EPI == MP_EPI_SWIGLU;
  // B tile rows: dense / F32 = 256 output columns; SWIGLU = 128 gate rows then the 128
  // matching up rows, so a wave's two 32-column fragments are gate j and up j
  constexpr int OUTC = SWI ? kBigBN / 2 : kBigBN;  // output columns per tile
  constexpr int WBN = SWI ? 32 : 64;               // wave column base step
  constexpr int BJ = SWI ? kBigBN / 2 : 32;        // B rows between a wave's two fragments
  // TMW = 4: 256-row tiles (waves of 128 x 64); TMW = 2: 128-row tiles (waves of 64 x 64, 48 KB of LDS
  // and <= 128 registers, two workgroups per CU) for grouped launches whose experts hold ~128 rows
  constexpr int BM = 64 * TMW, BN = kBigBN, BK = kBigBK, LD = kBigLD, NT = kBigThreads;
  constexpr int TM = TMW, TN = 2;              // 32x32 tiles per wave
  static_assert(TMW == 4 || EPI != MP_EPI_DENSE, "dense launches use 256-row tiles");
  constexpr int CPR = BK / 16;                 // 16-byte chunks per tile row
  constexpr int RPP = NT / CPR;                // tile rows covered per pass (128)
  constexpr int CA = BM / RPP, CB = BN / RPP;  // passes (2 each)
  extern __shared__ __attribute__((aligned(16))) int8_t smem_big[];
  int8_t *sa = smem_big;                // [2][BM*LD]
  int8_t *sb = smem_big + 2 * BM * LD;  // [2][BN*LD]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t k = p.k;

  // Tile schedule: the tiles of XCD x (workgroups id % 8 == x) form a contiguous
  // run in band order (big_tile_coords); workgroup id takes run entries id / 8,
  // id / 8 + stride, ...  With one workgroup per tile the stride ends the walk
  // after the first tile; a persistent launch (gridDim a multiple of 8) walks the
  // run, loading the next tile's first K steps before the current epilogue.
  // Grouped launches (grid: weight slices x row slots) take one tile: the row slot
  // walks group_offsets to the expert and its 256-row chunk.
  const int total = tiles_m * tiles_n;
  const int per = total / 8, rem = total % 8;
  const int xcd = blockIdx.x % 8;
  const int run_start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
  int run_len = per + (xcd < rem ? 1 : 0);
  const bool persist = !GROUPED && static_cast<int>(gridDim.x) < total;
  int stride = persist ? static_cast<int>(gridDim.x) / 8 : run_len;
  int t = blockIdx.x / 8;
  int64_t row_end = p.rows;
  const int8_t *bexp = p.b;
  const float *sbexp = p.s_b;
  int64_t g_m0 = 0;
  if (GROUPED) {
    int64_t slot = blockIdx.y;
    int e = 0;
    bool found = false;
    for (; e < p.n_experts; ++e) {
      const int64_t lo = p.offsets[e], hi = p.offsets[e + 1];
      const int64_t tiles_e = (hi - lo + BM - 1) / BM;
      if (slot < tiles_e) {
        g_m0 = lo + slot * BM;
        row_end = hi < g_m0 + BM ? hi : g_m0 + BM;
        found = true;
        break;
      }
      slot -= tiles_e;
    }
    if (!found) return;  // workgroup-uniform, before any barrier
    const int64_t nb_rows = SWI ? 2 * p.n : p.n;
    bexp = p.b + static_cast<int64_t>(e) * nb_rows * k;
    sbexp = p.s_b + static_cast<int64_t>(e) * nb_rows;
    t = 0;
    run_len = 1;
    stride = 1;
  }
  if (t >= run_len) return;  // workgroup-uniform, before any barrier
  auto coords = [&](int tt, int64_t &mm0, int64_t &nn0) {
    const int g = run_start + tt;
    const int band = g / (4 * tiles_n);
    const int inb = g % (4 * tiles_n);
    const int rows_in_band = (tiles_m - band * 4) < 4 ? (tiles_m - band * 4) : 4;
    mm0 = static_cast<int64_t>(band * 4 + inb % rows_in_band) * BM;
    nn0 = static_cast<int64_t>(inb / rows_in_band) * BN;
  };
  int64_t m0, n0;
  if (GROUPED) {
    m0 = g_m0;
    n0 = static_cast<int64_t>(blockIdx.x) * OUTC;
  } else {
    coords(t, m0, n0);
  }

  // pass i of this thread covers tile row (tid / CPR + i * RPP), bytes (tid % CPR) * 16
  // of the K step; rows past the matrix are clamped (computed, never stored)
  const int rloc = tid / CPR, cloc = (tid % CPR) * 16;
  const int cst = ((tid % CPR) ^ ((rloc >> 2) & 3)) * 16;  // swizzled slot (RPP % 16 == 0)
  // absolute A rows (clamped into the tile's valid rows) and B rows (clamped columns)
  int aoff[CA], boff[CB];
  const int8_t *abase = p.a + cloc, *bbase = bexp + cloc;
  auto set_tile = [&](int64_t mm0, int64_t nn0) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      int64_t r = mm0 + rloc + i * RPP;
      r = r < row_end ? r : row_end - 1;
      aoff[i] = static_cast<int>(r);
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int lr = rloc + i * RPP;
      if (SWI) {
        const int half = lr / (BN / 2);
        int64_t c = nn0 + lr % (BN / 2);
        c = c < p.n ? c : p.n - 1;
        boff[i] = static_cast<int>(half * p.n + c);
      } else {
        int64_t c = nn0 + lr;
        c = c < p.n ? c : p.n - 1;
        boff[i] = static_cast<int>(c);
      }
    }
  };
  set_tile(m0, n0);
  i4_t ra[CA + CB], rb[CA + CB];
  auto load_tile = [&](i4_t *r, int64_t kt) {
    const int64_t off = kt * BK;
#pragma unroll
    for (int i = 0; i < CA; ++i) r[i] = *reinterpret_cast<const i4_t *>(abase + static_cast<int64_t>(aoff[i]) * k + off);
#pragma unroll
    for (int i = 0; i < CB; ++i) r[CA + i] = *reinterpret_cast<const i4_t *>(bbase + static_cast<int64_t>(boff[i]) * k + off);
  };
  auto store_tile = [&](const i4_t *r, int buf) {
#pragma unroll
    for (int i = 0; i < CA; ++i)
      *reinterpret_cast<i4_t *>(&sa[buf * BM * LD + (rloc + i * RPP) * LD + cst]) = r[i];
#pragma unroll
    for (int i = 0; i < CB; ++i)
      *reinterpret_cast<i4_t *>(&sb[buf * BN * LD + (rloc + i * RPP) * LD + cst]) = r[CA + i];
  };

  i16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  const int rsw = 16 * ((lane >> 5) ^ ((lane >> 2) & 3));  // chunk (lane >> 5) of row lane & 31, swizzled
  const int arow = (wm * (32 * TM) + (lane & 31)) * LD + rsw;
  const int brow = (wn * WBN + (lane & 31)) * LD + rsw;
  // Software pipeline across the barrier.  Step s multiplies buffer b = s % 2:
  //   first half : global loads of K tile s+2; K32 half 0 MFMAs (fragments read in
  //                the previous step) interleaved with the reads of half 1's
  //                fragments and the LDS writes of tile s+1 into buffer b^1;
  //   barrier    : tile s+1 complete in b^1, every read of b's half 1 done;
  //   second half: K32 half 1 MFMAs interleaved with the reads of half 0's
  //                fragments of b^1 for step s+1.
  // After the barrier the MFMAs start at once (their fragments are in registers);
  // buffer b is rewritten only in step s+1's first half, after that barrier.
  i4_t af[2][TM], bf[2][TN];
  auto read_half = [&](int buf, int ks) {
    const int8_t *ca = sa + buf * BM * LD;
    const int8_t *cbp = sb + buf * BN * LD;
#pragma unroll
    for (int i = 0; i < TM; ++i) af[ks][i] = *reinterpret_cast<const i4_t *>(ca + (arow ^ (ks * 32)) + i * 32 * LD);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[ks][j] = *reinterpret_cast<const i4_t *>(cbp + (brow ^ (ks * 32)) + j * BJ * LD);
  };
  auto mfma_half = [&](int ks) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j], acc[i][j], 0, 0, 0);
  };
  auto first_half = [&](int buf, const i4_t *st, int nbuf, i4_t *ld, int64_t kt_ld) {
    load_tile(ld, kt_ld);
    read_half(buf, 1);
    mfma_half(0);
    store_tile(st, nbuf);
    __builtin_amdgcn_sched_group_barrier(0x020, CA + CB, 0);
    for (int r = 0; r < TM + TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    for (int r = 0; r < TM * TN - (TM + TN); ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
    }
  };
  auto second_half = [&](int nbuf) {
    read_half(nbuf, 0);
    mfma_half(1);
    for (int r = 0; r < TM + TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
  };

  // K is a multiple of 2 * BK (host check): the loop body is branch-free; the two
  // prefetches past the last tile are clamped to it and never multiplied
  const int64_t nkt = k / BK;
  load_tile(ra, 0);
  load_tile(rb, 1);
  __builtin_amdgcn_sched_barrier(0);
  store_tile(ra, 0);
  mp_lds_barrier();
  read_half(0, 0);
  while (true) {
    for (int64_t kt = 0; kt < nkt; kt += 2) {
      first_half(0, rb, 1, ra, kt + 2 < nkt ? kt + 2 : nkt - 1);
      mp_lds_barrier();
      second_half(1);
      __builtin_amdgcn_sched_barrier(0);
      first_half(1, ra, 0, rb, kt + 3 < nkt ? kt + 3 : nkt - 1);
      mp_lds_barrier();
      second_half(0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (GROUPED) {
      grouped_epilogue<EPI, TM>(p, acc, m0 + wm * (32 * TM) + 4 * (lane >> 5), row_end, n0 + wn * WBN, sbexp, lane);
      break;
    }
    // next tile's first two K steps go out before this tile's epilogue (LDS is
    // free: the last step's barrier has passed and the epilogue does not use it)
    const int tn_next = t + stride;
    const bool has_next = tn_next < run_len;
    int64_t m1 = m0, n1 = n0;
    if (has_next) {
      coords(tn_next, m1, n1);
      set_tile(m1, n1);
      load_tile(ra, 0);
      load_tile(rb, 1);
    }
    // epilogue: (acc * s_tok) * s_ch (+ bias) -> OUT_DT; 16-bit outputs of full tiles
    // go through LDS (the K loop is done with it: the last barrier has passed; only
    // the unused prefetch reads of buffer 0 may still be in flight in other waves)
    const bool staged = p.staged_epilogue && OUT_DT != MP_F32 && m0 + BM <= p.rows && n0 + BN <= p.n && (p.ldy & 7) == 0 &&
                        (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 &&
                        (reinterpret_cast<uintptr_t>(p.s_a) & 15) == 0;
    if constexpr (TM == 4) {
      if (staged)
        big_epilogue_staged<OUT_DT>(p, acc, m0 + wm * 128, n0 + wn * 64, lane, smem_big + wave * 8192);
      else
        big_epilogue<OUT_DT, TM, TN>(p, acc, m0 + wm * 128 + 4 * (lane >> 5), n0 + wn * 64, m0 + BM <= p.rows, lane);
    }
    if (!has_next) break;
    mp_lds_barrier();  // every wave's staging reads are done before buffer 0 is rewritten
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    store_tile(ra, 0);
    mp_lds_barrier();
    read_half(0, 0);
    t = tn_next;
    m0 = m1;
    n0 = n1;
  }
}

// Large-M GEMM with direct global->LDS loads (global_load_lds_dwordx4): 256x256
// tile, 8 waves of 128x64, 64-wide K steps, four LDS stages of 32 KB.  Tile kt+3
// is loaded straight into stage (kt+3) % 4 while tile kt is computed, so three
// tiles (96 KB per CU) are in flight without staging registers or LDS write
// instructions.  Each load instruction fills 1 KB of LDS (16 rows x 64 B, lane l
// at byte 16 l); a lane fetches the global chunk that the swizzled layout (chunk c
// of row r at slot c ^ ((r >> 2) & 3)) puts at its slot.  One barrier per step:
// after it every wave's loads of tile kt are complete and every read of stage
// (kt+3) % 4 from step kt-1 is done.
constexpr int kDmaStages = 4;

template <int OUT_DT, int EPI>
__global__ __launch_bounds__(512) void i8_gemm_dma_kernel(mp_i8_args p, int tiles_m, int tiles_n) {
  constexpr int BM = 256, BN = 256, BK = 64, LD = 64, TM = 4, TN = 2, S = kDmaStages;
  constexpr int STAGE = (BM + BN) * LD;  // bytes per stage (A rows then B rows)
  // grouped expert launches (F32 / SWIGLU epilogue): B tile layout as in i8_gemm_big_kernel
  constexpr bool GROUPED = EPI != MP_EPI_DENSE;
  constexpr bool SWI = EPI == MP_EPI_SWIGLU;
  constexpr int OUTC = SWI ? BN / 2 : BN, WBN = SWI ? 32 : 64, BJ = SWI ? BN / 2 : 32;
  extern __shared__ __attribute__((aligned(16))) int8_t smem_dma[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t k = p.k;
  int64_t m0, n0, row_end = p.rows;
  const int8_t *bexp = p.b;
  const float *sbexp = p.s_b;
  if (GROUPED) {
    int64_t slot = blockIdx.y;
    int e = 0;
    bool found = false;
    for (; e < p.n_experts; ++e) {
      const int64_t lo = p.offsets[e], hi = p.offsets[e + 1];
      const int64_t tiles_e = (hi - lo + BM - 1) / BM;
      if (slot < tiles_e) {
        m0 = lo + slot * BM;
        row_end = hi < m0 + BM ? hi : m0 + BM;
        found = true;
        break;
      }
      slot -= tiles_e;
    }
    if (!found) return;  // workgroup-uniform, before any barrier or load
    const int64_t nb_rows = SWI ? 2 * p.n : p.n;
    bexp = p.b + static_cast<int64_t>(e) * nb_rows * k;
    sbexp = p.s_b + static_cast<int64_t>(e) * nb_rows;
    n0 = static_cast<int64_t>(blockIdx.x) * OUTC;
  } else {
    int tm, tn;
    big_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    m0 = static_cast<int64_t>(tm) * BM;
    n0 = static_cast<int64_t>(tn) * BN;
  }

  // load instruction q (0..3) of this wave fills 16 rows: q < 2 -> A rows
  // (2 wave + q) * 16, else B rows (2 wave + q - 2) * 16.  Lane l: row + l / 4,
  // slot l % 4, global chunk slot ^ ((row >> 2) & 3).
  const int8_t *gsrc[4];
  int ldst[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const bool is_a = q < 2;
    const int r0 = (2 * wave + (q & 1)) * 16;
    const int r = r0 + lane / 4;
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    int64_t g;
    if (is_a) {
      g = m0 + r;
      g = g < row_end ? g : row_end - 1;
    } else if (SWI) {  // gate rows for r < 128, the matching up rows after
      int64_t cc = n0 + r % (BN / 2);
      cc = cc < p.n ? cc : p.n - 1;
      g = (r / (BN / 2)) * p.n + cc;
    } else {
      g = n0 + r;
      g = g < p.n ? g : p.n - 1;
    }
    gsrc[q] = (is_a ? p.a : bexp) + g * k + 16 * c;
    ldst[q] = (is_a ? 0 : BM * LD) + r0 * LD;
  }
  auto issue = [&](int64_t kt, int stage) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      __builtin_amdgcn_global_load_lds(gsrc[q] + kt * BK, smem_dma + stage * STAGE + ldst[q], 16, 0, 0);
  };

  i16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  const int rsw = 16 * ((lane >> 5) ^ ((lane >> 2) & 3));
  const int arow = (wm * 128 + (lane & 31)) * LD + rsw;
  const int brow = BM * LD + (wn * WBN + (lane & 31)) * LD + rsw;
  auto compute = [&](int stage) {
    const int8_t *st = smem_dma + stage * STAGE;
    i4_t af[2][TM], bf[2][TN];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < TM; ++i) af[ks][i] = *reinterpret_cast<const i4_t *>(st + (arow ^ (ks * 32)) + i * 32 * LD);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[ks][j] = *reinterpret_cast<const i4_t *>(st + (brow ^ (ks * 32)) + j * BJ * LD);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
    for (int r = 0; r < 6; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 10, 0);
  };

  const int64_t nkt = k / BK;
  auto kc = [&](int64_t t) { return t < nkt ? t : nkt - 1; };
  issue(0, 0);
  issue(kc(1), 1);
  issue(kc(2), 2);
  // step kt: own loads of tile kt done (8 newer load instructions may remain), barrier,
  // refill the stage read in step kt-1, compute
  for (int64_t kt = 0; kt < nkt; kt += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      // own loads of tile kt landed (vmcnt) and own reads of the stage refilled next are
      // done (lgkmcnt) before the barrier
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue(kc(kt + u + 3), (u + 3) % S);
      compute(u);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS DMA outstanding at exit

  if (GROUPED)
    grouped_epilogue<EPI, TM>(p, acc, m0 + wm * 128 + 4 * (lane >> 5), row_end, n0 + wn * WBN, sbexp, lane);
  else
    big_epilogue<OUT_DT, TM, TN>(p, acc, m0 + wm * 128 + 4 * (lane >> 5), n0 + wn * 64, m0 + BM <= p.rows, lane);
}

// Mid-M dense GEMM with direct global->LDS loads: a 128 x BN output tile per workgroup of four
// waves (BN = 128: 2 x 2 waves of 64x64; BN = 96: 4 x 1 waves of 32x96; MFMA i32_32x32x32_i8
// tiles), 128-byte K steps, four LDS stages (A rows 0..127, then B rows 0..BN-1, 128 bytes each).
// Tile kt+3 is loaded straight into stage (kt+3) % 4 while tile kt is multiplied: three K tiles in
// flight per workgroup with no staging registers and no LDS store instructions.  A load instruction
// fills 1 KB (8 rows x 128 B, lane l at byte 16 l); chunk c of row r sits at slot c ^ ((r >> 1) & 7),
// so the 16 lanes of a ds_read_b128 quarter (16 rows, one logical chunk) hit 16 distinct 16-byte bank
// groups.  One barrier per step: after it every wave's loads of tile kt have landed and every read of
// the stage refilled next is done.  The grid is 1-D: the row tiles of a column tile run on one XCD
// (blocks x and x + 8 ...), so their shared weight rows come from that XCD's L2.  BN = 96 gives a
// launch more tiles (more CUs streaming) for a quarter less weight per tile.
constexpr int kMidStages = 4, kMidBK = 128;
constexpr size_t mid_smem(int bn) { return static_cast<size_t>(kMidStages) * (128 + bn) * kMidBK; }

template <int OUT_DT, int BN>
__global__ __launch_bounds__(256) void i8_mid_kernel(mp_i8_args p, int tiles_m) {
  constexpr int BM = 128, BK = kMidBK, S = kMidStages;
  constexpr int WN = BN == 128 ? 2 : 1, WM = 4 / WN;  // waves along M and N
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // 32x32 tiles per wave
  constexpr int QW = (BM + BN) / 8 / 4;                // load instructions per wave per stage
  constexpr int STAGE = (BM + BN) * BK;
  static_assert((BN == 128 || BN == 96) && (BM + BN) % 32 == 0, "tile shapes");
  extern __shared__ __attribute__((aligned(16))) int8_t smem_mid[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int bx = static_cast<int>(blockIdx.x);
  const int tile_n = (bx / (8 * tiles_m)) * 8 + (bx & 7);
  const int64_t m0 = static_cast<int64_t>((bx >> 3) % tiles_m) * BM;
  const int64_t n0 = static_cast<int64_t>(tile_n) * BN;
  if (n0 >= p.n || m0 >= p.rows) return;  // grid padding; workgroup-uniform, before any barrier
  const int64_t k = p.k;

  // load instruction q of this wave fills 8-row group g = 4 q + wave of the stage: q < 4 (g < 16) -> A
  // rows 8 g .. + 8, else B rows 8 (g - 16) .. + 8.  Lane l: row + l / 8, slot l % 8, global chunk
  // slot ^ ((row >> 1) & 7).  Through buffer descriptors over the tile's valid A and B rows: a row
  // past M or N sits past its descriptor, reads zeros and moves no memory (the epilogue drops its
  // outputs).  The launcher bounds K below 2^23, so 128 K bytes of rows and the 0x80000000 dead
  // offset stay apart.
  constexpr uint32_t kOob = 0x80000000u;
  const int64_t a_rows = p.rows - m0 < BM ? p.rows - m0 : BM, b_rows = p.n - n0 < BN ? p.n - n0 : BN;
  const __amdgpu_buffer_rsrc_t arsrc = mp_rsrc(p.a + m0 * k, static_cast<uint32_t>(a_rows * k));
  const __amdgpu_buffer_rsrc_t brsrc = mp_rsrc(p.b + n0 * k, static_cast<uint32_t>(b_rows * k));
  uint32_t voff[QW];
  int ldst[QW];
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const bool is_a = q < BM / 32;
    const int r0 = (4 * q + wave - (is_a ? 0 : BM / 8)) * 8;
    const int r = r0 + lane / 8;
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    voff[q] = r < (is_a ? a_rows : b_rows) ? static_cast<uint32_t>(r * k + 16 * c) : kOob;
    ldst[q] = (is_a ? 0 : BM * BK) + r0 * BK;
  }
  auto issue = [&](int64_t kt, int stage) {
    const uint32_t kb = static_cast<uint32_t>(kt * BK);
#pragma unroll
    for (int q = 0; q < QW; ++q)
      mid_lds_load16(q < BM / 32 ? arsrc : brsrc, smem_mid + stage * STAGE + ldst[q],
                     voff[q] == kOob ? kOob : voff[q] + kb);
  };

  i16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  // fragment of K piece ks (32 bytes): lane l reads row l % 32 of its 32-row tile, logical chunk
  // 2 ks + l / 32, stored at slot (2 ks + l / 32) ^ ((l >> 1) & 7) (the tile's first row is a multiple
  // of 32, so the row's swizzle is that of l % 32)
  const int swz = (lane >> 1) & 7, half = lane >> 5;
  const int arow = (wm * TM * 32 + (lane & 31)) * BK;
  const int brow = BM * BK + (wn * TN * 32 + (lane & 31)) * BK;
  auto compute = [&](int stage) {
    const int8_t *st = smem_mid + stage * STAGE;
    i4_t af[4][TM], bf[4][TN];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int sl = 16 * ((2 * ks + half) ^ swz);
#pragma unroll
      for (int i = 0; i < TM; ++i) af[ks][i] = *reinterpret_cast<const i4_t *>(st + arow + i * 32 * BK + sl);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[ks][j] = *reinterpret_cast<const i4_t *>(st + brow + j * 32 * BK + sl);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks][i], bf[ks][j], acc[i][j], 0, 0, 0);
    // the fragments of K pieces ks + 1 (and 1 for ks = 0) are read while the MFMAs of piece ks run
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * (TM + TN), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * TM * TN, 0);
  };

  const int64_t nkt = k / BK;
  auto kc = [&](int64_t t) { return t < nkt ? t : nkt - 1; };
  issue(0, 0);
  issue(kc(1), 1);
  issue(kc(2), 2);
  // step kt: own loads of tile kt done (2 QW newer load instructions may remain), barrier, refill
  // the stage read in step kt-1, compute.  Loads past the last tile re-read it (never used).
  for (int64_t kt0 = 0; kt0 < nkt; kt0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      if (kt0 + u < nkt) {  // workgroup-uniform
        if constexpr (QW == 8) asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(14) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        static_assert(QW == 8 || QW == 7, "the wait counts two stages of loads");
        issue(kc(kt0 + u + 3), (u + 3) % S);
        compute(u);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS DMA outstanding at exit

  big_epilogue<OUT_DT, TM, TN>(p, acc, m0 + wm * TM * 32 + 4 * (lane >> 5), n0 + wn * TN * 32, m0 + BM <= p.rows,
                               lane);
}

// Any-shape dense fallback: one thread per output.
__global__ void i8_simple_kernel(mp_i8_args p) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= p.rows * p.n) return;
  const int64_t m = tid / p.n, col = tid % p.n;
  int acc = 0;
  for (int64_t c = 0; c < p.k; ++c)
    acc += static_cast<int>(p.a[m * p.k + c]) * static_cast<int>(p.b[col * p.k + c]);
  float v = mp_mul(mp_mul(static_cast<float>(acc), p.s_a[m]), p.s_b[col]);
  if (p.bias) v = mp_add(v, mp_load_as_f32(p.bias, col, p.bias_dtype));
  mp_store_from_f32(p.y, m * p.ldy + col, p.out_dtype, v);
}

constexpr int kTBM = 128, kTBN = 128, kTBK = 64;
// 128-byte K steps: a 64-lane load covers 8 rows x 128 bytes (a 64-byte step makes it
// 16 rows x 64 bytes, which costs the CU several times the load-issue slots)
constexpr int kTBK2 = 128;

}  // namespace

// Large-M kernel: 8 = register-staged interleaved kernel (default), 11 = direct
// global->LDS loads; MP_W8_BIG_VARIANT selects, for measurements.
static int mp_big_variant() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_BIG_VARIANT");
    return e ? atoi(e) : 8;
  }();
  return v;
}

// LDS-staged 16-byte-store epilogue (MP_W8_STAGED=0 turns it off, for measurements).
static int mp_staged_epilogue() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_STAGED");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// Grouped expert GEMMs on the large-M kernels: 1 = register-staged kernel with 128-row
// tiles for SwiGLU outputs (default), 2 = the same for fp32 outputs too, 3 = direct-to-LDS
// kernel with 256-row tiles, 0 = the tiled kernel (MP_W8_GROUPED_BIG, for measurements).
static int mp_grouped_big() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_GROUPED_BIG");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// Row-contiguous GEMV for M <= 2 (MP_W8_GEMV=0 routes those to the skinny MFMA
// kernel, =2/3/5 sets 1/2/4 rows per wave; for measurements).
static int mp_i8_gemv() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_GEMV");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// K step of the tiled kernel: 128 bytes when K allows (default), MP_W8_TILED_BK=64
// forces 64 (for measurements).
static int mp_tiled_bk() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_TILED_BK");
    return e ? atoi(e) : 128;
  }();
  return v;
}

// Tiled-kernel variant for a launch of `wgs` workgroups: 2 = 128-byte K steps with
// four register stages (one workgroup per CU: the grid fits the CUs once), 1 =
// 128-byte steps with one stage (two per CU), 0 = 64-byte steps (three per CU).
static int mp_tiled_variant(int64_t k, int64_t wgs) {
  if (k % kTBK2 != 0 || mp_tiled_bk() != 128) return 0;
  static const int forced = [] {  // MP_W8_TILED_VARIANT=0/1/2 forces a variant (for measurements)
    const char *e = mp_knob("MP_W8_TILED_VARIANT");
    return e ? atoi(e) : -1;
  }();
  if (forced >= 0 && forced <= 2) return forced;
  const int64_t cus = mp_cu_count() > 0 ? mp_cu_count() : 256;
  if (wgs <= cus) return 2;
  if (wgs <= 2 * cus) return 1;
  return 0;
}

// Whether the skinny kernel takes m (<= 64) rows of an n-column output: up to 32 rows, and up to 64
// where the tiled kernel's 128-column grid is small (<= 64 column tiles).  Measured at K = 4096: N = 11008
// (86 tiles) 30.2 against 38.6 us at 64 rows on the tiled kernel, even at 40; N = 4096 (32 tiles) the
// skinny kernel 19.3 against 29.5 us at 64 rows.  MP_W8_SKINNY_MAX_M (a row limit) overrides it, for
// measurements.
static bool mp_skinny_takes(int64_t m, int64_t n) {
  static const int forced = mp_knob("MP_W8_SKINNY_MAX_M") ? atoi(mp_knob("MP_W8_SKINNY_MAX_M")) : -1;
  if (m > 64) return false;
  if (forced >= 0) return m <= forced;
  return m <= 32 || mp_cdiv(n, 128) <= 64;
}

// Dense tiled launches with several row tiles on the XCD-paired 1-D grid (default); MP_W8_TILED_XCD=0
// keeps the 2-D grid, for measurements.
static bool mp_tiled_xcd() {
  static const bool v = !(mp_knob("MP_W8_TILED_XCD") && atoi(mp_knob("MP_W8_TILED_XCD")) == 0);
  return v;
}

// Column tiles (16 each) per workgroup of the direct-to-LDS skinny kernel for 3..32 rows, or 0 when it
// does not take the launch: the fewest that leave at most one workgroup per CU (MP_W8_SKDMA=0 keeps
// i8_skinny_kernel, for measurements).  Measured at K = 4096, N = 11008 against i8_skinny_kernel:
// M = 4 / 8 / 16 / 32 12.3 / 12.3 / 12.3 / 14.4 against 15.8 / 15.9 / 15.5 / 24.4 us; M = 16 at
// N = 4096 5.6 against 7.1 us, at K = 11008 13.4 against 17.5 us.
static int mp_skdma_nct(const mp_i8_args &a) {
  static const bool on = !(mp_knob("MP_W8_SKDMA") && atoi(mp_knob("MP_W8_SKDMA")) == 0);
  if (!on || a.rows < 3 || a.rows > 32 || a.k < 4 * 128 || a.k % 128 != 0 || a.k >= (int64_t(1) << 23)) return 0;
  const int64_t cus = mp_cu_count() > 0 ? mp_cu_count() : 256;
  for (int nct = 1; nct <= 4; ++nct)
    if (mp_cdiv(a.n, 16 * nct) <= cus) return nct;
  return 0;
}

static bool mp_skinny_one_chunk() {
  static const bool v = !(mp_knob("MP_W8_SKINNY_ONE_CHUNK") && atoi(mp_knob("MP_W8_SKINNY_ONE_CHUNK")) == 0);
  return v;
}

// Dense 16-bit outputs of the tiled kernel through its LDS-staged 16-byte-store epilogue: N and the row
// stride multiples of 8 elements, y 16-byte aligned (MP_W8_STAGED=0 turns it off, for measurements).
static int mp_tiled_staged_ok(const mp_i8_args &a, int epilogue) {
  return mp_staged_epilogue() && epilogue == MP_EPI_DENSE && a.out_dtype != MP_F32 && a.n % 8 == 0 &&
         a.ldy % 8 == 0 && mp_aligned(a.y, 16);
}

// Dense GEMMs below the large-M range on the direct-to-LDS mid-M kernel when its 128x128 tiles number
// from 64 to three quarters of the CUs (MP_W8_MID=0 keeps the register-staged tiled kernel, for
// measurements).  Measured at K = 4096 against the tiled kernel, with 128-column tiles: M = 256 / 128,
// N = 11008 (172 / 86 tiles) 27.3 / 25.5 against 32.1 / 29.9 us; M = 256 / 512, N = 4096 (64 / 128
// tiles) 21.5 / 23.4 against 28.3 / 30.8 us; M = 48 / 64 / 200 level with it (+-1 us), and faster with
// 96-column tiles (mp_mid_bn).  With 32 tiles (M = 96, N = 4096) it is slower (30 against 28 us), at
// 256 tiles (M = 1000, N = 4096) 34.0 against 33.0 us, and beyond one tile per CU (M = 384 .. 1000,
// N = 11008) the tiled kernel's two workgroups per CU win.
static int mp_mid_kernel() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_MID");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// The mid-M kernel's tile width for a launch, or 0 when it does not take it.  MP_W8_MID_BN=96 / 128
// forces the width (for measurements).
static int mp_mid_bn(const mp_i8_args &a) {
  const int64_t tiles = mp_cdiv(a.n, 128) * mp_cdiv(a.rows, 128);
  const int64_t cus = mp_cu_count() > 0 ? mp_cu_count() : 256;
  if (!(mp_mid_kernel() && a.k >= kMidBK && a.k % kMidBK == 0 && a.k < (int64_t(1) << 23) && tiles >= 64 &&
        4 * tiles <= 3 * cus))
    return 0;
  static const int forced = mp_knob("MP_W8_MID_BN") ? atoi(mp_knob("MP_W8_MID_BN")) : 0;
  if (forced == 96 || forced == 128) return forced;
  // 96-column tiles where they still fit one per CU: measured at K = 4096 against 128-column ones,
  // M = 256 / 128 / 64, N = 11008 25.2 / 22.5 / 25.9 against 27.2 / 25.5 / 29.5 us; M = 200, N = 8192
  // 24.6 against 29.6 us; M = 256 / 512, N = 4096 18.8 / 20.1 against 21.9 / 24.1 us
  return mp_cdiv(a.n, 96) * mp_cdiv(a.rows, 128) <= cus ? 96 : 128;
}

// Persistent large-M launch (MP_W8_PERSIST=0 turns it off, for measurements).
static int mp_persist() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_PERSIST");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// Grouped GEMMs of experts averaging <= 256 rows on i8_moe_kernel: 1 = on (default, two
// register stages in flight), 2 = three stages, 0 = off (MP_W8_MOE, for measurements).
static int mp_moe_kernel() {
  static int v = [] {
    const char *e = mp_knob("MP_W8_MOE");
    return e ? atoi(e) : 1;
  }();
  return v;
}

template <int EPI, int D>
static int mp_launch_moe_d(const mp_i8_args &a, hipStream_t stream) {
  const int64_t n_slices = mp_cdiv(a.n, EPI == MP_EPI_SWIGLU ? kMoeBN / 2 : kMoeBN);
  const int64_t items_ub = n_slices * (mp_cdiv(a.rows, kMoeBM) + a.n_experts);
  if (items_ub > INT32_MAX / 2) return MP_ERR_SHAPE;
  // persistent: one workgroup per CU (whole multiples of 8), or fewer when the items are fewer
  const int64_t cus = mp_cu_count() >= 8 ? mp_cu_count() / 8 * 8 : 256;
  const int64_t wgs = mp_cdiv(items_ub, 8) * 8;
  const dim3 grid(static_cast<unsigned>(wgs < cus ? wgs : cus));
  // > 64 KB of dynamic LDS must be allowed per kernel (idempotent, cheap)
  if (hipFuncSetAttribute(reinterpret_cast<const void *>(i8_moe_kernel<EPI, D>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMoeSmem)) != hipSuccess)
    return MP_ERR_HIP;
  hipLaunchKernelGGL((i8_moe_kernel<EPI, D>), grid, dim3(kMoeThreads), kMoeSmem, stream, a,
                     static_cast<int>(n_slices));
  MP_CHECK_LAUNCH();
  return MP_OK;
}

template <int EPI>
static int mp_launch_moe(const mp_i8_args &a, hipStream_t stream) {
  if (mp_moe_kernel() == 2) return mp_launch_moe_d<EPI, 2>(a, stream);
  return mp_launch_moe_d<EPI, 1>(a, stream);
}

// Shared launcher (dense + grouped).
int mp_launch_i8_gemm(const mp_i8_args &a, int epilogue, hipStream_t stream) {
  // the tiled kernel addresses a tile's 128 output rows, and its 128 activation rows, through one
  // descriptor each
  const bool aligned = mp_aligned(a.a, 16) && mp_aligned(a.b, 16) && a.ldy < (int64_t(1) << 23) &&
                       a.k < (int64_t(1) << 23);
  if (a.offsets) {
    // experts of a few hundred rows (serving-size MoE): one workgroup per 256 rows of an
    // expert and weight slice, so each slice streams once per expert
    if (mp_moe_kernel() && aligned && a.k % kMoeBK == 0 && a.k <= (1 << 17) && a.n_experts <= kMoeMaxExperts &&
        a.rows <= kMoeBM * static_cast<int64_t>(a.n_experts) && a.ldy <= (1 << 21) && a.n_partial <= (1 << 21)) {
      if (epilogue == MP_EPI_SWIGLU) return mp_launch_moe<MP_EPI_SWIGLU>(a, stream);
      if (epilogue == MP_EPI_F32) return mp_launch_moe<MP_EPI_F32>(a, stream);
      return mp_launch_moe<MP_EPI_DENSE>(a, stream);
    }
    // grouped: the large-M kernel (one 256-row chunk of one expert per workgroup, each
    // weight slice streamed once per chunk) for fp32 / SwiGLU outputs, else the tiled kernel
    // (fp32 outputs stay on the tiled kernel unless MP_W8_GROUPED_BIG >= 2: with N = hidden the
    // 256-column tiles leave most CUs idle)
    if (mp_grouped_big() && aligned && a.k % (2 * kBigBK) == 0 && a.k <= INT32_MAX &&
        ((epilogue == MP_EPI_F32 && mp_grouped_big() >= 2) ||
         (epilogue == MP_EPI_SWIGLU && a.n % (kBigBN / 2) == 0)) &&
        a.n <= INT32_MAX / 2 && a.rows <= INT32_MAX) {
      const bool swi = epilogue == MP_EPI_SWIGLU;
      const int64_t n_tiles = mp_cdiv(a.n, swi ? kBigBN / 2 : kBigBN);
      const int64_t m_slots = mp_cdiv(a.rows, kBigBM) + a.n_experts;
      // the expert weights stream from HBM once: the direct-to-LDS kernel keeps three
      // K tiles in flight per CU (K % 256), the register-staged one two
      if (a.k % (kDmaStages * kBigBK) == 0 && mp_grouped_big() == 3) {
        const size_t smemd = static_cast<size_t>(kDmaStages) * (kBigBM + kBigBN) * kBigBK;
        const void *fd = swi ? reinterpret_cast<const void *>(i8_gemm_dma_kernel<MP_F32, MP_EPI_SWIGLU>)
                             : reinterpret_cast<const void *>(i8_gemm_dma_kernel<MP_F32, MP_EPI_F32>);
        if (hipFuncSetAttribute(fd, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smemd)) !=
            hipSuccess)
          return MP_ERR_HIP;
        const dim3 gridd(static_cast<unsigned>(n_tiles), static_cast<unsigned>(m_slots));
        if (swi)
          hipLaunchKernelGGL((i8_gemm_dma_kernel<MP_F32, MP_EPI_SWIGLU>), gridd, dim3(512), smemd, stream, a, 1, 1);
        else
          hipLaunchKernelGGL((i8_gemm_dma_kernel<MP_F32, MP_EPI_F32>), gridd, dim3(512), smemd, stream, a, 1, 1);
        MP_CHECK_LAUNCH();
        return MP_OK;
      }
      // 128-row tiles: one tile per expert of up to 128 rows, 48 KB of LDS
      const size_t smem = static_cast<size_t>(2) * (128 + kBigBN) * kBigLD;
      const int64_t m_slots128 = mp_cdiv(a.rows, 128) + a.n_experts;
      const dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(m_slots128));
      if (swi)
        hipLaunchKernelGGL((i8_gemm_big_kernel<MP_F32, MP_EPI_SWIGLU, 2>), grid, dim3(kBigThreads), smem, stream, a, 1,
                           1);
      else
        hipLaunchKernelGGL((i8_gemm_big_kernel<MP_F32, MP_EPI_F32, 2>), grid, dim3(kBigThreads), smem, stream, a, 1,
                           1);
      MP_CHECK_LAUNCH();
      return MP_OK;
    }
    if (a.k % kTBK != 0 || !aligned) return MP_ERR_SHAPE;
    const int64_t n_tiles =
        mp_cdiv(a.n, epilogue == MP_EPI_SWIGLU ? kTBN / 2 : kTBN);
    const int64_t m_slots = mp_cdiv(a.rows, kTBM) + a.n_experts;
    const dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(m_slots));
    const int tv = mp_tiled_variant(a.k, n_tiles * m_slots);
    if (tv > 0) {
      if (epilogue == MP_EPI_SWIGLU) {
        if (tv == 2) hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_SWIGLU, 3>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_SWIGLU, 0>), grid, dim3(256), 0, stream, a);
      } else if (epilogue == MP_EPI_F32) {
        if (tv == 2) hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_F32, 3>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_F32, 0>), grid, dim3(256), 0, stream, a);
      } else {
        if (tv == 2) hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_DENSE, 3>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_DENSE, 0>), grid, dim3(256), 0, stream, a);
      }
      MP_CHECK_LAUNCH();
      return MP_OK;
    }
    if (epilogue == MP_EPI_SWIGLU)
      hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK, MP_EPI_SWIGLU>), grid, dim3(256), 0, stream, a);
    else if (epilogue == MP_EPI_F32)
      hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK, MP_EPI_F32>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK, MP_EPI_DENSE>), grid, dim3(256), 0, stream, a);
    MP_CHECK_LAUNCH();
    return MP_OK;
  }
  if (epilogue == MP_EPI_SWIGLU) return MP_ERR_ARG;
  if (a.rows <= 2 && mp_i8_gemv() && a.k % 16 == 0 && aligned && epilogue == MP_EPI_DENSE &&
      a.n * a.k < (int64_t(1) << 32) && a.rows * a.k < (int64_t(1) << 32)) {
    // row-contiguous int8 GEMV: R rows per wave (1: measured best on the 7B shapes), 4 waves per
    // workgroup
    const int64_t nch = mp_cdiv(a.k, 1024);
    const int rsel = mp_i8_gemv() >= 2 ? mp_i8_gemv() - 1 : 1;  // MP_W8_GEMV=2/3/5: 1/2/4 rows per wave
    const dim3 grid(static_cast<unsigned>(mp_cdiv(a.n, 4 * rsel)));
#define MP_I8_GEMV(R_)                                                                              \
  do {                                                                                              \
    if (a.rows == 1) {                                                                              \
      if (nch <= 4) hipLaunchKernelGGL((i8_gemv_kernel<R_, 1, 4>), grid, dim3(256), 0, stream, a); \
      else hipLaunchKernelGGL((i8_gemv_kernel<R_, 1, 2>), grid, dim3(256), 0, stream, a);          \
    } else {                                                                                        \
      hipLaunchKernelGGL((i8_gemv_kernel<R_, 2, 2>), grid, dim3(256), 0, stream, a);               \
    }                                                                                               \
  } while (0)
    if (rsel == 1) MP_I8_GEMV(1);
    else if (rsel == 4) MP_I8_GEMV(4);
    else MP_I8_GEMV(2);
#undef MP_I8_GEMV
  } else if (mp_skdma_nct(a) > 0 && aligned && epilogue == MP_EPI_DENSE) {
    const int nct = mp_skdma_nct(a);
    const int mt = a.rows <= 16 ? 1 : 2;
    const dim3 grid(static_cast<unsigned>(mp_cdiv(a.n, 16 * nct)));
#define MP_SD(MT_, NCT_)                                                                                      \
  do {                                                                                                       \
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(i8_skinny_dma_kernel<MT_, NCT_>),                 \
                            hipFuncAttributeMaxDynamicSharedMemorySize,                                      \
                            static_cast<int>(skdma_smem(MT_, NCT_))) != hipSuccess)                          \
      return MP_ERR_HIP;                                                                                     \
    hipLaunchKernelGGL((i8_skinny_dma_kernel<MT_, NCT_>), grid, dim3(256), skdma_smem(MT_, NCT_), stream, a); \
  } while (0)
    if (mt == 1) {
      if (nct == 1) MP_SD(1, 1);
      else if (nct == 2) MP_SD(1, 2);
      else if (nct == 3) MP_SD(1, 3);
      else MP_SD(1, 4);
    } else {
      if (nct == 1) MP_SD(2, 1);
      else if (nct == 2) MP_SD(2, 2);
      else if (nct == 3) MP_SD(2, 3);
      else MP_SD(2, 4);
    }
#undef MP_SD
  } else if (mp_skinny_takes(a.rows, a.n) && a.k % 64 == 0 && aligned && epilogue == MP_EPI_DENSE &&
             a.k <= INT32_MAX && a.n <= INT32_MAX) {
    const int mi = static_cast<int>(a.rows);
    const int mt = mi <= 16 ? 1 : (mi <= 32 ? 2 : 4);
    const int nw = mt == 4 ? 4 : 8;
    const int nblk = static_cast<int>(a.k / 64);
    int cb = (kMpXLdsBudget / mi - 16) / 64;
    cb = cb < 1 ? 1 : (cb > nblk ? nblk : cb);
    // the whole K in one chunk when it fits 76 KB (two workgroups per CU still fit) and the
    // workgroup's staging registers (skinny_pmax pieces per thread) hold it: no second
    // activation round trip and weight-pipeline restart (MP_W8_SKINNY_ONE_CHUNK=0: off)
    const int64_t stage_cap = static_cast<int64_t>(nw) * 64 * skinny_pmax(nw * 64);
    if (mp_skinny_one_chunk() && static_cast<int64_t>(mi) * (nblk * 64 + 16) + 16 <= 76 * 1024 &&
        static_cast<int64_t>(mi) * nblk * 4 <= stage_cap)
      cb = nblk;
    if (static_cast<int64_t>(mi) * cb * 4 > stage_cap) return MP_ERR_SHAPE;  // cannot happen with the rule above
    size_t smem = static_cast<size_t>(mi) * (cb * 64 + 16) + 16;
    const size_t red = static_cast<size_t>(nw) * mt * 1024;
    smem = smem > red ? smem : red;
    const dim3 grid(static_cast<unsigned>(mp_cdiv(a.n, 16)));
    if (mt == 1)
      hipLaunchKernelGGL((i8_skinny_kernel<1, 8>), grid, dim3(512), smem, stream, a, cb);
    else if (mt == 2)
      hipLaunchKernelGGL((i8_skinny_kernel<2, 8>), grid, dim3(512), smem, stream, a, cb);
    else
      hipLaunchKernelGGL((i8_skinny_kernel<4, 4>), grid, dim3(256), smem, stream, a, cb);
  } else if (a.rows >= 1024 && a.k % (2 * kBigBK) == 0 && aligned && epilogue == MP_EPI_DENSE) {
    const int tiles_m = static_cast<int>(mp_cdiv(a.rows, kBigBM));
    const int tiles_n = static_cast<int>(mp_cdiv(a.n, kBigBN));
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
    if (mp_big_variant() == 11 && a.k % (kDmaStages * kBigBK) == 0) {
      const size_t smemd = static_cast<size_t>(kDmaStages) * (kBigBM + kBigBN) * kBigBK;
      const void *fk[3] = {reinterpret_cast<const void *>(i8_gemm_dma_kernel<MP_F16, MP_EPI_DENSE>),
                           reinterpret_cast<const void *>(i8_gemm_dma_kernel<MP_BF16, MP_EPI_DENSE>),
                           reinterpret_cast<const void *>(i8_gemm_dma_kernel<MP_F32, MP_EPI_DENSE>)};
      for (const void *fn : fk)
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smemd)) !=
            hipSuccess)
          return MP_ERR_HIP;
      if (a.out_dtype == MP_F16)
        hipLaunchKernelGGL((i8_gemm_dma_kernel<MP_F16, MP_EPI_DENSE>), grid, dim3(512), smemd, stream, a, tiles_m, tiles_n);
      else if (a.out_dtype == MP_BF16)
        hipLaunchKernelGGL((i8_gemm_dma_kernel<MP_BF16, MP_EPI_DENSE>), grid, dim3(512), smemd, stream, a, tiles_m, tiles_n);
      else
        hipLaunchKernelGGL((i8_gemm_dma_kernel<MP_F32, MP_EPI_DENSE>), grid, dim3(512), smemd, stream, a, tiles_m, tiles_n);
    } else {
      // persistent when the tiles exceed one workgroup per CU (MP_W8_PERSIST=0 disables)
      const int cus = mp_cu_count();
      const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
      const dim3 pgrid(static_cast<unsigned>(mp_persist() && tiles > cus && cus >= 8 ? (cus / 8) * 8 : tiles));
      const size_t smem = static_cast<size_t>(2) * (kBigBM + kBigBN) * kBigLD;
      const void *fk[3] = {reinterpret_cast<const void *>(i8_gemm_big_kernel<MP_F16, MP_EPI_DENSE>),
                           reinterpret_cast<const void *>(i8_gemm_big_kernel<MP_BF16, MP_EPI_DENSE>),
                           reinterpret_cast<const void *>(i8_gemm_big_kernel<MP_F32, MP_EPI_DENSE>)};
      // > 64 KB of dynamic LDS must be allowed per kernel (idempotent, cheap)
      for (const void *fn : fk)
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)) !=
            hipSuccess)
          return MP_ERR_HIP;
      mp_i8_args am = a;
      am.staged_epilogue = mp_staged_epilogue();
      if (a.out_dtype == MP_F16)
        hipLaunchKernelGGL((i8_gemm_big_kernel<MP_F16, MP_EPI_DENSE>), pgrid, dim3(kBigThreads), smem, stream, am, tiles_m, tiles_n);
      else if (a.out_dtype == MP_BF16)
        hipLaunchKernelGGL((i8_gemm_big_kernel<MP_BF16, MP_EPI_DENSE>), pgrid, dim3(kBigThreads), smem, stream, am, tiles_m, tiles_n);
      else
        hipLaunchKernelGGL((i8_gemm_big_kernel<MP_F32, MP_EPI_DENSE>), pgrid, dim3(kBigThreads), smem, stream, am, tiles_m, tiles_n);
    }
  } else if (aligned && epilogue == MP_EPI_DENSE && mp_mid_bn(a) > 0) {
    const int bn = mp_mid_bn(a);
    const int64_t tn = mp_cdiv(a.n, bn), tm = mp_cdiv(a.rows, 128);
    const dim3 grid(static_cast<unsigned>(mp_cdiv(tn, 8) * 8 * tm));
    const int tmi = static_cast<int>(tm);
#define MP_MID(BN_)                                                                                          \
  do {                                                                                                       \
    const void *fk[3] = {reinterpret_cast<const void *>(i8_mid_kernel<MP_F16, BN_>),                         \
                         reinterpret_cast<const void *>(i8_mid_kernel<MP_BF16, BN_>),                        \
                         reinterpret_cast<const void *>(i8_mid_kernel<MP_F32, BN_>)};                        \
    for (const void *fn : fk)                                                                                \
      if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mid_smem(BN_))) != \
          hipSuccess)                                                                                        \
        return MP_ERR_HIP;                                                                                   \
    if (a.out_dtype == MP_F16)                                                                               \
      hipLaunchKernelGGL((i8_mid_kernel<MP_F16, BN_>), grid, dim3(256), mid_smem(BN_), stream, a, tmi);       \
    else if (a.out_dtype == MP_BF16)                                                                         \
      hipLaunchKernelGGL((i8_mid_kernel<MP_BF16, BN_>), grid, dim3(256), mid_smem(BN_), stream, a, tmi);      \
    else                                                                                                     \
      hipLaunchKernelGGL((i8_mid_kernel<MP_F32, BN_>), grid, dim3(256), mid_smem(BN_), stream, a, tmi);       \
  } while (0)
    if (bn == 96) MP_MID(96);
    else MP_MID(128);
#undef MP_MID
  } else if (aligned && mp_tiled_variant(a.k, mp_cdiv(a.n, kTBN) * mp_cdiv(a.rows, kTBM)) > 0) {
    // several row tiles: a 1-D grid whose row tiles of one column tile share an XCD (mp_tiled_xcd)
    const int64_t tn = mp_cdiv(a.n, kTBN), tm = mp_cdiv(a.rows, kTBM);
    mp_i8_args ax = a;
    ax.xcd_row_tiles = (tm > 1 && mp_tiled_xcd()) ? static_cast<int>(tm) : 0;
    ax.staged_epilogue = mp_tiled_staged_ok(a, epilogue);
    const dim3 grid = ax.xcd_row_tiles ? dim3(static_cast<unsigned>(mp_cdiv(tn, 8) * 8 * tm))
                                       : dim3(static_cast<unsigned>(tn), static_cast<unsigned>(tm));
    const int tv = mp_tiled_variant(a.k, tn * tm);
    if (epilogue == MP_EPI_F32) {
      if (tv == 2) hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_F32, 3>), grid, dim3(256), 0, stream, ax);
      else hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_F32, 0>), grid, dim3(256), 0, stream, ax);
    } else {
      if (tv == 2) hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_DENSE, 3>), grid, dim3(256), 0, stream, ax);
      else hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK2, MP_EPI_DENSE, 0>), grid, dim3(256), 0, stream, ax);
    }
  } else if (a.k % kTBK == 0 && aligned) {
    const int64_t tn = mp_cdiv(a.n, kTBN), tm = mp_cdiv(a.rows, kTBM);
    mp_i8_args ax = a;
    ax.xcd_row_tiles = (tm > 1 && mp_tiled_xcd()) ? static_cast<int>(tm) : 0;
    ax.staged_epilogue = mp_tiled_staged_ok(a, epilogue);
    const dim3 grid = ax.xcd_row_tiles ? dim3(static_cast<unsigned>(mp_cdiv(tn, 8) * 8 * tm))
                                       : dim3(static_cast<unsigned>(tn), static_cast<unsigned>(tm));
    if (epilogue == MP_EPI_F32)
      hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK, MP_EPI_F32>), grid, dim3(256), 0, stream, ax);
    else
      hipLaunchKernelGGL((i8_tiled_kernel<kTBM, kTBN, kTBK, MP_EPI_DENSE>), grid, dim3(256), 0, stream, ax);
  } else {
    if (epilogue != MP_EPI_DENSE) return MP_ERR_SHAPE;
    hipLaunchKernelGGL(i8_simple_kernel, dim3(static_cast<unsigned>(mp_cdiv(a.rows * a.n, 256))), dim3(256), 0,
                       stream, a);
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// ====================================================================== C ABI

// Row quantizer launch: the 16-byte kernel when the rows allow it, else the scalar one.
template <int RULE>
static void mp_launch_rowquant(const void *x, int x_dtype, int64_t rows, int64_t k, int8_t *q, float *s_f32,
                               uint16_t *s_src, int s_src_bf16, float min_scale, int32_t *bad, hipStream_t s) {
  const int per16 = x_dtype == MP_F32 ? 4 : 8;
  const dim3 g(static_cast<unsigned>(rows));
  if (k % per16 == 0 && mp_aligned(x, 16) && mp_aligned(q, 8)) {
    if (x_dtype == MP_F16)
      hipLaunchKernelGGL((rowquant_vec_kernel<RULE, MP_F16>), g, dim3(256), 0, s, x, k, q, s_f32, s_src, s_src_bf16,
                         min_scale, bad);
    else if (x_dtype == MP_BF16)
      hipLaunchKernelGGL((rowquant_vec_kernel<RULE, MP_BF16>), g, dim3(256), 0, s, x, k, q, s_f32, s_src, s_src_bf16,
                         min_scale, bad);
    else
      hipLaunchKernelGGL((rowquant_vec_kernel<RULE, MP_F32>), g, dim3(256), 0, s, x, k, q, s_f32, s_src, s_src_bf16,
                         min_scale, bad);
  } else {
    hipLaunchKernelGGL(rowquant_kernel<RULE>, g, dim3(256), 0, s, x, x_dtype, k, q, s_f32, s_src, s_src_bf16,
                       min_scale, bad);
  }
}

extern "C" int mp_quant_per_token_i8(const void *x, int64_t m, int64_t k, int x_dtype, int8_t *q,
                                     void *scale, int scale_rule, mp_stream_t stream) {
  if (!x || !q || !scale) return MP_ERR_ARG;
  if (x_dtype != MP_F16 && x_dtype != MP_BF16 && x_dtype != MP_F32) return MP_ERR_DTYPE;
  if (m < 0 || k <= 0) return MP_ERR_SHAPE;
  if (m == 0) return MP_OK;
  if (m > INT32_MAX) return MP_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (scale_rule == MP_SCALE_FP32) {
    mp_launch_rowquant<MP_SCALE_FP32>(x, x_dtype, m, k, q, static_cast<float *>(scale), nullptr, 0, 0.0f, nullptr, s);
  } else if (scale_rule == MP_SCALE_FAKE) {
    if (x_dtype != MP_F16 && x_dtype != MP_BF16) return MP_ERR_DTYPE;
    mp_launch_rowquant<MP_SCALE_FAKE>(x, x_dtype, m, k, q, nullptr, static_cast<uint16_t *>(scale),
                                      x_dtype == MP_BF16 ? 1 : 0, 0.0f, nullptr, s);
  } else {
    return MP_ERR_ARG;
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_fake_quant_rows(const void *x, int x_dtype, int64_t rows, int64_t k, int n_bits, int8_t *q,
                                  float *scale, mp_stream_t stream) {
  if (!x || !q || !scale) return MP_ERR_ARG;
  if (x_dtype != MP_F16 && x_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (n_bits < 2 || n_bits > 7) return MP_ERR_ARG;
  if (rows < 0 || k <= 0) return MP_ERR_SHAPE;
  if (rows == 0) return MP_OK;
  if (rows > INT32_MAX) return MP_ERR_SHAPE;
  hipLaunchKernelGGL(fake_rows_nbit_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), x, x_dtype, k,
                     static_cast<float>((1 << (n_bits - 1)) - 1), q, scale);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_w8_quantize_per_channel(const void *w, int64_t n, int64_t k, int w_dtype, int8_t *q,
                                          float *scale_f32, void *scale_src, int scale_rule,
                                          int32_t *bad_count, mp_stream_t stream) {
  if (!w || !q || !scale_f32) return MP_ERR_ARG;
  if (w_dtype != MP_F16 && w_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (n < 0 || k <= 0) return MP_ERR_SHAPE;
  if (n == 0) return MP_OK;
  if (n > INT32_MAX) return MP_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (scale_rule == MP_SCALE_FP32) {
    mp_launch_rowquant<MP_SCALE_FP32>(w, w_dtype, n, k, q, scale_f32, static_cast<uint16_t *>(scale_src),
                                      w_dtype == MP_BF16 ? 1 : 0, 1e-8f, bad_count, s);
  } else if (scale_rule == MP_SCALE_FAKE) {
    mp_launch_rowquant<MP_SCALE_FAKE>(w, w_dtype, n, k, q, scale_f32, static_cast<uint16_t *>(scale_src),
                                      w_dtype == MP_BF16 ? 1 : 0, 0.0f, bad_count, s);
  } else {
    return MP_ERR_ARG;
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_w8a8_gemm(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                            const void *bias, int bias_dtype, void *y, int out_dtype, int64_t m, int64_t n,
                            int64_t k, mp_stream_t stream) {
  if (!qx || !s_tok || !w || !s_ch || !y) return MP_ERR_ARG;
  if (out_dtype != MP_F16 && out_dtype != MP_BF16 && out_dtype != MP_F32) return MP_ERR_DTYPE;
  if (bias && bias_dtype != MP_F16 && bias_dtype != MP_BF16 && bias_dtype != MP_F32) return MP_ERR_DTYPE;
  if (m < 0 || n <= 0 || k <= 0) return MP_ERR_SHAPE;
  if (k > (1 << 17)) return MP_ERR_SHAPE;  // int32 accumulator: 127*127*K < 2^31
  if (m == 0) return MP_OK;
  mp_i8_args a{};
  a.a = qx;
  a.s_a = s_tok;
  a.b = w;
  a.s_b = s_ch;
  a.bias = bias;
  a.bias_dtype = bias_dtype;
  a.y = y;
  a.out_dtype = out_dtype;
  a.rows = m;
  a.n = n;
  a.k = k;
  a.ldy = n;
  return mp_launch_i8_gemm(a, MP_EPI_DENSE, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int mp_w8a8_gemm_fake(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                                 const void *bias, int act_dtype, void *y, int64_t m, int64_t n, int64_t k,
                                 mp_stream_t stream) {
  if (!qx || !s_tok || !w || !s_ch || !y) return MP_ERR_ARG;
  if (act_dtype != MP_F16 && act_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (m < 0 || n <= 0 || k <= 0) return MP_ERR_SHAPE;
  if (m == 0) return MP_OK;
  mp_dq_args d{};
  d.dt = act_dtype;
  d.a = qx;
  d.a_fmt = MP_DQ_I8ROW;
  d.a_scale = s_tok;
  d.b = w;
  d.b_fmt = MP_DQ_I8ROW;
  d.b_scale = s_ch;
  d.bias = bias;
  d.bias_dtype = act_dtype;
  d.y = y;
  d.out_dtype = act_dtype;
  d.ldy = n;
  d.rows = m;
  d.n = n;
  d.k = k;
  return mp_launch_dq_gemm(d, MP_EPI_DENSE, reinterpret_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------ output-quant W8A8 GEMM
// y = W8A8 GEMM output (16-bit), then its per-token int8 codes and scale -- the q/k/v output
// quant of SmoothQuantLinear(quantize_output=True) (fake_quant.py:77-82) returned as
// (int8, scale) (the return_scale form of vllm_ascend.patch:4019-4020).  The GEMM runs on
// i8_moe_kernel with every 256-row group multiplying the same weight (shared_b) and the AMAX
// epilogue: each wave stores its 64 columns of y and the abs-max of each row's rounded values
// over them.  The second launch reduces a row's partial maxima (2 per 128 columns, not the row),
// derives the scale and writes the codes from the 16-bit y.

__global__ void iota_groups_kernel(int64_t *__restrict__ off, int64_t groups, int64_t rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i <= groups) off[i] = i * kMoeBM < rows ? i * kMoeBM : rows;
}

// One workgroup per row: scale from the partial maxima (SIGNED: the bf16 fake rule's row sign
// also needs the row's extremes, read from y), codes of the row's 16-bit values.  VEC: four
// values per 8-byte load, four codes per store (n % 4 == 0, aligned rows).
template <int RULE, bool SIGNED, bool VEC, int DT>
__global__ __launch_bounds__(256) void rows_requant16_kernel(const uint16_t *__restrict__ y, const float *__restrict__ part,
                                                             int n_partial, int64_t n, int mode, int8_t *__restrict__ q,
                                                             float *__restrict__ s_out) {
  __shared__ float red[3][4];
  __shared__ int wbad[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t *row = y + r * n;
  auto val = [&](uint16_t b) { return DT == MP_BF16 ? mp_bf2f(b) : mp_h2f(b); };
  mp_rowstat st{0.f, -INFINITY, INFINITY, 0};
  if (SIGNED) {
    for (int64_t c = tid; c < n; c += 256) {
      const float v = val(row[c]);
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
    const uint2 *src = reinterpret_cast<const uint2 *>(row);
    uint32_t *dst = reinterpret_cast<uint32_t *>(q + r * n);
    for (int64_t c = tid; c < n / 4; c += 256) {
      const uint2 w = src[c];
      const float v0 = val(static_cast<uint16_t>(w.x & 0xFFFFu)), v1 = val(static_cast<uint16_t>(w.x >> 16));
      const float v2 = val(static_cast<uint16_t>(w.y & 0xFFFFu)), v3 = val(static_cast<uint16_t>(w.y >> 16));
      dst[c] = mp_row_code<RULE>(v0, s, sg, mode) | (mp_row_code<RULE>(v1, s, sg, mode) << 8) |
               (mp_row_code<RULE>(v2, s, sg, mode) << 16) | (mp_row_code<RULE>(v3, s, sg, mode) << 24);
    }
  } else {
    for (int64_t c = tid; c < n; c += 256)
      q[r * n + c] = static_cast<int8_t>(mp_row_code<RULE>(val(row[c]), s, sg, mode));
  }
}

static int64_t mp_qout_groups(int64_t m) { return mp_cdiv(m, kMoeBM); }
static int64_t mp_qout_partials(int64_t n) { return 2 * mp_cdiv(n, kMoeBN); }

extern "C" size_t mp_w8a8_gemm_quant_out_workspace_bytes(int64_t m, int64_t n) {
  if (m <= 0 || n <= 0) return 0;
  const int64_t off_bytes = mp_cdiv((mp_qout_groups(m) + 1) * 8, 256) * 256;
  return static_cast<size_t>(off_bytes + m * mp_qout_partials(n) * 4);
}

extern "C" int mp_w8a8_gemm_quant_out(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                                      const void *bias, int bias_dtype, int64_t m, int64_t n, int64_t k, int out_dtype,
                                      int scale_rule, void *y, int8_t *q_out, float *s_out, void *workspace,
                                      size_t workspace_bytes, mp_stream_t stream) {
  if (!qx || !s_tok || !w || !s_ch || !y || !q_out || !s_out) return MP_ERR_ARG;
  if (out_dtype != MP_F16 && out_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (bias && bias_dtype != MP_F16 && bias_dtype != MP_BF16 && bias_dtype != MP_F32) return MP_ERR_DTYPE;
  if (scale_rule != MP_SCALE_FP32 && scale_rule != MP_SCALE_FAKE) return MP_ERR_ARG;
  if (m < 0 || n <= 0 || k <= 0) return MP_ERR_SHAPE;
  if (k % kMoeBK != 0 || k > (1 << 17)) return MP_ERR_SHAPE;
  if (n > (1 << 20) || mp_qout_groups(m) > kMoeMaxExperts) return MP_ERR_SHAPE;
  if (m == 0) return MP_OK;
  if (!mp_aligned(qx, 16) || !mp_aligned(w, 16) || !mp_aligned(y, 4)) return MP_ERR_ALIGN;
  if (!workspace || workspace_bytes < mp_w8a8_gemm_quant_out_workspace_bytes(m, n)) return MP_ERR_WORKSPACE;
  if (!mp_aligned(workspace, 16)) return MP_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t groups = mp_qout_groups(m);
  auto *off = static_cast<int64_t *>(workspace);
  float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) + mp_cdiv((groups + 1) * 8, 256) * 256);
  hipLaunchKernelGGL(iota_groups_kernel, dim3(static_cast<unsigned>(mp_cdiv(groups + 1, 256))), dim3(256), 0, s, off,
                     groups, m);
  MP_CHECK_LAUNCH();
  mp_i8_args a{};
  a.a = qx;
  a.s_a = s_tok;
  a.b = w;
  a.s_b = s_ch;
  a.bias = bias;
  a.bias_dtype = bias_dtype;
  a.y = y;
  a.out_dtype = out_dtype;
  a.amax_partial = part;
  a.n_partial = static_cast<int>(mp_qout_partials(n));
  a.offsets = off;
  a.n_experts = static_cast<int>(groups);
  a.rows = m;
  a.n = n;
  a.k = k;
  a.ldy = n;
  a.shared_b = 1;
  const int rc = mp_launch_moe<MP_EPI_AMAX>(a, s);
  if (rc != MP_OK) return rc;
  const int mode = mp_round_mode_of(out_dtype);
  const bool vec = n % 4 == 0 && mp_aligned(y, 8) && mp_aligned(q_out, 4);
  const auto *yh = static_cast<const uint16_t *>(y);
  const dim3 g(static_cast<unsigned>(m));
#define MP_RQ16(RULE_, SIGNED_, VEC_)                                                                          \
  do {                                                                                                         \
    if (out_dtype == MP_BF16)                                                                                  \
      hipLaunchKernelGGL((rows_requant16_kernel<RULE_, SIGNED_, VEC_, MP_BF16>), g, dim3(256), 0, s, yh, part, \
                         a.n_partial, n, mode, q_out, s_out);                                                  \
    else                                                                                                       \
      hipLaunchKernelGGL((rows_requant16_kernel<RULE_, SIGNED_, VEC_, MP_F16>), g, dim3(256), 0, s, yh, part,  \
                         a.n_partial, n, mode, q_out, s_out);                                                  \
  } while (0)
  if (scale_rule == MP_SCALE_FP32) {
    if (vec) MP_RQ16(MP_SCALE_FP32, false, true);
    else MP_RQ16(MP_SCALE_FP32, false, false);
  } else if (mode == kRoundBF16) {  // the bf16 fake codes reach +-128: the row sign needs its extremes
    if (vec) MP_RQ16(MP_SCALE_FAKE, true, true);
    else MP_RQ16(MP_SCALE_FAKE, true, false);
  } else {
    if (vec) MP_RQ16(MP_SCALE_FAKE, false, true);
    else MP_RQ16(MP_SCALE_FAKE, false, false);
  }
#undef MP_RQ16
  MP_CHECK_LAUNCH();
  return MP_OK;
}
