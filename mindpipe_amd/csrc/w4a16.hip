// W4A16 group-quantized linear for gfx950: AWQ/GPTQ quantizers, the int4 pack
// format, the streaming decode GEMV (M <= 64) and the tiled prefill GEMM.
//
// Weight format (unchanged from the reference export, exporters/vllm.py:89-111):
// packed int32 [N, ceil(K/8)], column k in nibble k%8 of word k/8, plus fp16
// scales [N, K/g] and fp16 zeros [N, K/g] (AWQ) or an implicit zero point 8
// (GPTQ symmetric export, stored nibble = int + 8).
#include "dq_gemm.h"

namespace {

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024.0 in both halves

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t mp_as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

typedef __bf16 bf8w_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf2w_t __attribute__((ext_vector_type(2)));

// The eight weights of one packed word (K positions 0..7, natural order) as bf16 pairs, each
// R_bf16((u - z) s): the reference's bf16 pseudo-quantized weight, (q - z) exact and one rounding of
// the product (awq/quantize/quantizer.py:95-105 in bf16 arithmetic).  (w & 0x000F000F) | 0x64006400
// is the fp16 pair (1024 + u0, 1024 + u4) and the 0x00F000F0 mask gives (1024 + 16 u1, 1024 + 16 u5).
// Each v_fma_mix computes (1024 + u) s - (1024 + z) s, resp. (1024 + 16 u) (s / 16) - (64 + z) s,
// in one fp32 rounding that is exact: both subtracted products are exact in fp32 (at most 19
// significant bits) and so is the difference (u - z) s (at most 12).  v_cvt_pk_bf16_f32 then rounds
// to nearest even once.
__device__ __forceinline__ uint4 w4_bf16x8(uint32_t w, float s, float s16, float nce, float nco, uint32_t m0,
                                           uint32_t m1, uint32_t magic) {
  const uint32_t w8 = w >> 8;
  const h2_t e0 = mp_as_h2((w & m0) | magic), o0 = mp_as_h2((w & m1) | magic);
  const h2_t e1 = mp_as_h2((w8 & m0) | magic), o1 = mp_as_h2((w8 & m1) | magic);
  const bf2w_t p0 = {static_cast<__bf16>(fmaf(static_cast<float>(e0[0]), s, nce)),
                     static_cast<__bf16>(fmaf(static_cast<float>(o0[0]), s16, nco))};
  const bf2w_t p1 = {static_cast<__bf16>(fmaf(static_cast<float>(e1[0]), s, nce)),
                     static_cast<__bf16>(fmaf(static_cast<float>(o1[0]), s16, nco))};
  const bf2w_t p2 = {static_cast<__bf16>(fmaf(static_cast<float>(e0[1]), s, nce)),
                     static_cast<__bf16>(fmaf(static_cast<float>(o0[1]), s16, nco))};
  const bf2w_t p3 = {static_cast<__bf16>(fmaf(static_cast<float>(e1[1]), s, nce)),
                     static_cast<__bf16>(fmaf(static_cast<float>(o1[1]), s16, nco))};
  return make_uint4(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                    __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3));
}


// Eight nibbles of one packed word -> fp16 (1024 + u) in the order
// [k0, k4, k1, k5, k2, k6, k3, k7]: the "or 1024" trick turns a 4-bit integer
// into an fp16 bit pattern with one AND-OR per pair.
__device__ __forceinline__ h8_t dq_magic(uint32_t w) {
  union {
    uint32_t u[4];
    h8_t h;
  } r;
  r.u[0] = (w & 0x000F000Fu) | kMagic;
  r.u[1] = ((w >> 4) & 0x000F000Fu) | kMagic;
  r.u[2] = ((w >> 8) & 0x000F000Fu) | kMagic;
  r.u[3] = ((w >> 12) & 0x000F000Fu) | kMagic;
  return r.h;
}

// Natural-order 8 halves (x0..x7 in 4 dwords) -> [x0,x4,x1,x5,x2,x6,x3,x7],
// the order dq_magic produces, so that the MFMA pairs x_k with w_k.
__device__ __forceinline__ h8_t perm_to_magic(uint4 d) {
  union {
    uint32_t u[4];
    h8_t h;
  } r;
  r.u[0] = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  r.u[1] = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  r.u[2] = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  r.u[3] = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return r.h;
}

// Inverse of the magic order: [k0,k4,k1,k5,k2,k6,k3,k7] -> natural order.
__device__ __forceinline__ uint4 magic_to_natural(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  uint4 d;
  d.x = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  d.y = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  d.z = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  d.w = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
  return d;
}

// ------------------------------------------------------------------ quantizers

// One wave per quantization group (row segment of g elements).  The weight dtype's
// arithmetic (fp16 or bf16) restated as fp32 op + one rounding, as PyTorch does for half
// tensors; quantizer.py:63-105.
template <int DT>
__device__ __forceinline__ float awq_ld(uint16_t b) { return DT == MP_F16 ? mp_h2f(b) : mp_bf2f(b); }
template <int DT>
__device__ __forceinline__ float awq_r(float v) { return DT == MP_F16 ? mp_rh(v) : mp_rbf(v); }
template <int DT>
__device__ __forceinline__ uint16_t awq_st(float v) { return DT == MP_F16 ? mp_f2h(v) : mp_f2bf(v); }

template <int DT>
__global__ __launch_bounds__(256) void awq_quantize_kernel(
    const uint16_t *__restrict__ w, int64_t n_rows, int64_t k, int gs, int n_groups, int zero_point, int n_bit,
    uint32_t *__restrict__ packed, int64_t kw, uint16_t *__restrict__ scales,
    uint16_t *__restrict__ zeros, uint16_t *__restrict__ wdeq) {
  const int lane = threadIdx.x & 63;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grp >= n_rows * n_groups) return;
  const int64_t row = grp / n_groups;
  const int gi = static_cast<int>(grp % n_groups);
  const int64_t e0 = static_cast<int64_t>(gi) * gs;
  const uint16_t *src = w + row * k + e0;

  float mx = -INFINITY, mn = INFINITY;
  for (int i = lane; i < gs; i += 64) {
    const float v = awq_ld<DT>(src[i]);
    mx = fmaxf(mx, zero_point ? v : fabsf(v));
    mn = fminf(mn, v);
  }
  mx = mp_wave_max(mx);
  mn = mp_wave_min(mn);

  // n_bit-wide codes (1..8): [0, 2^n - 1] with a zero point, else [-2^(n-1), 2^(n-1) - 1];
  // every bound is exact in fp16 and bf16
  float s, z, qmin, qmax;
  if (zero_point) {
    qmin = 0.0f;
    qmax = static_cast<float>((1 << n_bit) - 1);
    float d = awq_r<DT>(mx - mn);
    if (d < 1e-5f) d = awq_r<DT>(1e-5f);
    s = awq_r<DT>(d / qmax);
    z = -rintf(awq_r<DT>(mn / s));
    if (z < 0.0f) z = 0.0f;   // keeps -0.0 like torch.clamp_
    if (z > qmax) z = qmax;
  } else {
    qmin = -static_cast<float>(1 << (n_bit - 1));
    qmax = static_cast<float>((1 << (n_bit - 1)) - 1);
    float a = mx;
    if (a < 1e-5f) a = awq_r<DT>(1e-5f);
    s = awq_r<DT>(a / qmax);
    z = 0.0f;
  }
  if (lane == 0) {
    scales[row * n_groups + gi] = awq_st<DT>(s);
    if (zero_point) zeros[row * n_groups + gi] = awq_st<DT>(z);
  }
  // pass 2: one packed word (8 consecutive columns) per lane iteration (4-bit codes only;
  // packed is null for other widths)
  const int nwords = (gs + 7) / 8;
  for (int c = lane; c < nwords; c += 64) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int idx = 8 * c + j;
      if (idx >= gs) break;
      const float v = awq_ld<DT>(src[idx]);
      const float t = rintf(awq_r<DT>(v / s));
      float q = awq_r<DT>(t + z);
      if (q < qmin) q = qmin;
      if (q > qmax) q = qmax;
      const float deq = awq_r<DT>(awq_r<DT>(q - z) * s);
      if (wdeq) wdeq[row * k + e0 + idx] = awq_st<DT>(deq);
      const uint32_t u = static_cast<uint32_t>(static_cast<int>(q) + (zero_point ? 0 : 8));
      word |= u << (4 * j);
    }
    if (packed) packed[row * kw + e0 / 8 + c] = word;
  }
}

// GPTQ symmetric RTN, fp32 math; one thread per (row, group).
__global__ void gptq_rtn_kernel(const void *__restrict__ w, int w_dtype, int64_t n_rows, int64_t k,
                                int gs, int8_t *__restrict__ iw, uint32_t *__restrict__ packed,
                                int64_t kw, uint16_t *__restrict__ scale) {
  const int n_groups = static_cast<int>(k / gs);
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= n_rows * n_groups) return;
  const int64_t row = tid / n_groups;
  const int gi = static_cast<int>(tid % n_groups);
  const int64_t base = row * k + static_cast<int64_t>(gi) * gs;
  float xmin = 0.0f, xmax = 0.0f;
  for (int i = 0; i < gs; ++i) {
    const float v = mp_load_as_f32(w, base + i, w_dtype);
    xmin = fminf(xmin, v);
    xmax = fmaxf(xmax, v);
  }
  xmax = fmaxf(fabsf(xmin), xmax);
  if (xmin < 0.0f) xmin = -xmax;
  if (xmin == 0.0f && xmax == 0.0f) {
    xmin = -1.0f;
    xmax = 1.0f;
  }
  const float s = (xmax - xmin) / 15.0f;
  scale[row * n_groups + gi] = mp_f2h(s);
  uint32_t word = 0;
  for (int i = 0; i < gs; ++i) {
    const float v = mp_load_as_f32(w, base + i, w_dtype);
    float q = rintf(v / s) + 8.0f;
    q = fminf(fmaxf(q, 0.0f), 15.0f);
    const int u = static_cast<int>(q);
    if (iw) iw[base + i] = static_cast<int8_t>(u - 8);
    const int64_t col = static_cast<int64_t>(gi) * gs + i;
    word |= static_cast<uint32_t>(u) << (4 * (col & 7));
    if ((col & 7) == 7 || i == gs - 1) {
      if (packed) packed[row * kw + col / 8] = word;
      word = 0;
    }
  }
}

__global__ void pack_int4_kernel(const int8_t *__restrict__ iw, int64_t n_rows, int64_t k,
                                 uint32_t *__restrict__ packed, int64_t kw, int32_t *__restrict__ bad) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= n_rows * kw) return;
  const int64_t row = tid / kw, c = tid % kw;
  uint32_t word = 0;
  int nbad = 0;
  for (int j = 0; j < 8; ++j) {
    const int64_t col = c * 8 + j;
    if (col >= k) break;
    const int v = iw[row * k + col];
    nbad += (v < -8 || v > 7);
    word |= (static_cast<uint32_t>(v + 8) & 0xFu) << (4 * j);
  }
  packed[tid] = word;
  if (nbad && bad) atomicAdd(bad, nbad);
}

__global__ void unpack_int4_kernel(const uint32_t *__restrict__ packed, int64_t n_rows, int64_t k,
                                   int64_t kw, int8_t *__restrict__ iw) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= n_rows * k) return;
  const int64_t row = tid / k, col = tid % k;
  const uint32_t word = packed[row * kw + col / 8];
  iw[tid] = static_cast<int8_t>(static_cast<int>((word >> (4 * (col & 7))) & 0xFu) - 8);
}

// ------------------------------------------------------------------ decode GEMV (M <= 64)
//
// Work split: a workgroup has 8 waves arranged as T = 8/S column tiles of 16
// output columns, S waves per tile splitting K into contiguous block ranges
// (a block = 128 K columns = one quantization group at g = 128).  S is chosen
// on the host so that about 2048 waves stream the weights; S = 1 needs no
// cross-wave reduction.  The activations are staged once per workgroup into
// LDS (K chunks within the LDS budget), already permuted into the order the
// nibble trick produces, with per-(row, block) sums.  Per block a lane loads
// 16 B of packed weights (32 columns of one output row); a wave load covers 16
// rows x 64 B.  One 32-bit load brings the fp16 scales (and zeros) of two
// consecutive blocks.  MFMA f32_16x16x32_f16: B = weights (column n =
// lane%16), A = activations (row m = lane%16).  Weights enter the MFMA as
// (1024 + u) from the bit trick; per group
//   sum_k x_k (u_k - z) s = s * (acc - (1024 + z) * sum_k x_k)
// removes the offset in fp32.  The hot path is straight-line code (clamped
// loads, surplus blocks masked by a zero scale): control-flow joins make the
// compiler wait for every outstanding load.

// (w & mask) | magic with both constants held in VGPRs: the compiler then
// emits one v_and_or_b32 per nibble pair (with literal operands it needs two
// instructions, since a gfx9 VOP3 instruction takes one literal / scalar
// operand).
__device__ __forceinline__ h8_t dq_magic_fast(uint32_t w, uint32_t mask_v, uint32_t magic_v) {
  union {
    uint32_t u[4];
    h8_t h;
  } r;
  r.u[0] = (w & mask_v) | magic_v;
  r.u[1] = ((w >> 4) & mask_v) | magic_v;
  r.u[2] = ((w >> 8) & mask_v) | magic_v;
  r.u[3] = ((w >> 12) & mask_v) | magic_v;
  return r.h;
}

// LDS layout of one K chunk (cb blocks), all offsets in bytes:
//   xs   [M][cb*256 + 16]  activations, permuted to the nibble-trick order
//   xsum [M][cb]            fp32 per-(row, block) sums
//   sz   [T*16][cb]         (scale | zero << 16) per (output row, group)
//   dummy 16 B              sink for masked stores
constexpr int kDecXPieces = 4;  // 16-B activation pieces staged per thread per chunk
constexpr int kDecSPieces = 2;  // scale (and zero) pieces staged per thread per chunk

struct DecodeLds {
  int xstride, xsum_off, sz_off, dummy_off, bytes;
  __host__ __device__ DecodeLds(int m, int cb, int tiles) {
    xstride = cb * 256 + 16;
    xsum_off = m * xstride;
    sz_off = xsum_off + m * cb * 4;
    dummy_off = sz_off + tiles * 16 * cb * 4;
    bytes = dummy_off + 16;
  }
};

template <int MT, int S, bool ZP, bool SZ16>
__global__ __launch_bounds__(512) void w4a16_decode_kernel(
    const uint16_t *__restrict__ x, int m_rows, int k, const uint32_t *__restrict__ wq, int n_cols,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, int cb) {
  constexpr int NW = 8, T = NW / S, U = 4, NT = NW * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const DecodeLds L(m_rows, cb, T);
  uint8_t *xs = smem;
  float *xsum = reinterpret_cast<float *>(smem + L.xsum_off);
  uint32_t *szl = reinterpret_cast<uint32_t *>(smem + L.sz_off);
  uint8_t *dummy = smem + L.dummy_off;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave / S, sw = wave % S;
  const int wg_col0 = blockIdx.x * T * 16;
  const int n = wg_col0 + tile * 16 + (lane & 15);
  const int nn = n < n_cols ? n : n_cols - 1;
  const int kq = lane >> 4;
  const int kw = k >> 3;
  const int nblk = k >> 7;
  const uint32_t *wrow = wq + static_cast<int64_t>(nn) * kw + 4 * kq;
  const int mlast = m_rows - 1;
  uint32_t magic_v = kMagic, mask_v = 0x000F000Fu;
  asm volatile("" : "+v"(magic_v), "+v"(mask_v));  // opaque: keep both constants in VGPRs

  f4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  const h8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  uint4 wa[U], wb[U];

  for (int c0 = 0; c0 < nblk; c0 += cb) {
    const int cbn = (nblk - c0) < cb ? (nblk - c0) : cb;
    const int lo = (cbn * sw) / S;
    const int hi = (cbn * (sw + 1)) / S;
    const int nmine = hi - lo;
    const int blast = c0 + cbn - 1;
    auto issue = [&](uint4 *w, int r0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int b = c0 + lo + r0 + u;
        b = b < blast ? b : blast;
        w[u] = *reinterpret_cast<const uint4 *>(wrow + b * 16);
      }
    };
    auto compute = [&](const uint4 *w, int r0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u;
        const bool live = r < nmine;
        int jl = lo + r;
        jl = jl < cbn - 1 ? jl : cbn - 1;
        const uint32_t wsel[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
        const uint32_t szv = szl[(tile * 16 + (lane & 15)) * cb + jl];
        const float su = live ? mp_h2f(static_cast<uint16_t>(szv)) : 0.0f;
        const float zu = 1024.0f + (ZP ? mp_h2f(static_cast<uint16_t>(szv >> 16)) : 8.0f);
        h8_t bq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) bq[q] = dq_magic_fast(wsel[q], mask_v, magic_v);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int ma = t * 16 + (lane & 15);
          const int mac = ma < mlast ? ma : mlast;
          f4_t cg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            h8_t a = *reinterpret_cast<const h8_t *>(xs + mac * L.xstride + (jl * 128 + 32 * kq + 8 * q) * 2);
            a = ma < m_rows ? a : zero8;
            cg = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[q], cg, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int mc = t * 16 + 4 * kq + i;
            const int mcc = mc < mlast ? mc : mlast;
            float xsv = xsum[mcc * cb + jl];
            xsv = mc < m_rows ? xsv : 0.f;
            acc[t][i] = fmaf(su, fmaf(-zu, xsv, cg[i]), acc[t][i]);
          }
        }
      }
    };

    // ---- staging loads (activations, then scales / zeros), then the weight
    // prefetch, so that the LDS writes wait only for the older staging loads
    // (the host sizes cb so that the pieces fit kDecXPieces / kDecSPieces per thread)
    constexpr int PMAX = kDecXPieces;
    const int pieces = m_rows * cbn * 16;
    uint4 xv[PMAX];
#pragma unroll
    for (int i = 0; i < PMAX; ++i) {
      int p = tid + i * NT;
      p = p < pieces ? p : pieces - 1;
      const int m = p / (cbn * 16), c8 = p % (cbn * 16);
      xv[i] = *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(m) * k + c0 * 128 + c8 * 8);
    }
    // scale / zero pieces: 8 groups (16 B) or 2 groups (4 B) of one output row
    constexpr int GPP = SZ16 ? 8 : 2;
    constexpr int SMAX = kDecSPieces;
    const int ppr = (cbn + GPP - 1) / GPP;               // pieces per row
    const int spieces = T * 16 * ppr;
    uint4 sv[SMAX], zv[SMAX];
#pragma unroll
    for (int i = 0; i < SMAX; ++i) {
      int p = tid + i * NT;
      p = p < spieces ? p : spieces - 1;
      const int r = p / ppr, c = p % ppr;
      int row = wg_col0 + r;
      row = row < n_cols ? row : n_cols - 1;
      const int64_t off = static_cast<int64_t>(row) * n_groups + c0 + c * GPP;
      if (SZ16) {
        sv[i] = *reinterpret_cast<const uint4 *>(sc + off);
        zv[i] = ZP ? *reinterpret_cast<const uint4 *>(zr + off) : make_uint4(0, 0, 0, 0);
      } else {
        sv[i] = make_uint4(*reinterpret_cast<const uint32_t *>(sc + off), 0u, 0u, 0u);
        zv[i] = make_uint4(ZP ? *reinterpret_cast<const uint32_t *>(zr + off) : 0u, 0u, 0u, 0u);
      }
    }
    issue(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (c0 > 0) mp_lds_barrier();
#pragma unroll
    for (int i = 0; i < PMAX; ++i) {
      const int p = tid + i * NT;
      const int pc = p < pieces ? p : pieces - 1;
      const int m = pc / (cbn * 16), c8 = pc % (cbn * 16);
      uint8_t *dst = p < pieces ? xs + m * L.xstride + c8 * 16 : dummy;
      const h8_t v = perm_to_magic(xv[i]);
      *reinterpret_cast<h8_t *>(dst) = v;
      // per-(row, block) sum: the 16 pieces of a block sit in 16 consecutive lanes
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) part += static_cast<float>(v[e]);
      part += __shfl_xor(part, 1, 64);
      part += __shfl_xor(part, 2, 64);
      part += __shfl_xor(part, 4, 64);
      part += __shfl_xor(part, 8, 64);
      float *sdst = (p < pieces && (c8 & 15) == 0) ? xsum + m * cb + (c8 >> 4) : reinterpret_cast<float *>(dummy);
      *sdst = part;
    }
#pragma unroll
    for (int i = 0; i < SMAX; ++i) {
      const int p = tid + i * NT;
      const int pc = p < spieces ? p : spieces - 1;
      const int r = pc / ppr, c = pc % ppr;
      const uint32_t s4[4] = {sv[i].x, sv[i].y, sv[i].z, sv[i].w};
      const uint32_t z4[4] = {zv[i].x, zv[i].y, zv[i].z, zv[i].w};
#pragma unroll
      for (int e = 0; e < GPP / 2; ++e) {
        const int j = c * GPP + 2 * e;
        const bool ok = p < spieces && j < cbn;
        uint32_t *d = ok ? szl + r * cb + j : reinterpret_cast<uint32_t *>(dummy);
        d[0] = (s4[e] & 0xFFFFu) | (z4[e] << 16);
        d = (ok && j + 1 < cbn) ? d + 1 : reinterpret_cast<uint32_t *>(dummy);
        d[0] = (s4[e] >> 16) | (z4[e] & 0xFFFF0000u);
      }
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

  if (S == 1) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = t * 16 + 4 * kq + i;
        if (m < m_rows && n < n_cols) {
          float v = acc[t][i];
          if (bias) v += mp_h2f(bias[n]);
          y[static_cast<int64_t>(m) * n_cols + n] = mp_f2h(v);
        }
      }
    return;
  }
  mp_lds_barrier();
  float *red = reinterpret_cast<float *>(smem);  // [NW][MT][4][64]
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * MT + t) * 4 + i) * 64 + lane] = acc[t][i];
  mp_lds_barrier();
  for (int o = tid; o < T * MT * 256; o += NT) {
    const int tl = o / (MT * 256), rem = o % (MT * 256);
    const int t = rem >> 8, r = rem & 255;
    const int l = r & 63, i = r >> 6;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < S; ++w) v += red[(((tl * S + w) * MT + t) * 4 + i) * 64 + l];
    const int m = t * 16 + 4 * (l >> 4) + i;
    const int col = wg_col0 + tl * 16 + (l & 15);
    if (m < m_rows && col < n_cols) {
      if (bias) v += mp_h2f(bias[col]);
      y[static_cast<int64_t>(m) * n_cols + col] = mp_f2h(v);
    }
  }
}

// ------------------------------------------------------------------ batched decode (4 < M <= 64)
//
// For small batches the activation bytes per weight byte grow with M: each wave
// owns NT column tiles (16 columns each) and a contiguous K range of whole 8-block
// steps, loads its activations once per 128-column block (reused by the NT tiles)
// and gets the per-row block sums from an MFMA against ones.  S waves of a
// workgroup split K; their partial sums meet in LDS.
//
// Load costs set the structure: a vector-memory instruction whose 64 lanes touch
// 16 rows costs the CU several times the issue slots of one reading a contiguous
// 1 KB, so the kernel keeps their number per weight byte low.  The scales and
// zeros of a tile come as one 16-byte load per 8 blocks (8 groups); activations
// come as contiguous row pieces (4 rows x 256 bytes per load, zeros past M) and
// reach the MFMA layout through the wave's LDS region.  All loads are raw buffer
// loads: the per-lane part of an address is fixed, the block offset is a
// wave-uniform scalar, and blocks past the wave's range point beyond the buffer,
// where loads return zeros without a memory access (no branches around loads: a
// join makes the compiler wait for every outstanding load).  Each block pair's
// activation loads are issued before the next pair's weight prefetch, so a
// compute step waits for its own data only.
//
// BF: bf16 activations, scales, zeros and output.  Every weight is rounded to bf16 as the reference's
// pseudo-quantized weight is (w4_bf16x8, natural K order), so the activation pieces go to the MFMA
// (f32_16x16x32_bf16) as they lie, the group scale is inside each weight and no sum against ones
// is needed.  The SwiGLU form rounds gate, up, silu and the product to bf16.
template <int MT, int NT, int S, bool ZP, bool SWI = false, bool XDB_ON = true, bool BF = false>
__global__ __launch_bounds__(S * 64) void w4a16_batch_kernel(
    const uint16_t *__restrict__ x, int m_rows, int k, const uint32_t *__restrict__ wq, int n_cols,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, int parts) {
  constexpr int U = 2;        // blocks per prefetch buffer
  constexpr int STEP = 8;     // blocks per scale / zero vector
  constexpr int XI = 4 * MT;  // activation loads per block (4 rows x 256 bytes each)
  constexpr bool XDB = MT == 1 && XDB_ON;  // double-buffered activations (registers allow it at 16 rows)
  __shared__ float red[S > 1 ? S : 1][MT * NT * 4][64];
  __shared__ uint4 xst[S][16 * MT * 16];  // per wave: one block of 16 MT rows x 256 bytes
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint4 *xsw = xst[wave];
  const int kq = lane >> 4;
  const uint32_t kw = static_cast<uint32_t>(k) >> 3;
  const int nblk = k >> 7;
  // SWI: tiles j < NT/2 are gate columns, tile j + NT/2 the matching up columns (rows
  // [I, 2I) of the weight, I = n_cols / 2); the output is act = silu(gate) * up, [M, I]
  constexpr int NO = SWI ? NT / 2 : NT;  // output tiles per wave
  static_assert(!SWI || NT % 2 == 0, "SwiGLU pairs tiles");
  const int n_out = SWI ? n_cols / 2 : n_cols;
  // parts > 1 (more rows than the 16 MT-row tiling): the parts workgroups of a column group take
  // rows [16 MT p, 16 MT (p + 1)).  They sit 8 apart in dispatch order, so on one XCD at nearly
  // the same time, and the later reads of the weight slab come from that XCD's L2.
  int bx = blockIdx.x;
  if (parts > 1) {
    const int part = (bx >> 3) % parts;
    bx = (bx / (8 * parts)) * 8 + (bx & 7);
    x += static_cast<int64_t>(part) * 16 * MT * k;
    y += static_cast<int64_t>(part) * 16 * MT * n_out;
    m_rows = min(16 * MT, m_rows - part * 16 * MT);
  }
  const int col0 = bx * NO * 16;
  if (col0 >= n_out || m_rows <= 0) return;  // padding workgroups of a parts grid; uniform, before any barrier
  // K range of this wave: whole steps; blocks at or past nblk are dead
  const int nst = (nblk + STEP - 1) / STEP;
  const int st_lo = (nst * wave) / S;
  const int nsteps = (nst * (wave + 1)) / S - st_lo;
  const int lo = st_lo * STEP;
  uint32_t magic_v = kMagic, mask_v = 0x000F000Fu, mask1_v = 0x00F000F0u;
  asm volatile("" : "+v"(magic_v), "+v"(mask_v), "+v"(mask1_v));
  const h8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};

  // buffer resources (the host checks that every size fits 32 bits)
  const uint32_t wbytes = static_cast<uint32_t>(n_cols) * kw * 4u;
  const uint32_t xbytes = static_cast<uint32_t>(m_rows) * static_cast<uint32_t>(k) * 2u;
  const uint32_t sbytes = static_cast<uint32_t>(n_cols) * static_cast<uint32_t>(n_groups) * 2u;
  const auto wr = mp_rsrc(wq, wbytes);
  const auto xr = mp_rsrc(x, xbytes);
  const auto sr = mp_rsrc(sc, sbytes);
  const auto zrr = mp_rsrc(ZP ? zr : sc, sbytes);
  uint32_t woff[NT], soff[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int n = col0 + (j % NO) * 16 + (lane & 15);
    n = n < n_out ? n : n_out - 1;
    if (SWI && j >= NO) n += n_out;
    woff[j] = (static_cast<uint32_t>(n) * kw + 4u * kq) * 4u;
    soff[j] = static_cast<uint32_t>(n) * static_cast<uint32_t>(n_groups) * 2u;
  }
  // activation load i, lane l: row 4 i + l / 16, 16-byte piece l % 16 of the block
  // (rows past M point beyond the buffer: zeros, no memory access)
  uint32_t xoff[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int m = 4 * i + (lane >> 4);
    xoff[i] = m < m_rows ? (static_cast<uint32_t>(m) * static_cast<uint32_t>(k) + 8u * (lane & 15)) * 2u : xbytes;
  }

  f4_t acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[t][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // block b (absolute) -> scalar byte offsets; dead blocks point past the buffers
  auto woffs = [&](int b) { return b < nblk ? static_cast<uint32_t>(b) * 64u : wbytes; };
  auto xoffs = [&](int b) { return b < nblk ? static_cast<uint32_t>(b) * 256u : xbytes; };
  uint4 wa[U][NT], wb[U][NT];
  auto issue_w = [&](uint4 (*w)[NT], int b0) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < NT; ++j) w[u][j] = mp_buf_load16(wr, woff[j], woffs(b0 + u));
  };
  uint4 xa[U][XI];
  uint4 xb[XDB ? U : 1][XDB ? XI : 1];  // second activation buffer (XDB)
  auto load_x_to = [&](uint4 (*xbuf)[XI], int b0) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < XI; ++i) xbuf[u][i] = mp_buf_load16(xr, xoff[i], xoffs(b0 + u));
  };
  auto load_x = [&](int b0) { load_x_to(xa, b0); };
  // scale / zero vectors (groups b0 .. b0+7 of each tile row; 4-byte aligned rows)
  uint4 sv[NT], zv[NT];
  auto load_sz = [&](int b0) {
    const uint32_t so = b0 < nblk ? static_cast<uint32_t>(b0) * 2u : sbytes;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      sv[j] = mp_buf_load16(sr, soff[j], so);
      if (ZP) zv[j] = mp_buf_load16(zrr, soff[j], so);
    }
  };
  // a block pair: weights w, activations xbuf, scale / zero words sw / zw of each tile
  auto compute_x = [&](uint4 (*w)[NT], uint4 (*xbuf)[XI], const uint32_t (&swd)[NT], const uint32_t (&zwd)[NT]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // transpose through the wave's LDS region into the MFMA layout (lane (m, kq), piece q
      // = row m, K [32 kq + 8 q, +8)); piece c of row r sits at slot c ^ (r % 16), so
      // the writes (16 pieces of one row) and the reads (16 rows, one piece) each
      // cover all 16 bank groups.  One wave writes and reads the region and its LDS
      // accesses execute in order: no barrier.
#pragma unroll
      for (int i = 0; i < XI; ++i) {
        const int r = 4 * i + (lane >> 4);
        xsw[r * 16 + ((lane & 15) ^ (r & 15))] = xbuf[u][i];
      }
      if constexpr (BF) {
        uint4 ab[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int r = 16 * t + (lane & 15);
#pragma unroll
          for (int q = 0; q < 4; ++q) ab[t][q] = xsw[r * 16 + ((4 * kq + q) ^ (r & 15))];
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const float su = mp_bf2f(static_cast<uint16_t>(swd[j] >> (16 * u)));
          const float zr_ = ZP ? mp_bf2f(static_cast<uint16_t>(zwd[j] >> (16 * u))) : 8.0f;
          const float s16 = su * 0.0625f, nce = -((1024.f + zr_) * su), nco = -((64.f + zr_) * su);
          const uint32_t wsel[4] = {w[u][j].x, w[u][j].y, w[u][j].z, w[u][j].w};
          uint4 bq[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) bq[q] = w4_bf16x8(wsel[q], su, s16, nce, nco, mask_v, mask1_v, magic_v);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8w_t, ab[t][q]),
                                                                  __builtin_bit_cast(bf8w_t, bq[q]), acc[t][j], 0, 0, 0);
        }
        continue;
      }
      h8_t af[MT][4];
      f4_t cs[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        cs[t] = f4_t{0.f, 0.f, 0.f, 0.f};
        const int r = 16 * t + (lane & 15);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          af[t][q] = perm_to_magic(xsw[r * 16 + ((4 * kq + q) ^ (r & 15))]);
          cs[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][q], ones, cs[t], 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const uint32_t sw = swd[j], zw = zwd[j];
        const float su = mp_h2f(static_cast<uint16_t>(sw >> (16 * u)));
        const float zu = 1024.0f + (ZP ? mp_h2f(static_cast<uint16_t>(zw >> (16 * u))) : 8.0f);
        const uint32_t wsel[4] = {w[u][j].x, w[u][j].y, w[u][j].z, w[u][j].w};
        h8_t bq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) bq[q] = dq_magic_fast(wsel[q], mask_v, magic_v);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          f4_t cg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q = 0; q < 4; ++q) cg = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t][q], bq[q], cg, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][j][i] = fmaf(su, fmaf(-zu, cs[t][i], cg[i]), acc[t][j][i]);
        }
      }
    }
  };
  // the scale / zero words of pair p (0..3) of the current step
  auto words = [&](int p, uint32_t (&swd)[NT], uint32_t (&zwd)[NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      swd[j] = p == 0 ? sv[j].x : (p == 1 ? sv[j].y : (p == 2 ? sv[j].z : sv[j].w));
      zwd[j] = p == 0 ? zv[j].x : (p == 1 ? zv[j].y : (p == 2 ? zv[j].z : zv[j].w));
    }
  };
  auto compute = [&](uint4 (*w)[NT], int p) {
    uint32_t swd[NT], zwd[NT];
    words(p, swd, zwd);
    compute_x(w, xa, swd, zwd);
  };

  // Steps of 4 block pairs, fully unrolled inside: each prefetch is used in the
  // basic block that issues it; scheduling barriers keep every group of loads
  // where it is written.  Dead blocks (past nblk) read zeros: zero scale, no
  // contribution.
  if constexpr (XDB) {
    // activations one pair ahead in two buffers, the next step's scales during the
    // current step's last pair (its words copied out first): a pair waits only for loads
    // issued a pair or more before it
    issue_w(wa, lo);
    load_x_to(xa, lo);
    load_sz(lo);
    for (int st = 0; st < nsteps; ++st) {
      const int b = lo + st * STEP;
      uint32_t swd[NT], zwd[NT];
      load_x_to(xb, b + 2);
      issue_w(wb, b + 2);
      __builtin_amdgcn_sched_barrier(0);
      words(0, swd, zwd);
      compute_x(wa, xa, swd, zwd);
      __builtin_amdgcn_sched_barrier(0);
      load_x_to(xa, b + 4);
      issue_w(wa, b + 4);
      __builtin_amdgcn_sched_barrier(0);
      words(1, swd, zwd);
      compute_x(wb, xb, swd, zwd);
      __builtin_amdgcn_sched_barrier(0);
      load_x_to(xb, b + 6);
      issue_w(wb, b + 6);
      __builtin_amdgcn_sched_barrier(0);
      words(2, swd, zwd);
      compute_x(wa, xa, swd, zwd);
      __builtin_amdgcn_sched_barrier(0);
      words(3, swd, zwd);
      const int nb = st + 1 < nsteps ? b + STEP : nblk;  // past the range: reads nothing
      load_x_to(xa, nb);
      issue_w(wa, nb);
      load_sz(nb);
      __builtin_amdgcn_sched_barrier(0);
      compute_x(wb, xb, swd, zwd);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
  issue_w(wa, lo);
  for (int st = 0; st < nsteps; ++st) {
    const int b = lo + st * STEP;
    load_sz(b);
    load_x(b);
    __builtin_amdgcn_sched_barrier(0);
    issue_w(wb, b + 2);
    __builtin_amdgcn_sched_barrier(0);
    compute(wa, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_x(b + 2);
    __builtin_amdgcn_sched_barrier(0);
    issue_w(wa, b + 4);
    __builtin_amdgcn_sched_barrier(0);
    compute(wb, 1);
    __builtin_amdgcn_sched_barrier(0);
    load_x(b + 4);
    __builtin_amdgcn_sched_barrier(0);
    issue_w(wb, b + 6);
    __builtin_amdgcn_sched_barrier(0);
    compute(wa, 2);
    __builtin_amdgcn_sched_barrier(0);
    load_x(b + 6);
    __builtin_amdgcn_sched_barrier(0);
    issue_w(wa, st + 1 < nsteps ? b + STEP : nblk);  // the last prefetch reads nothing
    __builtin_amdgcn_sched_barrier(0);
    compute(wb, 3);
    __builtin_amdgcn_sched_barrier(0);
  }
  }

  // biases of the lane's NO output columns (col0 + 16 j + lane % 16), read before any
  // store: a load after a store waits for it
  float bg[NO], bu[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    int col = col0 + j * 16 + (lane & 15);
    col = col < n_out ? col : n_out - 1;
    bg[j] = bias ? (BF ? mp_bf2f(bias[col]) : mp_h2f(bias[col])) : 0.f;
    bu[j] = (SWI && bias) ? (BF ? mp_bf2f(bias[n_out + col]) : mp_h2f(bias[n_out + col])) : 0.f;
  }
  auto emit = [&](int m, int j, float v, float u) {
    const int col = col0 + j * 16 + (lane & 15);
    if (m < m_rows && col < n_out) {
      if (SWI) {
        if (bias) {
          v += bg[j];
          u += bu[j];
        }
        y[static_cast<int64_t>(m) * n_out + col] = BF ? mp_swiglu_bf(mp_rbf(v), mp_rbf(u)) : mp_swiglu_h(mp_rh(v), mp_rh(u));
      } else {
        if (bias) v += bg[j];
        y[static_cast<int64_t>(m) * n_out + col] = BF ? mp_f2bf(v) : mp_f2h(v);
      }
    }
  };
  if (S > 1) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][(t * NT + j) * 4 + i][lane] = acc[t][j][i];
    __syncthreads();
    for (int o = threadIdx.x; o < MT * NO * 4 * 64; o += S * 64) {
      const int slot = o >> 6, l = o & 63;
      const int t = slot / (NO * 4), j = (slot / 4) % NO, i = slot % 4;
      const int sg = (t * NT + j) * 4 + i;  // gate (or plain) slot; its up slot is NO tiles on
      float v = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < S; ++w) {
        v += red[w][sg][l];
        if (SWI) u += red[w][sg + NO * 4][l];
      }
      emit(t * 16 + 4 * (l >> 4) + i, j, v, u);  // l == lane: the stride is a multiple of 64
    }
  } else {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < NO; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          emit(t * 16 + 4 * kq + i, j, acc[t][j][i], SWI ? acc[t][j + NO][i] : 0.f);
  }
}

// ------------------------------------------------------------------ prefill GEMM (M > 64)
//
// 128x128 output tile per workgroup of 4 waves (64x64 each, 2x2 MFMA
// f32_32x32x16_f16 tiles), BK = 64; from M = 256 a 256x128 tile of 8 waves.  Activations are staged to LDS as is; the
// packed weights are dequantised by (u - z) * s in fp16 (the exact fp16 values
// of the reference's pseudo-quantized weight) into LDS.  Double-buffered LDS and
// D + 1 register stages of K tiles in flight (the LDS-only barriers leave them
// outstanding).  Every load is unconditional (rows past M read zeros through the
// activation descriptor, K tiles past the end are clamped), so each wait is a
// partial one; the epilogue stores through a descriptor without branches.
constexpr int kPBM = 128, kPBN = 128, kPBK = 64, kPLD = kPBK + 8;  // row stride in halves
constexpr int kPrefillStages = 4;  // register stages of K tiles

// NTH = 512: a 256 x 128 tile of 8 waves (4 x 2 of 64 x 64): the weight tile is dequantised
// once per 256 rows, each thread two of its words.
// BF: bf16 activations, scales, zeros and output; each weight is dequantised to R_bf16((u - z) s) (the
// reference's bf16 pseudo-quantized weight, w4_bf16x8) and the MFMA is f32_32x32x16_bf16.
// SWI: the fused gate/up weight [2I, K] (n_cols = 2I): a workgroup's 128 weight rows are 64 gate
// rows and the matching 64 up rows, wave column half wn multiplies gate rows [32 wn, +32) (tile j = 0)
// and their up rows (j = 1), and the epilogue writes act [M, I] = silu(gate) * up with the rounding of
// the two-step path (gate and up rounded to the output type first).
template <int D, int NTH = 256, bool BF = false, bool SWI = false>
__global__ __launch_bounds__(NTH) void w4a16_prefill_kernel(
    const uint16_t *__restrict__ x, int m_rows, int k, const uint32_t *__restrict__ wq, int n_cols,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups, int gs,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y) {
  constexpr int BM = NTH / 2;         // 64 rows per wave pair
  constexpr int BW = 1024 / NTH;      // weight words per thread per K tile (a row holds 8)
  constexpr int TPR = 8 / BW;         // threads per weight row
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][BM * kPLD];
  __shared__ __attribute__((aligned(16))) uint16_t sb[2][kPBN * kPLD];
  constexpr uint32_t kOob = 0x80000000u;  // past every descriptor (sizes < 2^31, host check)
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * kPBN;
  const int kw = k >> 3;

  // A staging: 128 rows x 64 halves = 1024 chunks of 16 B, 4 per thread
  // B staging: 128 rows x 8 words = 256 chunks of 16 B (4 words), 1 per thread
  const auto xr = mp_rsrc(x, static_cast<uint32_t>(m_rows) * static_cast<uint32_t>(k) * 2);
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + i * NTH;
    const int m = m0 + (c >> 3);
    aoff[i] = m < m_rows ? (static_cast<uint32_t>(m) * static_cast<uint32_t>(k) + (c & 7) * 8) * 2 : kOob;
  }
  const int brow = tid / TPR, bhalf = tid % TPR;  // each thread: BW words = 8 BW columns
  const int n_out = SWI ? n_cols / 2 : n_cols;
  const int oc0 = SWI ? blockIdx.x * (kPBN / 2) : n0;  // first output column of the workgroup
  int bn;
  if constexpr (SWI) {
    const int oc = oc0 + (brow & (kPBN / 2 - 1));
    const int occ = oc < n_out ? oc : n_out - 1;
    bn = brow < kPBN / 2 ? occ : n_out + occ;
  } else {
    bn = n0 + brow < n_cols ? n0 + brow : n_cols - 1;
  }
  const uint32_t *bsrc = wq + static_cast<int64_t>(bn) * kw + BW * bhalf;
  const uint16_t *zsrc = zr ? zr : sc;  // (no zeros: the scale is read again and 8 used)

  uint4 areg[D + 1][4];
  uint32_t breg[D + 1][BW];
  uint32_t sz[D + 1];  // scale bits | zero bits << 16 of the thread's 32 columns
  const int nkt = k / kPBK;
  auto load_tile = [&](int set, int kt) {
    kt = kt < nkt ? kt : nkt - 1;
    const int kb = kt * kPBK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      areg[set][i] = __builtin_bit_cast(uint4, mp_buf_load16i(xr, aoff[i] + static_cast<uint32_t>(kb) * 2, 0));
    if constexpr (BW == 4) {
      const uint4 v = *reinterpret_cast<const uint4 *>(bsrc + kb / 8);
      breg[set][0] = v.x; breg[set][1] = v.y; breg[set][2] = v.z; breg[set][3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2 *>(bsrc + kb / 8);
      breg[set][0] = v.x; breg[set][1] = v.y;
    }
    const int64_t gi = static_cast<int64_t>(bn) * n_groups + (kb + 8 * BW * bhalf) / gs;
    sz[set] = static_cast<uint32_t>(sc[gi]) | (static_cast<uint32_t>(zsrc[gi]) << 16);
  };
  auto store_tile = [&](int set, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + i * NTH;
      const int r = c >> 3, cc = c & 7;
      *reinterpret_cast<uint4 *>(&sa[buf][r * kPLD + cc * 8]) = areg[set][i];
    }
    if constexpr (BF) {
      const float s_f = mp_bf2f(static_cast<uint16_t>(sz[set] & 0xFFFFu));
      const float z_f = zr ? mp_bf2f(static_cast<uint16_t>(sz[set] >> 16)) : 8.0f;
      const float s16 = s_f * 0.0625f, nce = -((1024.f + z_f) * s_f), nco = -((64.f + z_f) * s_f);
#pragma unroll
      for (int q = 0; q < BW; ++q)
        *reinterpret_cast<uint4 *>(&sb[buf][brow * kPLD + bhalf * 8 * BW + q * 8]) =
            w4_bf16x8(breg[set][q], s_f, s16, nce, nco, 0x000F000Fu, 0x00F000F0u, kMagic);
      return;
    }
    // exact fp16 dequant: (1024+u) - (1024+z) is exact, times s rounds once
    const float bz = zr ? mp_h2f(static_cast<uint16_t>(sz[set] >> 16)) : 8.0f;
    const __half2 off = __float2half2_rn(1024.0f + bz);
    const __half2 s2 = __float2half2_rn(mp_h2f(static_cast<uint16_t>(sz[set] & 0xFFFFu)));
#pragma unroll
    for (int q = 0; q < BW; ++q) {
      const uint32_t w = breg[set][q];
      uint32_t t[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        __half2 h = __builtin_bit_cast(__half2, ((w >> (4 * j)) & 0x000F000Fu) | kMagic);
        h = __hmul2(__hsub2(h, off), s2);
        t[j] = __builtin_bit_cast(uint32_t, h);
      }
      const uint4 nat = magic_to_natural(t[0], t[1], t[2], t[3]);
      *reinterpret_cast<uint4 *>(&sb[buf][brow * kPLD + bhalf * 8 * BW + q * 8]) = nat;
    }
  };

  f16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  auto mma = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < kPBK / 16; ++ks) {
      h8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const h8_t *>(&sa[cur][r * kPLD + ks * 16 + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = SWI ? j * 64 + wn * 32 + (lane & 31) : wn * 64 + j * 32 + (lane & 31);
        bf[j] = *reinterpret_cast<const h8_t *>(&sb[cur][r * kPLD + ks * 16 + 8 * (lane >> 5)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if constexpr (BF)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8w_t, af[i]),
                                                                 __builtin_bit_cast(bf8w_t, bf[j]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // Register set s holds tile t with t % (D + 1) == s; at step kt tiles kt+1 .. kt+D+1 are
  // in flight.  Tile kt+1 goes to LDS after tile kt is multiplied, and its set is refilled
  // with tile kt+D+2 (clamped past the end, never used).
#pragma unroll
  for (int d = 0; d <= D; ++d) load_tile(d, d);
  store_tile(0, 0);
  load_tile(0, D + 1);
  mp_lds_barrier();
  for (int kt0 = 0; kt0 < nkt; kt0 += D + 1) {
#pragma unroll
    for (int d = 0; d <= D; ++d) {
      const int kt = kt0 + d;
      const int nxt = (d + 1) % (D + 1);
      if (kt < nkt) {  // workgroup-uniform
        mma(kt & 1);
        if (kt + 1 < nkt) store_tile(nxt, (kt + 1) & 1);
      }
      load_tile(nxt, kt + D + 2);
      mp_lds_barrier();
    }
  }

  // epilogue: biases first, then stores through a descriptor (rows past M and columns past
  // N dropped without a branch)
  const auto yr = mp_rsrc(y, static_cast<uint32_t>(m_rows) * static_cast<uint32_t>(n_out) * 2);
  if constexpr (SWI) {
    const int col = oc0 + wn * 32 + (lane & 31);
    const bool cval = col < n_out;
    const int cc = cval ? col : n_out - 1;
    const float bg = bias ? (BF ? mp_bf2f(bias[cc]) : mp_h2f(bias[cc])) : 0.f;
    const float bu = bias ? (BF ? mp_bf2f(bias[n_out + cc]) : mp_h2f(bias[n_out + cc])) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const float g = acc[i][0][r] + bg, u = acc[i][1][r] + bu;
        const uint16_t a = BF ? mp_swiglu_bf(mp_rbf(g), mp_rbf(u)) : mp_swiglu_h(mp_rh(g), mp_rh(u));
        const uint32_t o = (cval && m < m_rows) ? (static_cast<uint32_t>(m) * static_cast<uint32_t>(n_out) + col) * 2 : kOob;
        mp_buf_store2(yr, o, a);
      }
    return;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 64 + j * 32 + (lane & 31);
    const bool cval = col < n_cols;
    const uint16_t bb = bias ? bias[cval ? col : n_cols - 1] : 0;
    const float bv = bias ? (BF ? mp_bf2f(bb) : mp_h2f(bb)) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const uint32_t o = (cval && m < m_rows) ? (static_cast<uint32_t>(m) * static_cast<uint32_t>(n_cols) + col) * 2 : kOob;
        mp_buf_store2(yr, o, BF ? mp_f2bf(acc[i][j][r] + bv) : mp_f2h(acc[i][j][r] + bv));
      }
  }
}

// ------------------------------------------------------------------ any-shape fallback
// One thread per output, exact fp16 dequant; used only for shapes the fast
// kernels do not take (tiny K, K not a multiple of 128 / 64, odd groups).
__global__ void w4a16_simple_kernel(const uint16_t *__restrict__ x, int64_t m_rows, int64_t k,
                                    const uint32_t *__restrict__ wq, int64_t n_cols, int64_t kw,
                                    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr,
                                    int n_groups, int gs, const uint16_t *__restrict__ bias,
                                    uint16_t *__restrict__ y) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= m_rows * n_cols) return;
  const int64_t m = tid / n_cols, n = tid % n_cols;
  float acc = 0.f;
  for (int64_t c = 0; c < k; ++c) {
    const uint32_t u = (wq[n * kw + c / 8] >> (4 * (c & 7))) & 0xFu;
    const int gi = static_cast<int>(c / gs);
    const float s = mp_h2f(sc[n * n_groups + gi]);
    const float z = zr ? mp_h2f(zr[n * n_groups + gi]) : 8.0f;
    const float w = mp_rh(mp_rh(static_cast<float>(u) - z) * s);
    acc = fmaf(mp_h2f(x[m * k + c]), w, acc);
  }
  if (bias) acc += mp_h2f(bias[n]);
  y[tid] = mp_f2h(acc);
}

}  // namespace


// ---------------------------------------------------------------- M = 1 GEMV
// Bandwidth kernel for one activation row.  A wave owns R output rows over all
// of K; lane l covers K positions [j*2048 + 32 l, +32) of chunk j, so its
// activation slice is loaded once per chunk and reused by the R rows.  Each
// 32-bit weight word is dequantised without a shift for half of its nibbles:
//   (w & 0x000F000F) | 0x6400_6400 -> 1024 + u    (nibbles 0, 4)
//   (w & 0x00F000F0) | 0x6400_6400 -> 1024 + 16 u (nibbles 1, 5)
// and the same two masks on w >> 8 for nibbles 2, 6 / 3, 7.  The two scalings
// go to separate fp32 dot-product chains d0 / d1, so with X0 / X1 the slice
// sums over the matching positions,
//   sum_k (u_k - z) x_k = d0 + d1 / 16 - (1024 X0 + 64 X1) - z (X0 + X1).
// Scale / zero pairs of the R rows x 16 groups are loaded by one coalesced
// load per 64 entries and handed to the lanes that use them by ds_bpermute.
// The R per-lane partials are reduced across the wave by a halving butterfly.

// NRM: the activation row is h = RMSNorm(x + residual) * w, computed by every
// workgroup in its prologue into LDS (the arithmetic of add_rmsnorm_quant_kernel
// with fp16 rows: fp32 sum, residual_out = round(sum), r = 1 / sqrt(mean(sum^2) +
// eps), h = round(round(sum * r) * w)); workgroup 0 writes residual_out.  One K
// iteration per wave (k = 2048 C S): the row's loads go out first, then the
// weights, so the norm runs while the weights stream in.
struct MpRowNorm {
  const uint16_t *x;    // row to normalise
  const uint16_t *res;  // residual added to it (nullable)
  const uint16_t *w;    // norm weight [k]
  uint16_t *res_out;    // round(x + res) (nullable)
  float eps;
};

template <int R, int C, int S, bool ZP, bool SWI = false, bool NRM = false>
__global__ __launch_bounds__(256) void w4a16_gemv_kernel(
    const uint16_t *__restrict__ x, int k, const uint32_t *__restrict__ wq, int n_cols,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y, const MpRowNorm nrm) {
  constexpr int SZN = R * 16 > 64 ? R * 16 / 64 : 1;  // scale / zero loads per chunk
  constexpr int LPR = 64 / R;                         // lanes per row after the butterfly
  constexpr int GPW = 4 / S;                          // row groups per workgroup (S waves split K)
  // SWI: rows [0, I) are gate rows and [I, 2I) the up rows (I = n_cols / 2); a wave owns
  // R/2 gate rows and the matching R/2 up rows and writes act = silu(gate) * up
  constexpr int RW = SWI ? R / 2 : R;                 // output rows per wave
  __shared__ float red[S > 1 ? 4 : 1][R];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sw = wave % S;
  const int n_out = SWI ? n_cols / 2 : n_cols;
  const int row0 = (blockIdx.x * GPW + wave / S) * RW;
  if (!NRM && S == 1 && row0 >= n_out) return;  // wave-uniform; with S == 1 there is no barrier
  const int kw = k >> 3;
  const int nch = (k + 2047) >> 11;
  uint32_t magic_v = kMagic, m0_v = 0x000F000Fu, m1_v = 0x00F000F0u;
  asm volatile("" : "+v"(magic_v), "+v"(m0_v), "+v"(m1_v));  // opaque: keep the constants in VGPRs
  // weight row of the wave's row r (clamped into its half)
  auto row_of = [&](int r) {
    const int rr = SWI ? r % RW : r;
    const int o = row0 + rr < n_out ? row0 + rr : n_out - 1;
    return SWI && r >= RW ? n_out + o : o;
  };

  const uint32_t *wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = wq + static_cast<int64_t>(row_of(r)) * kw;
  // scale / zero entry e = lane + 64 i: row e / 16 of the wave, group 16 j + e % 16, read as the
  // 32-bit word holding groups (2 t, 2 t + 1) (n_groups even, 4-byte aligned rows)
  const uint32_t *srow[SZN];
  const uint32_t *zrow[SZN];
#pragma unroll
  for (int i = 0; i < SZN; ++i) {
    const int e = lane + 64 * i;
    int r = e >> 4;
    r = r < R ? r : R - 1;
    const int n = row_of(r);
    srow[i] = reinterpret_cast<const uint32_t *>(sc + static_cast<int64_t>(n) * n_groups);
    zrow[i] = reinterpret_cast<const uint32_t *>(ZP ? zr + static_cast<int64_t>(n) * n_groups : sc);
  }
  const int gpair = (lane & 15) >> 1;
  // v_perm selector: (s, z) halves of this lane's group -> s in bits 0-15, z in bits 16-31
  const uint32_t sel = (lane & 1) ? 0x07060302u : 0x05040100u;  // bytes 0-3: s word, 4-7: z word

  struct Stage {
    uint4 w[R];
    uint4 xv[4];
    uint32_t s[SZN], z[SZN];
  };
  auto issue = [&](Stage &st, int j) {
    int kp = j * 2048 + 32 * lane;
    kp = kp < k ? kp : k - 32;
#pragma unroll
    for (int r = 0; r < R; ++r) st.w[r] = *reinterpret_cast<const uint4 *>(wrow[r] + (kp >> 3));
#pragma unroll
    for (int q = 0; q < 4; ++q) st.xv[q] = *reinterpret_cast<const uint4 *>(x + kp + 8 * q);
    int t = 8 * j + gpair;
    t = t < (n_groups >> 1) ? t : (n_groups >> 1) - 1;
#pragma unroll
    for (int i = 0; i < SZN; ++i) {
      st.s[i] = srow[i][t];
      st.z[i] = ZP ? zrow[i][t] : 0x48004800u;  // fp16 8.0
    }
  };
  auto issue_w = [&](Stage &st, int j) {  // issue() without the activation loads
    const int kp = j * 2048 + 32 * lane;
#pragma unroll
    for (int r = 0; r < R; ++r) st.w[r] = *reinterpret_cast<const uint4 *>(wrow[r] + (kp >> 3));
    const int t = 8 * j + gpair;
#pragma unroll
    for (int i = 0; i < SZN; ++i) {
      st.s[i] = srow[i][t];
      st.z[i] = ZP ? zrow[i][t] : 0x48004800u;  // fp16 8.0
    }
  };
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  auto compute = [&](const Stage &st, int j) {
    const bool live = j * 2048 + 32 * lane < k;
    union {
      uint32_t u[16];
      h8_t h[4];
    } xa;
    float x0 = 0.f, x1 = 0.f;
    const h2_t ones = mp_as_h2(0x3C003C00u);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xa.h[q] = perm_to_magic(st.xv[q]);  // a dead lane (clamped K) is removed by its zero scale
      x0 = __builtin_amdgcn_fdot2(mp_as_h2(xa.u[4 * q + 0]), ones, x0, false);
      x1 = __builtin_amdgcn_fdot2(mp_as_h2(xa.u[4 * q + 1]), ones, x1, false);
      x0 = __builtin_amdgcn_fdot2(mp_as_h2(xa.u[4 * q + 2]), ones, x0, false);
      x1 = __builtin_amdgcn_fdot2(mp_as_h2(xa.u[4 * q + 3]), ones, x1, false);
    }
    const float c_off = fmaf(1024.0f, x0, 64.0f * x1);
    const float c_sum = x0 + x1;
    uint32_t szw[SZN];
#pragma unroll
    for (int i = 0; i < SZN; ++i) {
      uint32_t sw = st.s[i], zw = st.z[i];
      asm volatile("" : "+v"(sw), "+v"(zw));  // keep the combine after the barrier: no early wait
      szw[i] = __builtin_amdgcn_perm(zw, sw, sel);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // (s, z) of row r, group 16 j + lane / 4: entry r * 16 + lane / 4
      const uint32_t v = __shfl(szw[(r * 16) >> 6], ((r * 16) & 63) + (lane >> 2), 64);
      const float s = live ? mp_h2f(static_cast<uint16_t>(v)) : 0.f;
      const float z = mp_h2f(static_cast<uint16_t>(v >> 16));
      const uint32_t wv[4] = {st.w[r].x, st.w[r].y, st.w[r].z, st.w[r].w};
      float d0 = 0.f, d1 = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = wv[q], w8 = w >> 8;
        d0 = __builtin_amdgcn_fdot2(mp_as_h2((w & m0_v) | magic_v), mp_as_h2(xa.u[4 * q + 0]), d0, false);
        d1 = __builtin_amdgcn_fdot2(mp_as_h2((w & m1_v) | magic_v), mp_as_h2(xa.u[4 * q + 1]), d1, false);
        d0 = __builtin_amdgcn_fdot2(mp_as_h2((w8 & m0_v) | magic_v), mp_as_h2(xa.u[4 * q + 2]), d0, false);
        d1 = __builtin_amdgcn_fdot2(mp_as_h2((w8 & m1_v) | magic_v), mp_as_h2(xa.u[4 * q + 3]), d1, false);
      }
      acc[r] = fmaf(s, fmaf(d1, 0.0625f, d0) - fmaf(z, c_sum, c_off), acc[r]);
    }
  };

  // C chunks per iteration, all issued before any is used; a chunk past the end
  // re-reads the last one (clamped) and adds nothing (zero scale).  No load
  // crosses an iteration, so every wait is a partial vmcnt and latency is
  // hidden by the other waves of the CU.
  Stage st[C];
  if constexpr (NRM) {
    constexpr int NV = C * S;          // 2048-element slices of the row: k == 2048 NV (host check)
    constexpr uint32_t kOob = 0x80000000u;
    __shared__ uint4 xs[NV * 256];     // the normalised row, fp16
    __shared__ float nred[4];
    const int tid = threadIdx.x;
    const uint32_t rb = static_cast<uint32_t>(k) * 2;
    const auto xr = mp_rsrc(nrm.x, rb);
    const auto rr = mp_rsrc(nrm.res ? nrm.res : nrm.x, nrm.res ? rb : 0);  // null: zeros, unused
    const auto wr = mp_rsrc(nrm.w, rb);
    // row loads first: their wait below leaves the weight loads in flight
    uint4 pw[NV], pa[NV], pr[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) pw[i] = mp_buf_load16(wr, (tid + 256 * i) * 16, 0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      pa[i] = mp_buf_load16(xr, (tid + 256 * i) * 16, 0);
      pr[i] = mp_buf_load16(rr, (tid + 256 * i) * 16, 0);
    }
    const int j = sw * C;
#pragma unroll
    for (int c = 0; c < C; ++c) issue_w(st[c], j + c);
    __builtin_amdgcn_sched_barrier(0);
    const bool has_res = nrm.res != nullptr;
    float v[NV][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t aw[4] = {pa[i].x, pa[i].y, pa[i].z, pa[i].w}, bw[4] = {pr[i].x, pr[i].y, pr[i].z, pr[i].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float f = mp_h2f(static_cast<uint16_t>(aw[e >> 1] >> (16 * (e & 1))));
        const float fb = mp_h2f(static_cast<uint16_t>(bw[e >> 1] >> (16 * (e & 1))));
        f = has_res ? mp_add(f, fb) : f;
        v[i][e] = f;
        ss = mp_add(ss, mp_mul(f, f));
      }
    }
    // residual_out from workgroup 0 (the other workgroups' stores are dropped)
    const auto ro = mp_rsrc(nrm.res_out ? nrm.res_out : nrm.x, nrm.res_out ? rb : 0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = static_cast<uint32_t>(mp_f2h(v[i][2 * e])) | (static_cast<uint32_t>(mp_f2h(v[i][2 * e + 1])) << 16);
      mp_buf_store16(ro, blockIdx.x == 0 ? (tid + 256 * i) * 16 : kOob, make_uint4(o[0], o[1], o[2], o[3]));
    }
    // workgroup sum in the fixed order of the norm kernel: wave butterfly, then the 4 waves
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) nred[wave] = ss;
    mp_lds_barrier();
    const float var = ((nred[0] + nred[1]) + (nred[2] + nred[3])) / static_cast<float>(k);
    const float rs = 1.0f / sqrtf(var + nrm.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t ww[4] = {pw[i].x, pw[i].y, pw[i].z, pw[i].w};
      uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float we = mp_h2f(static_cast<uint16_t>(ww[e >> 1] >> (16 * (e & 1))));
        const float yn = mp_rh(mp_mul(v[i][e], rs));
        o[e >> 1] |= static_cast<uint32_t>(mp_f2h(mp_mul(yn, we))) << (16 * (e & 1));
      }
      xs[tid + 256 * i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    mp_lds_barrier();
    if (S == 1 && row0 >= n_out) return;  // wave-uniform, after the last barrier of S == 1
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int kp = (j + c) * 2048 + 32 * lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) st[c].xv[q] = xs[(kp >> 3) + q];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      compute(st[c], j + c);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    for (int j = sw * C; j < nch; j += S * C) {
#pragma unroll
      for (int c = 0; c < C; ++c) issue(st[c], j + c < nch ? j + c : nch - 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        compute(st[c], j + c);
        __builtin_amdgcn_sched_barrier(0);  // chunk c + 1's waits stay after chunk c's math
      }
    }
  }

  // halving butterfly: after stage b the lane keeps the rows whose index bit matches lane bit (5 - b)
#pragma unroll
  for (int c = R, mask = 32; c > 1; c >>= 1, mask >>= 1) {
    const bool up = (lane & mask) != 0;
#pragma unroll
    for (int i = 0; i < c / 2; ++i) {
      const float send = up ? acc[i] : acc[i + c / 2];
      const float keep = up ? acc[i + c / 2] : acc[i];
      acc[i] = keep + __shfl_xor(send, mask, 64);
    }
  }
  float v = acc[0];
#pragma unroll
  for (int mask = LPR / 2; mask >= 1; mask >>= 1) v += __shfl_xor(v, mask, 64);
  if (S > 1) {  // the S waves of a row group add their K parts
    if ((lane % LPR) == 0) red[wave][lane / LPR] = v;
    __syncthreads();
    if (sw != 0) return;
#pragma unroll
    for (int t = 1; t < S; ++t) v += red[wave + t][lane / LPR];
  }
  if (SWI) {
    // lane r * LPR holds row r; gate row p pairs with up row p + RW (lane (p + RW) * LPR)
    const int r = lane / LPR;
    if (bias) v += mp_h2f(bias[row_of(r)]);
    const float up = __shfl(v, (lane + RW * LPR) & 63, 64);
    const int o = row0 + r;
    if ((lane % LPR) == 0 && r < RW && o < n_out) y[o] = mp_swiglu_h(mp_rh(v), mp_rh(up));
    return;
  }
  const int row = row0 + lane / LPR;
  if ((lane % LPR) == 0 && row < n_cols) {
    if (bias) v += mp_h2f(bias[row]);
    y[row] = mp_f2h(v);
  }
}

// One-row GEMV on the matrix cores: y[n] = sum_k x[k] * s(n, g) * (u(n, k) - z(n, g)) (+ bias),
// the product of ``VllmPackedInt4Linear``'s dequantised weight with one token row
// (reference: scripts/repro/dequant_vllm_int4.py:21-47 dequantisation, then F.linear).
// A workgroup of W waves owns 16 output rows; wave w takes the 512-wide K slices w, w + W, ...
// (NSL of them, K = 512 W NSL).  Lane l: output row n = l & 15, lane group g = l >> 4.
//  * Weights: per slice, four 16-byte loads per lane (row n, K offset 32 (4 i + g) of the slice,
//    i = the slice's 128-wide group); every load of every slice is issued before any arithmetic.
//  * Activations: one 16-byte load per lane per slice (K 8 l .. 8 l + 7 of the slice), permuted
//    into the nibble order of the dequantised words and staged in a wave-private LDS block (no
//    workgroup barrier before the MFMAs).
//  * Dequantisation: (w & 0x000F000F) | 0x64006400 is the fp16 pair 1024 + u, and the 0x00F000F0
//    mask gives 1024 + 16 u; subtracting 1024 + z (resp. 1024 + 16 z) in fp16 is exact, so the
//    MFMA (16x16x32 f16, the row broadcast over the 16 A rows) sums exact products x (u - z) into
//    fp32 and the group scale multiplies each group's sum.
//  * The W waves' partial rows meet in LDS; wave 0 adds them in wave order and stores.
template <int W, int NSL, bool ZP>
__global__ __launch_bounds__(W * 64) void w4a16_gemv_mfma_kernel(
    const uint16_t *__restrict__ x, int k, const uint32_t *__restrict__ wq, int n_rows,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y) {
  constexpr int KS = 512, NG = KS / 128;
  __shared__ uint4 xs[W][NSL][64];  // per slice: 32 blocks of 16 K, each (even 16 B, odd 16 B)
  __shared__ float red[W][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 16 + n;
  const int rowc = row < n_rows ? row : n_rows - 1;
  const int kw = k >> 3;
  // scale / zero words of the slice's four groups first, then the activations, then the weights
  uint2 sv[NSL], zv[NSL];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const int64_t e = static_cast<int64_t>(rowc) * n_groups + (wave + W * sl) * NG;
    sv[sl] = *reinterpret_cast<const uint2 *>(sc + e);
    zv[sl] = ZP ? *reinterpret_cast<const uint2 *>(zr + e) : make_uint2(0x48004800u, 0x48004800u);  // fp16 8
  }
  uint4 xv[NSL];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) xv[sl] = *reinterpret_cast<const uint4 *>(x + (wave + W * sl) * KS + 8 * lane);
  uint4 wv[NSL][NG];
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const uint32_t *wr = wq + static_cast<int64_t>(rowc) * kw + (wave + W * sl) * (KS / 8);
#pragma unroll
    for (int i = 0; i < NG; ++i) wv[sl][i] = *reinterpret_cast<const uint4 *>(wr + 4 * (4 * i + g));
  }
  __builtin_amdgcn_sched_barrier(0);
  // lane l holds K 8 l .. 8 l + 7 = half (l & 1) of block l >> 1: even positions (0 4 2 6) and
  // odd ones (1 5 3 7) of that half, in the order the dequantised words hold the nibbles
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const uint4 d = xv[sl];
    uint2 ev, od;
    ev.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);  // x0 x4
    ev.y = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);  // x2 x6
    od.x = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);  // x1 x5
    od.y = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);  // x3 x7
    uint2 *blk = reinterpret_cast<uint2 *>(&xs[wave][sl][2 * (lane >> 1)]);
    blk[lane & 1] = ev;
    blk[2 + (lane & 1)] = od;
  }
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl)  // keep the scale / zero loads ahead of the weights
    asm volatile("" : "+v"(sv[sl].x), "+v"(sv[sl].y), "+v"(zv[sl].x), "+v"(zv[sl].y));
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes land before its reads
  __builtin_amdgcn_wave_barrier();
  uint32_t magic_v = kMagic, m0_v = 0x000F000Fu, m1_v = 0x00F000F0u;
  asm volatile("" : "+v"(magic_v), "+v"(m0_v), "+v"(m1_v));  // opaque: keep the constants in VGPRs
  float total = 0.f;
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
    const uint32_t sw[2] = {sv[sl].x, sv[sl].y}, zw[2] = {zv[sl].x, zv[sl].y};
    f4_t accr[NG], accx[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const uint32_t zh = (zw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      const h2_t z2 = mp_as_h2(zh | (zh << 16));
      const h2_t ze = z2 + mp_as_h2(kMagic);                        // 1024 + z
      const h2_t zo = z2 * mp_as_h2(0x4C004C00u) + mp_as_h2(kMagic);  // 1024 + 16 z
      const uint32_t w4[4] = {wv[sl][i].x, wv[sl][i].y, wv[sl][i].z, wv[sl][i].w};
      accr[i] = f4_t{0.f, 0.f, 0.f, 0.f};
      accx[i] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t wa = w4[2 * t], wb = w4[2 * t + 1];
        const uint32_t wa8 = wa >> 8, wb8 = wb >> 8;
        h2_t br[4], bx[4];
        br[0] = mp_as_h2((wa & m0_v) | magic_v) - ze;
        br[1] = mp_as_h2((wa8 & m0_v) | magic_v) - ze;
        br[2] = mp_as_h2((wb & m0_v) | magic_v) - ze;
        br[3] = mp_as_h2((wb8 & m0_v) | magic_v) - ze;
        bx[0] = mp_as_h2((wa & m1_v) | magic_v) - zo;
        bx[1] = mp_as_h2((wa8 & m1_v) | magic_v) - zo;
        bx[2] = mp_as_h2((wb & m1_v) | magic_v) - zo;
        bx[3] = mp_as_h2((wb8 & m1_v) | magic_v) - zo;
        const int b = 2 * (4 * i + g) + t;  // 16-K block of the slice
        const uint4 ae = xs[wave][sl][2 * b], ao = xs[wave][sl][2 * b + 1];
        accr[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, ae), __builtin_bit_cast(h8_t, br),
                                                         accr[i], 0, 0, 0);
        accx[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, ao), __builtin_bit_cast(h8_t, bx),
                                                         accx[i], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < NG; ++i)
      total = fmaf(mp_h2f(static_cast<uint16_t>(sw[i >> 1] >> (16 * (i & 1)))), fmaf(accx[i][0], 0.0625f, accr[i][0]),
                   total);
  }
  if (W > 1) {
    if (g == 0) red[wave][n] = total;
    mp_lds_barrier();
    if (wave != 0) return;
    total = red[0][n];
#pragma unroll
    for (int w = 1; w < W; ++w) total += red[w][n];
  }
  if (g == 0 && row < n_rows) {
    if (bias) total += mp_h2f(bias[row]);
    y[row] = mp_f2h(total);
  }
}

// bf16 W4A16 for 1 to 16 activation rows on the matrix cores (group size 128):
// y[m][n] = sum_k x[m][k] R_bf16((u(n, k) - z(n, g)) s(n, g)) (+ bias[n]), F.linear on the
// reference's bf16 pseudo-quantized weight (fp32 accumulation, one rounding of the output).
// A workgroup of W waves owns 16 output rows; wave w takes the contiguous 128-wide K groups
// [w gpw, (w + 1) gpw) and streams them in rounds of two groups, the next round's weight loads in
// flight while the current one is dequantised (register ping-pong).  Lane l: output row
// n = l & 15 (MFMA B column), token l & 15 (A row), lane group g = l >> 4.
//  * Scale / zero: before the first round the wave copies the (s, z) pairs of its 16 rows x gpw
//    groups into LDS with coalesced loads (consecutive lanes, consecutive groups of a row); the
//    rounds read one 32-bit pair per group.  Per-group 16-bit loads scattered over 16 rows cost
//    more than the weight stream itself.  The copy's first batch shares round 0's round trip.
//  * Weights: per group one 16-byte load per lane, words 4 g .. 4 g + 3 of row n's group (K 32 g ..
//    32 g + 31 of the group); word j, dequantised by w4_bf16x8, is the B operand of MFMA j.
//  * Activations: the A operand of MFMA j is x[token][32 g + 8 j .. + 7] of the group, in natural
//    order.  One row (ONE): the wave's slice of x is copied into LDS before the first round and
//    every A row reads it back; several rows: each lane loads its token's row with the weights
//    (lanes past M repeat row M - 1, whose outputs are dropped).
//  * D: lane (n, g) holds tokens 4 g .. 4 g + 3 of output row n; the W partials meet in LDS and
//    wave 0 adds them in wave order.
// Dynamic LDS: W x 16 x (gpw + 1) pair words (row stride padded by one word), then, for ONE,
// W x gpw x 256 bytes of activations.
template <int W, bool ONE, bool ZP>
__global__ __launch_bounds__(W * 64) void w4a16_bf16_small_kernel(
    const uint16_t *__restrict__ x, int m_rows, int k, const uint32_t *__restrict__ wq, int n_rows,
    const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zr, int n_groups, int gpw,
    const uint16_t *__restrict__ bias, uint16_t *__restrict__ y) {
  constexpr int U = 2;
  extern __shared__ uint4 bf_lds[];
  __shared__ f4_t red[W][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int row = row0 + n;
  const int rowc = row < n_rows ? row : n_rows - 1;
  const int tok = ONE ? 0 : (n < m_rows ? n : m_rows - 1);
  const int gb = wave * gpw;
  const int ge = gb + gpw < n_groups ? gb + gpw : n_groups;
  const int cnt = ge > gb ? ge - gb : 0;  // groups of this wave (wave-uniform)
  const int nr = (cnt + U - 1) / U;       // rounds
  const int szst = gpw + 1;
  uint32_t *szw = reinterpret_cast<uint32_t *>(bf_lds) + wave * 16 * szst;
  uint4 *xw = bf_lds + (W * 16 * szst + 3) / 4 + static_cast<int64_t>(wave) * gpw * 16;
  const uint32_t *wr = wq + static_cast<int64_t>(rowc) * (k >> 3) + 4 * g;
  const uint16_t *xr = x + static_cast<int64_t>(tok) * k + 32 * g;
  uint32_t magic_v = kMagic, m0_v = 0x000F000Fu, m1_v = 0x00F000F0u;
  asm volatile("" : "+v"(magic_v), "+v"(m0_v), "+v"(m1_v));  // opaque: keep the constants in VGPRs
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  struct Round {
    uint4 w[U];
    uint4 xv[ONE ? 1 : U][ONE ? 1 : 4];
  };
  // loads of round r (group indices past the wave's range repeat its last group, never used)
  auto load = [&](Round &b, int r) {
    if constexpr (!ONE) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int gi = gb + r * U + u < ge ? gb + r * U + u : ge - 1;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          b.xv[u][j] = *reinterpret_cast<const uint4 *>(xr + static_cast<int64_t>(gi) * 128 + 8 * j);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gi = gb + r * U + u < ge ? gb + r * U + u : ge - 1;
      b.w[u] = *reinterpret_cast<const uint4 *>(wr + static_cast<int64_t>(gi) * 16);
    }
  };
  auto compute = [&](Round &b, int r) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int gl = r * U + u;
      if (gl < cnt) {  // wave-uniform
        const uint32_t szv = szw[n * szst + gl];
        const float s = __uint_as_float(szv << 16), z = __uint_as_float(szv & 0xFFFF0000u);
        const float s16 = s * 0.0625f, nce = -((1024.f + z) * s), nco = -((64.f + z) * s);
        const uint32_t w4[4] = {b.w[u].x, b.w[u].y, b.w[u].z, b.w[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 bw = w4_bf16x8(w4[j], s, s16, nce, nco, m0_v, m1_v, magic_v);
          const uint4 a = ONE ? xw[gl * 16 + 4 * g + j] : b.xv[ONE ? 0 : u][j];
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8w_t, a), __builtin_bit_cast(bf8w_t, bw),
                                                        acc, 0, 0, 0);
        }
      }
    }
  };
  if (nr > 0) {
    // Prologue.  The wave's (s, z) pairs (16 cnt elements, element e = row r * cnt + group c) and, for one
    // row, its activation slice (cnt chunks of 16 bytes per lane row) are copied into LDS.  The first
    // batch -- four pair loads per lane and four chunk loads per lane group -- is issued before round 0's
    // weights and stored after them, so one memory round trip covers the prologue and the first round;
    // a load-then-store loop costs one round trip per iteration, and every wave of the grid sits in
    // that prologue at once.  A wave with at least 16 groups fills every slot of the batch; shorter
    // ranges skip the slots without data (wave-uniform).  Longer ranges take further batches.
    const float rcp = 1.0f / static_cast<float>(cnt);  // (e + 0.5) / cnt rounds to the exact quotient
    auto sz_load = [&](int e) {
      const int ec = e < 16 * cnt ? e : 16 * cnt - 1;
      const int r = static_cast<int>((static_cast<float>(ec) + 0.5f) * rcp), c = ec - r * cnt;
      const int rr = row0 + r < n_rows ? row0 + r : n_rows - 1;
      const int64_t gi = static_cast<int64_t>(rr) * n_groups + gb + c;
      return static_cast<uint32_t>(sc[gi]) | (static_cast<uint32_t>(ZP ? zr[gi] : 0x4100u) << 16);
    };
    auto sz_store = [&](int e, uint32_t v) {
      if (e < 16 * cnt) {
        const int r = static_cast<int>((static_cast<float>(e) + 0.5f) * rcp), c = e - r * cnt;
        szw[r * szst + c] = v;
      }
    };
    auto x_load = [&](int c) {
      const int cc = c < cnt ? c : cnt - 1;
      return *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(gb + cc) * 128 + 8 * n);
    };
    uint32_t szv0[4];
    uint4 xv0[4];
    const bool fullb = cnt >= 16;
    if (fullb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) szv0[i] = sz_load(lane + 64 * i);
      if constexpr (ONE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) xv0[i] = x_load(g + 4 * i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (64 * i < 16 * cnt) szv0[i] = sz_load(lane + 64 * i);
      if constexpr (ONE) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * i < cnt) xv0[i] = x_load(g + 4 * i);
      }
    }
    Round A, B;
    load(A, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (fullb || 64 * i < 16 * cnt) sz_store(lane + 64 * i, szv0[i]);
    if constexpr (ONE) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g + 4 * i < cnt) xw[(g + 4 * i) * 16 + n] = xv0[i];
    }
    for (int e0 = 256; e0 < 16 * cnt; e0 += 256) {  // wave-uniform
      uint32_t v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = sz_load(e0 + lane + 64 * i);
#pragma unroll
      for (int i = 0; i < 4; ++i) sz_store(e0 + lane + 64 * i, v[i]);
    }
    if constexpr (ONE) {
      for (int c0 = 16; c0 < cnt; c0 += 16) {  // wave-uniform
        uint4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = x_load(c0 + g + 4 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (c0 + g + 4 * i < cnt) xw[(c0 + g + 4 * i) * 16 + n] = v[i];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes land before its reads
    __builtin_amdgcn_wave_barrier();
    int r = 0;
    for (; r + 2 < nr; r += 2) {
      load(B, r + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(A, r);
      __builtin_amdgcn_sched_barrier(0);
      load(A, r + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(B, r + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (r + 1 < nr) {
      load(B, r + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(A, r);
      __builtin_amdgcn_sched_barrier(0);
      compute(B, r + 1);
    } else {
      compute(A, r);
    }
  }
  if (W > 1) {
    red[wave][lane] = acc;
    mp_lds_barrier();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < W; ++w) acc += red[w][lane];
  }
  if (row >= n_rows) return;
  const float bv = bias ? mp_bf2f(bias[row]) : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * g + i;
    if (t < (ONE ? 1 : m_rows)) y[static_cast<int64_t>(t) * n_rows + row] = mp_f2bf(acc[i] + bv);
  }
}

// Measurement knobs for the one-row GEMV shape choice: MP_W4_GEMV_R (rows per
// wave), MP_W4_GEMV_C (chunks per iteration), MP_W4_GEMV_S (waves splitting K);
// MP_W4_GEMV_OFF=1 routes one-row calls to the general decode kernel.
static int mp_gemv_env(int which) {
  static const int v[4] = {
      mp_knob("MP_W4_GEMV_OFF") ? atoi(mp_knob("MP_W4_GEMV_OFF")) : 0,
      mp_knob("MP_W4_GEMV_R") ? atoi(mp_knob("MP_W4_GEMV_R")) : 0,
      mp_knob("MP_W4_GEMV_C") ? atoi(mp_knob("MP_W4_GEMV_C")) : 0,
      mp_knob("MP_W4_GEMV_S") ? atoi(mp_knob("MP_W4_GEMV_S")) : 0,
  };
  return v[which];
}

// MP_W4_GEMV_MFMA=0 routes the one-row shapes the matrix-core GEMV takes to the VALU GEMV (for
// measurements).
static bool mp_gemv_mfma() {
  static const bool v = !(mp_knob("MP_W4_GEMV_MFMA") && atoi(mp_knob("MP_W4_GEMV_MFMA")) == 0);
  return v;
}

// MP_W4_BF16_SMALL=0 routes bf16 calls of 1 to 64 rows to the dequantising GEMM (for measurements).
static bool mp_bf16_small() {
  static const bool v = !(mp_knob("MP_W4_BF16_SMALL") && atoi(mp_knob("MP_W4_BF16_SMALL")) == 0);
  return v;
}

// bf16 rows above which the batched kernel's bf16 form runs.  Default 1: measured against the small-M
// kernel at 2 to 16 rows on the 7B / 70B decode shapes, the batched form is faster from 4 rows on (at 16
// rows 6.0 against 8.0 us at 4096 x 4096, 38 against 66 us on the 70B gate/up GEMV) and at 2 rows on
// 4096 x 4096 and the 70B GEMV (5.5 / 32.8 against 5.9 / 38.8 us), 5% slower at 2 rows on the 7B gate/up
// and down projections.  MP_W4_BF16_BATCH_MIN_M overrides it, for measurements.
static int mp_bf16_batch_min_m() {
  static const int v = mp_knob("MP_W4_BF16_BATCH_MIN_M") ? atoi(mp_knob("MP_W4_BF16_BATCH_MIN_M")) : 1;
  return v;
}

// bf16 small-M kernel shape: waves per 16-row block, the fewest powers of two that give the grid
// about 4096 waves (measured on the 7B / 70B decode shapes: 2048 to 8192 land within 5%), at most 16
// and at least two rounds of two groups per wave; and its dynamic LDS (pair words + one-row slice).
static int mp_bf16_small_waves(int64_t blocks, int ng) {
  int w = 1;
  while (w < 16 && blocks * w < 4096 && ng >= 4 * w) w *= 2;
  return w;
}
static size_t mp_bf16_small_lds_for(int w, int gpw, bool one) {
  return ((static_cast<size_t>(w) * 16 * (gpw + 1) + 3) / 4) * 16 + (one ? static_cast<size_t>(w) * gpw * 256 : 0);
}
// dynamic LDS bound: one row up to K of about 38900 (the 70B down projection, K = 28672, takes 72 KiB
// at 8 waves), several rows far beyond any layer; above it the dequantising GEMM
constexpr size_t kBf16SmallLds = 96 * 1024;

template <int W, bool ONE, bool ZP>
static int mp_bf16_small_launch(int64_t blocks, size_t lds, hipStream_t s, const uint16_t *x, int m, int k,
                                const uint32_t *wq, int n, const uint16_t *sc, const uint16_t *zr, int ng, int gpw,
                                const uint16_t *bias, uint16_t *y) {
  // > 64 KiB of dynamic LDS must be allowed per kernel (idempotent, cheap)
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void *>(w4a16_bf16_small_kernel<W, ONE, ZP>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
    return MP_ERR_HIP;
  hipLaunchKernelGGL((w4a16_bf16_small_kernel<W, ONE, ZP>), dim3(static_cast<unsigned>(blocks)), dim3(W * 64), lds, s,
                     x, m, k, wq, n, sc, zr, ng, gpw, bias, y);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Batched-kernel shape knobs (for measurements): MP_W4_BATCH_NT (column tiles per
// wave), MP_W4_BATCH_S (waves splitting K), MP_W4_BATCH_WAVES (target wave count),
// MP_W4_BATCH_ALWAYS=0 (LDS-staged decode kernel above N = 16384 for M < 32).
static int mp_batch_env(int which) {
  static const int v[4] = {
      mp_knob("MP_W4_BATCH_NT") ? atoi(mp_knob("MP_W4_BATCH_NT")) : 0,
      mp_knob("MP_W4_BATCH_S") ? atoi(mp_knob("MP_W4_BATCH_S")) : 0,
      mp_knob("MP_W4_BATCH_WAVES") ? atoi(mp_knob("MP_W4_BATCH_WAVES")) : 0,  // 0: the shape's default
      mp_knob("MP_W4_BATCH_ALWAYS") ? atoi(mp_knob("MP_W4_BATCH_ALWAYS")) : 1,
  };
  return v[which];
}

// Double-buffered activations at <= 16 rows (MP_W4_BATCH_XDB=0 turns them off, for measurements).
static bool mp_batch_xdb() {
  static const bool v = !(mp_knob("MP_W4_BATCH_XDB") && atoi(mp_knob("MP_W4_BATCH_XDB")) == 0);
  return v;
}

// Row tiling of the batched kernel: MT 16-row tiles per wave, and parts = ceil(M / 16 MT)
// workgroups per column group when M exceeds them.  Default: MT = 1 up to 16 rows, 2 above
// (33..64 rows in two parts).  MP_W4_BATCH_PART_MT=1 / 2 / 4 fixes MT (for measurements).
static int mp_batch_part_mt(int64_t m) {
  static const int v = mp_knob("MP_W4_BATCH_PART_MT") ? atoi(mp_knob("MP_W4_BATCH_PART_MT")) : 0;
  if (v == 1 || v == 2 || v == 4) return v;
  return m <= 16 ? 1 : 2;
}
static bool mp_batch_part_mt_forced() {
  static const bool v = mp_knob("MP_W4_BATCH_PART_MT") != nullptr;
  return v;
}

// The batched kernel takes M > this value (default 1: every 2 <= M <= 64, measured faster than
// the LDS-staged kernel at 2..4 rows too, and the fused SwiGLU path then shares its sums);
// MP_W4_BATCH_MIN_M overrides it, for measurements.
static int mp_batch_min_m() {
  static int v = [] {
    const char *e = mp_knob("MP_W4_BATCH_MIN_M");
    return e ? atoi(e) : 1;
  }();
  return v;
}

// Whether the batched kernel (in 16- or 32-row parts) takes m rows of an n-column output: every
// m <= 64, and 64 < m <= 512 where the prefill kernel's grid (128 columns x 128 or 256 rows per
// workgroup) would fill at most half the CUs.  Measured at 96 to 512 rows (fp16 / bf16): 32 / 29 against
// 68 / 70 us at M = 256 and 4096 x 4096, 80 against 187 us at M = 256 and N = 4096, K = 11008, 37 against
// 59 us at M = 96 and N = 12288; the prefill kernel wins from grids of ~170 workgroups (N = 22016, M = 256:
// 77 against 97 us).  MP_W4_BATCH_MAX_M (a row limit) overrides it, for measurements.
static bool mp_batch_takes(int64_t m, int64_t n) {
  static const int forced = mp_knob("MP_W4_BATCH_MAX_M") ? atoi(mp_knob("MP_W4_BATCH_MAX_M")) : -1;
  if (forced >= 0) return m <= forced;
  if (m <= 64) return true;
  if (m > 512) return false;
  const int64_t wgs = mp_cdiv(n, 128) * (m >= 256 ? mp_cdiv(m, 256) : mp_cdiv(m, 128));
  return wgs <= 128;
}

// Prefill GEMM workgroup: 256 x 128 tiles of 8 waves from M = 256 (measured 8-13% faster than
// 128 x 128 tiles of 4 waves on the 7B linears at M = 2048); MP_W4_PREFILL_THREADS=256 selects the
// smaller tile (for measurements).
static int mp_prefill_threads() {
  static const int v = mp_knob("MP_W4_PREFILL_THREADS") ? atoi(mp_knob("MP_W4_PREFILL_THREADS")) : 512;
  return v;
}

// ====================================================================== C ABI

static int mp_launch_awq(const void *w, int w_dtype, int64_t n, int64_t k, int64_t gs, int zero_point, int n_bit,
                         int32_t *packed, void *scales, void *zeros, void *w_deq, mp_stream_t stream) {
  const int64_t n_groups = k / gs;
  const int64_t total = n * n_groups;
  const int64_t kw = mp_cdiv(k, 8);
#define MP_AWQ(DT_)                                                                                          \
  hipLaunchKernelGGL(awq_quantize_kernel<DT_>, dim3(static_cast<unsigned>(mp_cdiv(total, 4))), dim3(256), 0,  \
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(w), n, k,         \
                     static_cast<int>(gs), static_cast<int>(n_groups), zero_point, n_bit,                   \
                     reinterpret_cast<uint32_t *>(packed), kw, static_cast<uint16_t *>(scales),             \
                     static_cast<uint16_t *>(zeros), static_cast<uint16_t *>(w_deq))
  if (w_dtype == MP_F16) MP_AWQ(MP_F16);
  else MP_AWQ(MP_BF16);
#undef MP_AWQ
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_w4_quantize_awq(const void *w, int w_dtype, int64_t n, int64_t k, int group_size, int zero_point,
                                  int32_t *packed, void *scales, void *zeros, void *w_deq,
                                  mp_stream_t stream) {
  if (!w || !packed || !scales || (zero_point && !zeros)) return MP_ERR_ARG;
  if (w_dtype != MP_F16 && w_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (n <= 0 || k <= 0) return MP_ERR_SHAPE;
  const int64_t gs = (group_size > 0 && k % group_size == 0) ? group_size : k;
  if (gs % 8 != 0 && gs != k) return MP_ERR_SHAPE;
  if (gs > (1 << 30)) return MP_ERR_SHAPE;
  return mp_launch_awq(w, w_dtype, n, k, gs, zero_point, 4, packed, scales, zeros, w_deq, stream);
}

// Pseudo-quantization at any code width from 1 to 8 bits: the dequantized weight and, with a
// zero point, the group scales / zeros (no packed codes).
extern "C" int mp_awq_pseudo_quantize(const void *w, int w_dtype, int64_t n, int64_t k, int group_size,
                                      int zero_point, int n_bit, void *scales, void *zeros, void *w_deq,
                                      mp_stream_t stream) {
  if (!w || !scales || !w_deq || (zero_point && !zeros)) return MP_ERR_ARG;
  if (w_dtype != MP_F16 && w_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (n_bit < 1 || n_bit > 8 || (!zero_point && n_bit < 2)) return MP_ERR_ARG;
  if (n <= 0 || k <= 0) return MP_ERR_SHAPE;
  const int64_t gs = (group_size > 0 && k % group_size == 0) ? group_size : k;
  if (gs > (1 << 30)) return MP_ERR_SHAPE;
  return mp_launch_awq(w, w_dtype, n, k, gs, zero_point, n_bit, nullptr, scales, zeros, w_deq, stream);
}

extern "C" int mp_w4_quantize_gptq_rtn(const void *w, int w_dtype, int64_t n, int64_t k, int group_size,
                                       int8_t *int_weight, int32_t *packed, void *scale,
                                       mp_stream_t stream) {
  if (!w || !scale) return MP_ERR_ARG;
  if (w_dtype != MP_F32 && w_dtype != MP_F16 && w_dtype != MP_BF16) return MP_ERR_DTYPE;
  const int64_t gs = group_size > 0 ? group_size : k;
  if (n <= 0 || k <= 0 || k % gs != 0) return MP_ERR_SHAPE;
  const int64_t total = n * (k / gs);
  const int64_t kw = mp_cdiv(k, 8);
  if (packed && gs % 8 != 0 && gs != k) return MP_ERR_SHAPE;
  hipLaunchKernelGGL(gptq_rtn_kernel, dim3(static_cast<unsigned>(mp_cdiv(total, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w, w_dtype, n, k, static_cast<int>(gs),
                     int_weight, reinterpret_cast<uint32_t *>(packed), kw,
                     static_cast<uint16_t *>(scale));
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_pack_int4(const int8_t *int_weight, int64_t n, int64_t k, int32_t *packed,
                            int32_t *bad_count, mp_stream_t stream) {
  if (!int_weight || !packed) return MP_ERR_ARG;
  if (n < 0 || k < 0) return MP_ERR_SHAPE;
  const int64_t kw = mp_cdiv(k, 8);
  if (n * kw == 0) return MP_OK;
  hipLaunchKernelGGL(pack_int4_kernel, dim3(static_cast<unsigned>(mp_cdiv(n * kw, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), int_weight, n, k,
                     reinterpret_cast<uint32_t *>(packed), kw, bad_count);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_unpack_int4(const int32_t *packed, int64_t n, int64_t k, int8_t *int_weight,
                              mp_stream_t stream) {
  if (!int_weight || !packed) return MP_ERR_ARG;
  if (n < 0 || k < 0) return MP_ERR_SHAPE;
  if (n * k == 0) return MP_OK;
  hipLaunchKernelGGL(unpack_int4_kernel, dim3(static_cast<unsigned>(mp_cdiv(n * k, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t *>(packed), n,
                     k, mp_cdiv(k, 8), int_weight);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// One activation row through the norm-fused GEMV (see MpRowNorm): the fused
// add-RMSNorm and the M = 1 GEMV (or gate/up GEMV with SiLU-up) in one launch, the
// same bits as mp_add_rms_norm_quant (quant off) followed by mp_w4a16_gemm /
// mp_w4a16_gemm_swiglu.  K in {2048, 4096, 8192}: the K split the GEMV uses at
// that K, one iteration per wave.
extern "C" int mp_w4a16_gemv_rmsnorm(const void *x, const void *residual, const void *norm_weight, float eps,
                                     void *residual_out, int64_t k, const int32_t *w_packed, int64_t n,
                                     const void *scales, const void *zeros, int group_size, const void *bias,
                                     int swiglu, void *y, int x_dtype, mp_stream_t stream) {
  if (x_dtype != MP_F16) return MP_ERR_DTYPE;
  if (!x || !norm_weight || !w_packed || !scales || !y) return MP_ERR_ARG;
  if (group_size != 128 || (k != 2048 && k != 4096 && k != 8192) || n <= 0 || n > INT32_MAX ||
      (swiglu && (n & 1)))
    return MP_ERR_SHAPE;
  if (!mp_aligned(x, 16) || !mp_aligned(norm_weight, 16) || (residual && !mp_aligned(residual, 16)) ||
      (residual_out && !mp_aligned(residual_out, 16)) || !mp_aligned(w_packed, 16) || !mp_aligned(scales, 4) ||
      (zeros && !mp_aligned(zeros, 4)))
    return MP_ERR_ALIGN;
  // workgroup 0 writes residual_out while the others read x and residual: no overlap
  auto overlaps = [&](const void *a, const void *b) {
    const auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return a && b && pa < pb + static_cast<uintptr_t>(k) * 2 && pb < pa + static_cast<uintptr_t>(k) * 2;
  };
  if (overlaps(residual_out, x) || overlaps(residual_out, residual)) return MP_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const MpRowNorm nrm{static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(residual),
                      static_cast<const uint16_t *>(norm_weight), static_cast<uint16_t *>(residual_out), eps};
  const auto *wp = reinterpret_cast<const uint32_t *>(w_packed);
  const auto *sp = static_cast<const uint16_t *>(scales);
  const auto *zp = static_cast<const uint16_t *>(zeros);
  const auto *bp = static_cast<const uint16_t *>(bias);
  auto *yp = static_cast<uint16_t *>(y);
  const int ki = static_cast<int>(k), ni = static_cast<int>(n), n_groups = ki / 128;
  const int sk = k == 8192 ? 2 : 1;  // the GEMV's choice at these K (chunks C = K / 2048 / S)
  const int64_t groups = swiglu ? mp_cdiv(n / 2, 2) : mp_cdiv(n, 4);
  const dim3 grid(static_cast<unsigned>(mp_cdiv(groups, 4 / sk)));
#define MP_W4_GEMV_NRM(C_, S_, SWI_)                                                                          \
  do {                                                                                                        \
    if (zp)                                                                                                   \
      hipLaunchKernelGGL((w4a16_gemv_kernel<4, C_, S_, true, SWI_, true>), grid, dim3(256), 0, s, nrm.x, ki, wp, \
                         ni, sp, zp, n_groups, bp, yp, nrm);                                                  \
    else                                                                                                      \
      hipLaunchKernelGGL((w4a16_gemv_kernel<4, C_, S_, false, SWI_, true>), grid, dim3(256), 0, s, nrm.x, ki,   \
                         wp, ni, sp, zp, n_groups, bp, yp, nrm);                                              \
  } while (0)
  if (swiglu) {
    if (k == 2048) MP_W4_GEMV_NRM(1, 1, true);
    else if (k == 4096) MP_W4_GEMV_NRM(2, 1, true);
    else MP_W4_GEMV_NRM(2, 2, true);
  } else {
    if (k == 2048) MP_W4_GEMV_NRM(1, 1, false);
    else if (k == 4096) MP_W4_GEMV_NRM(2, 1, false);
    else MP_W4_GEMV_NRM(2, 2, false);
  }
#undef MP_W4_GEMV_NRM
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Launch of the batched kernel's SwiGLU form (fp16, or BF: bf16): NT/2 gate tiles paired with NT/2 up
// tiles per wave.  The caller has checked 1 <= m <= 512 (mp_batch_takes; above 64 rows it calls this
// once per 32-row part), K % 256 == 0, group 128, an even group count, the alignments and the 32-bit
// buffer sizes.
template <bool BF>
static void mp_launch_w4_batch_swiglu(hipStream_t s, const uint16_t *xp, int64_t m, int64_t k, const uint32_t *wp,
                                      int64_t n2, const uint16_t *sp, const uint16_t *zp, int n_groups,
                                      const uint16_t *bp, uint16_t *yp) {
  const int mi = static_cast<int>(m), ki = static_cast<int>(k), ni = static_cast<int>(n2);
  const int64_t half = n2 / 2;
  const int mt = BF && mp_batch_part_mt(m) > 2 ? 2 : mp_batch_part_mt(m);
  const int parts = static_cast<int>(mp_cdiv(m, 16 * mt));
  const bool xdb = mp_batch_xdb();
  // column tiles per wave: 4 for 17..32 rows from I = 8192 and up to 16 rows from I = 16384, else 2
  // (<= 16 rows: measured on the 7B gate/up, I = 11008, at M = 8, 17.4 -> 16.3 us with 2; on the 70B
  // one, I = 28672, at M = 16, 74.3 -> 68.0 us with 4; the 64-row tiling: registers)
  int nt = (half >= 8192 && mt == 2) || (half >= 16384 && mt == 1) ? 4 : 2;
  if (mp_batch_env(0) >= 2) nt = mp_batch_env(0) >= 4 ? 4 : 2;
  const int smax = mt * nt >= 8 ? 4 : 8;
  const int nblk = ki / 128;
  const int nsteps = (nblk + 7) / 8;
  const int64_t groups = mp_cdiv(half, 16 * (nt / 2));
  const int64_t wgs = groups * parts;
  int split = 1;
  while (split < smax && wgs * split < (mp_batch_env(2) > 0 ? mp_batch_env(2) : 1024) && nsteps / (split * 2) >= 1)
    split *= 2;
  if (mp_batch_env(1) > 0) split = mp_batch_env(1) < smax ? mp_batch_env(1) : smax;
  const dim3 grid(static_cast<unsigned>(parts > 1 ? mp_cdiv(groups, 8) * 8 * parts : groups));
  const int hv = parts;
#define MP_W4_BSWI(MT_, NT_, S_)                                                                              \
  do {                                                                                                       \
    if (zp && (xdb || MT_ != 1))                                                                             \
      hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, true, true, true, BF>), grid, dim3(S_ * 64), 0, s, xp, mi, ki,  \
                         wp, ni, sp, zp, n_groups, bp, yp, hv);                                              \
    else if (xdb || MT_ != 1)                                                                                \
      hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, false, true, true, BF>), grid, dim3(S_ * 64), 0, s, xp, mi, ki, \
                         wp, ni, sp, zp, n_groups, bp, yp, hv);                                              \
    else if (zp)                                                                                             \
      hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, true, true, false, BF>), grid, dim3(S_ * 64), 0, s, xp, mi, \
                         ki, wp, ni, sp, zp, n_groups, bp, yp, hv);                                          \
    else                                                                                                     \
      hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, false, true, false, BF>), grid, dim3(S_ * 64), 0, s, xp,   \
                         mi, ki, wp, ni, sp, zp, n_groups, bp, yp, hv);                                      \
  } while (0)
#define MP_W4_BSWI_S(MT_, NT_)                                                  \
  do {                                                                          \
    if (split == 1) MP_W4_BSWI(MT_, NT_, 1);                                    \
    else if (split == 2) MP_W4_BSWI(MT_, NT_, 2);                               \
    else if (split == 4) MP_W4_BSWI(MT_, NT_, 4);                               \
    else MP_W4_BSWI(MT_, NT_, (MT_ * NT_ >= 8 ? 4 : 8));                        \
  } while (0)
  if (mt == 1) {
    if (nt == 2) MP_W4_BSWI_S(1, 2);
    else MP_W4_BSWI_S(1, 4);
  } else if (mt == 2) {
    if (nt == 2) MP_W4_BSWI_S(2, 2);
    else MP_W4_BSWI_S(2, 4);
  } else if constexpr (!BF) {  // the bf16 form takes 16- and 32-row parts only
    if (nt == 2) MP_W4_BSWI_S(4, 2);
    else MP_W4_BSWI_S(4, 4);
  }
#undef MP_W4_BSWI_S
#undef MP_W4_BSWI
}

extern "C" int mp_w4a16_gemm_swiglu(const void *x, int64_t m, int64_t k, const int32_t *w_packed, int64_t n2,
                                    const void *scales, const void *zeros, int group_size, const void *bias,
                                    void *act, int x_dtype, mp_stream_t stream) {
  if (x_dtype != MP_F16 && x_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (m < 0 || n2 <= 0 || (n2 & 1) || k <= 0 || group_size != 128 || k % 256 != 0) return MP_ERR_SHAPE;
  if (m == 0) return MP_OK;
  if (!x || !w_packed || !scales || !act) return MP_ERR_ARG;
  if (n2 > INT32_MAX || k > INT32_MAX) return MP_ERR_SHAPE;
  const int n_groups = static_cast<int>(k / group_size);
  if (n_groups % 2 != 0) return MP_ERR_SHAPE;
  if (!mp_aligned(x, 16) || !mp_aligned(w_packed, 16) || !mp_aligned(scales, 4) ||
      (zeros != nullptr && !mp_aligned(zeros, 4)))
    return MP_ERR_ALIGN;
  if (n2 * (k / 2) >= (int64_t(1) << 32) || m * k * 2 >= (int64_t(1) << 32)) return MP_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto *xp = static_cast<const uint16_t *>(x);
  const auto *wp = reinterpret_cast<const uint32_t *>(w_packed);
  const auto *sp = static_cast<const uint16_t *>(scales);
  const auto *zp = static_cast<const uint16_t *>(zeros);
  const auto *bp = static_cast<const uint16_t *>(bias);
  auto *yp = static_cast<uint16_t *>(act);
  const int ki = static_cast<int>(k), ni = static_cast<int>(n2);
  const int64_t half = n2 / 2;
  if (m > 64 && !mp_batch_takes(m, n2)) {
    // the prefill kernel's SwiGLU form where w4a16_gemm takes the prefill kernel (else the batched
    // kernel's SwiGLU form in row parts, below): 64 output columns (their gate and up rows) per
    // workgroup; its descriptors cover the activation rows and the output (sizes < 2^31)
    if (m * k * 2 >= (int64_t(1) << 31) || m * half * 2 >= (int64_t(1) << 31) || m > INT32_MAX) return MP_ERR_SHAPE;
    const bool wide = mp_prefill_threads() == 512 && m >= 256;
    const dim3 grid(static_cast<unsigned>(mp_cdiv(half, kPBN / 2)), static_cast<unsigned>(mp_cdiv(m, wide ? 256 : kPBM)));
    const int mi = static_cast<int>(m);
#define MP_W4_PF_SWI(NTH_, BF_)                                                                                \
  hipLaunchKernelGGL((w4a16_prefill_kernel<kPrefillStages - 1, NTH_, BF_, true>), grid, dim3(NTH_), 0, s, xp, mi, ki, \
                     wp, ni, sp, zp, n_groups, group_size, bp, yp)
    if (x_dtype == MP_BF16) {
      if (wide) MP_W4_PF_SWI(512, true);
      else MP_W4_PF_SWI(256, true);
    } else {
      if (wide) MP_W4_PF_SWI(512, false);
      else MP_W4_PF_SWI(256, false);
    }
#undef MP_W4_PF_SWI
    MP_CHECK_LAUNCH();
    return MP_OK;
  }
  // one row, fp16: the VALU GEMV's SwiGLU form; otherwise the batched kernel's
  if (m == 1 && x_dtype == MP_F16) {
    // two gate rows and the matching two up rows per wave; chunk / split choice as the GEMV
    const int nch = (ki + 2047) / 2048;
    int c = 1, sk = 1;
    if (nch <= 2) c = nch;
    else if (nch % 4 == 0) { c = 2; sk = 2; }
    else if (nch % 2 == 0 && mp_cdiv(half, 2) < 2048) sk = 2;
    const int64_t groups = mp_cdiv(half, 2);
    const dim3 grid(static_cast<unsigned>(mp_cdiv(groups, 4 / sk)));
#define MP_W4_GEMV_SWI(C_, S_)                                                                               \
  do {                                                                                                       \
    if (zp)                                                                                                  \
      hipLaunchKernelGGL((w4a16_gemv_kernel<4, C_, S_, true, true>), grid, dim3(256), 0, s, xp, ki, wp, ni, sp, \
                         zp, n_groups, bp, yp, MpRowNorm{});                                                 \
    else                                                                                                     \
      hipLaunchKernelGGL((w4a16_gemv_kernel<4, C_, S_, false, true>), grid, dim3(256), 0, s, xp, ki, wp, ni,   \
                         sp, zp, n_groups, bp, yp, MpRowNorm{});                                             \
  } while (0)
    if (sk == 2) {
      if (c == 2) MP_W4_GEMV_SWI(2, 2);
      else MP_W4_GEMV_SWI(1, 2);
    } else {
      if (c == 2) MP_W4_GEMV_SWI(2, 1);
      else MP_W4_GEMV_SWI(1, 1);
    }
#undef MP_W4_GEMV_SWI
    MP_CHECK_LAUNCH();
    return MP_OK;
  }
  if (x_dtype == MP_BF16)
    mp_launch_w4_batch_swiglu<true>(s, xp, m, k, wp, n2, sp, zp, n_groups, bp, yp);
  else
    mp_launch_w4_batch_swiglu<false>(s, xp, m, k, wp, n2, sp, zp, n_groups, bp, yp);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Launch of the batched kernel (fp16, or BF: bf16) with the shape rules measured on the 7B / 70B
// decode shapes; the caller has checked 2 <= m <= 512 (mp_batch_takes), K % 256 == 0, group 128, an even group count,
// 16-byte alignment and the 32-bit buffer sizes.
template <bool BF>
static void mp_launch_w4_batch(hipStream_t s, const uint16_t *xp, int64_t m, int64_t k, const uint32_t *wp,
                               int64_t n, const uint16_t *sp, const uint16_t *zp, int n_groups_i, const uint16_t *bp,
                               uint16_t *yp) {
  const int mi = static_cast<int>(m), ki = static_cast<int>(k), ni = static_cast<int>(n);
  const int nblk = ki / 128;
  // 33..64 rows: one 64-row tile (fp16) where N <= 8192, else two 32-row parts (measured on the 70B
  // shapes at M = 64: o 34.4 -> 27.7 us and down 106.9 -> 80.0 us with the 64-row tile; q/k/v,
  // N = 10240, 40.1 -> 51.0 us)
  int mt = BF && mp_batch_part_mt(m) > 2 ? 2 : mp_batch_part_mt(m);
  if (!BF && mt == 2 && m > 32 && m <= 64 && n <= 8192 && !mp_batch_part_mt_forced()) mt = 4;
  const int parts = static_cast<int>(mp_cdiv(m, 16 * mt));
  const bool xdb = mp_batch_xdb();
  // column tiles per wave (measured on the 7B / 70B decode shapes, M = 8..64): one for N <= 4096
  // (enough workgroups), four from N = 12288 (activation loads shared by more tiles), and from
  // N = 10240 up to 16 rows (the 70B q/k/v at M = 16: 21.7 -> 19.3 us, where two tiles leave 320
  // workgroups for 256 CUs; at M = 64 four tiles are slower, 40.1 -> 42.3 us); the 64-row tiling
  // takes at most 2 (registers)
  int nt = n <= 4096 ? 1 : ((n >= 12288 || (n >= 10240 && m <= 16)) && mt < 4 ? 4 : 2);
  if (mp_batch_env(0) > 0) nt = mp_batch_env(0) >= 4 ? 4 : mp_batch_env(0);
  const int smax = mt * nt >= 8 ? 4 : (mt * nt > 1 ? 8 : 16);  // register budget per wave count
  const int64_t groups = mp_cdiv(n, 16 * nt);
  const int nsteps = (nblk + 7) / 8;                 // 8-block steps (one scale vector each)
  // waves splitting K, >= 1 step each, up to ~1024 waves (~2048 for one-tile waves of <= 16 rows,
  // measured on the 7B down projection at M = 8: 11.6 -> 10.2 us)
  const int64_t target = mp_batch_env(2) > 0 ? mp_batch_env(2) : (mt == 1 && nt == 1 ? 2048 : 1024);
  const int64_t wgs = groups * parts;
  int split = 1;
  while (split < smax && wgs * split < target && nsteps / (split * 2) >= 1) split *= 2;
  if (mp_batch_env(1) > 0) split = mp_batch_env(1) < smax ? mp_batch_env(1) : smax;
  const dim3 grid(static_cast<unsigned>(parts > 1 ? mp_cdiv(groups, 8) * 8 * parts : groups));
  const int hv = parts;
#define MP_W4_BATCH(MT_, NT_, S_)                                                                            \
do {                                                                                                       \
  if (zp && (xdb || MT_ != 1))                                                                             \
    hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, true, false, true, BF>), grid, dim3(S_ * 64), 0, s, xp, \
                       mi, ki, wp, ni, sp, zp, n_groups_i, bp, yp, hv);                                    \
  else if (xdb || MT_ != 1)                                                                                \
    hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, false, false, true, BF>), grid, dim3(S_ * 64), 0, s, xp, \
                       mi, ki, wp, ni, sp, zp, n_groups_i, bp, yp, hv);                                    \
  else if (zp)                                                                                             \
    hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, true, false, false, BF>), grid, dim3(S_ * 64), 0, s, xp, \
                       mi, ki, wp, ni, sp, zp, n_groups_i, bp, yp, hv);                                    \
  else                                                                                                     \
    hipLaunchKernelGGL((w4a16_batch_kernel<MT_, NT_, S_, false, false, false, BF>), grid, dim3(S_ * 64), 0, s, xp, \
                       mi, ki, wp, ni, sp, zp, n_groups_i, bp, yp, hv);                                    \
} while (0)
#define MP_W4_BATCH_S(MT_, NT_)                    \
do {                                             \
  if (split == 1) MP_W4_BATCH(MT_, NT_, 1);      \
  else if (split == 2) MP_W4_BATCH(MT_, NT_, 2); \
  else if (split == 4) MP_W4_BATCH(MT_, NT_, 4); \
  else if (split == 8 || MT_ * NT_ > 1) MP_W4_BATCH(MT_, NT_, (MT_ * NT_ >= 8 ? 4 : 8)); \
  else MP_W4_BATCH(MT_, NT_, (MT_ * NT_ >= 8 ? 4 : (MT_ * NT_ > 1 ? 8 : 16))); \
} while (0)
  if (mt == 1) {
    if (nt == 1) MP_W4_BATCH_S(1, 1);
    else if (nt == 2) MP_W4_BATCH_S(1, 2);
    else MP_W4_BATCH_S(1, 4);
  } else if (mt == 2) {
    if (nt == 1) MP_W4_BATCH_S(2, 1);
    else if (nt == 2) MP_W4_BATCH_S(2, 2);
    else MP_W4_BATCH_S(2, 4);
  } else if constexpr (!BF) {  // the bf16 form takes 16- and 32-row parts only
    if (nt == 1) MP_W4_BATCH_S(4, 1);
    else if (nt == 2) MP_W4_BATCH_S(4, 2);
    else MP_W4_BATCH_S(4, 4);
  }
#undef MP_W4_BATCH_S
#undef MP_W4_BATCH
}

extern "C" int mp_w4a16_gemm(const void *x, int64_t m, int64_t k, const int32_t *w_packed, int64_t n,
                             const void *scales, const void *zeros, int group_size, const void *bias,
                             void *y, int x_dtype, mp_stream_t stream) {
  if (x_dtype != MP_F16 && x_dtype != MP_BF16) return MP_ERR_DTYPE;
  if (m < 0 || n <= 0 || k <= 0 || group_size <= 0 || k % group_size != 0 || k % 8 != 0)
    return MP_ERR_SHAPE;
  if (m == 0) return MP_OK;
  if (!x || !w_packed || !scales || !y) return MP_ERR_ARG;
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return MP_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == MP_BF16) {
    // bf16: every dequantised weight rounded to bf16 as the reference's pseudo-quantized
    // weight is (bf16 keeps 8 significant bits: factoring the group scale out of the sum, as
    // the fp16 streaming kernels do, would miss the reference by ~1e-3).  Group 128: the batched
    // kernel's bf16 form for 2 to 64 rows and the mid-M shapes it takes (mp_batch_takes; activation
    // loads shared by column tiles; K % 256 == 0, an even group count), the matrix-core small-M kernel
    // for one row and the other shapes of up to 16 rows, the prefill kernel's bf16 form above 64 rows
    // (K % 64 == 0, group % 32 == 0); otherwise the dequantising GEMM.
    if (m > mp_bf16_batch_min_m() && mp_batch_takes(m, n) && mp_bf16_small() && k % 256 == 0 && group_size == 128 &&
        ((k / 128) % 2) == 0 &&
        mp_aligned(x, 16) && mp_aligned(w_packed, 16) && mp_aligned(scales, 4) &&
        (zeros == nullptr || mp_aligned(zeros, 4)) && n * (k / 2) < (int64_t(1) << 32) &&
        m * k * 2 < (int64_t(1) << 32)) {
      mp_launch_w4_batch<true>(s, static_cast<const uint16_t *>(x), m, k, reinterpret_cast<const uint32_t *>(w_packed),
                               n, static_cast<const uint16_t *>(scales), static_cast<const uint16_t *>(zeros),
                               static_cast<int>(k / group_size), static_cast<const uint16_t *>(bias),
                               static_cast<uint16_t *>(y));
      MP_CHECK_LAUNCH();
      return MP_OK;
    }
    if (m <= 16 && group_size == 128 && k % 128 == 0 && mp_bf16_small() && mp_aligned(x, 16) &&
        mp_aligned(w_packed, 16) && mp_aligned(scales, 2) && (zeros == nullptr || mp_aligned(zeros, 2)) &&
        (bias == nullptr || mp_aligned(bias, 2))) {
      const int64_t blocks = mp_cdiv(n, 16);
      const int ng = static_cast<int>(k / 128);
      const int w = mp_bf16_small_waves(blocks, ng);
      const int gpw = (ng + w - 1) / w;
      const size_t lds = mp_bf16_small_lds_for(w, gpw, m == 1);
      if (lds <= kBf16SmallLds) {
        const auto *xp = static_cast<const uint16_t *>(x);
        const auto *wp = reinterpret_cast<const uint32_t *>(w_packed);
        const auto *sp = static_cast<const uint16_t *>(scales);
        const auto *zp = static_cast<const uint16_t *>(zeros);
        const auto *bp = static_cast<const uint16_t *>(bias);
        auto *yp = static_cast<uint16_t *>(y);
        const bool one = m == 1;
        const int mi = static_cast<int>(m), ki = static_cast<int>(k), ni = static_cast<int>(n);
        int rc = MP_ERR_ARG;
#define MP_W4_BF16_W(W_)                                                                                        \
  do {                                                                                                          \
    if (one) rc = zp ? mp_bf16_small_launch<W_, true, true>(blocks, lds, s, xp, mi, ki, wp, ni, sp, zp, ng, gpw, bp, yp) \
                     : mp_bf16_small_launch<W_, true, false>(blocks, lds, s, xp, mi, ki, wp, ni, sp, zp, ng, gpw, bp, yp); \
    else rc = zp ? mp_bf16_small_launch<W_, false, true>(blocks, lds, s, xp, mi, ki, wp, ni, sp, zp, ng, gpw, bp, yp) \
                 : mp_bf16_small_launch<W_, false, false>(blocks, lds, s, xp, mi, ki, wp, ni, sp, zp, ng, gpw, bp, yp); \
  } while (0)
        if (w == 1) MP_W4_BF16_W(1);
        else if (w == 2) MP_W4_BF16_W(2);
        else if (w == 4) MP_W4_BF16_W(4);
        else if (w == 8) MP_W4_BF16_W(8);
        else MP_W4_BF16_W(16);
#undef MP_W4_BF16_W
        return rc;
      }
    }
    // above 64 rows: the prefill kernel's bf16 form
    if (m > 64 && k % kPBK == 0 && group_size % 32 == 0 && mp_aligned(x, 16) && mp_aligned(w_packed, 16) &&
        mp_aligned(scales, 2) && (zeros == nullptr || mp_aligned(zeros, 2)) && m * k * 2 < (int64_t(1) << 31) &&
        m * n * 2 < (int64_t(1) << 31) && n <= INT32_MAX && k <= INT32_MAX) {
      const auto *xp = static_cast<const uint16_t *>(x);
      const auto *wp = reinterpret_cast<const uint32_t *>(w_packed);
      const auto *sp = static_cast<const uint16_t *>(scales);
      const auto *zp = static_cast<const uint16_t *>(zeros);
      const auto *bp = static_cast<const uint16_t *>(bias);
      auto *yp = static_cast<uint16_t *>(y);
      const int ng = static_cast<int>(k / group_size);
      if (m >= 256) {
        const dim3 grid(static_cast<unsigned>(mp_cdiv(n, kPBN)), static_cast<unsigned>(mp_cdiv(m, 256)));
        hipLaunchKernelGGL((w4a16_prefill_kernel<kPrefillStages - 1, 512, true>), grid, dim3(512), 0, s, xp,
                           static_cast<int>(m), static_cast<int>(k), wp, static_cast<int>(n), sp, zp, ng, group_size,
                           bp, yp);
      } else {
        const dim3 grid(static_cast<unsigned>(mp_cdiv(n, kPBN)), static_cast<unsigned>(mp_cdiv(m, kPBM)));
        hipLaunchKernelGGL((w4a16_prefill_kernel<kPrefillStages - 1, 256, true>), grid, dim3(256), 0, s, xp,
                           static_cast<int>(m), static_cast<int>(k), wp, static_cast<int>(n), sp, zp, ng, group_size,
                           bp, yp);
      }
      MP_CHECK_LAUNCH();
      return MP_OK;
    }
    mp_dq_args a{};
    a.dt = MP_BF16;
    a.a = x;
    a.a_fmt = MP_DQ_DT;
    a.b = w_packed;
    a.b_fmt = MP_DQ_U4GRP;
    a.b_gscale = static_cast<const uint16_t *>(scales);
    a.b_gzero = static_cast<const uint16_t *>(zeros);
    a.group = group_size;
    a.bias = bias;
    a.bias_dtype = MP_BF16;
    a.y = y;
    a.out_dtype = MP_BF16;
    a.ldy = n;
    a.rows = m;
    a.n = n;
    a.k = k;
    return mp_launch_dq_gemm(a, MP_EPI_DENSE, s);
  }
  const int n_groups = static_cast<int>(k / group_size);
  const auto *xp = static_cast<const uint16_t *>(x);
  const auto *wp = reinterpret_cast<const uint32_t *>(w_packed);
  const auto *sp = static_cast<const uint16_t *>(scales);
  const auto *zp = static_cast<const uint16_t *>(zeros);
  const auto *bp = static_cast<const uint16_t *>(bias);
  auto *yp = static_cast<uint16_t *>(y);
  const bool aligned = mp_aligned(x, 16) && mp_aligned(w_packed, 16) && mp_aligned(scales, 4) &&
                       (zeros == nullptr || mp_aligned(zeros, 4));
  const int n_groups_i = n_groups;
  const int batch_min_m = mp_batch_min_m();
  // batched kernel for every N (MP_W4_BATCH_ALWAYS=0: the LDS-staged kernel for
  // N > 16384 below 32 rows, for measurements)
  const bool batch_shape = m >= 32 || n <= 16384 || mp_batch_env(3);
  // matrix-core GEMV at K = 2048 and 4096 (W = 4, 8 waves of 512-wide slices); measured against the
  // VALU GEMV on the 7B / 70B layer shapes: 4.24 vs 4.74 us at N = K = 4096, 11.3 vs 11.6 us at
  // N = 22016, 2.98 vs 3.24 us at N = K = 2048, but 26.5 vs 24.9 us at K = 8192, N = 28672 (with
  // 8 or 16 waves), where the VALU GEMV's contiguous 2048-wide row chunks stream faster
  const int mfma_slices = (k == 2048 || k == 4096) ? static_cast<int>(k / 512) : 0;
  const bool mfma_gemv = m == 1 && mp_gemv_env(0) == 0 && mp_gemv_mfma() && group_size == 128 &&
                         mfma_slices != 0 && mp_aligned(x, 16) &&
                         mp_aligned(w_packed, 16) && mp_aligned(scales, 8) && (zeros == nullptr || mp_aligned(zeros, 8));
  if (mfma_gemv) {
    const int ki = static_cast<int>(k), ni = static_cast<int>(n);
    const dim3 grid(static_cast<unsigned>(mp_cdiv(n, 16)));
#define MP_W4_GEMV_MFMA(W_, NSL_)                                                                          \
  do {                                                                                                     \
    if (zp)                                                                                                \
      hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<W_, NSL_, true>), grid, dim3(W_ * 64), 0, s, xp, ki, wp, ni, \
                         sp, zp, n_groups_i, bp, yp);                                                       \
    else                                                                                                   \
      hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<W_, NSL_, false>), grid, dim3(W_ * 64), 0, s, xp, ki, wp,   \
                         ni, sp, zp, n_groups_i, bp, yp);                                                   \
  } while (0)
    if (mfma_slices == 4) MP_W4_GEMV_MFMA(4, 1);
    else MP_W4_GEMV_MFMA(8, 1);
#undef MP_W4_GEMV_MFMA
  } else if (m == 1 && mp_gemv_env(0) == 0 && group_size == 128 && (n_groups_i % 2) == 0 && aligned) {
    const int ki = static_cast<int>(k), ni = static_cast<int>(n);
    const int nch = (ki + 2047) / 2048;  // 2048-wide K chunks
    // measured on the 7B / 70B layer shapes: all chunks up front for short K, two waves
    // splitting K when the chunk count is a multiple of 4 or the rows alone give under
    // 2048 waves, else one chunk per iteration
    int r = 4, c = 1, sk = 1;
    if (nch <= 2) {
      c = nch;
    } else if (n >= 16384 && nch % 2 == 0) {
      // wide layers (the 70B gate/up, down and LM head): 8 rows per wave, two waves splitting K,
      // two chunks per iteration: 26.8 / 44.2 / 27.8 us against 27.8 / 47.2 / 29.0 us with the
      // 4-row forms at K = 8192, N = 28672 / 57344 and K = 28672, N = 8192 (graph-timed, 8 rotated
      // copies, one box)
      r = 8;
      c = 2;
      sk = 2;
    } else if (nch % 4 == 0) {
      c = 2;
      sk = 2;
    } else if (nch % 2 == 0 && mp_cdiv(n, 4) < 2048) {
      sk = 2;
    }
    if (mp_gemv_env(1) > 0) r = mp_gemv_env(1) >= 8 ? 8 : (mp_gemv_env(1) >= 4 ? 4 : 2);
    if (mp_gemv_env(2) > 0) c = mp_gemv_env(2) >= 4 ? 4 : mp_gemv_env(2);
    if (mp_gemv_env(3) > 0) sk = mp_gemv_env(3) >= 4 ? 4 : mp_gemv_env(3);
    const int64_t groups = mp_cdiv(n, r);
    const dim3 grid(static_cast<unsigned>(mp_cdiv(groups, 4 / sk)));
#define MP_W4_GEMV(R_, C_, S_)                                                                               \
  do {                                                                                                       \
    if (zp)                                                                                                  \
      hipLaunchKernelGGL((w4a16_gemv_kernel<R_, C_, S_, true>), grid, dim3(256), 0, s, xp, ki, wp, ni, sp,  \
                         zp, n_groups_i, bp, yp, MpRowNorm{});                                               \
    else                                                                                                     \
      hipLaunchKernelGGL((w4a16_gemv_kernel<R_, C_, S_, false>), grid, dim3(256), 0, s, xp, ki, wp, ni, sp, \
                         zp, n_groups_i, bp, yp, MpRowNorm{});                                               \
  } while (0)
#define MP_W4_GEMV_C(R_, S_)           \
  do {                                 \
    if (c == 1) MP_W4_GEMV(R_, 1, S_); \
    else if (c == 2) MP_W4_GEMV(R_, 2, S_); \
    else MP_W4_GEMV(R_, 4, S_);        \
  } while (0)
#define MP_W4_GEMV_S(R_)               \
  do {                                 \
    if (sk == 1) MP_W4_GEMV_C(R_, 1);  \
    else if (sk == 2) MP_W4_GEMV_C(R_, 2); \
    else MP_W4_GEMV_C(R_, 4);          \
  } while (0)
    if (r == 2) MP_W4_GEMV_S(2);
    else if (r == 4) MP_W4_GEMV_S(4);
    else MP_W4_GEMV_S(8);
#undef MP_W4_GEMV_S
#undef MP_W4_GEMV_C
#undef MP_W4_GEMV
  } else if (m > batch_min_m && batch_shape && mp_batch_takes(m, n) && k % 256 == 0 && group_size == 128 && (n_groups_i % 2) == 0 &&
      aligned && n * (k / 2) < (int64_t(1) << 32) && m * k * 2 < (int64_t(1) << 32)) {
    mp_launch_w4_batch<false>(s, xp, m, k, wp, n, sp, zp, n_groups_i, bp, yp);
  } else if (m <= 64 && k % 256 == 0 && group_size == 128 && (n_groups_i % 2) == 0 && aligned) {
    const int mi = static_cast<int>(m), ki = static_cast<int>(k), ni = static_cast<int>(n);
    const int nblk = ki / 128;
    const int mt = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int cb_x = kDecXPieces * 512 / (16 * mi);  // blocks whose activations fit the staging registers
    const bool sz16 = (n_groups_i % 8) == 0 && cb_x >= 8 && mp_aligned(scales, 16) &&
                      (zeros == nullptr || mp_aligned(zeros, 16));
    const int gpp = sz16 ? 8 : 2;
    // waves sharing a 16-column tile: aim for ~2048 streaming waves, >= 4 blocks each
    const int64_t tiles = mp_cdiv(n, 16);
    int split = 1;
    while (split < 8 && tiles * split < 2048 && nblk / (split * 2) >= 4) split *= 2;
    const int t_per_wg = 8 / split;
    // chunk: as many blocks as fit the LDS budget, a multiple of the scale piece
    const int per_block = mi * 260 + t_per_wg * 16 * 4;
    int cb = (kMpXLdsBudget - 64) / per_block;
    const int cb_s = kDecSPieces * 512 * gpp / (t_per_wg * 16);            // scale pieces per thread
    cb = cb < cb_x ? cb : cb_x;
    cb = cb < cb_s ? cb : cb_s;
    cb = cb / gpp * gpp;
    cb = cb < gpp ? gpp : cb;
    cb = cb > nblk ? nblk : cb;
    const size_t smem_x = static_cast<size_t>(DecodeLds(mi, cb, t_per_wg).bytes);
    const size_t red = split > 1 ? static_cast<size_t>(8) * mt * 1024 : 0;
    const size_t smem = smem_x > red ? smem_x : red;
    const dim3 grid(static_cast<unsigned>(mp_cdiv(tiles, t_per_wg)));
#define MP_W4_DEC(MT_, S_, SZ_)                                                                             \
  do {                                                                                                      \
    if (zp)                                                                                                 \
      hipLaunchKernelGGL((w4a16_decode_kernel<MT_, S_, true, SZ_>), grid, dim3(512), smem, s, xp, mi, ki, wp, \
                         ni, sp, zp, n_groups_i, bp, yp, cb);                                               \
    else                                                                                                    \
      hipLaunchKernelGGL((w4a16_decode_kernel<MT_, S_, false, SZ_>), grid, dim3(512), smem, s, xp, mi, ki, wp, \
                         ni, sp, zp, n_groups_i, bp, yp, cb);                                               \
  } while (0)
#define MP_W4_DEC_S(MT_, SZ_)                 \
  do {                                        \
    if (split == 1) MP_W4_DEC(MT_, 1, SZ_);      \
    else if (split == 2) MP_W4_DEC(MT_, 2, SZ_); \
    else if (split == 4) MP_W4_DEC(MT_, 4, SZ_); \
    else MP_W4_DEC(MT_, 8, SZ_);                 \
  } while (0)
    if (sz16) {
      if (mt == 1) MP_W4_DEC_S(1, true);
      else if (mt == 2) MP_W4_DEC_S(2, true);
      else MP_W4_DEC_S(4, true);
    } else {
      if (mt == 1) MP_W4_DEC_S(1, false);
      else if (mt == 2) MP_W4_DEC_S(2, false);
      else MP_W4_DEC_S(4, false);
    }
#undef MP_W4_DEC_S
#undef MP_W4_DEC
  } else if (m > 64 && k % kPBK == 0 && group_size % 32 == 0 && aligned && m * k * 2 < (int64_t(1) << 31) &&
             m * n * 2 < (int64_t(1) << 31)) {
    if (mp_prefill_threads() == 512 && m >= 256) {
      const dim3 grid(static_cast<unsigned>(mp_cdiv(n, kPBN)), static_cast<unsigned>(mp_cdiv(m, 256)));
#define MP_W4_PF512(D_)                                                                                      \
  hipLaunchKernelGGL((w4a16_prefill_kernel<D_, 512>), grid, dim3(512), 0, s, xp, static_cast<int>(m),         \
                     static_cast<int>(k), wp, static_cast<int>(n), sp, zp, n_groups, group_size, bp, yp)
      const int st = mp_knob("MP_W4_PREFILL_STAGES") ? atoi(mp_knob("MP_W4_PREFILL_STAGES")) : kPrefillStages;
      if (st == 2) MP_W4_PF512(1);
      else if (st == 3) MP_W4_PF512(2);
      else if (st == 5) MP_W4_PF512(4);
      else MP_W4_PF512(kPrefillStages - 1);
#undef MP_W4_PF512
    } else {
      const dim3 grid(static_cast<unsigned>(mp_cdiv(n, kPBN)), static_cast<unsigned>(mp_cdiv(m, kPBM)));
      hipLaunchKernelGGL(w4a16_prefill_kernel<kPrefillStages - 1>, grid, dim3(256), 0, s, xp, static_cast<int>(m),
                         static_cast<int>(k), wp, static_cast<int>(n), sp, zp, n_groups, group_size, bp, yp);
    }
  } else {
    hipLaunchKernelGGL(w4a16_simple_kernel, dim3(static_cast<unsigned>(mp_cdiv(m * n, 256))), dim3(256), 0, s,
                       xp, m, k, wp, n, mp_cdiv(k, 8), sp, zp, n_groups, group_size, bp, yp);
  }
  MP_CHECK_LAUNCH();
  return MP_OK;
}
