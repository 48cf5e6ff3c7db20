// Decode-step kernels of the Llama-shaped measurement harness around the
// quantized linears: RoPE + KV-cache append, split-K decode attention (flash
// decoding) with its split merge (optionally with the RoPE and the append
// fused into the attention launch), and SiLU-multiply.  The reference has no
// counterpart (attention belongs to vLLM's backend); these exist so that one
// greedy decode step runs as 6-8 launches per layer and the W4A16 GEMVs, not
// launch gaps, set the step time.
//
// Shapes: head dim 128; q/k/v heads packed as one qkv row [B, (nh + 2 kvh) * 128]
// (the fused qkv W4A16 output); KV cache per layer K, V [B, kvh, T, 128] fp16
// (one 256-byte row per position).  The current position is read from device
// memory, so every launch has a fixed shape and a step can be graph-captured.
#include <climits>

#include "mp_common.h"

namespace {

constexpr int kHd = 128;
constexpr int kMergeMaxSplits = 1024;  // splits per head the merge kernel takes

// ---------------------------------------------------------------- RoPE + append
// One wave per (row b, head); lane i owns the interleaved pair (2i, 2i+1).
// Rounding follows PyTorch half ops: every product and the sum round to fp16.
__global__ __launch_bounds__(256) void rope_append_kernel(
    const uint16_t *__restrict__ qkv, int nh, int kvh, const uint16_t *__restrict__ cos_t,
    const uint16_t *__restrict__ sin_t, const int64_t *__restrict__ pos_p, int cap, uint16_t *__restrict__ q_out,
    uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache, int total_heads) {
  // no contraction: the compiler narrows these to fp16 ops and would fuse a product
  // into the subtraction (v_fma_f16), skipping the product's own rounding
#pragma clang fp contract(off)
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gw >= total_heads) return;  // wave-uniform, no barrier in the kernel
  const int lane = threadIdx.x & 63;
  const int heads = nh + 2 * kvh;
  const int b = gw / heads, h = gw % heads;
  const int64_t pos = pos_p[0];
  if (pos < 0 || pos >= cap) return;  // a position outside the cache writes nothing
  const uint32_t x2 = reinterpret_cast<const uint32_t *>(qkv + (static_cast<int64_t>(b) * heads + h) * kHd)[lane];
  if (h >= nh + kvh) {  // v: plain copy into the cache
    const int kh = h - nh - kvh;
    reinterpret_cast<uint32_t *>(v_cache + ((static_cast<int64_t>(b) * kvh + kh) * cap + pos) * kHd)[lane] = x2;
    return;
  }
  const float x1 = mp_h2f(static_cast<uint16_t>(x2)), xb = mp_h2f(static_cast<uint16_t>(x2 >> 16));
  const float c = mp_h2f(cos_t[pos * (kHd / 2) + lane]), s = mp_h2f(sin_t[pos * (kHd / 2) + lane]);
  const float o0 = mp_rh(mp_rh(x1 * c) - mp_rh(xb * s));
  const float o1 = mp_rh(mp_rh(x1 * s) + mp_rh(xb * c));
  const uint32_t o = static_cast<uint32_t>(mp_f2h(o0)) | (static_cast<uint32_t>(mp_f2h(o1)) << 16);
  if (h < nh) {
    reinterpret_cast<uint32_t *>(q_out + (static_cast<int64_t>(b) * nh + h) * kHd)[lane] = o;
  } else {
    const int kh = h - nh;
    reinterpret_cast<uint32_t *>(k_cache + ((static_cast<int64_t>(b) * kvh + kh) * cap + pos) * kHd)[lane] = o;
  }
}

// ---------------------------------------------------------------- decode attention
// Interleaved-pair RoPE of 8 consecutive dims (pairs 4 dl .. 4 dl + 3) given the
// four cos / sin values of those pairs, rounding like PyTorch half ops (every product
// and the sum round to fp16).
__device__ __forceinline__ void rope8(const uint4 xv, const uint2 cv, const uint2 sv, float (&o)[8]) {
  // no contraction: the compiler narrows these to fp16 ops and would fuse a product
  // into the subtraction (v_fma_f16), skipping the product's own rounding
#pragma clang fp contract(off)
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
  const uint32_t cw[2] = {cv.x, cv.y}, sw[2] = {sv.x, sv.y};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x1 = mp_h2f(static_cast<uint16_t>(xw[j])), xb = mp_h2f(static_cast<uint16_t>(xw[j] >> 16));
    const float c = mp_h2f(static_cast<uint16_t>(cw[j >> 1] >> (16 * (j & 1))));
    const float s = mp_h2f(static_cast<uint16_t>(sw[j >> 1] >> (16 * (j & 1))));
    o[2 * j] = mp_rh(mp_rh(x1 * c) - mp_rh(xb * s));
    o[2 * j + 1] = mp_rh(mp_rh(x1 * s) + mp_rh(xb * c));
  }
}

// Sum over each row of 16 lanes with DPP adds (full-rate VALU; __shfl_xor lowers to
// ds_bpermute chains): pairs (quad_perm 1,0,3,2), quads (2,3,0,1), then half-rows
// (row_half_mirror) and rows (row_mirror).  Every lane of the row gets the same value:
// each stage adds two equal partial sums in either order.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
  return fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF,
                                                                        false)));
}
// wave-wide max / sum: the 16-lane DPP stages, then the four rows (lanes l ^ 16, l ^ 32)
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = dpp_max<0xB1>(v);
  v = dpp_max<0x4E>(v);
  v = dpp_max<0x141>(v);
  v = dpp_max<0x140>(v);
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float dpp_sum16(float v);
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_sum16(v);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float dpp_sum16(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  return v;
}

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void h8_to_f32(const uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = mp_h2f(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
}

// Grid (splits, B * kvh), 256 threads.  A workgroup scores positions
// [s*chunk, min((s+1)*chunk, len)) for the GRP query heads of one kv head:
// 16 lanes per position (8 dims each, one 16-byte load), 4 positions per wave
// per step of 16, U steps per load round, fp32 dot products reduced over the 16
// lanes.  Scores go to LDS, softmax statistics are taken over the workgroup,
// then P.V accumulates in fp32 with the same lane layout.
//
// Memory round trips set the time of a short chunk, so the loads go out in this
// order before any of them is waited for: the query slices (and, with ROPE, the
// new key / value slices and their cos / sin), then the first K round, then the
// first V round.  With U * 16 >= chunk the whole chunk is one round.
//
// ROPE: the queries come from the fused qkv row [B, (nh + 2 kvh) * 128] and are
// rotated in registers.  The workgroup whose split holds position pos (the last
// used one) appends the rotated key and the value to the cache; its own use of
// that position takes the rows from registers, so no load has to see the append.
// len = pos + 1; a position outside [0, cap) appends nothing and yields zeros.
// Otherwise q is [B, nh, 128] and len = clamp(pos + 1, 0, cap).
//
// With one split the workgroup normalises and stores the output; otherwise it
// stores its unnormalised partial o, max m and sum l for attn_merge_kernel.
template <int GRP, bool ROPE, int U>
__global__ __launch_bounds__(256) void decode_attn_kernel(
    const uint16_t *__restrict__ qsrc, const uint16_t *__restrict__ cos_t, const uint16_t *__restrict__ sin_t,
    uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache, const int64_t *__restrict__ pos_p, int kvh,
    int cap, int chunk, int splits, float scale, float *__restrict__ part_o, float *__restrict__ part_ml,
    uint16_t *__restrict__ out) {
  constexpr uint32_t kOob = 0x80000000u;  // past the cache descriptors (host: cap * 256 < 2^31)
  extern __shared__ float sm[];  // [GRP][chunk] scores, then the [GRP][4][128] reduction
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x;
  const int bk = blockIdx.y;  // b * kvh + kh
  const int nh = kvh * GRP;
  const int b = bk / kvh, kh = bk % kvh;
  const int64_t pos = pos_p[0];
  int len;
  if (ROPE) {
    len = (pos < 0 || pos >= cap) ? 0 : static_cast<int>(pos) + 1;
  } else {
    const int64_t p1 = pos + 1;
    len = static_cast<int>(p1 < 0 ? 0 : (p1 > cap ? cap : p1));
  }
  const int t0 = s * chunk;
  if (t0 >= len) {  // workgroup-uniform, before any barrier
    if (len == 0 && s == 0 && splits == 1)  // (with splits the merge writes the zeros)
      for (int i = tid; i < GRP * kHd; i += 256)
        out[(static_cast<int64_t>(b) * nh + kh * GRP) * kHd + i] = 0;
    return;
  }
  const int used = (len + chunk - 1) / chunk;  // <= splits: the host sizes chunk * splits >= cap
  const int t1 = min(t0 + chunk, len);
  const int n = t1 - t0;
  const int dl = lane & 15;  // 8-dim slice of this lane
  const int pl = lane >> 4;  // position within the wave's group of 4
  const uint16_t *kbase = k_cache + static_cast<int64_t>(bk) * cap * kHd + dl * 8;
  const uint16_t *vbase = v_cache + static_cast<int64_t>(bk) * cap * kHd + dl * 8;
  // the appending workgroup: its last position (n - 1) is the new token's
  const bool app = ROPE && s == used - 1;
  auto tpos = [&](int base, int u) { return base + u * 16 + wave * 4 + pl; };  // unclamped

  // ---- loads: query (+ new key / value) slices, then the first K and V rounds
  auto load_round = [&](uint4 (&r)[U], const uint16_t *base_p, int base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = min(tpos(base, u), n - 1);
      r[u] = *reinterpret_cast<const uint4 *>(base_p + static_cast<int64_t>(t0 + t) * kHd);
    }
  };
  // the row a lane uses for (clamped) position t: the new token's from registers
  auto pick = [&](const uint4 cached, const uint4 fresh, int t) {
    return (app && min(t, n - 1) == n - 1) ? fresh : cached;
  };
  const uint32_t cbytes = static_cast<uint32_t>(cap) * kHd * 2;
  const auto krs = mp_rsrc(k_cache + static_cast<int64_t>(bk) * cap * kHd, cbytes);
  const auto vrs = mp_rsrc(v_cache + static_cast<int64_t>(bk) * cap * kHd, cbytes);
  const uint16_t *qkv_row = qsrc + static_cast<int64_t>(b) * (nh + 2 * kvh) * kHd;  // ROPE
  float *sc = sm;
  uint4 vv[U], vnv = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (GRP >= 4) {
    // ---- scores on MFMA (f32_16x16x16_f16): D[t][g] = K[t] . Q[g] for 16 positions of the
    // wave x 16 head slots (GRP used).  Lane l: position / head slot tl = l % 16 and the dims
    // [32 q4, +32), q4 = l / 16; MFMA j takes dims 32 q4 + 4 j + [0, 4) of both operands (one
    // permutation of the reduction index).  D: lane l holds positions 4 q4 + i of head tl.
    const int q4 = lane >> 4, tl = lane & 15;
    const int gq = tl < GRP ? tl : GRP - 1;
    uint4 q32[4], k32[4];
    uint2 c32[4], s32[4];
    if (ROPE) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        q32[c] = *reinterpret_cast<const uint4 *>(qkv_row + (kh * GRP + gq) * kHd + q4 * 32 + c * 8);
        k32[c] = *reinterpret_cast<const uint4 *>(qkv_row + (nh + kh) * kHd + q4 * 32 + c * 8);
        c32[c] = *reinterpret_cast<const uint2 *>(cos_t + pos * (kHd / 2) + (4 * q4 + c) * 4);
        s32[c] = *reinterpret_cast<const uint2 *>(sin_t + pos * (kHd / 2) + (4 * q4 + c) * 4);
      }
      vnv = *reinterpret_cast<const uint4 *>(qkv_row + (nh + kvh + kh) * kHd + dl * 8);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        q32[c] = *reinterpret_cast<const uint4 *>(qsrc + (static_cast<int64_t>(b) * nh + kh * GRP + gq) * kHd +
                                                  q4 * 32 + c * 8);
    }
    const uint16_t *kb32 = k_cache + static_cast<int64_t>(bk) * cap * kHd + q4 * 32;
    auto load_k = [&](uint4 (&r)[4], int base) {
      const int t = min(base + 16 * wave + tl, n - 1);
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] = *reinterpret_cast<const uint4 *>(kb32 + static_cast<int64_t>(t0 + t) * kHd + c * 8);
    };
    uint4 kc[4];
    load_k(kc, 0);
    load_round(vv, vbase, 0);
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the rotation waits

    // operands: rotated (ROPE) queries of head slot tl, zero for the unused slots
    h4_t qb[8];
    uint4 knew32[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (ROPE) {
        float f[8], kr[8];
        rope8(q32[c], c32[c], s32[c], f);
        rope8(k32[c], c32[c], s32[c], kr);
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = static_cast<uint32_t>(mp_f2h(kr[2 * j])) | (static_cast<uint32_t>(mp_f2h(kr[2 * j + 1])) << 16);
        knew32[c] = make_uint4(w[0], w[1], w[2], w[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qb[2 * c][e] = static_cast<_Float16>(f[e]);
          qb[2 * c + 1][e] = static_cast<_Float16>(f[4 + e]);
        }
      } else {
        knew32[c] = make_uint4(0u, 0u, 0u, 0u);
        qb[2 * c] = __builtin_bit_cast(h4_t, make_uint2(q32[c].x, q32[c].y));
        qb[2 * c + 1] = __builtin_bit_cast(h4_t, make_uint2(q32[c].z, q32[c].w));
      }
      const h4_t zero = {0, 0, 0, 0};
      qb[2 * c] = tl < GRP ? qb[2 * c] : zero;
      qb[2 * c + 1] = tl < GRP ? qb[2 * c + 1] : zero;
    }
    if (ROPE) {  // append: the key from wave 0's lanes with tl == 0, the value from lanes 16-31
#pragma unroll
      for (int c = 0; c < 4; ++c)
        mp_buf_store16(krs, app && tid < 64 && tl == 0 ? (static_cast<uint32_t>(pos) * kHd + q4 * 32 + c * 8) * 2 : kOob,
                       knew32[c]);
      mp_buf_store16(vrs, app && tid >= 16 && tid < 32 ? (static_cast<uint32_t>(pos) * kHd + dl * 8) * 2 : kOob,
                     vnv);
    }
    // the appending workgroup's last position is scored from the new key after the loop
    auto score_step = [&](const uint4 (&r)[4], int base) {
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 w = r[j >> 1];
        const h4_t a = __builtin_bit_cast(h4_t, (j & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y));
        d = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qb[j], d, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = base + 16 * wave + 4 * q4 + i;
        if (tl < GRP && t < n && !(app && t == n - 1)) sc[tl * chunk + t] = d[i] * scale;
      }
    };
    // two register sets in turn (n >= 1: at least one step); the prefetch past the end
    // re-reads the last row
    uint4 kd[4];
    int base = 0;
    while (true) {
      load_k(kd, base + 64);
      score_step(kc, base);
      base += 64;
      if (base >= n) break;
      load_k(kc, base + 64);
      score_step(kd, base);
      base += 64;
      if (base >= n) break;
    }
    if (app) {  // workgroup-uniform: every row of A is the new key, so D row 0 is its score
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 w = knew32[j >> 1];
        const h4_t a = __builtin_bit_cast(h4_t, (j & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y));
        d = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qb[j], d, 0, 0, 0);
      }
      if (wave == 0 && q4 == 0 && tl < GRP) sc[tl * chunk + n - 1] = d[0] * scale;
    }
  } else {
    uint4 qv[GRP], knv;
    uint2 cv, sv;
    if (ROPE) {
      const uint16_t *row = qkv_row + dl * 8;
#pragma unroll
      for (int g = 0; g < GRP; ++g) qv[g] = *reinterpret_cast<const uint4 *>(row + (kh * GRP + g) * kHd);
      knv = *reinterpret_cast<const uint4 *>(row + (nh + kh) * kHd);
      vnv = *reinterpret_cast<const uint4 *>(row + (nh + kvh + kh) * kHd);
      cv = *reinterpret_cast<const uint2 *>(cos_t + pos * (kHd / 2) + dl * 4);
      sv = *reinterpret_cast<const uint2 *>(sin_t + pos * (kHd / 2) + dl * 4);
    } else {
#pragma unroll
      for (int g = 0; g < GRP; ++g)
        qv[g] = *reinterpret_cast<const uint4 *>(qsrc + (static_cast<int64_t>(b) * nh + kh * GRP + g) * kHd + dl * 8);
    }
    uint4 kv[U];
    load_round(kv, kbase, 0);
    load_round(vv, vbase, 0);

    // queries to fp32; with ROPE rotate, and append the new row (lanes 0-15 the key,
    // 16-31 the value of the appending workgroup; every other store is dropped)
    float qf[GRP][8];
    uint4 knew = make_uint4(0, 0, 0, 0);
    if (ROPE) {
#pragma unroll
      for (int g = 0; g < GRP; ++g) rope8(qv[g], cv, sv, qf[g]);
      float kr[8];
      rope8(knv, cv, sv, kr);
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = static_cast<uint32_t>(mp_f2h(kr[2 * j])) | (static_cast<uint32_t>(mp_f2h(kr[2 * j + 1])) << 16);
      knew = make_uint4(w[0], w[1], w[2], w[3]);
      const uint32_t roff = (static_cast<uint32_t>(pos) * kHd + dl * 8) * 2;
      mp_buf_store16(krs, app && tid < 16 ? roff : kOob, knew);
      mp_buf_store16(vrs, app && tid >= 16 && tid < 32 ? roff : kOob, vnv);
    } else {
#pragma unroll
      for (int g = 0; g < GRP; ++g) h8_to_f32(qv[g], qf[g]);
    }

    // ---- scores on the VALU: 16 lanes per position, DPP sums
    auto score_round = [&](const uint4 (&r)[U], int base) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = tpos(base, u);
        float kf[8];
        h8_to_f32(ROPE ? pick(r[u], knew, t) : r[u], kf);
#pragma unroll
        for (int g = 0; g < GRP; ++g) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qf[g][e], kf[e], d);
          d = dpp_sum16(d);
          if (dl == 0 && t < n) sc[g * chunk + t] = d * scale;
        }
      }
    };
    score_round(kv, 0);
    for (int base = 16 * U; base < n; base += 16 * U) {
      uint4 k2[U];
      load_round(k2, kbase, base);
      score_round(k2, base);
    }
  }
  mp_lds_barrier();

  // ---- softmax statistics per head over the workgroup's positions
  float mx[GRP], sum[GRP];
  if constexpr (GRP >= 4) {
    // one wave per head (heads wave, wave + 4, ...): the statistics need a single barrier
    __shared__ float hstat[GRP][2];
#pragma unroll
    for (int hh = 0; hh < GRP / 4; ++hh) {
      const int g = wave + 4 * hh;
      float m = -INFINITY;
      for (int t = lane; t < n; t += 64) m = fmaxf(m, sc[g * chunk + t]);
      m = wave_max_dpp(m);
      float l = 0.f;
      for (int t = lane; t < n; t += 64) {
        const float p = expf(sc[g * chunk + t] - m);
        sc[g * chunk + t] = p;
        l += p;
      }
      l = wave_sum_dpp(l);
      if (lane == 0) {
        hstat[g][0] = m;
        hstat[g][1] = l;
      }
    }
    mp_lds_barrier();
#pragma unroll
    for (int g = 0; g < GRP; ++g) {
      mx[g] = hstat[g][0];
      sum[g] = hstat[g][1];
    }
  } else {
#pragma unroll
  for (int g = 0; g < GRP; ++g) {
    float m = -INFINITY;
    for (int t = tid; t < n; t += 256) m = fmaxf(m, sc[g * chunk + t]);
    m = mp_wave_max(m);
    if (lane == 0) red[wave] = m;
    mp_lds_barrier();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    mp_lds_barrier();
    float l = 0.f;
    for (int t = tid; t < n; t += 256) {
      const float p = expf(sc[g * chunk + t] - m);
      sc[g * chunk + t] = p;
      l += p;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) red[wave] = l;
    mp_lds_barrier();
    l = (red[0] + red[1]) + (red[2] + red[3]);
    mp_lds_barrier();
    mx[g] = m;
    sum[g] = l;
  }
  }

  // ---- P.V
  float acc[GRP][8];
#pragma unroll
  for (int g = 0; g < GRP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  auto pv_round = [&](const uint4 (&r)[U], int base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tpos(base, u);
      float vf[8];
      h8_to_f32(ROPE ? pick(r[u], vnv, t) : r[u], vf);
#pragma unroll
      for (int g = 0; g < GRP; ++g) {
        const float p = t < n ? sc[g * chunk + t] : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
      }
    }
  };
  pv_round(vv, 0);
  for (int base = 16 * U; base < n; base += 16 * U) {
    uint4 v2[U];
    load_round(v2, vbase, base);
    pv_round(v2, base);
  }
  // reduce over the 4 positions of a wave (lanes l, l^16, l^32, l^48), then over the waves
#pragma unroll
  for (int g = 0; g < GRP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[g][e] += __shfl_xor(acc[g][e], 16, 64);
      acc[g][e] += __shfl_xor(acc[g][e], 32, 64);
    }
  mp_lds_barrier();  // the score buffer is reused for the reduction
  float *rw = sm;    // [GRP][4 waves][128]
  if (pl == 0) {
#pragma unroll
    for (int g = 0; g < GRP; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) rw[(g * 4 + wave) * kHd + dl * 8 + e] = acc[g][e];
  }
  mp_lds_barrier();
  const int64_t head0 = static_cast<int64_t>(b) * nh + kh * GRP;
  if (splits == 1) {  // one split: normalise and store (what the merge computes for one split)
    for (int i = tid; i < GRP * kHd; i += 256) {
      const int g = i / kHd, d = i % kHd;
      const float o = (rw[(g * 4 + 0) * kHd + d] + rw[(g * 4 + 1) * kHd + d]) +
                      (rw[(g * 4 + 2) * kHd + d] + rw[(g * 4 + 3) * kHd + d]);
      out[head0 * kHd + i] = mp_f2h(o / sum[g]);
    }
    return;
  }
  for (int i = tid; i < GRP * kHd; i += 256) {
    const int g = i / kHd, d = i % kHd;
    const float o = (rw[(g * 4 + 0) * kHd + d] + rw[(g * 4 + 1) * kHd + d]) +
                    (rw[(g * 4 + 2) * kHd + d] + rw[(g * 4 + 3) * kHd + d]);
    part_o[((head0 + g) * splits + s) * kHd + d] = o;
    if (d == 0) {
      part_ml[((head0 + g) * splits + s) * 2 + 0] = mx[g];
      part_ml[((head0 + g) * splits + s) * 2 + 1] = sum[g];
    }
  }
}

// Merge of the used splits, one wave per (row, head), four heads per workgroup:
// lanes take the splits' (m, l) pairs for the max and the weights
// w_j = exp(m_j - max m), then each lane owns two dims and sums w_j o_j over the
// splits.  The partial outputs of the first kMergeRound splits are loaded right
// after the (m, l) pairs, before the weights are computed, so one memory round trip
// covers them.  Sums run in a fixed order (ascending j), so the result does not
// depend on timing.  An empty range (len 0) gives zeros.
constexpr int kMergeRound = 32;
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ part_o,
                                                         const float *__restrict__ part_ml,
                                                         const int64_t *__restrict__ pos_p, int cap, int chunk,
                                                         int splits, int rope, int64_t heads,
                                                         uint16_t *__restrict__ out) {
  __shared__ float wts[4][kMergeMaxSplits];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t head = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (head >= heads) return;  // wave-uniform; no barrier below
  const int64_t pos = pos_p[0];
  int len;
  if (rope) {
    len = (pos < 0 || pos >= cap) ? 0 : static_cast<int>(pos) + 1;
  } else {
    const int64_t p1 = pos + 1;
    len = static_cast<int>(p1 < 0 ? 0 : (p1 > cap ? cap : p1));
  }
  const int used = (len + chunk - 1) / chunk;
  uint32_t *o2 = reinterpret_cast<uint32_t *>(out + head * kHd) + lane;
  if (used == 0) {
    *o2 = 0u;
    return;
  }
  const float *ml = part_ml + head * splits * 2;
  const float2 *po = reinterpret_cast<const float2 *>(part_o + head * splits * kHd) + lane;
  // (m, l) of split lane (clamped into the used ones), then the first round of partials
  const float2 ml0 = reinterpret_cast<const float2 *>(ml)[min(lane, used - 1)];
  float2 v[kMergeRound];
#pragma unroll
  for (int u = 0; u < kMergeRound; ++u) v[u] = po[min(u, used - 1) * (kHd / 2)];
  float m = lane < used ? ml0.x : -INFINITY;
  for (int j = lane + 64; j < used; j += 64) m = fmaxf(m, ml[2 * j]);
  m = mp_wave_max(m);
  float den = 0.f;
  if (lane < used) {
    const float w = expf(ml0.x - m);
    wts[wave][lane] = w;
    den = w * ml0.y;  // fmaf(w, l, 0)
  }
  for (int j = lane + 64; j < used; j += 64) {
    const float w = expf(ml[2 * j] - m);
    wts[wave][j] = w;
    den = fmaf(w, ml[2 * j + 1], den);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float n0 = 0.f, n1 = 0.f;
#pragma unroll
  for (int u = 0; u < kMergeRound; ++u)
    if (u < used) {
      n0 = fmaf(wts[wave][u], v[u].x, n0);
      n1 = fmaf(wts[wave][u], v[u].y, n1);
    }
  int j = kMergeRound;
  for (; j + 8 <= used; j += 8) {
    float2 w8[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w8[u] = po[(j + u) * (kHd / 2)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      n0 = fmaf(wts[wave][j + u], w8[u].x, n0);
      n1 = fmaf(wts[wave][j + u], w8[u].y, n1);
    }
  }
  for (; j < used; ++j) {
    const float2 w1 = po[j * (kHd / 2)];
    n0 = fmaf(wts[wave][j], w1.x, n0);
    n1 = fmaf(wts[wave][j], w1.y, n1);
  }
  *o2 = static_cast<uint32_t>(mp_f2h(n0 / den)) | (static_cast<uint32_t>(mp_f2h(n1 / den)) << 16);
}

// ---------------------------------------------------------------- row argmax
// Greedy sampling of the decode step: idx[r] = the first index of the maximum of row r
// of x [rows, n] fp16 (torch.argmax's rules: the lowest index among equal maxima, and a
// NaN counts as the maximum).  One 1024-thread workgroup per row: each thread keeps the
// best (value, index) of a strided slice, then wave and workgroup reductions.
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}
// The row is read in batches whose loads all go out before any comparison (one memory round trip
// per batch, not one per element): VEC, 16-byte chunks of 8 values, 4 per thread per batch (rows
// 16-byte aligned, n % 8 == 0); otherwise 8 scalar loads per thread per batch.  am_better is a total
// order, so the visiting order does not change the result.
template <bool VEC>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const uint16_t *__restrict__ x, int n,
                                                          int64_t *__restrict__ idx) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const uint16_t *row = x + static_cast<int64_t>(blockIdx.x) * n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float bv = -INFINITY;
  int bi = INT_MAX;
  auto take = [&](float v, int i) {
    if (am_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  };
  if (VEC) {
    constexpr int U = 4;
    const int n8 = n >> 3;
    const uint4 *r4 = reinterpret_cast<const uint4 *>(row);
    for (int base = threadIdx.x; base < n8; base += 1024 * U) {
      uint4 c[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * 1024;
        c[u] = j < n8 ? r4[j] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * 1024;
        if (j >= n8) break;
        const uint32_t w[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          take(mp_h2f(static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu))), 8 * j + e);
      }
    }
  } else {
    constexpr int U = 8;
    for (int base = threadIdx.x; base < n; base += 1024 * U) {
      uint16_t c[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * 1024;
        c[u] = j < n ? row[j] : 0;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * 1024;
        if (j >= n) break;
        take(mp_h2f(c[u]), j);
      }
    }
  }
  auto reduce = [&](int width) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      if (o >= width) continue;
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (am_better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
  };
  reduce(64);
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (wave != 0) return;
  bv = lane < 16 ? sv[lane] : -INFINITY;
  bi = lane < 16 ? si[lane] : INT_MAX;
  reduce(16);
  if (lane == 0) idx[blockIdx.x] = bi;
}

// Split form for long rows (the LM head's vocabulary): a workgroup per 4096-value span of a row
// finds the span's best (value, index) and merges it into idx[row] by a 64-bit atomic max of a key
// that orders like am_better: the value's bits mapped to an unsigned order in the high word (NaN
// above everything, -0 as +0), the complement of the index in the low word (equal values: the
// smaller index wins).  idx[row] is cleared first and decoded after (three launches, no workspace).
__device__ __forceinline__ unsigned long long am_key(float v, int i) {
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  u = (v != v) ? 0xFFFFFFFFu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
  return (static_cast<unsigned long long>(u) << 32) | static_cast<uint32_t>(0xFFFFFFFFu - static_cast<uint32_t>(i));
}

__global__ void argmax_clear_kernel(int64_t *__restrict__ idx, int64_t rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r < rows) idx[r] = 0;
}

constexpr int kArgmaxSpan = 4096;

template <bool VEC>
__global__ __launch_bounds__(256) void argmax_span_kernel(const uint16_t *__restrict__ x, int n,
                                                          int64_t *__restrict__ idx) {
  __shared__ unsigned long long sk[4];
  const uint16_t *row = x + static_cast<int64_t>(blockIdx.y) * n;
  const int lo = blockIdx.x * kArgmaxSpan;
  const int hi = lo + kArgmaxSpan < n ? lo + kArgmaxSpan : n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long best = 0;
  if (VEC) {
    // 16 values per thread: two 16-byte chunks, both loaded before any comparison
    constexpr int C = kArgmaxSpan / 8 / 256;
    const uint4 *r4 = reinterpret_cast<const uint4 *>(row);
    uint4 c[C];
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int j = lo / 8 + threadIdx.x + u * 256;
      c[u] = 8 * j < hi ? r4[j] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int j = lo / 8 + threadIdx.x + u * 256;
      if (8 * j >= hi) break;
      const uint32_t w[4] = {c[u].x, c[u].y, c[u].z, c[u].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned long long k =
            am_key(mp_h2f(static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu))), 8 * j + e);
        best = k > best ? k : best;
      }
    }
  } else {
    constexpr int C = kArgmaxSpan / 256;
    uint16_t c[C];
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int j = lo + threadIdx.x + u * 256;
      c[u] = j < hi ? row[j] : 0;
    }
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int j = lo + threadIdx.x + u * 256;
      if (j >= hi) break;
      const unsigned long long k = am_key(mp_h2f(c[u]), j);
      best = k > best ? k : best;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long k = __shfl_xor(best, o, 64);
    best = k > best ? k : best;
  }
  if (lane == 0) sk[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = sk[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) k = sk[w] > k ? sk[w] : k;
    atomicMax(reinterpret_cast<unsigned long long *>(idx + blockIdx.y), k);
  }
}

__global__ void argmax_decode_kernel(int64_t *__restrict__ idx, int64_t rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r < rows) {
    const unsigned long long k = static_cast<unsigned long long>(idx[r]);
    idx[r] = static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(k & 0xFFFFFFFFull));
  }
}

// ---------------------------------------------------------------- SiLU * up
// gu [B, 2I] (gate | up) -> act [B, I] = round(round(silu(gate)) * up).
template <bool BF>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, int inter, int64_t total,
                                                       uint16_t *__restrict__ act) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / inter, c = i % inter;
  const uint16_t g = gu[b * 2 * inter + c], u = gu[b * 2 * inter + inter + c];
  act[i] = BF ? mp_swiglu_bf(mp_bf2f(g), mp_bf2f(u)) : mp_swiglu_h(mp_h2f(g), mp_h2f(u));
}

}  // namespace

extern "C" int mp_decode_rope_append(const void *qkv, int64_t batch, int nh, int kvh, int head_dim,
                                     const void *cos_t, const void *sin_t, const int64_t *pos, int64_t capacity,
                                     void *q_out, void *k_cache, void *v_cache, mp_stream_t stream) {
  if (!qkv || !cos_t || !sin_t || !pos || !q_out || !k_cache || !v_cache) return MP_ERR_ARG;
  if (head_dim != kHd) return MP_ERR_SHAPE;
  if (batch <= 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || capacity <= 0 || capacity > INT32_MAX) return MP_ERR_SHAPE;
  if (!mp_aligned(qkv, 4) || !mp_aligned(q_out, 4) || !mp_aligned(k_cache, 4) || !mp_aligned(v_cache, 4))
    return MP_ERR_ALIGN;
  const int64_t total = batch * (nh + 2 * kvh);
  if (total > INT32_MAX) return MP_ERR_SHAPE;
  hipLaunchKernelGGL(rope_append_kernel, dim3(static_cast<unsigned>(mp_cdiv(total, 4))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(qkv), nh, kvh,
                     static_cast<const uint16_t *>(cos_t), static_cast<const uint16_t *>(sin_t), pos,
                     static_cast<int>(capacity), static_cast<uint16_t *>(q_out), static_cast<uint16_t *>(k_cache),
                     static_cast<uint16_t *>(v_cache), static_cast<int>(total));
  MP_CHECK_LAUNCH();
  return MP_OK;
}

namespace {

// Prefill split: one thread per 16-byte piece (8 dims) of one head of one token row of the fused
// qkv output [B * T, (nh + 2 kvh) * 128].  Query and key pieces are rotated with the cos / sin rows
// of their position t (rope8: the reference's fp16 ops, each product and sum rounded), queries go
// to q_out [B, nh, T, 128] (the attention's layout), keys and values to the caches [B, kvh, cap, 128]
// at position t.  Replaces the slicing, rotation and cache-copy elementwise passes of a prefill.
__global__ __launch_bounds__(256) void prefill_rope_split_kernel(
    const uint16_t *__restrict__ qkv, int t_len, int nh, int kvh, const uint16_t *__restrict__ cos_t,
    const uint16_t *__restrict__ sin_t, int cap, uint16_t *__restrict__ q_out, uint16_t *__restrict__ k_cache,
    uint16_t *__restrict__ v_cache, int64_t pieces) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= pieces) return;
  const int heads = nh + 2 * kvh;
  const int d8 = static_cast<int>(i & 15);                      // 8-dim slice of the head
  const int64_t hrow = i >> 4;                                  // (row, head)
  const int h = static_cast<int>(hrow % heads);
  const int64_t row = hrow / heads;                             // b * T + t
  const int b = static_cast<int>(row / t_len), t = static_cast<int>(row % t_len);
  const uint4 x = *reinterpret_cast<const uint4 *>(qkv + (row * heads + h) * kHd + d8 * 8);
  uint4 o = x;
  if (h < nh + kvh) {
    const uint2 c = *reinterpret_cast<const uint2 *>(cos_t + static_cast<int64_t>(t) * (kHd / 2) + d8 * 4);
    const uint2 sn = *reinterpret_cast<const uint2 *>(sin_t + static_cast<int64_t>(t) * (kHd / 2) + d8 * 4);
    float f[8];
    rope8(x, c, sn, f);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(mp_f2h(f[2 * j])) | (static_cast<uint32_t>(mp_f2h(f[2 * j + 1])) << 16);
    o = make_uint4(w[0], w[1], w[2], w[3]);
  }
  uint16_t *dst;
  if (h < nh)
    dst = q_out + ((static_cast<int64_t>(b) * nh + h) * t_len + t) * kHd;
  else if (h < nh + kvh)
    dst = k_cache + ((static_cast<int64_t>(b) * kvh + (h - nh)) * cap + t) * kHd;
  else
    dst = v_cache + ((static_cast<int64_t>(b) * kvh + (h - nh - kvh)) * cap + t) * kHd;
  *reinterpret_cast<uint4 *>(dst + d8 * 8) = o;
}

}  // namespace

extern "C" int mp_prefill_rope_split(const void *qkv, int64_t batch, int64_t t_len, int nh, int kvh, int head_dim,
                                     const void *cos_t, const void *sin_t, int64_t capacity, void *q_out,
                                     void *k_cache, void *v_cache, mp_stream_t stream) {
  if (!qkv || !cos_t || !sin_t || !q_out || !k_cache || !v_cache) return MP_ERR_ARG;
  if (head_dim != kHd) return MP_ERR_SHAPE;
  if (batch <= 0 || t_len <= 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || capacity <= 0 || t_len > capacity ||
      capacity > INT32_MAX)
    return MP_ERR_SHAPE;
  if (!mp_aligned(qkv, 16) || !mp_aligned(q_out, 16) || !mp_aligned(k_cache, 16) || !mp_aligned(v_cache, 16) ||
      !mp_aligned(cos_t, 8) || !mp_aligned(sin_t, 8))
    return MP_ERR_ALIGN;
  const int64_t pieces = batch * t_len * (nh + 2 * kvh) * (kHd / 8);
  if (mp_cdiv(pieces, 256) > INT32_MAX) return MP_ERR_SHAPE;
  hipLaunchKernelGGL(prefill_rope_split_kernel, dim3(static_cast<unsigned>(mp_cdiv(pieces, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(qkv),
                     static_cast<int>(t_len), nh, kvh, static_cast<const uint16_t *>(cos_t),
                     static_cast<const uint16_t *>(sin_t), static_cast<int>(capacity), static_cast<uint16_t *>(q_out),
                     static_cast<uint16_t *>(k_cache), static_cast<uint16_t *>(v_cache), pieces);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Workspace: partial o [B, nh, splits, 128] fp32 | partial (m, l) [B, nh, splits, 2] fp32.
extern "C" size_t mp_decode_attention_workspace_bytes(int64_t batch, int nh, int splits) {
  if (batch <= 0 || nh <= 0 || splits <= 0) return 0;
  return static_cast<size_t>(batch) * nh * splits * (kHd + 2) * sizeof(float);
}

namespace {

// Shared launcher of the two attention entry points (ROPE: qsrc is the qkv row).
int launch_decode_attention(bool rope, const void *qsrc, int64_t batch, int nh, int kvh, int head_dim,
                            const void *cos_t, const void *sin_t, void *k_cache, void *v_cache, const int64_t *pos,
                            int64_t capacity, int splits, float scale, void *out, void *workspace,
                            size_t workspace_bytes, hipStream_t s) {
  if (!qsrc || !k_cache || !v_cache || !pos || !out || !workspace) return MP_ERR_ARG;
  if (rope && (!cos_t || !sin_t)) return MP_ERR_ARG;
  if (head_dim != kHd) return MP_ERR_SHAPE;
  // the fused append stores through a descriptor over one (row, kv head) cache slice
  if (rope && capacity * kHd * 2 >= (int64_t(1) << 31)) return MP_ERR_SHAPE;
  if (batch <= 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || capacity <= 0 || capacity > INT32_MAX) return MP_ERR_SHAPE;
  const int grp = nh / kvh;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8) return MP_ERR_SHAPE;
  if (splits <= 0 || splits > kMergeMaxSplits || batch * kvh > 65535) return MP_ERR_SHAPE;
  const int chunk = static_cast<int>(mp_cdiv(capacity, splits));
  // scores [GRP][chunk] and the [GRP][4][128] reduction share the dynamic LDS
  const size_t lds = static_cast<size_t>(grp) * (chunk > 4 * kHd ? chunk : 4 * kHd) * sizeof(float);
  if (lds > 64 * 1024) return MP_ERR_SHAPE;
  if (workspace_bytes < mp_decode_attention_workspace_bytes(batch, nh, splits)) return MP_ERR_WORKSPACE;
  if (!mp_aligned(qsrc, 16) || !mp_aligned(k_cache, 16) || !mp_aligned(v_cache, 16) || !mp_aligned(workspace, 16) ||
      !mp_aligned(out, 4))
    return MP_ERR_ALIGN;
  if (rope && (!mp_aligned(cos_t, 8) || !mp_aligned(sin_t, 8))) return MP_ERR_ALIGN;
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o + static_cast<size_t>(batch) * nh * splits * kHd;
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(batch * kvh));
  const auto *qp = static_cast<const uint16_t *>(qsrc);
  const auto *cp = static_cast<const uint16_t *>(cos_t);
  const auto *sp = static_cast<const uint16_t *>(sin_t);
  auto *kp = static_cast<uint16_t *>(k_cache);
  auto *vp = static_cast<uint16_t *>(v_cache);
  auto *op = static_cast<uint16_t *>(out);
  const int cap = static_cast<int>(capacity);
  // one load round covers a chunk of up to 80 positions (five steps of 16)
  const bool u5 = chunk <= 80;
#define MP_ATTN_LAUNCH(G, R)                                                                                   \
  do {                                                                                                         \
    if (u5)                                                                                                    \
      hipLaunchKernelGGL((decode_attn_kernel<G, R, 5>), grid, dim3(256), lds, s, qp, cp, sp, kp, vp, pos, kvh, \
                         cap, chunk, splits, scale, part_o, part_ml, op);                                      \
    else                                                                                                       \
      hipLaunchKernelGGL((decode_attn_kernel<G, R, 4>), grid, dim3(256), lds, s, qp, cp, sp, kp, vp, pos, kvh, \
                         cap, chunk, splits, scale, part_o, part_ml, op);                                      \
  } while (0)
  if (rope) {
    switch (grp) {
      case 1: MP_ATTN_LAUNCH(1, true); break;
      case 2: MP_ATTN_LAUNCH(2, true); break;
      case 4: MP_ATTN_LAUNCH(4, true); break;
      default: MP_ATTN_LAUNCH(8, true); break;
    }
  } else {
    switch (grp) {
      case 1: MP_ATTN_LAUNCH(1, false); break;
      case 2: MP_ATTN_LAUNCH(2, false); break;
      case 4: MP_ATTN_LAUNCH(4, false); break;
      default: MP_ATTN_LAUNCH(8, false); break;
    }
  }
#undef MP_ATTN_LAUNCH
  MP_CHECK_LAUNCH();
  if (splits > 1) {
    const int64_t heads = batch * nh;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(static_cast<unsigned>(mp_cdiv(heads, 4))), dim3(256), 0, s, part_o,
                       part_ml, pos, cap, chunk, splits, rope ? 1 : 0, heads, op);
    MP_CHECK_LAUNCH();
  }
  return MP_OK;
}

}  // namespace

extern "C" int mp_decode_attention(const void *q, int64_t batch, int nh, int kvh, int head_dim, const void *k_cache,
                                   const void *v_cache, const int64_t *pos, int64_t capacity, int splits, float scale,
                                   void *out, void *workspace, size_t workspace_bytes, mp_stream_t stream) {
  return launch_decode_attention(false, q, batch, nh, kvh, head_dim, nullptr, nullptr, const_cast<void *>(k_cache),
                                 const_cast<void *>(v_cache), pos, capacity, splits, scale, out, workspace,
                                 workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int mp_decode_rope_attention(const void *qkv, int64_t batch, int nh, int kvh, int head_dim,
                                        const void *cos_t, const void *sin_t, const int64_t *pos, int64_t capacity,
                                        void *k_cache, void *v_cache, int splits, float scale, void *out,
                                        void *workspace, size_t workspace_bytes, mp_stream_t stream) {
  return launch_decode_attention(true, qkv, batch, nh, kvh, head_dim, cos_t, sin_t, k_cache, v_cache, pos, capacity,
                                 splits, scale, out, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int mp_argmax_rows(const void *x, int64_t rows, int64_t n, int64_t *idx, mp_stream_t stream) {
  if (!x || !idx) return MP_ERR_ARG;
  if (rows < 0 || rows > UINT32_MAX || n <= 0 || n > INT32_MAX - 1024) return MP_ERR_SHAPE;
  if (rows == 0) return MP_OK;
  const bool vec = n % 8 == 0 && mp_aligned(x, 16);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t spans = mp_cdiv(n, kArgmaxSpan);
  if (spans >= 4 && rows <= 65535) {
    // long rows: spans of one row on many CUs (a single workgroup per row is bound by one CU's
    // outstanding loads)
    const dim3 g1(static_cast<unsigned>(mp_cdiv(rows, 256)));
    hipLaunchKernelGGL(argmax_clear_kernel, g1, dim3(256), 0, s, idx, rows);
    const dim3 g2(static_cast<unsigned>(spans), static_cast<unsigned>(rows));
    const auto *xp = static_cast<const uint16_t *>(x);
    if (vec) hipLaunchKernelGGL(argmax_span_kernel<true>, g2, dim3(256), 0, s, xp, static_cast<int>(n), idx);
    else hipLaunchKernelGGL(argmax_span_kernel<false>, g2, dim3(256), 0, s, xp, static_cast<int>(n), idx);
    hipLaunchKernelGGL(argmax_decode_kernel, g1, dim3(256), 0, s, idx, rows);
    MP_CHECK_LAUNCH();
    return MP_OK;
  }
  if (vec)
    hipLaunchKernelGGL(argmax_rows_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(x), static_cast<int>(n),
                       idx);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(x), static_cast<int>(n),
                       idx);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_silu_mul(const void *gate_up, int64_t rows, int64_t inter, void *act, int dtype,
                           mp_stream_t stream) {
  if (!gate_up || !act) return MP_ERR_ARG;
  if (dtype != MP_F16 && dtype != MP_BF16) return MP_ERR_DTYPE;
  if (rows < 0 || inter <= 0 || inter > INT32_MAX) return MP_ERR_SHAPE;
  const int64_t total = rows * inter;
  if (total == 0) return MP_OK;
  if (mp_cdiv(total, 256) > UINT32_MAX) return MP_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(mp_cdiv(total, 256)));
  const auto *gp = static_cast<const uint16_t *>(gate_up);
  auto *ap = static_cast<uint16_t *>(act);
  if (dtype == MP_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<true>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), gp,
                       static_cast<int>(inter), total, ap);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), gp,
                       static_cast<int>(inter), total, ap);
  MP_CHECK_LAUNCH();
  return MP_OK;
}
