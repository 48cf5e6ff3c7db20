// Decode-step kernels of the Llama-shaped measurement harness around the
// quantized linears: RoPE + KV-cache append, split-K decode attention (flash
// decoding) with its combine, and SiLU-multiply.  The reference has no
// counterpart (attention belongs to vLLM's backend); these exist so that one
// greedy decode step runs as ~10 launches per layer and the W4A16 GEMVs, not
// launch gaps, set the step time.
//
// Shapes: head dim 128; q/k/v heads packed as one qkv row [B, (nh + 2 kvh) * 128]
// (the fused qkv W4A16 output); KV cache per layer K, V [B, kvh, T, 128] fp16
// (one 256-byte row per position).  The current position is read from device
// memory, so every launch has a fixed shape and a step can be graph-captured.
#include "mp_common.h"

namespace {

constexpr int kHd = 128;

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
// Grid (splits, B * kvh), 256 threads.  A workgroup scores positions
// [s*chunk, min((s+1)*chunk, len)) for the GRP query heads of one kv head:
// 16 lanes per position (8 dims each, one 16-byte load), 4 positions per wave
// per step, fp32 dot products reduced over the 16 lanes.  Scores go to LDS,
// softmax statistics are taken over the workgroup, then P.V accumulates in
// fp32 with the same lane layout.  Output: unnormalised partial o, running max
// m and sum l per (row, head, split), merged by attn_combine_kernel.
template <int GRP>
__global__ __launch_bounds__(256) void decode_attn_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k_cache, const uint16_t *__restrict__ v_cache,
    const int64_t *__restrict__ pos_p, int kvh, int cap, int chunk, int splits, float scale,
    float *__restrict__ part_o, float *__restrict__ part_ml) {
  extern __shared__ float sm[];      // [GRP][chunk] scores, then [GRP][4][128] reduction
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = blockIdx.x;
  const int bk = blockIdx.y;         // b * kvh + kh
  const int64_t p1 = pos_p[0] + 1;   // valid positions [0, pos], clamped to the cache
  const int len = static_cast<int>(p1 < 0 ? 0 : (p1 > cap ? cap : p1));
  const int t0 = s * chunk;
  if (t0 >= len) return;             // workgroup-uniform; the combine reads only used splits
  const int t1 = min(t0 + chunk, len);
  const int n = t1 - t0;
  const int nh = kvh * GRP;
  const int b = bk / kvh, kh = bk % kvh;
  const int dl = lane & 15;          // 8-dim slice of this lane
  const int pl = lane >> 4;          // position within the wave's group of 4
  const uint16_t *kbase = k_cache + static_cast<int64_t>(bk) * cap * kHd + dl * 8;
  const uint16_t *vbase = v_cache + static_cast<int64_t>(bk) * cap * kHd + dl * 8;

  // query slices (fp32) of the GRP heads
  float qf[GRP][8];
#pragma unroll
  for (int g = 0; g < GRP; ++g) {
    const uint4 qv = *reinterpret_cast<const uint4 *>(q + (static_cast<int64_t>(b) * nh + kh * GRP + g) * kHd + dl * 8);
    const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[g][e] = mp_h2f(static_cast<uint16_t>(qw[e >> 1] >> (16 * (e & 1))));
  }

  // ---- scores: steps of 16 positions per workgroup, 4 steps in flight
  float *sc = sm;
  constexpr int U = 4;
  for (int base = 0; base < n; base += 16 * U) {
    uint4 kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int t = base + u * 16 + wave * 4 + pl;
      t = t < n ? t : n - 1;
      kv[u] = *reinterpret_cast<const uint4 *>(kbase + static_cast<int64_t>(t0 + t) * kHd);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = base + u * 16 + wave * 4 + pl;
      const uint32_t kw[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
      float kf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[e] = mp_h2f(static_cast<uint16_t>(kw[e >> 1] >> (16 * (e & 1))));
#pragma unroll
      for (int g = 0; g < GRP; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(qf[g][e], kf[e], d);
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);
        d += __shfl_xor(d, 4, 64);
        d += __shfl_xor(d, 8, 64);
        if (dl == 0 && t < n) sc[g * chunk + t] = d * scale;
      }
    }
  }
  __syncthreads();

  // ---- softmax statistics per head over the workgroup's positions
  float mx[GRP], sum[GRP];
#pragma unroll
  for (int g = 0; g < GRP; ++g) {
    float m = -INFINITY;
    for (int t = tid; t < n; t += 256) m = fmaxf(m, sc[g * chunk + t]);
    m = mp_wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (int t = tid; t < n; t += 256) {
      const float p = expf(sc[g * chunk + t] - m);
      sc[g * chunk + t] = p;
      l += p;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    l = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    mx[g] = m;
    sum[g] = l;
  }

  // ---- P.V
  float acc[GRP][8];
#pragma unroll
  for (int g = 0; g < GRP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  for (int base = 0; base < n; base += 16 * U) {
    uint4 vv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int t = base + u * 16 + wave * 4 + pl;
      t = t < n ? t : n - 1;
      vv[u] = *reinterpret_cast<const uint4 *>(vbase + static_cast<int64_t>(t0 + t) * kHd);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = base + u * 16 + wave * 4 + pl;
      const uint32_t vw[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
      float vf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) vf[e] = mp_h2f(static_cast<uint16_t>(vw[e >> 1] >> (16 * (e & 1))));
#pragma unroll
      for (int g = 0; g < GRP; ++g) {
        const float p = t < n ? sc[g * chunk + t] : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
      }
    }
  }
  // reduce over the 4 positions of a wave (lanes l, l^16, l^32, l^48), then over the waves
#pragma unroll
  for (int g = 0; g < GRP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[g][e] += __shfl_xor(acc[g][e], 16, 64);
      acc[g][e] += __shfl_xor(acc[g][e], 32, 64);
    }
  __syncthreads();  // the score buffer is reused for the reduction
  float *rw = sm;   // [GRP][4 waves][128]
  if (pl == 0) {
#pragma unroll
    for (int g = 0; g < GRP; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) rw[(g * 4 + wave) * kHd + dl * 8 + e] = acc[g][e];
  }
  __syncthreads();
  for (int i = tid; i < GRP * kHd; i += 256) {
    const int g = i / kHd, d = i % kHd;
    const float o = (rw[(g * 4 + 0) * kHd + d] + rw[(g * 4 + 1) * kHd + d]) +
                    (rw[(g * 4 + 2) * kHd + d] + rw[(g * 4 + 3) * kHd + d]);
    const int64_t head = static_cast<int64_t>(b) * nh + kh * GRP + g;
    part_o[(head * splits + s) * kHd + d] = o;
    if (d == 0) {
      part_ml[(head * splits + s) * 2 + 0] = mx[g];
      part_ml[(head * splits + s) * 2 + 1] = sum[g];
    }
  }
}

// One 128-thread workgroup per (row, head): merge the used splits.
__global__ __launch_bounds__(128) void attn_combine_kernel(const float *__restrict__ part_o,
                                                           const float *__restrict__ part_ml,
                                                           const int64_t *__restrict__ pos_p, int cap, int chunk,
                                                           int splits, uint16_t *__restrict__ out) {
  const int64_t head = blockIdx.x;
  const int d = threadIdx.x;
  const int64_t p1 = pos_p[0] + 1;
  const int len = static_cast<int>(p1 < 0 ? 0 : (p1 > cap ? cap : p1));
  int used = (len + chunk - 1) / chunk;
  used = used < splits ? used : splits;
  float m = -INFINITY;
  for (int s = 0; s < used; ++s) m = fmaxf(m, part_ml[(head * splits + s) * 2]);
  float num = 0.f, den = 0.f;
  for (int s = 0; s < used; ++s) {
    const float w = expf(part_ml[(head * splits + s) * 2] - m);
    num = fmaf(w, part_o[(head * splits + s) * kHd + d], num);
    den = fmaf(w, part_ml[(head * splits + s) * 2 + 1], den);
  }
  out[head * kHd + d] = mp_f2h(num / den);
}

// ---------------------------------------------------------------- SiLU * up
// gu [B, 2I] (gate | up) -> act [B, I] = round(round(silu(gate)) * up).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, int inter, int64_t total,
                                                       uint16_t *__restrict__ act) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / inter, c = i % inter;
  const float g = mp_h2f(gu[b * 2 * inter + c]);
  const float u = mp_h2f(gu[b * 2 * inter + inter + c]);
  const float sg = mp_rh(g / (1.0f + expf(-g)));
  act[i] = mp_f2h(sg * u);
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

extern "C" size_t mp_decode_attention_workspace_bytes(int64_t batch, int nh, int splits) {
  if (batch <= 0 || nh <= 0 || splits <= 0) return 0;
  return static_cast<size_t>(batch) * nh * splits * (kHd + 2) * sizeof(float);
}

extern "C" int mp_decode_attention(const void *q, int64_t batch, int nh, int kvh, int head_dim, const void *k_cache,
                                   const void *v_cache, const int64_t *pos, int64_t capacity, int splits, float scale,
                                   void *out, void *workspace, size_t workspace_bytes, mp_stream_t stream) {
  if (!q || !k_cache || !v_cache || !pos || !out || !workspace) return MP_ERR_ARG;
  if (head_dim != kHd) return MP_ERR_SHAPE;
  if (batch <= 0 || nh <= 0 || kvh <= 0 || nh % kvh != 0 || capacity <= 0 || capacity > INT32_MAX) return MP_ERR_SHAPE;
  const int grp = nh / kvh;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8) return MP_ERR_SHAPE;
  if (splits <= 0 || batch * kvh > 65535) return MP_ERR_SHAPE;
  const int chunk = static_cast<int>(mp_cdiv(capacity, splits));
  // scores [GRP][chunk] and the [GRP][4][128] reduction share the dynamic LDS
  const size_t lds = static_cast<size_t>(grp) * (chunk > 4 * kHd ? chunk : 4 * kHd) * sizeof(float);
  if (lds > 64 * 1024) return MP_ERR_SHAPE;
  if (workspace_bytes < mp_decode_attention_workspace_bytes(batch, nh, splits)) return MP_ERR_WORKSPACE;
  if (!mp_aligned(q, 16) || !mp_aligned(k_cache, 16) || !mp_aligned(v_cache, 16) || !mp_aligned(workspace, 16))
    return MP_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float *part_o = static_cast<float *>(workspace);
  float *part_ml = part_o + static_cast<size_t>(batch) * nh * splits * kHd;
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(batch * kvh));
  const auto *qp = static_cast<const uint16_t *>(q);
  const auto *kp = static_cast<const uint16_t *>(k_cache);
  const auto *vp = static_cast<const uint16_t *>(v_cache);
  const int cap = static_cast<int>(capacity);
  switch (grp) {
    case 1:
      hipLaunchKernelGGL(decode_attn_kernel<1>, grid, dim3(256), lds, s, qp, kp, vp, pos, kvh, cap, chunk, splits,
                         scale, part_o, part_ml);
      break;
    case 2:
      hipLaunchKernelGGL(decode_attn_kernel<2>, grid, dim3(256), lds, s, qp, kp, vp, pos, kvh, cap, chunk, splits,
                         scale, part_o, part_ml);
      break;
    case 4:
      hipLaunchKernelGGL(decode_attn_kernel<4>, grid, dim3(256), lds, s, qp, kp, vp, pos, kvh, cap, chunk, splits,
                         scale, part_o, part_ml);
      break;
    default:
      hipLaunchKernelGGL(decode_attn_kernel<8>, grid, dim3(256), lds, s, qp, kp, vp, pos, kvh, cap, chunk, splits,
                         scale, part_o, part_ml);
      break;
  }
  MP_CHECK_LAUNCH();
  hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>(batch * nh)), dim3(kHd), 0, s, part_o, part_ml,
                     pos, cap, chunk, splits, static_cast<uint16_t *>(out));
  MP_CHECK_LAUNCH();
  return MP_OK;
}

extern "C" int mp_silu_mul(const void *gate_up, int64_t rows, int64_t inter, void *act, mp_stream_t stream) {
  if (!gate_up || !act) return MP_ERR_ARG;
  if (rows < 0 || inter <= 0 || inter > INT32_MAX) return MP_ERR_SHAPE;
  const int64_t total = rows * inter;
  if (total == 0) return MP_OK;
  if (mp_cdiv(total, 256) > UINT32_MAX) return MP_ERR_SHAPE;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(mp_cdiv(total, 256))), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t *>(gate_up),
                     static_cast<int>(inter), total, static_cast<uint16_t *>(act));
  MP_CHECK_LAUNCH();
  return MP_OK;
}
