// Measurement-only library (libmindpipe_measure.so, not part of the product ABI): read probes
// that stream device memory through the vector memory path and do no other work, so a launch's
// duration is what launch, latency and transfer alone cost for that many bytes.  The kernels'
// roofline fractions are read against it.  No counterpart in the reference.
//
// Two forms, each with a choice of loads per lane (LOADS 16-byte loads, all issued before any
// arithmetic; consecutive lanes on consecutive 16-byte pieces):
//  * one-shot: one workgroup per THREADS * LOADS pieces (the one-row GEMVs' launch shape at
//    THREADS = 256, LOADS = 4);
//  * strided: a fixed grid; workgroup w reads pieces w * THREADS * LOADS + j * grid * THREADS *
//    LOADS, j = 0, 1, ... (a persistent streaming kernel).
#include "../csrc/mp_common.h"

namespace {

template <int THREADS, int LOADS>
__global__ __launch_bounds__(THREADS) void probe_read_kernel(const uint4 *__restrict__ p, int64_t n16, int64_t rounds,
                                                             uint32_t *__restrict__ sink) {
  constexpr int64_t kChunk = static_cast<int64_t>(THREADS) * LOADS;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kChunk;
  int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
  uint32_t x = 0;
  for (int64_t r = 0; r < rounds; ++r, base += stride) {
    uint4 v[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      int64_t idx = base + static_cast<int64_t>(i) * THREADS;
      idx = idx < n16 ? idx : n16 - 1;
      v[i] = p[idx];
    }
#pragma unroll
    for (int i = 0; i < LOADS; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  // data-dependent store that keeps the loads live; with any buffer content it writes at most one
  // word per workgroup, into sink[blockIdx.x]
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

template <int THREADS, int LOADS>
int launch(const void *buf, int64_t n16, int64_t grid, int64_t rounds, uint32_t *sink, hipStream_t s) {
  hipLaunchKernelGGL((probe_read_kernel<THREADS, LOADS>), dim3(static_cast<unsigned>(grid)), dim3(THREADS), 0, s,
                     static_cast<const uint4 *>(buf), n16, rounds, sink);
  MP_CHECK_LAUNCH();
  return MP_OK;
}

template <int THREADS>
int launch_loads(int loads, const void *buf, int64_t n16, int64_t grid, int64_t rounds, uint32_t *sink,
                 hipStream_t s) {
  switch (loads) {
    case 1: return launch<THREADS, 1>(buf, n16, grid, rounds, sink, s);
    case 2: return launch<THREADS, 2>(buf, n16, grid, rounds, sink, s);
    case 4: return launch<THREADS, 4>(buf, n16, grid, rounds, sink, s);
    case 8: return launch<THREADS, 8>(buf, n16, grid, rounds, sink, s);
    default: return MP_ERR_ARG;
  }
}

}  // namespace

// Workgroups of a read of `bytes` with `threads` threads and `loads` 16-byte loads per lane:
// `grid` > 0 fixes the grid (strided form), grid = 0 gives one-shot workgroups.
extern "C" int64_t mp_probe_read_grid(int64_t bytes, int threads, int loads, int64_t grid) {
  if (bytes < 16 || threads <= 0 || loads <= 0) return 0;
  const int64_t per = static_cast<int64_t>(threads) * loads;
  const int64_t need = mp_cdiv(bytes / 16, per);
  return grid > 0 ? (grid < need ? grid : need) : need;
}

// One launch reading `bytes` (a multiple of 16, 16-byte aligned buf); threads in {256, 512},
// loads in {1, 2, 4, 8}; sink: uint32 [mp_probe_read_grid(...)], written at most once per
// workgroup.
extern "C" int mp_probe_read_shape(const void *buf, int64_t bytes, int threads, int loads, int64_t grid,
                                   uint32_t *sink, mp_stream_t stream) {
  if (bytes < 16 || bytes % 16 != 0) return MP_ERR_SHAPE;
  if (!buf || !sink) return MP_ERR_ARG;
  if (!mp_aligned(buf, 16)) return MP_ERR_ALIGN;
  const int64_t n16 = bytes / 16;
  const int64_t g = mp_probe_read_grid(bytes, threads, loads, grid);
  if (g <= 0 || g > INT32_MAX) return MP_ERR_SHAPE;
  const int64_t rounds = mp_cdiv(n16, g * threads * loads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (threads == 256) return launch_loads<256>(loads, buf, n16, g, rounds, sink, s);
  if (threads == 512) return launch_loads<512>(loads, buf, n16, g, rounds, sink, s);
  return MP_ERR_ARG;
}
