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
// A third probe reads a row-major [rows, row_bytes] matrix in the order a tiled GEMM streams its
// weight operand: workgroup w owns rows [w * tile_rows, +tile_rows) and walks the row length in
// steps of step_bytes, each step reading step_bytes of every one of its rows, DEPTH steps' loads
// issued before any is used.
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

// tile-order read: 256 threads; per step tile_rows * step_bytes / 16 pieces, piece q = row
// q / (step_bytes / 16) of the tile, 16-byte column q % (step_bytes / 16) of the step
template <int DEPTH, int PPT>
__global__ __launch_bounds__(256) void probe_tiles_kernel(const uint4 *__restrict__ p, int64_t rows, int64_t row16,
                                                          int tile_rows, int step16, uint32_t *__restrict__ sink) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * tile_rows;
  const int64_t steps = row16 / step16;
  uint32_t x = 0;
  for (int64_t s0 = 0; s0 < steps; s0 += DEPTH) {
    uint4 v[DEPTH][PPT];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int q = static_cast<int>(threadIdx.x) + 256 * i;
        int64_t row = r0 + q / step16;
        row = row < rows ? row : rows - 1;
        int64_t st = s0 + d;
        st = st < steps ? st : steps - 1;
        v[d][i] = p[row * row16 + st * step16 + q % step16];
      }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int i = 0; i < PPT; ++i) x ^= v[d][i].x ^ v[d][i].y ^ v[d][i].z ^ v[d][i].w;
  }
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

// Per-CU read rate: every workgroup reads the region (blockIdx.x % nreg) of region16 16-byte pieces
// `passes` times, LOADS 16-byte loads per lane per step, two steps in flight.  With nreg = 8 and a
// grid that is a multiple of 8, the workgroups of one XCD share one region, which stays in that
// XCD's L2 after the first pass; large distinct regions come from HBM.  DMA: the loads go straight
// to LDS (buffer_load ... lds) instead of registers.
template <int THREADS, int LOADS, bool DMA>
__global__ __launch_bounds__(THREADS) void probe_cu_read_kernel(const uint4 *__restrict__ p, int64_t region16,
                                                               int nreg, int passes, uint32_t *__restrict__ sink) {
  constexpr int64_t kStep = static_cast<int64_t>(THREADS) * LOADS;
  __shared__ uint4 lds[DMA ? 2 * kStep : 1];
  const uint4 *base = p + static_cast<int64_t>(blockIdx.x % nreg) * region16;
  const uint32_t rbytes = static_cast<uint32_t>(region16 * 16);
  const auto rs = mp_rsrc(base, rbytes);
  const int wave = threadIdx.x >> 6;
  const int64_t steps = region16 / kStep;  // host: region16 a multiple of kStep, >= 2 steps
  uint32_t x = 0;
  uint4 v[2][LOADS];
  auto issue = [&](int64_t st, int slot) {
    const uint32_t off0 = static_cast<uint32_t>((st * kStep + threadIdx.x) * 16);
#pragma unroll
    for (int l = 0; l < LOADS; ++l) {
      const uint32_t off = off0 + static_cast<uint32_t>(l * THREADS * 16);
      if constexpr (DMA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, reinterpret_cast<__attribute__((address_space(3))) void *>(
                    reinterpret_cast<uintptr_t>(&lds[slot * kStep + l * THREADS + wave * 64])),
            16, off, 0, 0, 0);
      else
        v[slot][l] = mp_buf_load16(rs, off, 0);
    }
  };
  for (int ps = 0; ps < passes; ++ps) {
    issue(0, 0);
    for (int64_t st = 0; st < steps; st += 2) {
      issue(st + 1 < steps ? st + 1 : st, 1);
      if constexpr (DMA) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
      } else {
#pragma unroll
        for (int l = 0; l < LOADS; ++l) x ^= v[0][l].x ^ v[0][l].w;
      }
      issue(st + 2 < steps ? st + 2 : st, 0);
      if constexpr (DMA) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
      } else {
#pragma unroll
        for (int l = 0; l < LOADS; ++l) x ^= v[1][l].x ^ v[1][l].w;
      }
    }
    if constexpr (DMA) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
#pragma unroll
      for (int l = 0; l < LOADS; ++l) x ^= v[0][l].x ^ v[0][l].w;
    }
  }
  if constexpr (DMA) {
    __syncthreads();
    x = lds[threadIdx.x].x;
  }
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

// MFMA-operand weight read: an int8 [rows, row_bytes] matrix read the way a wave feeds it to
// v_mfma_i32_32x32x32_i8 as the B operand straight from memory.  A workgroup of four waves owns 32
// rows and a K range (kparts workgroups per 32 rows split K); wave w takes the w-th quarter of it.  Per
// 128-byte K step lane l loads 4 x 16 bytes of row l % 32 at K offset 64 (l / 32) + 16 i: each load
// instruction touches 32 rows x 32 bytes, the four of a step the same 32 cache lines.  DEPTH steps in
// flight.
template <int DEPTH>
__global__ __launch_bounds__(256) void probe_mfma_b_kernel(const int8_t *__restrict__ p, int64_t rows,
                                                          int64_t row_bytes, int kparts, uint32_t *__restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t rblk = blockIdx.x / kparts, kp = blockIdx.x % kparts;
  int64_t row = rblk * 32 + (lane & 31);
  row = row < rows ? row : rows - 1;
  const int64_t kspan = row_bytes / kparts / 4;  // bytes of K per wave (a multiple of 128)
  const int64_t k0 = kp * (row_bytes / kparts) + wave * kspan;
  const int8_t *src = p + row * row_bytes + k0 + 64 * (lane >> 5);
  const int64_t steps = kspan / 128;
  uint32_t x = 0;
  for (int64_t s0 = 0; s0 < steps; s0 += DEPTH) {
    uint4 v[DEPTH][4];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int64_t st = s0 + d < steps ? s0 + d : steps - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[d][i] = *reinterpret_cast<const uint4 *>(src + st * 128 + 16 * i);
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) x ^= v[d][i].x ^ v[d][i].w;
  }
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

}  // namespace

// MFMA-operand weight read (probe_mfma_b_kernel) of an int8 [rows, row_bytes] matrix: ceil(rows / 32) x
// kparts workgroups of 256 threads, depth in {1, 2, 4, 8}; row_bytes a multiple of 512 kparts; sink:
// uint32 [ceil(rows / 32) * kparts].
extern "C" int mp_probe_read_mfma_b(const void *buf, int64_t rows, int64_t row_bytes, int kparts, int depth,
                                    uint32_t *sink, mp_stream_t stream) {
  if (!buf || !sink || rows <= 0 || kparts <= 0) return MP_ERR_ARG;
  if (!mp_aligned(buf, 16)) return MP_ERR_ALIGN;
  if (row_bytes <= 0 || row_bytes % (512 * static_cast<int64_t>(kparts))) return MP_ERR_SHAPE;
  const int64_t grid = mp_cdiv(rows, 32) * kparts;
  if (grid > INT32_MAX) return MP_ERR_SHAPE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto *pp = static_cast<const int8_t *>(buf);
#define MP_PB(D_) hipLaunchKernelGGL((probe_mfma_b_kernel<D_>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, pp, rows, row_bytes, kparts, sink)
  if (depth == 1) MP_PB(1);
  else if (depth == 2) MP_PB(2);
  else if (depth == 4) MP_PB(4);
  else if (depth == 8) MP_PB(8);
  else return MP_ERR_ARG;
#undef MP_PB
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Per-CU read rate (probe_cu_read_kernel): `grid` workgroups of `threads` (256 / 512), `loads` (4 / 8)
// 16-byte loads per lane per step, each reading the region (w % nreg) of `region_bytes` bytes
// `passes` times; dma: loads straight into LDS.  buf holds nreg regions; region_bytes a multiple of
// 2 * threads * loads * 16 and below 4 GiB; sink: uint32 [grid].
extern "C" int mp_probe_cu_read(const void *buf, int64_t region_bytes, int nreg, int passes, int threads, int loads,
                                int dma, int grid, uint32_t *sink, mp_stream_t stream) {
  if (!buf || !sink || nreg <= 0 || passes <= 0 || grid <= 0) return MP_ERR_ARG;
  if (!mp_aligned(buf, 16)) return MP_ERR_ALIGN;
  const int64_t step = static_cast<int64_t>(threads) * loads * 16;
  if (region_bytes <= 0 || region_bytes % (2 * step) || region_bytes >= (int64_t(1) << 32)) return MP_ERR_SHAPE;
  if (dma && 2 * step > 64 * 1024) return MP_ERR_SHAPE;  // the two LDS steps fit 64 KB
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto *pp = static_cast<const uint4 *>(buf);
  const int64_t r16 = region_bytes / 16;
#define MP_PC(T_, L_, D_) hipLaunchKernelGGL((probe_cu_read_kernel<T_, L_, D_>), dim3(static_cast<unsigned>(grid)), dim3(T_), 0, s, pp, r16, nreg, passes, sink)
#define MP_PC_D(T_, L_) do { if (dma) MP_PC(T_, L_, true); else MP_PC(T_, L_, false); } while (0)
  if (threads == 256 && loads == 4) MP_PC_D(256, 4);
  else if (threads == 256 && loads == 8) MP_PC_D(256, 8);
  else if (threads == 512 && loads == 4) MP_PC_D(512, 4);
  else if (threads == 512 && loads == 8) MP_PC_D(512, 8);
  else return MP_ERR_ARG;
#undef MP_PC_D
#undef MP_PC
  MP_CHECK_LAUNCH();
  return MP_OK;
}

// Tile-order read of a row-major [rows, row_bytes] matrix (row_bytes a multiple of step_bytes,
// tile_rows * step_bytes / 16 a multiple of 256 and at most 4096): one workgroup per tile_rows
// rows, depth in {1, 2, 4} steps in flight; sink: uint32 [ceil(rows / tile_rows)].
extern "C" int mp_probe_read_tiles(const void *buf, int64_t rows, int64_t row_bytes, int tile_rows, int step_bytes,
                                   int depth, uint32_t *sink, mp_stream_t stream) {
  if (!buf || !sink || rows <= 0 || tile_rows <= 0 || step_bytes < 16 || step_bytes % 16 || row_bytes % step_bytes)
    return MP_ERR_ARG;
  if (!mp_aligned(buf, 16)) return MP_ERR_ALIGN;
  const int64_t pieces = static_cast<int64_t>(tile_rows) * (step_bytes / 16);
  if (pieces % 256 || pieces > 4096) return MP_ERR_SHAPE;
  const int ppt = static_cast<int>(pieces / 256);
  const int64_t grid = mp_cdiv(rows, tile_rows);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto *pp = static_cast<const uint4 *>(buf);
  const int64_t row16 = row_bytes / 16;
  const int step16 = step_bytes / 16;
#define MP_PT(D_, P_) hipLaunchKernelGGL((probe_tiles_kernel<D_, P_>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, pp, rows, row16, tile_rows, step16, sink)
#define MP_PT_D(P_) do { if (depth == 1) MP_PT(1, P_); else if (depth == 2) MP_PT(2, P_); else if (depth == 4) MP_PT(4, P_); else return MP_ERR_ARG; } while (0)
  switch (ppt) {
    case 1: MP_PT_D(1); break;
    case 2: MP_PT_D(2); break;
    case 4: MP_PT_D(4); break;
    case 8: MP_PT_D(8); break;
    case 16: MP_PT_D(16); break;
    default: return MP_ERR_SHAPE;
  }
#undef MP_PT_D
#undef MP_PT
  MP_CHECK_LAUNCH();
  return MP_OK;
}

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
