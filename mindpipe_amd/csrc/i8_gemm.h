// Internal launchers shared by the dense W8A8 and the MoE entry points.
#pragma once
#include "mp_common.h"

enum mp_i8_epilogue {
  MP_EPI_DENSE = 0,  // y = ((acc * s_tok) * s_ch) (+ bias) -> out dtype
  MP_EPI_F32 = 1,    // y = (acc * s_tok) * s_ch -> fp32 (grouped GEMM2)
  MP_EPI_SWIGLU = 2, // h = silu(g) * u -> fp32 workspace + per-row partial absmax
  MP_EPI_AMAX = 3    // y = ((acc * s_tok) * s_ch) (+ bias) -> 16-bit out dtype + per-row partial absmax
                     // of the rounded outputs (the output-quant GEMM; i8_moe_kernel only)
};

struct mp_i8_args {
  const int8_t *a;           // [R, K] rows (dense: M rows)
  const float *s_a;          // [R]
  const int8_t *b;           // [E?, N_b, K] weight rows
  const float *s_b;          // [E?, N_b]
  const void *bias;          // [N] or null (dense only)
  int bias_dtype;
  void *y;                   // output
  int out_dtype;
  float *amax_partial;       // SWIGLU: [R, n_partial]
  int n_partial;
  const int64_t *offsets;    // grouped: [E+1] cumulative row endpoints; null = dense
  int n_experts;
  int64_t rows;              // R (dense: M)
  int64_t n;                 // output columns (SWIGLU: I)
  int64_t k;
  int64_t ldy;               // output row stride (elements)
  int staged_epilogue;       // large-M kernel: 16-bit outputs through LDS, 16-byte stores
  int epi_round;             // SWIGLU: mp_round_mode of g, u, silu(g) and h (kRoundNone: fp32)
  int shared_b;              // grouped launches: every group multiplies the same b / s_b (a dense
                             // GEMM run as 256-row groups); 0: group e uses expert e's rows
  int xcd_row_tiles;         // dense tiled launches on a 1-D grid: the row tiles of a column tile sit
                             // 8 apart in dispatch order (one XCD); 0: the 2-D grid (x: columns, y: rows)
};

int mp_launch_i8_gemm(const mp_i8_args &args, int epilogue, hipStream_t stream);
