// Dequantising GEMM: Y = dq(A) . dq(B)^T with every operand element rounded to the
// activation dtype exactly as the reference's fake-quant / pseudo-quant tensors are, then
// fp16 / bf16 MFMA with fp32 accumulation (the arithmetic of F.linear on those tensors).
#pragma once
#include "i8_gemm.h"

// Operand formats.
enum mp_dq_fmt {
  MP_DQ_DT = 0,     // values in the arithmetic dtype, [rows, K]
  MP_DQ_I8ROW = 1,  // int8 codes [rows, K] + fp32 per-row scale (a value exact in the dtype): r(q * s)
  MP_DQ_U4GRP = 2   // B only: packed nibbles int32 [N, K/8] (column k in nibble k % 8 of word k / 8)
                    // + group scales [N, K/g] and zeros [N, K/g] in the dtype (null: zero point 8):
                    // r((u - z) * s)
};

struct mp_dq_args {
  int dt;                    // MP_F16 / MP_BF16: the rounding and MFMA dtype
  const void *a;             // [R, K] (dense: M rows)
  int a_fmt;                 // MP_DQ_DT or MP_DQ_I8ROW
  const float *a_scale;      // MP_DQ_I8ROW: [R]
  const void *b;             // [E?, N_b, K] (MP_DQ_U4GRP: [N_b, K/8] words, no experts)
  int b_fmt;
  const float *b_scale;      // MP_DQ_I8ROW: [E?, N_b]
  const uint16_t *b_gscale;  // MP_DQ_U4GRP: [N_b, K/g] in dt
  const uint16_t *b_gzero;   // MP_DQ_U4GRP: [N_b, K/g] in dt, or null (zero point 8)
  int group;                 // MP_DQ_U4GRP group size (a multiple of 32 dividing K)
  const void *bias;          // DENSE: [N] or null
  int bias_dtype;
  void *y;                   // DENSE: [R, ldy] in out_dtype; F32: fp32; SWIGLU: fp32 h [R, ldy]
  int out_dtype;
  int64_t ldy;
  float *amax_partial;       // SWIGLU: [R, n_partial], n_partial = 2 * ceil(I / 64)
  int n_partial;
  const int64_t *offsets;    // grouped: [E+1] cumulative row endpoints; null = dense
  int n_experts;
  int64_t rows, n, k;        // n = output columns (SWIGLU: I; B then holds 2I rows per expert)
};

// Launch on `stream`; returns MP_OK or an MP_ERR_* code (shapes checked here).  K % 64 == 0
// takes the tiled MFMA kernel, other K a one-output-per-thread kernel of the same arithmetic.
int mp_launch_dq_gemm(const mp_dq_args &args, int epilogue, hipStream_t stream);
