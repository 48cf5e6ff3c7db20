/*
 * mindpipe_amd: MI355X (gfx950) quantized-linear forward path, C ABI.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream, launches
 * asynchronously on that stream, never allocates, never synchronises, and
 * returns 0 on success or one of the MP_ERR_* codes below (mp_strerror gives
 * the text).  Shapes are validated on the host before any launch.  Tensors are
 * dense row-major; "[N,K]" means N rows of K contiguous elements.
 *
 * Layouts are the reference's on-disk / module layouts, unchanged:
 *   - W4 packed  : int32 [N, ceil(K/8)], column k in nibble k%8 of word k/8
 *                  (algorithm/quantization/exporters/vllm.py:89-111);
 *                  stored nibble u = int4 + 8 for the signed (GPTQ) export,
 *                  u = q for AWQ asymmetric codes.
 *   - W4 scales  : fp16 [N, K/g]; zeros fp16 [N, K/g] (AWQ, quantizer.py:63-105)
 *                  or NULL meaning the symmetric zero point 8.
 *   - W8 weight  : int8 [N, K] + fp32 per-row scale [N]
 *                  (export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195;
 *                  runtime weight_scale_fp32, vllm_ascend.patch:4030-4031).
 *   - MoE weights: gate_up int8 [E, 2I, H], down int8 [E, H, I] with per-row
 *                  fp32 scales [E, 2I] / [E, H] (fake_quant.py:124-160 layout).
 */
#ifndef MINDPIPE_AMD_H
#define MINDPIPE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *mp_stream_t; /* identical to hipStream_t */

enum mp_status {
  MP_OK = 0,
  MP_ERR_SHAPE = 1,    /* a size or group size the entry point cannot take */
  MP_ERR_DTYPE = 2,    /* unsupported dtype enum */
  MP_ERR_ALIGN = 3,    /* pointer not aligned as the kernel needs (16 B) */
  MP_ERR_HIP = 4,      /* a HIP launch failed */
  MP_ERR_ARG = 5,      /* NULL where a buffer is required, bad enum */
  MP_ERR_WORKSPACE = 6 /* workspace smaller than mp_*_workspace_bytes */
};

/* MP_I8: int8 codes with an fp32 per-row scale (pre-quantized input; mp_moe_permute_quant only). */
enum mp_dtype { MP_F16 = 0, MP_BF16 = 1, MP_F32 = 2, MP_I8 = 3 };

/* Scale rule of the int8 quantizers.
 * MP_SCALE_FP32 : s = fp32(absmax)/127, q = rint(x/s)   (runtime npu_dynamic_quant
 *                 contract, vllm_ascend.patch:1741, and the W8 export rule with
 *                 its 1e-8 clamp).
 * MP_SCALE_FAKE : the arithmetic of quantize_*_absmax (fake_quant.py:10-31) in the
 *                 input dtype r (fp16 or bf16): s = r(r(max(absmax,1e-5))/127),
 *                 q = rint(r(x/s)).  In fp16 |q| <= 127.  In bf16 q can reach
 *                 +-128: a row whose codes reach +128 but not -128 is stored as
 *                 (-q, -s) (same products q*s), a row reaching both clamps +128 to
 *                 127.  MP_SCALE_FP16 is the older name of this rule.           */
enum mp_scale_rule { MP_SCALE_FP32 = 0, MP_SCALE_FAKE = 1, MP_SCALE_FP16 = 1 };

const char *mp_strerror(int status);
int mp_abi_version(void);

/* ---------------------------------------------------------------- W4 (AWQ / GPTQ) */

/* AWQ pseudo_quantize_tensor(w, n_bit=4, zero_point, q_group_size=g,
 * get_scale_zp=True) in the arithmetic of w's dtype (fp16 or bf16); replaces
 * algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-105.
 * w [N,K].  Effective group = g if g > 0 and K % g == 0, else K (per row,
 * quantizer.py:67-68).  Outputs: packed int32 [N, ceil(K/8)] (u = q when
 * zero_point, u = q + 8 when symmetric), scales [N, K/g_eff], zeros
 * [N, K/g_eff] (zero_point only; pass NULL when symmetric), w_deq [N,K]
 * (optional, NULL to skip) = the tensor the reference returns; all in w_dtype. */
int mp_w4_quantize_awq(const void *w, int w_dtype, int64_t n, int64_t k, int group_size, int zero_point,
                       int32_t *packed, void *scales, void *zeros, void *w_deq, mp_stream_t stream);

/* pseudo_quantize_tensor(w, n_bit, zero_point, q_group_size, get_scale_zp=True) at any
 * code width n_bit = 1..8 (2..8 without a zero point) in the arithmetic of w's dtype;
 * replaces quantizer.py:63-105 for n_bit != 4.  Codes in [0, 2^n - 1] with a zero point,
 * else [-2^(n-1), 2^(n-1) - 1].  Outputs: scales [N, K/g_eff], zeros [N, K/g_eff]
 * (zero_point only), w_deq [N,K] (required); no packed codes. */
int mp_awq_pseudo_quantize(const void *w, int w_dtype, int64_t n, int64_t k, int group_size, int zero_point,
                           int n_bit, void *scales, void *zeros, void *w_deq, mp_stream_t stream);

/* GPTQ symmetric round-to-nearest group quantizer in fp32: Quantizer.find_params
 * (perchannel, sym) per group + quantize_with_qint and the signed export
 * q - 8; replaces algorithm/quantization/ptq/gptq/source/quant.py:13-17,44-82
 * and gptq.py:157-161 (without the Hessian error feedback).  w fp32 or fp16
 * [N,K] (w_dtype), K % g == 0.  Outputs (each optional): int_weight int8 [N,K]
 * in [-8,7], packed int32 [N, ceil(K/8)] in the pack_int4_for_vllm layout,
 * scale fp16 [N, K/g] (required). */
int mp_w4_quantize_gptq_rtn(const void *w, int w_dtype, int64_t n, int64_t k, int group_size,
                            int8_t *int_weight, int32_t *packed, void *scale, mp_stream_t stream);

/* pack_int4_for_vllm (algorithm/quantization/exporters/vllm.py:89-111):
 * int8 [N,K] in [-8,7] -> int32 [N, ceil(K/8)], K zero-padded.  Values out of
 * range are counted into *bad_count (device int32, caller zeroes it); the
 * caller raises like the reference's ValueError when it is non-zero. */
int mp_pack_int4(const int8_t *int_weight, int64_t n, int64_t k, int32_t *packed, int32_t *bad_count,
                 mp_stream_t stream);

/* Inverse of mp_pack_int4 (tests/test_vllm_real_quant_export.py:23-27). */
int mp_unpack_int4(const int32_t *packed, int64_t n, int64_t k, int8_t *int_weight, mp_stream_t stream);

/* Y[M,N] = X[M,K] . dequant(W)^T (+ bias[N]); dequant(w) = (u - z) * s with z
 * from zeros (or 8 when zeros == NULL).  Replaces the fp16 F.linear on AWQ
 * pseudo-quantized weights (quantizer.py:108-130 + the HF forward) and the
 * vLLM compressed-tensors WNA16 kernel the export targets
 * (scripts/repro/evaluate_vllm_real_int4_ppl.py:48-76).  x, scales, zeros, bias, y
 * in x_dtype; K % 8 == 0, K % g == 0.  fp16: M <= 64 runs the streaming (decode)
 * kernels, larger M the tiled (prefill) kernel.  bf16: the dequantising MFMA GEMM,
 * each weight rounded to bf16 as the reference's pseudo-quantized weight is. */
int mp_w4a16_gemm(const void *x, int64_t m, int64_t k, const int32_t *w_packed, int64_t n,
                  const void *scales, const void *zeros, int group_size, const void *bias, void *y,
                  int x_dtype, mp_stream_t stream);

/* act[M, I] = silu(G) * U with [G | U] = X . dequant(W)^T (+ bias[2I]) for the fused
 * gate/up weight W [2I, K] (gate rows first): the gate/up linear and the SiLU-mul
 * of the SwiGLU MLP (act_fn(gate_up) in the HF / vLLM Llama MLP the W4A16 export
 * serves) in one launch.  Every value is rounded as the two-step path rounds it
 * (fp16 / bf16 gate and up, then the rounded silu times up).  Group 128,
 * K % 256 == 0; fp16 or bf16.  The row ranges of mp_w4a16_gemm: the decode kernels up
 * to 64 rows and the batched kernel's row parts where its grid fills the chip better,
 * else the prefill kernel's SwiGLU form (M * K and M * I below 2^30). */
int mp_w4a16_gemm_swiglu(const void *x, int64_t m, int64_t k, const int32_t *w_packed, int64_t n2,
                         const void *scales, const void *zeros, int group_size, const void *bias, void *act,
                         int x_dtype, mp_stream_t stream);

/* One activation row x [K] (fp16): y = RMSNorm(x + residual) * norm_weight . dequant(W)^T
 * (+ bias), or with swiglu != 0 the SiLU-up product of the fused gate/up weight [N = 2I, K]
 * (y [I]); residual_out = round(x + residual) (optional; residual may be NULL).  No
 * counterpart in the reference: the fusion of mp_add_rms_norm_quant (quant off) with
 * mp_w4a16_gemm / mp_w4a16_gemm_swiglu at M = 1 for a decode step, bit-identical to
 * that two-launch chain.  K in {2048, 4096, 8192}, group 128; residual_out must not
 * overlap x or residual. */
int mp_w4a16_gemv_rmsnorm(const void *x, const void *residual, const void *norm_weight, float eps,
                          void *residual_out, int64_t k, const int32_t *w_packed, int64_t n, const void *scales,
                          const void *zeros, int group_size, const void *bias, int swiglu, void *y, int x_dtype,
                          mp_stream_t stream);

/* ---------------------------------------------------------------- W8A8 (SmoothQuant) */

/* Per-token dynamic symmetric int8 quant of x [M,K] (fp16/bf16/fp32).
 * MP_SCALE_FP32: replaces torch_npu.npu_dynamic_quant (vllm_ascend.patch:3950),
 *   scale fp32 [M].
 * MP_SCALE_FAKE: codes of quantize_activation_per_token_absmax
 *   (fake_quant.py:22-31), scale [M] in x's dtype (x fp16 or bf16; signed as the
 *   rule above stores the row). */
int mp_quant_per_token_i8(const void *x, int64_t m, int64_t k, int x_dtype, int8_t *q, void *scale,
                          int scale_rule, mp_stream_t stream);

/* Fused residual add + RMSNorm (+ per-token dynamic int8 quant) of x [M,H]
 * (fp16/bf16), replacing torch_npu.npu_add_rms_norm_dynamic_quant and the
 * npu_add_rms_norm -> npu_dynamic_quant chain of the W8A8 runtime
 * (vllm_ascend.patch:746-787).  sum = x + residual (fp32; residual may be NULL),
 * residual_out = sum in the input dtype (optional), y = round(round(sum * rstd)
 * * weight) (optional), q int8 [M,H] + scale fp32 [M] = per-token quant of y
 * with the MP_SCALE_FP32 rule of mp_quant_per_token_i8 (optional, both or
 * neither).  In-place calls (residual_out == residual, y == x) are allowed. */
int mp_add_rms_norm_quant(const void *x, const void *residual, const void *weight, float eps, int64_t m,
                          int64_t h, int dtype, void *residual_out, void *y, int8_t *q, float *scale,
                          mp_stream_t stream);

/* Per-output-channel symmetric int8 weight quant of w [N,K] (fp16/bf16).
 * MP_SCALE_FP32: quantize_weight_per_channel
 *   (scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195),
 *   scale_f32 [N] and scale_src [N] in the source dtype (optional).
 * MP_SCALE_FAKE: quantize_weight_per_channel_absmax (fake_quant.py:10-19) in the
 *   weight dtype, scale_f32 [N] holds the (signed) scale value exactly; scale_src [N]
 *   in the weight dtype.
 * Rows holding a non-finite value are counted into *bad_count (optional). */
int mp_w8_quantize_per_channel(const void *w, int64_t n, int64_t k, int w_dtype, int8_t *q,
                               float *scale_f32, void *scale_src, int scale_rule, int32_t *bad_count,
                               mp_stream_t stream);

/* Y[M,N] = ((int32 acc = Qx . Qw^T) * s_tok[m]) * s_ch[n] (+ bias[n]) rounded to
 * out_dtype (fp16/bf16/fp32).  Replaces torch_npu.npu_quant_matmul
 * (vllm_ascend.patch:4007-4015).  qx int8 [M,K], w int8 [N,K], K % 16 == 0. */
int mp_w8a8_gemm(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                 const void *bias, int bias_dtype, void *y, int out_dtype, int64_t m, int64_t n,
                 int64_t k, mp_stream_t stream);

/* y[M,N] = F.linear(r(qx * s_tok), r(w * s_ch), bias) in act_dtype (fp16 / bf16): the
 * fake path of SmoothQuantLinear.forward (fake_quant.py:85-88) on the fake rule's codes
 * (MP_SCALE_FAKE of mp_quant_per_token_i8 / mp_w8_quantize_per_channel), each operand
 * element rounded to act_dtype as the reference's fake-quant tensors are, fp32
 * accumulation, bias added in fp32, one rounding.  The int8 GEMM above multiplies the
 * unrounded q * s; in bf16 (8 significant bits) that differs from the fake path by ~3e-3,
 * so the bf16 fake-rule linear runs here.  bias in act_dtype or NULL. */
int mp_w8a8_gemm_fake(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                      const void *bias, int act_dtype, void *y, int64_t m, int64_t n, int64_t k,
                      mp_stream_t stream);

/* The fake-quant linear at any operand widths (fake_quant.py:85-88 with weight_bits /
 * activation_bits other than 8, SmoothQuantLinear of fake_quant.py:38-113): y[M,N] =
 * F.linear(A, B, bias) in dtype (fp16 / bf16) where A is int8 codes [M,K] with a_scale
 * [M] (the value r(q * s) of quantize_activation_per_token_absmax) or, with a_scale NULL,
 * plain values [M,K] in dtype (activation_bits >= 16); B likewise int8 [N,K] with
 * b_scale [N] or plain values (weight_bits >= 16).  fp32 accumulation, bias (dtype, or
 * NULL) added in fp32, one rounding. */
int mp_dq_linear(const void *a, const float *a_scale, const void *b, const float *b_scale, const void *bias,
                 int dtype, void *y, int64_t m, int64_t n, int64_t k, mp_stream_t stream);

/* quantize_activation_per_token_absmax / quantize_weight_per_channel_absmax
 * (fake_quant.py:10-31) at n_bits = 2..7, per row of x [rows, K] (fp16 / bf16), in the
 * arithmetic of x's dtype: q_max = 2^(n-1) - 1, s = r(r(max(amax, 1e-5)) / q_max),
 * q = rint(r(x / s)).  Outputs int8 codes [rows, K] (|q| <= q_max + 1) and scale fp32
 * [rows] (a value of x's dtype); the fake value is r(q * s).  8 bits: MP_SCALE_FAKE of
 * mp_quant_per_token_i8 / mp_w8_quantize_per_channel. */
int mp_fake_quant_rows(const void *x, int x_dtype, int64_t rows, int64_t k, int n_bits, int8_t *q, float *scale,
                       mp_stream_t stream);

/* Output-quant W8A8 linear: y[M,N] = mp_w8a8_gemm's output (out_dtype fp16 / bf16, bias in
 * bias_dtype or NULL) together with its per-token int8 codes q_out[M,N] and scale s_out[M]:
 * the q/k/v output quant of SmoothQuantLinear(quantize_output=True) (fake_quant.py:77-82),
 * returned as (int8, scale) in the return_scale form (vllm_ascend.patch:4019-4020).
 * scale_rule MP_SCALE_FP32: s = max|y|/127 in fp32, q = rint(y / s) (quantize_per_token_i8's
 * runtime rule on y); MP_SCALE_FAKE: quantize_activation_per_token_absmax in out_dtype.  The
 * GEMM epilogue rounds y and writes each row's partial abs-max per 64 columns; a second launch
 * reduces them and writes the codes.  K % 128 == 0, K <= 2^17, M <= 262144, N <= 2^20;
 * qx, w 16-byte aligned; workspace of mp_w8a8_gemm_quant_out_workspace_bytes(M, N), 16-byte
 * aligned.  Calls that share a workspace must not overlap. */
size_t mp_w8a8_gemm_quant_out_workspace_bytes(int64_t m, int64_t n);
int mp_w8a8_gemm_quant_out(const int8_t *qx, const float *s_tok, const int8_t *w, const float *s_ch,
                           const void *bias, int bias_dtype, int64_t m, int64_t n, int64_t k, int out_dtype,
                           int scale_rule, void *y, int8_t *q_out, float *s_out, void *workspace,
                           size_t workspace_bytes, mp_stream_t stream);

/* ---------------------------------------------------------------- W8A8 MoE */

/* Routing + per-token quant (replaces npu_moe_init_routing_quant,
 * vllm_ascend.patch:2369-2379).  topk_ids int32 [T, top_k] in [0,E).
 * Outputs: routed int8 [T*top_k, H] (token copies sorted by expert, stable in
 * (token, slot) order), routed_scale fp32 [T*top_k], row_of_slot int32
 * [T*top_k] (row in routed for assignment t*top_k+j), group_offsets int64
 * [E+1] (cumulative endpoints, offsets[0] = 0).  scale_rule MP_SCALE_FP32 is the
 * runtime rule; MP_SCALE_FAKE the act_quant of SmoothQuantPackedMoeExperts.forward
 * (fake_quant.py:183) in x's dtype (fp16 / bf16).  x_dtype MP_I8: x is already
 * quantized (int8 [T, H] with fp32 scales x_scale [T], the pertoken_scale input of
 * the runtime's fused_experts, vllm_ascend.patch:4447-4468) and is routed only;
 * x_scale is ignored otherwise.  workspace >= mp_moe_route_workspace_bytes(T, H, E). */
size_t mp_moe_route_workspace_bytes(int64_t t, int64_t h, int n_experts);
int mp_moe_permute_quant(const void *x, int x_dtype, const float *x_scale, int64_t t, int64_t h,
                         const int32_t *topk_ids, int top_k, int n_experts, int scale_rule, int8_t *routed,
                         float *routed_scale, int32_t *row_of_slot, int64_t *group_offsets, void *workspace,
                         size_t workspace_bytes, mp_stream_t stream);

/* GMM1 + SwiGLU + per-row requant (replaces npu_grouped_matmul_swiglu_quant,
 * vllm_ascend.patch:2391-2398, and the C++ loop-out bridge
 * acceleration/custom_ops/qwen2_5_vl/aclnn_grouped_swiglu_out_bridge.cpp:157-273).
 * For routed row r of expert e: g = (Qx_r . W13_e^T) * sx_r * s13_e (fp32),
 * h = silu(g[:I]) * g[I:], then h -> int8 q_out [R, I] + fp32 s_out [R].
 * scale_rule MP_SCALE_FP32: h in fp32, the runtime requant.  MP_SCALE_FAKE: the
 * arithmetic of SmoothQuantPackedMoeExperts.forward (fake_quant.py:184-186) in
 * act_dtype (fp16 / bf16): gate and up = F.linear of the fake-quant tensors
 * (sum_k r(qx_k * sx) * r(w_k * s13), fp32 accumulation, rounded), silu(gate)
 * rounded, the product rounded, then the fake per-token rule.
 * No limit on I (the CANN op rejects 2I > 10240, moe_mlp.py patch). */
size_t mp_moe_gmm1_workspace_bytes(int64_t rows, int64_t inter);
int mp_i8_gemm_swiglu_requant(const int8_t *routed, const float *routed_scale, const int8_t *w13,
                              const float *s13, const int64_t *group_offsets, int n_experts,
                              int64_t rows, int64_t h, int64_t inter, int scale_rule, int act_dtype,
                              int8_t *q_out, float *s_out, void *workspace, size_t workspace_bytes,
                              mp_stream_t stream);

/* mp_i8_gemm_swiglu_requant without a workspace argument: no counterpart in the reference.
 * For callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the scratch lives in a library-owned 64 MiB device array
 * per GPU, held until the process ends; the call allocates nothing.  Shapes whose
 * mp_moe_gmm1_workspace_bytes(rows, inter) exceeds 64 MiB return MP_ERR_WORKSPACE.  Every
 * call on one GPU uses that GPU's array: calls that overlap on one GPU (other streams or
 * threads) race.  Run with the stream's device current (the array is found per device). */
int mp_i8_gemm_swiglu_requant_noalloc(const int8_t *routed, const float *routed_scale, const int8_t *w13,
                                      const float *s13, const int64_t *group_offsets, int n_experts,
                                      int64_t rows, int64_t h, int64_t inter, int scale_rule, int act_dtype,
                                      int8_t *q_out, float *s_out, mp_stream_t stream);

/* GMM2: Y_r = (Qh_r . W2_e^T) * sh_r * s2_e -> out_dtype [R, N] (fp32 for the
 * combine).  Replaces npu_grouped_matmul with per_token_scale
 * (vllm_ascend.patch:2401-2412).  scale_rule MP_SCALE_FAKE: the reference's F.linear on
 * the fake-quant tensors instead, sum_k r(qh_k * sh) * r(w_k * s2) with r the rounding to
 * act_dtype (fp16 / bf16), fp32 accumulation (fake_quant.py:187).  K % 64 == 0 for the
 * runtime rule. */
int mp_w8a8_grouped_gemm(const int8_t *q, const float *s, const int8_t *w, const float *s_w,
                         const int64_t *group_offsets, int n_experts, int64_t rows, int64_t n,
                         int64_t k, int scale_rule, int act_dtype, void *y, int out_dtype,
                         mp_stream_t stream);

/* scale_rule MP_SCALE_FP32: out[t] = sum_j topk_w[t,j] * y[row_of_slot[t*top_k+j]]
 * in fp32 in slot order, rounded once (replaces npu_moe_token_unpermute,
 * vllm_ascend.patch:2415-2419).  MP_SCALE_FAKE: the index_add_ of
 * SmoothQuantPackedMoeExperts.forward (fake_quant.py:187-189) in out_dtype r
 * (fp16 / bf16): over the token's assignments in ascending expert order,
 * out = r(out + r(r(y) * topk_w)).  y fp32 [R, H]; topk_w fp32 [T, top_k];
 * out fp16/bf16/fp32 [T, H]; top_k <= 64. */
int mp_moe_unpermute_combine(const float *y, const int32_t *row_of_slot, const float *topk_w,
                             int64_t t, int top_k, int64_t h, int scale_rule, void *out, int out_dtype,
                             mp_stream_t stream);

/* ---------------------------------------------------------------- decode-step harness kernels
 * No counterpart in the reference (attention, RoPE and the MLP activation belong
 * to vLLM's model code); they let the Llama-shaped measurement harness run one
 * greedy decode step in ~10 launches per layer around the W4A16 GEMVs.  Head dim
 * 128; KV cache per layer K, V [B, kvh, capacity, 128] fp16; *pos is the position
 * of the new token (device memory, so launches are graph-capturable). */

/* RoPE (interleaved pairs, fp16 rounding after every op) on the q and k heads of
 * qkv [B, (nh + 2 kvh) * 128]; writes q_out [B, nh, 128] and the k, v rows of
 * position *pos into the caches.  cos_t / sin_t: fp16 [capacity, 64].  A position
 * outside [0, capacity) writes nothing. */
int mp_decode_rope_append(const void *qkv, int64_t batch, int nh, int kvh, int head_dim, const void *cos_t,
                          const void *sin_t, const int64_t *pos, int64_t capacity, void *q_out, void *k_cache,
                          void *v_cache, mp_stream_t stream);

/* Prefill counterpart of mp_decode_rope_append for positions 0 .. t_len - 1: qkv is
 * [B * t_len, (nh + 2 kvh) * 128] (token rows of each sequence in order); writes the
 * rotated queries q_out [B, nh, t_len, 128] and the rotated keys and the values into
 * the caches [B, kvh, capacity, 128] at positions 0 .. t_len - 1 (t_len <= capacity).
 * 16-byte aligned buffers; cos_t / sin_t fp16 [capacity, 64], 8-byte aligned. */
int mp_prefill_rope_split(const void *qkv, int64_t batch, int64_t t_len, int nh, int kvh, int head_dim,
                          const void *cos_t, const void *sin_t, int64_t capacity, void *q_out, void *k_cache,
                          void *v_cache, mp_stream_t stream);

/* Split-K decode attention (flash decoding) over positions [0, *pos] of one
 * layer's cache: out [B, nh, 128] fp16 = softmax(q k^T * scale) v, fp32 inside;
 * nh / kvh in {1, 2, 4, 8}.  splits workgroups per (row, kv head), each over
 * ceil(capacity / splits) positions (splits <= 1024), then a merge launch when
 * splits > 1.  workspace of mp_decode_attention_workspace_bytes(batch, nh,
 * splits), 16-byte aligned; calls that share a workspace must not overlap. */
size_t mp_decode_attention_workspace_bytes(int64_t batch, int nh, int splits);
int mp_decode_attention(const void *q, int64_t batch, int nh, int kvh, int head_dim, const void *k_cache,
                        const void *v_cache, const int64_t *pos, int64_t capacity, int splits, float scale,
                        void *out, void *workspace, size_t workspace_bytes, mp_stream_t stream);

/* mp_decode_rope_append followed by mp_decode_attention in one launch: the
 * queries are rotated from qkv [B, (nh + 2 kvh) * 128] in registers and the
 * workgroup whose split holds *pos appends the rotated key and the value before
 * it scores.  A position outside [0, capacity) appends nothing and gives zeros.
 * cos_t / sin_t fp16 [capacity, 64], 8-byte aligned; workspace as above. */
int mp_decode_rope_attention(const void *qkv, int64_t batch, int nh, int kvh, int head_dim, const void *cos_t,
                             const void *sin_t, const int64_t *pos, int64_t capacity, void *k_cache, void *v_cache,
                             int splits, float scale, void *out, void *workspace, size_t workspace_bytes,
                             mp_stream_t stream);

/* idx [rows] int64 = the first index of the maximum of each row of x [rows, n] fp16 (a NaN
 * counts as the maximum): the greedy sampling step of the decode harness, torch.argmax's
 * rules.  No counterpart in the reference. */
int mp_argmax_rows(const void *x, int64_t rows, int64_t n, int64_t *idx, mp_stream_t stream);

/* act [rows, I] = round(round(silu(gate)) * up) of gate_up [rows, 2I] (gate | up), in dtype
 * (MP_F16 / MP_BF16; every round is to that dtype). */
int mp_silu_mul(const void *gate_up, int64_t rows, int64_t inter, void *act, int dtype, mp_stream_t stream);

/* ---- SmoothQuant smoothing (offline) ----
 * colmax [k] fp32 = max(colmax, max over rows |x[r, :]|) for x [rows, k] row-major (fp16 / bf16 /
 * fp32, 16-byte aligned): the per-input-channel abs-max statistic of get_act_scales
 * (smoothquant/calibration.py:27-58) over a calibration batch, and the weight statistic
 * w_j = max_n |W_nj| of _compute_smooth_scales (smooth.py:16-20) over every fc sharing a norm.
 * accumulate = 0 starts from zeros; 1 keeps the running maxima (several fcs / batches).  Exact. */
int mp_colmax_abs(const void *x, int dtype, int64_t rows, int64_t k, int accumulate, float *colmax,
                  mp_stream_t stream);

/* scales [k] in dtype = (a^alpha / w^(1-alpha)).clamp(1e-5) of _compute_smooth_scales
 * (smooth.py:7-25): a = act_max cast to dtype, w = w_colmax clamped at 1e-5, every op rounded to
 * dtype, with the fp32 powers correctly rounded (square roots at alpha = 0.5, as torch's pow).  alpha
 * is a double, as the Python scalar is: the exponents are (float)alpha and (float)(1 - alpha), the
 * values torch applies. */
int mp_smooth_scales(const float *act_max, const float *w_colmax, int64_t k, double alpha, int dtype, void *scales,
                     mp_stream_t stream);

/* In place w[r, j] = w[r, j] * scales[j] (divide = 0: fc.weight.mul_(s.view(1, -1))) or
 * w[r, j] / scales[j] (divide = 1: ln.weight.div_(s), rows = 1), rounded to dtype
 * (smooth_ln_fcs_llama_like, smooth.py:91-101). */
int mp_scale_columns(void *w, int dtype, int64_t rows, int64_t k, const void *scales, int divide, mp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MINDPIPE_AMD_H */
