/*
 * lf_oracle.h - CPU correctness oracle for the FP8 projection path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (lunaflux_amd, liblunaflux_hip.so, the gfx950 code object) never
 * links, loads or calls it, and has no CPU fallback through it.
 *
 * Part 1 restates LunaFlux's MoonBit reference kernels
 * (/root/reference/kernels/reference) in C99:
 *   lfo_decode_bfloat16_le   <- kernels/reference/bfloat16.mbt:6-30
 *   lfo_project_values       <- kernels/reference/basic.mbt:71-98
 *   lfo_dense_projection     <- kernels/reference/basic.mbt:102-109
 *   lfo_qkv_projection       <- kernels/reference/basic.mbt:113-153
 *   lfo_silu_gated_mlp       <- kernels/reference/mlp.mbt:4-39
 *   lfo_rms_norm             <- kernels/reference/basic.mbt:32-68
 *   lfo_checked_element_count<- kernels/reference/limits.mbt:47-90
 * Numeric contract (kernels/reference/README.mbt.md:7-18): binary32 values,
 * sequential-K fp32 accumulation with separate multiply and add (this file is
 * compiled with -ffp-contract=off and without fast-math), non-finite inputs
 * and computed values rejected, outputs not rounded to bf16, weights stored
 * [output_width, input_width] row-major, Q|K|V concatenated in that order.
 *
 * Part 2 extends the oracle with what the reference does not have (there is
 * no FP8, quantization or MoE code in /root/reference): OCP E4M3 decode and
 * RNE-satfinite encode, bf16 RNE rounding, per-channel / 128x128-block weight
 * scales, per-token / per-token-per-group activation quantization, and the
 * MoE router, stable sort, grouped MLP and top-k combine. Every FP8 result
 * is defined as the reference's fp32 arithmetic applied to the dequantized
 * values (fp32(q) * s, one fp32 multiply).
 */
#ifndef LF_ORACLE_H
#define LF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. Part 1 codes mirror ReferenceKernelError
 * (kernels/reference/errors.mbt:43-52). */
enum lfo_status {
  LFO_OK = 0,
  LFO_INVALID_LIMIT = 1,
  LFO_LIMIT_EXCEEDED = 2,
  LFO_INVALID_SHAPE = 3,
  LFO_INVALID_SCALAR = 4,
  LFO_ARITHMETIC_OVERFLOW = 5,
  LFO_NON_FINITE = 6
};

/* Caller-owned allocation ceiling (kernels/reference/limits.mbt:7-13). A
 * NULL limits pointer means "no ceiling beyond int32 element counts". */
typedef struct lfo_limits {
  int32_t max_rows;
  int32_t max_columns;
  int32_t max_elements;
} lfo_limits;

int32_t lfo_limits_new(int32_t max_rows, int32_t max_columns,
                       int32_t max_elements, lfo_limits *out);
int32_t lfo_checked_element_count(int32_t rows, int32_t columns,
                                  const lfo_limits *limits, int32_t *out);

/* ---- Part 1: restated reference kernels -------------------------------- */

int32_t lfo_decode_bfloat16_le(const uint8_t *bytes, int64_t byte_count,
                               int32_t rows, int32_t columns,
                               const lfo_limits *limits, float *out);
/* out[r, n] = sum_{k=0..K-1} x[r, k] * w[n, k], k ascending, fp32. */
int32_t lfo_project_values(const float *x, int32_t rows, int32_t in_width,
                           const float *w, int32_t out_width,
                           int32_t w_columns, const lfo_limits *limits,
                           float *out);
int32_t lfo_dense_projection(const float *x, int32_t rows, int32_t in_width,
                             const float *w, int32_t out_width,
                             int32_t w_columns, const lfo_limits *limits,
                             float *out);
int32_t lfo_qkv_projection(const float *x, int32_t rows, int32_t in_width,
                           const float *wq, int32_t q_rows,
                           const float *wk, int32_t k_rows,
                           const float *wv, int32_t v_rows,
                           const lfo_limits *limits, float *out);
/* down(silu(gate(x)) * up(x)); if hidden_out is non-NULL the fp32 SiLU
 * product h [rows, inter] is also returned. round_hidden_bf16 != 0 rounds h
 * to bf16 (RNE) before the down projection; the reference keeps h in fp32
 * (mlp.mbt:27-31), so 0 is the reference semantics and 1 mirrors a device
 * pipeline that stores h as bf16 between two launches. */
int32_t lfo_silu_gated_mlp(const float *x, int32_t rows, int32_t hidden,
                           const float *wg, const float *wu, int32_t inter,
                           const float *wd, int32_t round_hidden_bf16,
                           const lfo_limits *limits, float *hidden_out,
                           float *out);
/* Row-wise RMS normalization: w is the [1, columns] norm weight; sequential
 * fp32 sum of squares, out = x * (1 / sqrt(sum / columns + epsilon)) * w. */
int32_t lfo_rms_norm(const float *x, int32_t rows, int32_t columns,
                     const float *w, int32_t w_rows, int32_t w_columns,
                     float epsilon, const lfo_limits *limits, float *out);
/* SiLU product for one element: g / (1 + expf(-g)) * u (mlp.mbt:30). */
float lfo_silu_mul(float g, float u);
/* out[i] = lfo_silu_mul(g[i], u[i]) for i < n. */
void lfo_silu_mul_array(const float *g, const float *u, int64_t n, float *out);

/* ---- Part 2: formats and quantizers ------------------------------------ */

uint16_t lfo_bf16_rne(float value);          /* fp32 -> bf16 bits, RNE  */
float lfo_bf16_to_f32(uint16_t bits);
void lfo_bf16_round_array(const float *in, int64_t n, uint16_t *out);
void lfo_bf16_decode_array(const uint16_t *in, int64_t n, float *out);

float lfo_e4m3_decode(uint8_t code);          /* OCP E4M3FN closed form  */
uint8_t lfo_e4m3_encode(float value);         /* RNE, saturate to +-448  */
void lfo_e4m3_encode_array(const float *in, int64_t n, uint8_t *out);
void lfo_e4m3_decode_array(const uint8_t *in, int64_t n, float *out);

/* Row quantizer used for weights (rows = output channels) and activations
 * (rows = tokens). For each row r and each K-group g of width `group`
 * (group == columns means one scale per row):
 *   amax = max |x[r, k]| over the group
 *   amax == 0: q = 0, scale = 0
 *   else:      ratio = 448 / amax, q = e4m3_rne_sat(x * ratio),
 *              scale = amax / 448
 * scales has rows * (columns / group) entries, row-major. */
int32_t lfo_quantize_rows(const float *x, int32_t rows, int32_t columns,
                          int32_t group, uint8_t *q, float *scales);
/* Same formula with the amax taken over square `block` x `block` tiles;
 * scales is [ceil(rows/block), ceil(columns/block)] row-major. */
int32_t lfo_quantize_blocks(const float *w, int32_t rows, int32_t columns,
                            int32_t block, uint8_t *q, float *scales);
/* fp32(q) * scale, the dequantized value every FP8 oracle result uses.
 * scale_mode 0: scales [rows]; 1: scales [rows, columns/group];
 * 2: scales [ceil(rows/group), ceil(columns/group)]. */
int32_t lfo_dequantize(const uint8_t *q, const float *scales, int32_t rows,
                       int32_t columns, int32_t scale_mode, int32_t group,
                       float *out);

/* ---- Part 2: MoE ------------------------------------------------------- */

enum lfo_route_mode {
  LFO_ROUTE_TOPK_SOFTMAX = 0,  /* top-k logits, softmax over the k picked */
  LFO_ROUTE_SOFTMAX_TOPK = 1   /* softmax over all experts, keep top-k   */
};
/* experts/weights are [tokens, k]; j-th pick is the j-th largest logit,
 * ties broken toward the lower expert id. */
int32_t lfo_route_topk(const float *logits, int32_t tokens, int32_t experts,
                       int32_t k, int32_t mode, int32_t *topk_experts,
                       float *topk_weights);
/* Stable counting sort of the tokens*k assignments a = t*k + j by expert.
 * sorted_assignments[p] = a, offsets[e] = first position of expert e,
 * offsets[experts] = tokens*k. */
int32_t lfo_moe_sort(const int32_t *topk_experts, int32_t tokens, int32_t k,
                     int32_t experts, int32_t *sorted_assignments,
                     int32_t *offsets);
/* Grouped SiLU MLP over dequantized expert weights and (optionally
 * quantized) activations. wg/wu: [E, inter, hidden], wd: [E, hidden, inter]
 * already dequantized fp32. x: [tokens, hidden] fp32 values (dequantized if
 * the caller quantized them). For each assignment a (token t, pick j):
 *   h_a = silu(x_t Wg_e^T) * (x_t Wu_e^T)               (fp32, per element)
 *   h_a is passed through `hidden_transform`, a bit set: bit 0 rounds h_a
 *   to bf16 (RNE); bits 1-2 then quantize-dequantize it to e4m3 with the
 *   lfo_quantize_rows formula (1: one scale per row, 2: one scale per 128
 *   columns). 0 keeps the fp32 h_a of the reference MLP (mlp.mbt:27-31).
 *   y_a = h_a Wd_e^T                                     (fp32; bit 3 of
 *   hidden_transform rounds it to bf16 (RNE), as a device that stores y in
 *   bf16 between the down GEMM and the combine)
 *   out_t = sum_j w_tj * y_(t,j), j ascending, fp32.
 * out is [tokens, hidden] fp32. */
int32_t lfo_moe_mlp(const float *x, int32_t tokens, int32_t hidden,
                    const float *wg, const float *wu, const float *wd,
                    int32_t experts, int32_t inter,
                    const int32_t *topk_experts, const float *topk_weights,
                    int32_t k, int32_t hidden_transform, int32_t threads,
                    float *out);

/* ---- Multithreaded projection (CPU baseline) --------------------------- */
/* Same per-element arithmetic as lfo_project_values; output elements are
 * split across `threads` POSIX threads. rows_limit restricts the work to
 * the first rows_limit rows (the CPU baseline times a bounded sample). */
int32_t lfo_project_values_mt(const float *x, int32_t rows, int32_t in_width,
                              const float *w, int32_t out_width,
                              int32_t threads, float *out);

#ifdef __cplusplus
}
#endif

#endif
