/*
 * lf_oracle.c - CPU correctness oracle (test infrastructure only; see
 * lf_oracle.h for the contract and the reference lines each function
 * restates). Build flags (oracle/Makefile): -O2 -ffp-contract=off, no
 * fast-math, so every fp32 multiply and add is a separately rounded IEEE
 * binary32 operation, as the reference's Float arithmetic is.
 */
#include "lf_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float v) {
  uint32_t u;
  memcpy(&u, &v, sizeof(u));
  return u;
}

static float bits_f32(uint32_t u) {
  float v;
  memcpy(&v, &u, sizeof(v));
  return v;
}

static int finite_f32(float v) { return !(isnan(v) || isinf(v)); }

/* kernels/reference/limits.mbt:16-31 */
int32_t lfo_limits_new(int32_t max_rows, int32_t max_columns,
                       int32_t max_elements, lfo_limits *out) {
  if (max_rows <= 0 || max_columns <= 0 || max_elements <= 0) {
    return LFO_INVALID_LIMIT;
  }
  out->max_rows = max_rows;
  out->max_columns = max_columns;
  out->max_elements = max_elements;
  return LFO_OK;
}

/* kernels/reference/limits.mbt:49-76 */
int32_t lfo_checked_element_count(int32_t rows, int32_t columns,
                                  const lfo_limits *limits, int32_t *out) {
  if (rows <= 0 || columns <= 0) return LFO_INVALID_SHAPE;
  if (limits != NULL) {
    if (rows > limits->max_rows) return LFO_LIMIT_EXCEEDED;
    if (columns > limits->max_columns) return LFO_LIMIT_EXCEEDED;
  }
  int64_t elements = (int64_t)rows * (int64_t)columns;
  if (limits != NULL && elements > (int64_t)limits->max_elements) {
    return LFO_LIMIT_EXCEEDED;
  }
  if (elements > 2147483647LL) return LFO_ARITHMETIC_OVERFLOW;
  *out = (int32_t)elements;
  return LFO_OK;
}

/* kernels/reference/bfloat16.mbt:6-30: each little-endian code unit is the
 * high half of a binary32; NaN and infinity are rejected. */
int32_t lfo_decode_bfloat16_le(const uint8_t *bytes, int64_t byte_count,
                               int32_t rows, int32_t columns,
                               const lfo_limits *limits, float *out) {
  int32_t elements = 0;
  int32_t status = lfo_checked_element_count(rows, columns, limits, &elements);
  if (status != LFO_OK) return status;
  if (byte_count != (int64_t)elements * 2) return LFO_INVALID_SHAPE;
  for (int32_t i = 0; i < elements; i += 1) {
    uint32_t low = bytes[2 * i];
    uint32_t high = bytes[2 * i + 1];
    float v = bits_f32(((high << 8) | low) << 16);
    if (!finite_f32(v)) return LFO_NON_FINITE;
    out[i] = v;
  }
  return LFO_OK;
}

/* kernels/reference/basic.mbt:71-98. One output element at a time, the
 * accumulator starts at 0.0 and adds x[k] * w[k] for k = 0, 1, ..., K-1.
 * A NaN or infinite accumulator is rejected (basic.mbt:91-93). */
int32_t lfo_project_values(const float *x, int32_t rows, int32_t in_width,
                           const float *w, int32_t out_width,
                           int32_t w_columns, const lfo_limits *limits,
                           float *out) {
  if (w_columns != in_width) return LFO_INVALID_SHAPE;
  int32_t elements = 0;
  int32_t status = lfo_checked_element_count(rows, out_width, limits,
                                             &elements);
  if (status != LFO_OK) return status;
  for (int32_t r = 0; r < rows; r += 1) {
    const float *xr = x + (int64_t)r * in_width;
    for (int32_t n = 0; n < out_width; n += 1) {
      const float *wn = w + (int64_t)n * w_columns;
      float acc = 0.0f;
      for (int32_t k = 0; k < in_width; k += 1) {
        float product = xr[k] * wn[k];
        acc = acc + product;
      }
      if (!finite_f32(acc)) return LFO_NON_FINITE;
      out[(int64_t)r * out_width + n] = acc;
    }
  }
  return LFO_OK;
}

/* kernels/reference/basic.mbt:102-109 (also language_model_head :175-181) */
int32_t lfo_dense_projection(const float *x, int32_t rows, int32_t in_width,
                             const float *w, int32_t out_width,
                             int32_t w_columns, const lfo_limits *limits,
                             float *out) {
  return lfo_project_values(x, rows, in_width, w, out_width, w_columns,
                            limits, out);
}

/* kernels/reference/basic.mbt:113-153: three projections, then each output
 * row is [Q | K | V]. K and V must have the same width. */
int32_t lfo_qkv_projection(const float *x, int32_t rows, int32_t in_width,
                           const float *wq, int32_t q_rows,
                           const float *wk, int32_t k_rows,
                           const float *wv, int32_t v_rows,
                           const lfo_limits *limits, float *out) {
  if (k_rows != v_rows) return LFO_INVALID_SHAPE;
  if (q_rows < 0 || k_rows < 0 || q_rows > 2147483647 - k_rows) {
    return LFO_ARITHMETIC_OVERFLOW;
  }
  int32_t qk = q_rows + k_rows;
  if (qk > 2147483647 - v_rows) return LFO_ARITHMETIC_OVERFLOW;
  int32_t width = qk + v_rows;
  int32_t elements = 0;
  int32_t status = lfo_checked_element_count(rows, width, limits, &elements);
  if (status != LFO_OK) return status;
  float *q = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)q_rows);
  float *k = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)k_rows);
  float *v = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)v_rows);
  if (q == NULL || k == NULL || v == NULL) {
    free(q);
    free(k);
    free(v);
    return LFO_ARITHMETIC_OVERFLOW;
  }
  status = lfo_project_values(x, rows, in_width, wq, q_rows, in_width,
                              limits, q);
  if (status == LFO_OK) {
    status = lfo_project_values(x, rows, in_width, wk, k_rows, in_width,
                                limits, k);
  }
  if (status == LFO_OK) {
    status = lfo_project_values(x, rows, in_width, wv, v_rows, in_width,
                                limits, v);
  }
  if (status == LFO_OK) {
    for (int32_t r = 0; r < rows; r += 1) {
      float *o = out + (int64_t)r * width;
      memcpy(o, q + (int64_t)r * q_rows, sizeof(float) * (size_t)q_rows);
      memcpy(o + q_rows, k + (int64_t)r * k_rows,
             sizeof(float) * (size_t)k_rows);
      memcpy(o + qk, v + (int64_t)r * v_rows, sizeof(float) * (size_t)v_rows);
    }
  }
  free(q);
  free(k);
  free(v);
  return status;
}

/* kernels/reference/mlp.mbt:30: gate / (1 + expf(-gate)) * up, left to
 * right in binary32. */
float lfo_silu_mul(float g, float u) {
  float denominator = 1.0f + expf(-g);
  float s = g / denominator;
  return s * u;
}

void lfo_silu_mul_array(const float *g, const float *u, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i += 1) out[i] = lfo_silu_mul(g[i], u[i]);
}

/* kernels/reference/basic.mbt:32-68: the weight must be one row of the
 * input's width (InvalidShape(NormalizationWeight)); epsilon must be finite
 * (NonFinite(Epsilon)) and > 0 (InvalidScalar(Epsilon)); per row the sum of
 * squares in ascending column order (a non-finite sum is
 * NonFinite(ComputedValue)), inverse_rms = 1 / sqrt(sum / width + epsilon),
 * out = x * inverse_rms * w evaluated left to right; a non-finite output is
 * NonFinite(ComputedValue) (values.mbt:117-133). sqrtf is the correctly
 * rounded IEEE square root. */
int32_t lfo_rms_norm(const float *x, int32_t rows, int32_t columns,
                     const float *w, int32_t w_rows, int32_t w_columns,
                     float epsilon, const lfo_limits *limits, float *out) {
  if (w_rows != 1 || w_columns != columns) return LFO_INVALID_SHAPE;
  if (!finite_f32(epsilon)) return LFO_NON_FINITE;
  if (epsilon <= 0.0f) return LFO_INVALID_SCALAR;
  int32_t elements = 0;
  int32_t st = lfo_checked_element_count(rows, columns, limits, &elements);
  if (st != LFO_OK) return st;
  const float width = (float)columns;
  for (int32_t r = 0; r < rows; r += 1) {
    const float *xr = x + (int64_t)r * columns;
    float square_sum = 0.0f;
    for (int32_t c = 0; c < columns; c += 1) {
      float square = xr[c] * xr[c];
      square_sum = square_sum + square;
    }
    if (!finite_f32(square_sum)) return LFO_NON_FINITE;
    float inverse_rms = 1.0f / sqrtf(square_sum / width + epsilon);
    for (int32_t c = 0; c < columns; c += 1) {
      float v = xr[c] * inverse_rms;
      v = v * w[c];
      if (!finite_f32(v)) return LFO_NON_FINITE;
      out[(int64_t)r * columns + c] = v;
    }
  }
  return LFO_OK;
}

/* kernels/reference/mlp.mbt:4-39 */
int32_t lfo_silu_gated_mlp(const float *x, int32_t rows, int32_t hidden,
                           const float *wg, const float *wu, int32_t inter,
                           const float *wd, int32_t round_hidden_bf16,
                           const lfo_limits *limits, float *hidden_out,
                           float *out) {
  int32_t elements = 0;
  int32_t status = lfo_checked_element_count(rows, inter, limits, &elements);
  if (status != LFO_OK) return status;
  float *g = (float *)malloc(sizeof(float) * (size_t)elements);
  float *u = (float *)malloc(sizeof(float) * (size_t)elements);
  if (g == NULL || u == NULL) {
    free(g);
    free(u);
    return LFO_ARITHMETIC_OVERFLOW;
  }
  status = lfo_project_values(x, rows, hidden, wg, inter, hidden, limits, g);
  if (status == LFO_OK) {
    status = lfo_project_values(x, rows, hidden, wu, inter, hidden, limits, u);
  }
  if (status == LFO_OK) {
    for (int32_t i = 0; i < elements; i += 1) {
      float h = lfo_silu_mul(g[i], u[i]);
      if (!finite_f32(h)) {
        status = LFO_NON_FINITE;
        break;
      }
      if (round_hidden_bf16) h = lfo_bf16_to_f32(lfo_bf16_rne(h));
      g[i] = h;
    }
  }
  if (status == LFO_OK && hidden_out != NULL) {
    memcpy(hidden_out, g, sizeof(float) * (size_t)elements);
  }
  if (status == LFO_OK) {
    status = lfo_project_values(g, rows, inter, wd, hidden, inter, limits,
                                out);
  }
  free(g);
  free(u);
  return status;
}

/* ---- formats ------------------------------------------------------------ */

/* IEEE round-to-nearest-even of the low 16 bits; NaN stays a quiet NaN and
 * values past the largest finite bf16 round to infinity. */
uint16_t lfo_bf16_rne(float value) {
  uint32_t u = f32_bits(value);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float lfo_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

void lfo_bf16_round_array(const float *in, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; i += 1) out[i] = lfo_bf16_rne(in[i]);
}

void lfo_bf16_decode_array(const uint16_t *in, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i += 1) out[i] = lfo_bf16_to_f32(in[i]);
}

/* OCP 8-bit floating point, E4M3 variant: sign, 4 exponent bits (bias 7), 3
 * mantissa bits, no infinities, S.1111.111 is NaN, largest finite 448,
 * subnormals m * 2^-9. */
float lfo_e4m3_decode(uint8_t code) {
  int exponent = (code >> 3) & 15;
  int mantissa = code & 7;
  float v;
  if (exponent == 15 && mantissa == 7) {
    v = NAN;
  } else if (exponent == 0) {
    v = ldexpf((float)mantissa, -9);
  } else {
    v = ldexpf((float)(8 + mantissa), exponent - 10);
  }
  return (code & 0x80) ? -v : v;
}

/* Round to nearest, ties to even, saturating: every finite |v| >= 448 and
 * infinity map to +-448; NaN maps to the NaN code; the sign of zero is kept. */
uint8_t lfo_e4m3_encode(float value) {
  uint32_t u = f32_bits(value);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu); /* >= 448 */
  if (a < 0x3c800000u) {                                 /* < 2^-6  */
    /* Subnormal grid step 2^-9: scale by 512 (exact) and round the result
     * (0 <= m < 8) to an integer with ties to even. */
    float m = bits_f32(a) * 512.0f;
    float r = (m + 8388608.0f) - 8388608.0f;
    return (uint8_t)(sign | (uint8_t)r);
  }
  uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  r &= 0xfff00000u;
  int32_t exponent = (int32_t)(r >> 23) - 127 + 7;
  uint32_t mantissa = (r >> 20) & 7u;
  return (uint8_t)(sign | (uint8_t)(((uint32_t)exponent << 3) | mantissa));
}

void lfo_e4m3_encode_array(const float *in, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; i += 1) out[i] = lfo_e4m3_encode(in[i]);
}

void lfo_e4m3_decode_array(const uint8_t *in, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i += 1) out[i] = lfo_e4m3_decode(in[i]);
}

static void quantize_span(const float *x, int64_t count, int64_t stride,
                          int64_t run, uint8_t *q, float *scale) {
  /* `count` runs of `run` contiguous values, `stride` apart. */
  float amax = 0.0f;
  for (int64_t i = 0; i < count; i += 1) {
    for (int64_t j = 0; j < run; j += 1) {
      float a = fabsf(x[i * stride + j]);
      if (a > amax) amax = a;
    }
  }
  if (amax == 0.0f) {
    for (int64_t i = 0; i < count; i += 1) {
      memset(q + i * stride, 0, (size_t)run);
    }
    *scale = 0.0f;
    return;
  }
  float ratio = 448.0f / amax;
  for (int64_t i = 0; i < count; i += 1) {
    for (int64_t j = 0; j < run; j += 1) {
      float scaled = x[i * stride + j] * ratio;
      q[i * stride + j] = lfo_e4m3_encode(scaled);
    }
  }
  *scale = amax / 448.0f;
}

int32_t lfo_quantize_rows(const float *x, int32_t rows, int32_t columns,
                          int32_t group, uint8_t *q, float *scales) {
  if (rows <= 0 || columns <= 0 || group <= 0 || columns % group != 0) {
    return LFO_INVALID_SHAPE;
  }
  int32_t groups = columns / group;
  for (int32_t r = 0; r < rows; r += 1) {
    for (int32_t g = 0; g < groups; g += 1) {
      int64_t base = (int64_t)r * columns + (int64_t)g * group;
      quantize_span(x + base, 1, 0, group, q + base,
                    scales + (int64_t)r * groups + g);
    }
  }
  return LFO_OK;
}

int32_t lfo_quantize_blocks(const float *w, int32_t rows, int32_t columns,
                            int32_t block, uint8_t *q, float *scales) {
  if (rows <= 0 || columns <= 0 || block <= 0) return LFO_INVALID_SHAPE;
  int32_t row_blocks = (rows + block - 1) / block;
  int32_t col_blocks = (columns + block - 1) / block;
  for (int32_t rb = 0; rb < row_blocks; rb += 1) {
    for (int32_t cb = 0; cb < col_blocks; cb += 1) {
      int32_t r0 = rb * block;
      int32_t c0 = cb * block;
      int32_t nr = rows - r0 < block ? rows - r0 : block;
      int32_t nc = columns - c0 < block ? columns - c0 : block;
      int64_t base = (int64_t)r0 * columns + c0;
      quantize_span(w + base, nr, columns, nc, q + base,
                    scales + (int64_t)rb * col_blocks + cb);
    }
  }
  return LFO_OK;
}

int32_t lfo_dequantize(const uint8_t *q, const float *scales, int32_t rows,
                       int32_t columns, int32_t scale_mode, int32_t group,
                       float *out) {
  if (rows <= 0 || columns <= 0) return LFO_INVALID_SHAPE;
  if (scale_mode != 0 && group <= 0) return LFO_INVALID_SHAPE;
  if (scale_mode == 1 && columns % group != 0) return LFO_INVALID_SHAPE;
  int32_t groups = scale_mode == 1 ? columns / group : 0;
  int32_t col_blocks = scale_mode == 2 ? (columns + group - 1) / group : 0;
  for (int32_t r = 0; r < rows; r += 1) {
    for (int32_t c = 0; c < columns; c += 1) {
      float s;
      if (scale_mode == 0) {
        s = scales[r];
      } else if (scale_mode == 1) {
        s = scales[(int64_t)r * groups + c / group];
      } else if (scale_mode == 2) {
        s = scales[(int64_t)(r / group) * col_blocks + c / group];
      } else {
        return LFO_INVALID_SHAPE;
      }
      int64_t i = (int64_t)r * columns + c;
      out[i] = lfo_e4m3_decode(q[i]) * s;
    }
  }
  return LFO_OK;
}

/* ---- MoE ----------------------------------------------------------------- */

int32_t lfo_route_topk(const float *logits, int32_t tokens, int32_t experts,
                       int32_t k, int32_t mode, int32_t *topk_experts,
                       float *topk_weights) {
  if (tokens <= 0 || experts <= 0 || k <= 0 || k > experts || k > 64) {
    return LFO_INVALID_SHAPE;
  }
  if (mode != LFO_ROUTE_TOPK_SOFTMAX && mode != LFO_ROUTE_SOFTMAX_TOPK) {
    return LFO_INVALID_SCALAR;
  }
  for (int32_t t = 0; t < tokens; t += 1) {
    const float *l = logits + (int64_t)t * experts;
    for (int32_t e = 0; e < experts; e += 1) {
      if (!finite_f32(l[e])) return LFO_NON_FINITE;
    }
    int32_t picked[64];
    for (int32_t j = 0; j < k; j += 1) {
      int32_t best = -1;
      for (int32_t e = 0; e < experts; e += 1) {
        int taken = 0;
        for (int32_t i = 0; i < j; i += 1) taken |= picked[i] == e;
        if (taken) continue;
        /* strict '>' keeps the lowest id among equal logits */
        if (best < 0 || l[e] > l[best]) best = e;
      }
      picked[j] = best;
      topk_experts[(int64_t)t * k + j] = best;
    }
    float top = l[picked[0]];
    if (mode == LFO_ROUTE_TOPK_SOFTMAX) {
      float sum = 0.0f;
      for (int32_t j = 0; j < k; j += 1) sum += expf(l[picked[j]] - top);
      for (int32_t j = 0; j < k; j += 1) {
        topk_weights[(int64_t)t * k + j] = expf(l[picked[j]] - top) / sum;
      }
    } else {
      float sum = 0.0f;
      for (int32_t e = 0; e < experts; e += 1) sum += expf(l[e] - top);
      for (int32_t j = 0; j < k; j += 1) {
        topk_weights[(int64_t)t * k + j] = expf(l[picked[j]] - top) / sum;
      }
    }
  }
  return LFO_OK;
}

int32_t lfo_moe_sort(const int32_t *topk_experts, int32_t tokens, int32_t k,
                     int32_t experts, int32_t *sorted_assignments,
                     int32_t *offsets) {
  if (tokens <= 0 || k <= 0 || experts <= 0) return LFO_INVALID_SHAPE;
  int64_t total = (int64_t)tokens * k;
  if (total > 2147483647LL) return LFO_ARITHMETIC_OVERFLOW;
  int32_t *cursor = (int32_t *)calloc((size_t)experts + 1, sizeof(int32_t));
  if (cursor == NULL) return LFO_ARITHMETIC_OVERFLOW;
  for (int64_t a = 0; a < total; a += 1) {
    int32_t e = topk_experts[a];
    if (e < 0 || e >= experts) {
      free(cursor);
      return LFO_INVALID_SHAPE;
    }
    cursor[e + 1] += 1;
  }
  for (int32_t e = 0; e < experts; e += 1) cursor[e + 1] += cursor[e];
  memcpy(offsets, cursor, sizeof(int32_t) * ((size_t)experts + 1));
  for (int64_t a = 0; a < total; a += 1) {
    int32_t e = topk_experts[a];
    sorted_assignments[cursor[e]] = (int32_t)a;
    cursor[e] += 1;
  }
  free(cursor);
  return LFO_OK;
}

static void transform_hidden(float *h, int32_t inter, int32_t transform) {
  if (transform & 1) {
    for (int32_t i = 0; i < inter; i += 1) {
      h[i] = lfo_bf16_to_f32(lfo_bf16_rne(h[i]));
    }
  }
  int32_t quant = (transform >> 1) & 3;
  if (quant == 0) return;
  int32_t group = quant == 1 ? inter : 128;
  for (int32_t g0 = 0; g0 < inter; g0 += group) {
    int32_t n = inter - g0 < group ? inter - g0 : group;
    float amax = 0.0f;
    for (int32_t i = 0; i < n; i += 1) {
      float a = fabsf(h[g0 + i]);
      if (a > amax) amax = a;
    }
    if (amax == 0.0f) {
      for (int32_t i = 0; i < n; i += 1) h[g0 + i] = 0.0f;
      continue;
    }
    float ratio = 448.0f / amax;
    float scale = amax / 448.0f;
    for (int32_t i = 0; i < n; i += 1) {
      uint8_t c = lfo_e4m3_encode(h[g0 + i] * ratio);
      h[g0 + i] = lfo_e4m3_decode(c) * scale;
    }
  }
}

typedef struct moe_job {
  const float *x;
  int32_t hidden, inter, k, transform;
  const float *wg, *wu, *wd;
  const int32_t *topk_experts;
  float *y; /* [tokens * k, hidden] */
  int64_t first, last;
  int32_t status;
} moe_job;

static void *moe_worker(void *arg) {
  moe_job *job = (moe_job *)arg;
  float *h = (float *)malloc(sizeof(float) * (size_t)job->inter);
  if (h == NULL) {
    job->status = LFO_ARITHMETIC_OVERFLOW;
    return NULL;
  }
  for (int64_t a = job->first; a < job->last; a += 1) {
    int32_t t = (int32_t)(a / job->k);
    int32_t e = job->topk_experts[a];
    const float *xt = job->x + (int64_t)t * job->hidden;
    const float *wg = job->wg + (int64_t)e * job->inter * job->hidden;
    const float *wu = job->wu + (int64_t)e * job->inter * job->hidden;
    const float *wd = job->wd + (int64_t)e * job->hidden * job->inter;
    for (int32_t i = 0; i < job->inter; i += 1) {
      float g = 0.0f;
      float u = 0.0f;
      const float *gi = wg + (int64_t)i * job->hidden;
      const float *ui = wu + (int64_t)i * job->hidden;
      for (int32_t c = 0; c < job->hidden; c += 1) {
        float pg = xt[c] * gi[c];
        g = g + pg;
      }
      for (int32_t c = 0; c < job->hidden; c += 1) {
        float pu = xt[c] * ui[c];
        u = u + pu;
      }
      h[i] = lfo_silu_mul(g, u);
    }
    transform_hidden(h, job->inter, job->transform);
    float *ya = job->y + a * job->hidden;
    for (int32_t n = 0; n < job->hidden; n += 1) {
      const float *dn = wd + (int64_t)n * job->inter;
      float acc = 0.0f;
      for (int32_t i = 0; i < job->inter; i += 1) {
        float p = h[i] * dn[i];
        acc = acc + p;
      }
      ya[n] = (job->transform & 8) ? lfo_bf16_to_f32(lfo_bf16_rne(acc)) : acc;
    }
  }
  free(h);
  job->status = LFO_OK;
  return NULL;
}

int32_t lfo_moe_mlp(const float *x, int32_t tokens, int32_t hidden,
                    const float *wg, const float *wu, const float *wd,
                    int32_t experts, int32_t inter,
                    const int32_t *topk_experts, const float *topk_weights,
                    int32_t k, int32_t hidden_transform, int32_t threads,
                    float *out) {
  if (tokens <= 0 || hidden <= 0 || experts <= 0 || inter <= 0 || k <= 0) {
    return LFO_INVALID_SHAPE;
  }
  int64_t total = (int64_t)tokens * k;
  for (int64_t a = 0; a < total; a += 1) {
    if (topk_experts[a] < 0 || topk_experts[a] >= experts) {
      return LFO_INVALID_SHAPE;
    }
  }
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  float *y = (float *)malloc(sizeof(float) * (size_t)total * (size_t)hidden);
  if (y == NULL) return LFO_ARITHMETIC_OVERFLOW;
  moe_job jobs[256];
  pthread_t ids[256];
  int started[256];
  for (int32_t i = 0; i < threads; i += 1) {
    moe_job j = {x, hidden, inter, k, hidden_transform, wg, wu, wd,
                 topk_experts, y, total * i / threads,
                 total * (i + 1) / threads, LFO_OK};
    jobs[i] = j;
    started[i] = threads > 1 &&
                 pthread_create(&ids[i], NULL, moe_worker, &jobs[i]) == 0;
    if (!started[i]) moe_worker(&jobs[i]);
  }
  int32_t status = LFO_OK;
  for (int32_t i = 0; i < threads; i += 1) {
    if (started[i]) pthread_join(ids[i], NULL);
    if (jobs[i].status != LFO_OK) status = jobs[i].status;
  }
  if (status == LFO_OK) {
    for (int32_t t = 0; t < tokens; t += 1) {
      for (int32_t n = 0; n < hidden; n += 1) {
        float acc = 0.0f;
        for (int32_t j = 0; j < k; j += 1) {
          float p = topk_weights[(int64_t)t * k + j] *
                    y[((int64_t)t * k + j) * hidden + n];
          acc = acc + p;
        }
        if (!finite_f32(acc)) status = LFO_NON_FINITE;
        out[(int64_t)t * hidden + n] = acc;
      }
    }
  }
  free(y);
  return status;
}

/* ---- multithreaded projection (CPU baseline) ---------------------------- */

typedef struct proj_job {
  const float *x, *w;
  int32_t in_width, out_width;
  int64_t first, last;
  float *out;
  int32_t status;
} proj_job;

static void *proj_worker(void *arg) {
  proj_job *job = (proj_job *)arg;
  job->status = LFO_OK;
  for (int64_t e = job->first; e < job->last; e += 1) {
    int64_t r = e / job->out_width;
    int64_t n = e % job->out_width;
    const float *xr = job->x + r * job->in_width;
    const float *wn = job->w + n * job->in_width;
    float acc = 0.0f;
    for (int32_t k = 0; k < job->in_width; k += 1) {
      float product = xr[k] * wn[k];
      acc = acc + product;
    }
    if (!finite_f32(acc)) job->status = LFO_NON_FINITE;
    job->out[e] = acc;
  }
  return NULL;
}

int32_t lfo_project_values_mt(const float *x, int32_t rows, int32_t in_width,
                              const float *w, int32_t out_width,
                              int32_t threads, float *out) {
  if (rows <= 0 || in_width <= 0 || out_width <= 0) return LFO_INVALID_SHAPE;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  int64_t total = (int64_t)rows * out_width;
  proj_job jobs[256];
  pthread_t ids[256];
  int started[256];
  for (int32_t i = 0; i < threads; i += 1) {
    proj_job j = {x, w, in_width, out_width, total * i / threads,
                  total * (i + 1) / threads, out, LFO_OK};
    jobs[i] = j;
    started[i] = threads > 1 &&
                 pthread_create(&ids[i], NULL, proj_worker, &jobs[i]) == 0;
    if (!started[i]) proj_worker(&jobs[i]);
  }
  int32_t status = LFO_OK;
  for (int32_t i = 0; i < threads; i += 1) {
    if (started[i]) pthread_join(ids[i], NULL);
    if (jobs[i].status != LFO_OK) status = jobs[i].status;
  }
  return status;
}
