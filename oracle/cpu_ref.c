/*
 * cpu_ref.c: TEST INFRASTRUCTURE ONLY. CPU restatement of the reference's
 * deterministic CPU backend (Vladislav-Kalinkin/ullis 0.10.0). See cpu_ref.h.
 *
 * The Rust reference cannot be built here (no cargo/rustc, crates not
 * vendored), so nothing under /root/reference is compiled or run; each
 * function below restates the cited reference lines, in the same loop and
 * summation order, in C compiled with -ffp-contract=off.
 *
 * How each function is pinned (tests/test_oracle.py):
 *  - ucr_f16_from_f32 / to_f32: numpy float16 casts over stratified and edge
 *    f32 patterns (numpy is independent of the reference); the reference's
 *    own specials test (src/precision.rs:219-228).
 *  - ucr_clipped_sgd / ucr_binaryconnect_sgd: the reference's precision tests
 *    (src/precision.rs:238-313) and the Metal bit-exact fixtures'
 *    inputs (src/metal.rs:4007-4042) against an independent numpy float32
 *    evaluation of the same formula with numpy float16 rounding.
 *  - packing: pack_bitplane known answer (tests/rosa.rs:151-157), brute force.
 *  - packed forward / backward_ste: closed forms of tests/binary_linear.rs:4-39
 *    and brute-force float64 dense +-1 matrix products on the Metal fixtures
 *    (src/metal.rs:3806-3844, :3908-3974), plus g_scale = sum(sign * G).
 *  - LayerNorm: closed form of tests/cmix.rs:19-31, float64 numpy LayerNorm,
 *    finite-difference gradient check.
 *  - head CE: float64 log-softmax CE and its gradient on the Metal fixture
 *    (src/metal.rs:4045-4085); sum_v gy = 0 per valid row; row_loss[T-1] = 0.
 *  - FP16 linear: float64 numpy matmul (src/metal.rs:3876-3905 fixture).
 *  - CMix: closed forms of tests/cmix.rs:33-72; finite differences of
 *    time-shift-mix backward.
 *  - ROSA y / g_e: float64 numpy.
 *  - heron step: tests/test_oracle_heron.py, an independent float64 numpy
 *    re-derivation of train_step_on at tiny sizes, including a case with
 *    large scales and learning rate in which any update-order mistake
 *    changes the result.
 */
#include "cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>


#define LAYER_NORM_EPS 1e-5f      /* src/model.rs:132 */
#define HEAD_BIAS_LR_MULT 8.0f    /* src/model.rs:97 */

/* ---------------------------------------------------------------- a1 ---- */

static inline uint32_t f32_bits(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return b;
}
static inline float bits_f32(uint32_t b) {
  float v;
  memcpy(&v, &b, 4);
  return v;
}

/* Fp16::from_f32, src/precision.rs:23-55 */
uint16_t ucr_f16_from_f32(float value) {
  uint32_t bits = f32_bits(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
  uint32_t mantissa = bits & 0x007fffffu;
  int32_t half_exponent;
  if (exponent == 0xff) {
    return (uint16_t)(sign | (mantissa == 0 ? 0x7c00u : 0x7e00u));
  }
  half_exponent = exponent - 127 + 15;
  if (half_exponent >= 31) {
    return (uint16_t)(sign | 0x7c00u);
  }
  if (half_exponent <= 0) {
    uint32_t significand, shift, rounded, remainder, halfway;
    if (half_exponent < -10) {
      return sign;
    }
    significand = mantissa | 0x00800000u;
    shift = (uint32_t)(14 - half_exponent);
    rounded = significand >> shift;
    remainder = significand & ((1u << shift) - 1u);
    halfway = 1u << (shift - 1u);
    if (remainder > halfway || (remainder == halfway && (rounded & 1u) != 0)) {
      rounded += 1u;
    }
    return (uint16_t)(sign | (uint16_t)rounded);
  }
  {
    uint16_t rounded = (uint16_t)(sign | (uint16_t)((uint32_t)half_exponent << 10) |
                                  (uint16_t)(mantissa >> 13));
    uint32_t remainder = mantissa & 0x1fffu;
    if (remainder > 0x1000u || (remainder == 0x1000u && (rounded & 1u) != 0)) {
      rounded = (uint16_t)(rounded + 1u);
    }
    return rounded;
  }
}

/* Fp16::to_f32, src/precision.rs:57-76 */
float ucr_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
  uint32_t exponent = (uint32_t)((h >> 10) & 0x1fu);
  uint32_t mantissa = (uint32_t)(h & 0x03ffu);
  uint32_t bits;
  if (exponent == 0 && mantissa == 0) {
    bits = sign;
  } else if (exponent == 0) {
    uint32_t significand = mantissa;
    int32_t e = -14;
    while ((significand & 0x0400u) == 0) {
      significand <<= 1;
      e -= 1;
    }
    bits = sign | ((uint32_t)(e + 127) << 23) | ((significand & 0x03ffu) << 13);
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  return bits_f32(bits);
}

void ucr_f16_from_f32_array(const float* src, uint16_t* dst, size_t n) {
  size_t i;
  for (i = 0; i < n; ++i) dst[i] = ucr_f16_from_f32(src[i]);
}

void ucr_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
  size_t i;
  for (i = 0; i < n; ++i) dst[i] = ucr_f16_to_f32(src[i]);
}

#define H2F(x) ucr_f16_to_f32(x)

static inline float clampf(float v, float lo, float hi) {
  /* f32::clamp: NaN passes through */
  if (v < lo) return lo;
  if (v > hi) return hi;
  return v;
}

/* ------------------------------------------------------------ a2 / a3 --- */

/* Fp16Storage::apply_clipped_sgd, src/precision.rs:106-113 */
static void clipped_sgd_one(uint16_t* value, float* residual, float gradient, float lr) {
  float current = H2F(*value);
  float update = lr * clampf(gradient, -1.0f, 1.0f);
  float desired = current - update + *residual;
  uint16_t rounded = ucr_f16_from_f32(desired);
  *residual = desired - H2F(rounded);
  *value = rounded;
}

/* Fp16Storage::apply_binaryconnect_sgd, src/precision.rs:124-134 */
static void binaryconnect_sgd_one(uint16_t* value, float* residual, float gradient, float lr) {
  float current, update, desired;
  uint16_t rounded;
  if (!isfinite(gradient) || gradient == 0.0f) {
    return;
  }
  current = H2F(*value);
  update = lr * clampf(gradient, -1.0f, 1.0f);
  desired = clampf(current - update + *residual, -1.0f, 1.0f);
  rounded = ucr_f16_from_f32(desired);
  *residual = desired - H2F(rounded);
  *value = rounded;
}

void ucr_clipped_sgd(uint16_t* values, float* residual, const float* gradient, size_t n,
                     float learning_rate) {
  size_t i;
  for (i = 0; i < n; ++i) clipped_sgd_one(&values[i], &residual[i], gradient[i], learning_rate);
}

/* gradient_scale multiplies first, as the caller does at src/model.rs:827
 * (g_w[i] * ste_scale) and the Metal kernel at rwkv8.metal:66. */
void ucr_binaryconnect_sgd(uint16_t* values, float* residual, const float* gradient, size_t n,
                           float learning_rate, float gradient_scale) {
  size_t i;
  for (i = 0; i < n; ++i) {
    binaryconnect_sgd_one(&values[i], &residual[i], gradient[i] * gradient_scale, learning_rate);
  }
}

/* ---------------------------------------------------------------- a4 ---- */

size_t ucr_packed_word_count(size_t weights) { return (weights + 31) / 32; } /* :142-144 */

static inline int bit_is_plus(const uint32_t* bits, size_t index) { /* :146-148 */
  return (bits[index / 32] & (1u << (index % 32))) != 0;
}

static inline float sign_at(const uint32_t* bits, size_t index) { /* :716-722 */
  return bit_is_plus(bits, index) ? 1.0f : -1.0f;
}

/* rebinarize, src/model.rs:878-884: latent.get(i) >= 0.0 (so -0.0 => +1) */
void ucr_pack_latent_bits(const uint16_t* latent, size_t n, uint32_t* bits) {
  size_t i;
  memset(bits, 0, ucr_packed_word_count(n) * 4);
  for (i = 0; i < n; ++i) {
    if (H2F(latent[i]) >= 0.0f) bits[i / 32] |= 1u << (i % 32);
  }
}

/* bit_from_activation (src/rosa.rs:372-374) + pack_bitplane (:400-411) */
void ucr_sign_pack_bits(const float* x, size_t n, uint32_t* bits) {
  size_t i;
  memset(bits, 0, ucr_packed_word_count(n) * 4);
  for (i = 0; i < n; ++i) {
    if (x[i] > 0.0f) bits[i / 32] |= 1u << (i % 32);
  }
}

/* Derived cache (no reference counterpart): bits of the [in, out] transpose. */
void ucr_transpose_bits(const uint32_t* bits, size_t out, size_t in, uint32_t* bits_t) {
  size_t o, i;
  memset(bits_t, 0, ucr_packed_word_count(out * in) * 4);
  for (o = 0; o < out; ++o) {
    for (i = 0; i < in; ++i) {
      if (bit_is_plus(bits, o * in + i)) {
        size_t t = i * out + o;
        bits_t[t / 32] |= 1u << (t % 32);
      }
    }
  }
}

size_t ucr_bit_flip_count(const uint32_t* before, const uint32_t* after, size_t words) {
  size_t i, n = 0;
  for (i = 0; i < words; ++i) n += (size_t)__builtin_popcount(before[i] ^ after[i]);
  return n;
}

/* ----------------------------------------------------------- a5 - a9 ---- */

/* PackedBinaryLinear::forward, src/model.rs:724-742 */
int ucr_packed_forward(const float* x, size_t rows, size_t in, size_t out, const uint32_t* bits,
                       const uint16_t* scale, const uint16_t* bias, float* y) {
  size_t row, o, i;
  for (row = 0; row < rows; ++row) {
    const float* x_row = x + row * in;
    for (o = 0; o < out; ++o) {
      float sum = 0.0f;
      size_t base = o * in;
      float b;
      for (i = 0; i < in; ++i) sum += sign_at(bits, base + i) * x_row[i];
      b = bias ? H2F(bias[o]) : 0.0f;
      y[row * out + o] = b + H2F(scale[o]) * sum;
    }
  }
  return 0;
}

/* PackedBinaryLinear::backward_ste, src/model.rs:745-796. All outputs accumulate. */
int ucr_packed_backward_ste(const float* x, const float* gy, size_t rows, size_t in, size_t out,
                            const uint32_t* bits, const uint16_t* scale, float* g_w, float* g_x,
                            float* g_scale, float* g_bias) {
  size_t row, o, i;
  for (row = 0; row < rows; ++row) {
    const float* x_row = x + row * in;
    const float* gy_row = gy + row * out;
    for (o = 0; o < out; ++o) {
      float sc = H2F(scale[o]);
      float gy_o = gy_row[o];
      float signed_dot = 0.0f;
      size_t base = o * in;
      for (i = 0; i < in; ++i) {
        float s = sign_at(bits, base + i);
        g_w[base + i] += gy_o * sc * x_row[i];
        if (g_x) g_x[row * in + i] += gy_o * sc * s;
        signed_dot += s * x_row[i];
      }
      g_scale[o] += gy_o * signed_dot;
      if (g_bias) g_bias[o] += gy_o;
    }
  }
  return 0;
}

/* PackedBinaryLinear::apply_packed_sgd + rebinarize, src/model.rs:808-837, 878-884 */
int ucr_packed_apply_sgd(size_t in, size_t out, uint16_t* latent, float* latent_res,
                         uint16_t* scale, float* scale_res, uint16_t* bias, float* bias_res,
                         uint32_t* bits, const float* g_w, const float* g_scale,
                         const float* g_bias, float learning_rate, float ste_scale) {
  size_t weights = out * in, i, o;
  for (i = 0; i < weights; ++i) {
    binaryconnect_sgd_one(&latent[i], &latent_res[i], g_w[i] * ste_scale, learning_rate);
  }
  for (o = 0; o < out; ++o) clipped_sgd_one(&scale[o], &scale_res[o], g_scale[o], learning_rate);
  if (bias && g_bias) {
    for (o = 0; o < out; ++o) clipped_sgd_one(&bias[o], &bias_res[o], g_bias[o], learning_rate);
  }
  ucr_pack_latent_bits(latent, weights, bits);
  return 0;
}

/* ---------------------------------------------------------- a10 / a11 --- */

/* LayerNorm::forward, src/model.rs:259-276 */
int ucr_layer_norm_forward(const float* x, size_t rows, size_t ch, const uint16_t* weight,
                           const uint16_t* bias, float* y) {
  size_t row, c;
  for (row = 0; row < rows; ++row) {
    const float* src = x + row * ch;
    float mean = 0.0f, var = 0.0f, inv;
    for (c = 0; c < ch; ++c) mean += src[c];
    mean = mean / (float)ch;
    for (c = 0; c < ch; ++c) var += (src[c] - mean) * (src[c] - mean);
    var = var / (float)ch;
    inv = 1.0f / sqrtf(var + LAYER_NORM_EPS);
    for (c = 0; c < ch; ++c) {
      y[row * ch + c] = (src[c] - mean) * inv * H2F(weight[c]) + H2F(bias[c]);
    }
  }
  return 0;
}

/* LayerNorm::backward, src/model.rs:278-316. gx overwritten, gw/gb zeroed here. */
int ucr_layer_norm_backward(const float* x, const float* gy, size_t rows, size_t ch,
                            const uint16_t* weight, float* gx, float* gw, float* gb) {
  size_t row, c;
  float* xhat = (float*)malloc(ch * sizeof(float));
  float* dxhat = (float*)malloc(ch * sizeof(float));
  if (!xhat || !dxhat) {
    free(xhat);
    free(dxhat);
    return -1;
  }
  memset(gw, 0, ch * sizeof(float));
  memset(gb, 0, ch * sizeof(float));
  for (row = 0; row < rows; ++row) {
    const float* src = x + row * ch;
    const float* g = gy + row * ch;
    float mean = 0.0f, var = 0.0f, inv, inv_n;
    float sum_dxhat = 0.0f, sum_dxhat_xhat = 0.0f;
    for (c = 0; c < ch; ++c) mean += src[c];
    mean = mean / (float)ch;
    for (c = 0; c < ch; ++c) var += (src[c] - mean) * (src[c] - mean);
    var = var / (float)ch;
    inv = 1.0f / sqrtf(var + LAYER_NORM_EPS);
    for (c = 0; c < ch; ++c) {
      xhat[c] = (src[c] - mean) * inv;
      dxhat[c] = g[c] * H2F(weight[c]);
      sum_dxhat += dxhat[c];
      sum_dxhat_xhat += dxhat[c] * xhat[c];
      gw[c] += g[c] * xhat[c];
      gb[c] += g[c];
    }
    inv_n = inv / (float)ch;
    for (c = 0; c < ch; ++c) {
      gx[row * ch + c] = inv_n * ((float)ch * dxhat[c] - sum_dxhat - xhat[c] * sum_dxhat_xhat);
    }
  }
  free(xhat);
  free(dxhat);
  return 0;
}

/* --------------------------------------------------------------- a12 ---- */

/* causal_ce_row_valid, src/model.rs:27-39 */
int ucr_causal_ce_row_valid(size_t row, size_t time, size_t horizon, const uint32_t* targets,
                            size_t n_targets, uint32_t ignore_id) {
  size_t target_row;
  if (time == 0 || row % time + horizon >= time) return 0;
  target_row = row + horizon;
  return target_row < n_targets && targets[target_row] != ignore_id;
}

/* causal_ce_gradient_scale, src/model.rs:49-55 */
float ucr_causal_ce_gradient_scale(size_t n_valid, size_t time) {
  if (n_valid == 0 || time < 2) return 0.0f;
  return 1.0f / (float)(time - 1);
}

/* --------------------------------------------------------------- a13 ---- */

/* CPU branch of UllisHeron::apply_head_ce, src/model.rs:3132-3145, 3195-3244:
 * per valid row, head.forward then head.backward_ste(row) accumulating g_w,
 * g_hidden (row), g_scale, g_bias. No parameter update here. g_w, g_scale,
 * g_bias, g_hidden and row_loss are zeroed first. */
int ucr_head_ce(const float* hidden, size_t rows, size_t time, size_t d, size_t vocab,
                const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                const uint32_t* targets, uint32_t ignore_id, float* mean_loss, size_t* n_valid,
                float* row_loss, float* g_hidden, float* g_w, float* g_scale, float* g_bias) {
  return ucr_head_ce_horizon(hidden, rows, time, 1, d, vocab, bits, scale, bias, targets,
                             ignore_id, mean_loss, n_valid, row_loss, g_hidden, g_w, g_scale,
                             g_bias);
}

/* The Metal method takes the horizon (src/metal.rs:3300-3316, causal_supervised_count
 * and the softmax_cross_entropy kernel); apply_head_ce passes 1. */
int ucr_head_ce_horizon(const float* hidden, size_t rows, size_t time, size_t horizon, size_t d,
                        size_t vocab, const uint32_t* bits, const uint16_t* scale,
                        const uint16_t* bias, const uint32_t* targets, uint32_t ignore_id,
                        float* mean_loss, size_t* n_valid, float* row_loss, float* g_hidden,
                        float* g_w, float* g_scale, float* g_bias) {
  size_t row, v, nv = 0;
  float loss_scale, loss_sum = 0.0f;
  float* logits = (float*)malloc(vocab * sizeof(float));
  float* exps = (float*)malloc(vocab * sizeof(float));
  float* gy = (float*)malloc(vocab * sizeof(float));
  if (!logits || !exps || !gy) {
    free(logits);
    free(exps);
    free(gy);
    return -1;
  }
  for (row = 0; row < rows; ++row) {
    if (ucr_causal_ce_row_valid(row, time, horizon, targets, rows, ignore_id)) nv += 1;
  }
  loss_scale = ucr_causal_ce_gradient_scale(nv, time);
  memset(g_w, 0, vocab * d * sizeof(float));
  memset(g_scale, 0, vocab * sizeof(float));
  if (g_bias) memset(g_bias, 0, vocab * sizeof(float));
  memset(g_hidden, 0, rows * d * sizeof(float));
  memset(row_loss, 0, rows * sizeof(float));
  for (row = 0; row < rows; ++row) {
    size_t target;
    const float* h;
    float mx = -INFINITY, exp_sum = 0.0f, ce;
    if (!ucr_causal_ce_row_valid(row, time, horizon, targets, rows, ignore_id)) continue;
    target = targets[row + horizon];
    h = hidden + row * d;
    ucr_packed_forward(h, 1, d, vocab, bits, scale, bias, logits);
    for (v = 0; v < vocab; ++v) mx = fmaxf(mx, logits[v]);
    for (v = 0; v < vocab; ++v) {
      exps[v] = expf(logits[v] - mx);
      exp_sum += exps[v];
    }
    ce = mx + logf(exp_sum) - logits[target];
    row_loss[row] = ce;
    loss_sum += ce;
    for (v = 0; v < vocab; ++v) {
      gy[v] = loss_scale * (exps[v] / exp_sum - (v == target ? 1.0f : 0.0f));
    }
    ucr_packed_backward_ste(h, gy, 1, d, vocab, bits, scale, g_w, g_hidden + row * d, g_scale,
                            g_bias);
  }
  *mean_loss = nv == 0 ? 0.0f : loss_sum / (float)nv;
  *n_valid = nv;
  free(logits);
  free(exps);
  free(gy);
  return 0;
}

/* ------------------------------------------------ CausalLoss statistics ---- */

/* rms, src/model.rs:3293-3299: sqrt(sum v^2 / n), sequential f32 sum */
float ucr_rms(const float* v, size_t n) {
  float s = 0.0f;
  size_t i;
  if (n == 0) return 0.0f;
  for (i = 0; i < n; ++i) s += v[i] * v[i];
  return sqrtf(s / (float)n);
}

/* rms_fp16, src/model.rs:3301-3312 */
float ucr_rms_fp16(const uint16_t* v, size_t n) {
  float s = 0.0f;
  size_t i;
  if (n == 0) return 0.0f;
  for (i = 0; i < n; ++i) {
    const float x = ucr_f16_to_f32(v[i]);
    s += x * x;
  }
  return sqrtf(s / (float)n);
}

/* mean_abs, src/model.rs:3314-3319 */
float ucr_mean_abs(const float* v, size_t n) {
  float s = 0.0f;
  size_t i;
  if (n == 0) return 0.0f;
  for (i = 0; i < n; ++i) s += fabsf(v[i]);
  return s / (float)n;
}

/* mean_abs_fp16, src/model.rs:3321-3327 */
float ucr_mean_abs_fp16(const uint16_t* v, size_t n) {
  float s = 0.0f;
  size_t i;
  if (n == 0) return 0.0f;
  for (i = 0; i < n; ++i) s += fabsf(ucr_f16_to_f32(v[i]));
  return s / (float)n;
}

/* mean_abs_delta_fp16, src/model.rs:3329-3339 */
float ucr_mean_abs_delta_fp16(const uint16_t* before, const uint16_t* after, size_t n) {
  float s = 0.0f;
  size_t i;
  if (n == 0) return 0.0f;
  for (i = 0; i < n; ++i) s += fabsf(ucr_f16_to_f32(before[i]) - ucr_f16_to_f32(after[i]));
  return s / (float)n;
}

/* f32::total_cmp as an unsigned key */
static uint32_t total_key(float v) {
  const uint32_t b = f32_bits(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static int cmp_total(const void* a, const void* b) {
  const uint32_t ka = total_key(*(const float*)a), kb = total_key(*(const float*)b);
  return ka < kb ? -1 : (ka > kb ? 1 : 0);
}

/* loss_percentiles, src/model.rs:3341-3363: finite losses of valid rows
 * (horizon 1), sorted by total_cmp; p-th = valid[min(round(p (n-1)), n-1)]
 * with the product and the rounding (half away from zero) in f32. */
void ucr_loss_percentiles(const float* row_loss, size_t rows, size_t time, const uint32_t* targets,
                          uint32_t ignore_id, float* out3) {
  const float ps[3] = {0.10f, 0.50f, 0.90f};
  float* valid = (float*)malloc((rows ? rows : 1) * sizeof(float));
  size_t n = 0, row;
  int q;
  out3[0] = out3[1] = out3[2] = 0.0f;
  if (!valid) return;
  for (row = 0; row < rows; ++row) {
    if (!ucr_causal_ce_row_valid(row, time, 1, targets, rows, ignore_id)) continue;
    if (!isfinite(row_loss[row])) continue;
    valid[n++] = row_loss[row];
  }
  if (n > 0) {
    qsort(valid, n, sizeof(float), cmp_total);
    for (q = 0; q < 3; ++q) {
      size_t at = (size_t)roundf(ps[q] * (float)(n - 1));
      if (at > n - 1) at = n - 1;
      out3[q] = valid[at];
    }
  }
  free(valid);
}

static int cmp_u32(const void* a, const void* b) {
  const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/* unigram_cross_entropy, src/model.rs:3365-3390: counts of targets[row + 1]
 * over valid rows; ce = -sum count * ln(count / n) / n (f32). The reference
 * iterates a HashMap, whose order is not fixed; here the counts are taken in
 * ascending target order. */
float ucr_unigram_cross_entropy(const uint32_t* targets, size_t rows, size_t time,
                                uint32_t ignore_id, size_t* unique) {
  uint32_t* ids = (uint32_t*)malloc((rows ? rows : 1) * sizeof(uint32_t));
  size_t n = 0, row, i, u = 0;
  float ce = 0.0f, nf;
  *unique = 0;
  if (!ids) return 0.0f;
  for (row = 0; row < rows; ++row) {
    if (!ucr_causal_ce_row_valid(row, time, 1, targets, rows, ignore_id)) continue;
    ids[n++] = targets[row + 1];
  }
  if (n == 0) {
    free(ids);
    return 0.0f;
  }
  qsort(ids, n, sizeof(uint32_t), cmp_u32);
  nf = (float)n;
  for (i = 0; i < n;) {
    size_t j = i;
    float count, p;
    while (j < n && ids[j] == ids[i]) ++j;
    count = (float)(j - i);
    p = count / nf;
    ce -= count * logf(p);
    u += 1;
    i = j;
  }
  free(ids);
  *unique = u;
  return ce / nf;
}

/* --------------------------------------------------------------- a14 ---- */

/* Fp16Linear::forward, src/model.rs:419-436 */
int ucr_fp16_forward(const float* x, size_t rows, size_t in, size_t out, const uint16_t* w,
                     float* y) {
  size_t row, o, i;
  for (row = 0; row < rows; ++row) {
    const float* x_row = x + row * in;
    for (o = 0; o < out; ++o) {
      float sum = 0.0f;
      size_t w_row = o * in;
      for (i = 0; i < in; ++i) sum += H2F(w[w_row + i]) * x_row[i];
      y[row * out + o] = sum;
    }
  }
  return 0;
}

/* Fp16Linear::backward, src/model.rs:438-460. g_x and g_w are zeroed here. */
int ucr_fp16_backward(const float* x, const float* gy, size_t rows, size_t in, size_t out,
                      const uint16_t* w, float* g_x, float* g_w) {
  size_t row, o, i;
  memset(g_x, 0, rows * in * sizeof(float));
  memset(g_w, 0, out * in * sizeof(float));
  for (row = 0; row < rows; ++row) {
    const float* x_row = x + row * in;
    const float* gy_row = gy + row * out;
    for (o = 0; o < out; ++o) {
      size_t base = o * in;
      float g = gy_row[o];
      for (i = 0; i < in; ++i) {
        g_w[base + i] += g * x_row[i];
        g_x[row * in + i] += g * H2F(w[base + i]);
      }
    }
  }
  return 0;
}

/* --------------------------------------------------------------- a15 ---- */

/* time_shift_delta, src/model.rs:186-212 */
int ucr_time_shift_delta(const float* x, size_t batch, size_t time, size_t ch, float* xx) {
  size_t b, t, c;
  if (time == 0 || ch == 0) return -1;
  for (b = 0; b < batch; ++b) {
    for (t = 0; t < time; ++t) {
      size_t row = (b * time + t) * ch;
      for (c = 0; c < ch; ++c) {
        float xt = x[row + c];
        xx[row + c] = t == 0 ? -xt : x[(b * time + t - 1) * ch + c] - xt;
      }
    }
  }
  return 0;
}

/* lerp_shift_backward, src/model.rs:1207-1240. g_x and g_mix accumulate. */
int ucr_lerp_shift_backward(const float* xx, const uint16_t* mix, const float* g_shifted,
                            size_t batch, size_t time, size_t ch, float* g_x, float* g_mix) {
  size_t b, t, c, n = batch * time * ch;
  float* g_xx = (float*)malloc(n * sizeof(float));
  if (!g_xx) return -1;
  for (b = 0; b < batch; ++b) {
    for (t = 0; t < time; ++t) {
      for (c = 0; c < ch; ++c) {
        size_t index = (b * time + t) * ch + c;
        g_mix[c] += g_shifted[index] * xx[index];
        g_x[index] += g_shifted[index];
        g_xx[index] = g_shifted[index] * H2F(mix[c]);
      }
    }
  }
  for (b = 0; b < batch; ++b) {
    for (t = 0; t < time; ++t) {
      for (c = 0; c < ch; ++c) {
        size_t index = (b * time + t) * ch + c;
        if (t > 0) g_x[(b * time + t - 1) * ch + c] += g_xx[index];
        g_x[index] -= g_xx[index];
      }
    }
  }
  free(g_xx);
  return 0;
}

/* shifted[i] = x[i] + xx[i] * mix[c], src/model.rs:1049-1057 */
static void lerp_mix(const float* x, const float* xx, const uint16_t* mix, size_t rows, size_t ch,
                     float* out) {
  size_t i, c;
  for (i = 0; i < rows; ++i) {
    for (c = 0; c < ch; ++c) {
      size_t index = i * ch + c;
      out[index] = x[index] + xx[index] * H2F(mix[c]);
    }
  }
}

/* --------------------------------------------------------------- a16 ---- */

/* y[index] = (2*idx - 1) * e[c], src/model.rs:1597-1599 (row-major idx). */
int ucr_rosa_y_from_idx(const uint8_t* idx, const uint16_t* e, size_t rows, size_t ch, float* y) {
  size_t i, c;
  for (i = 0; i < rows; ++i) {
    for (c = 0; c < ch; ++c) {
      size_t index = i * ch + c;
      y[index] = (2.0f * (float)idx[index] - 1.0f) * H2F(e[c]);
    }
  }
  return 0;
}

/* rosa_e_grad, src/model.rs:1608-1634 (g_e zeroed here) */
int ucr_rosa_e_grad(const float* g_y, const uint8_t* idx, size_t rows, size_t ch, float* g_e) {
  size_t row, c;
  memset(g_e, 0, ch * sizeof(float));
  for (row = 0; row < rows; ++row) {
    for (c = 0; c < ch; ++c) {
      size_t index = row * ch + c;
      g_e[c] += g_y[index] * (2.0f * (float)idx[index] - 1.0f);
    }
  }
  return 0;
}

/* ----------------------------------------------------------- embedding -- */

/* train_step_on's gather, src/model.rs:2866-2873 */
int ucr_embedding_gather(const uint16_t* table, size_t d, const uint32_t* tokens, size_t rows,
                         float* x) {
  size_t row, c;
  for (row = 0; row < rows; ++row) {
    size_t offset = (size_t)tokens[row] * d;
    for (c = 0; c < d; ++c) x[row * d + c] = H2F(table[offset + c]);
  }
  return 0;
}

/* train_step_on's scatter-SGD, src/model.rs:2986-2993: rows in order, so a
 * repeated token is stepped once per row, in row order */
int ucr_embedding_scatter_sgd(uint16_t* table, float* residual, size_t d,
                              const uint32_t* tokens, size_t rows, const float* g_x,
                              float learning_rate) {
  size_t row, c;
  for (row = 0; row < rows; ++row) {
    size_t offset = (size_t)tokens[row] * d;
    for (c = 0; c < d; ++c) {
      clipped_sgd_one(&table[offset + c], &residual[offset + c], g_x[row * d + c], learning_rate);
    }
  }
  return 0;
}

size_t ucr_heron_layout(const ullis_heron_dims* dims, ullis_tensor_desc* out, size_t cap,
                        uint64_t* bytes) {
  return ullis_heron_layout(dims, out, cap, bytes);
}

/* --------------------------------------------------------------- a17 ---- */

typedef struct arena_view {
  ullis_tensor_desc* descs;
  size_t n;
  uint8_t* base;
} arena_view;

static void* tensor_ptr(const arena_view* a, const char* name) {
  uint64_t off = ullis_heron_offset(a->descs, a->n, name);
  if (off == UINT64_MAX) return NULL;
  return a->base + off;
}

typedef struct packed_view {
  size_t out, in;
  uint32_t* bits;
  uint16_t *scale, *bias, *latent;
  float *scale_res, *bias_res, *latent_res;
} packed_view;

static int packed_bind(const arena_view* a, const char* prefix, size_t out, size_t in,
                       int has_bias, packed_view* p) {
  char buf[ULLIS_NAME_MAX];
  p->out = out;
  p->in = in;
#define BIND(field, suffix)                               \
  snprintf(buf, sizeof buf, "%s%s", prefix, suffix);      \
  p->field = tensor_ptr(a, buf);
  BIND(bits, ".bits");
  BIND(scale, ".scale");
  BIND(scale_res, ".scale.residual");
  BIND(latent, ".latent");
  BIND(latent_res, ".latent.residual");
  if (has_bias) {
    BIND(bias, ".bias");
    BIND(bias_res, ".bias.residual");
  } else {
    p->bias = NULL;
    p->bias_res = NULL;
  }
#undef BIND
  if (!p->bits || !p->scale || !p->latent) return -1;
  if (has_bias && !p->bias) return -1;
  return 0;
}

typedef struct ln_view {
  uint16_t *w, *b;
  float *w_res, *b_res;
} ln_view;

static int ln_bind(const arena_view* a, const char* prefix, ln_view* l) {
  char buf[ULLIS_NAME_MAX];
  snprintf(buf, sizeof buf, "%s.weight", prefix);
  l->w = tensor_ptr(a, buf);
  snprintf(buf, sizeof buf, "%s.weight.residual", prefix);
  l->w_res = tensor_ptr(a, buf);
  snprintf(buf, sizeof buf, "%s.bias", prefix);
  l->b = tensor_ptr(a, buf);
  snprintf(buf, sizeof buf, "%s.bias.residual", prefix);
  l->b_res = tensor_ptr(a, buf);
  return (l->w && l->b && l->w_res && l->b_res) ? 0 : -1;
}

/* LayerNorm::apply_clipped_sgd, src/model.rs:318-332 (weight then bias per channel) */
static void ln_sgd(ln_view* l, const float* gw, const float* gb, size_t ch, float lr) {
  size_t c;
  for (c = 0; c < ch; ++c) {
    clipped_sgd_one(&l->w[c], &l->w_res[c], gw[c], lr);
    clipped_sgd_one(&l->b[c], &l->b_res[c], gb[c], lr);
  }
}

typedef struct block_tape {
  float* ln0_in;     /* layer 0 only */
  float* after_rosa; /* [rows, d] */
  float* y;          /* ROSA output [rows, d] */
  uint8_t* idx;      /* row-major [rows, d] */
  float* xx;         /* CMix time-shift delta [rows, d] */
  float* shifted;    /* [rows, d] */
  float* key;        /* [rows, f] */
  float* relu2;      /* [rows, f] */
} block_tape;

#define XMALLOC(ptr, count)                                   \
  do {                                                        \
    (ptr) = calloc((count), sizeof(*(ptr)));                  \
    if (!(ptr)) {                                             \
      rc = -1;                                                \
      goto done;                                              \
    }                                                         \
  } while (0)

/*
 * UllisHeron::train_step_on, src/model.rs:2827-3025, CPU branch
 * (metal = None), rosa_grad = stop_grad_bits, starting from the gathered
 * embedding rows x_emb and ending with the embedding-row gradient g_emb.
 *
 * The ROSA suffix automaton is replaced by the caller's idx tape rosa_idx
 * ([n_layers][batch][d][time] u8, channel-major as produced by
 * rosa_qkv_batch_packed_channel_major, src/rosa.rs:486-513); y follows
 * rosa_qkv_out_batched_channel_major (src/rosa.rs:614-639). The Q/K/V
 * projections still run and their sign bit-planes (bit_from_activation +
 * pack_bitplane on row-major [rows, d]) are written to qkv_bits
 * ([n_layers][3][words]) when non-NULL.
 */
int ucr_heron_train_step(const ullis_heron_dims* dims, uint8_t* arena, const float* x_emb,
                         const uint32_t* labels, uint32_t ignore_id, size_t batch, size_t time,
                         float learning_rate, const uint8_t* rosa_idx, float* g_emb,
                         float* row_loss, uint32_t* qkv_bits, ucr_step_stats* stats) {
  int rc = 0;
  size_t d = dims->d_model, f = dims->dim_ffn, v = dims->vocab, L = dims->n_layers;
  size_t rows = batch * time, nd = rows * d, nf = rows * f, layer, i, c, b, t;
  size_t words_act = ucr_packed_word_count(nd);
  size_t max_w = d * d;
  float lr = learning_rate, ste;
  arena_view a;
  ln_view ln_out;
  packed_view head;
  block_tape* tapes = NULL;
  float *x = NULL, *tmp = NULL, *q = NULL, *k = NULL, *vv = NULL, *hidden = NULL, *pre_ln_out = NULL;
  float *g_x = NULL, *g_tmp = NULL, *g_tmp2 = NULL, *g_w = NULL, *g_scale = NULL, *g_bias = NULL;
  float *gw_ln = NULL, *gb_ln = NULL, *g_mix = NULL, *g_e = NULL, *g_f = NULL, *g_f2 = NULL;
  uint32_t* before = NULL;
  uint16_t* before_latent = NULL;
  float head_scale_grad_rms = 0.0f, head_latent_step_abs = 0.0f;
  uint64_t total;
  float mean_loss = 0.0f;
  size_t n_valid = 0, flips_head = 0, flips_cmix = 0, flips_rosa_o = 0;

  memset(&a, 0, sizeof a);
  if (time < 2 || !(learning_rate > 0.0f) || !isfinite(learning_rate) || batch == 0) return -2;
  a.n = ullis_heron_layout(dims, NULL, 0, &total);
  a.descs = (ullis_tensor_desc*)calloc(a.n, sizeof(ullis_tensor_desc));
  if (!a.descs) return -1;
  ullis_heron_layout(dims, a.descs, a.n, &total);
  a.base = arena;
  if (d * f > max_w) max_w = d * f;
  if (v * d > max_w) max_w = v * d;

  XMALLOC(tapes, L);
  XMALLOC(x, nd);
  XMALLOC(tmp, nd);
  XMALLOC(q, nd);
  XMALLOC(k, nd);
  XMALLOC(vv, nd);
  XMALLOC(hidden, nd);
  XMALLOC(pre_ln_out, nd);
  XMALLOC(g_x, nd);
  XMALLOC(g_tmp, nd);
  XMALLOC(g_tmp2, nd);
  XMALLOC(g_w, max_w);
  XMALLOC(g_scale, v > f ? v : f);
  XMALLOC(g_bias, v > d ? v : d);
  XMALLOC(gw_ln, d);
  XMALLOC(gb_ln, d);
  XMALLOC(g_mix, d);
  XMALLOC(g_e, d);
  XMALLOC(g_f, nf);
  XMALLOC(g_f2, nf);
  XMALLOC(before, ucr_packed_word_count(max_w));
  XMALLOC(before_latent, v * d);
  for (layer = 0; layer < L; ++layer) {
    block_tape* tp = &tapes[layer];
    if (layer == 0) XMALLOC(tp->ln0_in, nd);
    XMALLOC(tp->after_rosa, nd);
    XMALLOC(tp->y, nd);
    XMALLOC(tp->idx, nd);
    XMALLOC(tp->xx, nd);
    XMALLOC(tp->shifted, nd);
    XMALLOC(tp->key, nf);
    XMALLOC(tp->relu2, nf);
  }
  if (ln_bind(&a, "ln_out", &ln_out) || packed_bind(&a, "head", v, d, 1, &head)) {
    rc = -3;
    goto done;
  }

  memcpy(x, x_emb, nd * sizeof(float));

  /* forward, src/model.rs:2876-2915 */
  for (layer = 0; layer < L; ++layer) {
    block_tape* tp = &tapes[layer];
    char p[ULLIS_NAME_MAX];
    ln_view ln0, ln2, ln3;
    packed_view pq, pk, pv, po, key;
    uint16_t *x_q, *x_k, *x_v, *e, *cx_k, *value;
    snprintf(p, sizeof p, "blocks.%zu.ln2", layer);
    if (ln_bind(&a, p, &ln2)) { rc = -3; goto done; }
    snprintf(p, sizeof p, "blocks.%zu.ln3", layer);
    if (ln_bind(&a, p, &ln3)) { rc = -3; goto done; }
#define PBIND(view, name, out_, in_, bias_)                                  \
  snprintf(p, sizeof p, "blocks.%zu." name, layer);                          \
  if (packed_bind(&a, p, out_, in_, bias_, &view)) { rc = -3; goto done; }
    PBIND(pq, "rosa.q", d, d, 1);
    PBIND(pk, "rosa.k", d, d, 1);
    PBIND(pv, "rosa.v", d, d, 1);
    PBIND(po, "rosa.o", d, d, 1);
    PBIND(key, "ffn.key", f, d, 0);
#define TBIND(var, name)                                 \
  snprintf(p, sizeof p, "blocks.%zu." name, layer);      \
  var = tensor_ptr(&a, p);                               \
  if (!var) { rc = -3; goto done; }
    TBIND(x_q, "rosa.x_q");
    TBIND(x_k, "rosa.x_k");
    TBIND(x_v, "rosa.x_v");
    TBIND(e, "rosa.e");
    TBIND(cx_k, "ffn.x_k");
    TBIND(value, "ffn.value");
    if (layer == 0) {
      snprintf(p, sizeof p, "blocks.%zu.ln0", layer);
      if (ln_bind(&a, p, &ln0)) { rc = -3; goto done; }
      memcpy(tp->ln0_in, x, nd * sizeof(float));
      ucr_layer_norm_forward(tp->ln0_in, rows, d, ln0.w, ln0.b, x);
    }
    /* ROSA: ln3 -> time-shift mix3 -> Q/K/V -> [SAM] -> y -> O (src/model.rs:1354-1440) */
    ucr_layer_norm_forward(x, rows, d, ln3.w, ln3.b, tmp);
    ucr_time_shift_delta(tmp, batch, time, d, g_tmp); /* g_tmp holds xx here */
    lerp_mix(tmp, g_tmp, x_q, rows, d, g_tmp2);
    ucr_packed_forward(g_tmp2, rows, d, d, pq.bits, pq.scale, pq.bias, q);
    lerp_mix(tmp, g_tmp, x_k, rows, d, g_tmp2);
    ucr_packed_forward(g_tmp2, rows, d, d, pk.bits, pk.scale, pk.bias, k);
    lerp_mix(tmp, g_tmp, x_v, rows, d, g_tmp2);
    ucr_packed_forward(g_tmp2, rows, d, d, pv.bits, pv.scale, pv.bias, vv);
    if (qkv_bits) {
      uint32_t* dst = qkv_bits + layer * 3 * words_act;
      ucr_sign_pack_bits(q, nd, dst);
      ucr_sign_pack_bits(k, nd, dst + words_act);
      ucr_sign_pack_bits(vv, nd, dst + 2 * words_act);
    }
    {
      const uint8_t* src = rosa_idx + layer * nd;
      for (b = 0; b < batch; ++b)
        for (c = 0; c < d; ++c)
          for (t = 0; t < time; ++t)
            tp->idx[(b * time + t) * d + c] = src[(b * d + c) * time + t];
    }
    ucr_rosa_y_from_idx(tp->idx, e, rows, d, tp->y);
    ucr_packed_forward(tp->y, rows, d, d, po.bits, po.scale, po.bias, tmp);
    for (i = 0; i < nd; ++i) x[i] += tmp[i];
    memcpy(tp->after_rosa, x, nd * sizeof(float));
    /* CMix: ln2 -> forward_tape (src/model.rs:1018-1078) */
    ucr_layer_norm_forward(x, rows, d, ln2.w, ln2.b, tmp);
    ucr_time_shift_delta(tmp, batch, time, d, tp->xx);
    lerp_mix(tmp, tp->xx, cx_k, rows, d, tp->shifted);
    ucr_packed_forward(tp->shifted, rows, d, f, key.bits, key.scale, NULL, tp->key);
    for (i = 0; i < nf; ++i) {
      float kv = tp->key[i] > 0.0f ? tp->key[i] : 0.0f;
      tp->relu2[i] = kv * kv;
    }
    ucr_fp16_forward(tp->relu2, rows, f, d, value, tmp);
    for (i = 0; i < nd; ++i) x[i] += tmp[i];
#undef PBIND
#undef TBIND
  }
  memcpy(pre_ln_out, x, nd * sizeof(float));
  ucr_layer_norm_forward(x, rows, d, ln_out.w, ln_out.b, hidden);

  /* head + CE with update (src/model.rs:3132-3274) */
  {
    float loss;
    size_t nv;
    ucr_head_ce(hidden, rows, time, d, v, head.bits, head.scale, head.bias, labels, ignore_id,
                &loss, &nv, row_loss, g_x, g_w, g_scale, g_bias);
    memcpy(before, head.bits, ucr_packed_word_count(v * d) * 4);
    memcpy(before_latent, head.latent, v * d * sizeof(uint16_t));
    head_scale_grad_rms = ucr_rms(g_scale, v); /* rms(&g_scale), src/model.rs:3270 */
    /* flip_after_gradients(g_w, g_scale, None, lr, ste) then head bias at 8x lr */
    ucr_packed_apply_sgd(d, v, head.latent, head.latent_res, head.scale, head.scale_res, NULL,
                         NULL, head.bits, g_w, g_scale, NULL, lr, (float)(time - 1));
    for (c = 0; c < v; ++c) {
      clipped_sgd_one(&head.bias[c], &head.bias_res[c], g_bias[c], lr * HEAD_BIAS_LR_MULT);
    }
    flips_head = ucr_bit_flip_count(before, head.bits, ucr_packed_word_count(v * d));
    head_latent_step_abs = ucr_mean_abs_delta_fp16(before_latent, head.latent, v * d);
    mean_loss = loss;
    n_valid = nv;
  }
  ste = (float)(time - 1); /* binaryconnect_ste_scale(time - 1), src/model.rs:554-556 */

  /* ln_out backward + SGD (src/model.rs:2932-2937) */
  ucr_layer_norm_backward(pre_ln_out, g_x, rows, d, ln_out.w, g_tmp, gw_ln, gb_ln);
  ln_sgd(&ln_out, gw_ln, gb_ln, d, lr);
  memcpy(g_x, g_tmp, nd * sizeof(float));

  /* reverse blocks (src/model.rs:2941-2984) */
  for (layer = L; layer-- > 0;) {
    block_tape* tp = &tapes[layer];
    char p[ULLIS_NAME_MAX];
    ln_view ln2;
    packed_view po, key;
    uint16_t *e, *cx_k, *value;
    float *value_res, *e_res, *cx_k_res;
    snprintf(p, sizeof p, "blocks.%zu.ln2", layer);
    if (ln_bind(&a, p, &ln2)) { rc = -3; goto done; }
    snprintf(p, sizeof p, "blocks.%zu.rosa.o", layer);
    if (packed_bind(&a, p, d, d, 1, &po)) { rc = -3; goto done; }
    snprintf(p, sizeof p, "blocks.%zu.ffn.key", layer);
    if (packed_bind(&a, p, f, d, 0, &key)) { rc = -3; goto done; }
    snprintf(p, sizeof p, "blocks.%zu.rosa.e", layer);
    e = tensor_ptr(&a, p);
    snprintf(p, sizeof p, "blocks.%zu.rosa.e.residual", layer);
    e_res = tensor_ptr(&a, p);
    snprintf(p, sizeof p, "blocks.%zu.ffn.x_k", layer);
    cx_k = tensor_ptr(&a, p);
    snprintf(p, sizeof p, "blocks.%zu.ffn.x_k.residual", layer);
    cx_k_res = tensor_ptr(&a, p);
    snprintf(p, sizeof p, "blocks.%zu.ffn.value", layer);
    value = tensor_ptr(&a, p);
    snprintf(p, sizeof p, "blocks.%zu.ffn.value.residual", layer);
    value_res = tensor_ptr(&a, p);
    if (!e || !e_res || !cx_k || !cx_k_res || !value || !value_res) { rc = -3; goto done; }

    /* CMix backward_update, CPU branch (src/model.rs:1145-1177) */
    ucr_fp16_backward(tp->relu2, g_x, rows, f, d, value, g_f /* g_relu2 */, g_w /* g_value */);
    ucr_clipped_sgd(value, value_res, g_w, d * f, lr);
    for (i = 0; i < nf; ++i) { /* relu2_bwd_on, src/model.rs:1191-1205 */
      g_f2[i] = tp->key[i] > 0.0f ? 2.0f * tp->key[i] * g_f[i] : 0.0f;
    }
    memset(g_w, 0, f * d * sizeof(float));
    memset(g_scale, 0, f * sizeof(float));
    memset(g_tmp2, 0, nd * sizeof(float)); /* g_shifted */
    ucr_packed_backward_ste(tp->shifted, g_f2, rows, d, f, key.bits, key.scale, g_w, g_tmp2,
                            g_scale, NULL);
    memcpy(before, key.bits, ucr_packed_word_count(f * d) * 4);
    ucr_packed_apply_sgd(d, f, key.latent, key.latent_res, key.scale, key.scale_res, NULL, NULL,
                         key.bits, g_w, g_scale, NULL, lr, ste);
    flips_cmix += ucr_bit_flip_count(before, key.bits, ucr_packed_word_count(f * d));
    memset(g_mix, 0, d * sizeof(float));
    memset(g_tmp, 0, nd * sizeof(float)); /* g_ln2_out */
    ucr_lerp_shift_backward(tp->xx, cx_k, g_tmp2, batch, time, d, g_tmp, g_mix);
    ucr_clipped_sgd(cx_k, cx_k_res, g_mix, d, lr);

    /* ln2 backward + SGD, residual add (src/model.rs:2958-2963) */
    ucr_layer_norm_backward(tp->after_rosa, g_tmp, rows, d, ln2.w, g_tmp2, gw_ln, gb_ln);
    ln_sgd(&ln2, gw_ln, gb_ln, d, lr);
    for (i = 0; i < nd; ++i) g_x[i] += g_tmp2[i];

    /* ROSA backward_stop_grad, CPU branch (src/model.rs:1491-1522) */
    memset(g_w, 0, d * d * sizeof(float));
    memset(g_scale, 0, d * sizeof(float));
    memset(g_bias, 0, d * sizeof(float));
    memset(g_tmp2, 0, nd * sizeof(float)); /* g_y */
    ucr_packed_backward_ste(tp->y, g_x, rows, d, d, po.bits, po.scale, g_w, g_tmp2, g_scale,
                            g_bias);
    memcpy(before, po.bits, ucr_packed_word_count(d * d) * 4);
    ucr_packed_apply_sgd(d, d, po.latent, po.latent_res, po.scale, po.scale_res, po.bias,
                         po.bias_res, po.bits, g_w, g_scale, g_bias, lr, ste);
    flips_rosa_o += ucr_bit_flip_count(before, po.bits, ucr_packed_word_count(d * d));
    ucr_rosa_e_grad(g_tmp2, tp->idx, rows, d, g_e);
    ucr_clipped_sgd(e, e_res, g_e, d, lr);

    if (layer == 0) { /* ln0 backward + SGD (src/model.rs:2978-2982) */
      ln_view ln0;
      snprintf(p, sizeof p, "blocks.%zu.ln0", layer);
      if (ln_bind(&a, p, &ln0)) { rc = -3; goto done; }
      ucr_layer_norm_backward(tp->ln0_in, g_x, rows, d, ln0.w, g_tmp, gw_ln, gb_ln);
      ln_sgd(&ln0, gw_ln, gb_ln, d, lr);
      memcpy(g_x, g_tmp, nd * sizeof(float));
    }
  }
  memcpy(g_emb, g_x, nd * sizeof(float));
  if (stats) {
    /* CausalLoss, src/model.rs:2997-3024 */
    uint16_t* value0;
    size_t uniq = 0;
    float pct[3];
    stats->mean_loss = mean_loss;
    stats->n_valid = n_valid;
    stats->flips_head = flips_head;
    stats->flips_cmix = flips_cmix;
    stats->flips_rosa_o = flips_rosa_o;
    ucr_loss_percentiles(row_loss, rows, time, labels, ignore_id, pct);
    stats->loss_p10 = pct[0];
    stats->loss_p50 = pct[1];
    stats->loss_p90 = pct[2];
    stats->unigram_ce = ucr_unigram_cross_entropy(labels, rows, time, ignore_id, &uniq);
    stats->unique_targets = uniq;
    stats->embed_grad_rms = ucr_rms(g_emb, nd);
    stats->head_scale_grad_rms = head_scale_grad_rms;
    stats->head_scale_rms = ucr_rms_fp16(head.scale, v);
    value0 = tensor_ptr(&a, "blocks.0.ffn.value");
    stats->cmix_value_rms = value0 ? ucr_rms_fp16(value0, d * f) : 0.0f;
    stats->head_latent_abs_mean = ucr_mean_abs_fp16(head.latent, v * d);
    stats->head_latent_step_abs = head_latent_step_abs;
    stats->head_bias_rms = head.bias ? ucr_rms_fp16(head.bias, v) : 0.0f;
  }

done:
  if (tapes) {
    for (layer = 0; layer < L; ++layer) {
      free(tapes[layer].ln0_in);
      free(tapes[layer].after_rosa);
      free(tapes[layer].y);
      free(tapes[layer].idx);
      free(tapes[layer].xx);
      free(tapes[layer].shifted);
      free(tapes[layer].key);
      free(tapes[layer].relu2);
    }
  }
  free(tapes);
  free(x);
  free(tmp);
  free(q);
  free(k);
  free(vv);
  free(hidden);
  free(pre_ln_out);
  free(g_x);
  free(g_tmp);
  free(g_tmp2);
  free(g_w);
  free(g_scale);
  free(g_bias);
  free(gw_ln);
  free(gb_ln);
  free(g_mix);
  free(g_e);
  free(g_f);
  free(g_f2);
  free(before);
  free(before_latent);
  free(a.descs);
  return rc;
}

/* ------------------------------------------------------- T = 1 decode ---- */

/* time_shift_one, src/model.rs:214-228: prev - x, or -x without a previous token */
static void time_shift_one(const float* x, const float* prev, int has_prev, size_t d, float* xx) {
  size_t c;
  for (c = 0; c < d; ++c) xx[c] = has_prev ? prev[c] - x[c] : -x[c];
}

/*
 * One token per sequence of UllisHeron::generate_step (src/model.rs:2717-2753):
 * embedding row, every block's forward_one (src/model.rs:2243-2262; ROSA
 * forward_one src/model.rs:1320-1353, CMix forward_one src/model.rs:1003-1016),
 * ln_out, head. The suffix automaton's idx for this token is given
 * ([n_layers][batch][d] u8) instead of RosaSam::push; the Q/K/V sign bits it
 * would have been pushed (bit_from_activation = value > 0, src/rosa.rs:372)
 * go to qkv_bits ([n_layers][3][batch][d] u8) when non-NULL. rosa_prev /
 * cmix_prev ([n_layers][batch][d]) are the state's x_prev, read when has_prev
 * and overwritten with this token's values; logits [batch][vocab].
 */
int ucr_heron_decode_step(const ullis_heron_dims* dims, uint8_t* arena, const uint16_t* table,
                          const uint32_t* tokens, size_t batch, const uint8_t* idx,
                          float* rosa_prev, float* cmix_prev, int has_prev, float* logits,
                          uint8_t* qkv_bits) {
  size_t d = dims->d_model, f = dims->dim_ffn, v = dims->vocab, L = dims->n_layers;
  size_t b, layer, c, i;
  uint64_t total;
  arena_view a;
  ln_view ln_out;
  packed_view head;
  float *x = NULL, *h = NULL, *tmp = NULL, *xx = NULL, *qi = NULL, *q = NULL, *k = NULL;
  float *vv = NULL, *y = NULL, *key = NULL, *relu2 = NULL;
  int rc = 0;
  a.n = ullis_heron_layout(dims, NULL, 0, &total);
  a.descs = (ullis_tensor_desc*)calloc(a.n, sizeof(ullis_tensor_desc));
  if (!a.descs) return -1;
  ullis_heron_layout(dims, a.descs, a.n, &total);
  a.base = arena;
  XMALLOC(x, d);
  XMALLOC(h, d);
  XMALLOC(tmp, d);
  XMALLOC(xx, d);
  XMALLOC(qi, d);
  XMALLOC(q, d);
  XMALLOC(k, d);
  XMALLOC(vv, d);
  XMALLOC(y, d);
  XMALLOC(key, f);
  XMALLOC(relu2, f);
  if (ln_bind(&a, "ln_out", &ln_out) || packed_bind(&a, "head", v, d, 1, &head)) {
    rc = -3;
    goto done;
  }
  for (b = 0; b < batch; ++b) {
    if (tokens[b] >= v) { rc = -2; goto done; }
    for (c = 0; c < d; ++c) x[c] = ucr_f16_to_f32(table[(size_t)tokens[b] * d + c]);
    for (layer = 0; layer < L; ++layer) {
      char p[ULLIS_NAME_MAX];
      ln_view ln2, ln3;
      packed_view pq, pk, pv, po, kp;
      uint16_t *x_q, *x_k, *x_v, *e, *cx_k, *value;
      float* rp = rosa_prev + (layer * batch + b) * d;
      float* cp = cmix_prev + (layer * batch + b) * d;
      const uint8_t* id = idx + (layer * batch + b) * d;
#define DBIND(view, name, out_, in_, bias_)                                  \
  snprintf(p, sizeof p, "blocks.%zu." name, layer);                          \
  if (packed_bind(&a, p, out_, in_, bias_, &view)) { rc = -3; goto done; }
#define DTBIND(var, name)                                \
  snprintf(p, sizeof p, "blocks.%zu." name, layer);      \
  var = tensor_ptr(&a, p);                               \
  if (!var) { rc = -3; goto done; }
      snprintf(p, sizeof p, "blocks.%zu.ln2", layer);
      if (ln_bind(&a, p, &ln2)) { rc = -3; goto done; }
      snprintf(p, sizeof p, "blocks.%zu.ln3", layer);
      if (ln_bind(&a, p, &ln3)) { rc = -3; goto done; }
      DBIND(pq, "rosa.q", d, d, 1);
      DBIND(pk, "rosa.k", d, d, 1);
      DBIND(pv, "rosa.v", d, d, 1);
      DBIND(po, "rosa.o", d, d, 1);
      DBIND(kp, "ffn.key", f, d, 0);
      DTBIND(x_q, "rosa.x_q");
      DTBIND(x_k, "rosa.x_k");
      DTBIND(x_v, "rosa.x_v");
      DTBIND(e, "rosa.e");
      DTBIND(cx_k, "ffn.x_k");
      DTBIND(value, "ffn.value");
      if (layer == 0) { /* forward_one: h = ln0(x) */
        ln_view ln0;
        snprintf(p, sizeof p, "blocks.%zu.ln0", layer);
        if (ln_bind(&a, p, &ln0)) { rc = -3; goto done; }
        ucr_layer_norm_forward(x, 1, d, ln0.w, ln0.b, h);
      } else {
        memcpy(h, x, d * sizeof(float));
      }
      /* ROSA forward_one (src/model.rs:1320-1353) */
      ucr_layer_norm_forward(h, 1, d, ln3.w, ln3.b, tmp); /* rosa_in */
      time_shift_one(tmp, rp, has_prev, d, xx);
      for (c = 0; c < d; ++c) qi[c] = tmp[c] + xx[c] * ucr_f16_to_f32(x_q[c]);
      ucr_packed_forward(qi, 1, d, d, pq.bits, pq.scale, pq.bias, q);
      for (c = 0; c < d; ++c) qi[c] = tmp[c] + xx[c] * ucr_f16_to_f32(x_k[c]);
      ucr_packed_forward(qi, 1, d, d, pk.bits, pk.scale, pk.bias, k);
      for (c = 0; c < d; ++c) qi[c] = tmp[c] + xx[c] * ucr_f16_to_f32(x_v[c]);
      ucr_packed_forward(qi, 1, d, d, pv.bits, pv.scale, pv.bias, vv);
      if (qkv_bits) {
        uint8_t* qb = qkv_bits + (layer * 3) * batch * d + b * d;
        for (c = 0; c < d; ++c) {
          qb[c] = q[c] > 0.0f;
          qb[batch * d + c] = k[c] > 0.0f;
          qb[2 * batch * d + c] = vv[c] > 0.0f;
        }
      }
      for (c = 0; c < d; ++c) y[c] = (2.0f * (float)id[c] - 1.0f) * ucr_f16_to_f32(e[c]);
      memcpy(rp, tmp, d * sizeof(float)); /* layer.rosa_x_prev = Some(rosa_in) */
      ucr_packed_forward(y, 1, d, d, po.bits, po.scale, po.bias, tmp);
      for (c = 0; c < d; ++c) h[c] += tmp[c];
      /* CMix forward_one (src/model.rs:1003-1016) */
      ucr_layer_norm_forward(h, 1, d, ln2.w, ln2.b, tmp); /* ffn_in */
      time_shift_one(tmp, cp, has_prev, d, xx);
      for (c = 0; c < d; ++c) qi[c] = tmp[c] + xx[c] * ucr_f16_to_f32(cx_k[c]);
      memcpy(cp, tmp, d * sizeof(float)); /* layer.cmix_x_prev = Some(ffn_in) */
      ucr_packed_forward(qi, 1, d, f, kp.bits, kp.scale, NULL, key);
      for (i = 0; i < f; ++i) {
        const float kv = key[i] > 0.0f ? key[i] : 0.0f;
        relu2[i] = kv * kv;
      }
      ucr_fp16_forward(relu2, 1, f, d, value, tmp);
      for (c = 0; c < d; ++c) h[c] += tmp[c];
      memcpy(x, h, d * sizeof(float));
#undef DBIND
#undef DTBIND
    }
    ucr_layer_norm_forward(x, 1, d, ln_out.w, ln_out.b, h);
    ucr_packed_forward(h, 1, d, v, head.bits, head.scale, head.bias, logits + b * v);
  }
done:
  free(x);
  free(h);
  free(tmp);
  free(xx);
  free(qi);
  free(q);
  free(k);
  free(vv);
  free(y);
  free(key);
  free(relu2);
  free(a.descs);
  return rc;
}
