/*
 * cpu_ref: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's deterministic CPU backend for the
 * packed +-1 linear / LayerNorm / streamed-CE hot path (Vladislav-Kalinkin/ullis
 * 0.10.0, src/precision.rs and src/model.rs). It is the parity oracle for the
 * HIP library and the CPU throughput baseline in bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path never calls it.
 *
 * Conventions: activations f32, FP16 parameters as raw u16 bit patterns, FP32
 * carries, packed sign bits as LSB-first u32 words. Every loop keeps the
 * reference's order of f32 operations (Rust never contracts a*b+c into an
 * FMA; this file is compiled with -ffp-contract=off).
 *
 * Parity pins: see the header of cpu_ref.c for which check pins which function.
 */
#ifndef ULLIS_CPU_REF_H
#define ULLIS_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#include "../include/ullis_heron_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

/* a1: IEEE binary16 */
uint16_t ucr_f16_from_f32(float value);
float ucr_f16_to_f32(uint16_t bits);
void ucr_f16_from_f32_array(const float* src, uint16_t* dst, size_t n);
void ucr_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* a2 / a3: FP16 storage updates with FP32 carry (per element, in order) */
void ucr_clipped_sgd(uint16_t* values, float* residual, const float* gradient, size_t n,
                     float learning_rate);
void ucr_binaryconnect_sgd(uint16_t* values, float* residual, const float* gradient, size_t n,
                           float learning_rate, float gradient_scale);

/* a4: bit packing */
size_t ucr_packed_word_count(size_t weights);
void ucr_pack_latent_bits(const uint16_t* latent, size_t n, uint32_t* bits);
void ucr_sign_pack_bits(const float* x, size_t n, uint32_t* bits);
void ucr_transpose_bits(const uint32_t* bits, size_t out, size_t in, uint32_t* bits_t);
size_t ucr_bit_flip_count(const uint32_t* before, const uint32_t* after, size_t words);

/* a5-a8: packed +-1 linear */
int ucr_packed_forward(const float* x, size_t rows, size_t in, size_t out, const uint32_t* bits,
                       const uint16_t* scale, const uint16_t* bias, float* y);
int ucr_packed_backward_ste(const float* x, const float* gy, size_t rows, size_t in, size_t out,
                            const uint32_t* bits, const uint16_t* scale, float* g_w, float* g_x,
                            float* g_scale, float* g_bias);
/* a9: latent BinaryConnect SGD, then scale and bias clipped SGD, then rebinarize */
int ucr_packed_apply_sgd(size_t in, size_t out, uint16_t* latent, float* latent_res,
                         uint16_t* scale, float* scale_res, uint16_t* bias, float* bias_res,
                         uint32_t* bits, const float* g_w, const float* g_scale,
                         const float* g_bias, float learning_rate, float ste_scale);

/* a10 / a11: LayerNorm */
int ucr_layer_norm_forward(const float* x, size_t rows, size_t ch, const uint16_t* weight,
                           const uint16_t* bias, float* y);
int ucr_layer_norm_backward(const float* x, const float* gy, size_t rows, size_t ch,
                            const uint16_t* weight, float* gx, float* gw, float* gb);

/* a12 */
int ucr_causal_ce_row_valid(size_t row, size_t time, size_t horizon, const uint32_t* targets,
                            size_t n_targets, uint32_t ignore_id);
float ucr_causal_ce_gradient_scale(size_t n_valid, size_t time);

/* a13: packed head + next-token CE (CPU branch of apply_head_ce), no update */
int ucr_head_ce(const float* hidden, size_t rows, size_t time, size_t d, size_t vocab,
                const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                const uint32_t* targets, uint32_t ignore_id, float* mean_loss, size_t* n_valid,
                float* row_loss, float* g_hidden, float* g_w, float* g_scale, float* g_bias);
/* the same with the target of row r at targets[r + horizon] (horizon 1 above) */
int ucr_head_ce_horizon(const float* hidden, size_t rows, size_t time, size_t horizon, size_t d,
                        size_t vocab, const uint32_t* bits, const uint16_t* scale,
                        const uint16_t* bias, const uint32_t* targets, uint32_t ignore_id,
                        float* mean_loss, size_t* n_valid, float* row_loss, float* g_hidden,
                        float* g_w, float* g_scale, float* g_bias);

/* CausalLoss statistics (src/model.rs:3293-3390) */
float ucr_rms(const float* v, size_t n);
float ucr_rms_fp16(const uint16_t* v, size_t n);
float ucr_mean_abs(const float* v, size_t n);
float ucr_mean_abs_fp16(const uint16_t* v, size_t n);
float ucr_mean_abs_delta_fp16(const uint16_t* before, const uint16_t* after, size_t n);
/* p10 / p50 / p90 of the finite losses of valid rows (horizon 1) */
void ucr_loss_percentiles(const float* row_loss, size_t rows, size_t time, const uint32_t* targets,
                          uint32_t ignore_id, float* out3);
/* CE of the batch's target unigram over valid rows; *unique = distinct targets */
float ucr_unigram_cross_entropy(const uint32_t* targets, size_t rows, size_t time,
                                uint32_t ignore_id, size_t* unique);

/* a14: FP16 linear (CMix value) */
int ucr_fp16_forward(const float* x, size_t rows, size_t in, size_t out, const uint16_t* w,
                     float* y);
int ucr_fp16_backward(const float* x, const float* gy, size_t rows, size_t in, size_t out,
                      const uint16_t* w, float* g_x, float* g_w);

/* a15: CMix pieces */
int ucr_time_shift_delta(const float* x, size_t batch, size_t time, size_t ch, float* xx);
int ucr_lerp_shift_backward(const float* xx, const uint16_t* mix, const float* g_shifted,
                            size_t batch, size_t time, size_t ch, float* g_x, float* g_mix);

/* a16: ROSA output expansion and e gradient */
int ucr_rosa_y_from_idx(const uint8_t* idx, const uint16_t* e, size_t rows, size_t ch, float* y);
int ucr_rosa_e_grad(const float* g_y, const uint8_t* idx, size_t rows, size_t ch, float* g_e);

/* a17: one Heron train step on the parameter arena, embedding excluded */
/* The CausalLoss fields train_step_on fills (src/model.rs:2997-3024), except
 * residual_abs_mean (the embedding carry, outside the arena). */
typedef struct ucr_step_stats {
  float mean_loss;
  uint64_t n_valid;
  uint64_t flips_head;
  uint64_t flips_cmix;
  uint64_t flips_rosa_o;
  float loss_p10, loss_p50, loss_p90;
  float unigram_ce;
  uint64_t unique_targets;
  float embed_grad_rms;
  float head_scale_grad_rms;
  float head_scale_rms;
  float cmix_value_rms;
  float head_latent_abs_mean;
  float head_latent_step_abs;
  float head_bias_rms;
} ucr_step_stats;

int ucr_heron_train_step(const ullis_heron_dims* dims, uint8_t* arena, const float* x_emb,
                         const uint32_t* labels, uint32_t ignore_id, size_t batch, size_t time,
                         float learning_rate, const uint8_t* rosa_idx, float* g_emb,
                         float* row_loss, uint32_t* qkv_bits, ucr_step_stats* stats);

/* T = 1 decode of generate_step (src/model.rs:2717-2753) for `batch` sequences,
 * the automaton's indices of this token given ([n_layers][batch][d]);
 * rosa_prev / cmix_prev [n_layers][batch][d] are read when has_prev and
 * overwritten; logits [batch][vocab]; qkv_bits (optional) the Q/K/V sign bits
 * [n_layers][3][batch][d] u8. */
int ucr_heron_decode_step(const ullis_heron_dims* dims, uint8_t* arena, const uint16_t* table,
                          const uint32_t* tokens, size_t batch, const uint8_t* idx,
                          float* rosa_prev, float* cmix_prev, int has_prev, float* logits,
                          uint8_t* qkv_bits);

/* Embedding gather and sequential scatter SGD (src/model.rs:2866-2873, 2986-2993). */
int ucr_embedding_gather(const uint16_t* table, size_t d, const uint32_t* tokens, size_t rows,
                         float* x);
int ucr_embedding_scatter_sgd(uint16_t* table, float* residual, size_t d,
                              const uint32_t* tokens, size_t rows, const float* g_x,
                              float learning_rate);

/* Exported copy of the arena layout for ctypes callers. */
size_t ucr_heron_layout(const ullis_heron_dims* dims, ullis_tensor_desc* out, size_t cap,
                        uint64_t* bytes);

#ifdef __cplusplus
}
#endif

#endif /* ULLIS_CPU_REF_H */
