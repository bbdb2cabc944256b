// Internal launchers of libullis_hip (stream-ordered, device pointers, no
// host synchronisation). The C ABI in capi.hip validates arguments and calls
// these; the Heron step in heron.hip composes them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ullis {

enum ActDtype : int { kF16 = 1, kF32 = 2 };

inline long cdiv(long a, long b) { return (a + b - 1) / b; }

// Scaled-gradient operand: values are multiplied by a power of two derived from
// *amax (or by 1 when amax is null) before the fp16 conversion.
struct GradIn {
  const float* p;
  const float* amax;
  // Optional fp16 copy of p already multiplied by grad_scale_from_amax(*amax)
  // (f32_to_f16_sat); GEMMs that can stream fp16 straight to LDS use it.
  const uint16_t* p16 = nullptr;
};

// ------------------------------------------------------------ packed linear

// Output of a packed forward y = bias + scale * (x . S^T).
struct PackedFwdOut {
  float* y32 = nullptr;          // fp32 y, or resid + y when resid is set
  const float* resid = nullptr;  // residual stream input for fused x += y
  uint16_t* y16 = nullptr;       // fp16 y
  uint32_t* sign_bits = nullptr; // bit (row*out + o) = y > 0 (requires out % 32 == 0)
  uint16_t* relu2_16 = nullptr;  // fp16 max(y,0)^2 (CMix key)
};

hipError_t packed_forward(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                          const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                          const PackedFwdOut& o);

// Three packed forwards of one shape (Q, K, V) in one launch, each writing
// only its sign bit-plane (bit = y > 0).
hipError_t packed_forward_bits3(hipStream_t s, const uint16_t* const x[3], long rows, long in,
                               long out, const uint32_t* const bits[3],
                               const uint16_t* const scale[3], const uint16_t* const bias[3],
                               uint32_t* const sign_bits[3]);

// gX = (gY * scale) . S  via bits_t ([in, out] transpose bits) -> fp32 gx.
// gy is fp32 (scaled by amax) or fp16 (already scaled by 1/unscale); result is
// multiplied by out_mul (device scalar, may be null) and 1/gy-scale.
// accumulate: gx += result.
hipError_t packed_backward_input(hipStream_t s, GradIn gy32, const uint16_t* gy16, long rows,
                                 long in, long out, const uint32_t* bits_t, const uint16_t* scale,
                                 float* gx, const float* out_mul, int accumulate);

// Raw G = gY^T . X partials: part[z][out][in], z < splits. x is fp16 [rows, in];
// gy is fp32 scaled (GradIn) or fp16 [rows, out].
hipError_t packed_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* gy16,
                                       const uint16_t* x16, long rows, long in, long out,
                                       int splits, float* part);

// Reduces the partials and applies, per weight, the BinaryConnect latent step
// with g = scale[o] * G * gmul * ste, gmul = (1/gy-scale) * (*extra_mul);
// g_scale[o] = sum_i sign_old[o,i] * G * gmul. Optionally writes g_w.
struct PackedFinish {
  const float* part;
  int splits;
  long out, in;
  const uint16_t* scale;
  const uint32_t* bits_old;
  const float* amax;       // gy scale source (null: unscaled)
  const float* extra_mul;  // device scalar or null
  float ste;
  float lr;
  uint16_t* latent;        // null: no update
  float* latent_res;
  float* g_scale;          // may be null
  float* g_w;              // may be null
  // Fused tail of the update (optional, with latent set): clipped SGD of
  // scale[o] at lr with g_scale[o] (scale_upd/scale_res), and the repack of
  // the updated latent rows into bits_new (requires packed_finish_wave_ok,
  // or in % 64 == 0).
  uint16_t* scale_upd = nullptr;
  float* scale_res = nullptr;
  uint32_t* bits_new = nullptr;
  // Optional diagnostics of the one-wave-per-row finish (CausalLoss,
  // src/model.rs:58-80): row_flips[o] = sign bits of row o the repack
  // changed (bit_flip_count, src/model.rs:150-156); row_step[o] = sum over
  // row o of |latent_new - latent_old| (mean_abs_delta_fp16's terms,
  // src/model.rs:3329-3339).
  uint32_t* row_flips = nullptr;
  float* row_step = nullptr;
};
hipError_t packed_weight_finish(hipStream_t s, const PackedFinish& f);

// Arguments of packed_backward_input / packed_weight_grad_partials /
// fp16_backward_input, for the paired launches below.
// out is the contraction length. A column window of a wider layer (the
// streamed head): gy16 rows of ldgy halves, bits_t rows of ldb bits, k offset
// kofs into bits_t columns and scale (0: ldgy = ldb = out, kofs = 0).
struct PackedDxArgs {
  GradIn gy32;
  const uint16_t* gy16;
  long rows, in, out;
  const uint32_t* bits_t;
  const uint16_t* scale;
  float* gx;
  const float* out_mul;
  int accumulate;
  long ldgy = 0, ldb = 0, kofs = 0;
  // Signed column sums instead of gx (out_mul null, accumulate 0): with
  // col_part set, part[r / 16][c] = sum over 16-row groups of
  // gx[r][c] * (2 sign_idx[r][c] - 1) (sign_idx [rows][in] u8), exactly as
  // column_sum_partials over gx; gx is then only scratch for the non-LDS path.
  const uint8_t* sign_idx = nullptr;
  float* col_part = nullptr;
};
struct WeightGradArgs {
  GradIn gy32;
  const uint16_t* gy16;
  const uint16_t* x16;
  long rows, in, out;
  int splits;
  float* part;
};
struct Fp16DxArgs {
  GradIn gy32;
  long rows, in, out;
  const uint16_t* w;
  float* gx;
  const uint16_t* key16;
  uint16_t* gk16;
  // Optional W^T [in][out]: both operands then stream k-contiguous (same
  // results as with w: every output sums the same products in the same order).
  const uint16_t* w_t = nullptr;
};
// Whether an input gradient of this shape is worth a W^T cache: large
// products (at least 512 256x256 output tiles), where it measured faster.
bool fp16_dx_wants_w_t(long rows, long in, long out);
// Input and weight gradient of one layer in a single launch when both GEMMs
// take the streamed-LDS kernels (the blocks of both share the CUs), else the
// two launches of the functions above; same results either way.
hipError_t packed_backward_pair(hipStream_t s, const PackedDxArgs& dx, const WeightGradArgs& dw);
hipError_t fp16_backward_pair(hipStream_t s, const Fp16DxArgs& dx, const WeightGradArgs& dw);
// in % 32 == 0 and 16-byte aligned part / latent / latent_res / g_w: the
// finish runs one wave per row with vector loads.
bool packed_finish_wave_ok(const PackedFinish& f);
// n % 4 == 0, part / w_res / g_w 16-byte and w 8-byte aligned.
bool fp16_finish_vec_ok(const float* part, long n, const uint16_t* w, const float* w_res,
                        const float* g_w);

// Latent -> bits (row-major) and, if bits_t is non-null, the transposed bits.
hipError_t pack_latent_bits(hipStream_t s, const uint16_t* latent, long out, long in,
                            uint32_t* bits, uint32_t* bits_t);
hipError_t transpose_bits(hipStream_t s, const uint32_t* bits, long out, long in,
                          uint32_t* bits_t);

// Few-row forward products (rows <= kGemvMaxRows; T = 1 decode): the weights
// stream once, x stays in LDS. packed_forward / fp16_forward take these
// paths by themselves when the *_gemv_ok conditions hold.
constexpr int kGemvMaxRows = 8;
bool packed_gemv_ok(long rows, long in, long out, const void* x, int x_dtype,
                    const PackedFwdOut& o);
hipError_t packed_gemv(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                       const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                       const PackedFwdOut& o);
bool fp16_gemv_ok(long rows, long in, long out, const void* x, int x_dtype, const uint16_t* w);
hipError_t fp16_gemv(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                     const uint16_t* w, float* y32, const float* resid, uint16_t* y16);

// -------------------------------------------------------------- fp16 linear

// y = x . W^T (W f16 [out, in]); same output options as packed_forward (no
// bias/scale) plus the fused residual add.
hipError_t fp16_forward(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                        const uint16_t* w, float* y32, const float* resid, uint16_t* y16);

// gX = gY . W -> fp32, or with key16 set: fp16 2*k*gX for k > 0 (CMix ReLU^2
// backward, kept in the gy-scaled domain) written to gk16.
hipError_t fp16_backward_input(hipStream_t s, GradIn gy32, long rows, long in, long out,
                               const uint16_t* w, float* gx, const uint16_t* key16,
                               uint16_t* gk16);

// G = gY^T . X partials [z][out][in]; x fp16 [rows, in].
hipError_t fp16_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* x16, long rows,
                                     long in, long out, int splits, float* part);

// W clipped SGD from the reduced partials (g = G / gy-scale); optional g_w out.
hipError_t fp16_weight_finish(hipStream_t s, const float* part, int splits, long out, long in,
                              const float* amax, float lr, uint16_t* w, float* w_res,
                              float* g_w);

// ---------------------------------------------------------------- LayerNorm

// LayerNorm whose fp16 output feeds time_shift_mix (up to three mixes) in one
// kernel; same results as layer_norm_forward(y16) then time_shift_mix. y16
// receives the fp16 LayerNorm output when keep_y (it is scratch otherwise).
// With resid, the LayerNorm input is resid + x (fp32), written to sum_out.
hipError_t layer_norm_mix_forward(hipStream_t s, const float* x, long rows, long time, long ch,
                                  const uint16_t* w, const uint16_t* b, uint16_t* y16, bool keep_y,
                                  const uint16_t* mix0, uint16_t* out0, const uint16_t* mix1,
                                  uint16_t* out1, const uint16_t* mix2, uint16_t* out2,
                                  const float* resid = nullptr, float* sum_out = nullptr);

// out = a + b elementwise (fp32).
hipError_t add_f32(hipStream_t s, const float* a, const float* b, long n, float* out);
hipError_t layer_norm_forward(hipStream_t s, const float* x, long rows, long ch,
                              const uint16_t* w, const uint16_t* b, float* y32, uint16_t* y16);

// gx = LN backward; mode 0 store, 1 accumulate (gx += ...). amax (optional)
// receives max |gx result|. Column partials go to part[nblk][2][ch];
// returns nblk through *nblk_out.
hipError_t layer_norm_backward_rows(hipStream_t s, const float* x, const float* gy, long rows,
                                    long ch, const uint16_t* w, float* gx, int accumulate,
                                    float* amax, float* part, int* nblk_out);
int layer_norm_backward_blocks(long rows);
// The same backward with at most 256 column-partial blocks whatever the row
// count (rows are strided over a fixed grid): part[nblk][2][ch] with
// nblk = layer_norm_backward_capped_nblk(rows) <= 256.
hipError_t layer_norm_backward_rows_capped(hipStream_t s, const float* x, const float* gy,
                                           long rows, long ch, const uint16_t* w, float* gx,
                                           float* part, int* nblk_out);
int layer_norm_backward_capped_nblk(long rows);
// Partial blocks layer_norm_backward_rows uses for 16-byte aligned x / gy / gx.
int layer_norm_backward_nblk(long rows, long ch);
// LayerNorm backward fed by the backward of the time-shift mix that read its
// fp16 output x16: gy = time_shift_mix_backward(g_s, x16, mix) is formed in
// the same kernel (same values), the mix gradient partials go to
// part_mix[*nblk_mix_out][ch]; g_scratch [rows][ch] is used when the fused
// kernel does not apply. With aligned operands the partial counts are
// layer_norm_backward_nblk and layer_norm_mix_backward_mix_nblk.
hipError_t layer_norm_mix_backward_rows(hipStream_t s, const float* x, const float* g_s,
                                        const uint16_t* x16, const uint16_t* mix, long rows,
                                        long time, long ch, const uint16_t* w, float* gx,
                                        int accumulate, float* amax, float* part, float* part_mix,
                                        float* g_scratch, int* nblk_out, int* nblk_mix_out);
int layer_norm_mix_backward_mix_nblk(long rows, long ch);

// Sums part[nblk][2][ch] -> gw, gb (optional outputs) and, when lr > 0,
// clipped SGD on (w, b) with their carries.
// abort (device, optional): when *abort != 0 no step is applied.
hipError_t layer_norm_param_finish(hipStream_t s, const float* part, int nblk, long ch, float* gw,
                                   float* gb, float lr, uint16_t* w, float* w_res, uint16_t* b,
                                   float* b_res, const uint32_t* abort = nullptr);

// ---------------------------------------------------------------- elementwise

hipError_t fill_f32(hipStream_t s, float* p, long n, float v);
// dst [cols][rows] = src [rows][cols]^T, 16-bit elements.
hipError_t transpose_u16(hipStream_t s, const uint16_t* src, long rows, long cols, uint16_t* dst);
// Device-to-device byte copy as a kernel on stream s.
hipError_t copy_device(hipStream_t s, void* dst, const void* src, long bytes);
hipError_t clipped_sgd(hipStream_t s, uint16_t* values, float* residual, const float* grad, long n,
                       float lr);
hipError_t binaryconnect_sgd(hipStream_t s, uint16_t* values, float* residual, const float* grad,
                             long n, float lr, float grad_scale);
hipError_t sign_pack_bits(hipStream_t s, const float* x, long n, uint32_t* bits);
hipError_t amax_f32(hipStream_t s, const float* x, long n, float* slot);

// shifted_j = x + (x[t-1] - x) * mix_j for up to 3 mixes (time shift per
// sequence of length `time`; t == 0 uses -x). x fp16 [rows, ch].
hipError_t time_shift_mix(hipStream_t s, const uint16_t* x16, long rows, long time, long ch,
                          const uint16_t* mix0, uint16_t* out0, const uint16_t* mix1,
                          uint16_t* out1, const uint16_t* mix2, uint16_t* out2);

// lerp_shift_backward: g_x = g_s - g_s*mix + g_s[t+1]*mix (stored), and
// g_mix[c] = sum g_s * xx with xx recomputed from x16. g_mix column partials
// go to part[nblk][ch]; *nblk_out receives nblk.
hipError_t time_shift_mix_backward(hipStream_t s, const float* g_shifted, const uint16_t* x16,
                                   const uint16_t* mix, long rows, long time, long ch, float* g_x,
                                   float* part, int* nblk_out);

// Number of row chunks (partials) used by the column reductions below.
inline long column_partial_blocks(long rows) { return cdiv(rows, 16); }

// Column sums of v[rows][ch] (times +-1 from idx when idx != null, i.e.
// sum g_y * (2*idx - 1)) into part[nblk][ch].
hipError_t column_sum_partials(hipStream_t s, const float* v, const uint8_t* idx, long rows,
                               long ch, float* part, int* nblk_out, uint16_t* out16 = nullptr,
                               const float* amax = nullptr);
// out16 = f16_sat(v * grad_scale_from_amax(*amax)): the fp16 operand form of a
// scaled fp32 gradient (GradIn::p16). column_sum_partials writes the same
// copy when out16 / amax are given.
hipError_t scale_to_f16(hipStream_t s, const float* v, long n, const float* amax,
                        uint16_t* out16);
// out16 = f16 RNE of v (overflow to +-Inf, Fp16::from_f32).
hipError_t f32_to_f16(hipStream_t s, const float* v, long n, uint16_t* out16);
// Sums part[nblk][ch] -> out (optional) and optional clipped SGD with lr.
hipError_t vector_finish(hipStream_t s, const float* part, int nblk, long ch, float* out,
                         float lr, uint16_t* values, float* residual);

// Destination of a reduced vector: optional fp32 copy and optional clipped
// SGD of an f16 tensor with its carry; the sum is first multiplied by *mul.
struct VecTarget {
  float* out;
  uint16_t* values;
  float* residual;
  float lr;
  const float* mul;
  // optional (device): when *abort != 0 the step is skipped (refused step)
  const uint32_t* abort = nullptr;
};
// Fixed-order sum of part[nblk][ncols] over nblk; columns [0, split) go to a,
// [split, ncols) to b (index relative to split).
hipError_t partial_reduce(hipStream_t s, const float* part, int nblk, long ncols, long split,
                          const VecTarget& a, const VecTarget& b);

// ROSA: idx channel-major [batch][ch][time] u8 -> y16 row-major (2*idx-1)*e
// and the row-major idx tape.
hipError_t rosa_expand(hipStream_t s, const uint8_t* idx_cm, const uint16_t* e, long batch,
                       long time, long ch, uint16_t* y16, uint8_t* idx_rm);
// rosa_expand of `layers` consecutive layers in one launch: idx_cm, y16 and
// idx_rm advance by batch*time*ch per layer, layer l uses e_host[l] (host
// array) / e_dev[l] (the same pointers in device memory).
hipError_t rosa_expand_layers(hipStream_t s, const uint8_t* idx_cm, const uint16_t* const* e_host,
                              const uint16_t* const* e_dev, long layers, long batch, long time,
                              long ch, uint16_t* y16, uint8_t* idx_rm);

// ----------------------------------------------------------- T = 1 decode
// Fused decode kernels (decode.hip) for rows <= 8, d % 128 == 0, d <= 1024,
// f % 32 == 0 and the rows' fp16 inputs within 64 KiB of LDS.
bool decode_fused_ok(long rows, long d, long f);
struct DecodeQkv {
  const uint16_t* mix[3];
  const uint32_t* bits[3];
  const uint16_t* scale[3];
  const uint16_t* bias[3];
  uint32_t* planes[3];  // sign bits, bit b*d + c
};
struct DecodeO {
  const uint8_t* idx;  // u8 [rows][d], 4-byte aligned
  const uint16_t* e;
  const uint32_t* bits;
  const uint16_t* scale;
  const uint16_t* bias;
};
// x = f32 table rows of tokens (ids >= vocab: zero rows; *invalid = their
// count, when set), then LN0 in place when ln0_w is set (d <= 1024). rows <= 8.
hipError_t decode_embed(hipStream_t s, const uint16_t* table, long vocab, long d,
                        const uint32_t* tokens, long rows, float* x, uint32_t* invalid,
                        const uint16_t* ln0_w, const uint16_t* ln0_b);
// part 0: planes_j = sign(bias_j + scale_j * (mix_j(LN(x), prev_in) . S_j^T)),
// prev_out = LN(x); part 1: x2 = x + bias + scale * (((2 idx - 1) e) . S^T);
// part 2: both in one launch.
hipError_t decode_qkvo(hipStream_t s, const float* x, float* x2, long rows, long d, int part,
                       const uint16_t* ln_w, const uint16_t* ln_b, const float* prev_in,
                       float* prev_out, const DecodeQkv& p, const DecodeO& po);
// r2 = f16(max(k, 0)^2), k = scale * (mix(LN(x), prev_in) . S^T) [rows][f];
// prev_out = LN(x).
hipError_t decode_key(hipStream_t s, const float* x, long rows, long d, long f,
                      const uint16_t* ln_w, const uint16_t* ln_b, const float* prev_in,
                      float* prev_out, const uint16_t* mix, const uint32_t* bits,
                      const uint16_t* scale, uint16_t* r2);
// logits = bias + scale * (LN(x) . S^T) [rows][vocab].
hipError_t decode_head(hipStream_t s, const float* x, long rows, long d, long vocab,
                       const uint16_t* ln_w, const uint16_t* ln_b, const uint32_t* bits,
                       const uint16_t* scale, const uint16_t* bias, float* logits);
// General shapes: out_j = f16(x + (prev_in - x) * mix_j) for the given mixes
// (null: skipped), prev_out = x; x / prev fp32 [rows][d].
hipError_t decode_mix(hipStream_t s, const float* x, const float* prev_in, float* prev_out,
                      long rows, long d, const uint16_t* mix0, uint16_t* out0,
                      const uint16_t* mix1, uint16_t* out1, const uint16_t* mix2,
                      uint16_t* out2);
// next[r] = argmax_v logits[r][v] (lowest index among equal maxima).
hipError_t argmax_rows(hipStream_t s, const float* logits, long rows, long vocab, uint32_t* next);

// ---------------------------------------------------------------- embedding
// x = f32 rows of the f16 table at tokens (ids >= vocab: zero rows, counted
// into *invalid when non-null).
hipError_t embedding_gather(hipStream_t s, const uint16_t* table, long vocab, long d,
                            const uint32_t* tokens, long rows, float* x, uint32_t* invalid);
// Clipped SGD of table rows with g, rows sharing a token applied in row order.
// abort (device, optional): when *abort != 0 nothing is applied.
hipError_t embedding_scatter_sgd(hipStream_t s, uint16_t* table, float* residual, long vocab,
                                 long d, const uint32_t* tokens, long rows, const float* g,
                                 float lr, const uint32_t* abort = nullptr);

// --------------------------------------------------------------- head + CE

struct HeadCe {
  long rows, time, d, vocab;
  const uint16_t* hidden16;  // [rows, d]
  const uint32_t* bits;      // [vocab, d]
  const uint32_t* bits_t;    // [d, vocab]
  const uint16_t* scale;     // [vocab]
  const uint16_t* bias;      // [vocab] or null
  const uint32_t* targets;   // [rows]
  uint32_t ignore_id;
  long horizon = 1;          // target of row r is targets[r + horizon]
  // optional (device): += the number of targets >= vocab other than ignore_id
  // (their rows are left out of the loss and the gradient)
  uint32_t* invalid = nullptr;
  // outputs
  float* row_loss;      // [rows]
  float* stats;         // [4]: mean_loss, n_valid, gscale, loss_sum
  float* g_hidden;      // [rows, d] fp32
  float* g_scale;       // [vocab] or null
  float* g_bias;        // [vocab] or null
  float* g_w;           // [vocab, d] or null (tests)
  // update (lr > 0): latent step + scale clipped SGD (lr) + bias (8 lr)
  float lr;
  float ste;
  uint16_t* latent;
  float* latent_res;
  uint16_t* scale_upd;  // scale tensor to update (same as scale) or null
  float* scale_res;
  uint16_t* bias_upd;
  float* bias_res;
  uint32_t* bits_new;   // repacked bits (may alias bits only after all reads)
  uint32_t* bits_t_new;
  float* stats2 = nullptr;  // optional second copy of stats
  // Deferred mode (non-null): the weight-gradient partials of every vocab
  // chunk go to gpart_all[chunk][splits][vc][d] and no update runs; the
  // caller runs them later (head_ce_bias_partials, head_ce_chunk_cols,
  // head_ce_splits describe the layout).
  float* gpart_all = nullptr;
};
size_t head_ce_workspace_bytes(long rows, long d, long vocab);
hipError_t head_ce(hipStream_t s, const HeadCe& h, void* workspace);
long head_ce_chunk_cols(long vocab, long d);
int head_ce_splits(long rows, long d, long vocab);
// g_bias partials [ceil(rows/32)][vocab] (unscaled: multiply by gscale).
float* head_ce_bias_partials(void* workspace, long rows, long d, long vocab);

// ------------------------------------------------------- step diagnostics
// CausalLoss of a train step (src/model.rs:58-80): word indices of the fields
// of ullis_hip_causal_loss (include/ullis_hip.h), all 4 bytes wide.
enum DiagField : int {
  kDiagNextToken = 0,
  kDiagNextTokenCount,
  kDiagFlipsTotal,
  kDiagP10,
  kDiagP50,
  kDiagP90,
  kDiagUnigramCe,
  kDiagUniqueTargets,
  kDiagFlipsHead,
  kDiagFlipsCmix,
  kDiagFlipsRosaO,
  kDiagEmbedGradRms,
  kDiagHeadScaleGradRms,
  kDiagHeadScaleRms,
  kDiagResidualAbsMean,
  kDiagCmixValueRms,
  kDiagHeadLatentAbsMean,
  kDiagHeadLatentStepAbs,
  kDiagHeadBiasRms,
  kDiagFields
};
// One reduction of the diagnostics: field = sum / denom (sqrt of it for an
// rms), or, for kSumU32, the integer sum (a flip count).
struct DiagTask {
  enum Kind : int { kSqF32, kAbsF32, kSqF16, kAbsF16, kSumF32, kSumU32 };
  int kind;
  int field;
  int rms;
  const void* p;
  long n;
  long denom;
};
constexpr int kDiagMaxTasks = 16;
struct DiagOut {
  void* dst;  // device ullis_hip_causal_loss
};
struct DiagArgs {
  const float* row_loss;    // [rows]
  const uint32_t* targets;  // [rows] labels
  long rows, time, vocab;
  uint32_t ignore_id;
  const float* stats;       // the step's {mean_loss, n_valid, gscale, loss_sum}
  void* out;                // device ullis_hip_causal_loss
};
size_t diag_workspace_bytes(long vocab);
hipError_t causal_loss_diag(hipStream_t s, const DiagArgs& a, const DiagTask* tasks, int ntasks,
                            void* workspace);

// ------------------------------------------- batched end-of-step updates
// A train step can defer every parameter update to its end (no later kernel
// of the step reads an updated parameter), then run all updates of one kind
// in a single launch: blocks [block0, block0 + blocks) of the batched grid
// belong to one job. Job tables live in device memory, ordered by block0.

// Column reduction of part[nblk][ncols] with steps on up to two targets
// (see partial_reduce); a.lr / b.lr hold multipliers of the launch's lr.
struct VecJob {
  const float* part;
  int nblk;
  long ncols, split;
  VecTarget a, b;
  int block0;
};
inline int vec_job_blocks(long ncols) { return (int)cdiv(ncols, 64); }

// Four rows per block, one wave each (packed_finish_wave_ok must hold, with
// bits_new set or null); f.lr is ignored (the launch's lr is used).
inline int finish_job_blocks(long rows) { return (int)cdiv(rows, 4); }
struct FinishJob {
  PackedFinish f;
  int block0;
};

// fp16 weight finish, 1024 elements per block (fp16_finish_vec_ok must hold).
inline int f16_job_blocks(long n) { return (int)cdiv(n, 1024); }
struct F16Job {
  const float* part;
  int splits;
  long n;
  const float* amax;
  uint16_t* w;
  float* w_res;
  int block0;
};

// bits [out][in] -> bits_t [in][out], out % 32 == 0, in % 32 == 0; eight 32x32
// bit blocks per 256-thread block.
struct TransJob {
  const uint32_t* bits;
  long out, in;
  uint32_t* bits_t;
  int block0;
};

// abort (device, optional): when *abort != 0 the launches change nothing (a
// refused step); the finish then writes zero row flips / steps.
hipError_t run_vec_jobs(hipStream_t s, const VecJob* jobs, int njobs, int nblocks, float lr,
                        const uint32_t* abort = nullptr);
hipError_t run_finish_jobs(hipStream_t s, const FinishJob* jobs, int njobs, int nblocks, float lr,
                           const uint32_t* abort = nullptr);
hipError_t run_f16_jobs(hipStream_t s, const F16Job* jobs, int njobs, int nblocks, float lr,
                        const uint32_t* abort = nullptr);
hipError_t run_trans_jobs(hipStream_t s, const TransJob* jobs, int njobs, int nblocks,
                          const uint32_t* abort = nullptr);

}  // namespace ullis
