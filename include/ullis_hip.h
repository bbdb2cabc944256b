/*
 * libullis_hip: MI355X (gfx950) backend for the Ullis packed +-1 linear /
 * LayerNorm / streamed cross-entropy training hot path.
 *
 * This C ABI replaces the GPU runtime that Ullis' model code calls through
 * `Option<&MetalTrainRuntime>` (src/model.rs:1537-1542), i.e. the hot-path
 * methods of `MetalRuntime` (src/metal.rs). Every entry point names the
 * reference method it replaces. Differences by design:
 *   - arguments are DEVICE pointers that persist across calls (parameters,
 *     latents, carries, tapes); nothing is copied host<->device implicitly;
 *   - calls are stream-ordered and asynchronous; ullis_hip_sync() waits
 *     (MetalRuntime blocks in every submit, src/metal.rs:722-740);
 *   - GEMM operands (activations) are IEEE fp16, the residual stream and
 *     gradients fp32; parameters keep the reference's layouts exactly:
 *     f16 bit patterns as uint16_t, fp32 carries, LSB-first uint32_t sign
 *     words row-major [out, in] (src/model.rs:2266-2272);
 *   - errors are status codes (0 ok, negative failure) with a message from
 *     ullis_hip_last_error() instead of anyhow::Result; shape rules follow
 *     LinearDispatchShape / check_binary_shape (src/metal.rs:62-87, 3512-3546):
 *     zero-sized dimensions and > INT32_MAX extents are rejected.
 * A context is not thread safe (MetalRuntime is !Sync, src/metal.rs:456).
 */
#ifndef ULLIS_HIP_H
#define ULLIS_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "ullis_heron_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ULLIS_HIP_OK 0
#define ULLIS_HIP_ERR_INVALID (-1) /* shape or argument rejected before launch */
#define ULLIS_HIP_ERR_RUNTIME (-3) /* HIP runtime / kernel error */
#define ULLIS_HIP_ERR_NOMEM (-4)

#define ULLIS_HIP_F16 1
#define ULLIS_HIP_F32 2

typedef struct ullis_hip_ctx ullis_hip_ctx;
typedef struct ullis_hip_heron ullis_hip_heron;

/* ---- context, memory, timing (MetalRuntime::new, src/metal.rs:466-596;
 *      buffer pool src/metal.rs:342-414, 625-720) ---- */
int ullis_hip_version(void);
int ullis_hip_device_count(int* count);
int ullis_hip_create(int device, ullis_hip_ctx** out);
void ullis_hip_destroy(ullis_hip_ctx* ctx);
const char* ullis_hip_last_error(const ullis_hip_ctx* ctx);
int ullis_hip_sync(ullis_hip_ctx* ctx);
int ullis_hip_malloc(ullis_hip_ctx* ctx, size_t bytes, void** ptr);
int ullis_hip_free(ullis_hip_ctx* ctx, void* ptr);
/* synchronous copies */
int ullis_hip_upload(ullis_hip_ctx* ctx, void* dst_device, const void* src_host, size_t bytes);
int ullis_hip_download(ullis_hip_ctx* ctx, void* dst_host, const void* src_device, size_t bytes);
/* stream-ordered device copy */
int ullis_hip_copy(ullis_hip_ctx* ctx, void* dst_device, const void* src_device, size_t bytes);
/* Events on the context stream; slot in [0, 16). */
int ullis_hip_event_record(ullis_hip_ctx* ctx, int slot);
int ullis_hip_event_elapsed_ms(ullis_hip_ctx* ctx, int start_slot, int end_slot, float* ms);
/* No reference counterpart (measurement): the next kernel this thread
 * launches records its own start and end timestamps into event slots
 * start_slot / end_slot (hipExtLaunchKernel); read them with
 * ullis_hip_event_elapsed_ms. The arming is per thread and is consumed by
 * that one launch. */
int ullis_hip_time_next_launch(ullis_hip_ctx* ctx, int start_slot, int end_slot);

/* ---- unit operations ---- */

/* MetalRuntime::layer_norm, src/metal.rs:1590-1626. x fp32 [rows, channels];
 * weight/bias f16 [channels]; writes y32 and/or y16 (either may be NULL). */
int ullis_hip_layer_norm(ullis_hip_ctx* ctx, const float* x, const uint16_t* weight,
                         const uint16_t* bias, size_t rows, size_t channels, float* y32,
                         uint16_t* y16);

/* MetalRuntime::layer_norm_backward, src/metal.rs:1628-1703. */
int ullis_hip_layer_norm_backward(ullis_hip_ctx* ctx, const float* x, const float* gy,
                                  const uint16_t* weight, size_t rows, size_t channels, float* gx,
                                  float* gw, float* gb);

/* No counterpart in the reference: ullis_hip_layer_norm_backward for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). It calls no allocator: the
 * gamma / beta column partials live in a static 8 MiB device array that the
 * library holds on every GPU it runs on until the process ends, which limits
 * channels to 4096 (larger values are rejected with ULLIS_HIP_ERR_INVALID).
 * gx, gw and gb are the same quantities as ullis_hip_layer_norm_backward's
 * (the partials are grouped differently, so gw / gb may differ in the last
 * bits). Calls on one GPU share the array: calls that overlap on that GPU
 * (other streams, other threads) race. */
int ullis_hip_layer_norm_backward_static(ullis_hip_ctx* ctx, const float* x, const float* gy,
                                         const uint16_t* weight, size_t rows, size_t channels,
                                         float* gx, float* gw, float* gb);

/* MetalRuntime::binary_linear, src/metal.rs:1705-1751:
 * y = bias + scale * (x . S^T). x is [rows, in] of x_dtype (ULLIS_HIP_F16 or
 * ULLIS_HIP_F32); bias may be NULL; y32 / y16 may be NULL. */
int ullis_hip_binary_linear(ullis_hip_ctx* ctx, const void* x, int x_dtype, const uint32_t* bits,
                            const uint16_t* scale, const uint16_t* bias, size_t rows, size_t in,
                            size_t out, float* y32, uint16_t* y16);

/* MetalRuntime::binary_linear_backward, src/metal.rs:2578-2682 (the STE of
 * PackedBinaryLinear::backward_ste, src/model.rs:745-796): gx, gw, g_scale and
 * (has_bias) g_bias, all overwritten, fp32. x fp16 [rows, in], gy fp32 [rows, out].
 * gx / g_bias may be NULL. */
int ullis_hip_binary_linear_backward(ullis_hip_ctx* ctx, const uint16_t* x16, const float* gy,
                                     const uint32_t* bits, const uint16_t* scale, int has_bias,
                                     size_t rows, size_t in, size_t out, float* gx, float* gw,
                                     float* g_scale, float* g_bias);

/* MetalRuntime::apply_latent_sgd, src/metal.rs:3006-3051: BinaryConnect step
 * on latent/residual with gradient * ste_scale, then bits = latent >= 0
 * (and bits_t, the [in, out] transpose bits, when non-NULL). In place. */
int ullis_hip_apply_latent_sgd(ullis_hip_ctx* ctx, uint16_t* latent, float* residual,
                               const float* gradient, size_t out, size_t in, float learning_rate,
                               float ste_scale, uint32_t* bits, uint32_t* bits_t);

/* MetalRuntime::fp16_linear, src/metal.rs:2790-2827: y = x . W^T, W f16 [out, in]. */
int ullis_hip_fp16_linear(ullis_hip_ctx* ctx, const void* x, int x_dtype, const uint16_t* w,
                          size_t rows, size_t in, size_t out, float* y32, uint16_t* y16);

/* MetalRuntime::fp16_linear_backward, src/metal.rs:2829-2908: gx = gy . W,
 * gw = gy^T . x (fp32, overwritten). gx may be NULL. */
int ullis_hip_fp16_linear_backward(ullis_hip_ctx* ctx, const uint16_t* x16, const float* gy,
                                   const uint16_t* w, size_t rows, size_t in, size_t out,
                                   float* gx, float* gw);

/* MetalRuntime::clipped_sgd_fp16 / binaryconnect_sgd_fp16, src/metal.rs:3053-3102. In place. */
int ullis_hip_clipped_sgd_fp16(ullis_hip_ctx* ctx, uint16_t* params, float* residual,
                               const float* gradient, size_t n, float learning_rate);
int ullis_hip_binaryconnect_sgd_fp16(ullis_hip_ctx* ctx, uint16_t* params, float* residual,
                                     const float* gradient, size_t n, float learning_rate);

/* MetalRuntime::sign_pack_bits (kernel ullis_sign_pack_bits, rwkv8.metal:112-129):
 * bit i = x[i] > 0, LSB-first. */
int ullis_hip_sign_pack_bits(ullis_hip_ctx* ctx, const float* x, size_t n, uint32_t* bits);

/* No reference counterpart: bits of the [in, out] transpose of a packed
 * [out, in] matrix (the GPU input-gradient operand). */
int ullis_hip_transpose_bits(ullis_hip_ctx* ctx, const uint32_t* bits, size_t out, size_t in,
                             uint32_t* bits_t);

/* MetalRuntime::packed_head_train_sgd, src/metal.rs:3300-3510, as driven by
 * UllisHeron::apply_head_ce (src/model.rs:3145-3193): CE of row r against
 * targets[r + horizon] over the packed head (causal_ce_row_valid,
 * src/model.rs:27-39; apply_head_ce passes horizon 1), streamed over vocab
 * tiles (no [rows, vocab] buffer), then the head update: BinaryConnect latent
 * step (ste_scale), scale clipped SGD at learning_rate and bias clipped SGD
 * at 8 x learning_rate, then bits / bits_t repack. learning_rate == 0
 * computes gradients only. stats4 (device) receives {mean_loss, n_valid,
 * gradient_scale, loss_sum}. g_scale / g_bias / g_w (device, optional)
 * receive the gradients. A target >= vocab other than ignore_id (which the
 * reference's train step refuses, src/model.rs:2852-2861) leaves its row out
 * of the loss and the gradient and is counted into *invalid (device u32,
 * optional, accumulated); the caller decides whether to keep the update. */
int ullis_hip_packed_head_train_sgd(ullis_hip_ctx* ctx, const uint16_t* hidden16, uint32_t* bits,
                                    uint32_t* bits_t, uint16_t* scale, uint16_t* bias,
                                    uint16_t* latent, float* latent_residual,
                                    float* scale_residual, float* bias_residual,
                                    const uint32_t* targets, size_t rows, size_t time, size_t d,
                                    size_t vocab, size_t horizon, uint32_t ignore_id,
                                    float learning_rate, float ste_scale, float* row_loss,
                                    float* stats4, float* g_hidden, float* g_scale, float* g_bias,
                                    float* g_w, uint32_t* invalid);

/* Embedding gather of UllisHeron::train_step_on (src/model.rs:2866-2873):
 * x[r] = the f16 table row tokens[r] as fp32 (table [vocab, d]). The
 * reference rejects an id >= vocab before the step (src/model.rs:2852-2861);
 * here tokens are device data, so such a row is written as zeros and counted
 * into *invalid (device u32, accumulated; optional) for the caller to check. */
int ullis_hip_embedding_gather(ullis_hip_ctx* ctx, const uint16_t* table, size_t vocab, size_t d,
                               const uint32_t* tokens, size_t rows, float* x, uint32_t* invalid);

/* Embedding scatter-SGD of UllisHeron::train_step_on (src/model.rs:2986-2993):
 * for r in row order, clipped SGD (Fp16Storage::apply_clipped_sgd) of table
 * row tokens[r] with g[r] ([rows, d] fp32), in place with its fp32 carry.
 * Rows sharing a token are applied in row order, as the reference's
 * sequential loop does; ids >= vocab are skipped. */
int ullis_hip_embedding_scatter_sgd(ullis_hip_ctx* ctx, uint16_t* table, float* residual,
                                    size_t vocab, size_t d, const uint32_t* tokens, size_t rows,
                                    const float* g, float learning_rate);

/* ---- block-level methods of the Metal train step ----
 * The reference moves train tapes as MetalBuffers from a block's forward to
 * its backward (src/model.rs:1242-1256, 1525-1535); here the caller owns the
 * tape: a device buffer of *_tape_bytes() bytes, 256-byte aligned, filled by
 * the forward and read by the backward of the same block. GEMM operands
 * (block inputs, tapes) are fp16; an fp32 x is rounded to fp16 first. The
 * parameter updates the reference runs on the GPU inside these methods run
 * here too, in place (latent, residual, bits, and bits_t when non-NULL;
 * NULL bits_t is rebuilt in scratch for the input gradient); the small
 * vectors the reference steps on the host (key / O scale, O bias, e, the mix
 * vectors) are returned as gradients, for ullis_hip_clipped_sgd_fp16. */
size_t ullis_hip_cmix_tape_bytes(size_t rows, size_t d_model, size_t dim_ffn);
size_t ullis_hip_rosa_tape_bytes(size_t rows, size_t channels);

/* MetalRuntime::cmix_block_forward, src/metal.rs:1891 (CMix forward_tape,
 * src/model.rs:1018-1078): s = x + (x[t-1] - x) * mix, k = key(s) (packed,
 * no bias), r = max(k, 0)^2, out = r . value_weight^T (value_weight f16
 * [d_model, dim_ffn]). x [batch*time, d_model] of x_dtype; out fp32, the
 * block's contribution without the residual. */
int ullis_hip_cmix_block_forward(ullis_hip_ctx* ctx, const void* x, int x_dtype,
                                 const uint16_t* mix, const uint32_t* key_bits,
                                 const uint16_t* key_scale, const uint16_t* value_weight,
                                 size_t batch, size_t time, size_t d_model, size_t dim_ffn,
                                 float* out, void* tape);

/* MetalRuntime::cmix_block_backward_sgd, src/metal.rs:2165 (driven by CMix
 * backward_update, src/model.rs:1080-1143): from gy (fp32 [batch*time,
 * d_model], gradient of out) on the pre-update weights: g_x (overwritten),
 * g_mix [d_model], g_key_scale [dim_ffn]; then the value weight clipped SGD
 * and the key BinaryConnect step (gradient x ste_scale) with the repack. */
int ullis_hip_cmix_block_backward_sgd(ullis_hip_ctx* ctx, const void* tape, const float* gy,
                                      const uint16_t* mix, uint32_t* key_bits,
                                      uint32_t* key_bits_t, const uint16_t* key_scale,
                                      uint16_t* key_latent, float* key_residual,
                                      uint16_t* value_weight, float* value_residual,
                                      size_t batch, size_t time, size_t d_model, size_t dim_ffn,
                                      float learning_rate, float ste_scale, float* g_x,
                                      float* g_mix, float* g_key_scale);

/* MetalRuntime::rosa_block_forward, src/metal.rs:1334-1484, up to the
 * suffix automaton: q/k/v inputs x + (x[t-1] - x) * mix_{q,k,v}, the three
 * packed projections with bias, and their sign bit-planes (bit
 * row*channels + c = projection > 0, LSB-first u32, ceil(batch*time*
 * channels / 32) words each) for rosa_qkv_batch_packed_channel_major
 * (src/rosa.rs:486-513), which stays with the caller. */
int ullis_hip_rosa_qkv_forward(ullis_hip_ctx* ctx, const void* x, int x_dtype,
                               const uint16_t* mix_q, const uint16_t* mix_k,
                               const uint16_t* mix_v, const uint32_t* q_bits,
                               const uint16_t* q_scale, const uint16_t* q_bias,
                               const uint32_t* k_bits, const uint16_t* k_scale,
                               const uint16_t* k_bias, const uint32_t* v_bits,
                               const uint16_t* v_scale, const uint16_t* v_bias, size_t batch,
                               size_t time, size_t channels, uint32_t* q_plane,
                               uint32_t* k_plane, uint32_t* v_plane);

/* The rest of MetalRuntime::rosa_block_forward (src/metal.rs:1485-1511):
 * y = (2 idx - 1) * e (rosa_qkv_out_batched_channel_major, src/rosa.rs:
 * 614-639) from the automaton's output idx (u8, channel-major [batch]
 * [channels][time]), out = O(y) with bias, fp32 [batch*time, channels].
 * The tape keeps y (fp16) and idx (row-major). */
int ullis_hip_rosa_out_forward(ullis_hip_ctx* ctx, const uint8_t* idx, const uint16_t* e,
                               const uint32_t* o_bits, const uint16_t* o_scale,
                               const uint16_t* o_bias, size_t batch, size_t time,
                               size_t channels, float* out, void* tape);

/* MetalRuntime::rosa_o_stop_grad_sgd, src/metal.rs:2409 (RwkvRosaQkv1Bit::
 * backward_stop_grad, src/model.rs:1442-1490): from gy (fp32 [rows,
 * channels], gradient of out): g_e[c] = sum_r g_y[r,c] (2 idx - 1) with g_y
 * the O input gradient (never stored), g_scale, g_bias [channels]; then the
 * O BinaryConnect step (gradient x ste_scale) with the repack. The
 * reference's y / out / bias arguments are the tape here (its scale
 * gradient from outputs is sum_i sign * G, the same quantity). */
int ullis_hip_rosa_o_stop_grad_sgd(ullis_hip_ctx* ctx, const void* tape, const float* gy,
                                   uint32_t* o_bits, uint32_t* o_bits_t, const uint16_t* o_scale,
                                   uint16_t* o_latent, float* o_residual, size_t rows,
                                   size_t channels, float learning_rate, float ste_scale,
                                   float* g_e, float* g_scale, float* g_bias);

/* ---- one Heron train step on the device (UllisHeron::train_step_on,
 *      src/model.rs:2827-3025, metal branch; rosa_grad = stop_grad_bits) ---- */

/* The parameter arena follows ullis_heron_layout.h. */
size_t ullis_hip_heron_layout(const ullis_heron_dims* dims, ullis_tensor_desc* out, size_t cap,
                              uint64_t* bytes);
int ullis_hip_heron_create(ullis_hip_ctx* ctx, const ullis_heron_dims* dims, size_t batch,
                           size_t time, ullis_hip_heron** out);
void ullis_hip_heron_destroy(ullis_hip_heron* h);
/* Device pointer and byte size of the arena. */
int ullis_hip_heron_arena(ullis_hip_heron* h, void** device_ptr, uint64_t* bytes);
/* Rebuilds every derived "<prefix>.bits_t" from "<prefix>.bits" (after an upload). */
int ullis_hip_heron_refresh_derived(ullis_hip_heron* h);
/*
 * One step from the gathered embedding rows x_emb (fp32 [batch*time, d]) to
 * the embedding-row gradient g_emb (fp32, same shape); the embedding gather and
 * scatter stay with the caller, as in the reference's GPU path
 * (src/model.rs:2866-2873, 2986-2993). labels u32 [batch*time]. rosa_idx is the
 * suffix-automaton output per layer, channel-major u8 [n_layers][batch][d][time]
 * (rosa_qkv_batch_packed_channel_major, src/rosa.rs:486-513). Outputs (device):
 * row_loss fp32 [batch*time]; stats4 {mean_loss, n_valid, gscale, loss_sum};
 * qkv_bits (may be NULL) u32 [n_layers][3][ceil(batch*time*d/32)], the Q/K/V
 * sign bit-planes handed to the automaton. All pointers are device pointers.
 * invalid (may be NULL) receives the number of labels >= vocab other than
 * ignore_id. train_step_on refuses such a step before any update
 * (src/model.rs:2852-2861); labels are device data here, so the step runs,
 * but when the count is non-zero its update launches change no parameter,
 * and the loss and gradients leave those rows out.
 */
int ullis_hip_heron_step(ullis_hip_heron* h, const float* x_emb, const uint32_t* labels,
                         uint32_t ignore_id, float learning_rate, const uint8_t* rosa_idx,
                         float* g_emb, float* row_loss, float* stats4, uint32_t* qkv_bits,
                         uint32_t* invalid);
/*
 * One step from token ids (UllisHeron::train_step_on with its embedding
 * gather and scatter-SGD, src/model.rs:2866-2873, 2986-2993): gathers
 * table[tokens] (f16 [vocab, d]) into x_emb, runs ullis_hip_heron_step, and
 * applies the clipped SGD of g_emb to the table rows (table_residual: fp32
 * carry, [vocab, d]) in row order, as soon as g_emb is complete. invalid
 * (may be NULL) receives the number of token ids >= vocab plus labels >=
 * vocab other than ignore_id; when it is non-zero the step changed no
 * parameter and no table row (the reference refuses the step,
 * src/model.rs:2852-2861). Replayed from the step graph like
 * ullis_hip_heron_step when that is on.
 */
int ullis_hip_heron_step_tokens(ullis_hip_heron* h, uint16_t* table, float* table_residual,
                                size_t vocab, const uint32_t* tokens, const uint32_t* labels,
                                uint32_t ignore_id, float learning_rate, const uint8_t* rosa_idx,
                                float* x_emb, float* g_emb, float* row_loss, float* stats4,
                                uint32_t* qkv_bits, uint32_t* invalid);
/*
 * The suffix automaton driven live, layer by layer (MetalRuntime::
 * rosa_block_forward's hand-off, src/metal.rs:1411-1511; the automaton is
 * rosa_qkv_batch_packed_channel_major, src/rosa.rs:486-513, and stays with the
 * caller). ullis_hip_heron_step_sam runs the step of ullis_hip_heron_step
 * (from token ids when table is non-NULL, as ullis_hip_heron_step_tokens,
 * else from the rows in x_emb), except that no indices are given up front:
 * for each layer l it computes the Q/K/V sign bit-planes, copies them to
 * pinned host memory and calls sam(user, l, planes, idx) on the calling
 * thread. planes holds 3 x ceil(batch*time*d/32) u32 words (Q, K, V; bit
 * row*d + c = projection > 0, LSB-first); the callback writes the layer's
 * indices into idx (batch*d*time u8, channel-major [batch][d][time], pinned
 * host memory) and returns 0, or non-zero to abort the step before any
 * parameter changes. Both buffers are the library's and are reused for the
 * next layer once the callback returns. The call blocks the host on each
 * layer's planes; it never replays a step graph. Other arguments as for
 * ullis_hip_heron_step / ullis_hip_heron_step_tokens.
 */
typedef int (*ullis_hip_sam_fn)(void* user, size_t layer, const uint32_t* planes, uint8_t* idx);
int ullis_hip_heron_step_sam(ullis_hip_heron* h, uint16_t* table, float* table_residual,
                             size_t vocab, const uint32_t* tokens, float* x_emb,
                             const uint32_t* labels, uint32_t ignore_id, float learning_rate,
                             ullis_hip_sam_fn sam, void* sam_user, float* g_emb, float* row_loss,
                             float* stats4, uint32_t* qkv_bits, uint32_t* invalid);

/*
 * T = 1 greedy decode (UllisHeron::generate_step, src/model.rs:2717-2753; the
 * reference runs it on the CPU): one token for each of `batch` sequences
 * (1..8) through every block's forward_one (src/model.rs:2243-2262) on the
 * trainer's parameters. ullis_hip_heron_decode_init(h, batch) sizes the
 * decode state and starts new sequences (no previous token: the time-shift
 * mixes see -x, as time_shift_one, src/model.rs:214-228); each
 * ullis_hip_heron_decode_step then takes tokens (device u32 [batch]; an id
 * >= vocab gathers a zero row and is counted into *invalid, device u32,
 * optional), writes logits (device fp32 [batch][vocab]) and, when non-NULL,
 * next_tokens (device u32 [batch], the argmax, lowest index on ties), and keeps
 * each layer's LayerNorm outputs as the next token's previous values. The
 * suffix automaton's indices of this token come either from rosa_idx (device
 * u8 [n_layers][batch][d]) or from the callback, called per layer with the
 * Q/K/V sign bits (3 x ceil(batch*d/32) words, bit b*d + c) and writing idx
 * [batch][d] (sam / sam_user as for ullis_hip_heron_step_sam); exactly one
 * of the two. The reference's context_len limit is the caller's to keep.
 */
#define ULLIS_HIP_DECODE_EAGER 1
int ullis_hip_heron_decode_init(ullis_hip_heron* h, size_t batch, int flags);
int ullis_hip_heron_decode_step(ullis_hip_heron* h, const uint16_t* table, size_t vocab,
                                const uint32_t* tokens, const uint8_t* rosa_idx,
                                ullis_hip_sam_fn sam, void* sam_user, float* logits,
                                uint32_t* next_tokens, uint32_t* invalid);

/*
 * CausalLoss of the last step (src/model.rs:58-80, as train_step_on fills it,
 * src/model.rs:2997-3024), into *out (DEVICE memory, sizeof(ullis_hip_causal_loss)
 * bytes): loss, valid count, sign-bit flips per class (head, CMix key, ROSA
 * O) and their total, row-loss percentiles, unigram CE and unique targets,
 * and the rms / mean-abs statistics of the embedding gradient (g_emb), the
 * head scale gradient, head scale / bias / latent, the first block's CMix
 * value weight and the head's mean latent step; residual_abs_mean is the
 * mean |carry| of the embedding table when table_residual (table_elems
 * floats) is given, else 0. Call after a step and before the next one, with
 * the g_emb, labels, ignore_id and row_loss (NULL: the step wrote none) of
 * that step. Stream-ordered; statistics are fixed-order sums, so they match
 * the reference's sequential sums to rounding.
 */
typedef struct ullis_hip_causal_loss {
  float next_token;
  uint32_t next_token_count;
  uint32_t binary_flip_count;
  float loss_p10;
  float loss_p50;
  float loss_p90;
  float unigram_ce;
  uint32_t unique_targets;
  uint32_t flips_head;
  uint32_t flips_cmix;
  uint32_t flips_rosa_o;
  float embed_grad_rms;
  float head_scale_grad_rms;
  float head_scale_rms;
  float residual_abs_mean;
  float cmix_value_rms;
  float head_latent_abs_mean;
  float head_latent_step_abs;
  float head_bias_rms;
} ullis_hip_causal_loss;
int ullis_hip_heron_causal_loss(ullis_hip_heron* h, const float* g_emb, const uint32_t* labels,
                                uint32_t ignore_id, const float* row_loss,
                                const float* table_residual, size_t table_elems,
                                ullis_hip_causal_loss* out);

/*
 * Step graph (no counterpart in the reference, whose Metal backend encodes
 * command buffers per step): with enable != 0, ullis_hip_heron_step and
 * ullis_hip_heron_step_tokens capture their launches on both streams into a
 * HIP graph the first time and replay the graph while they are called with
 * the same pointers, vocab, ignore_id and learning_rate (other arguments
 * capture again). Probed steps run eagerly.
 * enable = 0 drops the graph.
 */
int ullis_hip_heron_set_graph(ullis_hip_heron* h, int enable);

/*
 * Kernel probe, the device-side counterpart of the reference's per-phase
 * TrainStepProfile (src/model.rs:101-124): while a probe id is set, every
 * launch of that class inside ullis_hip_heron_step records its execution
 * interval: a streamed-LDS GEMM launch has each workgroup write its start and
 * end on the device wall clock (earliest start to latest end; with
 * ULLIS_HIP_PROBE_EVENTS, kernel-timestamp events as below), other kernels
 * use kernel-timestamp events (hipExtLaunchKernel); HEAD_CE, which is several
 * kernels, is bracketed by event records on the step's stream. At most 512
 * launches are recorded. probe_read waits for the step and returns the summed
 * time and the number of launches, then restarts the count.
 */
#define ULLIS_HIP_PROBE_NONE 0
#define ULLIS_HIP_PROBE_KEY_FORWARD 1       /* CMix key packed GEMM + ReLU^2, per layer */
#define ULLIS_HIP_PROBE_VALUE_FORWARD 2     /* CMix value fp16 GEMM + residual add */
#define ULLIS_HIP_PROBE_HEAD_CE 3           /* whole head + streamed CE (several kernels) */
#define ULLIS_HIP_PROBE_VALUE_BACKWARD 4    /* value dX (+ ReLU^2 bwd) and dW in one launch */
#define ULLIS_HIP_PROBE_KEY_BACKWARD 5      /* key dX (packed) and dW in one launch */
#define ULLIS_HIP_PROBE_O_BACKWARD 6        /* ROSA O dX (packed) and dW in one launch */
#define ULLIS_HIP_PROBE_LN_FORWARD 7        /* ln2 forward fused with the CMix time-shift mix */
#define ULLIS_HIP_PROBE_LN_BACKWARD 8       /* CMix mix backward fused with the ln2 backward */
#define ULLIS_HIP_PROBE_COUNT 9
/* OR-ed into probe_id: time the GEMM launches of the class by kernel-timestamp
 * events as well (the start / end of the dispatch that rocprofv3's kernel
 * trace reports) instead of workgroup wall-clock stamps. */
#define ULLIS_HIP_PROBE_EVENTS 0x100
int ullis_hip_heron_probe(ullis_hip_heron* h, int probe_id);
int ullis_hip_heron_probe_read(ullis_hip_heron* h, float* total_ms, int* launches);

/*
 * Step phases: the reference's TrainStepProfile (src/model.rs:101-124,
 * 2864-2994) names its wall-clock phases embed, fwd_ln, fwd_rosa, fwd_cmix,
 * head, bwd_ln, bwd_cmix, bwd_rosa, embed_sgd (ULLIS_HIP_PHASE_* order below).
 * ullis_hip_heron_phases(h, 1) times the steps that follow (run eagerly, not
 * from a graph) with events on the main stream at those phase boundaries;
 * ullis_hip_heron_phases_read waits for the device and writes, per phase, the
 * milliseconds of the main stream's segments summed over those steps (*steps
 * = their number). The main stream carries the step's dependent chain; work
 * the second stream runs beside it (the Q/K/V branch, the O products and
 * backward, the deferred updates) is inside those segments, and the wait for
 * its tail at the step's end counts as bwd_rosa. At most about 2000 phase
 * boundaries (about 25 config-4 steps) between enabling and reading.
 */
#define ULLIS_HIP_PHASE_EMBED 0
#define ULLIS_HIP_PHASE_FWD_LN 1
#define ULLIS_HIP_PHASE_FWD_ROSA 2
#define ULLIS_HIP_PHASE_FWD_CMIX 3
#define ULLIS_HIP_PHASE_HEAD 4
#define ULLIS_HIP_PHASE_BWD_LN 5
#define ULLIS_HIP_PHASE_BWD_CMIX 6
#define ULLIS_HIP_PHASE_BWD_ROSA 7
#define ULLIS_HIP_PHASE_EMBED_SGD 8
#define ULLIS_HIP_PHASE_COUNT 9
int ullis_hip_heron_phases(ullis_hip_heron* h, int enable);
int ullis_hip_heron_phases_read(ullis_hip_heron* h, float* ms, int* steps);

#ifdef __cplusplus
}
#endif

#endif /* ULLIS_HIP_H */
