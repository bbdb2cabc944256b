// One Heron train step on the device: UllisHeron::train_step_on
// (src/model.rs:2827-3025) with rosa_grad = stop_grad_bits, from the gathered
// embedding rows to the embedding-row gradient, as a single stream of kernel
// launches with no host synchronisation.
//
// Order of operations (and which weights each GEMM sees) follows the
// reference: per block forward LN0 (block 0) -> LN3 -> time-shift mix3 ->
// Q/K/V (sign bit-planes for the automaton) -> y = (2 idx - 1) e -> O (+x)
// -> LN2 -> mix -> key (ReLU^2) -> value (+x); LN_out; head + CE with the head
// update; LN_out backward; per block in reverse: CMix backward (value input
// gradient with the pre-update value weights, value step, key input gradient
// with the pre-update bits, key latent / scale steps, x_k step), LN2
// backward (+= into g_x), ROSA O stop-grad backward (e step from g_y, O
// latent / scale / bias steps), LN0 backward at block 0.
// Tapes stay resident in HBM between the forward and the backward.
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/ullis_hip.h"
#include "common.hpp"
#include "context.hpp"
#include "ops.hpp"

using namespace ullis;

namespace {

struct Ln {
  uint16_t *w = nullptr, *b = nullptr;
  float *w_res = nullptr, *b_res = nullptr;
};

struct Packed {
  long out = 0, in = 0;
  uint32_t *bits = nullptr, *bits_t = nullptr;
  uint16_t *scale = nullptr, *bias = nullptr, *latent = nullptr;
  float *scale_res = nullptr, *bias_res = nullptr, *latent_res = nullptr;
};

struct Block {
  bool has_ln0 = false;
  Ln ln0, ln2, ln3;
  uint16_t *x_q = nullptr, *x_k = nullptr, *x_v = nullptr, *e = nullptr;
  float* e_res = nullptr;
  Packed q, k, v, o, key;
  uint16_t* cx_k = nullptr;
  float* cx_k_res = nullptr;
  uint16_t* value = nullptr;
  float* value_res = nullptr;
};

}  // namespace

struct ullis_hip_heron {
  ullis_hip_ctx* ctx = nullptr;
  ullis_heron_dims dims{};
  long batch = 0, time = 0, rows = 0, D = 0, F = 0, V = 0, L = 0;
  std::vector<ullis_tensor_desc> descs;
  uint8_t* arena = nullptr;
  uint64_t arena_bytes = 0;
  Ln ln_out;
  Packed head;
  std::vector<Block> blocks;
  void* act = nullptr;  // one allocation for activations, tapes and scratch
  // activations / tapes
  float *resid = nullptr, *after_rosa = nullptr;
  uint16_t *ln16 = nullptr, *q16 = nullptr, *k16 = nullptr, *v16 = nullptr;
  uint16_t *y16 = nullptr, *ln2_16 = nullptr, *shifted16 = nullptr;
  uint8_t* idx_rm = nullptr;
  uint16_t *key16 = nullptr, *relu2_16 = nullptr, *gk16 = nullptr, *gx16 = nullptr;
  float *g_x = nullptr, *g_a = nullptr, *g_b = nullptr;
  float *gpart = nullptr, *part = nullptr, *vec = nullptr, *slots = nullptr, *stats = nullptr;
  float* row_loss = nullptr;
  uint32_t* qkv = nullptr;
  void* head_ws = nullptr;
  int splits_o = 1, splits_key = 1, splits_value = 1;
  // kernel probe: events around every launch of one launch class
  int probe = 0;
  int probe_used = 0;
  std::vector<hipEvent_t> probe_events;

  template <class T>
  T* tensor(const std::string& name) {
    const uint64_t off = ullis_heron_offset(descs.data(), descs.size(), name.c_str());
    if (off == UINT64_MAX) return nullptr;
    return reinterpret_cast<T*>(arena + off);
  }
};

namespace {

bool bind_ln(ullis_hip_heron* h, const std::string& p, Ln& l) {
  l.w = h->tensor<uint16_t>(p + ".weight");
  l.b = h->tensor<uint16_t>(p + ".bias");
  l.w_res = h->tensor<float>(p + ".weight.residual");
  l.b_res = h->tensor<float>(p + ".bias.residual");
  return l.w && l.b && l.w_res && l.b_res;
}

bool bind_packed(ullis_hip_heron* h, const std::string& p, long out, long in, bool bias,
                 bool transpose, Packed& k) {
  k.out = out;
  k.in = in;
  k.bits = h->tensor<uint32_t>(p + ".bits");
  k.bits_t = transpose ? h->tensor<uint32_t>(p + ".bits_t") : nullptr;
  k.scale = h->tensor<uint16_t>(p + ".scale");
  k.scale_res = h->tensor<float>(p + ".scale.residual");
  k.latent = h->tensor<uint16_t>(p + ".latent");
  k.latent_res = h->tensor<float>(p + ".latent.residual");
  if (bias) {
    k.bias = h->tensor<uint16_t>(p + ".bias");
    k.bias_res = h->tensor<float>(p + ".bias.residual");
  }
  return k.bits && (!transpose || k.bits_t) && k.scale && k.scale_res && k.latent &&
         k.latent_res && (!bias || (k.bias && k.bias_res));
}

#define STEP(expr, what)                              \
  do {                                                \
    if (int rc_ = c->hip((expr), (what))) return rc_; \
  } while (0)

constexpr int kProbeMax = 512;

// When `id` is the probed launch class, the kernel that `expr` launches
// records its own start and end timestamps into the next event pair
// (LaunchProbe). `expr` must launch exactly one kernel.
#define PROBED(id, expr, what)                                                     \
  do {                                                                             \
    const bool on_ = h->probe == (id) && h->probe_used < kProbeMax;                \
    LaunchProbe lp_;                                                               \
    if (on_) {                                                                     \
      lp_.start = h->probe_events[2 * h->probe_used];                              \
      lp_.stop = h->probe_events[2 * h->probe_used + 1];                           \
      t_launch_probe = &lp_;                                                       \
    }                                                                              \
    const int rc_ = c->hip((expr), (what));                                        \
    const bool consumed_ = t_launch_probe == nullptr;                              \
    t_launch_probe = nullptr;                                                      \
    if (rc_) return rc_;                                                           \
    if (on_) {                                                                     \
      if (!consumed_) return c->fail(ULLIS_HIP_ERR_RUNTIME, "probe: no kernel launched"); \
      ++h->probe_used;                                                             \
    }                                                                              \
  } while (0)

// Brackets a multi-kernel operation with events when `id` is the probed class.
#define PROBED_SPAN(id, expr, what)                                                \
  do {                                                                             \
    const bool on_ = h->probe == (id) && h->probe_used < kProbeMax;                \
    if (on_) STEP(hipEventRecord(h->probe_events[2 * h->probe_used], s), "probe"); \
    STEP(expr, what);                                                              \
    if (on_) {                                                                     \
      STEP(hipEventRecord(h->probe_events[2 * h->probe_used + 1], s), "probe");    \
      ++h->probe_used;                                                             \
    }                                                                              \
  } while (0)

}  // namespace

extern "C" {

int ullis_hip_heron_create(ullis_hip_ctx* c, const ullis_heron_dims* dims, size_t batch,
                           size_t time, ullis_hip_heron** out) {
  if (!c || !dims || !out) return ULLIS_HIP_ERR_INVALID;
  *out = nullptr;
  if (dims->d_model == 0 || dims->n_layers == 0 || dims->dim_ffn == 0 || dims->vocab == 0 ||
      batch == 0 || time < 2)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron dims must be non-zero and time >= 2");
  if (dims->d_model % 32 != 0)
    return c->fail(ULLIS_HIP_ERR_INVALID, "d_model must be a multiple of 32 (sign bit-planes)");
  if ((double)batch * time * dims->dim_ffn > (double)INT32_MAX ||
      (double)dims->vocab * dims->d_model > (double)INT32_MAX)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron shape exceeds int32 extents");
  auto* h = new ullis_hip_heron();
  h->ctx = c;
  h->dims = *dims;
  h->batch = (long)batch;
  h->time = (long)time;
  h->rows = (long)(batch * time);
  h->D = dims->d_model;
  h->F = dims->dim_ffn;
  h->V = dims->vocab;
  h->L = dims->n_layers;
  const size_t n = ullis_heron_layout(dims, nullptr, 0, &h->arena_bytes);
  h->descs.resize(n);
  ullis_heron_layout(dims, h->descs.data(), n, &h->arena_bytes);
  if (hipMalloc(&h->arena, h->arena_bytes) != hipSuccess) {
    delete h;
    return c->fail(ULLIS_HIP_ERR_NOMEM, "heron arena allocation failed");
  }
  (void)hipMemsetAsync(h->arena, 0, h->arena_bytes, c->stream);

  bool ok = bind_ln(h, "ln_out", h->ln_out) && bind_packed(h, "head", h->V, h->D, true, true, h->head);
  h->blocks.resize(h->L);
  for (long l = 0; l < h->L && ok; ++l) {
    Block& b = h->blocks[l];
    const std::string p = "blocks." + std::to_string(l);
    b.has_ln0 = l == 0;
    if (b.has_ln0) ok = ok && bind_ln(h, p + ".ln0", b.ln0);
    ok = ok && bind_ln(h, p + ".ln2", b.ln2) && bind_ln(h, p + ".ln3", b.ln3);
    b.x_q = h->tensor<uint16_t>(p + ".rosa.x_q");
    b.x_k = h->tensor<uint16_t>(p + ".rosa.x_k");
    b.x_v = h->tensor<uint16_t>(p + ".rosa.x_v");
    b.e = h->tensor<uint16_t>(p + ".rosa.e");
    b.e_res = h->tensor<float>(p + ".rosa.e.residual");
    b.cx_k = h->tensor<uint16_t>(p + ".ffn.x_k");
    b.cx_k_res = h->tensor<float>(p + ".ffn.x_k.residual");
    b.value = h->tensor<uint16_t>(p + ".ffn.value");
    b.value_res = h->tensor<float>(p + ".ffn.value.residual");
    ok = ok && b.x_q && b.x_k && b.x_v && b.e && b.e_res && b.cx_k && b.cx_k_res && b.value &&
         b.value_res;
    ok = ok && bind_packed(h, p + ".rosa.q", h->D, h->D, true, false, b.q) &&
         bind_packed(h, p + ".rosa.k", h->D, h->D, true, false, b.k) &&
         bind_packed(h, p + ".rosa.v", h->D, h->D, true, false, b.v) &&
         bind_packed(h, p + ".rosa.o", h->D, h->D, true, true, b.o) &&
         bind_packed(h, p + ".ffn.key", h->F, h->D, false, true, b.key);
  }
  if (!ok) {
    (void)hipFree(h->arena);
    delete h;
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron arena layout is missing a tensor");
  }

  const long R = h->rows, D = h->D, F = h->F, L = h->L, V = h->V;
  const long nd = R * D, nf = R * F;
  const long words = cdiv(nd, 32);
  h->splits_o = dw_splits(D, D, R);
  h->splits_key = dw_splits(F, D, R);
  h->splits_value = dw_splits(D, F, R);
  long gpart = (long)h->splits_o * D * D;
  if ((long)h->splits_key * F * D > gpart) gpart = (long)h->splits_key * F * D;
  if ((long)h->splits_value * D * F > gpart) gpart = (long)h->splits_value * D * F;
  long part = 2L * layer_norm_backward_blocks(R) * D;
  if (column_partial_blocks(R) * D > part) part = column_partial_blocks(R) * D;
  const long vec = F > V ? F : (V > D ? V : D);
  const size_t head_ws = head_ce_workspace_bytes(R, D, V);

  size_t bytes = 0;
  auto add = [&](size_t b) { bytes += Carver::bytes_for(b); };
  add(4ul * nd * (L + 1));   // resid
  add(4ul * nd * L);         // after_rosa
  for (int i = 0; i < 4; ++i) add(2ul * nd);  // ln16 q16 k16 v16
  add(2ul * nd * L);         // y16
  add(2ul * nd * L);         // ln2_16
  add(2ul * nd * L);         // shifted16
  add(1ul * nd * L);         // idx_rm
  add(2ul * nf * L);         // key16
  add(2ul * nf * L);         // relu2_16
  add(2ul * nf);             // gk16
  add(2ul * nd);             // gx16
  add(4ul * nd * 3);         // g_x g_a g_b
  add(4ul * gpart);
  add(4ul * part);
  add(4ul * vec);
  add(4ul * (L + 2));        // slots
  add(4ul * 4);              // stats
  add(4ul * R);              // row_loss
  add(4ul * words * 3 * L);  // qkv bit-planes
  add(head_ws);
  if (hipMalloc(&h->act, bytes) != hipSuccess) {
    (void)hipFree(h->arena);
    delete h;
    return c->fail(ULLIS_HIP_ERR_NOMEM, "heron activation allocation of " +
                                            std::to_string(bytes) + " bytes failed");
  }
  Carver cv(h->act);
  h->resid = cv.take<float>(nd * (L + 1));
  h->after_rosa = cv.take<float>(nd * L);
  h->ln16 = cv.take<uint16_t>(nd);
  h->q16 = cv.take<uint16_t>(nd);
  h->k16 = cv.take<uint16_t>(nd);
  h->v16 = cv.take<uint16_t>(nd);
  h->y16 = cv.take<uint16_t>(nd * L);
  h->ln2_16 = cv.take<uint16_t>(nd * L);
  h->shifted16 = cv.take<uint16_t>(nd * L);
  h->idx_rm = cv.take<uint8_t>(nd * L);
  h->key16 = cv.take<uint16_t>(nf * L);
  h->relu2_16 = cv.take<uint16_t>(nf * L);
  h->gk16 = cv.take<uint16_t>(nf);
  h->gx16 = cv.take<uint16_t>(nd);
  h->g_x = cv.take<float>(nd);
  h->g_a = cv.take<float>(nd);
  h->g_b = cv.take<float>(nd);
  h->gpart = cv.take<float>(gpart);
  h->part = cv.take<float>(part);
  h->vec = cv.take<float>(vec);
  h->slots = cv.take<float>(L + 2);
  h->stats = cv.take<float>(4);
  h->row_loss = cv.take<float>(R);
  h->qkv = cv.take<uint32_t>(words * 3 * L);
  h->head_ws = cv.take<char>(head_ws);
  h->probe_events.resize(2 * kProbeMax);
  for (auto& e : h->probe_events) {
    if (hipEventCreate(&e) != hipSuccess) {
      e = nullptr;
      ullis_hip_heron_destroy(h);
      return c->fail(ULLIS_HIP_ERR_RUNTIME, "probe event creation failed");
    }
  }
  if (int rc = c->hip(hipStreamSynchronize(c->stream), "heron create")) {
    ullis_hip_heron_destroy(h);
    return rc;
  }
  *out = h;
  return 0;
}

void ullis_hip_heron_destroy(ullis_hip_heron* h) {
  if (!h) return;
  if (h->ctx) (void)hipStreamSynchronize(h->ctx->stream);
  for (auto& e : h->probe_events) (void)hipEventDestroy(e);
  if (h->arena) (void)hipFree(h->arena);
  if (h->act) (void)hipFree(h->act);
  delete h;
}

int ullis_hip_heron_arena(ullis_hip_heron* h, void** device_ptr, uint64_t* bytes) {
  if (!h || !device_ptr || !bytes) return ULLIS_HIP_ERR_INVALID;
  *device_ptr = h->arena;
  *bytes = h->arena_bytes;
  return 0;
}

int ullis_hip_heron_probe(ullis_hip_heron* h, int probe_id) {
  if (!h || probe_id < 0 || probe_id >= ULLIS_HIP_PROBE_COUNT) return ULLIS_HIP_ERR_INVALID;
  h->probe = probe_id;
  h->probe_used = 0;
  return 0;
}

int ullis_hip_heron_probe_read(ullis_hip_heron* h, float* total_ms, int* launches) {
  if (!h || !total_ms || !launches) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  double sum = 0.0;
  for (int i = 0; i < h->probe_used; ++i) {
    float ms = 0.0f;
    STEP(hipEventSynchronize(h->probe_events[2 * i + 1]), "probe sync");
    STEP(hipEventElapsedTime(&ms, h->probe_events[2 * i], h->probe_events[2 * i + 1]),
         "probe elapsed");
    sum += ms;
  }
  *total_ms = (float)sum;
  *launches = h->probe_used;
  h->probe_used = 0;
  return 0;
}

int ullis_hip_heron_refresh_derived(ullis_hip_heron* h) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  hipStream_t s = c->stream;
  STEP(transpose_bits(s, h->head.bits, h->head.out, h->head.in, h->head.bits_t), "head bits_t");
  for (auto& b : h->blocks) {
    STEP(transpose_bits(s, b.o.bits, b.o.out, b.o.in, b.o.bits_t), "o bits_t");
    STEP(transpose_bits(s, b.key.bits, b.key.out, b.key.in, b.key.bits_t), "key bits_t");
  }
  return 0;
}

int ullis_hip_heron_step(ullis_hip_heron* h, const float* x_emb, const uint32_t* labels,
                         uint32_t ignore_id, float lr, const uint8_t* rosa_idx, float* g_emb,
                         float* row_loss, float* stats4, uint32_t* qkv_bits) {
  if (!h) return ULLIS_HIP_ERR_INVALID;
  ullis_hip_ctx* c = h->ctx;
  if (!x_emb || !labels || !rosa_idx || !g_emb)
    return c->fail(ULLIS_HIP_ERR_INVALID, "heron step needs x_emb, labels, rosa_idx and g_emb");
  if (!(lr > 0.0f) || !__builtin_isfinite(lr))
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "train step requires a positive learning rate and time >= 2");
  hipStream_t s = c->stream;
  const long R = h->rows, D = h->D, F = h->F, L = h->L, T = h->time, B = h->batch;
  const long nd = R * D, nf = R * F;
  const long words = cdiv(nd, 32);
  const float ste = (float)(T - 1);  // binaryconnect_ste_scale(time - 1), src/model.rs:554-556
  // latent rows of the packed weights are whole 64-weight chunks: the latent
  // step, scale step and repack run in one kernel per matrix
  const bool fuse_pack = D % 64 == 0;
  float* rl = row_loss ? row_loss : h->row_loss;
  float* st = stats4 ? stats4 : h->stats;
  uint32_t* qkv = qkv_bits ? qkv_bits : h->qkv;
  int nb = 0;

  STEP(fill_f32(s, h->slots, L + 2, 0.0f), "clear amax slots");

  // ------------------------------------------------------------- forward
  for (long l = 0; l < L; ++l) {
    Block& b = h->blocks[l];
    float* x_l = h->resid + l * nd;
    if (b.has_ln0) {
      STEP(layer_norm_forward(s, x_emb, R, D, b.ln0.w, b.ln0.b, x_l, nullptr), "ln0");
    } else if (l == 0) {
      STEP(copy_device(s, x_l, x_emb, (long)sizeof(float) * nd), "copy x");
    }
    // ROSA block (src/model.rs:1354-1440)
    STEP(layer_norm_forward(s, x_l, R, D, b.ln3.w, b.ln3.b, nullptr, h->ln16), "ln3");
    STEP(time_shift_mix(s, h->ln16, R, T, D, b.x_q, h->q16, b.x_k, h->k16, b.x_v, h->v16), "mix3");
    const Packed* qkvp[3] = {&b.q, &b.k, &b.v};
    const uint16_t* qkv_in[3] = {h->q16, h->k16, h->v16};
    for (int j = 0; j < 3; ++j) {
      PackedFwdOut o;
      o.sign_bits = qkv + (l * 3 + j) * words;
      STEP(packed_forward(s, qkv_in[j], kF16, R, D, D, qkvp[j]->bits, qkvp[j]->scale,
                          qkvp[j]->bias, o),
           "qkv");
    }
    uint16_t* y16 = h->y16 + l * nd;
    STEP(rosa_expand(s, rosa_idx + l * nd, b.e, B, T, D, y16, h->idx_rm + l * nd), "rosa y");
    float* ar = h->after_rosa + l * nd;
    {
      PackedFwdOut o;
      o.y32 = ar;
      o.resid = x_l;
      STEP(packed_forward(s, y16, kF16, R, D, D, b.o.bits, b.o.scale, b.o.bias, o), "o");
    }
    // CMix (src/model.rs:1018-1078)
    uint16_t* ln2 = h->ln2_16 + l * nd;
    uint16_t* sh = h->shifted16 + l * nd;
    uint16_t* key = h->key16 + l * nf;
    uint16_t* r2 = h->relu2_16 + l * nf;
    PROBED(ULLIS_HIP_PROBE_LN_FORWARD,
           layer_norm_forward(s, ar, R, D, b.ln2.w, b.ln2.b, nullptr, ln2), "ln2");
    STEP(time_shift_mix(s, ln2, R, T, D, b.cx_k, sh, nullptr, nullptr, nullptr, nullptr), "mix");
    {
      PackedFwdOut o;
      o.y16 = key;
      o.relu2_16 = r2;
      PROBED(ULLIS_HIP_PROBE_KEY_FORWARD,
             packed_forward(s, sh, kF16, R, D, F, b.key.bits, b.key.scale, nullptr, o), "key");
    }
    PROBED(ULLIS_HIP_PROBE_VALUE_FORWARD,
           fp16_forward(s, r2, kF16, R, F, D, b.value, h->resid + (l + 1) * nd, ar, nullptr),
           "value");
  }
  float* x_last = h->resid + L * nd;
  STEP(layer_norm_forward(s, x_last, R, D, h->ln_out.w, h->ln_out.b, nullptr, h->ln16), "ln_out");

  // ------------------------------------------------- head + CE with update
  {
    HeadCe hc{};
    hc.rows = R;
    hc.time = T;
    hc.d = D;
    hc.vocab = h->V;
    hc.hidden16 = h->ln16;
    hc.bits = h->head.bits;
    hc.bits_t = h->head.bits_t;
    hc.scale = h->head.scale;
    hc.bias = h->head.bias;
    hc.targets = labels;
    hc.ignore_id = ignore_id;
    hc.row_loss = rl;
    hc.stats = st;
    hc.g_hidden = h->g_a;
    hc.g_scale = h->vec;
    hc.lr = lr;
    hc.ste = ste;
    hc.latent = h->head.latent;
    hc.latent_res = h->head.latent_res;
    hc.scale_upd = h->head.scale;
    hc.scale_res = h->head.scale_res;
    hc.bias_upd = h->head.bias;
    hc.bias_res = h->head.bias_res;
    hc.bits_new = h->head.bits;
    hc.bits_t_new = h->head.bits_t;
    PROBED_SPAN(ULLIS_HIP_PROBE_HEAD_CE, head_ce(s, hc, h->head_ws), "head ce");
  }
  // LN_out backward + step (src/model.rs:2932-2937)
  STEP(layer_norm_backward_rows(s, x_last, h->g_a, R, D, h->ln_out.w, h->g_x, 0, h->slots + L,
                                h->part, &nb),
       "ln_out bwd");
  STEP(layer_norm_param_finish(s, h->part, nb, D, nullptr, nullptr, lr, h->ln_out.w,
                               h->ln_out.w_res, h->ln_out.b, h->ln_out.b_res),
       "ln_out step");
  STEP(scale_to_f16(s, h->g_x, nd, h->slots + L, h->gx16), "g_x fp16");

  // ------------------------------------------------------------ backward
  for (long l = L - 1; l >= 0; --l) {
    Block& b = h->blocks[l];
    const float* slot_in = h->slots + l + 1;
    float* slot_mid = h->slots + l;
    const uint16_t* ln2 = h->ln2_16 + l * nd;
    const uint16_t* sh = h->shifted16 + l * nd;
    const uint16_t* key = h->key16 + l * nf;
    const uint16_t* r2 = h->relu2_16 + l * nf;
    const float* ar = h->after_rosa + l * nd;

    // CMix backward_update (src/model.rs:1145-1177)
    PROBED(ULLIS_HIP_PROBE_VALUE_INPUT_GRAD,
           fp16_backward_input(s, GradIn{h->g_x, slot_in, h->gx16}, R, F, D, b.value, nullptr, key,
                               h->gk16),
           "value input grad + relu2 bwd");
    STEP(fp16_weight_grad_partials(s, GradIn{h->g_x, slot_in, h->gx16}, r2, R, F, D,
                                   h->splits_value,
                                   h->gpart),
         "value weight grad");
    STEP(fp16_weight_finish(s, h->gpart, h->splits_value, D, F, slot_in, lr, b.value, b.value_res,
                            nullptr),
         "value step");
    PROBED(ULLIS_HIP_PROBE_KEY_INPUT_GRAD,
           packed_backward_input(s, GradIn{nullptr, slot_in}, h->gk16, R, D, F, b.key.bits_t,
                                 b.key.scale, h->g_a, nullptr, 0),
           "key input grad");
    PROBED(ULLIS_HIP_PROBE_KEY_WEIGHT_GRAD,
           packed_weight_grad_partials(s, GradIn{nullptr, slot_in}, h->gk16, sh, R, D, F,
                                       h->splits_key, h->gpart),
           "key weight grad");
    {
      PackedFinish f;
      f.part = h->gpart;
      f.splits = h->splits_key;
      f.out = F;
      f.in = D;
      f.scale = b.key.scale;
      f.bits_old = b.key.bits;
      f.amax = slot_in;
      f.extra_mul = nullptr;
      f.ste = ste;
      f.lr = lr;
      f.latent = b.key.latent;
      f.latent_res = b.key.latent_res;
      f.g_scale = h->vec;
      f.g_w = nullptr;
      if (fuse_pack) {
        f.scale_upd = b.key.scale;
        f.scale_res = b.key.scale_res;
        f.bits_new = b.key.bits;
      }
      STEP(packed_weight_finish(s, f), "key latent step");
    }
    if (fuse_pack) {
      STEP(transpose_bits(s, b.key.bits, F, D, b.key.bits_t), "key bits_t");
    } else {
      STEP(clipped_sgd(s, b.key.scale, b.key.scale_res, h->vec, F, lr), "key scale step");
      STEP(pack_latent_bits(s, b.key.latent, F, D, b.key.bits, b.key.bits_t), "key repack");
    }
    STEP(time_shift_mix_backward(s, h->g_a, ln2, b.cx_k, R, T, D, h->g_b, h->part, &nb),
         "mix bwd");
    STEP(vector_finish(s, h->part, nb, D, nullptr, lr, b.cx_k, b.cx_k_res), "x_k step");

    // LN2 backward, += into g_x (src/model.rs:2958-2963)
    PROBED(ULLIS_HIP_PROBE_LN_BACKWARD,
           layer_norm_backward_rows(s, ar, h->g_b, R, D, b.ln2.w, h->g_x, 1, slot_mid, h->part,
                                    &nb),
           "ln2 bwd");
    STEP(layer_norm_param_finish(s, h->part, nb, D, nullptr, nullptr, lr, b.ln2.w, b.ln2.w_res,
                                 b.ln2.b, b.ln2.b_res),
         "ln2 step");
    // O bias gradient (column sums of g_x) and the fp16 copy of g_x for the
    // O GEMMs here and the CMix GEMMs of the block below.
    STEP(column_sum_partials(s, h->g_x, nullptr, R, D, h->part, &nb, h->gx16, slot_mid),
         "o g_bias + g_x fp16");
    STEP(vector_finish(s, h->part, nb, D, nullptr, lr, b.o.bias, b.o.bias_res), "o bias step");

    // ROSA O stop-grad backward (src/model.rs:1491-1522)
    STEP(packed_backward_input(s, GradIn{h->g_x, slot_mid, h->gx16}, nullptr, R, D, D, b.o.bits_t,
                               b.o.scale, h->g_a, nullptr, 0),
         "o input grad");
    STEP(column_sum_partials(s, h->g_a, h->idx_rm + l * nd, R, D, h->part, &nb), "g_e");
    STEP(vector_finish(s, h->part, nb, D, nullptr, lr, b.e, b.e_res), "e step");
    STEP(packed_weight_grad_partials(s, GradIn{h->g_x, slot_mid, h->gx16}, nullptr, h->y16 + l * nd, R, D,
                                     D, h->splits_o, h->gpart),
         "o weight grad");
    {
      PackedFinish f;
      f.part = h->gpart;
      f.splits = h->splits_o;
      f.out = D;
      f.in = D;
      f.scale = b.o.scale;
      f.bits_old = b.o.bits;
      f.amax = slot_mid;
      f.extra_mul = nullptr;
      f.ste = ste;
      f.lr = lr;
      f.latent = b.o.latent;
      f.latent_res = b.o.latent_res;
      f.g_scale = h->vec;
      f.g_w = nullptr;
      if (fuse_pack) {
        f.scale_upd = b.o.scale;
        f.scale_res = b.o.scale_res;
        f.bits_new = b.o.bits;
      }
      STEP(packed_weight_finish(s, f), "o latent step");
    }
    if (fuse_pack) {
      STEP(transpose_bits(s, b.o.bits, D, D, b.o.bits_t), "o bits_t");
    } else {
      STEP(clipped_sgd(s, b.o.scale, b.o.scale_res, h->vec, D, lr), "o scale step");
      STEP(pack_latent_bits(s, b.o.latent, D, D, b.o.bits, b.o.bits_t), "o repack");
    }

    if (b.has_ln0) {  // (src/model.rs:2978-2982)
      STEP(layer_norm_backward_rows(s, x_emb, h->g_x, R, D, b.ln0.w, g_emb, 0, nullptr, h->part,
                                    &nb),
           "ln0 bwd");
      STEP(layer_norm_param_finish(s, h->part, nb, D, nullptr, nullptr, lr, b.ln0.w, b.ln0.w_res,
                                   b.ln0.b, b.ln0.b_res),
           "ln0 step");
    } else if (l == 0) {
      STEP(copy_device(s, g_emb, h->g_x, (long)sizeof(float) * nd), "copy g_emb");
    }
  }
  (void)F;
  return 0;
}

}  // extern "C"
