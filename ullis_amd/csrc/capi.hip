// C ABI: context, memory and the unit operations of include/ullis_hip.h.
// Every entry point validates shapes on the host (LinearDispatchShape rules,
// src/metal.rs:62-87) before anything is launched.
#include <hip/hip_runtime.h>

#include <climits>
#include <string>

#include "../../include/ullis_hip.h"
#include "context.hpp"
#include "ops.hpp"

using namespace ullis;

namespace {
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

namespace {

constexpr int kVersion = 1;

bool dim_ok(size_t v) { return v > 0 && v <= (size_t)INT32_MAX; }

bool prod_ok(size_t a, size_t b) {
  return a > 0 && b > 0 && a <= (size_t)LONG_MAX / b;
}

int check_linear(ullis_hip_ctx* c, size_t rows, size_t in, size_t out) {
  if (!dim_ok(rows) || !dim_ok(in) || !dim_ok(out) || !prod_ok(rows, in) || !prod_ok(rows, out) ||
      !prod_ok(in, out))
    return c->fail(ULLIS_HIP_ERR_INVALID, "linear dimensions must be non-zero and fit in int32");
  return 0;
}

#define NEED(ptr, name)                                                         \
  do {                                                                          \
    if (!(ptr)) return c->fail(ULLIS_HIP_ERR_INVALID, std::string(name) + " is NULL"); \
  } while (0)

#define HIPCALL(expr, what)                     \
  do {                                          \
    if (int rc_ = c->hip((expr), (what))) return rc_; \
  } while (0)

}  // namespace

extern "C" {

int ullis_hip_version(void) { return kVersion; }

int ullis_hip_device_count(int* count) {
  if (!count) return ULLIS_HIP_ERR_INVALID;
  *count = 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return ULLIS_HIP_ERR_RUNTIME;
  *count = n;
  return 0;
}

int ullis_hip_create(int device, ullis_hip_ctx** out) {
  if (!out) return ULLIS_HIP_ERR_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return ULLIS_HIP_ERR_RUNTIME;
  if (hipSetDevice(device) != hipSuccess) return ULLIS_HIP_ERR_RUNTIME;
  ullis_hip_ctx* c = new ullis_hip_ctx();
  c->device = device;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return ULLIS_HIP_ERR_RUNTIME;
  }
  for (auto& e : c->events) {
    if (hipEventCreate(&e) != hipSuccess) {
      ullis_hip_destroy(c);
      return ULLIS_HIP_ERR_RUNTIME;
    }
  }
  // the no-allocation entry points' scratch: its address on this device
  const hipError_t se = static_scratch_address(device, &c->static_scratch);
  if (se != hipSuccess) {
    c->static_scratch = nullptr;
    c->static_scratch_err = hipGetErrorString(se);
  }
  *out = c;
  return 0;
}

void ullis_hip_destroy(ullis_hip_ctx* c) {
  if (!c) return;
  if (t_launch_probe == &c->next_launch) t_launch_probe = nullptr;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (auto& e : c->events)
    if (e) (void)hipEventDestroy(e);
  if (c->scratch) (void)hipFree(c->scratch);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* ullis_hip_last_error(const ullis_hip_ctx* c) { return c ? c->err.c_str() : "null context"; }

int ullis_hip_sync(ullis_hip_ctx* c) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  HIPCALL(hipStreamSynchronize(c->stream), "stream synchronize");
  HIPCALL(hipGetLastError(), "pending kernel error");
  return 0;
}

int ullis_hip_malloc(ullis_hip_ctx* c, size_t bytes, void** ptr) {
  if (!c || !ptr) return ULLIS_HIP_ERR_INVALID;
  *ptr = nullptr;
  if (bytes == 0) return c->fail(ULLIS_HIP_ERR_INVALID, "zero-byte allocation");
  if (hipMalloc(ptr, bytes) != hipSuccess) {
    *ptr = nullptr;
    return c->fail(ULLIS_HIP_ERR_NOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  return 0;
}

int ullis_hip_free(ullis_hip_ctx* c, void* ptr) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (!ptr) return 0;
  HIPCALL(hipStreamSynchronize(c->stream), "sync before free");
  HIPCALL(hipFree(ptr), "hipFree");
  return 0;
}

int ullis_hip_upload(ullis_hip_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (bytes == 0) return 0;
  NEED(dst, "dst");
  NEED(src, "src");
  HIPCALL(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "upload");
  HIPCALL(hipStreamSynchronize(c->stream), "upload sync");
  return 0;
}

int ullis_hip_download(ullis_hip_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (bytes == 0) return 0;
  NEED(dst, "dst");
  NEED(src, "src");
  HIPCALL(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "download");
  HIPCALL(hipStreamSynchronize(c->stream), "download sync");
  return 0;
}

int ullis_hip_copy(ullis_hip_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (bytes == 0) return 0;
  NEED(dst, "dst");
  NEED(src, "src");
  if (bytes > (size_t)INT64_MAX) return c->fail(ULLIS_HIP_ERR_INVALID, "copy size too large");
  HIPCALL(copy_device(c->stream, dst, src, (long)bytes), "device copy");
  return 0;
}

int ullis_hip_event_record(ullis_hip_ctx* c, int slot) {
  if (!c || slot < 0 || slot >= 16) return ULLIS_HIP_ERR_INVALID;
  HIPCALL(hipEventRecord(c->events[slot], c->stream), "event record");
  return 0;
}

int ullis_hip_time_next_launch(ullis_hip_ctx* c, int start_slot, int end_slot) {
  if (!c || start_slot < 0 || start_slot >= 16 || end_slot < 0 || end_slot >= 16 ||
      start_slot == end_slot)
    return ULLIS_HIP_ERR_INVALID;
  c->next_launch = LaunchProbe{};
  c->next_launch.start = c->events[start_slot];
  c->next_launch.stop = c->events[end_slot];
  t_launch_probe = &c->next_launch;
  return 0;
}

int ullis_hip_event_elapsed_ms(ullis_hip_ctx* c, int a, int b, float* ms) {
  if (!c || !ms || a < 0 || a >= 16 || b < 0 || b >= 16) return ULLIS_HIP_ERR_INVALID;
  HIPCALL(hipEventSynchronize(c->events[b]), "event sync");
  HIPCALL(hipEventElapsedTime(ms, c->events[a], c->events[b]), "event elapsed");
  return 0;
}

// ------------------------------------------------------------------ unit ops

int ullis_hip_layer_norm(ullis_hip_ctx* c, const float* x, const uint16_t* weight,
                         const uint16_t* bias, size_t rows, size_t channels, float* y32,
                         uint16_t* y16) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (!dim_ok(rows) || !dim_ok(channels) || !prod_ok(rows, channels))
    return c->fail(ULLIS_HIP_ERR_INVALID, "LayerNorm input shape mismatch");
  NEED(x, "x");
  NEED(weight, "weight");
  NEED(bias, "bias");
  if (!y32 && !y16) return c->fail(ULLIS_HIP_ERR_INVALID, "LayerNorm needs an output");
  HIPCALL(layer_norm_forward(c->stream, x, (long)rows, (long)channels, weight, bias, y32, y16),
          "layer_norm");
  return 0;
}

int ullis_hip_layer_norm_backward(ullis_hip_ctx* c, const float* x, const float* gy,
                                  const uint16_t* weight, size_t rows, size_t channels, float* gx,
                                  float* gw, float* gb) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (!dim_ok(rows) || !dim_ok(channels) || !prod_ok(rows, channels))
    return c->fail(ULLIS_HIP_ERR_INVALID, "LayerNorm backward shape mismatch");
  NEED(x, "x");
  NEED(gy, "gy");
  NEED(weight, "weight");
  NEED(gx, "gx");
  const int nblk = layer_norm_backward_blocks((long)rows);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(Carver::bytes_for(sizeof(float) * 2 * nblk * channels), &ws))
    return rc;
  int nb = 0;
  HIPCALL(layer_norm_backward_rows(c->stream, x, gy, (long)rows, (long)channels, weight, gx, 0,
                                   nullptr, static_cast<float*>(ws), &nb),
          "layer_norm_backward");
  HIPCALL(layer_norm_param_finish(c->stream, static_cast<float*>(ws), nb, (long)channels, gw, gb,
                                  0.0f, nullptr, nullptr, nullptr, nullptr),
          "layer_norm_param_finish");
  return 0;
}

int ullis_hip_binary_linear(ullis_hip_ctx* c, const void* x, int x_dtype, const uint32_t* bits,
                            const uint16_t* scale, const uint16_t* bias, size_t rows, size_t in,
                            size_t out, float* y32, uint16_t* y16) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_linear(c, rows, in, out)) return rc;
  NEED(x, "x");
  NEED(bits, "bits");
  NEED(scale, "scale");
  if (x_dtype != ULLIS_HIP_F16 && x_dtype != ULLIS_HIP_F32)
    return c->fail(ULLIS_HIP_ERR_INVALID, "x_dtype must be ULLIS_HIP_F16 or ULLIS_HIP_F32");
  if (!y32 && !y16) return c->fail(ULLIS_HIP_ERR_INVALID, "binary_linear needs an output");
  PackedFwdOut o;
  o.y32 = y32;
  o.y16 = y16;
  HIPCALL(packed_forward(c->stream, x, x_dtype, (long)rows, (long)in, (long)out, bits, scale, bias,
                         o),
          "binary_linear");
  return 0;
}

int ullis_hip_binary_linear_backward(ullis_hip_ctx* c, const uint16_t* x16, const float* gy,
                                     const uint32_t* bits, const uint16_t* scale, int has_bias,
                                     size_t rows, size_t in, size_t out, float* gx, float* gw,
                                     float* g_scale, float* g_bias) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_linear(c, rows, in, out)) return rc;
  NEED(x16, "x");
  NEED(gy, "gy");
  NEED(bits, "bits");
  NEED(scale, "scale");
  NEED(gw, "gw");
  NEED(g_scale, "g_scale");
  const long R = (long)rows, I = (long)in, O = (long)out;
  const int splits = dw_splits(O, I, R);
  const long words = cdiv(I * O, 32);
  const long nb = column_partial_blocks(R);
  const size_t need = Carver::bytes_for(4 * words) + Carver::bytes_for(4ul * splits * O * I) +
                      Carver::bytes_for(4) + Carver::bytes_for(4ul * nb * O) +
                      Carver::bytes_for(2ul * R * O);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(need, &ws)) return rc;
  Carver cv(ws);
  uint32_t* bits_t = cv.take<uint32_t>(words);
  float* part = cv.take<float>((size_t)splits * O * I);
  float* slot = cv.take<float>(1);
  float* cpart = cv.take<float>((size_t)nb * O);
  uint16_t* gy16 = cv.take<uint16_t>((size_t)R * O);
  HIPCALL(fill_f32(c->stream, slot, 1, 0.0f), "fill");
  HIPCALL(amax_f32(c->stream, gy, R * O, slot), "amax");
  // fp16 operand copy of the scaled gradient (the GEMMs use it when their
  // shapes allow the streamed-LDS kernels)
  const GradIn g{gy, slot, aligned16(gy) ? gy16 : nullptr};
  if (g.p16) HIPCALL(scale_to_f16(c->stream, gy, R * O, slot, gy16), "gy fp16");
  if (gx) {
    HIPCALL(transpose_bits(c->stream, bits, O, I, bits_t), "transpose_bits");
    HIPCALL(packed_backward_input(c->stream, g, nullptr, R, I, O, bits_t, scale, gx, nullptr, 0),
            "binary_linear input grad");
  }
  HIPCALL(packed_weight_grad_partials(c->stream, g, nullptr, x16, R, I, O, splits, part),
          "binary_linear weight grad");
  PackedFinish f;
  f.part = part;
  f.splits = splits;
  f.out = O;
  f.in = I;
  f.scale = scale;
  f.bits_old = bits;
  f.amax = slot;
  f.extra_mul = nullptr;
  f.ste = 1.0f;
  f.lr = 0.0f;
  f.latent = nullptr;
  f.latent_res = nullptr;
  f.g_scale = g_scale;
  f.g_w = gw;
  HIPCALL(packed_weight_finish(c->stream, f), "binary_linear finish");
  if (has_bias && g_bias) {
    int nblk = 0;
    HIPCALL(column_sum_partials(c->stream, gy, nullptr, R, O, cpart, &nblk), "g_bias");
    HIPCALL(vector_finish(c->stream, cpart, nblk, O, g_bias, 0.0f, nullptr, nullptr), "g_bias");
  }
  return 0;
}

int ullis_hip_apply_latent_sgd(ullis_hip_ctx* c, uint16_t* latent, float* residual,
                               const float* gradient, size_t out, size_t in, float learning_rate,
                               float ste_scale, uint32_t* bits, uint32_t* bits_t) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (!dim_ok(out) || !dim_ok(in) || !prod_ok(out, in))
    return c->fail(ULLIS_HIP_ERR_INVALID, "latent SGD length mismatch");
  NEED(latent, "latent");
  NEED(residual, "residual");
  NEED(gradient, "gradient");
  NEED(bits, "bits");
  const long n = (long)(out * in);
  HIPCALL(binaryconnect_sgd(c->stream, latent, residual, gradient, n, learning_rate, ste_scale),
          "binaryconnect_sgd");
  HIPCALL(pack_latent_bits(c->stream, latent, (long)out, (long)in, bits, bits_t), "pack bits");
  return 0;
}

int ullis_hip_fp16_linear(ullis_hip_ctx* c, const void* x, int x_dtype, const uint16_t* w,
                          size_t rows, size_t in, size_t out, float* y32, uint16_t* y16) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_linear(c, rows, in, out)) return rc;
  NEED(x, "x");
  NEED(w, "w");
  if (x_dtype != ULLIS_HIP_F16 && x_dtype != ULLIS_HIP_F32)
    return c->fail(ULLIS_HIP_ERR_INVALID, "x_dtype must be ULLIS_HIP_F16 or ULLIS_HIP_F32");
  if (!y32 && !y16) return c->fail(ULLIS_HIP_ERR_INVALID, "fp16_linear needs an output");
  HIPCALL(fp16_forward(c->stream, x, x_dtype, (long)rows, (long)in, (long)out, w, y32, nullptr, y16),
          "fp16_linear");
  return 0;
}

int ullis_hip_fp16_linear_backward(ullis_hip_ctx* c, const uint16_t* x16, const float* gy,
                                   const uint16_t* w, size_t rows, size_t in, size_t out,
                                   float* gx, float* gw) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_linear(c, rows, in, out)) return rc;
  NEED(x16, "x");
  NEED(gy, "gy");
  NEED(w, "w");
  NEED(gw, "gw");
  const long R = (long)rows, I = (long)in, O = (long)out;
  const int splits = dw_splits(O, I, R);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(Carver::bytes_for(4ul * splits * O * I) + Carver::bytes_for(4) +
                                     Carver::bytes_for(2ul * R * O),
                                 &ws))
    return rc;
  Carver cv(ws);
  float* part = cv.take<float>((size_t)splits * O * I);
  float* slot = cv.take<float>(1);
  uint16_t* gy16 = cv.take<uint16_t>((size_t)R * O);
  HIPCALL(fill_f32(c->stream, slot, 1, 0.0f), "fill");
  HIPCALL(amax_f32(c->stream, gy, R * O, slot), "amax");
  const GradIn g{gy, slot, aligned16(gy) ? gy16 : nullptr};
  if (g.p16) HIPCALL(scale_to_f16(c->stream, gy, R * O, slot, gy16), "gy fp16");
  if (gx)
    HIPCALL(fp16_backward_input(c->stream, g, R, I, O, w, gx, nullptr, nullptr),
            "fp16_linear input grad");
  HIPCALL(fp16_weight_grad_partials(c->stream, g, x16, R, I, O, splits, part),
          "fp16_linear weight grad");
  HIPCALL(fp16_weight_finish(c->stream, part, splits, O, I, slot, 0.0f, nullptr, nullptr, gw),
          "fp16_linear finish");
  return 0;
}

int ullis_hip_clipped_sgd_fp16(ullis_hip_ctx* c, uint16_t* params, float* residual,
                               const float* gradient, size_t n, float learning_rate) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (n == 0) return 0;
  NEED(params, "params");
  NEED(residual, "residual");
  NEED(gradient, "gradient");
  HIPCALL(clipped_sgd(c->stream, params, residual, gradient, (long)n, learning_rate), "clipped_sgd");
  return 0;
}

int ullis_hip_binaryconnect_sgd_fp16(ullis_hip_ctx* c, uint16_t* params, float* residual,
                                     const float* gradient, size_t n, float learning_rate) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (n == 0) return 0;
  NEED(params, "params");
  NEED(residual, "residual");
  NEED(gradient, "gradient");
  HIPCALL(binaryconnect_sgd(c->stream, params, residual, gradient, (long)n, learning_rate, 1.0f),
          "binaryconnect_sgd");
  return 0;
}

int ullis_hip_sign_pack_bits(ullis_hip_ctx* c, const float* x, size_t n, uint32_t* bits) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (n == 0) return 0;
  NEED(x, "x");
  NEED(bits, "bits");
  HIPCALL(sign_pack_bits(c->stream, x, (long)n, bits), "sign_pack_bits");
  return 0;
}

int ullis_hip_transpose_bits(ullis_hip_ctx* c, const uint32_t* bits, size_t out, size_t in,
                             uint32_t* bits_t) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (!dim_ok(out) || !dim_ok(in) || !prod_ok(out, in))
    return c->fail(ULLIS_HIP_ERR_INVALID, "transpose_bits shape mismatch");
  NEED(bits, "bits");
  NEED(bits_t, "bits_t");
  HIPCALL(transpose_bits(c->stream, bits, (long)out, (long)in, bits_t), "transpose_bits");
  return 0;
}

int ullis_hip_packed_head_train_sgd(ullis_hip_ctx* c, const uint16_t* hidden16, uint32_t* bits,
                                    uint32_t* bits_t, uint16_t* scale, uint16_t* bias,
                                    uint16_t* latent, float* latent_residual,
                                    float* scale_residual, float* bias_residual,
                                    const uint32_t* targets, size_t rows, size_t time, size_t d,
                                    size_t vocab, size_t horizon, uint32_t ignore_id,
                                    float learning_rate, float ste_scale, float* row_loss,
                                    float* stats4, float* g_hidden, float* g_scale, float* g_bias,
                                    float* g_w, uint32_t* invalid) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_linear(c, rows, d, vocab)) return rc;
  if (time == 0 || rows % time != 0)
    return c->fail(ULLIS_HIP_ERR_INVALID, "packed head SGD shape mismatch: rows % time != 0");
  if (vocab > (size_t)UINT32_MAX || horizon > (size_t)INT32_MAX)
    return c->fail(ULLIS_HIP_ERR_INVALID, "packed head SGD: vocab or horizon out of range");
  NEED(hidden16, "hidden");
  NEED(bits, "bits");
  NEED(scale, "scale");
  NEED(targets, "targets");
  NEED(row_loss, "row_loss");
  NEED(stats4, "stats4");
  NEED(g_hidden, "g_hidden");
  const bool upd = learning_rate > 0.0f;
  if (!(learning_rate >= 0.0f)) return c->fail(ULLIS_HIP_ERR_INVALID, "learning rate must be >= 0");
  if (upd) {
    NEED(latent, "latent");
    NEED(latent_residual, "latent_residual");
    NEED(scale_residual, "scale_residual");
    if (bias) NEED(bias_residual, "bias_residual");
  }
  const long R = (long)rows, D = (long)d, V = (long)vocab;
  const long words = cdiv(V * D, 32);
  const size_t head_ws = head_ce_workspace_bytes(R, D, V);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(Carver::bytes_for(4 * words) + head_ws, &ws)) return rc;
  Carver cv(ws);
  uint32_t* bt = bits_t;
  uint32_t* bt_scratch = cv.take<uint32_t>(words);
  void* hws = cv.take<char>(head_ws);
  if (!bt) {
    bt = bt_scratch;
    HIPCALL(transpose_bits(c->stream, bits, V, D, bt), "transpose_bits");
  }
  HeadCe h{};
  h.rows = R;
  h.time = (long)time;
  h.d = D;
  h.vocab = V;
  h.hidden16 = hidden16;
  h.bits = bits;
  h.bits_t = bt;
  h.scale = scale;
  h.bias = bias;
  h.targets = targets;
  h.ignore_id = ignore_id;
  h.horizon = (long)horizon;
  h.invalid = invalid;
  h.row_loss = row_loss;
  h.stats = stats4;
  h.g_hidden = g_hidden;
  h.g_scale = g_scale;
  h.g_bias = g_bias;
  h.g_w = g_w;
  h.lr = learning_rate;
  h.ste = ste_scale;
  h.latent = latent;
  h.latent_res = latent_residual;
  h.scale_upd = upd ? scale : nullptr;
  h.scale_res = scale_residual;
  h.bias_upd = upd ? bias : nullptr;
  h.bias_res = bias_residual;
  h.bits_new = upd ? bits : nullptr;
  h.bits_t_new = upd ? bits_t : nullptr;
  HIPCALL(head_ce(c->stream, h, hws), "packed_head_train_sgd");
  return 0;
}

size_t ullis_hip_heron_layout(const ullis_heron_dims* dims, ullis_tensor_desc* out, size_t cap,
                              uint64_t* bytes) {
  if (!dims) return 0;
  return ullis_heron_layout(dims, out, cap, bytes);
}

}  // extern "C"
