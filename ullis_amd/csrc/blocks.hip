// C ABI: the block-level methods of the reference's Metal train step
// (MetalRuntime::rosa_block_forward, cmix_block_forward,
// cmix_block_backward_sgd, rosa_o_stop_grad_sgd; src/metal.rs:1334, 1891,
// 2165, 2409), with device pointers and caller-owned tapes. They run the same
// internal launchers as the fused Heron step (heron.hip), so a caller that
// drives the model block by block (e.g. to run the suffix automaton between
// the Q/K/V projections and O) gets the step's arithmetic.
#include <hip/hip_runtime.h>

#include <climits>
#include <string>

#include "../../include/ullis_hip.h"
#include "context.hpp"
#include "ops.hpp"

using namespace ullis;

namespace {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned256(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 255u) == 0; }

#define NEED(ptr, name)                                                                  \
  do {                                                                                   \
    if (!(ptr)) return c->fail(ULLIS_HIP_ERR_INVALID, std::string(name) + " is NULL");   \
  } while (0)

#define HIPCALL(expr, what)                           \
  do {                                                \
    if (int rc_ = c->hip((expr), (what))) return rc_; \
  } while (0)

// batch, time, channels (and dim_ffn) non-zero, products within int32 rows
// and int64 elements (MetalDispatchShape / LinearDispatchShape, src/metal.rs:37-87)
int check_block(ullis_hip_ctx* c, size_t batch, size_t time, size_t d, size_t f, const char* what) {
  const size_t lim = (size_t)INT32_MAX;
  if (batch == 0 || time == 0 || d == 0 || f == 0 || batch > lim || time > lim || d > lim ||
      f > lim || batch * time > lim || (batch * time) > (size_t)LONG_MAX / (d > f ? d : f) ||
      d > (size_t)LONG_MAX / f)
    return c->fail(ULLIS_HIP_ERR_INVALID, std::string(what) + " shape must be non-zero and fit");
  return 0;
}

// Tape layouts (each piece 256-byte aligned from a 256-byte aligned base).
struct CmixTape {
  uint16_t* x16;   // [rows][d] block input, fp16
  uint16_t* sh16;  // [rows][d] x + xx * mix
  uint16_t* key16; // [rows][f] key pre-activation
  uint16_t* r2;    // [rows][f] max(key, 0)^2
};
CmixTape carve_cmix(void* base, long rows, long d, long f) {
  Carver cv(base);
  CmixTape t;
  t.x16 = cv.take<uint16_t>((size_t)(rows * d));
  t.sh16 = cv.take<uint16_t>((size_t)(rows * d));
  t.key16 = cv.take<uint16_t>((size_t)(rows * f));
  t.r2 = cv.take<uint16_t>((size_t)(rows * f));
  return t;
}
size_t cmix_tape_bytes(long rows, long d, long f) {
  return 2 * Carver::bytes_for(2ul * rows * d) + 2 * Carver::bytes_for(2ul * rows * f);
}

struct RosaTape {
  uint16_t* y16;    // [rows][d] (2 idx - 1) * e
  uint8_t* idx_rm;  // [rows][d] suffix-automaton output, row-major
};
RosaTape carve_rosa(void* base, long rows, long d) {
  Carver cv(base);
  RosaTape t;
  t.y16 = cv.take<uint16_t>((size_t)(rows * d));
  t.idx_rm = cv.take<uint8_t>((size_t)(rows * d));
  return t;
}
size_t rosa_tape_bytes(long rows, long d) {
  return Carver::bytes_for(2ul * rows * d) + Carver::bytes_for(1ul * rows * d);
}

// x of either dtype -> fp16 copy at dst (the GEMM operand precision).
hipError_t to_f16(hipStream_t s, const void* x, int x_dtype, long n, uint16_t* dst) {
  if (x_dtype == ULLIS_HIP_F16) return copy_device(s, dst, x, 2 * n);
  return f32_to_f16(s, static_cast<const float*>(x), n, dst);
}

}  // namespace

extern "C" {

size_t ullis_hip_cmix_tape_bytes(size_t rows, size_t d_model, size_t dim_ffn) {
  if (rows == 0 || d_model == 0 || dim_ffn == 0) return 0;
  return cmix_tape_bytes((long)rows, (long)d_model, (long)dim_ffn);
}

size_t ullis_hip_rosa_tape_bytes(size_t rows, size_t channels) {
  if (rows == 0 || channels == 0) return 0;
  return rosa_tape_bytes((long)rows, (long)channels);
}

int ullis_hip_cmix_block_forward(ullis_hip_ctx* c, const void* x, int x_dtype, const uint16_t* mix,
                                 const uint32_t* key_bits, const uint16_t* key_scale,
                                 const uint16_t* value_weight, size_t batch, size_t time,
                                 size_t d_model, size_t dim_ffn, float* out, void* tape) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_block(c, batch, time, d_model, dim_ffn, "CMix block")) return rc;
  NEED(x, "x");
  NEED(mix, "mix");
  NEED(key_bits, "key_bits");
  NEED(key_scale, "key_scale");
  NEED(value_weight, "value_weight");
  NEED(out, "out");
  NEED(tape, "tape");
  if (x_dtype != ULLIS_HIP_F16 && x_dtype != ULLIS_HIP_F32)
    return c->fail(ULLIS_HIP_ERR_INVALID, "x_dtype must be ULLIS_HIP_F16 or ULLIS_HIP_F32");
  if (!aligned256(tape)) return c->fail(ULLIS_HIP_ERR_INVALID, "tape must be 256-byte aligned");
  const long R = (long)(batch * time), T = (long)time, D = (long)d_model, F = (long)dim_ffn;
  hipStream_t s = c->stream;
  const CmixTape t = carve_cmix(tape, R, D, F);
  HIPCALL(to_f16(s, x, x_dtype, R * D, t.x16), "cmix x fp16");
  // s = x + (x[t-1] - x) * mix (time_shift_delta, src/model.rs:186-212)
  HIPCALL(time_shift_mix(s, t.x16, R, T, D, mix, t.sh16, nullptr, nullptr, nullptr, nullptr),
          "cmix mix");
  PackedFwdOut k;
  k.y16 = t.key16;
  k.relu2_16 = t.r2;
  HIPCALL(packed_forward(s, t.sh16, kF16, R, D, F, key_bits, key_scale, nullptr, k), "cmix key");
  HIPCALL(fp16_forward(s, t.r2, kF16, R, F, D, value_weight, out, nullptr, nullptr), "cmix value");
  return 0;
}

int ullis_hip_cmix_block_backward_sgd(ullis_hip_ctx* c, const void* tape, const float* gy,
                                      const uint16_t* mix, uint32_t* key_bits,
                                      uint32_t* key_bits_t, const uint16_t* key_scale,
                                      uint16_t* key_latent, float* key_residual,
                                      uint16_t* value_weight, float* value_residual,
                                      size_t batch, size_t time, size_t d_model, size_t dim_ffn,
                                      float learning_rate, float ste_scale, float* g_x,
                                      float* g_mix, float* g_key_scale) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_block(c, batch, time, d_model, dim_ffn, "CMix block backward")) return rc;
  NEED(tape, "tape");
  NEED(gy, "gy");
  NEED(mix, "mix");
  NEED(key_bits, "key_bits");
  NEED(key_scale, "key_scale");
  NEED(key_latent, "key_latent");
  NEED(key_residual, "key_residual");
  NEED(value_weight, "value_weight");
  NEED(value_residual, "value_residual");
  NEED(g_x, "g_x");
  NEED(g_mix, "g_mix");
  NEED(g_key_scale, "g_key_scale");
  if (!aligned256(tape)) return c->fail(ULLIS_HIP_ERR_INVALID, "tape must be 256-byte aligned");
  if (!(learning_rate >= 0.0f) || !__builtin_isfinite(learning_rate) ||
      !__builtin_isfinite(ste_scale))
    return c->fail(ULLIS_HIP_ERR_INVALID, "learning rate / ste scale must be finite, lr >= 0");
  const long R = (long)(batch * time), T = (long)time, D = (long)d_model, F = (long)dim_ffn;
  hipStream_t s = c->stream;
  const CmixTape t = carve_cmix(const_cast<void*>(tape), R, D, F);
  const int sv = pair_dw_splits(D, F, R), sk = pair_dw_splits(F, D, R);
  const long nbm = column_partial_blocks(R);  // time_shift_mix_backward's 16-row partials
  const long words = cdiv(F * D, 32);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(
          Carver::bytes_for(4) + Carver::bytes_for(2ul * R * D) + Carver::bytes_for(2ul * R * F) +
              Carver::bytes_for(4ul * R * D) + Carver::bytes_for(4ul * sv * D * F) +
              Carver::bytes_for(4ul * sk * F * D) + Carver::bytes_for(4ul * nbm * D) +
              Carver::bytes_for(4ul * words),
          &ws))
    return rc;
  Carver cv(ws);
  float* slot = cv.take<float>(1);
  uint16_t* gy16 = cv.take<uint16_t>((size_t)(R * D));
  uint16_t* gk16 = cv.take<uint16_t>((size_t)(R * F));
  float* g_sh = cv.take<float>((size_t)(R * D));
  float* pv = cv.take<float>((size_t)sv * D * F);
  float* pk = cv.take<float>((size_t)sk * F * D);
  float* pm = cv.take<float>((size_t)(nbm * D));
  uint32_t* bt_scratch = cv.take<uint32_t>((size_t)words);
  const uint32_t* bt = key_bits_t;
  if (!bt) {
    HIPCALL(transpose_bits(s, key_bits, F, D, bt_scratch), "key bits_t");
    bt = bt_scratch;
  }
  // gradient scaling of the fp16 GEMM operands: one power of two from max|gy|
  HIPCALL(fill_f32(s, slot, 1, 0.0f), "clear amax");
  HIPCALL(amax_f32(s, gy, R * D, slot), "gy amax");
  const bool g16 = aligned16(gy);
  if (g16) HIPCALL(scale_to_f16(s, gy, R * D, slot, gy16), "gy fp16");
  // value input gradient with the ReLU^2 backward (into gk16, gy-scaled) and
  // the value weight gradient; then the key input and weight gradients, all
  // on the pre-update weights (src/model.rs:1145-1168)
  const GradIn g{gy, slot, g16 ? gy16 : nullptr};
  const GradIn scaled_only{nullptr, slot};
  HIPCALL(fp16_backward_pair(s, Fp16DxArgs{g, R, F, D, value_weight, nullptr, t.key16, gk16},
                             WeightGradArgs{g, g16 ? gy16 : nullptr, t.r2, R, F, D, sv, pv}),
          "cmix value backward");
  HIPCALL(packed_backward_pair(s, PackedDxArgs{scaled_only, gk16, R, D, F, bt, key_scale, g_sh,
                                               nullptr, 0},
                               WeightGradArgs{scaled_only, gk16, t.sh16, R, D, F, sk, pk}),
          "cmix key backward");
  // lerp_shift_backward (src/model.rs:1207-1240): g_x and the mix gradient
  int nb = 0;
  HIPCALL(time_shift_mix_backward(s, g_sh, t.x16, mix, R, T, D, g_x, pm, &nb), "cmix mix backward");
  if (nb != nbm) return c->fail(ULLIS_HIP_ERR_RUNTIME, "mix backward partial count");
  HIPCALL(vector_finish(s, pm, nb, D, g_mix, 0.0f, nullptr, nullptr), "g_mix");
  // value clipped SGD, key BinaryConnect step + repack; the key scale and
  // the mix vector are stepped by the caller from g_key_scale / g_mix, as
  // the reference's host does (src/model.rs:1117-1137)
  HIPCALL(fp16_weight_finish(s, pv, sv, D, F, slot, learning_rate, value_weight, value_residual,
                             nullptr),
          "value step");
  PackedFinish f;
  f.part = pk;
  f.splits = sk;
  f.out = F;
  f.in = D;
  f.scale = key_scale;
  f.bits_old = key_bits;
  f.amax = slot;
  f.extra_mul = nullptr;
  f.ste = ste_scale;
  f.lr = learning_rate;
  f.latent = key_latent;
  f.latent_res = key_residual;
  f.g_scale = g_key_scale;
  f.g_w = nullptr;
  f.bits_new = key_bits;
  HIPCALL(packed_weight_finish(s, f), "key step");
  if (key_bits_t) HIPCALL(transpose_bits(s, key_bits, F, D, key_bits_t), "key bits_t");
  return 0;
}

int ullis_hip_rosa_qkv_forward(ullis_hip_ctx* c, const void* x, int x_dtype,
                               const uint16_t* mix_q, const uint16_t* mix_k,
                               const uint16_t* mix_v, const uint32_t* q_bits,
                               const uint16_t* q_scale, const uint16_t* q_bias,
                               const uint32_t* k_bits, const uint16_t* k_scale,
                               const uint16_t* k_bias, const uint32_t* v_bits,
                               const uint16_t* v_scale, const uint16_t* v_bias, size_t batch,
                               size_t time, size_t channels, uint32_t* q_plane,
                               uint32_t* k_plane, uint32_t* v_plane) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_block(c, batch, time, channels, channels, "ROSA block")) return rc;
  NEED(x, "x");
  NEED(mix_q, "mix_q");
  NEED(mix_k, "mix_k");
  NEED(mix_v, "mix_v");
  NEED(q_bits, "q_bits");
  NEED(q_scale, "q_scale");
  NEED(q_bias, "q_bias");
  NEED(k_bits, "k_bits");
  NEED(k_scale, "k_scale");
  NEED(k_bias, "k_bias");
  NEED(v_bits, "v_bits");
  NEED(v_scale, "v_scale");
  NEED(v_bias, "v_bias");
  NEED(q_plane, "q_plane");
  NEED(k_plane, "k_plane");
  NEED(v_plane, "v_plane");
  if (x_dtype != ULLIS_HIP_F16 && x_dtype != ULLIS_HIP_F32)
    return c->fail(ULLIS_HIP_ERR_INVALID, "x_dtype must be ULLIS_HIP_F16 or ULLIS_HIP_F32");
  const long R = (long)(batch * time), T = (long)time, D = (long)channels;
  hipStream_t s = c->stream;
  const bool fused = D % 32 == 0;
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(4 * Carver::bytes_for(2ul * R * D) +
                                     (fused ? 0 : Carver::bytes_for(4ul * R * D)),
                                 &ws))
    return rc;
  Carver cv(ws);
  uint16_t* x16 = cv.take<uint16_t>((size_t)(R * D));
  uint16_t* in16[3] = {cv.take<uint16_t>((size_t)(R * D)), cv.take<uint16_t>((size_t)(R * D)),
                       cv.take<uint16_t>((size_t)(R * D))};
  HIPCALL(to_f16(s, x, x_dtype, R * D, x16), "rosa x fp16");
  // q/k/v inputs x + xx * x_{q,k,v} (ullis_time_shift_mix3)
  HIPCALL(time_shift_mix(s, x16, R, T, D, mix_q, in16[0], mix_k, in16[1], mix_v, in16[2]),
          "rosa mix3");
  const uint16_t* const xin[3] = {in16[0], in16[1], in16[2]};
  const uint32_t* const wb[3] = {q_bits, k_bits, v_bits};
  const uint16_t* const sc[3] = {q_scale, k_scale, v_scale};
  const uint16_t* const bi[3] = {q_bias, k_bias, v_bias};
  uint32_t* const planes[3] = {q_plane, k_plane, v_plane};
  if (fused) {
    // bit (row * channels + c) = projection > 0, from the GEMM epilogue
    HIPCALL(packed_forward_bits3(s, xin, R, D, D, wb, sc, bi, planes), "rosa qkv");
    return 0;
  }
  float* y32 = cv.take<float>((size_t)(R * D));
  for (int j = 0; j < 3; ++j) {
    PackedFwdOut o;
    o.y32 = y32;
    HIPCALL(packed_forward(s, xin[j], kF16, R, D, D, wb[j], sc[j], bi[j], o), "rosa qkv");
    HIPCALL(sign_pack_bits(s, y32, R * D, planes[j]), "rosa sign bits");
  }
  return 0;
}

int ullis_hip_rosa_out_forward(ullis_hip_ctx* c, const uint8_t* idx, const uint16_t* e,
                               const uint32_t* o_bits, const uint16_t* o_scale,
                               const uint16_t* o_bias, size_t batch, size_t time,
                               size_t channels, float* out, void* tape) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_block(c, batch, time, channels, channels, "ROSA output")) return rc;
  NEED(idx, "idx");
  NEED(e, "e");
  NEED(o_bits, "o_bits");
  NEED(o_scale, "o_scale");
  NEED(o_bias, "o_bias");
  NEED(out, "out");
  NEED(tape, "tape");
  if (!aligned256(tape)) return c->fail(ULLIS_HIP_ERR_INVALID, "tape must be 256-byte aligned");
  const long B = (long)batch, T = (long)time, D = (long)channels, R = B * T;
  hipStream_t s = c->stream;
  const RosaTape t = carve_rosa(tape, R, D);
  // y = (2 idx - 1) * e (rosa_qkv_out_batched_channel_major, src/rosa.rs:614-639)
  HIPCALL(rosa_expand(s, idx, e, B, T, D, t.y16, t.idx_rm), "rosa y");
  PackedFwdOut o;
  o.y32 = out;
  HIPCALL(packed_forward(s, t.y16, kF16, R, D, D, o_bits, o_scale, o_bias, o), "rosa o");
  return 0;
}

int ullis_hip_rosa_o_stop_grad_sgd(ullis_hip_ctx* c, const void* tape, const float* gy,
                                   uint32_t* o_bits, uint32_t* o_bits_t, const uint16_t* o_scale,
                                   uint16_t* o_latent, float* o_residual, size_t rows,
                                   size_t channels, float learning_rate, float ste_scale,
                                   float* g_e, float* g_scale, float* g_bias) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (int rc = check_block(c, 1, rows, channels, channels, "ROSA O backward")) return rc;
  NEED(tape, "tape");
  NEED(gy, "gy");
  NEED(o_bits, "o_bits");
  NEED(o_scale, "o_scale");
  NEED(o_latent, "o_latent");
  NEED(o_residual, "o_residual");
  NEED(g_e, "g_e");
  NEED(g_scale, "g_scale");
  NEED(g_bias, "g_bias");
  if (!aligned256(tape)) return c->fail(ULLIS_HIP_ERR_INVALID, "tape must be 256-byte aligned");
  if (!(learning_rate >= 0.0f) || !__builtin_isfinite(learning_rate) ||
      !__builtin_isfinite(ste_scale))
    return c->fail(ULLIS_HIP_ERR_INVALID, "learning rate / ste scale must be finite, lr >= 0");
  const long R = (long)rows, D = (long)channels;
  hipStream_t s = c->stream;
  const RosaTape t = carve_rosa(const_cast<void*>(tape), R, D);
  const int so = pair_dw_splits(D, D, R);
  const long nb_col = column_partial_blocks(R);
  const long words = cdiv(D * D, 32);
  void* ws = nullptr;
  if (int rc = c->ensure_scratch(
          Carver::bytes_for(4) + Carver::bytes_for(2ul * R * D) + Carver::bytes_for(4ul * R * D) +
              Carver::bytes_for(4ul * so * D * D) + 2 * Carver::bytes_for(4ul * nb_col * D) +
              Carver::bytes_for(4ul * words),
          &ws))
    return rc;
  Carver cv(ws);
  float* slot = cv.take<float>(1);
  uint16_t* gy16 = cv.take<uint16_t>((size_t)(R * D));
  float* g_y = cv.take<float>((size_t)(R * D));
  float* po = cv.take<float>((size_t)so * D * D);
  float* pe = cv.take<float>((size_t)(nb_col * D));
  float* pb = cv.take<float>((size_t)(nb_col * D));
  uint32_t* bt_scratch = cv.take<uint32_t>((size_t)words);
  const uint32_t* bt = o_bits_t;
  if (!bt) {
    HIPCALL(transpose_bits(s, o_bits, D, D, bt_scratch), "o bits_t");
    bt = bt_scratch;
  }
  HIPCALL(fill_f32(s, slot, 1, 0.0f), "clear amax");
  HIPCALL(amax_f32(s, gy, R * D, slot), "gy amax");
  // O bias gradient (column sums of gy) and the scaled fp16 copy of gy
  int nb = 0;
  const bool g16 = aligned16(gy);
  HIPCALL(column_sum_partials(s, gy, nullptr, R, D, pb, &nb, g16 ? gy16 : nullptr,
                              g16 ? slot : nullptr),
          "o g_bias");
  if (nb != nb_col) return c->fail(ULLIS_HIP_ERR_RUNTIME, "o bias partial count");
  HIPCALL(vector_finish(s, pb, nb, D, g_bias, 0.0f, nullptr, nullptr), "g_bias");
  // O input gradient reduced straight to the e gradient partials
  // (rosa_e_grad, src/model.rs:1608-1634: g_e[c] = sum g_y * (2 idx - 1)) and
  // the O weight gradient, in one launch
  const GradIn g{gy, slot, g16 ? gy16 : nullptr};
  PackedDxArgs dx{g, g16 ? gy16 : nullptr, R, D, D, bt, o_scale, g_y, nullptr, 0};
  dx.sign_idx = t.idx_rm;
  dx.col_part = pe;
  HIPCALL(packed_backward_pair(
              s, dx, WeightGradArgs{g, g16 ? gy16 : nullptr, t.y16, R, D, D, so, po}),
          "rosa o backward");
  HIPCALL(vector_finish(s, pe, (int)nb_col, D, g_e, 0.0f, nullptr, nullptr), "g_e");
  // O BinaryConnect step + repack; scale, bias and e are stepped by the
  // caller from the returned gradients (src/model.rs:1481-1490)
  PackedFinish f;
  f.part = po;
  f.splits = so;
  f.out = D;
  f.in = D;
  f.scale = o_scale;
  f.bits_old = o_bits;
  f.amax = slot;
  f.extra_mul = nullptr;
  f.ste = ste_scale;
  f.lr = learning_rate;
  f.latent = o_latent;
  f.latent_res = o_residual;
  f.g_scale = g_scale;
  f.g_w = nullptr;
  f.bits_new = o_bits;
  HIPCALL(packed_weight_finish(s, f), "o step");
  if (o_bits_t) HIPCALL(transpose_bits(s, o_bits, D, D, o_bits_t), "o bits_t");
  return 0;
}

}  // extern "C"
