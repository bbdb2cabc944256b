/*
 * Heron parameter arena: one contiguous block holding every trainable tensor
 * of the model, in the element layouts of the reference's checkpoint v2.
 *
 * Tensor names are the reference's safetensors names
 * (src/model.rs:3426-3468 push_*, :3878-3932; train carry :3742-3803):
 *   embedding is NOT part of the arena (the reference gathers and scatters it
 *   on the host in its GPU path too, src/model.rs:2866-2873, :2986-2993);
 *   ln_out.{weight,bias}; head.{bits,scale,bias}; blocks.{i}.{ln0,ln2,ln3}.*;
 *   blocks.{i}.rosa.{x_q,x_k,x_v,e}; blocks.{i}.rosa.{q,k,v,o}.{bits,scale,bias};
 *   blocks.{i}.ffn.{x_k,value}; blocks.{i}.ffn.key.{bits,scale};
 *   train carry <prefix>.latent (f16) and <name>.residual (f32).
 *
 * Element layouts (src/model.rs:2266-2272):
 *   bits   little-endian u32 words, row-major [out, in], bit 0 of word 0 is
 *          weight [0,0], 1 means +1, no per-row padding;
 *   f16    IEEE binary16 bit patterns stored as u16;
 *   f32    FP32 error-diffusion carry, same element count as its f16 tensor.
 *
 * One derived tensor has no checkpoint counterpart: "<prefix>.bits_t", the
 * sign bits of the TRANSPOSED matrix ([in, out], same LSB-first packing). The
 * GPU keeps it beside "<prefix>.bits" for the input-gradient GEMMs; it is
 * rebuilt from the latents on every update and is never serialised.
 *
 * Plain C99, header-only, shared by the HIP library, the CPU oracle and the
 * Python bindings (which call the exported copies of these functions).
 */
#ifndef ULLIS_HERON_LAYOUT_H
#define ULLIS_HERON_LAYOUT_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ullis_dtype { ULLIS_DT_F16 = 1, ULLIS_DT_F32 = 2, ULLIS_DT_U32 = 3, ULLIS_DT_U8 = 4 };

#define ULLIS_NAME_MAX 64
#define ULLIS_ARENA_ALIGN 256u

typedef struct ullis_tensor_desc {
  char name[ULLIS_NAME_MAX];
  int32_t dtype;     /* enum ullis_dtype */
  int32_t derived;   /* 1: GPU cache with no checkpoint counterpart */
  uint64_t count;    /* elements */
  uint64_t offset;   /* bytes from arena base, ULLIS_ARENA_ALIGN aligned */
} ullis_tensor_desc;

typedef struct ullis_heron_dims {
  uint32_t d_model;
  uint32_t n_layers;
  uint32_t dim_ffn;
  uint32_t vocab;
} ullis_heron_dims;

static inline uint64_t ullis_dtype_size(int dtype) {
  switch (dtype) {
    case ULLIS_DT_F16: return 2;
    case ULLIS_DT_F32: return 4;
    case ULLIS_DT_U32: return 4;
    case ULLIS_DT_U8: return 1;
    default: return 0;
  }
}

/* packed_word_count, src/model.rs:142-144 */
static inline uint64_t ullis_packed_words(uint64_t weights) { return (weights + 31u) / 32u; }

typedef struct ullis_layout_builder {
  ullis_tensor_desc* out;
  size_t cap;
  size_t n;
  uint64_t cursor;
} ullis_layout_builder;

static inline void ullis_lb_add(ullis_layout_builder* b, const char* name, int dtype,
                                uint64_t count, int derived) {
  if (b->out && b->n < b->cap) {
    ullis_tensor_desc* d = &b->out[b->n];
    memset(d, 0, sizeof(*d));
    strncpy(d->name, name, ULLIS_NAME_MAX - 1);
    d->dtype = dtype;
    d->derived = derived;
    d->count = count;
    d->offset = b->cursor;
  }
  b->n += 1;
  b->cursor += count * ullis_dtype_size(dtype);
  b->cursor = (b->cursor + ULLIS_ARENA_ALIGN - 1) / ULLIS_ARENA_ALIGN * ULLIS_ARENA_ALIGN;
}

static inline void ullis_lb_f16_with_carry(ullis_layout_builder* b, const char* name,
                                           uint64_t count) {
  char buf[ULLIS_NAME_MAX];
  ullis_lb_add(b, name, ULLIS_DT_F16, count, 0);
  snprintf(buf, sizeof buf, "%s.residual", name);
  ullis_lb_add(b, buf, ULLIS_DT_F32, count, 0);
}

static inline void ullis_lb_ln(ullis_layout_builder* b, const char* prefix, uint64_t d) {
  char buf[ULLIS_NAME_MAX];
  snprintf(buf, sizeof buf, "%s.weight", prefix);
  ullis_lb_f16_with_carry(b, buf, d);
  snprintf(buf, sizeof buf, "%s.bias", prefix);
  ullis_lb_f16_with_carry(b, buf, d);
}

static inline void ullis_lb_packed(ullis_layout_builder* b, const char* prefix, uint64_t out,
                                   uint64_t in, int has_bias, int with_transpose) {
  char buf[ULLIS_NAME_MAX];
  uint64_t w = out * in;
  snprintf(buf, sizeof buf, "%s.bits", prefix);
  ullis_lb_add(b, buf, ULLIS_DT_U32, ullis_packed_words(w), 0);
  if (with_transpose) {
    snprintf(buf, sizeof buf, "%s.bits_t", prefix);
    ullis_lb_add(b, buf, ULLIS_DT_U32, ullis_packed_words(w), 1);
  }
  snprintf(buf, sizeof buf, "%s.scale", prefix);
  ullis_lb_f16_with_carry(b, buf, out);
  if (has_bias) {
    snprintf(buf, sizeof buf, "%s.bias", prefix);
    ullis_lb_f16_with_carry(b, buf, out);
  }
  snprintf(buf, sizeof buf, "%s.latent", prefix);
  ullis_lb_f16_with_carry(b, buf, w);
}

/*
 * Enumerates the arena. Returns the number of tensors; writes up to `cap`
 * descriptors into `out` (may be NULL) and the total byte size into *bytes.
 * Order follows to_safetensors_bytes (src/model.rs:3426-3445).
 */
static inline size_t ullis_heron_layout(const ullis_heron_dims* dims, ullis_tensor_desc* out,
                                        size_t cap, uint64_t* bytes) {
  ullis_layout_builder b;
  char p[ULLIS_NAME_MAX];
  char q[ULLIS_NAME_MAX];
  uint64_t d = dims->d_model, f = dims->dim_ffn, v = dims->vocab;
  uint32_t i;
  b.out = out;
  b.cap = cap;
  b.n = 0;
  b.cursor = 0;
  ullis_lb_ln(&b, "ln_out", d);
  ullis_lb_packed(&b, "head", v, d, 1, 1);
  for (i = 0; i < dims->n_layers; ++i) {
    if (i == 0) {
      snprintf(p, sizeof p, "blocks.%u.ln0", i);
      ullis_lb_ln(&b, p, d);
    }
    snprintf(p, sizeof p, "blocks.%u.ln2", i);
    ullis_lb_ln(&b, p, d);
    snprintf(p, sizeof p, "blocks.%u.ln3", i);
    ullis_lb_ln(&b, p, d);
    snprintf(q, sizeof q, "blocks.%u.rosa.x_q", i);
    ullis_lb_f16_with_carry(&b, q, d);
    snprintf(q, sizeof q, "blocks.%u.rosa.x_k", i);
    ullis_lb_f16_with_carry(&b, q, d);
    snprintf(q, sizeof q, "blocks.%u.rosa.x_v", i);
    ullis_lb_f16_with_carry(&b, q, d);
    snprintf(q, sizeof q, "blocks.%u.rosa.e", i);
    ullis_lb_f16_with_carry(&b, q, d);
    snprintf(p, sizeof p, "blocks.%u.rosa.q", i);
    ullis_lb_packed(&b, p, d, d, 1, 0);
    snprintf(p, sizeof p, "blocks.%u.rosa.k", i);
    ullis_lb_packed(&b, p, d, d, 1, 0);
    snprintf(p, sizeof p, "blocks.%u.rosa.v", i);
    ullis_lb_packed(&b, p, d, d, 1, 0);
    snprintf(p, sizeof p, "blocks.%u.rosa.o", i);
    ullis_lb_packed(&b, p, d, d, 1, 1);
    snprintf(q, sizeof q, "blocks.%u.ffn.x_k", i);
    ullis_lb_f16_with_carry(&b, q, d);
    snprintf(p, sizeof p, "blocks.%u.ffn.key", i);
    ullis_lb_packed(&b, p, f, d, 0, 1);
    snprintf(q, sizeof q, "blocks.%u.ffn.value", i);
    ullis_lb_f16_with_carry(&b, q, d * f);
  }
  if (bytes) *bytes = b.cursor;
  return b.n;
}

/* Byte offset of a named tensor, or UINT64_MAX. Linear scan: set-up only. */
static inline uint64_t ullis_heron_offset(const ullis_tensor_desc* descs, size_t n,
                                          const char* name) {
  size_t i;
  for (i = 0; i < n; ++i) {
    if (strcmp(descs[i].name, name) == 0) return descs[i].offset;
  }
  return UINT64_MAX;
}

#ifdef __cplusplus
}
#endif

#endif /* ULLIS_HERON_LAYOUT_H */
