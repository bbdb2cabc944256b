// Parameter-update bodies shared by the immediate launchers (linear.hip,
// elementwise.hip) and the batched end-of-step update kernels (deferred.hip).
//
// Reference semantics: PackedBinaryLinear::apply_packed_sgd / rebinarize
// (src/model.rs:808-884), Fp16Linear::apply_clipped_sgd (src/model.rs:463-470),
// Fp16Storage::apply_clipped_sgd / apply_binaryconnect_sgd
// (src/precision.rs:106-134).
#pragma once

#include "common.hpp"
#include "ops.hpp"

namespace ullis {

// Row o of a packed latent finish, 256 threads (red: 256 floats of LDS):
// G = sum of split partials * gmul; g_scale[o] = sum_i sign_old * G;
// BinaryConnect step on g_w * ste with g_w = scale[o] * G; optionally the
// scale step and the repack of row o (whole waves over 64-weight chunks).
__device__ __forceinline__ void packed_finish_row(const PackedFinish& f, long o, float lr,
                                                  float* red) {
  float gmul = f.amax ? 1.0f / grad_scale_from_amax(*f.amax) : 1.0f;
  if (f.extra_mul) gmul *= *f.extra_mul;
  const float sc = f16_bits_to_f32(f.scale[o]);
  const long wn = f.out * f.in;
  float gs = 0.0f;
  const int lane = threadIdx.x & 63;
  for (long i = threadIdx.x; i < f.in; i += blockDim.x) {
    const long w = o * f.in + i;
    float G = 0.0f;
    for (int z = 0; z < f.splits; ++z) G += f.part[(long)z * wn + w];
    G *= gmul;
    const bool plus = (f.bits_old[w >> 5] >> (w & 31)) & 1u;
    gs += plus ? G : -G;
    const float gw = sc * G;
    if (f.g_w) f.g_w[w] = gw;
    if (f.latent) {
      binaryconnect_sgd_one(f.latent[w], f.latent_res[w], gw * f.ste, lr);
      if (f.bits_new) {
        // whole waves cover 64 consecutive weights of row o (in % 64 == 0);
        // each word of the row is read above before it is rewritten here
        const unsigned long long m = __ballot(latent_is_plus(f.latent[w]));
        if (lane == 0) f.bits_new[w >> 5] = (uint32_t)m;
        if (lane == 32) f.bits_new[w >> 5] = (uint32_t)(m >> 32);
      }
    }
  }
  red[threadIdx.x] = gs;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (f.g_scale) f.g_scale[o] = red[0];
    if (f.scale_upd && lr > 0.0f) clipped_sgd_one(f.scale_upd[o], f.scale_res[o], red[0], lr);
  }
}

// One wave per row o of a packed latent finish (the same steps as
// packed_finish_row), eight consecutive weights per lane and pass with 16-byte
// loads; requires packed_finish_wave_ok. The repack assembles each 32-bit
// word from four lanes, so whole words of row o (in % 32 == 0) are written
// after the wave has read them.
// With f.row_flips / f.row_step it also records row o's bit flips and summed
// |latent step| (no effect on the update).
__device__ __forceinline__ void packed_finish_row_wave(const PackedFinish& f, long o, float lr) {
  float gmul = f.amax ? 1.0f / grad_scale_from_amax(*f.amax) : 1.0f;
  if (f.extra_mul) gmul *= *f.extra_mul;
  const float sc = f16_bits_to_f32(f.scale[o]);
  const long wn = f.out * f.in;
  const int lane = threadIdx.x & 63;
  float gs = 0.0f;
  uint32_t flips = 0;
  float step = 0.0f;
  for (long i0 = lane * 8; i0 < f.in; i0 += 512) {
    const long w = o * f.in + i0;
    floatx4 g0 = {0.0f, 0.0f, 0.0f, 0.0f}, g1 = g0;
    for (int z = 0; z < f.splits; ++z) {
      const floatx4* p = reinterpret_cast<const floatx4*>(f.part + (long)z * wn + w);
      g0 += p[0];
      g1 += p[1];
    }
    float G[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
    const uint32_t old_word = f.bits_old[w >> 5];
    const uint32_t signs = old_word >> (w & 31);
    float gw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      G[j] *= gmul;
      gs += ((signs >> j) & 1u) ? G[j] : -G[j];
      gw[j] = sc * G[j];
    }
    if (f.g_w) {
      floatx4* q = reinterpret_cast<floatx4*>(f.g_w + w);
      q[0] = floatx4{gw[0], gw[1], gw[2], gw[3]};
      q[1] = floatx4{gw[4], gw[5], gw[6], gw[7]};
    }
    if (f.latent) {
      u32x4 lat = *reinterpret_cast<const u32x4*>(f.latent + w);
      floatx4* rp = reinterpret_cast<floatx4*>(f.latent_res + w);
      floatx4 r0 = rp[0], r1 = rp[1];
      uint16_t v[8];
      float r[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
      uint32_t plus = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] = (uint16_t)(lat[j >> 1] >> (16 * (j & 1)));
        const uint16_t before = v[j];
        binaryconnect_sgd_one(v[j], r[j], gw[j] * f.ste, lr);
        plus |= (latent_is_plus(v[j]) ? 1u : 0u) << j;
        if (f.row_step) step += __builtin_fabsf(f16_bits_to_f32(before) - f16_bits_to_f32(v[j]));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) lat[j] = (uint32_t)v[2 * j] | ((uint32_t)v[2 * j + 1] << 16);
      *reinterpret_cast<u32x4*>(f.latent + w) = lat;
      rp[0] = floatx4{r[0], r[1], r[2], r[3]};
      rp[1] = floatx4{r[4], r[5], r[6], r[7]};
      if (f.bits_new) {
        uint32_t word = plus << (8 * (lane & 3));
        word |= __shfl_xor(word, 1, 64);
        word |= __shfl_xor(word, 2, 64);
        if ((lane & 3) == 0) {
          f.bits_new[w >> 5] = word;
          flips += (uint32_t)__builtin_popcount(word ^ old_word);
        }
      }
    }
  }
  gs = wave_sum(gs);
  if (f.row_flips) {
    const uint32_t n = wave_sum_u32(flips);
    if (lane == 0) f.row_flips[o] = n;
  }
  if (f.row_step) {
    step = wave_sum(step);
    if (lane == 0) f.row_step[o] = step;
  }
  if (lane == 0) {
    if (f.g_scale) f.g_scale[o] = gs;
    if (f.scale_upd && lr > 0.0f) clipped_sgd_one(f.scale_upd[o], f.scale_res[o], gs, lr);
  }
}

// Element i of an fp16 weight finish: G = sum of split partials / gy-scale,
// optional g_w output, clipped SGD on w[i].
__device__ __forceinline__ void fp16_finish_one(const float* part, int splits, long n, long i,
                                                const float* amax, float lr, uint16_t* w,
                                                float* w_res, float* g_w) {
  const float m = amax ? 1.0f / grad_scale_from_amax(*amax) : 1.0f;
  float G = 0.0f;
  for (int z = 0; z < splits; ++z) G += part[(long)z * n + i];
  G *= m;
  if (g_w) g_w[i] = G;
  if (w) clipped_sgd_one(w[i], w_res[i], G, lr);
}

// Elements [i, i + 4) of an fp16 weight finish with vector loads (n % 4 == 0,
// part / w_res / g_w 16-byte and w 8-byte aligned; fp16_finish_vec_ok).
__device__ __forceinline__ void fp16_finish_four(const float* part, int splits, long n, long i,
                                                 const float* amax, float lr, uint16_t* w,
                                                 float* w_res, float* g_w) {
  const float m = amax ? 1.0f / grad_scale_from_amax(*amax) : 1.0f;
  floatx4 G = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int z = 0; z < splits; ++z) G += *reinterpret_cast<const floatx4*>(part + (long)z * n + i);
#pragma unroll
  for (int j = 0; j < 4; ++j) G[j] *= m;
  if (g_w) *reinterpret_cast<floatx4*>(g_w + i) = G;
  if (!w) return;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x2 wv = *reinterpret_cast<const u32x2*>(w + i);
  floatx4 rv = *reinterpret_cast<const floatx4*>(w_res + i);
  uint16_t v[4] = {(uint16_t)wv[0], (uint16_t)(wv[0] >> 16), (uint16_t)wv[1],
                   (uint16_t)(wv[1] >> 16)};
  float r[4] = {rv[0], rv[1], rv[2], rv[3]};
#pragma unroll
  for (int j = 0; j < 4; ++j) clipped_sgd_one(v[j], r[j], G[j], lr);
  wv[0] = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  wv[1] = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
  *reinterpret_cast<u32x2*>(w + i) = wv;
  *reinterpret_cast<floatx4*>(w_res + i) = floatx4{r[0], r[1], r[2], r[3]};
}

// 32x32 bit-block `blk` of bits [out][in] -> bits_t [in][out], one half-wave
// per block (out % 32 == 0, in % 32 == 0); every lane of the wave calls it.
__device__ __forceinline__ void transpose_bits_block(const uint32_t* bits, long out, long in,
                                                     uint32_t* bits_t, long blk, bool active) {
  const int lane = threadIdx.x & 63;
  const long ib = in / 32;
  const long bo = active ? blk / ib : 0, bi = active ? blk % ib : 0;
  const long o = bo * 32 + (lane & 31);
  const uint32_t word = active ? bits[(o * in + bi * 32) >> 5] : 0u;
  for (int b = 0; b < 32; ++b) {
    const unsigned long long m = __ballot((word >> b) & 1u);
    if ((lane & 31) == 0 && active) {
      const long i = bi * 32 + b;
      bits_t[(i * out + bo * 32) >> 5] = (lane < 32) ? (uint32_t)m : (uint32_t)(m >> 32);
    }
  }
}

// Block of a fixed-order column reduction of part[nblk][ncols], 1024 threads
// = 16 groups of four adjacent columns x 64 partial subsets (subset k sums
// rows k, k + 64, ...; then a tree over subsets; red: LDS [64][64]), so each
// partial row is read as 256 contiguous bytes. Columns [0, split) go to a,
// the rest to b; lr_a / lr_b are the learning rates of the steps.
__device__ __forceinline__ void vec_reduce_block(const float* part, int nblk, long ncols,
                                                 long split, const VecTarget& a, float lr_a,
                                                 const VecTarget& b, float lr_b, long colblk,
                                                 float (*red)[64]) {
  const int lg = threadIdx.x & 15, sub = threadIdx.x >> 4;
  const long c0 = colblk * 64 + lg * 4;
  floatx4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ncols % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15u) == 0) {
    if (c0 < ncols) {
#pragma unroll 4
      for (int k = sub; k < nblk; k += 64)
        s += *reinterpret_cast<const floatx4*>(part + (long)k * ncols + c0);
    }
  } else {
    for (int k = sub; k < nblk; k += 64)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c0 + j < ncols) s[j] += part[(long)k * ncols + c0 + j];
  }
  *reinterpret_cast<floatx4*>(&red[sub][lg * 4]) = s;
  __syncthreads();
  for (int st = 32; st > 0; st >>= 1) {
    if (sub < st) {
      floatx4 v = *reinterpret_cast<floatx4*>(&red[sub][lg * 4]);
      v += *reinterpret_cast<floatx4*>(&red[sub + st][lg * 4]);
      *reinterpret_cast<floatx4*>(&red[sub][lg * 4]) = v;
    }
    __syncthreads();
  }
  const long col = colblk * 64 + threadIdx.x;
  if (threadIdx.x < 64 && col < ncols) {
    const bool first = col < split;
    const VecTarget& t = first ? a : b;
    const float lr = first ? lr_a : lr_b;
    const long i = first ? col : col - split;
    float v = red[0][threadIdx.x];
    if (t.mul) v *= *t.mul;
    if (t.out) t.out[i] = v;
    if (t.values && lr > 0.0f && !(t.abort && *t.abort))
      clipped_sgd_one(t.values[i], t.residual[i], v, lr);
  }
}

}  // namespace ullis
