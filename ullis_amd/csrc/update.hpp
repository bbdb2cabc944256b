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
// = 16 columns x 64 partial subsets (red: LDS [64][16]); columns [0, split)
// go to a, the rest to b. lr_a / lr_b are the learning rates of the steps.
__device__ __forceinline__ void vec_reduce_block(const float* part, int nblk, long ncols,
                                                 long split, const VecTarget& a, float lr_a,
                                                 const VecTarget& b, float lr_b, long colblk,
                                                 float (*red)[16]) {
  const int lc = threadIdx.x & 15, sub = threadIdx.x >> 4;
  const long col = colblk * 16 + lc;
  float s = 0.0f;
  if (col < ncols)
    for (int k = sub; k < nblk; k += 64) s += part[(long)k * ncols + col];
  red[sub][lc] = s;
  __syncthreads();
  for (int st = 32; st > 0; st >>= 1) {
    if (sub < st) red[sub][lc] += red[sub + st][lc];
    __syncthreads();
  }
  if (sub == 0 && col < ncols) {
    const bool first = col < split;
    const VecTarget& t = first ? a : b;
    const float lr = first ? lr_a : lr_b;
    const long i = first ? col : col - split;
    float v = red[0][lc];
    if (t.mul) v *= *t.mul;
    if (t.out) t.out[i] = v;
    if (t.values && lr > 0.0f) clipped_sgd_one(t.values[i], t.residual[i], v, lr);
  }
}

}  // namespace ullis
