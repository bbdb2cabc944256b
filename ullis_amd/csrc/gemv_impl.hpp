// Device building blocks of the few-row forward products (rows <= 8: T = 1
// decode): x staged in LDS as fp16, and the packed product's 32-row weight
// tile on MFMA. Shared by gemv.hip (the standalone products) and decode.hip
// (the decode step's fused kernels, which stage LayerNorm / mix outputs or
// ROSA's expanded y instead of a plain x).
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"
#include "ops.hpp"

namespace ullis {
namespace gemv {

constexpr int kThreads = 256;
constexpr long kLds = 64 * 1024;
// LDS of the packed tile: the sign table (32 words) and four 16 x 64 partial tiles
constexpr int kLutWords = 32;
constexpr int kRedFloats = 4 * 16 * 64;

// x rows 0 .. rows_m -> LDS fp16 [rows_m][in] with 16-byte loads (in % 8 ==
// 0, n8 >= 1; x 16-byte aligned), a thread's loads issued before its stores:
// 8 loads in flight per thread for fp16 x, 8 pairs for fp32 x (16 for fp16
// measured slower in the value product at 8 rows: 15.9 against 10.7 us).
// Every load is issued (indices past the end reload the last chunk, whose
// store is skipped): with the loads under a condition the compiler kept the
// chunks in scratch memory and waited for each load before the next.
template <int DEPTH, bool F32>
__device__ __forceinline__ void stage_x_rows_n(uint16_t* xs, const void* x, int n8) {
  for (int base = 0; base < n8; base += DEPTH * kThreads) {
    uint4 v[DEPTH];
#pragma unroll
    for (int t = 0; t < DEPTH; ++t) {
      const int i = min(base + (int)threadIdx.x + t * kThreads, n8 - 1);
      {
        const long e = 8L * i;
        if (!F32) {
          v[t] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + e);
        } else {
          const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + e);
          const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + e + 4);
          v[t] = make_uint4(f32_to_f16_bits(a.x) | ((uint32_t)f32_to_f16_bits(a.y) << 16),
                            f32_to_f16_bits(a.z) | ((uint32_t)f32_to_f16_bits(a.w) << 16),
                            f32_to_f16_bits(b.x) | ((uint32_t)f32_to_f16_bits(b.y) << 16),
                            f32_to_f16_bits(b.z) | ((uint32_t)f32_to_f16_bits(b.w) << 16));
        }
      }
    }
#pragma unroll
    for (int t = 0; t < DEPTH; ++t) {
      const int i = base + threadIdx.x + t * kThreads;
      if (i < n8) *reinterpret_cast<uint4*>(xs + 8L * i) = v[t];
    }
  }
}

__device__ __forceinline__ void stage_x_rows(uint16_t* xs, const void* x, int x_dtype, int in,
                                             int rows_m) {
  const int n8 = rows_m * in / 8;
  if (x_dtype == kF16)
    stage_x_rows_n<8, false>(xs, x, n8);
  else
    stage_x_rows_n<8, true>(xs, x, n8);
}

// Sign table: entry n (4 weight bits) = fp16 sign bits of 4 halves, 0x8000
// where bit j of n is 0 (threads 0..31 write it).
__device__ __forceinline__ void init_sign_lut(uint32_t* lut) {
  if (threadIdx.x < 32) {
    const int n = threadIdx.x >> 1, h = threadIdx.x & 1;
    const uint32_t nb = ~(uint32_t)n >> (2 * h);
    lut[threadIdx.x] = ((nb & 1u) << 15) | ((nb & 2u) << 30);
  }
}

// The packed product of one 32-row weight tile with rows_m (<= 32) rows of x:
// sign bits expanded to +-1 fp16 through the sign table are the A operand of
// v_mfma_f32_32x32x16_f16 and x^T (rows of x as columns; columns >= rows_m
// zero) the B operand, so one instruction covers 32 weight rows x 16 inputs
// for every row of x at once. The four waves split the inputs into four
// ranges of whole 4-word (128-input) groups, the unit of one 16-byte sign
// load (short dependent chains, four times the loads in flight; with fewer
// than four groups some waves own none), and their partial tiles are summed
// in LDS in wave order, so results are deterministic.
//
// begin() issues the first sign loads and those of the row scales and biases
// the thread's outputs use (call it before staging x, so they are in flight
// meanwhile); finish() runs after x is staged and the block has synchronised,
// and calls epi(m, o, y) once for each row m < rows_m and weight row o < out
// of the tile, y = bias[o] + scale[o] * sum (bias null: 0).
struct PackedTile {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const uint32_t* br;
  long row;
  int out, wbeg, wend;
  uint4 bw[4];
  float sc[4], bi[4];  // of the thread's output entries t + 256 k

  __device__ __forceinline__ void load(int w0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int w = w0 + 4 * u;
      bw[u] = (row < out && w < wend) ? *reinterpret_cast<const uint4*>(br + w)
                                      : make_uint4(0, 0, 0, 0);
    }
  }

  __device__ __forceinline__ void begin(const uint32_t* bits, int in, int out_rows, long tile,
                                        const uint16_t* scale, const uint16_t* bias) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int groups = in >> 7;  // in % 128 == 0
    wbeg = 4 * (wave * groups / 4);
    wend = 4 * ((wave + 1) * groups / 4);
    out = out_rows;
    row = tile * 32 + (lane & 31);
    br = bits + (row < out ? row : 0) * (long)(in >> 5);
    load(wbeg);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = threadIdx.x + k * kThreads;
      const long o = tile * 32 + mfma32_row(e >> 6, e & 63);
      sc[k] = o < out ? f16_bits_to_f32(scale[o]) : 0.0f;
      bi[k] = o < out && bias ? f16_bits_to_f32(bias[o]) : 0.0f;
    }
  }

  template <class Epi>
  __device__ __forceinline__ void finish(const uint32_t* lut, const uint16_t* xs, int in,
                                         int rows_m, long tile, float* red, Epi&& epi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = lane & 31;         // B column: the row of x this lane feeds
    const bool mok = m < rows_m;
    const int kh = 8 * (lane >> 5);  // this lane's 8 inputs within a 16-input step
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for (int w0 = wbeg; w0 < wend; w0 += 16) {
      if (w0 != wbeg) load(w0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (w0 + 4 * u >= wend) break;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t word = q == 0 ? bw[u].x : q == 1 ? bw[u].y : q == 2 ? bw[u].z : bw[u].w;
          const int kw = 32 * (w0 + 4 * u + q);
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int sh = 16 * hf + kh;
            const u32x2 lo = *reinterpret_cast<const u32x2*>(lut + 2 * ((word >> sh) & 15u));
            const u32x2 hi =
                *reinterpret_cast<const u32x2*>(lut + 2 * ((word >> (sh + 4)) & 15u));
            u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
            a |= 0x3C003C00u;
            u32x4 b = {0u, 0u, 0u, 0u};
            if (mok) b = *reinterpret_cast<const u32x4*>(xs + (long)m * in + kw + 16 * hf + kh);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                         __builtin_bit_cast(half8, b), acc, 0, 0,
                                                         0);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
    // thread t sums entries (r, l) = t, t + 256, t + 512, t + 768 of the tile
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = threadIdx.x + k * kThreads;
      const int r = e >> 6, l = e & 63;
      if ((l & 31) >= rows_m) continue;
      const float v = red[e] + red[1024 + e] + red[2048 + e] + red[3072 + e];
      const long o = tile * 32 + mfma32_row(r, l);
      if (o < out) epi(l & 31, o, bi[k] + sc[k] * v);
    }
  }
};

}  // namespace gemv
}  // namespace ullis
