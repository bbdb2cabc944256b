// Kernels of the T = 1 decode step (UllisHeron::generate_step,
// src/model.rs:2717-2753) for up to 8 sequences.
//
// Fused path (decode_fused_ok): three launches per layer. Each product
// kernel stages its own input rows in LDS, so LayerNorm, the time-shift
// mixes and ROSA's output expansion never make a round trip through HBM:
//   decode_qkvo LN3 + the Q/K/V mixes (time_shift_one against the previous
//               token's LayerNorm output, src/model.rs:214-228, 1320-1353),
//               the three packed products and their sign bits (the planes
//               the suffix automaton takes) written straight from the tile;
//               and, in the same launch when the automaton's indices are
//               given, y = (2 idx - 1) e and the O product into x2 = x + O(y)
//               (a live automaton splits the launch in two around its call);
//   decode_key  LN2 + the CMix mix (src/model.rs:1003-1016), the packed key
//               product and ReLU^2;
//   value       the fp16 few-row product (gemv.hip): x = x2 + value(r2).
// Every block of a product recomputes the LayerNorm of the (<= 8) rows it
// needs, with all its loads issued at once, which costs no launch and no
// barrier. The previous token's LayerNorm outputs are double-buffered
// (prev_in read, prev_out written by one block), since other blocks of the
// same launch still read prev_in. decode_embed gathers the embedding rows and
// applies LN0; decode_head applies the final LayerNorm in the head product's
// staging; argmax_rows picks the greedy next tokens.
//
// General path (any shape): decode_mix beside the standalone products.
#include <type_traits>

#include "common.hpp"
#include "gemv_impl.hpp"
#include "ops.hpp"

namespace ullis {

namespace {

using gemv::kThreads;

// LDS bytes of a fused product kernel: sign table, x rows [rows][d] fp16,
// the four partial tiles, and one fp32 tile row per sequence.
long fused_lds(long rows, long d) {
  return 4L * gemv::kLutWords + 2 * rows * d + 4L * gemv::kRedFloats + 4L * 8 * 32;
}

struct FusedLds {
  uint32_t* lut;
  uint16_t* xs;
  float* red;
  float* ys;  // [8][32]
};

__device__ __forceinline__ FusedLds fused_lds_layout(uint32_t* smem, int rows, int d) {
  FusedLds l;
  l.lut = smem;
  l.xs = reinterpret_cast<uint16_t*>(smem + gemv::kLutWords);
  l.red = reinterpret_cast<float*>(smem + gemv::kLutWords + rows * d / 2);
  l.ys = l.red + gemv::kRedFloats;
  return l;
}

// 4 consecutive fp16 values (8-byte aligned) as floats.
__device__ __forceinline__ floatx4 load_h4(const uint16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return {f16_bits_to_f32((uint16_t)(u.x & 0xffffu)), f16_bits_to_f32((uint16_t)(u.x >> 16)),
          f16_bits_to_f32((uint16_t)(u.y & 0xffffu)), f16_bits_to_f32((uint16_t)(u.y >> 16))};
}

__device__ __forceinline__ void store_h4(uint16_t* p, uint16_t a, uint16_t b, uint16_t c,
                                         uint16_t e) {
  *reinterpret_cast<uint2*>(p) = make_uint2(a | ((uint32_t)b << 16), c | ((uint32_t)e << 16));
}

// The rows of x [rows][d] (rows <= 8, d <= 256 NV, d % 4 == 0) that wave w
// normalises: rows w and w + 4. Lane l holds the float4 chunks at channel
// 4 l + 256 j of both rows; every load of x, gamma and beta is issued before
// the first reduction, so a block pays one memory round trip for its
// LayerNorm (src/model.rs:259-283: population variance, eps 1e-5).
template <int NV>
struct WaveRows {
  floatx4 v[2][NV];

  __device__ __forceinline__ static int row(int r) { return (threadIdx.x >> 6) + 4 * r; }
  __device__ __forceinline__ static int chan(int j) { return 4 * (threadIdx.x & 63) + 256 * j; }

  __device__ __forceinline__ void load(const float* x, int rows, int d) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const bool ok = row(r) < rows && chan(j) < d;
        v[r][j] = ok ? *reinterpret_cast<const floatx4*>(x + (long)row(r) * d + chan(j))
                     : (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
      }
  }

  // v = LayerNorm(v) for the rows < rows.
  __device__ __forceinline__ void normalise(int rows, int d, const uint16_t* w,
                                            const uint16_t* b) {
    floatx4 gw[NV], gb[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const bool ok = chan(j) < d;
      gw[j] = ok ? load_h4(w + chan(j)) : (floatx4){};
      gb[j] = ok ? load_h4(b + chan(j)) : (floatx4){};
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      if (row(r) >= rows) continue;  // uniform over the wave
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < NV; ++j) s += (v[r][j][0] + v[r][j][1]) + (v[r][j][2] + v[r][j][3]);
      const float mean = wave_sum(s) / (float)d;
      float q = 0.0f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (chan(j) < d) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float dv = v[r][j][e] - mean;
            q += dv * dv;
          }
        }
      const float var = wave_sum(q) / (float)d;
      const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[r][j][e] = (v[r][j][e] - mean) * inv * gw[j][e] + gb[j][e];
    }
  }
};

// Time-shift mix of one LayerNorm output y against the previous token's p:
// f16(y + (p - y) * mix) (p = 0 before the first token gives -y, as
// time_shift_one without a previous state).
__device__ __forceinline__ uint16_t mix_f16(float y, float p, float mix) {
  return f32_to_f16_bits(y + (p - y) * mix);
}

// LN(x) mixed against prev_in into xs (fp16 [rows][d]); prev_out = LN(x) when set.
template <int NV>
__device__ __forceinline__ void stage_ln_mix(uint16_t* xs, const float* x, int rows, int d,
                                             const uint16_t* ln_w, const uint16_t* ln_b,
                                             const float* prev_in, float* prev_out,
                                             const uint16_t* mix) {
  WaveRows<NV> wr, pv;
  floatx4 mx[NV];
  wr.load(x, rows, d);
  pv.load(prev_in, rows, d);
#pragma unroll
  for (int j = 0; j < NV; ++j)
    mx[j] = WaveRows<NV>::chan(j) < d ? load_h4(mix + WaveRows<NV>::chan(j)) : (floatx4){};
  wr.normalise(rows, d, ln_w, ln_b);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int m = WaveRows<NV>::row(r);
    if (m >= rows) continue;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = WaveRows<NV>::chan(j);
      if (c >= d) continue;
      const long i = (long)m * d + c;
      const floatx4 y = wr.v[r][j], pp = pv.v[r][j];
      store_h4(xs + i, mix_f16(y[0], pp[0], mx[j][0]), mix_f16(y[1], pp[1], mx[j][1]),
               mix_f16(y[2], pp[2], mx[j][2]), mix_f16(y[3], pp[3], mx[j][3]));
      if (prev_out) *reinterpret_cast<floatx4*>(prev_out + i) = y;
    }
  }
}

// One block: the embedding rows of tokens [rows] (ids >= vocab give zero rows;
// *invalid = their count), LN0 applied when ln0_w is set.
template <int NV>
__global__ __launch_bounds__(kThreads) void decode_embed_kernel(
    const uint16_t* __restrict__ table, long vocab, int d, const uint32_t* __restrict__ tokens,
    int rows, float* __restrict__ x, uint32_t* __restrict__ invalid,
    const uint16_t* __restrict__ ln0_w, const uint16_t* __restrict__ ln0_b) {
  WaveRows<NV> wr;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int m = WaveRows<NV>::row(r);
    const uint32_t tok = m < rows ? tokens[m] : 0u;
    const bool ok = m < rows && tok < (uint64_t)vocab;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = WaveRows<NV>::chan(j);
      wr.v[r][j] = ok && c < d ? load_h4(table + (long)tok * d + c) : (floatx4){};
    }
  }
  if (ln0_w) wr.normalise(rows, d, ln0_w, ln0_b);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int m = WaveRows<NV>::row(r);
    if (m >= rows) continue;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = WaveRows<NV>::chan(j);
      if (c < d) *reinterpret_cast<floatx4*>(x + (long)m * d + c) = wr.v[r][j];
    }
  }
  if (invalid && threadIdx.x == 0) {
    uint32_t n = 0;
    for (int m = 0; m < rows; ++m) n += tokens[m] >= (uint64_t)vocab ? 1u : 0u;
    *invalid = n;
  }
}

// Blocks [first, first + count) of the roles [0, 4T) (T = d / 32): role
// j T + t (j < 3) is projection j's weight tile t, role 3 T + t the O tile t.
// Q/K/V: sign bits of bias + scale * (mix_j(LN3(x), prev_in) . S_j^T);
// O: x2 = x + bias + scale * (((2 idx - 1) e) . S^T). The O roles write x2,
// not x, since Q/K/V blocks of the same launch may still read x.
template <int NV>
__global__ __launch_bounds__(kThreads) void decode_qkvo_kernel(
    const float* __restrict__ x, float* __restrict__ x2, int rows, int d, int first,
    const uint16_t* __restrict__ ln_w, const uint16_t* __restrict__ ln_b,
    const float* __restrict__ prev_in, float* __restrict__ prev_out, DecodeQkv p, DecodeO po) {
  extern __shared__ uint32_t smem[];
  const FusedLds l = fused_lds_layout(smem, rows, d);
  const int tiles = d >> 5;
  const int role = (int)blockIdx.x + first;
  gemv::init_sign_lut(l.lut);
  gemv::PackedTile pt;
  if (role < 3 * tiles) {
    const int j = role / tiles;
    const long tile = role % tiles;
    pt.begin(p.bits[j], d, d, tile, p.scale[j], p.bias[j]);
    // layer.rosa_x_prev = Some(rosa_in), kept by the first Q tile
    stage_ln_mix<NV>(l.xs, x, rows, d, ln_w, ln_b, prev_in, role == 0 ? prev_out : nullptr,
                     p.mix[j]);
    __syncthreads();
    pt.finish(l.lut, l.xs, d, rows, tile, l.red,
              [&](int m, long o, float y) { l.ys[m * 32 + (int)(o - tile * 32)] = y; });
    __syncthreads();
    // bit b d + c of the plane = (output c of row b) > 0 (src/rosa.rs:372); the
    // tile's 32 outputs of row m are one word, rows m and m + 1 one ballot
    const int t = threadIdx.x, m = t >> 5;
    const bool bit = m < rows && l.ys[t] > 0.0f;
    const unsigned long long bal = __ballot(bit);
    if ((t & 31) == 0 && m < rows)
      p.planes[j][(long)m * tiles + tile] = (uint32_t)(bal >> (32 * ((t >> 5) & 1)));
  } else {
    const long tile = role - 3 * tiles;
    pt.begin(po.bits, d, d, tile, po.scale, po.bias);
    // y = (2 idx - 1) e, four channels per thread
    const int n4 = rows * d / 4;
    for (int i4 = threadIdx.x; i4 < n4; i4 += kThreads) {
      const uint32_t id = *reinterpret_cast<const uint32_t*>(po.idx + 4L * i4);
      const floatx4 e = load_h4(po.e + (4 * i4) % d);
      uint16_t h[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        h[k] = f32_to_f16_bits((2.0f * (float)((id >> (8 * k)) & 0xffu) - 1.0f) * e[k]);
      store_h4(l.xs + 4L * i4, h[0], h[1], h[2], h[3]);
    }
    __syncthreads();
    pt.finish(l.lut, l.xs, d, rows, tile, l.red, [&](int m, long o, float y) {
      const long i = (long)m * d + o;
      x2[i] = x[i] + y;
    });
  }
}

// Blocks [F / 32): key tile; r2 = f16(max(k, 0)^2), k = scale * (mix(LN2(x)) . S^T).
template <int NV>
__global__ __launch_bounds__(kThreads) void decode_key_kernel(
    const float* __restrict__ x, int rows, int d, int f, const uint16_t* __restrict__ ln_w,
    const uint16_t* __restrict__ ln_b, const float* __restrict__ prev_in,
    float* __restrict__ prev_out, const uint16_t* __restrict__ mix,
    const uint32_t* __restrict__ bits, const uint16_t* __restrict__ scale,
    uint16_t* __restrict__ r2) {
  extern __shared__ uint32_t smem[];
  const FusedLds l = fused_lds_layout(smem, rows, d);
  const long tile = blockIdx.x;
  gemv::init_sign_lut(l.lut);
  gemv::PackedTile pt;
  pt.begin(bits, d, f, tile, scale, nullptr);
  // layer.cmix_x_prev = Some(ffn_in), kept by the first tile
  stage_ln_mix<NV>(l.xs, x, rows, d, ln_w, ln_b, prev_in, tile == 0 ? prev_out : nullptr, mix);
  __syncthreads();
  pt.finish(l.lut, l.xs, d, rows, tile, l.red, [&](int m, long o, float k) {
    const float kp = k > 0.0f ? k : 0.0f;
    r2[(long)m * f + o] = __builtin_bit_cast(uint16_t, (_Float16)(kp * kp));
  });
}

// Blocks [ceil(V / 32)): head tile; logits = bias + scale * (LN_out(x) . S^T).
template <int NV>
__global__ __launch_bounds__(kThreads) void decode_head_kernel(
    const float* __restrict__ x, int rows, int d, int vocab, const uint16_t* __restrict__ ln_w,
    const uint16_t* __restrict__ ln_b, const uint32_t* __restrict__ bits,
    const uint16_t* __restrict__ scale, const uint16_t* __restrict__ bias,
    float* __restrict__ logits) {
  extern __shared__ uint32_t smem[];
  const FusedLds l = fused_lds_layout(smem, rows, d);
  const long tile = blockIdx.x;
  gemv::init_sign_lut(l.lut);
  gemv::PackedTile pt;
  pt.begin(bits, d, vocab, tile, scale, bias);
  {
    WaveRows<NV> wr;
    wr.load(x, rows, d);
    wr.normalise(rows, d, ln_w, ln_b);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int m = WaveRows<NV>::row(r);
      if (m >= rows) continue;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = WaveRows<NV>::chan(j);
        if (c >= d) continue;
        const floatx4 y = wr.v[r][j];
        store_h4(l.xs + (long)m * d + c, f32_to_f16_bits(y[0]), f32_to_f16_bits(y[1]),
                 f32_to_f16_bits(y[2]), f32_to_f16_bits(y[3]));
      }
    }
  }
  __syncthreads();
  pt.finish(l.lut, l.xs, d, rows, tile, l.red,
            [&](int m, long o, float y) { logits[(long)m * vocab + o] = y; });
}

// General shapes: the embedding rows (one block, any d % 4 == 0).
__global__ __launch_bounds__(kThreads) void decode_embed_any_kernel(
    const uint16_t* __restrict__ table, long vocab, int d, const uint32_t* __restrict__ tokens,
    int rows, float* __restrict__ x, uint32_t* __restrict__ invalid) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int m = wave; m < rows; m += kThreads / 64) {
    const uint32_t tok = tokens[m];
    const bool ok = tok < (uint64_t)vocab;
    for (int c = 4 * lane; c < d; c += 256)
      *reinterpret_cast<floatx4*>(x + (long)m * d + c) =
          ok ? load_h4(table + (long)tok * d + c) : (floatx4){};
  }
  if (invalid && threadIdx.x == 0) {
    uint32_t n = 0;
    for (int m = 0; m < rows; ++m) n += tokens[m] >= (uint64_t)vocab ? 1u : 0u;
    *invalid = n;
  }
}

// Element i of [rows][d]: out_j = f16(x + (prev_in - x) * mix_j[c]) for the
// given mixes, prev_out = x.
__global__ __launch_bounds__(256) void decode_mix_kernel(const float* __restrict__ x,
                                                         const float* prev_in, float* prev_out,
                                                         long n, int d, const uint16_t* mix0,
                                                         uint16_t* out0, const uint16_t* mix1,
                                                         uint16_t* out1, const uint16_t* mix2,
                                                         uint16_t* out2) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int c = (int)(i % d);
  const float xv = x[i];
  const float pv = prev_in[i];
  if (out0) out0[i] = mix_f16(xv, pv, f16_bits_to_f32(mix0[c]));
  if (out1) out1[i] = mix_f16(xv, pv, f16_bits_to_f32(mix1[c]));
  if (out2) out2[i] = mix_f16(xv, pv, f16_bits_to_f32(mix2[c]));
  prev_out[i] = xv;
}

// One block of 1024 threads per row: the index of the row's largest logit
// (the lowest index among equal maxima; NaN logits are never chosen). Each
// thread scans float4 chunks with eight loads in flight, then waves and the
// block reduce (value, index) pairs.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_take(float v, long i, float& best, long& at) {
  if (v > best || (v == best && i < at)) {
    best = v;
    at = i;
  }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits,
                                                                long vocab,
                                                                uint32_t* __restrict__ next) {
  __shared__ float bv[kArgmaxThreads / 64];
  __shared__ long bi[kArgmaxThreads / 64];
  const float* row = logits + (long)blockIdx.x * vocab;
  float best = -__builtin_inff();
  long at = vocab;
  const bool vec = (vocab & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  if (vec) {
    const long n4 = vocab / 4;
    for (long base = 0; base < n4; base += 8L * kArgmaxThreads) {
      floatx4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const long i4 = base + threadIdx.x + (long)u * kArgmaxThreads;
        v[u] = i4 < n4 ? *reinterpret_cast<const floatx4*>(row + 4 * i4)
                       : (floatx4){-__builtin_inff(), -__builtin_inff(), -__builtin_inff(),
                                   -__builtin_inff()};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const long i4 = base + threadIdx.x + (long)u * kArgmaxThreads;
#pragma unroll
        for (int e = 0; e < 4; ++e) argmax_take(v[u][e], 4 * i4 + e, best, at);
      }
    }
  } else {
    for (long v = threadIdx.x; v < vocab; v += kArgmaxThreads) argmax_take(row[v], v, best, at);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const long oi = __shfl_xor(at, off, 64);
    argmax_take(ov, oi, best, at);
  }
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = at;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_take(bv[w], bi[w], best, at);
    next[blockIdx.x] = at < vocab ? (uint32_t)at : 0u;
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// The fused kernels keep two rows of d <= 1024 channels per wave in
// registers: NV = ceil(d / 256) float4 chunks per lane and row.
constexpr long kFusedMaxD = 1024;

template <class F>
hipError_t by_nv(long d, F&& f) {
  const long nv = cdiv(d, 256);
  if (nv <= 1) return f(std::integral_constant<int, 1>{});
  if (nv <= 2) return f(std::integral_constant<int, 2>{});
  if (nv <= 4) return f(std::integral_constant<int, 4>{});
  return hipErrorInvalidValue;
}

bool decode_fused_ok(long rows, long d, long f) {
  return rows >= 1 && rows <= 8 && d % 128 == 0 && d <= kFusedMaxD && f % 32 == 0 &&
         f <= INT32_MAX && fused_lds(rows, d) <= gemv::kLds;
}

hipError_t decode_embed(hipStream_t s, const uint16_t* table, long vocab, long d,
                        const uint32_t* tokens, long rows, float* x, uint32_t* invalid,
                        const uint16_t* ln0_w, const uint16_t* ln0_b) {
  if (rows < 1 || rows > 8 || d % 4 != 0 || d > INT32_MAX || !al16(x) || (ln0_w && !ln0_b))
    return hipErrorInvalidValue;
  if (d > kFusedMaxD) {
    // general shapes: LN0 runs as its own launch
    if (ln0_w) return hipErrorInvalidValue;
    launch(decode_embed_any_kernel, dim3(1), dim3(kThreads), 0, s, table, vocab, (int)d, tokens,
           (int)rows, x, invalid);
    return hipGetLastError();
  }
  return by_nv(d, [&](auto nv) {
    launch(decode_embed_kernel<decltype(nv)::value>, dim3(1), dim3(kThreads), 0, s, table, vocab,
           (int)d, tokens, (int)rows, x, invalid, ln0_w, ln0_b);
    return hipGetLastError();
  });
}

hipError_t decode_qkvo(hipStream_t s, const float* x, float* x2, long rows, long d, int part,
                       const uint16_t* ln_w, const uint16_t* ln_b, const float* prev_in,
                       float* prev_out, const DecodeQkv& p, const DecodeO& po) {
  if (!decode_fused_ok(rows, d, d) || !al16(x) || part < 0 || part > 2) return hipErrorInvalidValue;
  const int tiles = (int)(d / 32);
  if (part != 1) {
    for (int j = 0; j < 3; ++j)
      if (!al16(p.bits[j]) || !p.planes[j] || !p.mix[j] || !p.scale[j] || !p.bias[j] ||
          !prev_in || !prev_out)
        return hipErrorInvalidValue;
  }
  if (part != 0 && (!al16(po.bits) || !po.idx || !po.e || !x2 ||
                    (reinterpret_cast<uintptr_t>(po.idx) & 3u) != 0))
    return hipErrorInvalidValue;
  // part 0: Q/K/V roles, 1: O roles, 2: both
  const int first = part == 1 ? 3 * tiles : 0;
  const int count = part == 0 ? 3 * tiles : part == 1 ? tiles : 4 * tiles;
  return by_nv(d, [&](auto nv) {
    launch(decode_qkvo_kernel<decltype(nv)::value>, dim3((unsigned)count), dim3(kThreads),
           (uint32_t)fused_lds(rows, d), s, x, x2, (int)rows, (int)d, first, ln_w, ln_b, prev_in,
           prev_out, p, po);
    return hipGetLastError();
  });
}

hipError_t decode_key(hipStream_t s, const float* x, long rows, long d, long f,
                      const uint16_t* ln_w, const uint16_t* ln_b, const float* prev_in,
                      float* prev_out, const uint16_t* mix, const uint32_t* bits,
                      const uint16_t* scale, uint16_t* r2) {
  if (!decode_fused_ok(rows, d, f) || !al16(x) || !al16(bits)) return hipErrorInvalidValue;
  return by_nv(d, [&](auto nv) {
    launch(decode_key_kernel<decltype(nv)::value>, dim3((unsigned)(f / 32)), dim3(kThreads),
           (uint32_t)fused_lds(rows, d), s, x, (int)rows, (int)d, (int)f, ln_w, ln_b, prev_in,
           prev_out, mix, bits, scale, r2);
    return hipGetLastError();
  });
}

hipError_t decode_head(hipStream_t s, const float* x, long rows, long d, long vocab,
                       const uint16_t* ln_w, const uint16_t* ln_b, const uint32_t* bits,
                       const uint16_t* scale, const uint16_t* bias, float* logits) {
  if (!decode_fused_ok(rows, d, 32) || vocab < 1 || vocab > INT32_MAX || !al16(x) ||
      !al16(bits))
    return hipErrorInvalidValue;
  return by_nv(d, [&](auto nv) {
    launch(decode_head_kernel<decltype(nv)::value>, dim3((unsigned)cdiv(vocab, 32)),
           dim3(kThreads), (uint32_t)fused_lds(rows, d), s, x, (int)rows, (int)d, (int)vocab, ln_w,
           ln_b, bits, scale, bias, logits);
    return hipGetLastError();
  });
}

hipError_t decode_mix(hipStream_t s, const float* x, const float* prev_in, float* prev_out,
                      long rows, long d, const uint16_t* mix0, uint16_t* out0,
                      const uint16_t* mix1, uint16_t* out1, const uint16_t* mix2,
                      uint16_t* out2) {
  const long n = rows * d;
  if (n <= 0) return hipSuccess;
  if (d > INT32_MAX) return hipErrorInvalidValue;
  launch(decode_mix_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, x, prev_in, prev_out,
         n, (int)d, mix0, out0, mix1, out1, mix2, out2);
  return hipGetLastError();
}

hipError_t argmax_rows(hipStream_t s, const float* logits, long rows, long vocab, uint32_t* next) {
  if (rows <= 0 || vocab <= 0) return hipSuccess;
  if (rows > INT32_MAX) return hipErrorInvalidValue;
  launch(argmax_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, s, logits, vocab, next);
  return hipGetLastError();
}

}  // namespace ullis
