// Forward products at a few rows (T = 1 decode, batch <= 8): the weights
// stream from HBM once and the activations stay in LDS, where the streamed
// MFMA GEMMs would spend their time loading 64-row activation tiles that are
// almost all padding.
//
// packed: y[m][o] = bias[o] + scale[o] * sum_i sign[o][i] x[m][i] on MFMA,
//   weight rows as the A operand and the rows of x as the columns of B.
// fp16:   y[m][o] = sum_i W[o][i] x[m][i] with v_dot2_f32_f16 on 16-byte
//   weight loads.
// x is rounded to fp16 (the GEMM operand precision) and sums are fp32 in a
// fixed order, so results are deterministic.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "ops.hpp"

namespace ullis {

bool gemv_ok(long rows, long in, long out);

namespace {

constexpr int kGemvThreads = 256;
constexpr long kGemvLds = 64 * 1024;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

struct GemvOut {
  float* y32;
  const float* resid;
  uint16_t* y16;
  uint16_t* relu2_16;
};

__device__ __forceinline__ void gemv_store(const GemvOut& o, long idx, float y) {
  if (o.y32) o.y32[idx] = o.resid ? o.resid[idx] + y : y;
  if (o.y16) o.y16[idx] = __builtin_bit_cast(uint16_t, (_Float16)y);
  if (o.relu2_16) {
    const float k = y > 0.0f ? y : 0.0f;
    o.relu2_16[idx] = __builtin_bit_cast(uint16_t, (_Float16)(k * k));
  }
}

// x rows 0 .. rows_m -> LDS fp16 [rows_m][in] with 16-byte loads (in % 8 ==
// 0; x 16-byte aligned), a thread's loads issued before its stores.
__device__ __forceinline__ void stage_x_rows(uint16_t* xs, const void* x, int x_dtype, int in,
                                             int rows_m) {
  const int n8 = rows_m * in / 8;
  for (int base = 0; base < n8; base += 8 * kGemvThreads) {
    uint4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int i = base + threadIdx.x + t * kGemvThreads;
      if (i < n8) {
        const long e = 8L * i;
        if (x_dtype == kF16) {
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
    for (int t = 0; t < 8; ++t) {
      const int i = base + threadIdx.x + t * kGemvThreads;
      if (i < n8) *reinterpret_cast<uint4*>(xs + 8L * i) = v[t];
    }
  }
}

// Packed product on MFMA: a block owns a 32-row tile of the weight matrix,
// the A operand of v_mfma_f32_32x32x16_f16 (sign bits expanded to +-1 fp16
// through a 16-entry table in LDS, as the streamed GEMM does), and x^T is the
// B operand (rows m of x as columns; columns >= M are zero), so one
// instruction covers 32 weight rows x 16 inputs for every row of x at once.
// The four waves split the inputs into four ranges of whole 4-word
// (128-input) groups, the unit of one 16-byte sign load (short dependent
// chains, four times the loads in flight; with fewer than four groups some
// waves own none), and their partial tiles are summed in LDS in wave order.
// LDS: the sign table (128 B), x [M][in] fp16, 4 partial tiles.
__global__ __launch_bounds__(kGemvThreads) void gemv_bits_kernel(
    const void* x, int x_dtype, int rows_m, int in, int out, const uint32_t* bits,
    const uint16_t* scale, const uint16_t* bias, GemvOut o) {
  extern __shared__ uint32_t gsm[];
  uint32_t* lut = gsm;
  uint16_t* xs = reinterpret_cast<uint16_t*>(gsm + 32);
  float* red = reinterpret_cast<float*>(gsm + 32 + rows_m * in / 2);  // [4][16][64]
  if (threadIdx.x < 32) {
    // entry n (4 weight bits) = fp16 sign bits of 4 halves: 0x8000 where bit j of n is 0
    const int n = threadIdx.x >> 1, h = threadIdx.x & 1;
    const uint32_t nb = ~(uint32_t)n >> (2 * h);
    lut[threadIdx.x] = ((nb & 1u) << 15) | ((nb & 2u) << 30);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int groups = in >> 7;  // in % 128 == 0
  const int wbeg = 4 * (wave * groups / 4), wend = 4 * ((wave + 1) * groups / 4);
  const int m = lane & 31;         // B column: the row of x this lane feeds
  const bool mok = m < rows_m;
  const int kh = 8 * (lane >> 5);  // this lane's 8 inputs within a 16-input step
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const long tile = blockIdx.x;
  const long row = tile * 32 + (lane & 31);
  const uint32_t* br = bits + (row < out ? row : 0) * (long)(in >> 5);
  uint4 bw[4];
  auto load_words = [&](int w0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int w = w0 + 4 * u;
      bw[u] = (row < out && w < wend) ? *reinterpret_cast<const uint4*>(br + w)
                                      : make_uint4(0, 0, 0, 0);
    }
  };
  // the first sign words are on their way while x is staged
  load_words(wbeg);
  stage_x_rows(xs, x, x_dtype, in, rows_m);
  __syncthreads();
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  for (int w0 = wbeg; w0 < wend; w0 += 16) {
    if (w0 != wbeg) load_words(w0);
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
          const u32x2 hi = *reinterpret_cast<const u32x2*>(lut + 2 * ((word >> (sh + 4)) & 15u));
          u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          a |= 0x3C003C00u;
          u32x4 b = {0u, 0u, 0u, 0u};
          if (mok) b = *reinterpret_cast<const u32x4*>(xs + (long)m * in + kw + 16 * hf + kh);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                       __builtin_bit_cast(half8, b), acc, 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
  __syncthreads();
  // thread t sums entries (r, l) = t, t + 256, t + 512, t + 768 of the tile
#pragma unroll
  for (int e = threadIdx.x; e < 16 * 64; e += kGemvThreads) {
    const int r = e >> 6, l = e & 63;
    if ((l & 31) >= rows_m) continue;
    const float v = red[e] + red[1024 + e] + red[2048 + e] + red[3072 + e];
    const long orow = tile * 32 + mfma32_row(r, l);
    if (orow < out) {
      const float sc = f16_bits_to_f32(scale[orow]);
      const float bi = bias ? f16_bits_to_f32(bias[orow]) : 0.0f;
      gemv_store(o, (long)(l & 31) * out + orow, bi + sc * v);
    }
  }
}

// y = x . W^T for M rows; LDS: x [M][in] fp16. One wave per output row,
// lanes over 8-column chunks: up to eight 16-byte weight loads per lane are
// issued before they are used.
template <int M>
__global__ __launch_bounds__(kGemvThreads) void gemv_f16_kernel(const void* x, int x_dtype,
                                                                int in, int out,
                                                                const uint16_t* w, GemvOut o) {
  extern __shared__ uint16_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long row0 = (long)blockIdx.x * 4 + wave;
  uint4 wv[8];
  auto load_w = [&](long row, int k0) {
    const uint16_t* wr = w + row * in;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u * 512;
      wv[u] = (row < out && k < in) ? *reinterpret_cast<const uint4*>(wr + k)
                                    : make_uint4(0, 0, 0, 0);
    }
  };
  // the first weights are on their way while x is staged
  load_w(row0, lane * 8);
  stage_x_rows(xs, x, x_dtype, in, M);
  __syncthreads();
  for (long row = row0; row < out; row += (long)gridDim.x * 4) {
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    for (int k0 = lane * 8; k0 < in; k0 += 64 * 8 * 8) {
      if (row != row0 || k0 != lane * 8) load_w(row, k0);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u * 512;
        if (k < in) {
          const half2v* wh = reinterpret_cast<const half2v*>(&wv[u]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xs + m * in + k);
            const half2v* xh = reinterpret_cast<const half2v*>(&xv);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[m] = __builtin_amdgcn_fdot2(wh[q], xh[q], acc[m], false);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = wave_sum(acc[m], 64);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m) gemv_store(o, (long)m * out + row, acc[m]);
    }
  }
}

template <class F>
hipError_t with_m(int m, F&& f) {
  switch (m) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 5: return f(std::integral_constant<int, 5>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 7: return f(std::integral_constant<int, 7>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return hipErrorInvalidValue;
  }
}

unsigned gemv_grid(long units, long cap) {
  long g = cdiv(units, 4);
  if (g > cap) g = cap;
  return (unsigned)(g > 0 ? g : 1);
}

}  // namespace

bool gemv_ok(long rows, long in, long out) {
  return rows >= 1 && rows <= kGemvMaxRows && in >= 32 && in <= INT32_MAX && out >= 1 &&
         out <= INT32_MAX;
}

bool x_aligned(const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15u) == 0; }

// LDS bytes of the packed kernel: sign table, x rows, four partial tiles
long packed_gemv_lds(long rows, long in) { return 128 + 2 * rows * in + 4 * 16 * 64 * 4; }

bool packed_gemv_ok(long rows, long in, long out, const void* x, int x_dtype,
                    const PackedFwdOut& o) {
  return gemv_ok(rows, in, out) && in % 128 == 0 && packed_gemv_lds(rows, in) <= kGemvLds &&
         !o.sign_bits && (!o.resid || o.y32) && (x_dtype == kF16 || x_dtype == kF32) &&
         x != nullptr && x_aligned(x);
}

hipError_t packed_gemv(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                       const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                       const PackedFwdOut& o) {
  if (!packed_gemv_ok(rows, in, out, x, x_dtype, o) ||
      (reinterpret_cast<uintptr_t>(bits) & 15u) != 0)
    return hipErrorInvalidValue;
  const GemvOut go{o.y32, o.resid, o.y16, o.relu2_16};
  if (cdiv(out, 32) > INT32_MAX) return hipErrorInvalidValue;
  launch(gemv_bits_kernel, dim3((unsigned)cdiv(out, 32)), dim3(kGemvThreads),
         (uint32_t)packed_gemv_lds(rows, in), s, x, x_dtype, (int)rows, (int)in, (int)out, bits,
         scale, bias, go);
  return hipGetLastError();
}

bool fp16_gemv_ok(long rows, long in, long out, const void* x, int x_dtype, const uint16_t* w) {
  return gemv_ok(rows, in, out) && in % 8 == 0 && 2L * rows * in <= kGemvLds &&
         (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
         (x_dtype == kF16 || x_dtype == kF32) && x != nullptr && x_aligned(x);
}

hipError_t fp16_gemv(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                     const uint16_t* w, float* y32, const float* resid, uint16_t* y16) {
  if (!fp16_gemv_ok(rows, in, out, x, x_dtype, w) || (resid && !y32))
    return hipErrorInvalidValue;
  const GemvOut go{y32, resid, y16, nullptr};
  return with_m((int)rows, [&](auto mt) -> hipError_t {
    constexpr int M = decltype(mt)::value;
    launch(gemv_f16_kernel<M>, dim3(gemv_grid(out, 1024)), dim3(kGemvThreads),
           (uint32_t)(2 * M * in), s, x, x_dtype, (int)in, (int)out, w, go);
    return hipGetLastError();
  });
}

}  // namespace ullis
