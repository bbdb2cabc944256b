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
#include "gemv_impl.hpp"
#include "ops.hpp"

namespace ullis {

bool gemv_ok(long rows, long in, long out);

namespace {

constexpr int kGemvThreads = gemv::kThreads;
constexpr long kGemvLds = gemv::kLds;
using gemv::stage_x_rows;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v, int width) {
  if (width == 64) return ullis::wave_sum(v);
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

// Packed product on MFMA (gemv::PackedTile): a block owns a 32-row tile of
// the weight matrix. LDS: the sign table (128 B), x [M][in] fp16, 4 partial
// tiles.
__global__ __launch_bounds__(kGemvThreads) void gemv_bits_kernel(
    const void* x, int x_dtype, int rows_m, int in, int out, const uint32_t* bits,
    const uint16_t* scale, const uint16_t* bias, GemvOut o) {
  extern __shared__ uint32_t gsm[];
  uint32_t* lut = gsm;
  uint16_t* xs = reinterpret_cast<uint16_t*>(gsm + gemv::kLutWords);
  float* red = reinterpret_cast<float*>(gsm + gemv::kLutWords + rows_m * in / 2);
  gemv::init_sign_lut(lut);
  const long tile = blockIdx.x;
  gemv::PackedTile pt;
  // the first sign words are on their way while x is staged
  pt.begin(bits, in, out, tile, scale, bias);
  stage_x_rows(xs, x, x_dtype, in, rows_m);
  __syncthreads();
  pt.finish(lut, xs, in, rows_m, tile, red,
            [&](int m, long orow, float y) { gemv_store(o, (long)m * out + orow, y); });
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
