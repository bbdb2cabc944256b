// Embedding gather and scatter-SGD on the device (the two host loops of
// UllisHeron::train_step_on, src/model.rs:2866-2873 and 2986-2993) and their
// C ABI entry points.
#include <hip/hip_runtime.h>

#include <climits>
#include <string>

#include "../../include/ullis_hip.h"
#include "common.hpp"
#include "context.hpp"
#include "ops.hpp"

namespace ullis {
namespace {

// x[r][c] = f16 table[tokens[r]][c] as f32; a token >= vocab gives a zero row
// and one count in *invalid. Grid (rows, channel chunks of 1024); vec: d % 4
// == 0 with 8-byte aligned table and 16-byte aligned x (4 channels per load).
__global__ __launch_bounds__(256) void embedding_gather_kernel(const uint16_t* table, int d,
                                                               const uint32_t* tokens,
                                                               uint32_t vocab, float* x,
                                                               uint32_t* invalid, bool vec) {
  const long r = blockIdx.x;
  const uint32_t id = tokens[r];
  const bool ok = id < vocab;
  if (!ok && invalid && blockIdx.y == 0 && threadIdx.x == 0) atomicAdd(invalid, 1u);
  const long src = ok ? (long)id * d : 0;
  float* dst = x + r * d;
  const int c4 = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (vec) {
    if (c4 < d) {
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (ok) {
        const uint2 w = *reinterpret_cast<const uint2*>(table + src + c4);
        v = make_float4(f16_bits_to_f32((uint16_t)(w.x & 0xffffu)), f16_bits_to_f32((uint16_t)(w.x >> 16)),
                        f16_bits_to_f32((uint16_t)(w.y & 0xffffu)), f16_bits_to_f32((uint16_t)(w.y >> 16)));
      }
      *reinterpret_cast<float4*>(dst + c4) = v;
    }
  } else {
    for (int c = c4; c < c4 + 4 && c < d; ++c) dst[c] = ok ? f16_bits_to_f32(table[src + c]) : 0.0f;
  }
}

// Token reads a thread keeps in flight in the scans below.
constexpr int kScanBatch = 16;
// Rows of one pass of the walk: their matches are marked in an LDS bitmap
// (kScatterWindow bits) with one summary bit per non-empty bitmap word.
constexpr int kScatterWindow = 16384;
constexpr int kScatterWords = kScatterWindow / 64;
// Channels a thread carries through the walk in registers (256 threads:
// widths up to 2048 in one walk, wider tables walk once per 2048 channels).
constexpr int kScatterChannels = 8;

// Clipped SGD of table[tokens[r]] with g[r] for every row r, in row order for
// rows that share a token, as the reference's sequential loop applies them.
// Block r does the work only if r is the first row holding its token: the
// block checks rows [0, r) for its token (kScanBatch reads in flight per
// thread), then marks the rows [r, rows) holding it in an LDS bitmap and
// applies their gradients in row order, each channel's value and carry kept
// in registers between applications (the same arithmetic as storing and
// reloading them).
__global__ __launch_bounds__(256) void embedding_scatter_sgd_kernel(uint16_t* table,
                                                                    float* residual, int d,
                                                                    const uint32_t* tokens,
                                                                    int rows, uint32_t vocab,
                                                                    const float* g, float lr,
                                                                    const uint32_t* abort) {
  __shared__ unsigned long long s_bits[kScatterWords];
  __shared__ unsigned long long s_sum[kScatterWords / 64];
  const int r = blockIdx.x;
  const int t = threadIdx.x;
  if (abort && *abort) return;  // refused step
  const uint32_t id = tokens[r];
  if (id >= vocab) return;
  bool earlier = false;
  for (int base = 0; base < r; base += 256 * kScanBatch) {
    uint32_t tk[kScanBatch];
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) {
      const int j = base + u * 256 + t;
      tk[u] = tokens[j < r ? j : r - 1];  // past r - 1: row r - 1 again, also an earlier row
    }
#pragma unroll
    for (int u = 0; u < kScanBatch; ++u) earlier = earlier || tk[u] == id;
  }
  if (__syncthreads_or(earlier)) return;  // an earlier row owns this token
  for (int cg = 0; cg < d; cg += 256 * kScatterChannels) {
    uint16_t v[kScatterChannels];
    float res[kScatterChannels];
    const long row0 = (long)id * d;
#pragma unroll
    for (int k = 0; k < kScatterChannels; ++k) {
      const int c = cg + k * 256 + t;
      v[k] = 0;
      res[k] = 0.0f;
      if (c < d) {
        v[k] = table[row0 + c];
        res[k] = residual[row0 + c];
      }
    }
    for (int w0 = r; w0 < rows; w0 += kScatterWindow) {
      const int wn = rows - w0 < kScatterWindow ? rows - w0 : kScatterWindow;
      for (int q = t; q < kScatterWords; q += 256) s_bits[q] = 0ull;
      if (t < kScatterWords / 64) s_sum[t] = 0ull;
      __syncthreads();
      for (int base = 0; base < wn; base += 256 * kScanBatch) {
        uint32_t tk[kScanBatch];
#pragma unroll
        for (int u = 0; u < kScanBatch; ++u) {
          const int j = base + u * 256 + t;
          tk[u] = tokens[w0 + (j < wn ? j : wn - 1)];
        }
#pragma unroll
        for (int u = 0; u < kScanBatch; ++u) {
          const int j = base + u * 256 + t;
          if (j < wn && tk[u] == id) {
            atomicOr(&s_bits[j >> 6], 1ull << (j & 63));
            atomicOr(&s_sum[j >> 12], 1ull << ((j >> 6) & 63));
          }
        }
      }
      __syncthreads();
      for (int sw = 0; sw < kScatterWords / 64; ++sw) {
        unsigned long long sm = s_sum[sw];
        while (sm) {
          const int q = sw * 64 + __builtin_ctzll(sm);
          sm &= sm - 1;
          unsigned long long m = s_bits[q];
          while (m) {
            const long j = w0 + q * 64 + __builtin_ctzll(m);
            m &= m - 1;
#pragma unroll
            for (int k = 0; k < kScatterChannels; ++k) {
              const int c = cg + k * 256 + t;
              if (c < d) clipped_sgd_one(v[k], res[k], g[j * d + c], lr);
            }
          }
        }
      }
      __syncthreads();  // every thread has read the bitmap before the next window clears it
    }
#pragma unroll
    for (int k = 0; k < kScatterChannels; ++k) {
      const int c = cg + k * 256 + t;
      if (c < d) {
        table[row0 + c] = v[k];
        residual[row0 + c] = res[k];
      }
    }
  }
}

}  // namespace

hipError_t embedding_gather(hipStream_t s, const uint16_t* table, long vocab, long d,
                            const uint32_t* tokens, long rows, float* x, uint32_t* invalid) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  if (rows > INT32_MAX || cdiv(d, 1024) > 65535 || vocab > (long)UINT32_MAX)
    return hipErrorInvalidValue;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(table) & 7u) == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  launch(embedding_gather_kernel, dim3((unsigned)rows, (unsigned)cdiv(d, 1024)), dim3(256), 0, s,
         table, (int)d, tokens, (uint32_t)vocab, x, invalid, vec);
  return hipGetLastError();
}

hipError_t embedding_scatter_sgd(hipStream_t s, uint16_t* table, float* residual, long vocab,
                                 long d, const uint32_t* tokens, long rows, const float* g,
                                 float lr, const uint32_t* abort) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  if (rows > INT32_MAX || vocab > (long)UINT32_MAX) return hipErrorInvalidValue;
  launch(embedding_scatter_sgd_kernel, dim3((unsigned)rows), dim3(256), 0, s, table, residual,
         (int)d, tokens, (int)rows, (uint32_t)vocab, g, lr, abort);
  return hipGetLastError();
}

}  // namespace ullis

using namespace ullis;

extern "C" {

int ullis_hip_embedding_gather(ullis_hip_ctx* c, const uint16_t* table, size_t vocab, size_t d,
                               const uint32_t* tokens, size_t rows, float* x, uint32_t* invalid) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (vocab == 0 || d == 0 || rows == 0 || vocab > (size_t)UINT32_MAX || d > (size_t)INT32_MAX ||
      rows > (size_t)INT32_MAX || vocab > (size_t)LONG_MAX / d || rows > (size_t)LONG_MAX / d)
    return c->fail(ULLIS_HIP_ERR_INVALID, "embedding shape must be non-zero and fit");
  if (!table || !tokens || !x) return c->fail(ULLIS_HIP_ERR_INVALID, "embedding gather: NULL pointer");
  if (int rc = c->hip(embedding_gather(c->stream, table, (long)vocab, (long)d, tokens, (long)rows,
                                       x, invalid),
                      "embedding gather"))
    return rc;
  return 0;
}

int ullis_hip_embedding_scatter_sgd(ullis_hip_ctx* c, uint16_t* table, float* residual,
                                    size_t vocab, size_t d, const uint32_t* tokens, size_t rows,
                                    const float* g, float learning_rate) {
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (vocab == 0 || d == 0 || rows == 0 || vocab > (size_t)UINT32_MAX || d > (size_t)INT32_MAX ||
      rows > (size_t)INT32_MAX || vocab > (size_t)LONG_MAX / d || rows > (size_t)LONG_MAX / d)
    return c->fail(ULLIS_HIP_ERR_INVALID, "embedding shape must be non-zero and fit");
  if (!table || !residual || !tokens || !g)
    return c->fail(ULLIS_HIP_ERR_INVALID, "embedding scatter: NULL pointer");
  if (!__builtin_isfinite(learning_rate))
    return c->fail(ULLIS_HIP_ERR_INVALID, "learning rate must be finite");
  if (int rc = c->hip(embedding_scatter_sgd(c->stream, table, residual, (long)vocab, (long)d, tokens,
                                            (long)rows, g, learning_rate),
                      "embedding scatter sgd"))
    return rc;
  return 0;
}

}  // extern "C"
