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

// Clipped SGD of table[tokens[r]] with g[r] for every row r, in row order for
// rows that share a token, as the reference's sequential loop applies them.
// Block r does the work only if r is the first row holding its token; it then
// walks the later rows with the same token (64 at a time by wave ballot),
// keeping each channel's value and carry in registers between applications,
// which is the same arithmetic as storing and reloading them.
__global__ __launch_bounds__(256) void embedding_scatter_sgd_kernel(uint16_t* table,
                                                                    float* residual, int d,
                                                                    const uint32_t* tokens,
                                                                    int rows, uint32_t vocab,
                                                                    const float* g, float lr,
                                                                    const uint32_t* abort) {
  const int r = blockIdx.x;
  if (abort && *abort) return;  // refused step
  const uint32_t id = tokens[r];
  if (id >= vocab) return;
  const int lane = threadIdx.x & 63;
  for (int base = 0; base < r; base += 64) {
    const int j = base + lane;
    if (__ballot(j < r && tokens[j] == id)) return;  // an earlier row owns this token
  }
  const long row0 = (long)id * d;
  for (int c0 = 0; c0 < d; c0 += 256) {
    const int c = c0 + threadIdx.x;
    const bool active = c < d;
    uint16_t v = 0;
    float res = 0.0f;
    if (active) {
      v = table[row0 + c];
      res = residual[row0 + c];
    }
    for (int base = r; base < rows; base += 64) {
      const int j = base + lane;
      unsigned long long m = __ballot(j < rows && tokens[j] == id);
      while (m) {
        const int k = __builtin_ctzll(m);
        m &= m - 1;
        if (active) clipped_sgd_one(v, res, g[(long)(base + k) * d + c], lr);
      }
    }
    if (active) {
      table[row0 + c] = v;
      residual[row0 + c] = res;
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
