// Kernels of the T = 1 decode step (UllisHeron::generate_step,
// src/model.rs:2717-2753): the time-shift mixes against the previous token's
// values kept in the decode state (time_shift_one, src/model.rs:214-228, and
// the mixes of ROSA / CMix forward_one, src/model.rs:1320-1353, 1003-1016),
// and the greedy argmax over the last token's logits. The products are the
// few-row forward kernels of gemv.hip, reached through packed_forward /
// fp16_forward.
#include "common.hpp"
#include "ops.hpp"

namespace ullis {

namespace {

// Element i of [rows][d]: xx = prev - x (-x without a previous token),
// out_j = f16(x + xx * mix_j[c]) for the given mixes, then prev = x.
__global__ __launch_bounds__(256) void decode_mix_kernel(const float* __restrict__ x,
                                                         float* __restrict__ prev, int has_prev,
                                                         long n, int d, const uint16_t* mix0,
                                                         uint16_t* out0, const uint16_t* mix1,
                                                         uint16_t* out1, const uint16_t* mix2,
                                                         uint16_t* out2) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int c = (int)(i % d);
  const float xv = x[i];
  const float xx = has_prev ? prev[i] - xv : -xv;
  if (out0) out0[i] = f32_to_f16_bits(xv + xx * f16_bits_to_f32(mix0[c]));
  if (out1) out1[i] = f32_to_f16_bits(xv + xx * f16_bits_to_f32(mix1[c]));
  if (out2) out2[i] = f32_to_f16_bits(xv + xx * f16_bits_to_f32(mix2[c]));
  prev[i] = xv;
}

// One block per row: the index of the row's largest logit (the lowest index
// among equal maxima; NaN logits are never chosen).
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, long vocab,
                                                     uint32_t* __restrict__ next) {
  __shared__ float bv[4];
  __shared__ long bi[4];
  const float* row = logits + (long)blockIdx.x * vocab;
  float best = -__builtin_inff();
  long at = vocab;
  for (long v = threadIdx.x; v < vocab; v += blockDim.x) {
    const float l = row[v];
    if (l > best || (l == best && v < at)) {
      best = l;
      at = v;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const long oi = __shfl_xor(at, off, 64);
    if (ov > best || (ov == best && oi < at)) {
      best = ov;
      at = oi;
    }
  }
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = at;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] < at)) {
        best = bv[w];
        at = bi[w];
      }
    next[blockIdx.x] = at < vocab ? (uint32_t)at : 0u;
  }
}

}  // namespace

hipError_t decode_mix(hipStream_t s, const float* x, float* prev, bool has_prev, long rows,
                      long d, const uint16_t* mix0, uint16_t* out0, const uint16_t* mix1,
                      uint16_t* out1, const uint16_t* mix2, uint16_t* out2) {
  const long n = rows * d;
  if (n <= 0) return hipSuccess;
  if (d > INT32_MAX) return hipErrorInvalidValue;
  launch(decode_mix_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, x, prev,
         has_prev ? 1 : 0, n, (int)d, mix0, out0, mix1, out1, mix2, out2);
  return hipGetLastError();
}

hipError_t argmax_rows(hipStream_t s, const float* logits, long rows, long vocab, uint32_t* next) {
  if (rows <= 0 || vocab <= 0) return hipSuccess;
  if (rows > INT32_MAX) return hipErrorInvalidValue;
  launch(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, s, logits, vocab, next);
  return hipGetLastError();
}

}  // namespace ullis
