// Element-wise and reduction kernels around the GEMMs (HBM-bound).
//
// Reference semantics:
//   clipped SGD          Fp16Storage::apply_clipped_sgd   src/precision.rs:106-113
//   BinaryConnect SGD    apply_binaryconnect_sgd          src/precision.rs:124-134
//   sign bit-planes      bit_from_activation + pack_bitplane src/rosa.rs:372-374, 400-411
//   time-shift mix       time_shift_delta + lerp          src/model.rs:186-212, 1049-1057, 1385-1396
//   its backward         lerp_shift_backward              src/model.rs:1207-1240
//   ROSA output          (2*idx-1)*e                      src/rosa.rs:614-639
//   ROSA e gradient      rosa_e_grad                      src/model.rs:1608-1634
// Column reductions (g_mix, g_e, g_bias) are two-stage with fixed-order
// partial sums: deterministic, unlike the Metal float CAS atomics
// (rwkv8.metal:12-25, :295-323).
#include <algorithm>

#include "common.hpp"
#include "ops.hpp"
#include "update.hpp"

namespace ullis {

namespace {

constexpr int kColChunkRows = 16;

__global__ void fill_kernel(float* p, long n, float v) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// 16-byte vector copy, grid-stride; the head/tail bytes outside the aligned
// middle are copied one byte per thread by block 0.
__global__ void copy_kernel(uint8_t* dst, const uint8_t* src, long head, long vecs, long bytes) {
  const long stride = (long)gridDim.x * blockDim.x;
  const u32x4* s = reinterpret_cast<const u32x4*>(src + head);
  u32x4* d = reinterpret_cast<u32x4*>(dst + head);
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < vecs; i += stride) d[i] = s[i];
  if (blockIdx.x == 0) {
    const long tail0 = head + vecs * 16;
    for (long i = threadIdx.x; i < head; i += blockDim.x) dst[i] = src[i];
    for (long i = tail0 + threadIdx.x; i < bytes; i += blockDim.x) dst[i] = src[i];
  }
}

__global__ void clipped_sgd_kernel(uint16_t* values, float* residual, const float* grad, long n,
                                   float lr) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) clipped_sgd_one(values[i], residual[i], grad[i], lr);
}

__global__ void binaryconnect_sgd_kernel(uint16_t* values, float* residual, const float* grad,
                                         long n, float lr, float grad_scale) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) binaryconnect_sgd_one(values[i], residual[i], grad[i] * grad_scale, lr);
}

__global__ void sign_pack_kernel(const float* x, long n, uint32_t* bits) {
  const long w = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long base = w * 32;
  if (base >= n) return;
  uint32_t packed = 0;
  for (int j = 0; j < 32; ++j) {
    const long i = base + j;
    if (i < n && x[i] > 0.0f) packed |= 1u << j;
  }
  bits[w] = packed;
}

__global__ __launch_bounds__(256) void amax_kernel(const float* x, long n, float* slot) {
  float m = 0.0f;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    m = __builtin_fmaxf(m, finite_abs(x[i]));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomic_amax(slot, m);
}

// One thread per (row, 8-channel group) when ch % 8 == 0, else per element.
__global__ void time_shift_mix_kernel(const uint16_t* x16, long rows, long time, long ch,
                                      const uint16_t* mix0, uint16_t* out0,
                                      const uint16_t* mix1, uint16_t* out1,
                                      const uint16_t* mix2, uint16_t* out2, int group) {
  const long gi = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long groups_per_row = ch / group;
  const long row = gi / groups_per_row;
  if (row >= rows) return;
  const long c0 = (gi % groups_per_row) * group;
  const long t = row % time;
  for (int j = 0; j < group; ++j) {
    const long idx = row * ch + c0 + j;
    const float xt = f16_bits_to_f32(x16[idx]);
    const float xx = t == 0 ? -xt : f16_bits_to_f32(x16[idx - ch]) - xt;
    const long c = c0 + j;
    if (out0) out0[idx] = f32_to_f16_bits(xt + xx * f16_bits_to_f32(mix0[c]));
    if (out1) out1[idx] = f32_to_f16_bits(xt + xx * f16_bits_to_f32(mix1[c]));
    if (out2) out2[idx] = f32_to_f16_bits(xt + xx * f16_bits_to_f32(mix2[c]));
  }
}

// Vector form: 8 channels per thread, 32-bit index math (rows * ch < 2^31,
// ch % 8 == 0, 16-byte aligned rows).
__device__ __forceinline__ void mix8_one(const half8& x, const half8& p, const uint16_t* mix,
                                         uint16_t* out, int c, long idx) {
  const half8 m = *reinterpret_cast<const half8*>(mix + c);
  half8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xt = (float)x[e];
    const float xx = (float)p[e] - xt;  // p = 0 at t == 0: xx = -x
    o[e] = (half_t)(xt + xx * (float)m[e]);
  }
  *reinterpret_cast<half8*>(out + idx) = o;
}

__global__ void time_shift_mix8_kernel(const uint16_t* x16, int rows, int time, int ch,
                                       const uint16_t* mix0, uint16_t* out0,
                                       const uint16_t* mix1, uint16_t* out1,
                                       const uint16_t* mix2, uint16_t* out2) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  const int gpr = ch >> 3;
  if (g >= rows * gpr) return;
  const int row = g / gpr;
  const int c = (g - row * gpr) * 8;
  const int t = row % time;
  const long idx = (long)row * ch + c;
  const half8 x = *reinterpret_cast<const half8*>(x16 + idx);
  half8 p = {};
  if (t > 0) p = *reinterpret_cast<const half8*>(x16 + idx - ch);
  if (out0) mix8_one(x, p, mix0, out0, c, idx);
  if (out1) mix8_one(x, p, mix1, out1, c, idx);
  if (out2) mix8_one(x, p, mix2, out2, c, idx);
}

// Column-reduction blocks: 16 rows x 64 channels, 4 channels per thread; the
// per-column partial of the block's rows is summed in row order through LDS.
constexpr int kColBlockCh = 64;

__device__ __forceinline__ void col_block_reduce(float (&red)[16][kColBlockCh], const float (&v)[4],
                                                 int tx, int ty, long c, long ch, float* dst) {
#pragma unroll
  for (int e = 0; e < 4; ++e) red[ty][tx * 4 + e] = v[e];
  __syncthreads();
  if (threadIdx.x < kColBlockCh) {
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += red[r][threadIdx.x];
    const long cc = (long)blockIdx.x * kColBlockCh + threadIdx.x;
    if (cc < ch) dst[cc] = s;
  }
  (void)c;
}

// grid (ch / 64, ceil(rows / 16)), 256 threads; ch % 4 == 0, aligned rows.
__global__ __launch_bounds__(256) void time_shift_mix_bwd4_kernel(
    const float* g_s, const uint16_t* x16, const uint16_t* mix, int rows, int time, int ch,
    float* g_x, float* part) {
  __shared__ float red[16][kColBlockCh];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const long c = (long)blockIdx.x * kColBlockCh + tx * 4;
  const int row = blockIdx.y * 16 + ty;
  float gm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (row < rows && c < ch) {
    const int t = row % time;
    const long idx = (long)row * ch + c;
    const floatx4 gs = *reinterpret_cast<const floatx4*>(g_s + idx);
    const half4 x = *reinterpret_cast<const half4*>(x16 + idx);
    half4 p = {};
    if (t > 0) p = *reinterpret_cast<const half4*>(x16 + idx - ch);
    floatx4 gn = {};
    const bool has_next = t + 1 < time;
    if (has_next) gn = *reinterpret_cast<const floatx4*>(g_s + idx + ch);
    const half4 m = *reinterpret_cast<const half4*>(mix + c);
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xt = (float)x[e];
      const float xx = (t == 0 ? 0.0f : (float)p[e]) - xt;
      const float mm = (float)m[e];
      gm[e] = gs[e] * xx;
      float gx = gs[e] - gs[e] * mm;
      if (has_next) gx = gx + gn[e] * mm;
      o[e] = gx;
    }
    *reinterpret_cast<floatx4*>(g_x + idx) = o;
  }
  col_block_reduce(red, gm, tx, ty, c, ch, part + (long)blockIdx.y * ch);
}

// grid (ch / 64, ceil(rows / 16)), 256 threads; ch % 4 == 0, aligned rows.
__global__ __launch_bounds__(256) void column_sum4_kernel(const float* v, const uint8_t* idx,
                                                          int rows, int ch, float* part,
                                                          uint16_t* out16, const float* amax) {
  __shared__ float red[16][kColBlockCh];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const long c = (long)blockIdx.x * kColBlockCh + tx * 4;
  const int row = blockIdx.y * 16 + ty;
  float sv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (row < rows && c < ch) {
    const long i = (long)row * ch + c;
    const floatx4 x = *reinterpret_cast<const floatx4*>(v + i);
    if (idx) {
      const uint32_t b = *reinterpret_cast<const uint32_t*>(idx + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = x[e] * (2.0f * (float)((b >> (8 * e)) & 0xFFu) - 1.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = x[e];
    }
    if (out16) {
      const float sc = grad_scale_from_amax(*amax);
      half4 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = f32_to_f16_sat(x[e] * sc);
      *reinterpret_cast<half4*>(out16 + i) = h;
    }
  }
  col_block_reduce(red, sv, tx, ty, c, ch, part + (long)blockIdx.y * ch);
}

// grid (ceil(ch/256), ceil(rows/64)); thread = one channel over a 64-row chunk.
__global__ void time_shift_mix_bwd_kernel(const float* g_s, const uint16_t* x16,
                                          const uint16_t* mix, long rows, long time, long ch,
                                          float* g_x, float* part) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ch) return;
  const long r0 = (long)blockIdx.y * kColChunkRows;
  const long r1 = r0 + kColChunkRows < rows ? r0 + kColChunkRows : rows;
  const float m = f16_bits_to_f32(mix[c]);
  float gm = 0.0f;
  for (long row = r0; row < r1; ++row) {
    const long idx = row * ch + c;
    const long t = row % time;
    const float gs = g_s[idx];
    const float xt = f16_bits_to_f32(x16[idx]);
    const float xx = t == 0 ? -xt : f16_bits_to_f32(x16[idx - ch]) - xt;
    gm += gs * xx;
    float gx = gs - gs * m;
    if (t + 1 < time) gx = gx + g_s[idx + ch] * m;
    g_x[idx] = gx;
  }
  part[(long)blockIdx.y * ch + c] = gm;
}

__global__ void column_sum_kernel(const float* v, const uint8_t* idx, long rows, long ch,
                                  float* part, uint16_t* out16, const float* amax) {
  const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ch) return;
  const long r0 = (long)blockIdx.y * kColChunkRows;
  const long r1 = r0 + kColChunkRows < rows ? r0 + kColChunkRows : rows;
  const float sc = out16 ? grad_scale_from_amax(*amax) : 1.0f;
  float s = 0.0f;
  for (long row = r0; row < r1; ++row) {
    const long i = row * ch + c;
    const float x = v[i];
    s += idx ? x * (2.0f * (float)idx[i] - 1.0f) : x;
    if (out16) out16[i] = __builtin_bit_cast(uint16_t, f32_to_f16_sat(x * sc));
  }
  part[(long)blockIdx.y * ch + c] = s;
}

// out16 = f16_sat(v * grad_scale_from_amax(*amax)), 4 elements per thread.
__global__ void scale_to_f16_kernel(const float* v, long n, const float* amax, uint16_t* out16) {
  const float sc = grad_scale_from_amax(*amax);
  const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    const floatx4 x = *reinterpret_cast<const floatx4*>(v + i);
    uint32_t lo = __builtin_bit_cast(uint16_t, f32_to_f16_sat(x[0] * sc)) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_sat(x[1] * sc)) << 16);
    uint32_t hi = __builtin_bit_cast(uint16_t, f32_to_f16_sat(x[2] * sc)) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_sat(x[3] * sc)) << 16);
    *reinterpret_cast<uint2*>(out16 + i) = make_uint2(lo, hi);
  } else {
    for (long j = i; j < n; ++j) out16[j] = __builtin_bit_cast(uint16_t, f32_to_f16_sat(v[j] * sc));
  }
}

// Sums part[nblk][ncols] over nblk: 16 columns per block, 64 partial subsets
// per column summed in a fixed order (strided, then an LDS tree), so the result
// does not depend on scheduling. Columns < split go to target a, the rest to b.
__global__ void f32_to_f16_kernel(const float* v, long n, uint16_t* out16) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out16[i] = f32_to_f16_bits(v[i]);
}

__global__ void add_f32_kernel(const float* a, const float* b, long n, float* out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(1024) void partial_reduce_kernel(const float* part, int nblk,
                                                              long ncols, long split, VecTarget a,
                                                              VecTarget b) {
  __shared__ float red[64][64];
  vec_reduce_block(part, nblk, ncols, split, a, a.lr, b, b.lr, blockIdx.x, red);
}

__global__ void rosa_expand_kernel(const uint8_t* idx_cm, const uint16_t* e, long batch, long time,
                                   long ch, uint16_t* y16, uint8_t* idx_rm) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long n = batch * time * ch;
  if (i >= n) return;
  const long c = i % ch;
  const long row = i / ch;
  const long b = row / time, t = row % time;
  const uint8_t bit = idx_cm[(b * ch + c) * time + t];
  const float y = (2.0f * (float)bit - 1.0f) * f16_bits_to_f32(e[c]);
  y16[i] = f32_to_f16_bits(y);
  if (idx_rm) idx_rm[i] = bit;
}

// Channel-major [B][C][T] bits -> row-major [B*T][C] through a 64 x 64 LDS
// tile (coalesced 16-byte reads along T and writes along C).
// grid (T / 64, C / 64, B * layers); requires T % 64 == 0, C % 64 == 0.
// Layer l = blockIdx.z / B reads idx_cm and writes y16 / idx_rm at offset
// l * B * T * C, with e = e_tab[l] (e_tab null: one layer, e).
__global__ __launch_bounds__(256) void rosa_expand_tile_kernel(const uint8_t* idx_cm,
                                                               const uint16_t* e,
                                                               const uint16_t* const* e_tab,
                                                               int batch, int time, int ch,
                                                               uint16_t* y16, uint8_t* idx_rm) {
  __shared__ uint8_t tile[64][64 + 16];
  const int t0 = blockIdx.x * 64, c0 = blockIdx.y * 64, b = blockIdx.z % batch;
  const int l = blockIdx.z / batch;
  if (e_tab) {
    const long lofs = (long)l * batch * time * ch;
    e = e_tab[l];
    idx_cm += lofs;
    y16 += lofs;
    if (idx_rm) idx_rm += lofs;
  }
  {
    const int cl = threadIdx.x >> 2, tl = (threadIdx.x & 3) * 16;
    const u32x4 v = *reinterpret_cast<const u32x4*>(
        idx_cm + ((long)b * ch + c0 + cl) * time + t0 + tl);
    *reinterpret_cast<u32x4*>(&tile[cl][tl]) = v;
  }
  __syncthreads();
  const int tl = threadIdx.x >> 2, cl = (threadIdx.x & 3) * 16;
  const long row = (long)b * time + t0 + tl;
  uint8_t bits[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) bits[k] = tile[cl + k][tl];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const half8 ev = *reinterpret_cast<const half8*>(e + c0 + cl + 8 * q);
    half8 y;
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (half_t)((2.0f * (float)bits[8 * q + k] - 1.0f) * (float)ev[k]);
    *reinterpret_cast<half8*>(y16 + row * ch + c0 + cl + 8 * q) = y;
  }
  if (idx_rm) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w[q] = (uint32_t)bits[4 * q] | ((uint32_t)bits[4 * q + 1] << 8) |
             ((uint32_t)bits[4 * q + 2] << 16) | ((uint32_t)bits[4 * q + 3] << 24);
    *reinterpret_cast<u32x4*>(idx_rm + row * ch + c0 + cl) = w;
  }
}

inline dim3 grid1d(long n, int threads = 256) { return dim3((unsigned)cdiv(n, threads)); }
inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t add_f32(hipStream_t s, const float* a, const float* b, long n, float* out) {
  if (n <= 0) return hipSuccess;
  launch(add_f32_kernel, grid1d(n), dim3(256), 0, s, a, b, n, out);
  return hipGetLastError();
}

hipError_t fill_f32(hipStream_t s, float* p, long n, float v) {
  if (n <= 0) return hipSuccess;
  launch(fill_kernel, grid1d(n), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

namespace {

// dst[c][r] = src[r][c] for one 64 x 64 tile of 16-bit values through LDS
// (a padded row keeps the column reads free of bank conflicts).
__global__ __launch_bounds__(256) void transpose_u16_kernel(const uint16_t* __restrict__ src,
                                                            long rows, long cols,
                                                            uint16_t* __restrict__ dst) {
  __shared__ uint16_t t[64][66];
  const long r0 = (long)blockIdx.y * 64, c0 = (long)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int r = ty + 4 * k;
    if (r0 + r < rows && c0 + tx < cols) t[r][tx] = src[(r0 + r) * cols + c0 + tx];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = ty + 4 * k;
    if (c0 + c < cols && r0 + tx < rows) dst[(c0 + c) * rows + r0 + tx] = t[tx][c];
  }
}

}  // namespace

hipError_t transpose_u16(hipStream_t s, const uint16_t* src, long rows, long cols, uint16_t* dst) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (cdiv(rows, 64) > 65535 || cdiv(cols, 64) > INT32_MAX) return hipErrorInvalidValue;
  launch(transpose_u16_kernel, dim3((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64)),
         dim3(256), 0, s, src, rows, cols, dst);
  return hipGetLastError();
}

hipError_t copy_device(hipStream_t s, void* dst, const void* src, long bytes) {
  if (bytes <= 0) return hipSuccess;
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst), b = reinterpret_cast<uintptr_t>(src);
  long head = 0, vecs = 0;
  if ((a & 15) == (b & 15)) {
    head = std::min<long>((long)((16 - (a & 15)) & 15), bytes);
    vecs = (bytes - head) / 16;
  } else {
    head = bytes;  // no common alignment: block 0 copies byte by byte
  }
  const long blocks = std::max<long>(1, std::min<long>(cdiv(vecs, 256), 8192));
  launch(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     static_cast<uint8_t*>(dst), static_cast<const uint8_t*>(src), head, vecs,
                     bytes);
  return hipGetLastError();
}

hipError_t clipped_sgd(hipStream_t s, uint16_t* values, float* residual, const float* grad, long n,
                       float lr) {
  if (n <= 0) return hipSuccess;
  launch(clipped_sgd_kernel, grid1d(n), dim3(256), 0, s, values, residual, grad, n, lr);
  return hipGetLastError();
}

hipError_t binaryconnect_sgd(hipStream_t s, uint16_t* values, float* residual, const float* grad,
                             long n, float lr, float grad_scale) {
  if (n <= 0) return hipSuccess;
  launch(binaryconnect_sgd_kernel, grid1d(n), dim3(256), 0, s, values, residual, grad,
                     n, lr, grad_scale);
  return hipGetLastError();
}

hipError_t sign_pack_bits(hipStream_t s, const float* x, long n, uint32_t* bits) {
  if (n <= 0) return hipSuccess;
  launch(sign_pack_kernel, grid1d(cdiv(n, 32)), dim3(256), 0, s, x, n, bits);
  return hipGetLastError();
}

hipError_t amax_f32(hipStream_t s, const float* x, long n, float* slot) {
  if (n <= 0) return hipSuccess;
  long blocks = cdiv(n, 256 * 8);
  if (blocks > 1024) blocks = 1024;
  launch(amax_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, slot);
  return hipGetLastError();
}

hipError_t time_shift_mix(hipStream_t s, const uint16_t* x16, long rows, long time, long ch,
                          const uint16_t* mix0, uint16_t* out0, const uint16_t* mix1,
                          uint16_t* out1, const uint16_t* mix2, uint16_t* out2) {
  if (rows <= 0 || ch <= 0 || time <= 0) return hipSuccess;
  if (ch % 8 == 0 && rows * ch < (1L << 31) && a16(x16) && (!out0 || (a16(out0) && a16(mix0))) &&
      (!out1 || (a16(out1) && a16(mix1))) && (!out2 || (a16(out2) && a16(mix2)))) {
    launch(time_shift_mix8_kernel, grid1d(rows * ch / 8), dim3(256), 0, s, x16, (int)rows,
           (int)time, (int)ch, mix0, out0, mix1, out1, mix2, out2);
    return hipGetLastError();
  }
  const int group = ch % 8 == 0 ? 8 : 1;
  const long n = rows * (ch / group);
  launch(time_shift_mix_kernel, grid1d(n), dim3(256), 0, s, x16, rows, time, ch, mix0,
                     out0, mix1, out1, mix2, out2, group);
  return hipGetLastError();
}

hipError_t time_shift_mix_backward(hipStream_t s, const float* g_shifted, const uint16_t* x16,
                                   const uint16_t* mix, long rows, long time, long ch, float* g_x,
                                   float* part, int* nblk_out) {
  const long nblk = cdiv(rows, kColChunkRows);
  if (nblk_out) *nblk_out = (int)nblk;
  if (rows <= 0 || ch <= 0) return hipSuccess;
  if (ch % 4 == 0 && rows * ch < (1L << 31) && a16(g_shifted) && a16(g_x) &&
      (reinterpret_cast<uintptr_t>(x16) & 7u) == 0 && (reinterpret_cast<uintptr_t>(mix) & 7u) == 0) {
    launch(time_shift_mix_bwd4_kernel, dim3((unsigned)cdiv(ch, kColBlockCh), (unsigned)nblk),
           dim3(256), 0, s, g_shifted, x16, mix, (int)rows, (int)time, (int)ch, g_x, part);
    return hipGetLastError();
  }
  launch(time_shift_mix_bwd_kernel, dim3((unsigned)cdiv(ch, 256), (unsigned)nblk),
                     dim3(256), 0, s, g_shifted, x16, mix, rows, time, ch, g_x, part);
  return hipGetLastError();
}

hipError_t column_sum_partials(hipStream_t s, const float* v, const uint8_t* idx, long rows,
                               long ch, float* part, int* nblk_out, uint16_t* out16,
                               const float* amax) {
  const long nblk = cdiv(rows, kColChunkRows);
  if (nblk_out) *nblk_out = (int)nblk;
  if (rows <= 0 || ch <= 0) return hipSuccess;
  if (out16 && !amax) return hipErrorInvalidValue;
  if (ch % 4 == 0 && rows * ch < (1L << 31) && a16(v) &&
      (reinterpret_cast<uintptr_t>(idx) & 3u) == 0 &&
      (reinterpret_cast<uintptr_t>(out16) & 7u) == 0) {
    launch(column_sum4_kernel, dim3((unsigned)cdiv(ch, kColBlockCh), (unsigned)nblk), dim3(256), 0,
           s, v, idx, (int)rows, (int)ch, part, out16, amax);
    return hipGetLastError();
  }
  launch(column_sum_kernel, dim3((unsigned)cdiv(ch, 256), (unsigned)nblk), dim3(256), 0, s, v,
         idx, rows, ch, part, out16, amax);
  return hipGetLastError();
}

hipError_t scale_to_f16(hipStream_t s, const float* v, long n, const float* amax,
                        uint16_t* out16) {
  if (n <= 0) return hipSuccess;
  if ((reinterpret_cast<uintptr_t>(v) & 15u) != 0 || (reinterpret_cast<uintptr_t>(out16) & 7u) != 0)
    return hipErrorInvalidValue;
  launch(scale_to_f16_kernel, dim3((unsigned)cdiv(cdiv(n, 4), 256)), dim3(256), 0, s, v, n, amax,
         out16);
  return hipGetLastError();
}

hipError_t f32_to_f16(hipStream_t s, const float* v, long n, uint16_t* out16) {
  if (n <= 0) return hipSuccess;
  launch(f32_to_f16_kernel, grid1d(n), dim3(256), 0, s, v, n, out16);
  return hipGetLastError();
}

hipError_t partial_reduce(hipStream_t s, const float* part, int nblk, long ncols, long split,
                          const VecTarget& a, const VecTarget& b) {
  if (ncols <= 0) return hipSuccess;
  launch(partial_reduce_kernel, dim3((unsigned)vec_job_blocks(ncols)), dim3(1024), 0, s, part, nblk,
         ncols, split, a, b);
  return hipGetLastError();
}

hipError_t vector_finish(hipStream_t s, const float* part, int nblk, long ch, float* out,
                         float lr, uint16_t* values, float* residual) {
  VecTarget a{out, values, residual, lr, nullptr};
  return partial_reduce(s, part, nblk, ch, ch, a, a);
}

hipError_t rosa_expand(hipStream_t s, const uint8_t* idx_cm, const uint16_t* e, long batch,
                       long time, long ch, uint16_t* y16, uint8_t* idx_rm) {
  const long n = batch * time * ch;
  if (n <= 0) return hipSuccess;
  if (time % 64 == 0 && ch % 64 == 0 && time * ch < (1L << 31) && a16(idx_cm) && a16(e) &&
      a16(y16) && (!idx_rm || a16(idx_rm))) {
    launch(rosa_expand_tile_kernel, dim3((unsigned)(time / 64), (unsigned)(ch / 64), (unsigned)batch),
           dim3(256), 0, s, idx_cm, e, (const uint16_t* const*)nullptr, (int)batch, (int)time,
           (int)ch, y16, idx_rm);
    return hipGetLastError();
  }
  launch(rosa_expand_kernel, grid1d(n), dim3(256), 0, s, idx_cm, e, batch, time, ch,
                     y16, idx_rm);
  return hipGetLastError();
}

hipError_t rosa_expand_layers(hipStream_t s, const uint8_t* idx_cm, const uint16_t* const* e_host,
                              const uint16_t* const* e_dev, long layers, long batch, long time,
                              long ch, uint16_t* y16, uint8_t* idx_rm) {
  const long nd = batch * time * ch;
  if (nd <= 0 || layers <= 0) return hipSuccess;
  bool tile = time % 64 == 0 && ch % 64 == 0 && time * ch < (1L << 31) &&
              batch * layers <= 65535 && a16(idx_cm) && a16(y16) && (!idx_rm || a16(idx_rm)) &&
              e_dev != nullptr;
  for (long l = 0; l < layers && tile; ++l) tile = a16(e_host[l]);
  if (tile) {
    launch(rosa_expand_tile_kernel,
           dim3((unsigned)(time / 64), (unsigned)(ch / 64), (unsigned)(batch * layers)), dim3(256),
           0, s, idx_cm, (const uint16_t*)nullptr, e_dev, (int)batch, (int)time, (int)ch, y16,
           idx_rm);
    return hipGetLastError();
  }
  for (long l = 0; l < layers; ++l) {
    hipError_t e = rosa_expand(s, idx_cm + l * nd, e_host[l], batch, time, ch, y16 + l * nd,
                               idx_rm ? idx_rm + l * nd : nullptr);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ullis
