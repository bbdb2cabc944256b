// Packed +-1 BinaryConnect linear and FP16 linear on gfx950 MFMA.
//
// Reference semantics (Vladislav-Kalinkin/ullis 0.10.0):
//   forward      y[r,o]  = bias[o] + scale[o] * sum_i sign[o,i] x[r,i]   src/model.rs:724-742
//   input grad   gx[r,i] = sum_o gy[r,o] scale[o] sign[o,i]             src/model.rs:783
//   weight grad  gw[o,i] = sum_r gy[r,o] scale[o] x[r,i]                src/model.rs:782
//   scale grad   gs[o]   = sum_r gy[r,o] sum_i sign[o,i] x[r,i]         src/model.rs:787
//                        = sum_i sign[o,i] G[o,i],  G = gy^T x  (computed that way here)
//   latent SGD   BinaryConnect step on g = gw * ste, then rebinarize    src/model.rs:808-884
//   FP16 linear  y = x W^T, gx = gy W, gW = gy^T x, clipped SGD          src/model.rs:419-470
// The Metal kernels these replace are ullis_binary_linear*, ullis_fp16_linear*
// (src/metal/rwkv8.metal:370-841).
#include <type_traits>

#include "gemm.hpp"
#include "gemm_lds.hpp"
#include "ops.hpp"
#include "update.hpp"

namespace ullis {

namespace {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int vec_ok_f16(const void* p, long ld) { return aligned16(p) && ld % 8 == 0; }
inline int vec_ok_f32(const void* p, long ld) { return aligned16(p) && ld % 4 == 0; }

inline int bits_aligned(long ldb, long kofs, const void* kscale) {
  return ldb % 8 == 0 && kofs % 8 == 0 && (!kscale || aligned16(kscale));
}

// 128x128 tiles when they alone give ~one block per CU, else 64x64.
template <class F>
hipError_t with_tile(long M, long N, F&& f) {
  if (cdiv(M, 128) * cdiv(N, 128) >= 240) return f(CfgLarge{});
  return f(CfgSmall{});
}

template <class T, class LA, class LB, class Epi>
hipError_t launch_gemm(hipStream_t s, const LA& la, const LB& lb, const Epi& epi, long M, long N,
                       long K, int splits) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return hipErrorInvalidValue;
  if (splits < 1) splits = 1;
  const long tiles = cdiv(M, T::bm) * cdiv(N, T::bn);
  const int ks = (int)(cdiv(cdiv(K, splits), T::bk) * T::bk);
  launch((gemm_kernel<T::bm, T::bn, T::bk, T::stages, LA, LB, Epi>),
                     dim3((unsigned)tiles, 1, splits), dim3(kThreads), 0, s, la, lb, epi, (int)M,
                     (int)N, (int)K, ks > 0 ? ks : T::bk);
  return hipGetLastError();
}

__device__ __forceinline__ float unscale_of(const float* amax) {
  return amax ? 1.0f / grad_scale_from_amax(*amax) : 1.0f;
}

// ---------------------------------------------------------------- epilogues

// Output set of a packed forward, fixed at compile time so each instantiation
// carries only the stores it makes (a generic epilogue keeps every path live
// and spills at 128x128 tiles).
enum : int { kOutY32 = 1, kOutResid = 2, kOutY16 = 4, kOutRelu2 = 8, kOutBits = 16 };

template <int OUT>
struct EpiPackedFwd {
  const uint16_t* scale;
  const uint16_t* bias;
  PackedFwdOut o;
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = col0 + j * 32 + (lane & 31);
        const bool colok = col < N;
        const float sc = colok ? f16_bits_to_f32(scale[col]) : 0.0f;
        const float bi = (bias && colok) ? f16_bits_to_f32(bias[col]) : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row0 + i * 32 + mfma32_row(r, lane);
          const bool ok = colok && row < M;
          const float y = bi + sc * acc[i][j][r];
          const long idx = (long)row * N + col;
          if (ok) {
            if constexpr ((OUT & kOutY32) != 0) {
              if constexpr ((OUT & kOutResid) != 0)
                o.y32[idx] = o.resid[idx] + y;
              else
                o.y32[idx] = y;
            }
            if constexpr ((OUT & kOutY16) != 0) o.y16[idx] = __builtin_bit_cast(uint16_t, (half_t)y);
            if constexpr ((OUT & kOutRelu2) != 0) {
              const float k = y > 0.0f ? y : 0.0f;
              o.relu2_16[idx] = __builtin_bit_cast(uint16_t, (half_t)(k * k));
            }
          }
          if constexpr ((OUT & kOutBits) != 0) {
            const unsigned long long m = __ballot(ok && y > 0.0f);
            if ((lane & 31) == 0 && row < M && col0 + j * 32 < N) {
              const long word = ((long)row * N + col0 + j * 32) >> 5;
              o.sign_bits[word] = (lane < 32) ? (uint32_t)m : (uint32_t)(m >> 32);
            }
          }
        }
      }
  }
  // Streamed-LDS kernels: 16 consecutive columns of one row (lds::epilogue_rows).
  __device__ void row16(int row, int col, float (&v)[16], int lane, int M, int N, float*, int,
                        int) {
    const bool rok = row < M;
    const bool full = col + 16 <= N && N % 8 == 0;
    float sc[16], bi[16];
    lds::get16h(scale, col, N, full && lds::al16(scale), sc);
    if (bias) {
      lds::get16h(bias, col, N, full && lds::al16(bias), bi);
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) bi[k] = 0.0f;
    }
    float y[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) y[k] = bi[k] + sc[k] * v[k];
    if constexpr ((OUT & kOutBits) != 0) {
      // out % 32 == 0: lanes 2r and 2r+1 hold the two halves of one word
      uint32_t m = 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) m |= (uint32_t)(rok && col + k < N && y[k] > 0.0f) << k;
      const uint32_t other = (uint32_t)__shfl_xor((int)m, 1, 64);
      if (rok && (lane & 1) == 0 && col < N)
        o.sign_bits[((long)row * N + col) >> 5] = m | (other << 16);
    }
    if (!rok) return;
    const long idx = (long)row * N + col;
    if constexpr ((OUT & kOutY32) != 0) {
      float z[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) z[k] = y[k];
      if (full && lds::al16(o.y32) && (!((OUT & kOutResid) != 0) || lds::al16(o.resid))) {
        if constexpr ((OUT & kOutResid) != 0) {
          float rv[16];
          lds::load16f(o.resid + idx, rv);
#pragma unroll
          for (int k = 0; k < 16; ++k) z[k] = rv[k] + y[k];
        }
        lds::store16f(o.y32 + idx, z);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          o.y32[idx + k] = ((OUT & kOutResid) != 0) ? o.resid[idx + k] + y[k] : y[k];
      }
    }
    if constexpr ((OUT & kOutY16) != 0) {
      if (full && lds::al16(o.y16)) {
        lds::store16h(o.y16 + idx, y);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          o.y16[idx + k] = __builtin_bit_cast(uint16_t, (half_t)y[k]);
      }
    }
    if constexpr ((OUT & kOutRelu2) != 0) {
      float r2[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float kk = y[k] > 0.0f ? y[k] : 0.0f;
        r2[k] = kk * kk;
      }
      if (full && lds::al16(o.relu2_16)) {
        lds::store16h(o.relu2_16 + idx, r2);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          o.relu2_16[idx + k] = __builtin_bit_cast(uint16_t, (half_t)r2[k]);
      }
    }
  }
};

// The ROSA e gradient from the O input gradient g (never stored): column sums
// of g * (2 idx - 1) over 16-row groups, with the same products and summation
// order as column_sum_partials over the stored g (streamed-LDS kernels only).
struct EpiSignedColSum {
  const float* amax;  // operand scale to divide out
  const uint8_t* idx;  // [M][N]
  float* part;         // [ceil(M/16)][N]
  __device__ void row16(int row, int col, float (&v)[16], int lane, int M, int N, float* buf,
                        int brow, int bcol) {
    const float m = unscale_of(amax);
    float g[16];
    if (row < M) {
      const long i = (long)row * N + col;
      if (col + 16 <= N && N % 16 == 0 && lds::al16(idx)) {
        const u32x4 b = *reinterpret_cast<const u32x4*>(idx + i);
#pragma unroll
        for (int k = 0; k < 16; ++k)
          g[k] = (v[k] * m) * (2.0f * (float)((b[k >> 2] >> (8 * (k & 3))) & 0xFFu) - 1.0f);
      } else {
#pragma unroll
        for (int k = 0; k < 16; ++k)
          g[k] = col + k < N ? (v[k] * m) * (2.0f * (float)idx[i + k] - 1.0f) : 0.0f;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) g[k] = 0.0f;
    }
    float* rowp = buf + (lane >> 1) * lds::kBufPitch + (lane & 1) * 16;
#pragma unroll
    for (int k = 0; k < 16; ++k) rowp[k] = g[k];
    lds::lds_fence();
    // half-wave h sums rows [16 h, 16 h + 16) of column lane % 32
    const int c = lane & 31, h = lane >> 5;
    float cs = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) cs += buf[(16 * h + r) * lds::kBufPitch + c];
    const int prow = brow + 16 * h;
    if (bcol + c < N && prow < M) part[(long)(prow / 16) * N + bcol + c] = cs;
  }
};

struct EpiStoreF32 {
  float* out;
  const float* amax;  // operand scale to divide out
  const float* mul;   // extra device scalar
  int accumulate;
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
    float m = unscale_of(amax);
    if (mul) m *= *mul;
    for_each_acc(acc, row0, col0, lane, M, N, [&](int row, int col, float v) {
      const long idx = (long)row * N + col;
      const float g = v * m;
      out[idx] = accumulate ? out[idx] + g : g;
    });
  }
  __device__ void row16(int row, int col, float (&v)[16], int, int M, int N, float*, int, int) {
    if (row >= M) return;
    float m = unscale_of(amax);
    if (mul) m *= *mul;
    const long idx = (long)row * N + col;
    if (col + 16 <= N && N % 8 == 0 && lds::al16(out)) {
      float g[16];
      if (accumulate) lds::load16f(out + idx, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) g[k] = accumulate ? g[k] + v[k] * m : v[k] * m;
      lds::store16f(out + idx, g);
    } else {
      for (int k = 0; k < 16 && col + k < N; ++k)
        out[idx + k] = accumulate ? out[idx + k] + v[k] * m : v[k] * m;
    }
  }
};

struct EpiF16Fwd {
  float* y32;
  const float* resid;
  uint16_t* y16;
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
    for_each_acc(acc, row0, col0, lane, M, N, [&](int row, int col, float y) {
      const long idx = (long)row * N + col;
      if (y32) y32[idx] = resid ? resid[idx] + y : y;
      if (y16) y16[idx] = __builtin_bit_cast(uint16_t, (half_t)y);
    });
  }
  __device__ void row16(int row, int col, float (&v)[16], int, int M, int N, float*, int, int) {
    if (row >= M) return;
    const long idx = (long)row * N + col;
    const bool full = col + 16 <= N && N % 8 == 0;
    if (y32) {
      if (full && lds::al16(y32) && (!resid || lds::al16(resid))) {
        float z[16];
        if (resid) lds::load16f(resid + idx, z);
#pragma unroll
        for (int k = 0; k < 16; ++k) z[k] = resid ? z[k] + v[k] : v[k];
        lds::store16f(y32 + idx, z);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          y32[idx + k] = resid ? resid[idx + k] + v[k] : v[k];
      }
    }
    if (y16) {
      if (full && lds::al16(y16)) {
        lds::store16h(y16 + idx, v);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          y16[idx + k] = __builtin_bit_cast(uint16_t, (half_t)v[k]);
      }
    }
  }
};

// ReLU^2 backward fused into the value input-gradient: gk = 2 k g (k > 0),
// src/model.rs:1191-1205, stored in the scaled fp16 domain of g.
struct EpiRelu2Bwd {
  const uint16_t* key16;
  uint16_t* gk16;
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
    for_each_acc(acc, row0, col0, lane, M, N, [&](int row, int col, float g) {
      const long idx = (long)row * N + col;
      const float k = f16_bits_to_f32(key16[idx]);
      const float gk = k > 0.0f ? 2.0f * k * g : 0.0f;
      gk16[idx] = __builtin_bit_cast(uint16_t, f32_to_f16_sat(gk));
    });
  }
  __device__ void row16(int row, int col, float (&v)[16], int, int M, int N, float*, int, int) {
    if (row >= M) return;
    const long idx = (long)row * N + col;
    const bool full = col + 16 <= N && N % 8 == 0 && lds::al16(key16) && lds::al16(gk16);
    float k[16];
    lds::get16h(key16 + idx - col, col, N, full, k);
    float gk[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float t = k[e] > 0.0f ? 2.0f * k[e] * v[e] : 0.0f;
      gk[e] = __builtin_fminf(__builtin_fmaxf(t, -65504.0f), 65504.0f);  // f32_to_f16_sat
    }
    if (full) {
      lds::store16h(gk16 + idx, gk);
    } else {
      for (int e = 0; e < 16 && col + e < N; ++e)
        gk16[idx + e] = __builtin_bit_cast(uint16_t, (half_t)gk[e]);
    }
  }
};

// ------------------------------------------------------------ finish kernels

__global__ __launch_bounds__(256) void packed_finish_kernel(PackedFinish f) {
  __shared__ float red[256];
  const long o = blockIdx.x;
  if (o >= f.out) return;
  packed_finish_row(f, o, f.lr, red);
}

__global__ __launch_bounds__(256) void packed_finish_wave_kernel(PackedFinish f) {
  const long o = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o < f.out) packed_finish_row_wave(f, o, f.lr);
}

__global__ void fp16_finish_kernel(const float* part, int splits, long n, const float* amax,
                                   float lr, uint16_t* w, float* w_res, float* g_w) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  fp16_finish_one(part, splits, n, i, amax, lr, w, w_res, g_w);
}

__global__ __launch_bounds__(256) void fp16_finish4_kernel(const float* part, int splits, long n,
                                                           const float* amax, float lr,
                                                           uint16_t* w, float* w_res, float* g_w) {
  const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i < n) fp16_finish_four(part, splits, n, i, amax, lr, w, w_res, g_w);
}

// One thread per word: bit j of word w is latent[32w + j] >= 0 (ullis_pack_latent_bits).
__global__ void pack_bits_kernel(const uint16_t* latent, long n, uint32_t* bits) {
  const long w = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long base = w * 32;
  if (base >= n) return;
  uint32_t packed = 0;
  for (int j = 0; j < 32; ++j) {
    const long i = base + j;
    if (i < n && latent_is_plus(latent[i])) packed |= 1u << j;
  }
  bits[w] = packed;
}

// bits_t[i*out + o] = bits[o*in + i]. Aligned path: one half-wave transposes a
// 32x32 bit block with 32 ballots.
__global__ void transpose_bits_aligned_kernel(const uint32_t* bits, long out, long in,
                                              uint32_t* bits_t) {
  const long blk = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // one block per half-wave
  transpose_bits_block(bits, out, in, bits_t, blk, blk < (out / 32) * (in / 32));
}

__global__ void transpose_bits_generic_kernel(const uint32_t* bits, long out, long in,
                                              uint32_t* bits_t) {
  const long w = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long n = out * in;
  const long base = w * 32;
  if (base >= n) return;
  uint32_t packed = 0;
  for (int j = 0; j < 32; ++j) {
    const long t = base + j;
    if (t >= n) break;
    const long i = t / out, o = t % out;
    const long src = o * in + i;
    if ((bits[src >> 5] >> (src & 31)) & 1u) packed |= 1u << j;
  }
  bits_t[w] = packed;
}

}  // namespace

// ------------------------------------------------------------------ packed

hipError_t packed_forward(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                          const uint32_t* bits, const uint16_t* scale, const uint16_t* bias,
                          const PackedFwdOut& o) {
  if (o.sign_bits && out % 32 != 0) return hipErrorInvalidValue;
  const int mask = (o.y32 ? kOutY32 : 0) | (o.y32 && o.resid ? kOutResid : 0) |
                   (o.y16 ? kOutY16 : 0) | (o.relu2_16 ? kOutRelu2 : 0) |
                   (o.sign_bits ? kOutBits : 0);
  if (packed_gemv_ok(rows, in, out, x, x_dtype, o)) {
    switch (mask) {
      case kOutY32:
      case kOutY16:
      case kOutY32 | kOutY16:
      case kOutY32 | kOutResid:
      case kOutY16 | kOutRelu2:
        return packed_gemv(s, x, x_dtype, rows, in, out, bits, scale, bias, o);
      default:
        return hipErrorInvalidValue;
    }
  }
  auto run = [&](auto out_tag) {
    constexpr int OUT = decltype(out_tag)::value;
    EpiPackedFwd<OUT> epi{scale, bias, o};
    hipError_t err = hipSuccess;
    // very large products: 256x256 tiles over sign bits expanded once per
    // stage in LDS
    if (x_dtype == kF16 && lds::mk_ok(x, in) && lds::giant_ok(rows, out, in)) {
      lds::OpMK<lds::LdsGiant::bm, lds::LdsGiant::bk> a{static_cast<const half_t*>(x), in,
                                                        (int)rows};
      lds::OpBitsX<lds::LdsGiant::bn, lds::LdsGiant::bk> b{bits, in / 32, (int)out};
      return lds::launch_lds<lds::LdsGiant>(s, a, b, epi, rows, out, in, 1);
    }
    if (x_dtype == kF16 && lds::mk_ok(x, in) &&
        lds::with_lds(rows, out, in, 1, &err, [&](auto t) {
          using T = decltype(t);
          lds::OpMK<T::bm, T::bk> a{static_cast<const half_t*>(x), in, (int)rows};
          lds::OpBits<T::bn, T::bk, false> b{bits, in / 32, (int)out, nullptr, 0};
          return lds::launch_lds<T>(s, a, b, epi, rows, out, in, 1);
        }))
      return err;
    return with_tile(rows, out, [&](auto t) {
      using T = decltype(t);
      LoadBits<T::bn, T::bk> lb{bits, in, 0, nullptr, bits_aligned(in, 0, nullptr)};
      if (x_dtype == kF16) {
        LoadF16K<T::bm, T::bk> la{static_cast<const half_t*>(x), in, vec_ok_f16(x, in)};
        return launch_gemm<T>(s, la, lb, epi, rows, out, in, 1);
      }
      LoadF32K<T::bm, T::bk> la{static_cast<const float*>(x), in, vec_ok_f32(x, in), nullptr,
                                1.0f};
      return launch_gemm<T>(s, la, lb, epi, rows, out, in, 1);
    });
  };
  switch (mask) {
    case kOutY32: return run(std::integral_constant<int, kOutY32>{});
    case kOutY16: return run(std::integral_constant<int, kOutY16>{});
    case kOutY32 | kOutY16: return run(std::integral_constant<int, kOutY32 | kOutY16>{});
    case kOutY32 | kOutResid: return run(std::integral_constant<int, kOutY32 | kOutResid>{});
    case kOutY16 | kOutRelu2: return run(std::integral_constant<int, kOutY16 | kOutRelu2>{});
    case kOutBits: return run(std::integral_constant<int, kOutBits>{});
    default: return hipErrorInvalidValue;
  }
}

hipError_t packed_forward_bits3(hipStream_t s, const uint16_t* const x[3], long rows, long in,
                               long out, const uint32_t* const bits[3],
                               const uint16_t* const scale[3], const uint16_t* const bias[3],
                               uint32_t* const sign_bits[3]) {
  if (out % 32 != 0) return hipErrorInvalidValue;
  bool lds_ok = true;
  for (int j = 0; j < 3; ++j) lds_ok = lds_ok && lds::mk_ok(x[j], in);
  hipError_t err = hipSuccess;
  if (lds_ok && lds::with_lds(rows, out, in, 1, &err, [&](auto t) {
        using T = decltype(t);
        lds::Group<lds::OpMK<T::bm, T::bk>, 3> a;
        lds::Group<lds::OpBits<T::bn, T::bk, false>, 3> b;
        lds::Group<EpiPackedFwd<kOutBits>, 3> e;
        for (int j = 0; j < 3; ++j) {
          a.v[j] = {reinterpret_cast<const half_t*>(x[j]), in, (int)rows};
          b.v[j] = {bits[j], in / 32, (int)out, nullptr, 0};
          PackedFwdOut o;
          o.sign_bits = sign_bits[j];
          e.v[j] = {scale[j], bias[j], o};
        }
        return lds::launch_lds_group<T>(s, a, b, e, rows, out, in);
      }))
    return err;
  for (int j = 0; j < 3; ++j) {
    PackedFwdOut o;
    o.sign_bits = sign_bits[j];
    if ((err = packed_forward(s, x[j], kF16, rows, in, out, bits[j], scale[j], bias[j], o)) !=
        hipSuccess)
      return err;
  }
  return hipSuccess;
}

namespace {

// Streamed-LDS problems of the backward GEMMs: each calls f(problem) and
// returns true when the operands allow the LDS kernels (false: f not called).
long ldgy_of(const PackedDxArgs& d) { return d.ldgy ? d.ldgy : d.out; }
long ldb_of(const PackedDxArgs& d) { return d.ldb ? d.ldb : d.out; }

template <class F>
bool packed_dx_lds(const PackedDxArgs& d, hipError_t* err, F&& f) {
  const uint16_t* g16 = d.gy16 ? d.gy16 : d.gy32.p16;
  const long ldgy = ldgy_of(d), ldb = ldb_of(d);
  // the scaled-bits operand keeps the scales of the block's k range in LDS
  if (!lds::mk_ok(g16, ldgy) || d.out > 8192 || ldb % 32 != 0 || d.kofs % 32 != 0) return false;
  EpiStoreF32 epi{d.gx, d.gy32.amax, d.out_mul, d.accumulate};
  return lds::with_lds(d.rows, d.in, d.out, 1, err, [&](auto t) {
    using T = decltype(t);
    lds::OpMK<T::bm, T::bk> a{reinterpret_cast<const half_t*>(g16), ldgy, (int)d.rows};
    lds::OpBits<T::bn, T::bk, true> b{d.bits_t, ldb / 32, (int)d.in, d.scale, (int)d.kofs};
    if (d.col_part)
      return f(lds::lds_problem<T>(a, b, EpiSignedColSum{d.gy32.amax, d.sign_idx, d.col_part},
                                   d.rows, d.in, d.out, 1));
    return f(lds::lds_problem<T>(a, b, epi, d.rows, d.in, d.out, 1));
  });
}

template <class F>
bool weight_grad_lds(const WeightGradArgs& d, hipError_t* err, F&& f) {
  // G[out][in]: M = out, N = in, K = rows; both operands are row-contiguous.
  const uint16_t* g16 = d.gy16 ? d.gy16 : d.gy32.p16;
  if (!lds::km_ok(g16, d.out, d.out) || !lds::km_ok(d.x16, d.in, d.in)) return false;
  EpiPartial epi{d.part};
  return lds::with_lds(d.out, d.in, d.rows, d.splits, err, [&](auto t) {
    using T = decltype(t);
    lds::OpKM<T::bm, T::bk> a{reinterpret_cast<const half_t*>(g16), d.out, (int)d.out};
    lds::OpKM<T::bn, T::bk> b{reinterpret_cast<const half_t*>(d.x16), d.in, (int)d.in};
    return f(lds::lds_problem<T>(a, b, epi, d.out, d.in, d.rows, d.splits));
  });
}

template <class F>
bool fp16_dx_lds(const Fp16DxArgs& d, hipError_t* err, F&& f) {
  // gX[rows][in] = gY[rows][out] . W[out][in]: B(n = i, k = o) = W[o*in + i].
  if (!lds::mk_ok(d.gy32.p16, d.out) || !lds::km_ok(d.w, d.in, d.in)) return false;
  return lds::with_lds(d.rows, d.in, d.out, 1, err, [&](auto t) {
    using T = decltype(t);
    lds::OpMK<T::bm, T::bk> a{reinterpret_cast<const half_t*>(d.gy32.p16), d.out, (int)d.rows};
    lds::OpKM<T::bn, T::bk> b{reinterpret_cast<const half_t*>(d.w), d.in, (int)d.in};
    if (d.gk16)
      return f(lds::lds_problem<T>(a, b, EpiRelu2Bwd{d.key16, d.gk16}, d.rows, d.in, d.out, 1));
    return f(lds::lds_problem<T>(a, b, EpiStoreF32{d.gx, d.gy32.amax, nullptr, 0}, d.rows, d.in,
                                 d.out, 1));
    // 128x128 tiles: 256 blocks next to the weight gradient's in the pair
    // launch (measured 33.3 -> 25.3 us for the pair against 64x64 tiles)
  }, lds::LdsPolicy::kBig);
}

auto launch_one(hipStream_t s) {
  return [s](const auto& p) { return lds::launch_lds_problem(s, p); };
}

}  // namespace

// gx (+)= gy . (scale * S) over the window of PackedDxArgs.
hipError_t packed_dx(hipStream_t s, const PackedDxArgs& d) {
  if (d.col_part && (d.out_mul || d.accumulate || !d.sign_idx)) return hipErrorInvalidValue;
  hipError_t err = hipSuccess;
  if (packed_dx_lds(d, &err, launch_one(s))) return err;
  if (d.col_part) {
    // store gx, then the signed column sums over it
    PackedDxArgs st = d;
    st.col_part = nullptr;
    if ((err = packed_dx(s, st)) != hipSuccess) return err;
    return column_sum_partials(s, d.gx, d.sign_idx, d.rows, d.in, d.col_part, nullptr);
  }
  const long ldgy = ldgy_of(d), ldb = ldb_of(d);
  EpiStoreF32 epi{d.gx, d.gy32.amax, d.out_mul, d.accumulate};
  return with_tile(d.rows, d.in, [&](auto t) {
    using T = decltype(t);
    LoadBits<T::bn, T::bk, true> lb{d.bits_t, ldb, d.kofs, d.scale,
                                    bits_aligned(ldb, d.kofs, d.scale)};
    if (d.gy16) {
      LoadF16K<T::bm, T::bk> la{reinterpret_cast<const half_t*>(d.gy16), ldgy,
                                vec_ok_f16(d.gy16, ldgy)};
      return launch_gemm<T>(s, la, lb, epi, d.rows, d.in, d.out, 1);
    }
    LoadF32K<T::bm, T::bk> la{d.gy32.p, ldgy, vec_ok_f32(d.gy32.p, ldgy), d.gy32.amax, 1.0f};
    return launch_gemm<T>(s, la, lb, epi, d.rows, d.in, d.out, 1);
  });
}

hipError_t packed_backward_input(hipStream_t s, GradIn gy32, const uint16_t* gy16, long rows,
                                 long in, long out, const uint32_t* bits_t, const uint16_t* scale,
                                 float* gx, const float* out_mul, int accumulate) {
  return packed_dx(s, PackedDxArgs{gy32, gy16, rows, in, out, bits_t, scale, gx, out_mul,
                                   accumulate});
}

// Input gradient over a column window of the output features: contraction
// over k in [kofs, kofs + k_len) of a bits_t matrix with ldb bits per row, gy
// fp16 [rows][ldgy] holding only that window (unscaled), scale indexed kofs + k.
hipError_t packed_backward_input_ex(hipStream_t s, const uint16_t* gy16, long ldgy, long rows,
                                    long in, long k_len, const uint32_t* bits_t, long ldb,
                                    long kofs, const uint16_t* scale, float* gx,
                                    const float* out_mul, int accumulate) {
  return packed_dx(s, PackedDxArgs{GradIn{nullptr, nullptr}, gy16, rows, in, k_len, bits_t, scale,
                                   gx, out_mul, accumulate, ldgy, ldb, kofs});
}

hipError_t packed_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* gy16,
                                       const uint16_t* x16, long rows, long in, long out,
                                       int splits, float* part) {
  EpiPartial epi{part};
  hipError_t err = hipSuccess;
  if (weight_grad_lds(WeightGradArgs{gy32, gy16, x16, rows, in, out, splits, part}, &err,
                      launch_one(s)))
    return err;
  return with_tile(out, in, [&](auto t) {
    using T = decltype(t);
    LoadF16T<T::bn, T::bk> lb{reinterpret_cast<const half_t*>(x16), in, vec_ok_f16(x16, in)};
    if (gy16) {
      LoadF16T<T::bm, T::bk> la{reinterpret_cast<const half_t*>(gy16), out, vec_ok_f16(gy16, out)};
      return launch_gemm<T>(s, la, lb, epi, out, in, rows, splits);
    }
    LoadF32T<T::bm, T::bk> la{gy32.p, out, vec_ok_f32(gy32.p, out), gy32.amax, 1.0f};
    return launch_gemm<T>(s, la, lb, epi, out, in, rows, splits);
  });
}

bool packed_finish_wave_ok(const PackedFinish& f) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  return f.in % 32 == 0 && a16(f.part) && (!f.latent || (a16(f.latent) && a16(f.latent_res))) &&
         (!f.g_w || a16(f.g_w));
}

bool fp16_finish_vec_ok(const float* part, long n, const uint16_t* w, const float* w_res,
                        const float* g_w) {
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & m) == 0; };
  return n % 4 == 0 && al(part, 15u) && (!w || (al(w, 7u) && al(w_res, 15u))) &&
         (!g_w || al(g_w, 15u));
}

hipError_t packed_weight_finish(hipStream_t s, const PackedFinish& f) {
  if (f.out <= 0 || f.in <= 0) return hipSuccess;
  const bool wave = packed_finish_wave_ok(f);
  if (f.bits_new && (!f.latent || (!wave && f.in % 64 != 0))) return hipErrorInvalidValue;
  if (f.scale_upd && !f.scale_res) return hipErrorInvalidValue;
  if (wave)
    launch(packed_finish_wave_kernel, dim3((unsigned)finish_job_blocks(f.out)), dim3(256), 0, s, f);
  else
    launch(packed_finish_kernel, dim3((unsigned)f.out), dim3(256), 0, s, f);
  return hipGetLastError();
}

hipError_t pack_latent_bits(hipStream_t s, const uint16_t* latent, long out, long in,
                            uint32_t* bits, uint32_t* bits_t) {
  const long n = out * in;
  if (n <= 0) return hipSuccess;
  const long words = cdiv(n, 32);
  launch(pack_bits_kernel, dim3((unsigned)cdiv(words, 256)), dim3(256), 0, s, latent,
                     n, bits);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bits_t) return e;
  return transpose_bits(s, bits, out, in, bits_t);
}

hipError_t transpose_bits(hipStream_t s, const uint32_t* bits, long out, long in,
                          uint32_t* bits_t) {
  const long n = out * in;
  if (n <= 0) return hipSuccess;
  if (out % 32 == 0 && in % 32 == 0) {
    const long blocks32 = (out / 32) * (in / 32);
    const long threads = blocks32 * 32;
    launch(transpose_bits_aligned_kernel, dim3((unsigned)cdiv(threads, 256)),
                       dim3(256), 0, s, bits, out, in, bits_t);
  } else {
    launch(transpose_bits_generic_kernel, dim3((unsigned)cdiv(cdiv(n, 32), 256)),
                       dim3(256), 0, s, bits, out, in, bits_t);
  }
  return hipGetLastError();
}

// -------------------------------------------------------------------- fp16

hipError_t fp16_forward(hipStream_t s, const void* x, int x_dtype, long rows, long in, long out,
                        const uint16_t* w, float* y32, const float* resid, uint16_t* y16) {
  if (fp16_gemv_ok(rows, in, out, x, x_dtype, w) && (!resid || y32))
    return fp16_gemv(s, x, x_dtype, rows, in, out, w, y32, resid, y16);
  EpiF16Fwd epi{y32, resid, y16};
  hipError_t err = hipSuccess;
  if (x_dtype == kF16 && lds::mk_ok(x, in) && lds::mk_ok(w, in) &&
      lds::with_lds(rows, out, in, 1, &err, [&](auto t) {
        using T = decltype(t);
        lds::OpMK<T::bm, T::bk> a{static_cast<const half_t*>(x), in, (int)rows};
        lds::OpMK<T::bn, T::bk> b{reinterpret_cast<const half_t*>(w), in, (int)out};
        return lds::launch_lds<T>(s, a, b, epi, rows, out, in, 1);
        // one block per CU at heron sizes, reading an operand fresh from HBM:
        // the four-stage ring (measured 18.9 -> 15.2 us in the step)
      }, lds::LdsPolicy::kDeepGiant))
    return err;
  return with_tile(rows, out, [&](auto t) {
    using T = decltype(t);
    LoadF16K<T::bn, T::bk> lb{reinterpret_cast<const half_t*>(w), in, vec_ok_f16(w, in)};
    if (x_dtype == kF16) {
      LoadF16K<T::bm, T::bk> la{static_cast<const half_t*>(x), in, vec_ok_f16(x, in)};
      return launch_gemm<T>(s, la, lb, epi, rows, out, in, 1);
    }
    LoadF32K<T::bm, T::bk> la{static_cast<const float*>(x), in, vec_ok_f32(x, in), nullptr, 1.0f};
    return launch_gemm<T>(s, la, lb, epi, rows, out, in, 1);
  });
}

hipError_t fp16_backward_input(hipStream_t s, GradIn gy32, long rows, long in, long out,
                               const uint16_t* w, float* gx, const uint16_t* key16,
                               uint16_t* gk16) {
  hipError_t err = hipSuccess;
  if (fp16_dx_lds(Fp16DxArgs{gy32, rows, in, out, w, gx, key16, gk16}, &err, launch_one(s)))
    return err;
  return with_tile(rows, in, [&](auto t) {
    using T = decltype(t);
    LoadF32K<T::bm, T::bk> la{gy32.p, out, vec_ok_f32(gy32.p, out), gy32.amax, 1.0f};
    LoadF16T<T::bn, T::bk> lb{reinterpret_cast<const half_t*>(w), in, vec_ok_f16(w, in)};
    if (gk16) {
      EpiRelu2Bwd epi{key16, gk16};
      return launch_gemm<T>(s, la, lb, epi, rows, in, out, 1);
    }
    EpiStoreF32 epi{gx, gy32.amax, nullptr, 0};
    return launch_gemm<T>(s, la, lb, epi, rows, in, out, 1);
  });
}

hipError_t fp16_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* x16, long rows,
                                     long in, long out, int splits, float* part) {
  return packed_weight_grad_partials(s, gy32, nullptr, x16, rows, in, out, splits, part);
}

// Both GEMMs of a backward in one launch when both take the streamed-LDS path
// (their blocks share the CUs); otherwise the two separate launches.
hipError_t packed_backward_pair(hipStream_t s, const PackedDxArgs& dx, const WeightGradArgs& dw) {
  hipError_t err = hipSuccess;
  bool dw_ok = false;
  if (packed_dx_lds(dx, &err, [&](const auto& p1) {
        hipError_t e2 = hipSuccess;
        dw_ok = weight_grad_lds(dw, &e2, [&](const auto& p2) {
          return lds::launch_lds_pair(s, p1, p2);
        });
        return dw_ok ? e2 : hipSuccess;
      }) &&
      dw_ok)
    return err;
  if ((err = packed_dx(s, dx)) != hipSuccess) return err;
  return packed_weight_grad_partials(s, dw.gy32, dw.gy16, dw.x16, dw.rows, dw.in, dw.out,
                                     dw.splits, dw.part);
}

hipError_t fp16_backward_pair(hipStream_t s, const Fp16DxArgs& dx, const WeightGradArgs& dw) {
  hipError_t err = hipSuccess;
  bool dw_ok = false;
  if (fp16_dx_lds(dx, &err, [&](const auto& p1) {
        hipError_t e2 = hipSuccess;
        dw_ok = weight_grad_lds(dw, &e2, [&](const auto& p2) {
          return lds::launch_lds_pair(s, p1, p2);
        });
        return dw_ok ? e2 : hipSuccess;
      }) &&
      dw_ok)
    return err;
  if ((err = fp16_backward_input(s, dx.gy32, dx.rows, dx.in, dx.out, dx.w, dx.gx, dx.key16,
                                 dx.gk16)) != hipSuccess)
    return err;
  return packed_weight_grad_partials(s, dw.gy32, dw.gy16, dw.x16, dw.rows, dw.in, dw.out,
                                     dw.splits, dw.part);
}

hipError_t fp16_weight_finish(hipStream_t s, const float* part, int splits, long out, long in,
                              const float* amax, float lr, uint16_t* w, float* w_res,
                              float* g_w) {
  const long n = out * in;
  if (n <= 0) return hipSuccess;
  if (fp16_finish_vec_ok(part, n, w, w_res, g_w))
    launch(fp16_finish4_kernel, dim3((unsigned)f16_job_blocks(n)), dim3(256), 0, s, part, splits,
           n, amax, lr, w, w_res, g_w);
  else
    launch(fp16_finish_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, part, splits, n,
           amax, lr, w, w_res, g_w);
  return hipGetLastError();
}

}  // namespace ullis
