// Shared pieces of the packed +-1 and FP16 linear translation units
// (linear.hip: forwards and parameter finishes; linear_bwd.hip: input- and
// weight-gradient products): tile helpers, GEMM epilogues and the
// streamed-LDS problem builders of the backward products.
//
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
#pragma once


#include "context.hpp"
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
  // the residual segment of a row16 call, loaded ahead (epilogue_rows)
  struct Pre {
    floatx4 r[4];
    bool ok;
  };
  __device__ __forceinline__ Pre pre16(int row, int col, int M, int N) const {
    Pre p;
    p.ok = y32 && resid && row < M && col + 16 <= N && N % 8 == 0 && lds::al16(y32) &&
           lds::al16(resid);
    if (p.ok) {
      const floatx4* src = reinterpret_cast<const floatx4*>(resid + (long)row * N + col);
#pragma unroll
      for (int q = 0; q < 4; ++q) p.r[q] = src[q];
    }
    return p;
  }
  __device__ void row16p(int row, int col, float (&v)[16], const Pre& p, int lane, int M, int N,
                         float* buf, int brow, int bcol) {
    if (!p.ok) {
      row16(row, col, v, lane, M, N, buf, brow, bcol);
      return;
    }
    const long idx = (long)row * N + col;
    float z[16];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) z[4 * q + e] = p.r[q][e] + v[4 * q + e];
    lds::store16f(y32 + idx, z);
    if (y16) {
      if (lds::al16(y16)) {
        lds::store16h(y16 + idx, v);
      } else {
        for (int k = 0; k < 16; ++k) y16[idx + k] = __builtin_bit_cast(uint16_t, (half_t)v[k]);
      }
    }
  }
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
  // the key tape's segment of a row16 call, loaded ahead (epilogue_rows)
  struct Pre {
    half8 k[2];
    bool ok;
  };
  __device__ __forceinline__ Pre pre16(int row, int col, int M, int N) const {
    Pre p;
    p.ok = row < M && col + 16 <= N && N % 8 == 0 && lds::al16(key16) && lds::al16(gk16);
    if (p.ok) {
      const half8* src = reinterpret_cast<const half8*>(key16 + (long)row * N + col);
      p.k[0] = src[0];
      p.k[1] = src[1];
    }
    return p;
  }
  __device__ void row16p(int row, int col, float (&v)[16], const Pre& p, int lane, int M, int N,
                         float* buf, int brow, int bcol) {
    if (!p.ok) {
      row16(row, col, v, lane, M, N, buf, brow, bcol);
      return;
    }
    float gk[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float k = (float)p.k[e >> 3][e & 7];
      const float t = k > 0.0f ? 2.0f * k * v[e] : 0.0f;
      gk[e] = clamp_f16_range(t);  // as f32_to_f16_sat
    }
    lds::store16h(gk16 + (long)row * N + col, gk);
  }
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
      gk[e] = clamp_f16_range(t);  // as f32_to_f16_sat
    }
    if (full) {
      lds::store16h(gk16 + idx, gk);
    } else {
      for (int e = 0; e < 16 && col + e < N; ++e)
        gk16[idx + e] = __builtin_bit_cast(uint16_t, (half_t)gk[e]);
    }
  }
};

}  // namespace

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
  // very large products: 256x256 tiles over the scaled sign bits expanded in
  // LDS, on the interleaved K loop
  if (lds::giant_ok(d.rows, d.in, d.out) && d.out % lds::LdsGiantBits::bk == 0) {
    using T = lds::LdsGiantBits;
    lds::OpMK<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(g16), ldgy, (int)d.rows};
    lds::OpBitsX<T::bn, T::bk, T::nw, true> b{d.bits_t, ldb / 32, (int)d.in, d.scale,
                                              (int)d.kofs};
    if (d.col_part)
      *err = f(lds::lds_problem<T>(a, b, EpiSignedColSum{d.gy32.amax, d.sign_idx, d.col_part},
                                   d.rows, d.in, d.out, 1));
    else
      *err = f(lds::lds_problem<T>(a, b, epi, d.rows, d.in, d.out, 1));
    return true;
  }
  return lds::with_lds(d.rows, d.in, d.out, 1, err, [&](auto t) {
    using T = decltype(t);
    lds::OpMK<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(g16), ldgy, (int)d.rows};
    lds::OpBits<T::bn, T::bk, true, T::nw> b{d.bits_t, ldb / 32, (int)d.in, d.scale, (int)d.kofs};
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
  if (dw_giant(d.out, d.in, d.rows) && d.rows % (lds::LdsGiant8::bk * d.splits) == 0) {
    using T = lds::LdsGiant8;
    lds::OpKM<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(g16), d.out, (int)d.out};
    lds::OpKM<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(d.x16), d.in, (int)d.in};
    *err = f(lds::lds_problem<T>(a, b, epi, d.out, d.in, d.rows, d.splits));
    return true;
  }
  return lds::with_lds(d.out, d.in, d.rows, d.splits, err, [&](auto t) {
    using T = decltype(t);
    lds::OpKM<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(g16), d.out, (int)d.out};
    lds::OpKM<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(d.x16), d.in, (int)d.in};
    return f(lds::lds_problem<T>(a, b, epi, d.out, d.in, d.rows, d.splits));
  });
}

template <class F>
bool fp16_dx_lds(const Fp16DxArgs& d, hipError_t* err, F&& f) {
  // gX[rows][in] = gY[rows][out] . W[out][in]: B(n = i, k = o) = W[o*in + i],
  // or W^T[i*out + o] k-contiguous when given. With W^T, 128x256 eight-wave
  // tiles of two k-contiguous operands on the interleaved K loop: at config 5
  // the value backward pair took 969 us, against 995 us with four waves, 1136
  // us on 128x128 tiles and 1389 us with the transposed operand (256x256
  // tiles: 1752 us).
  if (d.w_t && lds::mk_ok(d.gy32.p16, d.out) && lds::mk_ok(d.w_t, d.out) &&
      d.out % lds::LdsHuge::bk == 0 && d.rows % lds::LdsHuge::bm == 0 &&
      d.in % lds::LdsHuge8::bn == 0) {
    using T = lds::LdsHuge8;
    lds::OpMK<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(d.gy32.p16), d.out, (int)d.rows};
    lds::OpMK<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(d.w_t), d.out, (int)d.in};
    if (d.gk16)
      *err = f(lds::lds_problem<T>(a, b, EpiRelu2Bwd{d.key16, d.gk16}, d.rows, d.in, d.out, 1));
    else
      *err = f(lds::lds_problem<T>(a, b, EpiStoreF32{d.gx, d.gy32.amax, nullptr, 0}, d.rows,
                                   d.in, d.out, 1));
    return true;
  }
  if (!lds::mk_ok(d.gy32.p16, d.out) || !lds::km_ok(d.w, d.in, d.in)) return false;
  return lds::with_lds(d.rows, d.in, d.out, 1, err, [&](auto t) {
    using T = decltype(t);
    lds::OpMK<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(d.gy32.p16), d.out, (int)d.rows};
    lds::OpKM<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(d.w), d.in, (int)d.in};
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
}  // namespace ullis
