// LayerNorm forward / backward (HBM-bound), one wave64 per row.
//
// Reference: LayerNorm::forward / backward, src/model.rs:259-316 (affine,
// population variance, eps = 1e-5, inv = 1/sqrt(var + eps)); the Metal kernels
// replaced are ullis_layer_norm, ullis_layer_norm_backward and
// ullis_layer_norm_param_bwd (src/metal/rwkv8.metal:154-269), which run one
// thread per row. Here a row is spread over the 64 lanes of a wave: each lane
// keeps its float4 chunks in registers and row sums are wave (DPP) reductions.
// gamma/beta gradients are column sums written as per-block partials and
// reduced in a fixed order by layer_norm_param_finish, so results do not
// depend on scheduling.
#include <type_traits>

#include "common.hpp"
#include "ops.hpp"

namespace ullis {

namespace {

constexpr int kRowsPerBlock = 4;

// LayerNorm of one row by one wave: lane holds channels [4 (lane + 64 j), +4)
// of chunk j (NV float4 chunks per lane, ch <= 256 * NV, ch % 4 == 0).
// With rr, the row normalised is xr + rr (fp32 sums), and sum_out (if set)
// receives it.
template <int NV>
__device__ __forceinline__ void ln_row_vec(const float* __restrict__ xr, int ch, int lane,
                                           const uint16_t* __restrict__ w,
                                           const uint16_t* __restrict__ b, floatx4 (&out)[NV],
                                           const float* __restrict__ rr = nullptr,
                                           float* __restrict__ sum_out = nullptr) {
  floatx4 v[NV];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    v[j] = c < ch ? *reinterpret_cast<const floatx4*>(xr + c) : (floatx4){};
    if (rr && c < ch) {
      const floatx4 r = *reinterpret_cast<const floatx4*>(rr + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] = r[e] + v[j][e];
      if (sum_out) *reinterpret_cast<floatx4*>(sum_out + c) = v[j];
    }
    s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  }
  const float mean = wave_sum(s) / (float)ch;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[j][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / (float)ch;
  const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[j][e] = (v[j][e] - mean) * inv * f16_bits_to_f32(w[c + e]) + f16_bits_to_f32(b[c + e]);
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void ln_fwd_vec_kernel(const float* __restrict__ x, long rows,
                                                         int ch, const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ b,
                                                         float* __restrict__ y32,
                                                         uint16_t* __restrict__ y16) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  floatx4 y[NV];
  ln_row_vec<NV>(x + row * ch, ch, lane, w, b, y);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
      const floatx4 o = y[j];
      if (y32) *reinterpret_cast<floatx4*>(y32 + row * ch + c) = o;
      if (y16) {
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (half_t)o[e];
        *reinterpret_cast<half4*>(y16 + row * ch + c) = h;
      }
    }
  }
}

// The arithmetic of ln_row_vec on a row whose chunks (x, or resid + x; zero
// past ch) and LayerNorm weights are already in registers.
template <int NV>
__device__ __forceinline__ void ln_row_regs(const floatx4 (&v)[NV], int ch, int lane,
                                            const half4 (&wv)[NV], const half4 (&bv)[NV],
                                            floatx4 (&out)[NV]) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  const float mean = wave_sum(s) / (float)ch;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[j][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / (float)ch;
  const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[j][e] = (v[j][e] - mean) * inv * (float)wv[j][e] + (float)bv[j][e];
    }
  }
}

// mix one 4-channel chunk with its mix vector in registers: out = f16(x +
// (prev - x) * mix), prev = 0 at t = 0 (time_shift_mix on the fp16 LayerNorm
// output).
__device__ __forceinline__ void mix4_store(const half4& x, const half4& p, const half4& m,
                                           uint16_t* out, long idx) {
  half4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float xt = (float)x[e];
    const float xx = (float)p[e] - xt;
    o[e] = (half_t)(xt + xx * (float)m[e]);
  }
  *reinterpret_cast<half4*>(out + idx) = o;
}

// LayerNorm fused with the time-shift mixes that read its fp16 output: each
// wave normalises its row and the previous row of the same sequence (the
// same per-row arithmetic as ln_fwd_vec_kernel), so out_i = mix_i of the
// fp16 rows without the LayerNorm output making a round trip through HBM.
// y16 (optional) also receives the fp16 LayerNorm output. With resid, the
// LayerNorm input is resid + x (a residual add), which sum_out receives.
// Every load of both rows, the LayerNorm weights and the mix vectors is
// issued before the first is used, so their round trips overlap instead of
// following one another (a row's chunks, then its weights, then the next
// row's).
template <int NV>
__global__ __launch_bounds__(256) void ln_mix_kernel(const float* __restrict__ x, long rows,
                                                     int time, int ch,
                                                     const uint16_t* __restrict__ w,
                                                     const uint16_t* __restrict__ b,
                                                     uint16_t* __restrict__ y16,
                                                     const uint16_t* mix0, uint16_t* out0,
                                                     const uint16_t* mix1, uint16_t* out1,
                                                     const uint16_t* mix2, uint16_t* out2,
                                                     const float* __restrict__ resid,
                                                     float* __restrict__ sum_out) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool has_prev = row % time != 0;  // uniform over the wave
  const long prow = has_prev ? row - 1 : row;
  floatx4 vc[NV], vp[NV];
  half4 wv[NV], bv[NV], m0[NV], m1[NV], m2[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    const int cc = c < ch ? c : 0;  // in bounds; chunks past ch are zeroed below
    vc[j] = *reinterpret_cast<const floatx4*>(x + row * ch + cc);
    vp[j] = *reinterpret_cast<const floatx4*>(x + prow * ch + cc);
    wv[j] = *reinterpret_cast<const half4*>(w + cc);
    bv[j] = *reinterpret_cast<const half4*>(b + cc);
    if (out0) m0[j] = *reinterpret_cast<const half4*>(mix0 + cc);
    if (out1) m1[j] = *reinterpret_cast<const half4*>(mix1 + cc);
    if (out2) m2[j] = *reinterpret_cast<const half4*>(mix2 + cc);
  }
  if (resid) {
    floatx4 rc[NV], rp[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 4;
      const int cc = c < ch ? c : 0;
      rc[j] = *reinterpret_cast<const floatx4*>(resid + row * ch + cc);
      rp[j] = *reinterpret_cast<const floatx4*>(resid + prow * ch + cc);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vc[j][e] = rc[j][e] + vc[j][e];
        vp[j][e] = rp[j][e] + vp[j][e];
      }
      const int c = (lane + 64 * j) * 4;
      if (sum_out && c < ch) *reinterpret_cast<floatx4*>(sum_out + row * ch + c) = vc[j];
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if ((lane + 64 * j) * 4 >= ch) vc[j] = vp[j] = (floatx4){};
  floatx4 cur[NV], prev[NV];
  ln_row_regs<NV>(vc, ch, lane, wv, bv, cur);
  if (has_prev) ln_row_regs<NV>(vp, ch, lane, wv, bv, prev);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
      half4 xh, ph;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[e] = (half_t)cur[j][e];
        ph[e] = has_prev ? (half_t)prev[j][e] : (half_t)0.0f;
      }
      const long idx = row * ch + c;
      if (y16) *reinterpret_cast<half4*>(y16 + idx) = xh;
      if (out0) mix4_store(xh, ph, m0[j], out0, idx);
      if (out1) mix4_store(xh, ph, m1[j], out1, idx);
      if (out2) mix4_store(xh, ph, m2[j], out2, idx);
    }
  }
}

// Any ch: two passes over global memory, lane-strided.
__global__ __launch_bounds__(256) void ln_fwd_any_kernel(const float* x, long rows, int ch,
                                                         const uint16_t* w, const uint16_t* b,
                                                         float* y32, uint16_t* y16) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * ch;
  float s = 0.0f;
  for (int c = lane; c < ch; c += 64) s += xr[c];
  const float mean = wave_sum(s) / (float)ch;
  float q = 0.0f;
  for (int c = lane; c < ch; c += 64) {
    const float d = xr[c] - mean;
    q += d * d;
  }
  const float var = wave_sum(q) / (float)ch;
  const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
  for (int c = lane; c < ch; c += 64) {
    const float o = (xr[c] - mean) * inv * f16_bits_to_f32(w[c]) + f16_bits_to_f32(b[c]);
    if (y32) y32[row * ch + c] = o;
    if (y16) y16[row * ch + c] = f32_to_f16_bits(o);
  }
}

// Backward, ch % 4 == 0 and ch <= 1024 (block LDS reduction of the column
// partials). Rows are distributed wave-strided over a fixed grid.
template <int NV>
__global__ __launch_bounds__(256) void ln_bwd_vec_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ gy, long rows,
                                                         int ch, const uint16_t* __restrict__ w,
                                                         float* gx, int accumulate, float* amax,
                                                         float* __restrict__ part) {
  __shared__ float red[kRowsPerBlock][2][1024];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  floatx4 pw[NV], pb[NV], wv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    pw[j] = (floatx4){};
    pb[j] = (floatx4){};
    const int c = (lane + 64 * j) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[j][e] = c < ch ? f16_bits_to_f32(w[c + e]) : 0.0f;
  }
  float local_max = 0.0f;
  for (long row = (long)blockIdx.x * kRowsPerBlock + wave; row < rows;
       row += (long)gridDim.x * kRowsPerBlock) {
    const float* xr = x + row * ch;
    const float* gr = gy + row * ch;
    floatx4 v[NV], g[NV];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 4;
      v[j] = c < ch ? *reinterpret_cast<const floatx4*>(xr + c) : (floatx4){};
      g[j] = c < ch ? *reinterpret_cast<const floatx4*>(gr + c) : (floatx4){};
      s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
    }
    const float mean = wave_sum(s) / (float)ch;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 4;
      if (c < ch) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = v[j][e] - mean;
          q += d * d;
        }
      }
    }
    const float var = wave_sum(q) / (float)ch;
    const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
    float sd = 0.0f, sdx = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xhat = (v[j][e] - mean) * inv;
        const float dxhat = g[j][e] * wv[j][e];
        v[j][e] = xhat;  // keep xhat
        sd += dxhat;
        sdx += dxhat * xhat;
        pw[j][e] += g[j][e] * xhat;
        pb[j][e] += g[j][e];
      }
    }
    const float sum_dxhat = wave_sum(sd);
    const float sum_dxhat_xhat = wave_sum(sdx);
    const float inv_n = inv / (float)ch;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 4;
      if (c < ch) {
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float dxhat = g[j][e] * wv[j][e];
          o[e] = inv_n * ((float)ch * dxhat - sum_dxhat - v[j][e] * sum_dxhat_xhat);
        }
        floatx4* dst = reinterpret_cast<floatx4*>(gx + row * ch + c);
        if (accumulate) {
          const floatx4 old = *dst;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = old[e] + o[e];
        }
        *dst = o;
#pragma unroll
        for (int e = 0; e < 4; ++e) local_max = __builtin_fmaxf(local_max, finite_abs(o[e]));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        red[wave][0][c + e] = pw[j][e];
        red[wave][1][c + e] = pb[j][e];
      }
    }
  }
  if (amax) {
    const float m = wave_max(local_max);
    if (lane == 0) atomic_amax(amax, m);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < ch; c += blockDim.x) {
    float a = 0.0f, bsum = 0.0f;
#pragma unroll
    for (int k = 0; k < kRowsPerBlock; ++k) {
      a += red[k][0][c];
      bsum += red[k][1][c];
    }
    part[((long)blockIdx.x * 2 + 0) * ch + c] = a;
    part[((long)blockIdx.x * 2 + 1) * ch + c] = bsum;
  }
}

// Backward, one row per wave (4 rows per block), ch % 4 == 0, ch <= 1024: all
// of a row's loads (x, gy and, when accumulating, the old gx) are issued
// before the first reduction, and the grid has one wave per row, so the
// memory latency of every row overlaps. Column partials per block as above.
// MIX: the output gradient gy is that of a time-shift mix's input, computed
// here from the mix's output gradient g_s (rows t, t + 1), its fp16 input
// x16 = this LayerNorm's output (rows t, t - 1) and the mix vector, with the
// arithmetic of time_shift_mix_bwd4_kernel; the mix-vector gradient goes to
// part_mix[block][ch] (the block's rows summed in order).
template <int NV, bool MIX = false>
__global__ __launch_bounds__(256) void ln_bwd_row_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ gy, long rows,
                                                         int ch, const uint16_t* __restrict__ w,
                                                         float* gx, int accumulate, float* amax,
                                                         float* __restrict__ part,
                                                         const uint16_t* __restrict__ x16 = nullptr,
                                                         const uint16_t* __restrict__ mix = nullptr,
                                                         int time = 1,
                                                         float* __restrict__ part_mix = nullptr) {
  constexpr int kParts = MIX ? 3 : 2;
  __shared__ float red[kRowsPerBlock][kParts][1024];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long row = (long)blockIdx.x * kRowsPerBlock + wave;
  const bool live = row < rows;
  // Loads go to in-bounds addresses unconditionally (a dead wave reads the
  // last row, a chunk past ch reads chunk 0, a missing neighbour row reads
  // the row itself) and the values are selected afterwards, so no load waits
  // behind a branch.
  const long lrow = live ? row : rows - 1;
  floatx4 v[NV], g[NV], old[NV], wv[NV], gmix[NV];
  const int t = MIX ? (int)(lrow % time) : 0;
  const bool has_next = t + 1 < time;
  const long prow = t > 0 ? lrow - 1 : lrow;
  const long nrow = has_next ? lrow + 1 : lrow;
  floatx4 xv[NV], gv[NV], nv[NV];
  half4 xh[NV], ph[NV], mv[NV], wh[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    const int cc = c < ch ? c : 0;
    xv[j] = *reinterpret_cast<const floatx4*>(x + lrow * ch + cc);
    gv[j] = *reinterpret_cast<const floatx4*>(gy + lrow * ch + cc);
    wh[j] = *reinterpret_cast<const half4*>(w + cc);
    if constexpr (MIX) {
      nv[j] = *reinterpret_cast<const floatx4*>(gy + nrow * ch + cc);
      xh[j] = *reinterpret_cast<const half4*>(x16 + lrow * ch + cc);
      ph[j] = *reinterpret_cast<const half4*>(x16 + prow * ch + cc);
      mv[j] = *reinterpret_cast<const half4*>(mix + cc);
    }
  }
  if (accumulate) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 4;
      old[j] = *reinterpret_cast<const floatx4*>(gx + lrow * ch + (c < ch ? c : 0));
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    const bool ok = live && c < ch;
    v[j] = ok ? xv[j] : (floatx4){};
    if constexpr (MIX) {
      const floatx4 gs = ok ? gv[j] : (floatx4){};
      const floatx4 gn = ok && has_next ? nv[j] : (floatx4){};
      const half4 xo = ok ? xh[j] : (half4){};
      const half4 po = ok && t > 0 ? ph[j] : (half4){};
      const half4 m = ok ? mv[j] : (half4){};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xt = (float)xo[e];
        const float xx = (t == 0 ? 0.0f : (float)po[e]) - xt;
        const float mm = (float)m[e];
        gmix[j][e] = gs[e] * xx;
        float gb = gs[e] - gs[e] * mm;
        if (has_next) gb = gb + gn[e] * mm;
        g[j][e] = gb;
      }
    } else {
      g[j] = ok ? gv[j] : (floatx4){};
    }
    if (!(ok && accumulate)) old[j] = (floatx4){};
    const half4 wo = c < ch ? wh[j] : (half4){};
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[j][e] = (float)wo[e];
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  const float mean = wave_sum(s) / (float)ch;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (c < ch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[j][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / (float)ch;
  const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
  float sd = 0.0f, sdx = 0.0f;
  floatx4 pw[NV], pb[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xhat = (v[j][e] - mean) * inv;
      const float dxhat = g[j][e] * wv[j][e];
      v[j][e] = xhat;
      sd += dxhat;
      sdx += dxhat * xhat;
      pw[j][e] = g[j][e] * xhat;
      pb[j][e] = g[j][e];
    }
  }
  const float sum_dxhat = wave_sum(sd);
  const float sum_dxhat_xhat = wave_sum(sdx);
  const float inv_n = inv / (float)ch;
  float local_max = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 4;
    if (live && c < ch) {
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dxhat = g[j][e] * wv[j][e];
        o[e] = inv_n * ((float)ch * dxhat - sum_dxhat - v[j][e] * sum_dxhat_xhat);
        if (accumulate) o[e] = old[j][e] + o[e];
        local_max = __builtin_fmaxf(local_max, finite_abs(o[e]));
      }
      *reinterpret_cast<floatx4*>(gx + row * ch + c) = o;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c < ch) {
        red[wave][0][c + e] = pw[j][e];
        red[wave][1][c + e] = pb[j][e];
        if constexpr (MIX) red[wave][kParts - 1][c + e] = live ? gmix[j][e] : 0.0f;
      }
  }
  __shared__ float wmax[kRowsPerBlock];
  if (amax) {
    const float m = wave_max(local_max);
    if (lane == 0) wmax[wave] = m;
  }
  __syncthreads();
  if (amax && threadIdx.x == 0) {
    float m = wmax[0];
#pragma unroll
    for (int k = 1; k < kRowsPerBlock; ++k) m = __builtin_fmaxf(m, wmax[k]);
    atomic_amax(amax, m);
  }
  for (int c = threadIdx.x; c < ch; c += blockDim.x) {
    float a = 0.0f, bsum = 0.0f;
#pragma unroll
    for (int k = 0; k < kRowsPerBlock; ++k) {
      a += red[k][0][c];
      bsum += red[k][1][c];
    }
    part[((long)blockIdx.x * 2 + 0) * ch + c] = a;
    part[((long)blockIdx.x * 2 + 1) * ch + c] = bsum;
    if constexpr (MIX) {
      float mg = 0.0f;
#pragma unroll
      for (int k = 0; k < kRowsPerBlock; ++k) mg += red[k][kParts - 1][c];
      part_mix[(long)blockIdx.x * ch + c] = mg;
    }
  }
}

// Any ch: one wave per (block, row slot); per-wave partials (block = 1 wave).
__global__ __launch_bounds__(64) void ln_bwd_any_kernel(const float* x, const float* gy, long rows,
                                                        int ch, const uint16_t* w, float* gx,
                                                        int accumulate, float* amax, float* part) {
  const int lane = threadIdx.x & 63;
  float local_max = 0.0f;
  float* pw = part + ((long)blockIdx.x * 2 + 0) * ch;
  float* pb = part + ((long)blockIdx.x * 2 + 1) * ch;
  for (int c = lane; c < ch; c += 64) {
    pw[c] = 0.0f;
    pb[c] = 0.0f;
  }
  for (long row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * ch;
    const float* gr = gy + row * ch;
    float s = 0.0f;
    for (int c = lane; c < ch; c += 64) s += xr[c];
    const float mean = wave_sum(s) / (float)ch;
    float q = 0.0f;
    for (int c = lane; c < ch; c += 64) {
      const float d = xr[c] - mean;
      q += d * d;
    }
    const float var = wave_sum(q) / (float)ch;
    const float inv = 1.0f / __builtin_sqrtf(var + kLayerNormEps);
    float sd = 0.0f, sdx = 0.0f;
    for (int c = lane; c < ch; c += 64) {
      const float xhat = (xr[c] - mean) * inv;
      const float dxhat = gr[c] * f16_bits_to_f32(w[c]);
      sd += dxhat;
      sdx += dxhat * xhat;
      pw[c] += gr[c] * xhat;
      pb[c] += gr[c];
    }
    const float sum_dxhat = wave_sum(sd);
    const float sum_dxhat_xhat = wave_sum(sdx);
    const float inv_n = inv / (float)ch;
    for (int c = lane; c < ch; c += 64) {
      const float xhat = (xr[c] - mean) * inv;
      const float dxhat = gr[c] * f16_bits_to_f32(w[c]);
      float o = inv_n * ((float)ch * dxhat - sum_dxhat - xhat * sum_dxhat_xhat);
      if (accumulate) o = gx[row * ch + c] + o;
      gx[row * ch + c] = o;
      local_max = __builtin_fmaxf(local_max, finite_abs(o));
    }
  }
  if (amax) {
    const float m = wave_max(local_max);
    if (lane == 0) atomic_amax(amax, m);
  }
}

template <class F>
hipError_t by_nv(long ch, F&& f) {
  const long nv = cdiv(ch, 256);
  if (nv <= 1) return f(std::integral_constant<int, 1>{});
  if (nv <= 2) return f(std::integral_constant<int, 2>{});
  if (nv <= 4) return f(std::integral_constant<int, 4>{});
  if (nv <= 8) return f(std::integral_constant<int, 8>{});
  return f(std::integral_constant<int, 16>{});
}

inline bool vec_ok(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t layer_norm_forward(hipStream_t s, const float* x, long rows, long ch,
                              const uint16_t* w, const uint16_t* b, float* y32, uint16_t* y16) {
  if (rows <= 0 || ch <= 0) return hipSuccess;
  const dim3 grid((unsigned)cdiv(rows, kRowsPerBlock));
  const bool vec = ch % 4 == 0 && ch <= 4096 && vec_ok(x) && (!y32 || vec_ok(y32)) &&
                   (!y16 || (reinterpret_cast<uintptr_t>(y16) & 7u) == 0);
  if (vec) {
    return by_nv(ch, [&](auto nv) {
      launch(ln_fwd_vec_kernel<decltype(nv)::value>, grid, dim3(256), 0, s, x, rows,
                         (int)ch, w, b, y32, y16);
      return hipGetLastError();
    });
  }
  launch(ln_fwd_any_kernel, grid, dim3(256), 0, s, x, rows, (int)ch, w, b, y32, y16);
  return hipGetLastError();
}

hipError_t layer_norm_mix_forward(hipStream_t s, const float* x, long rows, long time, long ch,
                                  const uint16_t* w, const uint16_t* b, uint16_t* y16, bool keep_y,
                                  const uint16_t* mix0, uint16_t* out0, const uint16_t* mix1,
                                  uint16_t* out1, const uint16_t* mix2, uint16_t* out2,
                                  const float* resid, float* sum_out) {
  if (rows <= 0 || ch <= 0 || time <= 0) return hipSuccess;
  if (resid && !sum_out) return hipErrorInvalidValue;
  auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; };
  const bool fused = ch % 4 == 0 && ch <= 4096 && time <= INT32_MAX && vec_ok(x) && a8(y16) &&
                     (!out0 || (a8(out0) && a8(mix0))) && (!out1 || (a8(out1) && a8(mix1))) &&
                     (!out2 || (a8(out2) && a8(mix2))) &&
                     (!resid || (vec_ok(resid) && vec_ok(sum_out)));
  if (fused) {
    return by_nv(ch, [&](auto nv) {
      launch(ln_mix_kernel<decltype(nv)::value>, dim3((unsigned)cdiv(rows, kRowsPerBlock)),
             dim3(256), 0, s, x, rows, (int)time, (int)ch, w, b, keep_y ? y16 : nullptr, mix0,
             out0, mix1, out1, mix2, out2, resid, sum_out);
      return hipGetLastError();
    });
  }
  if (resid) {
    const hipError_t e = add_f32(s, resid, x, rows * ch, sum_out);
    if (e != hipSuccess) return e;
    x = sum_out;
  }
  hipError_t e = layer_norm_forward(s, x, rows, ch, w, b, nullptr, y16);
  if (e != hipSuccess) return e;
  return time_shift_mix(s, y16, rows, time, ch, mix0, out0, mix1, out1, mix2, out2);
}

static bool ln_bwd_vec_path(long ch) { return ch % 4 == 0 && ch <= 1024; }

// Blocks of the vector path (one row per wave) and of the any-ch path.
static bool ln_bwd_row_path(long rows, long ch) { return ln_bwd_vec_path(ch) && rows <= (1L << 20); }

static int ln_bwd_blocks_any(long rows) {
  long nblk = cdiv(rows, 2 * kRowsPerBlock);
  if (nblk > 256) nblk = 256;
  if (nblk < 1) nblk = 1;
  return (int)nblk;
}

int layer_norm_backward_nblk(long rows, long ch) {
  return ln_bwd_row_path(rows, ch) ? (int)cdiv(rows, kRowsPerBlock) : ln_bwd_blocks_any(rows);
}

int layer_norm_backward_blocks(long rows) {
  // Upper bound over both paths (sizes the partial buffers).
  long nblk = cdiv(rows, kRowsPerBlock);
  if (nblk < 256) nblk = 256;
  return (int)nblk;
}


hipError_t layer_norm_backward_rows(hipStream_t s, const float* x, const float* gy, long rows,
                                    long ch, const uint16_t* w, float* gx, int accumulate,
                                    float* amax, float* part, int* nblk_out) {
  if (rows <= 0 || ch <= 0) {
    if (nblk_out) *nblk_out = 0;
    return hipSuccess;
  }
  if (ln_bwd_row_path(rows, ch) && vec_ok(x) && vec_ok(gy) && vec_ok(gx) &&
      (reinterpret_cast<uintptr_t>(w) & 7u) == 0) {
    const int nblk = (int)cdiv(rows, kRowsPerBlock);
    if (nblk_out) *nblk_out = nblk;
    return by_nv(ch, [&](auto nv) {
      launch(ln_bwd_row_kernel<decltype(nv)::value>, dim3(nblk), dim3(256), 0, s, x, gy, rows,
             (int)ch, w, gx, accumulate, amax, part, (const uint16_t*)nullptr,
             (const uint16_t*)nullptr, 1, (float*)nullptr);
      return hipGetLastError();
    });
  }
  const int nblk = ln_bwd_blocks_any(rows);
  if (nblk_out) *nblk_out = nblk;
  if (ln_bwd_vec_path(ch) && vec_ok(x) && vec_ok(gy) && vec_ok(gx)) {
    return by_nv(ch, [&](auto nv) {
      launch(ln_bwd_vec_kernel<decltype(nv)::value>, dim3(nblk), dim3(256), 0, s, x,
                         gy, rows, (int)ch, w, gx, accumulate, amax, part);
      return hipGetLastError();
    });
  }
  launch(ln_bwd_any_kernel, dim3(nblk), dim3(64), 0, s, x, gy, rows, (int)ch, w, gx,
                     accumulate, amax, part);
  return hipGetLastError();
}

int layer_norm_backward_capped_nblk(long rows) { return ln_bwd_blocks_any(rows); }

hipError_t layer_norm_backward_rows_capped(hipStream_t s, const float* x, const float* gy,
                                           long rows, long ch, const uint16_t* w, float* gx,
                                           float* part, int* nblk_out) {
  if (rows <= 0 || ch <= 0) {
    if (nblk_out) *nblk_out = 0;
    return hipSuccess;
  }
  const int nblk = ln_bwd_blocks_any(rows);
  if (nblk_out) *nblk_out = nblk;
  if (ln_bwd_vec_path(ch) && vec_ok(x) && vec_ok(gy) && vec_ok(gx)) {
    return by_nv(ch, [&](auto nv) {
      launch(ln_bwd_vec_kernel<decltype(nv)::value>, dim3(nblk), dim3(256), 0, s, x, gy, rows,
             (int)ch, w, gx, 0, (float*)nullptr, part);
      return hipGetLastError();
    });
  }
  launch(ln_bwd_any_kernel, dim3(nblk), dim3(64), 0, s, x, gy, rows, (int)ch, w, gx, 0,
         (float*)nullptr, part);
  return hipGetLastError();
}

int layer_norm_mix_backward_mix_nblk(long rows, long ch) {
  return ln_bwd_row_path(rows, ch) ? (int)cdiv(rows, kRowsPerBlock) : (int)cdiv(rows, 16);
}

hipError_t layer_norm_mix_backward_rows(hipStream_t s, const float* x, const float* g_s,
                                        const uint16_t* x16, const uint16_t* mix, long rows,
                                        long time, long ch, const uint16_t* w, float* gx,
                                        int accumulate, float* amax, float* part, float* part_mix,
                                        float* g_scratch, int* nblk_out, int* nblk_mix_out) {
  if (rows <= 0 || ch <= 0 || time <= 0) {
    if (nblk_out) *nblk_out = 0;
    if (nblk_mix_out) *nblk_mix_out = 0;
    return hipSuccess;
  }
  auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; };
  if (ln_bwd_row_path(rows, ch) && time <= INT32_MAX && vec_ok(x) && vec_ok(g_s) && vec_ok(gx) &&
      a8(w) && a8(x16) && a8(mix)) {
    const int nblk = (int)cdiv(rows, kRowsPerBlock);
    if (nblk_out) *nblk_out = nblk;
    if (nblk_mix_out) *nblk_mix_out = nblk;
    return by_nv(ch, [&](auto nv) {
      launch(ln_bwd_row_kernel<decltype(nv)::value, true>, dim3(nblk), dim3(256), 0, s, x, g_s,
             rows, (int)ch, w, gx, accumulate, amax, part, x16, mix, (int)time, part_mix);
      return hipGetLastError();
    });
  }
  hipError_t e = time_shift_mix_backward(s, g_s, x16, mix, rows, time, ch, g_scratch, part_mix,
                                         nblk_mix_out);
  if (e != hipSuccess) return e;
  return layer_norm_backward_rows(s, x, g_scratch, rows, ch, w, gx, accumulate, amax, part,
                                  nblk_out);
}

hipError_t layer_norm_param_finish(hipStream_t s, const float* part, int nblk, long ch, float* gw,
                                   float* gb, float lr, uint16_t* w, float* w_res, uint16_t* b,
                                   float* b_res, const uint32_t* abort) {
  if (ch <= 0) return hipSuccess;
  // part is [nblk][2][ch]: columns [0, ch) are gamma sums, [ch, 2 ch) beta sums.
  // LayerNorm::apply_clipped_sgd, src/model.rs:318-332.
  VecTarget a{gw, lr > 0.0f ? w : nullptr, w_res, lr, nullptr, abort};
  VecTarget bt{gb, lr > 0.0f ? b : nullptr, b_res, lr, nullptr, abort};
  return partial_reduce(s, part, nblk, 2 * ch, ch, a, bt);
}

}  // namespace ullis
