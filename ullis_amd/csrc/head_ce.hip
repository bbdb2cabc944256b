// Packed vocab head fused with streamed next-token cross-entropy.
//
// Reference: the CPU branch of UllisHeron::apply_head_ce (src/model.rs:3132-3274)
// with causal_ce_row_valid / causal_ce_gradient_scale (src/model.rs:27-55):
// per valid row, ce = max + ln sum exp(l - max) - l[target], gy = gscale *
// (softmax - onehot), gscale = 1/(T-1); then the head's backward_ste, the
// BinaryConnect latent step with ste = T-1 and scale SGD, and the head bias
// step at 8x the learning rate (src/model.rs:3118-3130). The Metal path it
// replaces (packed_head_train_sgd, src/metal.rs:3300-3510) materialises
// [rows, vocab] fp32 logits and their gradient.
//
// Here the [rows, vocab] logits are never stored:
//  1. logits GEMM with an online log-sum-exp epilogue: per (row, 32-column
//     block) max and sum-exp, plus the target logit;
//  2. a per-row combine gives lse, row loss, n_valid, mean loss and gscale on
//     the device (no host round trip);
//  3. the vocabulary is streamed in chunks of Vc columns: the logits of the
//     chunk are recomputed, turned into the unscaled fp16 gradient p - onehot
//     (a [rows, Vc] scratch, never [rows, vocab]), and consumed by the input
//     gradient GEMM (accumulated into g_hidden, times gscale) and the
//     weight-gradient GEMM of those Vc head rows, whose finish kernel applies
//     the latent step and g_scale = sum_i sign * G;
//  4. g_bias, the scale / bias steps and the bit repack run after the last
//     chunk, so every GEMM above reads the pre-update bits and scales.
#include <math.h>

#include "gemm.hpp"
#include "context.hpp"
#include "gemm_lds.hpp"
#include "ops.hpp"

namespace ullis {

hipError_t packed_backward_input_ex(hipStream_t s, const uint16_t* gy16, long ldgy, long rows,
                                    long in, long k_len, const uint32_t* bits_t, long ldb,
                                    long kofs, const uint16_t* scale, float* gx,
                                    const float* out_mul, int accumulate);

namespace {

// causal_ce_row_valid(row, time, horizon, targets, ignore_id), src/model.rs:27-39,
// with one addition: a target >= vocab (other than ignore_id) makes no row
// valid. The reference refuses such a label before the step
// (src/model.rs:2852-2861); here labels are device data, so those rows are
// left out of the loss and the gradient, and ce_invalid_labels_kernel counts
// them for the caller.
struct CeRows {
  long rows, time, horizon, vocab;
  const uint32_t* targets;
  uint32_t ignore_id;
  __device__ __forceinline__ bool valid(long row) const {
    if (time == 0 || row % time + horizon >= time) return false;
    const long t = row + horizon;
    if (t >= rows) return false;
    const uint32_t id = targets[t];
    return id != ignore_id && (long)id < vocab;
  }
  __device__ __forceinline__ long target(long row) const { return (long)targets[row + horizon]; }
};

struct EpiCeStats {
  const uint16_t* scale;
  const uint16_t* bias;
  CeRows ce;
  float* part_m;  // [M][nb32], nb32 = ceil(N / 32): one row's blocks contiguous
  float* part_s;
  float* tgt;     // [M]
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int cbase = col0 + j * 32;
        const int col = cbase + (lane & 31);
        const bool colok = col < N;
        const float sc = colok ? f16_bits_to_f32(scale[col]) : 0.0f;
        const float bi = (bias && colok) ? f16_bits_to_f32(bias[col]) : 0.0f;
        const long cb = cbase / 32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row0 + i * 32 + mfma32_row(r, lane);
          const float logit = colok ? bi + sc * acc[i][j][r] : -INFINITY;
          const float m = halfwave_max(logit);
          const float e = (colok && m > -INFINITY) ? expf(logit - m) : 0.0f;
          const float ssum = halfwave_sum(e);
          if (row < M && cbase < N) {
            if ((lane & 31) == 0) {
              const long nb = (N + 31) / 32;
              part_m[(long)row * nb + cb] = m;
              part_s[(long)row * nb + cb] = ssum;
            }
            if (colok && ce.valid(row) && ce.target(row) == (long)col) tgt[row] = logit;
          }
        }
      }
  }
  // Streamed-LDS kernels: lanes 2r, 2r+1 hold the two 16-column halves of one
  // row of a 32-column block; their (max, sum-exp) pairs merge in registers.
  __device__ void row16(int row, int col, float (&v)[16], int lane, int M, int N, float*, int,
                        int) {
    const bool full = col + 16 <= N && N % 8 == 0;
    float sc[16], bi[16];
    lds::get16h(scale, col, N, full && lds::al16(scale), sc);
    if (bias) {
      lds::get16h(bias, col, N, full && lds::al16(bias), bi);
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) bi[k] = 0.0f;
    }
    float l[16];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      l[k] = col + k < N ? bi[k] + sc[k] * v[k] : -INFINITY;
      m = __builtin_fmaxf(m, l[k]);
    }
    float se = 0.0f;
    if (m > -INFINITY) {
#pragma unroll
      for (int k = 0; k < 16; ++k) se += col + k < N ? expf(l[k] - m) : 0.0f;
    }
    const float pm = __shfl_xor(m, 1, 64), ps = __shfl_xor(se, 1, 64);
    const float mm = __builtin_fmaxf(m, pm);
    float ss = 0.0f;
    if (mm > -INFINITY) {
      if (m > -INFINITY) ss += se * expf(m - mm);
      if (pm > -INFINITY) ss += ps * expf(pm - mm);
    }
    if (row >= M) return;
    if ((lane & 1) == 0 && col < N) {
      const long nb = (N + 31) / 32;
      part_m[(long)row * nb + (col >> 5)] = mm;
      part_s[(long)row * nb + (col >> 5)] = ss;
    }
    if (ce.valid(row)) {
      const long t = ce.target(row) - col;
      if (t >= 0 && t < 16 && col + t < N) {
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (k == t) tgt[row] = l[k];
      }
    }
  }
};

struct EpiCeGrad {
  const uint16_t* scale;  // chunk-offset
  const uint16_t* bias;   // chunk-offset or null
  CeRows ce;
  long col_base;          // global vocab index of chunk column 0
  long vocab;
  const float* lse;
  uint16_t* gy16;         // [M][N] chunk scratch
  float* part_bias;       // [ceil(M/32)][vocab]
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
        const long vcol = col_base + col;
        float csum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row0 + i * 32 + mfma32_row(r, lane);
          if (row < M && colok) {
            float g = 0.0f;
            if (ce.valid(row)) {
              const float logit = bi + sc * acc[i][j][r];
              const float p = expf(logit - lse[row]);
              g = ce.target(row) == vcol ? p - 1.0f : p;
            }
            gy16[(long)row * N + col] = __builtin_bit_cast(uint16_t, (half_t)g);
            csum += g;
          }
        }
        csum += __shfl_xor(csum, 32, 64);
        const int tile_row = row0 + i * 32;
        if (lane < 32 && colok && tile_row < M) part_bias[(long)(tile_row / 32) * vocab + vcol] = csum;
      }
  }
  // Streamed-LDS kernels: gradient for 16 columns of one row, then the block's
  // column sums over its 32 rows from the LDS block buffer (fixed order).
  __device__ void row16(int row, int col, float (&v)[16], int lane, int M, int N, float* buf,
                        int brow, int bcol) {
    const bool rok = row < M;
    const bool valid = rok && ce.valid(row);
    const bool full = col + 16 <= N && N % 8 == 0;
    float g[16];
    if (valid) {
      float sc[16], bi[16];
      lds::get16h(scale, col, N, full && lds::al16(scale), sc);
      if (bias) {
        lds::get16h(bias, col, N, full && lds::al16(bias), bi);
      } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) bi[k] = 0.0f;
      }
      const float ls = lse[row];
      const long t = ce.target(row) - (col_base + col);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float p = expf(bi[k] + sc[k] * v[k] - ls);
        g[k] = col + k < N ? (k == t ? p - 1.0f : p) : 0.0f;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) g[k] = 0.0f;
    }
    if (rok) {
      const long idx = (long)row * N + col;
      if (full && lds::al16(gy16)) {
        lds::store16h(gy16 + idx, g);
      } else {
        for (int k = 0; k < 16 && col + k < N; ++k)
          gy16[idx + k] = __builtin_bit_cast(uint16_t, (half_t)g[k]);
      }
    }
    // g over the block's 32 rows -> per-column sums (rows past M hold 0)
    float* rowp = buf + (lane >> 1) * lds::kBufPitch + (lane & 1) * 16;
#pragma unroll
    for (int k = 0; k < 16; ++k) rowp[k] = g[k];
    lds::lds_fence();
    if (lane < 32) {
      float cs = 0.0f;
#pragma unroll
      for (int r = 0; r < 32; ++r) cs += buf[r * lds::kBufPitch + lane];
      if (bcol + lane < N && brow < M)
        part_bias[(long)(brow / 32) * vocab + col_base + bcol + lane] = cs;
    }
  }
};

// One wave per row: merge the per-block (max, sum-exp) pairs.
__global__ __launch_bounds__(256) void ce_combine_kernel(const float* part_m, const float* part_s,
                                                         long nb, CeRows ce, const float* tgt,
                                                         float* lse, float* row_loss) {
  const long rows = ce.rows;
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float m = -INFINITY;
  const float* pm = part_m + row * nb;
  const float* ps = part_s + row * nb;
  for (long b = lane; b < nb; b += 64) m = __builtin_fmaxf(m, pm[b]);
  m = wave_max(m);
  float s = 0.0f;
  for (long b = lane; b < nb; b += 64) {
    const float mb = pm[b];
    if (mb > -INFINITY) s += ps[b] * expf(mb - m);
  }
  s = wave_sum(s);
  if (lane == 0) {
    const float l = m + logf(s);
    lse[row] = l;
    row_loss[row] = ce.valid(row) ? l - tgt[row] : 0.0f;
  }
}

// Adds to *invalid the number of targets that are neither ignore_id nor a
// vocabulary index (every row, as the reference's check of labels does).
__global__ __launch_bounds__(256) void ce_invalid_labels_kernel(const uint32_t* targets, long rows,
                                                                long vocab, uint32_t ignore_id,
                                                                uint32_t* invalid) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool bad = r < rows && targets[r] != ignore_id && (long)targets[r] >= vocab;
  const unsigned long long m = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && m) atomicAdd(invalid, (uint32_t)__popcll(m));
}

// Single block: n_valid, loss sum (fixed-order tree), mean and gscale.
__global__ __launch_bounds__(1024) void ce_mean_kernel(const float* row_loss, CeRows ce,
                                                       float* stats, float* stats2) {
  const long rows = ce.rows, time = ce.time;
  __shared__ float ls[1024];
  __shared__ float nv[1024];
  float a = 0.0f, n = 0.0f;
  for (long r = threadIdx.x; r < rows; r += blockDim.x) {
    if (ce.valid(r)) {
      a += row_loss[r];
      n += 1.0f;
    }
  }
  ls[threadIdx.x] = a;
  nv[threadIdx.x] = n;
  __syncthreads();
  for (int st = 512; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) {
      ls[threadIdx.x] += ls[threadIdx.x + st];
      nv[threadIdx.x] += nv[threadIdx.x + st];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float count = nv[0];
    stats[0] = count > 0.0f ? ls[0] / count : 0.0f;
    stats[1] = count;
    stats[2] = (count > 0.0f && time >= 2) ? 1.0f / (float)(time - 1) : 0.0f;  // :49-55
    stats[3] = ls[0];
    if (stats2) {
      stats2[0] = stats[0];
      stats2[1] = stats[1];
      stats2[2] = stats[2];
      stats2[3] = stats[3];
    }
  }
}

long chunk_cols(long vocab, long d) {
  // The whole vocabulary up to 8192 columns (the scaled-bits operand of the
  // input-gradient GEMM keeps the scales of its k range in LDS), multiple of 32.
  (void)d;
  const long vc = vocab < 8192 ? vocab : 8192;
  return cdiv(vc, 32) * 32;
}

struct Ws {
  float *part_m, *part_s, *tgt, *lse, *part_bias, *gpart, *g_scale, *g_bias;
  uint16_t* gy16;
};

Ws carve(void* base, long rows, long d, long vocab) {
  const long nb32 = cdiv(vocab, 32);
  const long vc = chunk_cols(vocab, d);
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) {
    char* r = p;
    p += (bytes + 255) / 256 * 256;
    return r;
  };
  Ws w;
  w.part_m = reinterpret_cast<float*>(take(sizeof(float) * nb32 * rows));
  w.part_s = reinterpret_cast<float*>(take(sizeof(float) * nb32 * rows));
  w.tgt = reinterpret_cast<float*>(take(sizeof(float) * rows));
  w.lse = reinterpret_cast<float*>(take(sizeof(float) * rows));
  w.part_bias = reinterpret_cast<float*>(take(sizeof(float) * cdiv(rows, 32) * vocab));
  w.gpart = reinterpret_cast<float*>(take(sizeof(float) * pair_dw_splits(vc, d, rows) * vc * d));
  w.g_scale = reinterpret_cast<float*>(take(sizeof(float) * vocab));
  w.g_bias = reinterpret_cast<float*>(take(sizeof(float) * vocab));
  w.gy16 = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * rows * vc));
  return w;
}

template <class Epi>
hipError_t logits_gemm(hipStream_t s, const uint16_t* hidden16, long rows, long d,
                       const uint32_t* bits_rows, long ncols, const Epi& epi) {
  // C[rows][ncols] = hidden . S^T ; S rows start at bits_rows (word aligned).
  hipError_t err = hipSuccess;
  if (lds::mk_ok(hidden16, d) &&
      lds::with_lds(rows, ncols, d, 1, &err, [&](auto t) {
        using T = decltype(t);
        lds::OpMK<T::bm, T::bk, T::nw> a{reinterpret_cast<const half_t*>(hidden16), d, (int)rows};
        lds::OpBits<T::bn, T::bk, false, T::nw> b{bits_rows, d / 32, (int)ncols, nullptr, 0};
        return lds::launch_lds<T>(s, a, b, epi, rows, ncols, d, 1);
      }, lds::LdsPolicy::kNoBig))
    return err;
  const bool vec = (reinterpret_cast<uintptr_t>(hidden16) & 15u) == 0 && d % 8 == 0;
  auto run = [&](auto cfg) {
    using T = decltype(cfg);
    using LA = LoadF16K<T::bm, T::bk>;
    using LB = LoadBits<T::bn, T::bk>;
    LA la{reinterpret_cast<const half_t*>(hidden16), d, vec};
    LB lb{bits_rows, d, 0, nullptr, d % 8 == 0};
    launch((gemm_kernel<T::bm, T::bn, T::bk, T::stages, LA, LB, Epi>),
                       dim3((unsigned)(cdiv(rows, T::bm) * cdiv(ncols, T::bn))), dim3(kThreads),
                       0, s, la, lb, epi, (int)rows, (int)ncols, (int)d,
                       (int)(cdiv(d, T::bk) * T::bk));
    return hipGetLastError();
  };
  if (cdiv(rows, 128) * cdiv(ncols, 128) >= 240) return run(CfgLarge{});
  return run(CfgSmall{});
}

}  // namespace

size_t head_ce_workspace_bytes(long rows, long d, long vocab) {
  const long nb32 = cdiv(vocab, 32);
  const long vc = chunk_cols(vocab, d);
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  return al(4 * nb32 * rows) * 2 + al(4 * rows) * 2 + al(4 * cdiv(rows, 32) * vocab) +
         al(4 * pair_dw_splits(vc, d, rows) * vc * d) + al(4 * vocab) * 2 + al(2 * rows * vc) + 256;
}

long head_ce_chunk_cols(long vocab, long d) { return chunk_cols(vocab, d); }

int head_ce_splits(long rows, long d, long vocab) {
  return pair_dw_splits(chunk_cols(vocab, d), d, rows);
}

float* head_ce_bias_partials(void* workspace, long rows, long d, long vocab) {
  return carve(workspace, rows, d, vocab).part_bias;
}

hipError_t head_ce(hipStream_t s, const HeadCe& h, void* workspace) {
  const long rows = h.rows, d = h.d, V = h.vocab;
  if (rows <= 0 || d <= 0 || V <= 0) return hipErrorInvalidValue;
  Ws w = carve(workspace, rows, d, V);
  const long nb32 = cdiv(V, 32);
  hipError_t e;

  // 1. forward statistics (fills every part_m/part_s entry and tgt of valid rows)
  const CeRows ce{rows, h.time, h.horizon, V, h.targets, h.ignore_id};
  if (h.invalid) {
    launch(ce_invalid_labels_kernel, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, s, h.targets,
           rows, V, h.ignore_id, h.invalid);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  EpiCeStats st{h.scale, h.bias, ce, w.part_m, w.part_s, w.tgt};
  if ((e = logits_gemm(s, h.hidden16, rows, d, h.bits, V, st)) != hipSuccess) return e;
  // 2. combine
  launch(ce_combine_kernel, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, w.part_m,
                     w.part_s, nb32, ce, w.tgt, w.lse, h.row_loss);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  launch(ce_mean_kernel, dim3(1), dim3(1024), 0, s, h.row_loss, ce, h.stats, h.stats2);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  // 3. stream the vocabulary in chunks
  const long vc = chunk_cols(V, d);
  const bool upd = h.lr > 0.0f;
  const bool fuse = upd && h.scale_upd && h.bits_new && d % 64 == 0 && h.bits_new == h.bits;
  const float* gscale = h.stats + 2;
  float* g_scale = h.g_scale ? h.g_scale : w.g_scale;
  for (long c0 = 0, ci = 0; c0 < V; c0 += vc, ++ci) {
    const long n = V - c0 < vc ? V - c0 : vc;
    const uint32_t* bits_rows = h.bits + (c0 * d) / 32;
    EpiCeGrad gr{h.scale + c0, h.bias ? h.bias + c0 : nullptr, ce, c0,
                 V, w.lse, w.gy16, w.part_bias};
    if ((e = logits_gemm(s, h.hidden16, rows, d, bits_rows, n, gr)) != hipSuccess) return e;
    // g_hidden (+)= gscale * gy_chunk . (scale * S)_chunk and G_chunk =
    // gy_chunk^T . hidden in one launch, then the latent step for these rows
    const int sp = pair_dw_splits(vc, d, rows);  // the workspace holds this many [vc][d] partials
    float* gp = h.gpart_all ? h.gpart_all + ci * sp * vc * d : w.gpart;
    const PackedDxArgs dx{GradIn{nullptr, nullptr}, w.gy16, rows, d, n, h.bits_t, h.scale,
                          h.g_hidden, gscale, ci > 0 ? 1 : 0, n, V, c0};
    const WeightGradArgs dw{GradIn{nullptr, nullptr}, w.gy16, h.hidden16, rows, d, n, sp, gp};
    if ((e = packed_backward_pair(s, dx, dw)) != hipSuccess) return e;
    if (h.gpart_all) continue;  // deferred: the caller runs the update
    PackedFinish f;
    f.part = w.gpart;
    f.splits = sp;
    f.out = n;
    f.in = d;
    f.scale = h.scale + c0;
    f.bits_old = h.bits + (c0 * d) / 32;
    f.amax = nullptr;
    f.extra_mul = gscale;
    f.ste = h.ste;
    f.lr = h.lr;
    f.latent = h.lr > 0.0f ? h.latent + c0 * d : nullptr;
    f.latent_res = h.lr > 0.0f ? h.latent_res + c0 * d : nullptr;
    f.g_scale = g_scale + c0;
    f.g_w = h.g_w ? h.g_w + c0 * d : nullptr;
    if (fuse) {
      // this chunk's rows are not read again in this call except through
      // bits_t (rebuilt at the end): step their scales and repack them now
      f.scale_upd = h.scale_upd + c0;
      f.scale_res = h.scale_res + c0;
      f.bits_new = h.bits_new + (c0 * d) / 32;
    }
    if ((e = packed_weight_finish(s, f)) != hipSuccess) return e;
  }

  if (h.gpart_all) return hipSuccess;
  // 4. bias gradient, vector steps, repack
  // g_bias = gscale * sum over row tiles; head bias step at 8 lr (src/model.rs:3118-3130)
  VecTarget bias_t{h.g_bias ? h.g_bias : w.g_bias, upd ? h.bias_upd : nullptr, h.bias_res,
                   h.lr * kHeadBiasLrMult, gscale};
  if ((e = partial_reduce(s, w.part_bias, (int)cdiv(rows, 32), V, V, bias_t, bias_t)) !=
      hipSuccess)
    return e;
  if (fuse) return h.bits_t_new ? transpose_bits(s, h.bits_new, V, d, h.bits_t_new) : hipSuccess;
  if (upd && h.scale_upd) {
    if ((e = clipped_sgd(s, h.scale_upd, h.scale_res, g_scale, V, h.lr)) != hipSuccess) return e;
  }
  if (upd && h.bits_new) return pack_latent_bits(s, h.latent, V, d, h.bits_new, h.bits_t_new);
  return hipSuccess;
}

}  // namespace ullis
