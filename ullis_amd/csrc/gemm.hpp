// Tiled fp16 MFMA GEMM for gfx950:  C[m][n] = sum_k A(m, k) * B(n, k).
//
// One block = 256 threads = 4 wave64s in a 2x2 grid; each wave owns a
// (BM/2) x (BN/2) sub-tile made of 32x32 v_mfma_f32_32x32x16_f16 tiles with
// fp32 accumulation. The K loop steps BK = 32 with two LDS buffers: global
// loads for step k+1 are issued before the MFMAs of step k and stored to the
// other LDS buffer afterwards, so one barrier per step suffices.
//
// Operands reach LDS as fp16 in a [row][k] layout (k contiguous, rows padded
// to 40 halves = 80 B so the ds_read_b128 fragment reads of 16 lanes hit 16
// distinct bank quads). Loaders convert on the way in:
//   LoadF16K   fp16 source, k contiguous            (activations [rows][k])
//   LoadF32K   fp32 source, k contiguous, x scale   (fp32 gradients)
//   LoadF16T   fp16 source, row contiguous          ([k][rows]: transposed)
//   LoadF32T   fp32 source, row contiguous, x scale
//   LoadBits   packed sign bits, LSB-first u32; each bit becomes +-1 (or
//              +-scale[k] when a per-k scale vector is given) in fp16.
// Out-of-range elements are zero, so any M, N, K works; the vector fast paths
// need 16-byte aligned rows and are selected per launch by the host.
//
// The epilogue functor receives the accumulators with their tile origin.
#pragma once

#include "common.hpp"

namespace ullis {

constexpr int kBK = 32;
constexpr int kLDK = kBK + 8;  // padded LDS row, in halves
constexpr int kThreads = 256;

// ------------------------------------------------------------------ loaders

// Element (row, k) at p[row * ld + k].
template <int ROWS>
struct LoadF16K {
  const half_t* p;
  long ld;
  int vec_ok;  // ld % 8 == 0 and p 16-byte aligned
  static constexpr int U = (ROWS * kBK / 8 + kThreads - 1) / kThreads;
  struct Regs {
    half8 v[U];
  };
  __device__ void prepare() {}
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      half8 v = {};
      if (c < ROWS * kBK / 8) {
        const int row = row0 + (c >> 2);
        const int k = k0 + (c & 3) * 8;
        if (row < rows) {
          const half_t* src = p + (long)row * ld + k;
          if (vec_ok && k + 8 <= kend) {
            v = *reinterpret_cast<const half8*>(src);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (k + j < kend) ? src[j] : (half_t)0.0f;
          }
        }
      }
      r.v[u] = v;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < ROWS * kBK / 8) *reinterpret_cast<half8*>(&s[(c >> 2) * kLDK + (c & 3) * 8]) = r.v[u];
    }
  }
};

// Element (row, k) = p[row * ld + k] * scale (fp32 source).
template <int ROWS>
struct LoadF32K {
  const float* p;
  long ld;
  int vec_ok;  // ld % 4 == 0 and p 16-byte aligned
  const float* amax;  // optional: scale = grad_scale_from_amax(*amax)
  float scale;
  static constexpr int U = (ROWS * kBK / 8 + kThreads - 1) / kThreads;
  struct Regs {
    half8 v[U];
  };
  __device__ void prepare() {
    if (amax) scale = grad_scale_from_amax(*amax);
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      half8 v = {};
      if (c < ROWS * kBK / 8) {
        const int row = row0 + (c >> 2);
        const int k = k0 + (c & 3) * 8;
        if (row < rows) {
          const float* src = p + (long)row * ld + k;
          if (vec_ok && k + 8 <= kend) {
            const floatx4 a = *reinterpret_cast<const floatx4*>(src);
            const floatx4 b = *reinterpret_cast<const floatx4*>(src + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              v[j] = f32_to_f16_sat(a[j] * scale);
              v[j + 4] = f32_to_f16_sat(b[j] * scale);
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              v[j] = (k + j < kend) ? f32_to_f16_sat(src[j] * scale) : (half_t)0.0f;
          }
        }
      }
      r.v[u] = v;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < ROWS * kBK / 8) *reinterpret_cast<half8*>(&s[(c >> 2) * kLDK + (c & 3) * 8]) = r.v[u];
    }
  }
};

// Transposed fp16 source: element (row, k) at p[k * ld + row].
// Work item = (k pair, 8 consecutive rows); written to LDS as 8 b32 pairs.
template <int ROWS>
struct LoadF16T {
  const half_t* p;
  long ld;
  int vec_ok;  // ld % 8 == 0 and p 16-byte aligned
  static constexpr int ITEMS = (kBK / 2) * (ROWS / 8);
  static constexpr int U = (ITEMS + kThreads - 1) / kThreads;
  struct Regs {
    uint32_t w[U][8];
  };
  __device__ void prepare() {}
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
      if (c < ITEMS) {
        const int kp = c & 15;
        const int rc = c >> 4;
        const int k = k0 + 2 * kp;
        const int row = row0 + 8 * rc;
        if (vec_ok && row + 8 <= rows) {
          if (k < kend) lo = *reinterpret_cast<const u32x4*>(q + (long)k * ld + row);
          if (k + 1 < kend) hi = *reinterpret_cast<const u32x4*>(q + (long)(k + 1) * ld + row);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (row + j < rows) {
              const uint32_t sh = (j & 1) * 16;
              if (k < kend) lo[j >> 1] |= (uint32_t)q[(long)k * ld + row + j] << sh;
              if (k + 1 < kend) hi[j >> 1] |= (uint32_t)q[(long)(k + 1) * ld + row + j] << sh;
            }
          }
        }
      }
      // dword j = {row + j at k, row + j at k + 1}: low halves of lo/hi for
      // even j, high halves for odd j (v_perm_b32 byte selects).
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        r.w[u][2 * m] = __builtin_amdgcn_perm(hi[m], lo[m], 0x05040100u);
        r.w[u][2 * m + 1] = __builtin_amdgcn_perm(hi[m], lo[m], 0x07060302u);
      }
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < ITEMS) {
        const int kp = c & 15;
        const int rc = c >> 4;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<uint32_t*>(&s[(8 * rc + j) * kLDK + 2 * kp]) = r.w[u][j];
      }
    }
  }
};

// Transposed fp32 source with scale: element (row, k) = p[k * ld + row] * scale.
template <int ROWS>
struct LoadF32T {
  const float* p;
  long ld;
  int vec_ok;  // ld % 4 == 0 and p 16-byte aligned
  const float* amax;
  float scale;
  static constexpr int ITEMS = (kBK / 2) * (ROWS / 8);
  static constexpr int U = (ITEMS + kThreads - 1) / kThreads;
  struct Regs {
    uint32_t w[U][8];
  };
  __device__ void prepare() {
    if (amax) scale = grad_scale_from_amax(*amax);
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      float lo[8], hi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        lo[j] = 0.0f;
        hi[j] = 0.0f;
      }
      if (c < ITEMS) {
        const int kp = c & 15;
        const int rc = c >> 4;
        const int k = k0 + 2 * kp;
        const int row = row0 + 8 * rc;
        if (vec_ok && row + 8 <= rows) {
          if (k < kend) {
            const floatx4* s0 = reinterpret_cast<const floatx4*>(p + (long)k * ld + row);
            const floatx4 a = s0[0], b = s0[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              lo[j] = a[j];
              lo[j + 4] = b[j];
            }
          }
          if (k + 1 < kend) {
            const floatx4* s1 = reinterpret_cast<const floatx4*>(p + (long)(k + 1) * ld + row);
            const floatx4 a = s1[0], b = s1[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              hi[j] = a[j];
              hi[j + 4] = b[j];
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (row + j < rows) {
              if (k < kend) lo[j] = p[(long)k * ld + row + j];
              if (k + 1 < kend) hi[j] = p[(long)(k + 1) * ld + row + j];
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const half_t l = f32_to_f16_sat(lo[j] * scale);
        const half_t h = f32_to_f16_sat(hi[j] * scale);
        r.w[u][j] = (uint32_t)__builtin_bit_cast(uint16_t, l) |
                    ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
      }
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < ITEMS) {
        const int kp = c & 15;
        const int rc = c >> 4;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<uint32_t*>(&s[(8 * rc + j) * kLDK + 2 * kp]) = r.w[u][j];
      }
    }
  }
};

// Packed sign bits: element (row, k) is bit (row * ldb + kofs + k) of the
// LSB-first u32 array `bits` (src/model.rs:146-148), 1 => +1, 0 => -1.
// With `kscale` (f16 bits, indexed kofs + k) the element is +-kscale[k].
template <int ROWS>
struct LoadBits {
  const uint32_t* bits;
  long ldb;   // bits per row
  long kofs;  // bit offset of k = 0 within each row
  const uint16_t* kscale;
  int aligned;  // ldb % 8 == 0 and kofs % 8 == 0: each byte lies in one word
  static constexpr int ITEMS = ROWS * kBK / 8;
  static constexpr int U = (ITEMS + kThreads - 1) / kThreads;
  struct Regs {
    u32x4 v[U];
  };
  __device__ void prepare() {}
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      uint32_t byte = 0, valid = 0;
      const int row = row0 + (c >> 2);
      const int k = k0 + (c & 3) * 8;
      if (c < ITEMS && row < rows && k < kend) {
        const int nv = kend - k < 8 ? kend - k : 8;
        valid = nv >= 8 ? 0xffu : ((1u << nv) - 1u);
        const long g = (long)row * ldb + kofs + k;
        const uint32_t w0 = bits[g >> 5];
        const uint32_t sh = (uint32_t)(g & 31);
        byte = (w0 >> sh) & 0xffu;
        // The next word is read only when valid bits spill into it, so the
        // last word of the array is never overrun.
        if (!aligned && sh + (uint32_t)nv > 32u) byte = (byte | (bits[(g >> 5) + 1] << (32u - sh))) & 0xffu;
      }
      u32x4 out;
      if (kscale) {
        uint16_t sc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (valid) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if ((valid >> j) & 1u) sc[j] = kscale[kofs + k + j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t b0 = (byte >> (2 * j)) & 1u, b1 = (byte >> (2 * j + 1)) & 1u;
          const uint32_t lo = (uint32_t)sc[2 * j] ^ ((b0 ^ 1u) << 15);
          const uint32_t hi = (uint32_t)sc[2 * j + 1] ^ ((b1 ^ 1u) << 15);
          out[j] = (((valid >> (2 * j)) & 1u) ? lo : 0u) |
                   ((((valid >> (2 * j + 1)) & 1u) ? hi : 0u) << 16);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t b0 = (byte >> (2 * j)) & 1u, b1 = (byte >> (2 * j + 1)) & 1u;
          const uint32_t lo = 0xBC00u ^ (b0 << 15);  // 0x3C00 = +1.0, 0xBC00 = -1.0
          const uint32_t hi = 0xBC00u ^ (b1 << 15);
          out[j] = (((valid >> (2 * j)) & 1u) ? lo : 0u) |
                   ((((valid >> (2 * j + 1)) & 1u) ? hi : 0u) << 16);
        }
      }
      r.v[u] = out;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < ITEMS) *reinterpret_cast<u32x4*>(&s[(c >> 2) * kLDK + (c & 3) * 8]) = r.v[u];
    }
  }
};

// ------------------------------------------------------------------ kernel

// Maps blockIdx.x to a tile so that consecutive dispatches on one XCD (blocks
// b, b+8, b+16, ... land on the same XCD) walk along N for a fixed M panel,
// which keeps the A panel resident in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int t = bid;
  if (total % 8 == 0) t = (bid % 8) * (total / 8) + bid / 8;
  tm = t / tiles_n;
  tn = t % tiles_n;
}

template <int BM, int BN, class LA, class LB, class Epi>
__global__ __launch_bounds__(256) void gemm_kernel(LA la, LB lb, Epi epi, int M, int N, int K,
                                                   int k_split) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) half_t sA[2][BM * kLDK];
  __shared__ __attribute__((aligned(16))) half_t sB[2][BN * kLDK];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = blockIdx.z * k_split;
  const int kend = min(K, kbeg + k_split);

  la.prepare();
  lb.prepare();

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (floatx16){};

  const int nk = kend > kbeg ? (kend - kbeg + kBK - 1) / kBK : 0;
  typename LA::Regs ra;
  typename LB::Regs rb;
  if (nk > 0) {
    la.load(ra, m0, kbeg, M, kend);
    lb.load(rb, n0, kbeg, N, kend);
    la.store(ra, sA[0]);
    lb.store(rb, sB[0]);
  }
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(ra, m0, kbeg + (kt + 1) * kBK, M, kend);
      lb.load(rb, n0, kbeg + (kt + 1) * kBK, N, kend);
    }
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const half8*>(
            &sA[cur][(wm * WM + i * 32 + frag_row) * kLDK + ks * 16 + frag_k]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const half8*>(
            &sB[cur][(wn * WN + j * 32 + frag_row) * kLDK + ks * 16 + frag_k]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(ra, sA[cur ^ 1]);
      lb.store(rb, sB[cur ^ 1]);
    }
    __syncthreads();
  }

  epi.template run<TM, TN>(acc, m0 + wm * WM, n0 + wn * WN, lane, M, N);
}

// Convenience: visit every in-range accumulator element as (row, col, value).
template <int TM, int TN, class F>
__device__ __forceinline__ void for_each_acc(floatx16 (&acc)[TM][TN], int row0, int col0, int lane,
                                             int M, int N, F&& f) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = col0 + j * 32 + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + i * 32 + mfma32_row(r, lane);
        if (row < M && col < N) f(row, col, acc[i][j][r]);
      }
    }
}

// Split-K partial: writes fp32 C for split blockIdx.z to part[z][M][N].
struct EpiPartial {
  float* part;
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
    float* dst = part + (long)blockIdx.z * M * N;
    for_each_acc(acc, row0, col0, lane, M, N,
                 [&](int row, int col, float v) { dst[(long)row * N + col] = v; });
  }
};

}  // namespace ullis
