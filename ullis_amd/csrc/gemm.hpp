// Tiled fp16 MFMA GEMM for gfx950:  C[m][n] = sum_k A(m, k) * B(n, k).
//
// One block = 256 threads = 4 wave64s in a 2x2 grid; each wave owns a
// (BM/2) x (BN/2) sub-tile made of 32x32 v_mfma_f32_32x32x16_f16 tiles with
// fp32 accumulation. The K loop steps BK (32 or 64) with two LDS buffers and a
// ring of S register stages: at step t the loads of tile t+S are issued, the
// MFMAs of tile t run from LDS, then tile t+1 (loaded S-1 steps earlier) is
// written to the other LDS buffer. S-1 steps of global-load latency are hidden
// behind MFMA work, which matters because the heron grids give one block per
// CU. One barrier per step (it waits for LDS traffic only).
//
// Each loader has a checked path (zero fill outside M / N / K, scalar
// fallbacks for unaligned rows) and a fast path for full, aligned tiles with
// straight-line vector loads. The fast path is chosen once per block, so the
// loads it issues stay in flight across steps; per-element branches would make
// the compiler wait for every load at the branch join.
//
// Operands reach LDS as fp16 in a [row][k] layout (k contiguous, rows padded
// by 8 halves: 80 B rows for BK 32, 144 B for BK 64, so the ds_read_b128
// fragment reads of 16 lanes hit 16 distinct bank quads). Loaders:
//   LoadF16K   fp16 source, k contiguous            (activations [rows][k])
//   LoadF32K   fp32 source, k contiguous, x scale   (fp32 gradients)
//   LoadF16T   fp16 source, row contiguous          ([k][rows]: transposed)
//   LoadF32T   fp32 source, row contiguous, x scale
//   LoadBits   packed sign bits, LSB-first u32; each bit becomes +-1 (or
//              +-scale[k] when a per-k scale vector is given) in fp16.
//
// The epilogue functor receives the accumulators with their tile origin.
#pragma once

#include "common.hpp"

namespace ullis {

constexpr int kThreads = 256;

template <int BK>
struct Lds {
  static constexpr int ldk = BK + 8;  // padded LDS row, in halves
};

constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ loaders

// Element (row, k) at p[row * ld + k].
template <int ROWS, int BK>
struct LoadF16K {
  const half_t* p;
  long ld;
  int vec_ok;  // ld % 8 == 0 and p 16-byte aligned
  static constexpr int CPR = BK / 8;
  static constexpr int ITEMS = ROWS * CPR;
  static constexpr int U = ceil_div(ITEMS, kThreads);
  struct Regs {
    half8 v[U];
  };
  __device__ void prepare() {}
  __device__ bool fast(int row0, int rows) const { return vec_ok && row0 + ROWS <= rows; }
  __device__ __forceinline__ void load_fast(Regs& r, int row0, int k0) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS)
        r.v[u] = *reinterpret_cast<const half8*>(p + (long)(row0 + c / CPR) * ld + k0 + (c % CPR) * 8);
    }
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      half8 v = {};
      if (c < ITEMS) {
        const int row = row0 + c / CPR;
        const int k = k0 + (c % CPR) * 8;
        if (row < rows) {
          const half_t* src = p + (long)row * ld + k;
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = (k + j < kend) ? src[j] : (half_t)0.0f;
        }
      }
      r.v[u] = v;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS)
        *reinterpret_cast<half8*>(&s[(c / CPR) * Lds<BK>::ldk + (c % CPR) * 8]) = r.v[u];
    }
  }
};

// Element (row, k) = p[row * ld + k] * scale (fp32 source).
template <int ROWS, int BK>
struct LoadF32K {
  const float* p;
  long ld;
  int vec_ok;  // ld % 4 == 0 and p 16-byte aligned
  const float* amax;  // optional: scale = grad_scale_from_amax(*amax)
  float scale;
  static constexpr int CPR = BK / 8;
  static constexpr int ITEMS = ROWS * CPR;
  static constexpr int U = ceil_div(ITEMS, kThreads);
  struct Regs {
    floatx4 a[U], b[U];
  };
  __device__ void prepare() {
    if (amax) scale = grad_scale_from_amax(*amax);
  }
  __device__ bool fast(int row0, int rows) const { return vec_ok && row0 + ROWS <= rows; }
  __device__ __forceinline__ void load_fast(Regs& r, int row0, int k0) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const float* src = p + (long)(row0 + c / CPR) * ld + k0 + (c % CPR) * 8;
        r.a[u] = *reinterpret_cast<const floatx4*>(src);
        r.b[u] = *reinterpret_cast<const floatx4*>(src + 4);
      }
    }
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      floatx4 a = {}, b = {};
      if (c < ITEMS) {
        const int row = row0 + c / CPR;
        const int k = k0 + (c % CPR) * 8;
        if (row < rows) {
          const float* src = p + (long)row * ld + k;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            a[j] = (k + j < kend) ? src[j] : 0.0f;
            b[j] = (k + 4 + j < kend) ? src[4 + j] : 0.0f;
          }
        }
      }
      r.a[u] = a;
      r.b[u] = b;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        half8 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = f32_to_f16_sat(r.a[u][j] * scale);
          v[j + 4] = f32_to_f16_sat(r.b[u][j] * scale);
        }
        *reinterpret_cast<half8*>(&s[(c / CPR) * Lds<BK>::ldk + (c % CPR) * 8]) = v;
      }
    }
  }
};

// Transposed fp16 source: element (row, k) at p[k * ld + row].
// Work item = (k pair, 8 consecutive rows), written to LDS as 8 b32 pairs;
// consecutive lanes take consecutive k pairs of one row block, so each LDS
// write instruction of 32 lanes covers 128 contiguous bytes.
template <int ROWS, int BK>
struct LoadF16T {
  const half_t* p;
  long ld;
  int vec_ok;  // ld % 8 == 0 and p 16-byte aligned
  static constexpr int KP = BK / 2;
  static constexpr int ITEMS = KP * (ROWS / 8);
  static constexpr int U = ceil_div(ITEMS, kThreads);
  struct Regs {
    u32x4 lo[U], hi[U];
  };
  __device__ void prepare() {}
  __device__ bool fast(int row0, int rows) const { return vec_ok && row0 + ROWS <= rows; }
  __device__ __forceinline__ void load_fast(Regs& r, int row0, int k0) const {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const uint16_t* src = q + (long)(k0 + 2 * (c % KP)) * ld + row0 + 8 * (c / KP);
        r.lo[u] = *reinterpret_cast<const u32x4*>(src);
        r.hi[u] = *reinterpret_cast<const u32x4*>(src + ld);
      }
    }
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
      if (c < ITEMS) {
        const int k = k0 + 2 * (c % KP);
        const int row = row0 + 8 * (c / KP);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (row + j < rows) {
            const uint32_t sh = (j & 1) * 16;
            if (k < kend) lo[j >> 1] |= (uint32_t)q[(long)k * ld + row + j] << sh;
            if (k + 1 < kend) hi[j >> 1] |= (uint32_t)q[(long)(k + 1) * ld + row + j] << sh;
          }
        }
      }
      r.lo[u] = lo;
      r.hi[u] = hi;
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const int kp = c % KP;
        const int rc = c / KP;
        // dword j = {row + j at k, row + j at k + 1}: low halves of lo/hi for
        // even j, high halves for odd j (v_perm_b32 byte selects).
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          *reinterpret_cast<uint32_t*>(&s[(8 * rc + 2 * m) * Lds<BK>::ldk + 2 * kp]) =
              __builtin_amdgcn_perm(r.hi[u][m], r.lo[u][m], 0x05040100u);
          *reinterpret_cast<uint32_t*>(&s[(8 * rc + 2 * m + 1) * Lds<BK>::ldk + 2 * kp]) =
              __builtin_amdgcn_perm(r.hi[u][m], r.lo[u][m], 0x07060302u);
        }
      }
    }
  }
};

// Transposed fp32 source with scale: element (row, k) = p[k * ld + row] * scale.
template <int ROWS, int BK>
struct LoadF32T {
  const float* p;
  long ld;
  int vec_ok;  // ld % 4 == 0 and p 16-byte aligned
  const float* amax;
  float scale;
  static constexpr int KP = BK / 2;
  static constexpr int ITEMS = KP * (ROWS / 8);
  static constexpr int U = ceil_div(ITEMS, kThreads);
  struct Regs {
    floatx4 lo0[U], lo1[U], hi0[U], hi1[U];
  };
  __device__ void prepare() {
    if (amax) scale = grad_scale_from_amax(*amax);
  }
  __device__ bool fast(int row0, int rows) const { return vec_ok && row0 + ROWS <= rows; }
  __device__ __forceinline__ void load_fast(Regs& r, int row0, int k0) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const float* src = p + (long)(k0 + 2 * (c % KP)) * ld + row0 + 8 * (c / KP);
        r.lo0[u] = *reinterpret_cast<const floatx4*>(src);
        r.lo1[u] = *reinterpret_cast<const floatx4*>(src + 4);
        r.hi0[u] = *reinterpret_cast<const floatx4*>(src + ld);
        r.hi1[u] = *reinterpret_cast<const floatx4*>(src + ld + 4);
      }
    }
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
        const int k = k0 + 2 * (c % KP);
        const int row = row0 + 8 * (c / KP);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (row + j < rows) {
            if (k < kend) lo[j] = p[(long)k * ld + row + j];
            if (k + 1 < kend) hi[j] = p[(long)(k + 1) * ld + row + j];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r.lo0[u][j] = lo[j];
        r.lo1[u][j] = lo[j + 4];
        r.hi0[u][j] = hi[j];
        r.hi1[u][j] = hi[j + 4];
      }
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const int kp = c % KP;
        const int rc = c / KP;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float lo = j < 4 ? r.lo0[u][j & 3] : r.lo1[u][j & 3];
          const float hi = j < 4 ? r.hi0[u][j & 3] : r.hi1[u][j & 3];
          const uint32_t l = __builtin_bit_cast(uint16_t, f32_to_f16_sat(lo * scale));
          const uint32_t h = __builtin_bit_cast(uint16_t, f32_to_f16_sat(hi * scale));
          *reinterpret_cast<uint32_t*>(&s[(8 * rc + j) * Lds<BK>::ldk + 2 * kp]) = l | (h << 16);
        }
      }
    }
  }
};

// Packed sign bits: element (row, k) is bit (row * ldb + kofs + k) of the
// LSB-first u32 array `bits` (src/model.rs:146-148), 1 => +1, 0 => -1.
// With SCALED, `kscale` (f16 bits, indexed kofs + k) is applied: the element is
// +-kscale[k] (a compile-time choice: a runtime null check would put a branch
// join after the loads, where the compiler waits for them).
// Work item = 8 consecutive k of one row: one byte of sign bits -> 8 halves.
template <int ROWS, int BK, bool SCALED = false>
struct LoadBits {
  const uint32_t* bits;
  long ldb;   // bits per row
  long kofs;  // bit offset of k = 0 within each row
  const uint16_t* kscale;  // used iff SCALED
  int aligned;  // ldb % 8 == 0, kofs % 8 == 0, kscale 16-byte aligned
  static constexpr int BPR = BK / 8;
  static constexpr int ITEMS = ROWS * BPR;
  static constexpr int U = ceil_div(ITEMS, kThreads);
  struct Regs {
    uint32_t word[U];  // raw sign word; the byte is extracted in store()
    uint32_t sh[U];    // bit offset of the byte within word
    u32x4 sc[U];
  };
  __device__ void prepare() {}
  __device__ bool fast(int row0, int rows) const { return aligned && row0 + ROWS <= rows; }
  __device__ __forceinline__ void load_fast(Regs& r, int row0, int k0) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const int k = k0 + (c % BPR) * 8;
        const long g = (long)(row0 + c / BPR) * ldb + kofs + k;
        r.word[u] = bits[g >> 5];
        r.sh[u] = (uint32_t)(g & 31);
        if constexpr (SCALED) r.sc[u] = *reinterpret_cast<const u32x4*>(kscale + kofs + k);
      }
    }
  }
  __device__ __forceinline__ void load(Regs& r, int row0, int k0, int rows, int kend) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      const int row = row0 + c / BPR;
      const int k = k0 + (c % BPR) * 8;
      uint32_t byte = 0;
      u32x4 sc = {0u, 0u, 0u, 0u};
      if (c < ITEMS && row < rows && k < kend) {
        const int nv = kend - k < 8 ? kend - k : 8;
        const long g = (long)row * ldb + kofs + k;
        const uint32_t sh = (uint32_t)(g & 31);
        byte = bits[g >> 5] >> sh;
        // The next word is read only when valid bits spill into it, so the
        // last word of the array is never overrun.
        if (sh + (uint32_t)nv > 32u) byte |= bits[(g >> 5) + 1] << (32u - sh);
        // Out-of-range elements become zero: with a scale, a zero scale; without,
        // the +-1 expansion is masked in store() through sc = 0x3C00 per valid half.
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t base = (j < nv) ? (SCALED ? (uint32_t)kscale[kofs + k + j] : 0x3C00u) : 0u;
          sc[j >> 1] |= base << ((j & 1) * 16);
        }
      }
      r.word[u] = byte;
      r.sh[u] = 0;
      r.sc[u] = sc;
    }
  }
  // Expansion: sign bit 15 of each half is set for a 0 bit (-1 / -scale).
  template <bool FAST>
  __device__ __forceinline__ void store_t(const Regs& r, half_t* s) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (ITEMS % kThreads == 0 || c < ITEMS) {
        const uint32_t byte = r.word[u] >> r.sh[u];
        u32x4 out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t neg = ((~byte >> (2 * j)) & 1u) << 15 | ((~byte >> (2 * j + 1)) & 1u) << 31;
          // Masked elements have a zero base; flipping its sign leaves a zero.
          const uint32_t base = (FAST && !SCALED) ? 0x3C003C00u : r.sc[u][j];
          out[j] = base ^ neg;
        }
        *reinterpret_cast<u32x4*>(&s[(c / BPR) * Lds<BK>::ldk + (c % BPR) * 8]) = out;
      }
    }
  }
  __device__ __forceinline__ void store(const Regs& r, half_t* s) const { store_t<false>(r, s); }
  __device__ __forceinline__ void store_fast(const Regs& r, half_t* s) const { store_t<true>(r, s); }
};

// Loaders other than LoadBits store the same way on both paths.
template <class L>
__device__ __forceinline__ auto store_fast_of(const L& l, const typename L::Regs& r, half_t* s,
                                              int) -> decltype(l.store_fast(r, s)) {
  return l.store_fast(r, s);
}
template <class L>
__device__ __forceinline__ void store_fast_of(const L& l, const typename L::Regs& r, half_t* s,
                                              long) {
  l.store(r, s);
}

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

template <bool FAST, int BM, int BN, int BK, int S, class LA, class LB, int TM, int TN>
__device__ __forceinline__ void gemm_mainloop(const LA& la, const LB& lb, floatx16 (&acc)[TM][TN],
                                              half_t (*sA)[BM * Lds<BK>::ldk],
                                              half_t (*sB)[BN * Lds<BK>::ldk], int m0, int n0,
                                              int kbeg, int kend, int M, int N) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int LDK = Lds<BK>::ldk;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  typename LA::Regs ra[S];
  typename LB::Regs rb[S];
  auto load = [&](typename LA::Regs& a, typename LB::Regs& b, int k0) {
    if constexpr (FAST) {
      la.load_fast(a, m0, k0);
      lb.load_fast(b, n0, k0);
    } else {
      la.load(a, m0, k0, M, kend);
      lb.load(b, n0, k0, N, kend);
    }
  };
  auto store = [&](const typename LA::Regs& a, const typename LB::Regs& b, int buf) {
    if constexpr (FAST) {
      store_fast_of(la, a, sA[buf], 0);
      store_fast_of(lb, b, sB[buf], 0);
    } else {
      la.store(a, sA[buf]);
      lb.store(b, sB[buf]);
    }
  };
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < nk) load(ra[s], rb[s], kbeg + s * BK);
  if (nk > 0) store(ra[0], rb[0], 0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  auto compute = [&](int cur) {
    const half_t* a_t = sA[cur];
    const half_t* b_t = sB[cur];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const half8*>(
            &a_t[(wm * WM + i * 32 + frag_row) * LDK + ks * 16 + frag_k]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const half8*>(
            &b_t[(wn * WN + j * 32 + frag_row) * LDK + ks * 16 + frag_k]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  int kt = 0;
  // Steady state: every step issues its loads and stores unconditionally, so
  // the waits before the LDS stores only cover loads issued S-1 steps earlier.
  for (; kt + 2 * S <= nk; kt += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = kt + s;
      const int cur = t & 1;
      load(ra[s], rb[s], kbeg + (t + S) * BK);
      compute(cur);
      const int nxt = (s + 1) % S;  // constant once the s loop is unrolled
      store(ra[nxt], rb[nxt], cur ^ 1);
      __syncthreads();
    }
  }
  // Tail: the last (fewer than 2 S) tiles, with bounds on every action.
  for (; kt < nk; kt += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = kt + s;  // tile computed now; register slot s held it
      if (t < nk) {
        const int cur = t & 1;
        if (t + S < nk) load(ra[s], rb[s], kbeg + (t + S) * BK);
        compute(cur);
        if (t + 1 < nk) {
          const int nxt = (s + 1) % S;
          store(ra[nxt], rb[nxt], cur ^ 1);
        }
        __syncthreads();
      }
    }
  }
}

template <int BM, int BN, int BK, int S, class LA, class LB, class Epi>
__global__ __launch_bounds__(256) void gemm_kernel(LA la, LB lb, Epi epi, int M, int N, int K,
                                                   int k_split) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int LDK = Lds<BK>::ldk;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(S >= 1, "at least one register stage");
  __shared__ __attribute__((aligned(16))) half_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) half_t sB[2][BN * LDK];

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

  const bool fast = la.fast(m0, M) && lb.fast(n0, N) && (kend - kbeg) % BK == 0;
  if (fast)
    gemm_mainloop<true, BM, BN, BK, S>(la, lb, acc, sA, sB, m0, n0, kbeg, kend, M, N);
  else
    gemm_mainloop<false, BM, BN, BK, S>(la, lb, acc, sA, sB, m0, n0, kbeg, kend, M, N);

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

// Split-K partial: writes fp32 C of split z to part[z][M][N] (z = blockIdx.z
// in gemm_kernel; the streamed-LDS kernels pass their split via set_split).
struct EpiPartial {
  float* part;
  int split = 0;
  __device__ void set_split(int z) { split = z; }
  template <int TM, int TN>
  __device__ void run(floatx16 (&acc)[TM][TN], int row0, int col0, int lane, int M, int N) {
    float* dst = part + (long)blockIdx.z * M * N;
    for_each_acc(acc, row0, col0, lane, M, N,
                 [&](int row, int col, float v) { dst[(long)row * N + col] = v; });
  }
  // 16 consecutive columns of one row (streamed-LDS kernels).
  __device__ void row16(int row, int col, float (&v)[16], int, int M, int N, float*, int, int) {
    if (row >= M) return;
    float* dst = part + (long)split * M * N + (long)row * N + col;
    if (col + 16 <= N && N % 8 == 0 && (reinterpret_cast<uintptr_t>(part) & 15u) == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        floatx4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = v[4 * q + e];
        *reinterpret_cast<floatx4*>(dst + 4 * q) = t;
      }
    } else {
      for (int k = 0; k < 16 && col + k < N; ++k) dst[k] = v[k];
    }
  }
};

// Tile configurations: 128x128 tiles (BK 32, 2 register stages: 16 MFMAs per
// wave per step already cover a load, and a third stage spills) when they
// alone give about one block per CU, else 64x64 tiles (BK 64, 3 stages).
struct CfgLarge {
  static constexpr int bm = 128, bn = 128, bk = 32, stages = 2;
};
struct CfgSmall {
  static constexpr int bm = 64, bn = 64, bk = 64, stages = 3;
};

}  // namespace ullis
