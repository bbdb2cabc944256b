// Streamed-LDS fp16 MFMA GEMM for gfx950:  C[m][n] = sum_k A(m, k) * B(n, k).
//
// Operands move from HBM straight into LDS with global_load_lds_dwordx4 /
// global_load_lds_dword (LDS DMA: lane i of a wave writes 16 or 4 bytes at
// M0 + 16 i or M0 + 4 i), so no registers hold tiles in flight and the K loop
// can keep NS-1 stages of loads outstanding in an NS-buffer LDS ring. Each
// step waits for its own stage with an exact `s_waitcnt vmcnt(n)` (every wave
// issues the same number of loads per stage), then one s_barrier; the loads
// of stage t+NS-1 go out right after that barrier, into the buffer that stage
// t-1 used.
//
// Block = NW wave64s (4 or 8) in a 2 x (NW/2) grid, each owning a (BM/2) x
// (BN/(NW/2)) sub-tile of 32x32 v_mfma_f32_32x32x16_f16 tiles with fp32
// accumulation (the same accumulator layout and epilogue interface as
// gemm.hpp). With 8 waves two run on each SIMD, so one wave's LDS reads and
// waits overlap the other's MFMAs.
//
// Operand layouts in LDS (one stage):
//   OpMK    fp16 [row][k], k contiguous in HBM. LDS rows of BK halves with the
//           16-byte chunks XOR-swizzled by row, so the ds_read_b128 fragment
//           reads of 16 consecutive rows hit 16 distinct 16-byte slots of a
//           256-byte bank window.
//   OpKM    fp16 [k][row], rows contiguous in HBM (a transposed operand, e.g.
//           activations for a weight gradient). LDS keeps [k][row]; fragments
//           come from ds_read_b64_tr_b16, which hands each lane of a 16-lane
//           group 4 k-consecutive values of one row: with lane q of the group
//           pointing at (k0 + q/4, m0 + 4 (q%4)), lane L receives
//           (k0 + j, m0 + L) for j = 0..3. Chunks are swizzled by 2 (k%4).
//   OpBits  LSB-first u32 sign words [row][k/32]; the raw words are streamed
//           (1/16 of the bytes of an fp16 operand) and each fragment expands
//           its 8 bits, one nibble at a time through a 16-entry LDS table of
//           fp16 sign bits, to +-1 fp16, or to +-scale[k] when a per-k scale
//           vector is given (staged in LDS once for the block's K range).
//
// Requirements (checked by the launchers, which fall back to gemm.hpp):
// every split's K range is a multiple of BK, operand pointers are 16-byte
// aligned with row pitches a multiple of 8 halves (4 words for bits), and
// OpKM extents are multiples of 8. Tile rows past M / N read a clamped,
// in-bounds row; their results are never stored.
#pragma once

#include <type_traits>
#include <utility>

#include "common.hpp"
#include "gemm.hpp"
#include "ops.hpp"

namespace ullis {
namespace lds {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void gbl_void_t;

// Per-lane 16-byte (or 4-byte) copy HBM -> LDS at wave-uniform base + lane * size.
__device__ __forceinline__ void dma16(const void* src, char* lds_base) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, char* lds_base) {
  __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)lds_base, 4, 0, 0);
}

// Wait until at most N vector-memory operations of this wave are in flight
// and its LDS operations are done, then barrier. No compiler fence: the
// fence of __syncthreads() would wait for every load in flight.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// fp16 [row][k] with k contiguous.
template <int ROWS, int BK, int NW = 4>
struct OpMK {
  const half_t* p;
  long ld;   // halves between rows
  int rows;  // valid rows (tile rows past it are clamped)
  static constexpr int CPR = BK / 8;  // 16-byte chunks per row
  static constexpr int kBytes = ROWS * BK * 2;
  static_assert(kBytes % (NW * 1024) == 0, "a stage must be whole wave-loads for NW waves");
  static constexpr int kInst = kBytes / (NW * 1024);  // loads per wave per stage
  static constexpr int kExtra = 0;
  static constexpr bool kPlain = true;  // fragments are plain LDS reads
  static constexpr int kFragReads = 1;  // LDS read instructions per fragment
  static constexpr int kNW = NW;        // the block's wave count issue() assumes
  static_assert(CPR == 4 || CPR == 8 || CPR == 16 || CPR == 32, "BK 32, 64, 128 or 256");
  // LDS serves 16 lanes of a ds_read_b128 per cycle from a 256-byte bank
  // window: 16 consecutive rows must land in 16 distinct 16-byte slots.
  // Rows are 64 B (BK 32: 4 rows per window), 128 B (BK 64: 2 per window) or
  // whole windows (BK 128 / 256), so the chunk index is XORed with the row
  // bits above those.
  __device__ static int swz(int row) {
    if constexpr (CPR >= 16)
      return row & 15;
    else if constexpr (CPR == 8)
      return (row >> 1) & 7;
    else
      return (row >> 2) & 3;
  }
  __device__ void prepare(char*, int, int) const {}
  __device__ __forceinline__ void issue(char* stage, int row0, int k0, int wave, int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int id = (wave * kInst + t) * 64 + lane;
      const int row = id / CPR, pos = id % CPR;
      const int c = pos ^ swz(row);
      const int r = min(row0 + row, rows - 1);
      dma16(p + (long)r * ld + k0 + 8 * c, stage + (wave * kInst + t) * 1024);
    }
  }
  // Fragment of the 32-row block starting at tile row `base`, k offset ks16 of
  // the stage: lane l gets row base + l%32, k = ks16 + 8 (l/32) .. +7.
  __device__ __forceinline__ half8 frag(const char* stage, const char*, int base, int ks16,
                                        int lane, int) const {
    const int row = base + (lane & 31);
    const int c = (ks16 >> 3) + (lane >> 5);
    return *reinterpret_cast<const half8*>(stage + row * (BK * 2) + 16 * (c ^ swz(row)));
  }
  // Phases of the pipelined K loop: pre() does the LDS read; lut() and fix()
  // have nothing to do for an fp16 operand.
  using Pre = half8;
  using Raw = half8;
  __device__ __forceinline__ Pre pre(const char* stage, const char* extra, int base, int ks16,
                                     int lane, int k0rel) const {
    return frag(stage, extra, base, ks16, lane, k0rel);
  }
  __device__ __forceinline__ Raw lut(const Pre& p, const char*) const { return p; }
  __device__ __forceinline__ half8 fix(const Raw& r) const { return r; }
};

// fp16 [k][row] with rows contiguous (a transposed operand).
template <int ROWS, int BK, int NW = 4>
struct OpKM {
  const half_t* p;
  long ld;   // halves between k rows
  int rows;  // valid rows (multiple of 8)
  static constexpr int CPR = ROWS / 8;  // chunks per k row
  static_assert(CPR >= 8, "OpKM needs at least 64 rows per tile");
  static constexpr int kBytes = ROWS * BK * 2;
  static_assert(kBytes % (NW * 1024) == 0, "a stage must be whole wave-loads for NW waves");
  static constexpr int kInst = kBytes / (NW * 1024);
  static constexpr int kExtra = 0;
  static constexpr bool kPlain = true;
  static constexpr int kFragReads = 2;
  static constexpr int kNW = NW;
  __device__ static int swz(int k) { return 2 * (k & 3); }
  __device__ void prepare(char*, int, int) const {}
  __device__ __forceinline__ void issue(char* stage, int row0, int k0, int wave, int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int id = (wave * kInst + t) * 64 + lane;
      const int kr = id / CPR, pos = id % CPR;
      const int c = pos ^ swz(kr);
      const int m = min(row0 + 8 * c, rows - 8);
      dma16(p + (long)(k0 + kr) * ld + m, stage + (wave * kInst + t) * 1024);
    }
  }
  // issue() through registers: the same chunks into r (rload), then into the
  // stage at the places the DMA writes them (rstore).
  __device__ __forceinline__ void rload(u32x4 (&r)[kInst], int row0, int k0, int wave,
                                        int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int id = (wave * kInst + t) * 64 + lane;
      const int kr = id / CPR, pos = id % CPR;
      const int c = pos ^ swz(kr);
      const int m = min(row0 + 8 * c, rows - 8);
      r[t] = *reinterpret_cast<const u32x4*>(p + (long)(k0 + kr) * ld + m);
    }
  }
  __device__ __forceinline__ void rstore(const u32x4 (&r)[kInst], char* stage, int wave,
                                         int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t)
      *reinterpret_cast<u32x4*>(stage + (wave * kInst + t) * 1024 + lane * 16) = r[t];
  }
  __device__ __forceinline__ half8 frag(const char* stage, const char*, int base, int ks16,
                                        int lane, int) const {
    const int g = lane >> 4, q = lane & 15;
    const int m = base + 16 * (g & 1) + 4 * (q & 3);
    const int kq = ks16 + 8 * (g >> 1) + (q >> 2);
    const int k0 = kq, k1 = kq + 4;
    const char* a0 = stage + k0 * (ROWS * 2) + 16 * ((m >> 3) ^ swz(k0)) + 2 * (m & 7);
    const char* a1 = stage + k1 * (ROWS * 2) + 16 * ((m >> 3) ^ swz(k1)) + 2 * (m & 7);
    typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const h4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (__attribute__((address_space(3))) h4*)(a0));
    const h4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (__attribute__((address_space(3))) h4*)(a1));
    const u32x2 l = __builtin_bit_cast(u32x2, lo), h = __builtin_bit_cast(u32x2, hi);
    const u32x4 r = {l[0], l[1], h[0], h[1]};
    return __builtin_bit_cast(half8, r);
  }
  using Pre = half8;
  using Raw = half8;
  __device__ __forceinline__ Pre pre(const char* stage, const char* extra, int base, int ks16,
                                     int lane, int k0rel) const {
    return frag(stage, extra, base, ks16, lane, k0rel);
  }
  __device__ __forceinline__ Raw lut(const Pre& p, const char*) const { return p; }
  __device__ __forceinline__ half8 fix(const Raw& r) const { return r; }
};

// Packed sign bits [row][k/32] (LSB-first u32 words, row pitch `ldw` words).
// With `scale` (fp16 bits, indexed by k), bit b becomes +-scale[k] instead of
// +-1. The block's scale range is staged in LDS by prepare().
template <int ROWS, int BK, bool SCALED, int NW = 4>
struct OpBits {
  const uint32_t* p;
  long ldw;  // words between rows
  int rows;
  const uint16_t* scale;  // SCALED only, indexed by kofs + k
  int kofs;               // k offset into the rows (multiple of 32)
  static constexpr int WPR = BK / 32;  // words per row per stage
  static constexpr int kWords = ROWS * WPR;
  // one word per lane per load
  static constexpr int kInst = kWords <= NW * 64 ? 1 : kWords / (NW * 64);
  static_assert(kWords % NW == 0 && (kInst == 1 || kWords % (NW * 64) == 0),
                "bit tile must split into whole wave loads");
  static constexpr int kWordsPerWave = kWords / NW;
  static constexpr int kBytes = ((kWords * 4 + 255) / 256) * 256;
  static constexpr int kMaxScaleK = 8192;
  static constexpr int kNW = NW;
  // extra: 16-entry sign table (128 B), then the scale range when SCALED.
  static constexpr int kLut = 128;
  static constexpr int kExtra = kLut + (SCALED ? kMaxScaleK * 2 : 0);
  // Sign words sit in LDS as [row][WPR] with word w of row r in slot
  // w ^ swzw(r): the 32 rows one fragment read touches then hit 32 distinct
  // banks instead of 32 / WPR.
  __device__ static int swzw(int row) {
    if constexpr (WPR == 1)
      return 0;
    else
      return (row >> (WPR == 2 ? 4 : WPR == 4 ? 3 : 2)) & (WPR - 1);
  }
  __device__ void prepare(char* extra, int kbeg, int kend) const {
    // Entry n (4 weight bits) = 4 halves: +-1 (the sign from bit j of n, 0 is
    // -1) for the plain operand, only the sign bits for the scaled one (they
    // are XORed into the scales). Every entry is 8 bytes, so 16 entries cover
    // the 32 banks of a 128-byte row once: lookups never conflict.
    if (threadIdx.x < 32) {
      const int n = threadIdx.x >> 1, h = threadIdx.x & 1;
      const uint32_t nb = ~(uint32_t)n >> (2 * h);
      const uint32_t sign = ((nb & 1u) << 15) | ((nb & 2u) << 30);
      reinterpret_cast<uint32_t*>(extra)[threadIdx.x] = SCALED ? sign : (sign | 0x3C003C00u);
    }
    if constexpr (SCALED) {
      uint16_t* s = reinterpret_cast<uint16_t*>(extra + kLut);
      for (int k = kbeg + (int)threadIdx.x; k < kend; k += NW * 64) s[k - kbeg] = scale[kofs + k];
    }
  }
  __device__ __forceinline__ void issue(char* stage, int row0, int k0, int wave, int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int base = (wave * kInst + t) * (kWordsPerWave / kInst);
      if (lane < kWordsPerWave / kInst) {
        const int id = base + lane;
        const int row = id / WPR, w = (id % WPR) ^ swzw(row);
        const int r = min(row0 + row, rows - 1);
        dma4(p + (long)r * ldw + ((kofs + k0) >> 5) + w, stage + base * 4);
      }
    }
  }
  // k0rel: the stage's first k relative to the block's kbeg (scale index).
  __device__ __forceinline__ half8 frag(const char* stage, const char* extra, int base, int ks16,
                                        int lane, int k0rel) const {
    const int row = base + (lane & 31);
    const int kk = ks16 + 8 * (lane >> 5);  // k offset within the stage
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const uint32_t word =
        reinterpret_cast<const uint32_t*>(stage)[row * WPR + ((kk >> 5) ^ swzw(row))];
    const int sh = kk & 31;
    const u32x2 lo = *reinterpret_cast<const u32x2*>(extra + 8 * ((word >> sh) & 15u));
    const u32x2 hi = *reinterpret_cast<const u32x2*>(extra + 8 * ((word >> (sh + 4)) & 15u));
    u32x4 o = {lo[0], lo[1], hi[0], hi[1]};
    if constexpr (SCALED) o ^= *reinterpret_cast<const u32x4*>(extra + kLut + 2 * (k0rel + kk));
    return __builtin_bit_cast(half8, o);
  }
  // Phases of the pipelined K loop: pre() reads the lane's 8 sign bits (and
  // its 8 scales), lut() reads their halves from the table, fix() applies
  // the signs to the scales (scaled operand only).
  struct Pre {
    uint32_t word;  // the sign word holding the lane's 8 weight bits
    int sh;         // their offset in it
    u32x4 sc;       // SCALED: the fp16 scales of those 8 inputs
  };
  __device__ __forceinline__ Pre pre(const char* stage, const char* extra, int base, int ks16,
                                     int lane, int k0rel) const {
    const int row = base + (lane & 31);
    const int kk = ks16 + 8 * (lane >> 5);
    Pre p;
    p.word = reinterpret_cast<const uint32_t*>(stage)[row * WPR + ((kk >> 5) ^ swzw(row))];
    p.sh = kk & 31;
    if constexpr (SCALED) {
      p.sc = *reinterpret_cast<const u32x4*>(extra + kLut + 2 * (k0rel + kk));
    } else {
      p.sc = u32x4{0u, 0u, 0u, 0u};
    }
    return p;
  }
  struct Raw {
    u32x4 sign;  // sign bits of the 8 halves
    u32x4 sc;
  };
  __device__ __forceinline__ Raw lut(const Pre& p, const char* extra) const {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const uint32_t bits8 = p.word >> p.sh;
    const u32x2 lo = *reinterpret_cast<const u32x2*>(extra + 8 * (bits8 & 15u));
    const u32x2 hi = *reinterpret_cast<const u32x2*>(extra + 8 * ((bits8 >> 4) & 15u));
    return Raw{u32x4{lo[0], lo[1], hi[0], hi[1]}, p.sc};
  }
  __device__ __forceinline__ half8 fix(const Raw& r) const {
    u32x4 o = r.sign;
    if constexpr (SCALED) o ^= r.sc;
    return __builtin_bit_cast(half8, o);
  }
};

// Packed sign bits [row][k/32] expanded once per stage into an fp16 tile in
// LDS: +-1, or with SCALED +-scale[kofs + k] (the input gradient's operand;
// the block's scale range is staged in LDS by prepare(), as for OpBits). The
// raw words stream in as for OpBits; after the stage has landed, each thread
// expands the words its own loads brought in into the stage's fp16 tile (laid
// out and swizzled as OpMK's), and the fragments are then plain ds_read_b128
// reads. One expansion serves every wave that reads the tile, which pays for
// 256-row tiles (four waves share each column).
template <int ROWS, int BK, int NW = 4, bool SCALED = false>
struct OpBitsX {
  const uint32_t* p;
  long ldw;  // words between rows
  int rows;
  const uint16_t* scale = nullptr;  // SCALED only, indexed by kofs + k
  int kofs = 0;                     // k offset into the rows (multiple of 32)
  static constexpr int WPR = BK / 32;  // words per row per stage
  static constexpr int kWords = ROWS * WPR;
  // one word per lane per load
  static constexpr int kInst = kWords <= NW * 64 ? 1 : kWords / (NW * 64);
  static_assert(kWords % (NW * 64) == 0, "the stage's words must be whole block loads");
  static constexpr int kWordsPerWave = kWords / NW;
  static constexpr int kWordBytes = ((kWords * 4 + 1023) / 1024) * 1024;
  static constexpr int CPR = BK / 8;  // 16-byte chunks per tile row
  static constexpr int kBytes = kWordBytes + ROWS * BK * 2;
  static constexpr int kMaxScaleK = 8192;
  static constexpr int kExtra = SCALED ? kMaxScaleK * 2 : 0;
  static constexpr bool kExpand = true;
  static constexpr bool kPlain = true;
  static constexpr int kFragReads = 1;
  static constexpr int kNW = NW;
  static_assert(CPR == 4 || CPR == 8 || CPR == 16 || CPR == 32, "BK 32, 64, 128 or 256");
  __device__ static int swz(int row) { return OpMK<ROWS, BK, NW>::swz(row); }
  __device__ void prepare(char* extra, int kbeg, int kend) const {
    if constexpr (SCALED) {
      uint16_t* sc = reinterpret_cast<uint16_t*>(extra);
      for (int k = kbeg + (int)threadIdx.x; k < kend; k += NW * 64) sc[k - kbeg] = scale[kofs + k];
    }
  }
  __device__ __forceinline__ void issue(char* stage, int row0, int k0, int wave, int lane) const {
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int id = (wave * kInst + t) * 64 + lane;
      const int row = id / WPR, w = id % WPR;
      const int r = min(row0 + row, rows - 1);
      dma4(p + (long)r * ldw + ((kofs + k0) >> 5) + w, stage + (wave * kInst + t) * 256);
    }
  }
  // Word id (row id / WPR, k 32 (id % WPR) .. +31) -> four 16-byte chunks of
  // the tile; bit j (LSB first) is +1 (+scale) when set, -1 (-scale) when
  // clear. Each thread expands the words its own loads brought in (issue()'s
  // ids), so once its own loads have landed it needs no barrier before
  // expanding. k0rel: the stage's first k relative to the block's first.
  __device__ __forceinline__ void expand(char* stage, const char* extra, int k0rel, int wave,
                                         int lane) const {
    char* tile = stage + kWordBytes;
#pragma unroll
    for (int t = 0; t < kInst; ++t) {
      const int id = (wave * kInst + t) * 64 + lane;
      const uint32_t word = reinterpret_cast<const uint32_t*>(stage)[id];
      const int row = id / WPR, w = id % WPR;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t byte = word >> (8 * q);
        u32x4 o;
        if constexpr (SCALED) {
          // the sign bit of each half flips where the weight bit is clear
          const u32x4 sc =
              *reinterpret_cast<const u32x4*>(extra + 2 * (k0rel + 32 * w + 8 * q));
#pragma unroll
          for (int m = 0; m < 4; ++m)
            o[m] = sc[m] ^ ((((~byte) >> (2 * m)) & 1u) << 15) ^
                   ((((~byte) >> (2 * m + 1)) & 1u) << 31);
        } else {
#pragma unroll
          for (int m = 0; m < 4; ++m)
            o[m] = 0xBC00BC00u ^ (((byte >> (2 * m)) & 1u) << 15) ^
                   (((byte >> (2 * m + 1)) & 1u) << 31);
        }
        const int c = 4 * w + q;
        *reinterpret_cast<u32x4*>(tile + row * (BK * 2) + 16 * (c ^ swz(row))) = o;
      }
    }
  }
  __device__ __forceinline__ half8 frag(const char* stage, const char*, int base, int ks16,
                                        int lane, int) const {
    const int row = base + (lane & 31);
    const int c = (ks16 >> 3) + (lane >> 5);
    return *reinterpret_cast<const half8*>(stage + kWordBytes + row * (BK * 2) +
                                           16 * (c ^ swz(row)));
  }
  using Pre = half8;
  using Raw = half8;
  __device__ __forceinline__ Pre pre(const char* stage, const char* extra, int base, int ks16,
                                     int lane, int k0rel) const {
    return frag(stage, extra, base, ks16, lane, k0rel);
  }
  __device__ __forceinline__ Raw lut(const Pre& p, const char*) const { return p; }
  __device__ __forceinline__ half8 fix(const Raw& r) const { return r; }
};

template <class O>
inline constexpr bool kIsKM = false;
template <int R, int B, int W>
inline constexpr bool kIsKM<OpKM<R, B, W>> = true;

// Operands that expand a landed stage in LDS before its fragments are read.
template <class O, class = void>
inline constexpr bool kExpands = false;
template <class O>
inline constexpr bool kExpands<O, std::enable_if_t<O::kExpand>> = true;

// Operands whose fragments are plain LDS reads (no sign table, no per-k
// scales): the interleaved K loop takes these.
template <class O, class = void>
inline constexpr bool kPlainFrag = false;
template <class O>
inline constexpr bool kPlainFrag<O, std::enable_if_t<O::kPlain>> = true;

// s_waitcnt vmcnt(IPS * later), no barrier, for a runtime `later` in [0, S].
template <int IPS, int S>
__device__ __forceinline__ void wait_vm_stages(int later) {
  if constexpr (S == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    if (later >= S)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(IPS * S) : "memory");
    else
      wait_vm_stages<IPS, S - 1>(later);
  }
}

// wait_barrier<IPS * later>() for a runtime `later` in [0, S] (the K-loop tail).
template <int IPS, int S>
__device__ __forceinline__ void wait_stages(int later) {
  if constexpr (S == 0) {
    wait_barrier<0>();
  } else {
    if (later >= S)
      wait_barrier<IPS * S>();
    else
      wait_stages<IPS, S - 1>(later);
  }
}

// ------------------------------------------------------------ epilogue
// Row-wise epilogue: each 32x32 accumulator block of a wave is scattered into
// a per-wave LDS buffer [32][kBufPitch] fp32 and read back so that lane l
// holds row l/2, columns 16 (l%2) .. +15 of the block. The epilogue functor's
// row16(row, col, v, lane, M, N, buf, brow, bcol) then works on 16 consecutive
// columns of one row (vector loads / stores, in-register row reductions);
// (brow, bcol) is the block origin and buf the block in LDS, which a functor
// may overwrite for column reductions (it must leave the lanes in step).
constexpr int kBufPitch = 36;  // floats; 144-byte rows keep both passes conflict-light
constexpr int kBufFloats = 32 * kBufPitch;

__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Epilogues that read global memory per 16-value row segment (a residual, a
// tape) may define `Pre` with `pre16(row, col, M, N)`, which issues those
// loads, and `row16p(..., const Pre&, ...)`, which consumes them: the driver
// then issues the loads of up to kEpiAhead segments ahead of the one it
// stores, so their latency overlaps instead of adding up segment by segment.
template <class E, class = void>
inline constexpr bool kHasPre16 = false;
template <class E>
inline constexpr bool kHasPre16<E, std::void_t<typename E::Pre>> = true;
constexpr int kEpiAhead = 4;

template <class Epi, int TM, int TN>
__device__ __forceinline__ void epilogue_rows(Epi& epi, floatx16 (&acc)[TM][TN], float* buf,
                                              int row0, int col0, int lane, int M, int N) {
  const int rr = lane >> 1, cc = (lane & 1) * 16;
  if constexpr (kHasPre16<Epi>) {
    constexpr int S = TM * TN;
    constexpr int P = S < kEpiAhead ? S : kEpiAhead;
    typename Epi::Pre ring[P];
    auto at = [&](int sidx, int& r, int& c) {
      r = row0 + (sidx / TN) * 32 + rr;
      c = col0 + (sidx % TN) * 32 + cc;
    };
#pragma unroll
    for (int t = 0; t < P; ++t) {
      int r, c;
      at(t, r, c);
      ring[t] = epi.pre16(r, c, M, N);
    }
#pragma unroll
    for (int sidx = 0; sidx < S; ++sidx) {
      const int i = sidx / TN, j = sidx % TN;
#pragma unroll
      for (int r = 0; r < 16; ++r) buf[mfma32_row(r, lane) * kBufPitch + (lane & 31)] = acc[i][j][r];
      lds_fence();
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 t = *reinterpret_cast<const floatx4*>(buf + rr * kBufPitch + cc + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
      }
      lds_fence();
      const int brow = row0 + i * 32, bcol = col0 + j * 32;
      const typename Epi::Pre cur = ring[sidx % P];
      if (sidx + P < S) {
        int r, c;
        at(sidx + P, r, c);
        ring[sidx % P] = epi.pre16(r, c, M, N);
      }
      epi.row16p(brow + rr, bcol + cc, v, cur, lane, M, N, buf, brow, bcol);
      lds_fence();
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) buf[mfma32_row(r, lane) * kBufPitch + (lane & 31)] = acc[i][j][r];
      lds_fence();
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 t = *reinterpret_cast<const floatx4*>(buf + rr * kBufPitch + cc + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
      }
      lds_fence();
      const int brow = row0 + i * 32, bcol = col0 + j * 32;
      epi.row16(brow + rr, bcol + cc, v, lane, M, N, buf, brow, bcol);
      lds_fence();
    }
}

// 16 consecutive fp16 / fp32 values at p (16-byte aligned).
__device__ __forceinline__ void load16h(const uint16_t* p, float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const half8 h = *reinterpret_cast<const half8*>(p + 8 * q);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[8 * q + e] = (float)h[e];
  }
}
__device__ __forceinline__ void store16h(uint16_t* p, const float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (half_t)v[8 * q + e];
    *reinterpret_cast<half8*>(p + 8 * q) = h;
  }
}
__device__ __forceinline__ void load16f(const float* p, float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const floatx4 t = *reinterpret_cast<const floatx4*>(p + 4 * q);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
  }
}
__device__ __forceinline__ void store16f(float* p, const float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    floatx4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = v[4 * q + e];
    *reinterpret_cast<floatx4*>(p + 4 * q) = t;
  }
}

__device__ __forceinline__ bool al16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
// p[col .. col+15] as float; entries past n read as 0. vec: whole and aligned.
__device__ __forceinline__ void get16h(const uint16_t* p, int col, int n, bool vec,
                                       float (&v)[16]) {
  if (vec) {
    load16h(p + col, v);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = col + k < n ? f16_bits_to_f32(p[col + k]) : 0.0f;
  }
}

// XCD-aware tile order. Blocks are dealt round-robin to the 8 XCDs
// (bid % 8), each with its own L2, and the blocks of one XCD run together. XCD
// x takes one rectangle of gm x gn output tiles (gm | tiles_m, gn | tiles_n,
// gm * gn = tiles / 8, all powers of two) that minimises the operand bytes
// its L2 streams, gm * wa + gn * wb (wa / wb: bytes of one tile row of A /
// one tile column of B per K step); row-major inside the rectangle. The
// host picks the rectangle (tile_map); other tile counts keep the row-major
// order.
struct TileMap {
  int log_gm = -1;  // < 0: row-major order
  int log_gn = 0, log_groups_n = 0;
};

inline int log2_exact(long v) {  // log2 of a power of two, else -1
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int l = 0;
  while ((1L << l) < v) ++l;
  return l;
}

inline TileMap tile_map(long tiles_m, long tiles_n, long wa, long wb) {
  TileMap m;
  const long total = tiles_m * tiles_n;
  if (total % 8 != 0) return m;
  const long per = total / 8;
  long best = -1;
  for (long gm = 1; gm <= tiles_m && gm <= per; gm *= 2) {
    if (tiles_m % gm != 0 || per % gm != 0) continue;
    const long gn = per / gm;
    if (tiles_n % gn != 0 || log2_exact(gn) < 0 || log2_exact(tiles_n / gn) < 0) continue;
    const long cost = gm * wa + gn * wb;
    if (best < 0 || cost < best) {
      best = cost;
      m.log_gm = log2_exact(gm);
      m.log_gn = log2_exact(gn);
      m.log_groups_n = log2_exact(tiles_n / gn);
    }
  }
  return m;
}

__device__ __forceinline__ void tile_of_block_map(int bid, int tiles_n, const TileMap& map,
                                                  int& tm, int& tn) {
  if (map.log_gm >= 0) {
    const int xcd = bid & 7, local = bid >> 3;
    tm = ((xcd >> map.log_groups_n) << map.log_gm) + (local >> map.log_gn);
    tn = ((xcd & ((1 << map.log_groups_n) - 1)) << map.log_gn) + (local & ((1 << map.log_gn) - 1));
  } else {
    tm = bid / tiles_n;
    tn = bid - tm * tiles_n;
  }
}

template <class T, class OA, class OB>
TileMap tile_map_for(long M, long N) {
  return tile_map(cdiv(M, T::bm), cdiv(N, T::bn), OA::kBytes, OB::kBytes);
}

// Epilogues of split-K outputs take the block's K split through set_split(kz).
template <class E, class = void>
inline constexpr bool kHasSplit = false;
template <class E>
inline constexpr bool kHasSplit<E, decltype(std::declval<E&>().set_split(0))> = true;

// Ring depth of a config for an operand pair: the config's stage count, cut
// to what fits in kRingCap bytes (a deep ring of sign-bit stages is cheap; of
// fp16 stages it is not).
constexpr int kRingCap = 128 * 1024;
template <int NS, class OA, class OB>
constexpr int ring_ns() {
  constexpr int STAGE = OA::kBytes + OB::kBytes;
  return NS * STAGE <= kRingCap ? NS : (kRingCap / STAGE < 2 ? 2 : kRingCap / STAGE);
}

// LDS bytes of one block of the streamed-LDS GEMM: the stage ring (which the
// epilogue reuses) and the operands' extra tables.
template <int BM, int BN, int BK, int NS_CFG, class OA, class OB, int NW = 4>
constexpr int lds_ring_bytes() {
  constexpr int STAGE = OA::kBytes + OB::kBytes;
  constexpr int NS = ring_ns<NS_CFG, OA, OB>();
  return NS * STAGE > NW * kBufFloats * 4 ? NS * STAGE : NW * kBufFloats * 4;
}
template <int BM, int BN, int BK, int NS, class OA, class OB, int NW = 4>
constexpr int lds_smem_bytes() {
  return lds_ring_bytes<BM, BN, BK, NS, OA, OB, NW>() + OA::kExtra + OB::kExtra;
}

// Tiles with at least this many MFMAs per wave per 16-deep step and plain
// fragment operands take the interleaved K loop (128x128 four-wave tiles
// included: config 4's value backward pair 22.2 -> 22.0 us).
constexpr int kInterleaveMfmas = 4;
template <int BM, int BN, int BK, class OA, class OB, int NW>
inline constexpr bool kInterleaved = kPlainFrag<OA> && kPlainFrag<OB> && BK >= 32 &&
                                     (BM / 64) * (BN / (NW * 16)) >= kInterleaveMfmas;

// The interleaved K loop for large tiles. A wave's MFMAs of one 16-deep step
// are issued with the LDS fragment reads of the next step between them, so the
// reads complete while the MFMA pipe is busy instead of before it starts. Each
// stage has one barrier, before its last step: by then every wave has read the
// whole stage (its buffer is refilled with stage kt + NS right after) and has
// waited for stage kt + 1 to land (and expanded it, for sign-bit operands), so
// the last step's MFMAs overlap the first reads of the next stage. Every
// output sums the same products in the same k order as gemm_lds_body's loop.
template <int BM, int BN, int BK, int NS_CFG, class OA, class OB, class Epi, int NW>
__device__ __forceinline__ void gemm_lds_body_il(char* smem, int bid, int kz, const OA& a,
                                                 const OB& b, Epi& epi, int M, int N, int K,
                                                 int k_split, const TileMap& map) {
  constexpr int NS = ring_ns<NS_CFG, OA, OB>();
  static_assert(OA::kNW == NW && OB::kNW == NW, "operands built for another wave count");
  constexpr int WGN = NW / 2;
  constexpr int WM = BM / 2, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = OA::kBytes + OB::kBytes;
  constexpr int IPS = OA::kInst + OB::kInst;
  constexpr int S = BK / 16;
  static_assert(S >= 2 && S % 2 == 0, "an even number of 16-deep steps per stage");
  static_assert(NS >= 2 && IPS * (NS - 1) < 64, "pipeline depth");
  constexpr int RING = lds_ring_bytes<BM, BN, BK, NS_CFG, OA, OB, NW>();
  char* extra_a = smem + RING;
  char* extra_b = extra_a + OA::kExtra;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of_block_map(bid, tiles_n, map, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = kz * k_split;
  const int kend = min(K, kbeg + k_split);
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (floatx16){};

  a.prepare(extra_a, kbeg, kend);
  b.prepare(extra_b, kbeg, kend);
  // staged tables (scales) are read by other threads' expansions
  if constexpr (OA::kExtra > 0 || OB::kExtra > 0)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  auto stage_at = [&](int kt) { return smem + (kt % NS) * STAGE; };
  // Loads of stage `kt` into its ring buffer; stages past the last reload the
  // last one (in bounds, never read), so every wave issues the same loads in
  // every iteration and each wait below is one fixed vmcnt, with no branch
  // to split the interleaved instruction stream.
  auto issue = [&](int kt) {
    char* st = stage_at(kt);
    const int k0 = kbeg + min(kt, nk - 1) * BK;
    a.issue(st, m0, k0, wave, lane);
    b.issue(st + OA::kBytes, n0, k0, wave, lane);
  };
  auto expand = [&](int kt) {
    const int k0rel = min(kt, nk - 1) * BK;  // the stage issue() loaded
    if constexpr (kExpands<OA>) a.expand(stage_at(kt), extra_a, k0rel, wave, lane);
    if constexpr (kExpands<OB>) b.expand(stage_at(kt) + OA::kBytes, extra_b, k0rel, wave, lane);
  };
  half8 fa[2][TM], fb[2][TN];
  auto read = [&](int kt, int s, half8(&af)[TM], half8(&bf)[TN]) {
    const char* st = stage_at(kt);
#pragma unroll
    for (int i = 0; i < TM; ++i) af[i] = a.frag(st, extra_a, wm * WM + i * 32, 16 * s, lane, 0);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      bf[j] = b.frag(st + OA::kBytes, extra_b, wn * WN + j * 32, 16 * s, lane, 0);
  };
  auto mma = [&](const half8(&af)[TM], const half8(&bf)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
  };
  // Issue order inside a step: MFMAs in pairs, one fragment read (and, in
  // the last step of a stage, one operand load) after each pair.
  constexpr int kReads = TM * OA::kFragReads + TN * OB::kFragReads;
  auto interleave = [&](bool loads) {
    constexpr int P = TM * TN / 2;
    constexpr int Q = P > kReads ? (P > IPS ? P : IPS) : (kReads > IPS ? kReads : IPS);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (q < P) __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);            // MFMA
      if (q < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // LDS read
      if (loads && q < IPS) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    }
  };

  if (nk > 0) {
    // prologue: fill the whole ring, wait for stage 0, read its first step
#pragma unroll
    for (int s = 0; s < NS; ++s) issue(s);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(IPS * (NS - 1)) : "memory");
    expand(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read(0, 0, fa[0], fb[0]);
  }
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int s = 0; s < S - 1; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      mma(fa[s & 1], fb[s & 1]);
      read(kt, s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
      interleave(false);
      __builtin_amdgcn_sched_barrier(0);
    }
    // this wave's reads of stage kt are complete (lgkmcnt); stage kt + 1 has
    // landed (vmcnt): expand it, then the barrier frees buffer kt for stage
    // kt + NS
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(IPS * (NS - 2)) : "memory");
    expand(kt + 1);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue(kt + NS);
    mma(fa[(S - 1) & 1], fb[(S - 1) & 1]);
    read(kt + 1, 0, fa[0], fb[0]);  // past the last stage: a stale buffer, never used
    interleave(true);
    __builtin_amdgcn_sched_barrier(0);
  }
  wait_barrier<0>();  // every wave is done reading the ring
  if constexpr (kHasSplit<Epi>) epi.set_split(kz);
  epilogue_rows(epi, acc, reinterpret_cast<float*>(smem) + wave * kBufFloats, m0 + wm * WM,
                n0 + wn * WN, lane, M, N);
}

// One output tile (bid: tile index, kz: K split) of C = A . B^T in the block's
// LDS (smem: lds_smem_bytes, 1024-byte aligned).
template <int BM, int BN, int BK, int NS_CFG, class OA, class OB, class Epi, int NW = 4>
__device__ __forceinline__ void gemm_lds_body(char* smem, int bid, int kz, const OA& a,
                                              const OB& b, Epi& epi, int M, int N, int K,
                                              int k_split, const TileMap& map) {
  constexpr int NS = ring_ns<NS_CFG, OA, OB>();
  // Eight waves (a 2 x 4 grid) run only on the interleaved loop. (An early
  // eight-wave trial returned non-finite products because its operands were
  // built for four waves: waves 4-7 loaded past the stage. The kNW check
  // below rules that out.)
  static_assert(NW == 4 || kInterleaved<BM, BN, BK, OA, OB, NW>, "wave count");
  static_assert(OA::kNW == NW && OB::kNW == NW, "operands built for another wave count");
  if constexpr (kInterleaved<BM, BN, BK, OA, OB, NW>) {
    gemm_lds_body_il<BM, BN, BK, NS_CFG, OA, OB, Epi, NW>(smem, bid, kz, a, b, epi, M, N, K,
                                                          k_split, map);
    return;
  }
  constexpr int WGN = NW / 2;  // waves along N
  constexpr int WM = BM / 2, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = OA::kBytes + OB::kBytes;
  constexpr int IPS = OA::kInst + OB::kInst;  // loads per wave per stage
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(NS >= 2 && IPS * (NS - 2) < 64, "pipeline depth");
  constexpr int RING = lds_ring_bytes<BM, BN, BK, NS_CFG, OA, OB, NW>();
  char* extra_a = smem + RING;
  char* extra_b = extra_a + OA::kExtra;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of_block_map(bid, tiles_n, map, tm, tn);
  (void)tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = kz * k_split;
  const int kend = min(K, kbeg + k_split);
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (floatx16){};

  a.prepare(extra_a, kbeg, kend);
  b.prepare(extra_b, kbeg, kend);
  auto issue = [&](int kt) {
    char* st = smem + (kt % NS) * STAGE;
    a.issue(st, m0, kbeg + kt * BK, wave, lane);
    b.issue(st + OA::kBytes, n0, kbeg + kt * BK, wave, lane);
  };
  // Two transposed operands on a two-stage ring (the 64x64 weight gradients)
  // are staged through registers instead of the DMA: a stage's loads go out
  // three steps before its MFMAs, and are stored into LDS the step before
  // (config 4's value backward pair 22.0 -> 20.4 us). The register ring has
  // two slots, so that K loop runs in pairs of steps (slot indices stay
  // compile-time), with an odd last step peeled off; every other operand pair
  // keeps the one-step loop (the pairs cost config 5's head logits, on this
  // loop over sign bits, 11 -> 15 ms).
  constexpr bool kRegStage = kIsKM<OA> && kIsKM<OB> && NS == 2;
  u32x4 ra0[OA::kInst], ra1[OA::kInst], rb0[OB::kInst], rb1[OB::kInst];
  if constexpr (kRegStage) {
    // stage 0 through the registers into LDS, then stages 1 and 2 into them
    // (none for a block with an empty K range: its loop does not run)
    if (nk > 0) {
      a.rload(ra1, m0, kbeg, wave, lane);
      b.rload(rb1, n0, kbeg, wave, lane);
      a.rstore(ra1, smem, wave, lane);
      b.rstore(rb1, smem + OA::kBytes, wave, lane);
      const int k1 = 1 < nk ? 1 : nk - 1, k2 = 2 < nk ? 2 : nk - 1;
      a.rload(ra1, m0, kbeg + k1 * BK, wave, lane);
      b.rload(rb1, n0, kbeg + k1 * BK, wave, lane);
      a.rload(ra0, m0, kbeg + k2 * BK, wave, lane);
      b.rload(rb0, n0, kbeg + k2 * BK, wave, lane);
    }
  } else {
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < nk) issue(s);
  }

  // One K step: P is the parity of kt (which register slot holds stage kt + 1).
  auto step = [&](int kt, auto parity) {
    if constexpr (kRegStage) {
      constexpr int P = decltype(parity)::value;
      // every wave's stores of stage kt are done, and its reads of stage
      // kt - 1 (the slot stage kt + 1 now takes)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int k3 = kt + 3 < nk ? kt + 3 : nk - 1;  // past the end: the last stage again
      char* st1 = smem + ((kt + 1) % NS) * STAGE;
      auto& rsa = P == 0 ? ra1 : ra0;
      auto& rsb = P == 0 ? rb1 : rb0;
      a.rstore(rsa, st1, wave, lane);
      b.rstore(rsb, st1 + OA::kBytes, wave, lane);
      a.rload(rsa, m0, kbeg + k3 * BK, wave, lane);
      b.rload(rsb, n0, kbeg + k3 * BK, wave, lane);
    } else {
      (void)parity;
      // Stage kt is complete once at most the later stages' loads are in flight.
      wait_stages<IPS, NS - 2>(nk - 1 - kt);
      if (kt + NS - 1 < nk) issue(kt + NS - 1);
    }
    if constexpr (kExpands<OA> || kExpands<OB>) {
      // the stage's words have landed for every wave: expand them, then
      // barrier again (LDS writes only; the loads in flight stay in flight)
      if constexpr (kExpands<OA>) a.expand(smem + (kt % NS) * STAGE, extra_a, kt * BK, wave, lane);
      if constexpr (kExpands<OB>)
        b.expand(smem + (kt % NS) * STAGE + OA::kBytes, extra_b, kt * BK, wave, lane);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const char* st = smem + (kt % NS) * STAGE;
    const int k0rel = kt * BK;
    // Software pipeline over the stage's 16-deep K steps. Step s's MFMAs use
    // sign patterns read from the table kLut steps earlier, whose LDS words
    // were read kLut + 1 steps earlier (an fp16 operand is read kLut + 1
    // steps early). Scheduling barriers keep the LDS reads of later steps
    // ahead of this step's MFMAs, so the LDS latency hides behind the MFMAs
    // of the steps in between: at these tile sizes a wave runs alone on its
    // SIMD, and nothing else would hide it.
    constexpr int S = BK / 16;
    // how many steps ahead a sign-bit fragment's table lookup runs: with one
    // wave per SIMD the pipeline alone hides the LDS latency; with two, the
    // other wave does, and a deep register ring would only cut occupancy
    constexpr int kDepth = NW == 4 ? 3 : 1;
    constexpr int kLut = S > kDepth ? kDepth : S - 1;
    constexpr int kPre = kLut + 1;
    constexpr int RP = kPre + 1, RR = kLut + 1;  // ring sizes
    typename OA::Pre pa[RP][TM];
    typename OB::Pre pb[RP][TN];
    typename OA::Raw ra[RR][TM];
    typename OB::Raw rb[RR][TN];
    auto pre = [&](int s) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        pa[s % RP][i] = a.pre(st, extra_a, wm * WM + i * 32, 16 * s, lane, k0rel);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        pb[s % RP][j] = b.pre(st + OA::kBytes, extra_b, wn * WN + j * 32, 16 * s, lane, k0rel);
    };
    auto lut = [&](int s) {
#pragma unroll
      for (int i = 0; i < TM; ++i) ra[s % RR][i] = a.lut(pa[s % RP][i], extra_a);
#pragma unroll
      for (int j = 0; j < TN; ++j) rb[s % RR][j] = b.lut(pb[s % RP][j], extra_b);
    };
#pragma unroll
    for (int t = 0; t < kPre && t < S; ++t) pre(t);
#pragma unroll
    for (int t = 0; t < kLut; ++t) lut(t);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (s + kPre < S) pre(s + kPre);
      if (s + kLut < S) lut(s + kLut);
      __builtin_amdgcn_sched_barrier(0);
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = a.fix(ra[s % RR][i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = b.fix(rb[s % RR][j]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (kRegStage) {
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      step(kt, std::integral_constant<int, 0>{});
      step(kt + 1, std::integral_constant<int, 1>{});
    }
    if (kt < nk) step(kt, std::integral_constant<int, 0>{});
  } else {
    for (int kt = 0; kt < nk; ++kt) step(kt, std::integral_constant<int, 0>{});
  }
  wait_barrier<0>();  // every wave is done reading the ring
  if constexpr (kHasSplit<Epi>) epi.set_split(kz);
  epilogue_rows(epi, acc, reinterpret_cast<float*>(smem) + wave * kBufFloats, m0 + wm * WM,
                n0 + wn * WN, lane, M, N);
}

template <int BM, int BN, int BK, int NS, class OA, class OB, class Epi, int NW = 4>
__global__ __launch_bounds__(NW * 64) void gemm_lds_kernel(OA a, OB b, Epi epi, int M, int N,
                                                           int K, int k_split, TileMap map,
                                                           unsigned long long* stamps) {
  __shared__ __attribute__((aligned(1024)))
  char smem[lds_smem_bytes<BM, BN, BK, NS, OA, OB, NW>()];
  stamp_block_start(stamps);
  gemm_lds_body<BM, BN, BK, NS, OA, OB, Epi, NW>(smem, blockIdx.x, blockIdx.z, a, b, epi, M, N, K,
                                                 k_split, map);
  stamp_block_end(stamps);
}

template <class T, int G>
struct Group {
  T v[G];
};

// G independent problems of one shape in one launch (blockIdx.y = problem).
template <int BM, int BN, int BK, int NS, class OA, class OB, class Epi, int G, int NW = 4>
__global__ __launch_bounds__(NW * 64) void gemm_lds_group_kernel(Group<OA, G> a, Group<OB, G> b,
                                                                 Group<Epi, G> epi, int M, int N,
                                                                 int K, int k_split, TileMap map,
                                                                 unsigned long long* stamps) {
  __shared__ __attribute__((aligned(1024)))
  char smem[lds_smem_bytes<BM, BN, BK, NS, OA, OB, NW>()];
  const int g = blockIdx.y;
  stamp_block_start(stamps);
  gemm_lds_body<BM, BN, BK, NS, OA, OB, Epi, NW>(smem, blockIdx.x, blockIdx.z, a.v[g], b.v[g],
                                                 epi.v[g], M, N, K, k_split, map);
  stamp_block_end(stamps);
}

// One GEMM of a pair launch: tile config T, operands, epilogue and shape;
// tiles * splits blocks.
template <class T, class OA, class OB, class Epi>
struct LdsProblem {
  OA a;
  OB b;
  Epi epi;
  int M, N, K, k_split, tiles, blocks;
  TileMap map;
};

constexpr int max_of(int a) { return a; }
template <class... R>
constexpr int max_of(int a, R... r) {
  const int m = max_of(r...);
  return a > m ? a : m;
}

template <class P>
struct LdsProblemSmem;
template <class T, class OA, class OB, class Epi>
struct LdsProblemSmem<LdsProblem<T, OA, OB, Epi>> {
  static constexpr int value = lds_smem_bytes<T::bm, T::bn, T::bk, T::ns, OA, OB, T::nw>();
  static constexpr int nw = T::nw;
};

template <class T, class OA, class OB, class Epi>
__device__ __forceinline__ void run_lds_problem(char* smem, const LdsProblem<T, OA, OB, Epi>& p,
                                                int bid) {
  const int z = p.blocks == p.tiles ? 0 : bid / p.tiles;
  Epi epi = p.epi;
  gemm_lds_body<T::bm, T::bn, T::bk, T::ns, OA, OB, Epi, T::nw>(smem, bid - z * p.tiles, z, p.a,
                                                                 p.b, epi, p.M, p.N, p.K,
                                                                 p.k_split, p.map);
}

// Independent GEMMs (possibly of different tile configs, operand kinds and
// epilogues) in one launch: the first ps[0].blocks blocks run ps[0], the next
// ps[1].blocks run ps[1], ..., so the blocks of all of them share the CUs.
// The problems of one launch share the wave count (launch_lds_multi launches
// problems of different wave counts one after another instead).
template <class... Ps>
constexpr int multi_nw() {
  constexpr int nw[] = {LdsProblemSmem<Ps>::nw...};
  for (int w : nw)
    if (w != nw[0]) return -1;
  return nw[0];
}

template <class... Ps>
__global__ __launch_bounds__(multi_nw<Ps...>() * 64) void gemm_lds_multi_kernel(
    unsigned long long* stamps, Ps... ps) {
  static_assert(multi_nw<Ps...>() > 0, "the problems of one launch share the wave count");
  constexpr int S = max_of(LdsProblemSmem<Ps>::value...);
  __shared__ __attribute__((aligned(1024))) char smem[S];
  int bid = blockIdx.x;
  bool done = false;
  stamp_block_start(stamps);
  auto one = [&](const auto& p) {
    if (done) return;
    if (bid < p.blocks) {
      run_lds_problem(smem, p, bid);
      done = true;
    } else {
      bid -= p.blocks;
    }
  };
  (one(ps), ...);
  stamp_block_end(stamps);
}

// ------------------------------------------------------------ host dispatch
// Measured on MI355X for the heron shapes (2048 rows): 64x64 tiles with BK 64
// beat 128x128 tiles (one block per CU) everywhere except very wide outputs
// (the vocab head), where 128x128 tiles win; a 4-stage ring was best inside
// the train step (2, 3 and 6 stages were slower).
// Tile configs: 64x64 output tiles (one 32x32 MFMA block per wave). A
// two-stage ring of BK = 128 halves the barrier round trips per MFMA of a
// four-stage ring of BK = 64 in the same 64 KiB of LDS (two blocks per CU),
// and measured faster at every heron shape (value fwd 12.7 -> 11.8 us, value
// dW 16.7 -> 13.7 us, head dW 46.7 -> 36.8 us); 128x128 tiles were slower or
// equal. BK = 64 serves contraction lengths that are not multiples of 128.
struct LdsMid {
  static constexpr int bm = 64, bn = 64, bk = 128, ns = 2, nw = 4;
};
struct LdsShort {
  static constexpr int bm = 64, bn = 64, bk = 64, ns = 4, nw = 4;
};
struct LdsDeep {
  static constexpr int bm = 64, bn = 64, bk = 128, ns = 4, nw = 4;
};
struct LdsBig {
  static constexpr int bm = 128, bn = 128, bk = 32, ns = 4, nw = 4;
};
struct LdsHuge {
  static constexpr int bm = 128, bn = 256, bk = 32, ns = 4, nw = 4;
};
struct LdsGiant {
  static constexpr int bm = 256, bn = 256, bk = 32, ns = 4, nw = 4;
};
// 256x256 tiles over sign bits expanded in LDS: BK 64 halves the expansion
// barriers and makes every row's stage segment a whole 128-byte line (config-5
// key forward 400 -> 377 us; the fp16 forward measured 310 -> 318-328 us
// with it, so it keeps LdsGiant), and eight waves, two per SIMD (the packed
// forward alone 396 -> 362 us; the fp16 forward 343 -> 351 us with them).
struct LdsGiantBits {
  static constexpr int bm = 256, bn = 256, bk = 64, ns = 2, nw = 8;
};
// 128x256 tiles of eight waves (64x64 per wave, two waves per SIMD): config
// 5's value dX from the value^T cache (its pair 995 -> 969 us).
struct LdsHuge8 {
  static constexpr int bm = 128, bn = 256, bk = 32, ns = 4, nw = 8;
};
// 256x256 tiles of eight waves for the weight gradients over many rows
// (paired in one launch with the input gradients' eight-wave tiles).
struct LdsGiant8 {
  static constexpr int bm = 256, bn = 256, bk = 32, ns = 4, nw = 8;
};

constexpr long kBigAutoBlocks = 512;
constexpr long kHugeAutoBlocks = 1024;
constexpr long kGiantAutoBlocks = 512;
// Per-call-site choice (with_lds): kAuto = LdsBig for large products, else
// LdsMid / LdsShort by K; kDeep =
// the four-stage BK 128 ring for launches of one block per CU whose operands
// come from HBM; kBig = 128x128 tiles; kNoBig = kAuto without the 128x128
// rule (config 4's head logits, 1024 such tiles: 64x64 tiles measured faster,
// the head op 170 -> 156 us). 256x256 tiles are not chosen here: the call
// sites that want them (giant_ok) name them, so that no pair launch carries
// an unused four-wave 256x256 problem.
enum class LdsPolicy { kAuto, kDeep, kBig, kNoBig };

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool mk_ok(const void* p, long ld) { return p && aligned16(p) && ld % 8 == 0; }
inline bool km_ok(const void* p, long ld, long rows) {
  return p && aligned16(p) && ld % 8 == 0 && rows % 8 == 0 && rows >= 8;
}

// Runs f(T) with the streamed-LDS tile config for an M x N output when K
// splits into whole BK steps; returns false (and runs nothing) otherwise.
template <class F>
bool with_lds(long M, long N, long K, int splits, hipError_t* err, F&& f,
              LdsPolicy policy = LdsPolicy::kAuto) {
  if (M <= 0 || N <= 0 || K <= 0 || splits < 1) return false;
  if (policy == LdsPolicy::kBig && K % LdsBig::bk == 0 && M % 128 == 0 && N % 128 == 0) {
    *err = f(LdsBig{});
    return true;
  }
  // Very large products (four or more 128x256 tiles per CU) take 128x256
  // tiles, eight MFMAs per fragment step per wave; large ones (two or more
  // 128x128 tiles per CU) 128x128 tiles, half the operand bytes per MFMA of
  // a 64x64 tile. Both before the kDeep policy, which is tuned for config
  // 4's shapes (config-5 value forward 708 -> 415 us); the value dX keeps
  // its 128x128 tiles (kBig: 128x256 measured 1.45x slower for it). Deeper
  // rings for the 128x256 tiles measured slower: fewer blocks fit per CU.
  // 256x256 tiles: 16 MFMAs per fragment step per wave (config-5 value
  // forward 418 -> 335 us).
  if (K % LdsHuge::bk == 0 && M % 128 == 0 && N % 256 == 0 &&
      (M / 128) * (N / 256) * splits >= kHugeAutoBlocks) {
    *err = f(LdsHuge{});
    return true;
  }
  if (policy != LdsPolicy::kNoBig && K % LdsBig::bk == 0 && M % 128 == 0 && N % 128 == 0 &&
      (M / 128) * (N / 128) * splits >= kBigAutoBlocks) {
    *err = f(LdsBig{});
    return true;
  }
  if (policy == LdsPolicy::kDeep && K % LdsDeep::bk == 0) {
    *err = f(LdsDeep{});
    return true;
  }
  if (K % LdsMid::bk == 0) {
    *err = f(LdsMid{});
    return true;
  }
  if (K % LdsShort::bk == 0) {
    *err = f(LdsShort{});
    return true;
  }
  return false;
}

// The 256x256-tile product for an M x N output with K in whole BK steps.
inline bool giant_ok(long M, long N, long K) {
  return K > 0 && K % LdsGiant::bk == 0 && M % 256 == 0 && N % 256 == 0 &&
         (M / 256) * (N / 256) >= kGiantAutoBlocks;
}

template <class T, class OA, class OB, class Epi, int G>
hipError_t launch_lds_group(hipStream_t s, const Group<OA, G>& a, const Group<OB, G>& b,
                            const Group<Epi, G>& epi, long M, long N, long K) {
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return hipErrorInvalidValue;
  const long tiles = cdiv(M, T::bm) * cdiv(N, T::bn);
  const int ks = (int)(cdiv(K, T::bk) * T::bk);
  unsigned long long* stamps = take_probe_stamps(tiles * G);
  launch((gemm_lds_group_kernel<T::bm, T::bn, T::bk, T::ns, OA, OB, Epi, G, T::nw>),
         dim3((unsigned)tiles, G, 1), dim3(T::nw * 64), 0, s, a, b, epi, (int)M, (int)N, (int)K, ks,
         tile_map_for<T, OA, OB>(M, N), stamps);
  return hipGetLastError();
}

template <class T, class OA, class OB, class Epi>
hipError_t launch_lds(hipStream_t s, const OA& a, const OB& b, const Epi& epi, long M, long N,
                      long K, int splits) {
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return hipErrorInvalidValue;
  if (splits < 1) splits = 1;
  const long tiles = cdiv(M, T::bm) * cdiv(N, T::bn);
  const int ks = (int)(cdiv(cdiv(K, splits), T::bk) * T::bk);
  unsigned long long* stamps = take_probe_stamps(tiles * splits);
  launch((gemm_lds_kernel<T::bm, T::bn, T::bk, T::ns, OA, OB, Epi, T::nw>),
         dim3((unsigned)tiles, 1, splits), dim3(T::nw * 64), 0, s, a, b, epi, (int)M, (int)N, (int)K,
         ks, tile_map_for<T, OA, OB>(M, N), stamps);
  return hipGetLastError();
}

template <class T, class OA, class OB, class Epi>
LdsProblem<T, OA, OB, Epi> lds_problem(const OA& a, const OB& b, const Epi& epi, long M, long N,
                                       long K, int splits) {
  if (splits < 1) splits = 1;
  const int tiles = (int)(cdiv(M, T::bm) * cdiv(N, T::bn));
  const int ks = (int)(cdiv(cdiv(K, splits), T::bk) * T::bk);
  return LdsProblem<T, OA, OB, Epi>{a,  b,     epi,          (int)M, (int)N, (int)K,
                                    ks, tiles, tiles * splits, tile_map_for<T, OA, OB>(M, N)};
}

template <class T, class OA, class OB, class Epi>
hipError_t launch_lds_problem(hipStream_t s, const LdsProblem<T, OA, OB, Epi>& p) {
  unsigned long long* stamps = take_probe_stamps(p.blocks);
  launch((gemm_lds_kernel<T::bm, T::bn, T::bk, T::ns, OA, OB, Epi, T::nw>),
         dim3((unsigned)p.tiles, 1, (unsigned)(p.blocks / p.tiles)), dim3(T::nw * 64), 0, s, p.a,
         p.b,
         p.epi, p.M, p.N, p.K, p.k_split, p.map, stamps);
  return hipGetLastError();
}

// Shapes must fit int32 (lds_problem's callers check M, N, K).
// Problems of different wave counts (an eight-wave 256x256 product beside a
// four-wave one, a shape pair config 4 and 5 never form) run as separate
// launches, in order, on the stream.
template <class... Ps>
hipError_t launch_lds_multi(hipStream_t s, const Ps&... ps) {
  if constexpr (multi_nw<Ps...>() > 0) {
    unsigned long long* stamps = take_probe_stamps(0L + (0L + ... + ps.blocks));
    launch((gemm_lds_multi_kernel<Ps...>), dim3((unsigned)(0 + ... + ps.blocks)),
           dim3(multi_nw<Ps...>() * 64), 0,
           s, stamps, ps...);
    return hipGetLastError();
  } else {
    hipError_t e = hipSuccess;
    ((e = e == hipSuccess ? launch_lds_problem(s, ps) : e), ...);
    return e;
  }
}

template <class P1, class P2>
hipError_t launch_lds_pair(hipStream_t s, const P1& p1, const P2& p2) {
  return launch_lds_multi(s, p1, p2);
}

}  // namespace lds
}  // namespace ullis
