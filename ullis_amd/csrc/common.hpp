// Shared device helpers for the gfx950 kernels of libullis_hip.
//
// Numeric contract (matches the reference CPU backend, src/precision.rs):
//  - f32 -> f16 conversion is IEEE round-to-nearest-even with subnormals
//    (v_cvt_f16_f32 in the default RNE mode; f16 denormals are not flushed);
//  - SGD updates evaluate (current - lr*clamp(g)) + residual with two
//    roundings, never an FMA: every translation unit is built with
//    -ffp-contract=off.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ullis {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLayerNormEps = 1e-5f;  // src/model.rs:132
constexpr float kHeadBiasLrMult = 8.0f;  // src/model.rs:97

// Dynamic power-of-two scaling of fp32 gradients that feed fp16 MFMA operands:
// amax * scale lands in [2^(kGradTargetExp-1), 2^kGradTargetExp). The scale is
// exact, so dividing it back out in an epilogue is exact.
constexpr int kGradTargetExp = 6;

// amax is the largest FINITE |value| of the tensor (non-finite values are
// left out of it and pass through the fp16 conversion as NaN / Inf, so they
// reach the products and the updates as they do in the reference's fp32
// arithmetic).
__device__ __forceinline__ float grad_scale_from_amax(float amax) {
  if (!(amax > 0.0f) || !__builtin_isfinite(amax)) return 1.0f;
  int e;
  (void)__builtin_frexpf(amax, &e);  // amax = m * 2^e, m in [0.5, 1)
  return __builtin_ldexpf(1.0f, kGradTargetExp - e);
}

// Fp16::from_f32 (src/precision.rs:23-55): RNE with subnormals; a NaN becomes
// the canonical quiet NaN 0x7e00 with the input's sign, whatever its payload.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  if (__builtin_isnan(v)) return (uint16_t)(((__float_as_uint(v) >> 16) & 0x8000u) | 0x7e00u);
  half_t h = (half_t)v;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(half_t, b);
}

// Finite values clamped to the fp16 range; NaN and +-Inf pass unchanged (so a
// non-finite gradient stays non-finite in the fp16 operand, as in fp32).
__device__ __forceinline__ float clamp_f16_range(float v) {
  return __builtin_isfinite(v) ? __builtin_fminf(__builtin_fmaxf(v, -65504.0f), 65504.0f) : v;
}

// Conversion of a scaled gradient to its fp16 operand: finite values saturate
// (a finite value never becomes Inf), NaN and +-Inf are kept.
__device__ __forceinline__ half_t f32_to_f16_sat(float v) { return (half_t)clamp_f16_range(v); }

// |v| as it enters a gradient's amax: 0 for NaN and +-Inf (see
// grad_scale_from_amax).
__device__ __forceinline__ float finite_abs(float v) {
  return __builtin_isfinite(v) ? __builtin_fabsf(v) : 0.0f;
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
  // f32::clamp semantics: NaN passes through.
  return v < lo ? lo : (v > hi ? hi : v);
}

// Fp16Storage::apply_clipped_sgd, src/precision.rs:106-113.
__device__ __forceinline__ void clipped_sgd_one(uint16_t& value, float& residual, float gradient,
                                                float lr) {
  const float current = f16_bits_to_f32(value);
  const float update = lr * clampf(gradient, -1.0f, 1.0f);
  const float desired = current - update + residual;
  const uint16_t rounded = f32_to_f16_bits(desired);
  residual = desired - f16_bits_to_f32(rounded);
  value = rounded;
}

// Fp16Storage::apply_binaryconnect_sgd, src/precision.rs:124-134.
// Returns false when the gradient was skipped (zero or non-finite).
__device__ __forceinline__ bool binaryconnect_sgd_one(uint16_t& value, float& residual,
                                                      float gradient, float lr) {
  if (!__builtin_isfinite(gradient) || gradient == 0.0f) return false;
  const float current = f16_bits_to_f32(value);
  const float update = lr * clampf(gradient, -1.0f, 1.0f);
  const float desired = clampf(current - update + residual, -1.0f, 1.0f);
  const uint16_t rounded = f32_to_f16_bits(desired);
  residual = desired - f16_bits_to_f32(rounded);
  value = rounded;
  return true;
}

// rebinarize (src/model.rs:878-884): latent >= 0.0, so -0.0 packs as +1.
__device__ __forceinline__ bool latent_is_plus(uint16_t latent_bits) {
  return f16_bits_to_f32(latent_bits) >= 0.0f;
}

// Cross-lane moves of a xor butterfly with no LDS round trip: v_permlane32_swap
// and v_permlane16_swap give lane ^ 32 and lane ^ 16, DPP row_ror:8 lane ^ 8,
// DPP row_ror:4 lane ^ 4 or ^ 12 (the same value once the ^ 8 step has run),
// and quad permutations lane ^ 2 and ^ 1. (A __shfl_xor is a ds_bpermute,
// one LDS round trip per step, each waited for before the next.) The lane
// layouts were checked on gfx950, and the butterflies below are bit-identical
// to the __shfl_xor ones with the same offsets.
namespace xlane {
__device__ __forceinline__ uint32_t swap32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
}
__device__ __forceinline__ uint32_t swap16(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
// The partner value of butterfly step OFF (steps run from large to small).
template <int OFF>
__device__ __forceinline__ uint32_t step(uint32_t v) {
  if constexpr (OFF == 32) return swap32(v);
  else if constexpr (OFF == 16) return swap16(v);
  else if constexpr (OFF == 8) return dpp<0x128>(v);  // row_ror:8
  else if constexpr (OFF == 4) return dpp<0x124>(v);  // row_ror:4
  else if constexpr (OFF == 2) return dpp<0x4E>(v);   // quad_perm 2,3,0,1
  else return dpp<0xB1>(v);                           // quad_perm 1,0,3,2
}
// v = op(v, partner) for OFF = FROM, FROM / 2, ..., 1 (FROM 8 or more, so
// that the ^ 4 step follows the ^ 8 one).
template <int FROM, class T, class Op>
__device__ __forceinline__ T butterfly(T v, Op op) {
  static_assert(FROM >= 8 && (FROM & (FROM - 1)) == 0 && FROM <= 32, "butterfly width");
  if constexpr (FROM >= 32) v = op(v, __builtin_bit_cast(T, step<32>(__builtin_bit_cast(uint32_t, v))));
  if constexpr (FROM >= 16) v = op(v, __builtin_bit_cast(T, step<16>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(T, step<8>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(T, step<4>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(T, step<2>(__builtin_bit_cast(uint32_t, v))));
  v = op(v, __builtin_bit_cast(T, step<1>(__builtin_bit_cast(uint32_t, v))));
  return v;
}
}  // namespace xlane

// Wave64 reductions; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) {
  return xlane::butterfly<32>(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return xlane::butterfly<32>(v, [](float a, float b) { return __builtin_fmaxf(a, b); });
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return xlane::butterfly<32>(v, [](uint32_t a, uint32_t b) { return a + b; });
}

// Max / sum over the 32 lanes of each half-wave (lanes 0-31 and 32-63 separately).
__device__ __forceinline__ float halfwave_max(float v) {
  return xlane::butterfly<16>(v, [](float a, float b) { return __builtin_fmaxf(a, b); });
}

__device__ __forceinline__ float halfwave_sum(float v) {
  return xlane::butterfly<16>(v, [](float a, float b) { return a + b; });
}

// Non-negative floats order like their bit patterns, so a u32 atomicMax on the
// bits is an exact, order-independent max.
// The slot only grows, so a value not above a (possibly stale) read of it
// cannot change it: skipping those atomics keeps same-address contention low.
// Non-finite values are not counted (callers pass maxima of finite_abs).
__device__ __forceinline__ void atomic_amax(float* slot, float v) {
  v = finite_abs(v);
  unsigned int* p = reinterpret_cast<unsigned int*>(slot);
  if (__float_as_uint(v) > __atomic_load_n(p, __ATOMIC_RELAXED))
    atomicMax(p, __float_as_uint(v));
}

// Row/column of accumulator register r of a 32x32x16 MFMA tile held by `lane`:
// column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4.
__device__ __forceinline__ int mfma32_row(int r, int lane) {
  return ((r >> 2) << 3) + ((lane >> 5) << 2) + (r & 3);
}

// ------------------------------------------------------------ launching
// Launch probe, armed on the launching thread for the next launch:
//  - kernels that take a stamps slot (the streamed-LDS GEMMs) get `stamps`
//    as an argument: every block writes the device wall clock
//    (s_memrealtime) at its start and end into its own (start, end) pair, and
//    the host takes the earliest start and the latest end, i.e. the launch's
//    execution interval, which waiting for CUs held by another stream's
//    kernels does not inflate; the launcher sets used_stamps;
//  - any other launch() records its kernel into the events
//    (hipExtLaunchKernelGGL).
// The launcher that consumes the probe disarms it.
struct LaunchProbe {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  unsigned long long* stamps = nullptr;  // [stamp_cap][2]: per block (start, end)
  long stamp_cap = 0;                    // blocks the stamps slot holds
  long blocks = 0;                       // blocks of the launch that took the slot
  bool used_stamps = false;
};
inline thread_local LaunchProbe* t_launch_probe = nullptr;

// The stamps slot for the next launch, of `blocks` workgroups, of a kernel
// that records them (the probe is consumed), or null: no probe, or a grid
// larger than the slot (the launch is then timed by the probe's events).
inline unsigned long long* take_probe_stamps(long blocks) {
  LaunchProbe* p = t_launch_probe;
  if (!p || !p->stamps || blocks > p->stamp_cap) return nullptr;
  t_launch_probe = nullptr;
  p->used_stamps = true;
  p->blocks = blocks;
  return p->stamps;
}

// Each block writes its own (start, end) pair of the device wall clock, so
// stamping adds no contended atomics; the kernel's interval is the earliest
// start to the latest end.
__device__ __forceinline__ long stamp_slot() {
  return blockIdx.x + (long)gridDim.x * (blockIdx.y + (long)gridDim.y * blockIdx.z);
}
__device__ __forceinline__ void stamp_block_start(unsigned long long* stamps) {
  if (stamps && threadIdx.x == 0) stamps[2 * stamp_slot()] = __builtin_amdgcn_s_memrealtime();
}
// Call from every thread after the block's last store.
__device__ __forceinline__ void stamp_block_end(unsigned long long* stamps) {
  if (stamps) {
    __syncthreads();
    if (threadIdx.x == 0) stamps[2 * stamp_slot() + 1] = __builtin_amdgcn_s_memrealtime();
  }
}

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes,
                   hipStream_t s, Args... args) {
  if (LaunchProbe* p = t_launch_probe) {
    t_launch_probe = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, s, p->start, p->stop, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds_bytes, s, args...);
  }
}

}  // namespace ullis
