// Host-side context shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "ops.hpp"

struct ullis_hip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  hipEvent_t events[16] = {};
  ullis::LaunchProbe next_launch;  // armed by ullis_hip_time_next_launch
  // device address of the static scratch array on this context's device
  // (ullis_hip_layer_norm_backward_static), looked up at create
  void* static_scratch = nullptr;
  std::string static_scratch_err;

  int fail(int code, const std::string& msg) {
    err = msg;
    return code;
  }
  int hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    err = std::string(what) + ": " + hipGetErrorString(e);
    return -3;
  }
  // Grow-only scratch; waits for the stream before replacing the buffer.
  int ensure_scratch(size_t bytes, void** out) {
    if (bytes > scratch_bytes) {
      if (scratch) {
        if (int rc = hip(hipStreamSynchronize(stream), "scratch sync")) return rc;
        if (int rc = hip(hipFree(scratch), "scratch free")) return rc;
        scratch = nullptr;
        scratch_bytes = 0;
      }
      const size_t want = (bytes + (1u << 20) - 1) / (1u << 20) * (1u << 20);
      if (hipMalloc(&scratch, want) != hipSuccess) {
        scratch = nullptr;
        return fail(-4, "scratch allocation of " + std::to_string(want) + " bytes failed");
      }
      scratch_bytes = want;
    }
    *out = scratch;
    return 0;
  }
};

namespace ullis {

// noalloc.hip: device address of the library's static scratch array on
// `device` (the current device), looked up once per device.
hipError_t static_scratch_address(int device, void** out);

// Carves 256-byte aligned sub-buffers from one allocation.
struct Carver {
  char* p;
  size_t used = 0;
  explicit Carver(void* base) : p(static_cast<char*>(base)) {}
  template <class T>
  T* take(size_t count) {
    T* r = reinterpret_cast<T*>(p + used);
    used += (count * sizeof(T) + 255) / 256 * 256;
    return r;
  }
  static size_t bytes_for(size_t bytes) { return (bytes + 255) / 256 * 256; }
};

// Counts the bytes a sequence of Carver::take calls needs (returns null pointers).
struct CarveSizer {
  size_t used = 0;
  template <class T>
  T* take(size_t count) {
    used += Carver::bytes_for(count * sizeof(T));
    return nullptr;
  }
};

// Weight gradients over many rows with 256x256-tileable outputs run on
// 256x256 tiles, split over the rows for one block per CU (config 5's value,
// key and O weight gradients: the pairs 1295 -> 1152, 902 -> 757 and
// 532 -> 424 us, the step 104.0 -> 96.9 ms, against 64x64 tiles over all rows).
inline bool dw_giant(long out, long in, long rows) {
  return out % 256 == 0 && in % 256 == 0 && (out / 256) * (in / 256) >= 16 && rows >= 16384 &&
         rows % 4096 == 0;
}

// Split-K factor for a weight-gradient GEMM [out, in] over `rows`: enough
// 64x64-tile blocks for two per CU (512), at least 256 rows per split, at most 8
// (256x256 tiles: one block per CU, at most 8, whole 32-row steps per split).
inline int dw_splits(long out, long in, long rows, long target_blocks = 512) {
  if (dw_giant(out, in, rows)) {
    long s = cdiv(256, (out / 256) * (in / 256));
    if (s > 8) s = 8;
    while (s > 1 && rows % (32 * s) != 0) --s;
    return (int)s;
  }
  const long tiles = cdiv(out, 64) * cdiv(in, 64);
  long s = cdiv(target_blocks, tiles > 0 ? tiles : 1);
  const long by_rows = rows / 256;
  if (s > by_rows) s = by_rows;
  if (s > 8) s = 8;
  if (s < 1) s = 1;
  return (int)s;
}

// Split-K factor of a weight gradient paired with its layer's input gradient
// in one launch (packed_backward_pair / fp16_backward_pair): the input
// gradient supplies blocks too, so one per CU (256) is enough, and fewer
// splits mean fewer fp32 partials to write and reduce.
inline int pair_dw_splits(long out, long in, long rows) { return dw_splits(out, in, rows, 256); }

}  // namespace ullis
