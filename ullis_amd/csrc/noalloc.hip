// LayerNorm backward that allocates nothing: ullis_hip_layer_norm_backward_static.
//
// ullis_hip_layer_norm_backward keeps its gamma / beta column partials in the
// context's grow-only scratch, which hipMallocs on first use (and again when
// a larger call comes). Callers that cannot allocate (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc) use this
// variant instead: the partials live in `scratch`, a fixed device array that
// every GPU the library runs on holds until the process ends. The row kernel
// here takes at most kStaticPartBlocks blocks whatever the row count, so the
// array bounds the channel count only: 2 * 256 * channels floats <= 8 MiB,
// i.e. channels <= 4096.
//
// The array's name is a host-side stand-in in host code; its device address
// is looked up once per device (hipGetSymbolAddress, with that device
// current) when a context is created, and only that address is passed to
// kernels. Every call on a GPU shares the GPU's array: the row kernel writes
// every partial it later reads (nothing needs clearing), and calls that
// overlap on one GPU (two streams, two threads) race on it.
#include <hip/hip_runtime.h>

#include <climits>
#include <mutex>
#include <string>

#include "../../include/ullis_hip.h"
#include "context.hpp"
#include "ops.hpp"

namespace {

constexpr size_t kStaticScratchBytes = size_t(8) << 20;
constexpr long kStaticPartBlocks = 256;  // upper bound of layer_norm_backward_capped_nblk
constexpr long kStaticMaxChannels =
    (long)(kStaticScratchBytes / sizeof(float) / (2 * kStaticPartBlocks));
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace ullis {

// Device address of `scratch` on `device`, which must be the current device;
// looked up once per device.
hipError_t static_scratch_address(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!ptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace ullis

extern "C" int ullis_hip_layer_norm_backward_static(ullis_hip_ctx* c, const float* x,
                                                    const float* gy, const uint16_t* weight,
                                                    size_t rows, size_t channels, float* gx,
                                                    float* gw, float* gb) {
  using namespace ullis;
  if (!c) return ULLIS_HIP_ERR_INVALID;
  if (rows == 0 || channels == 0 || rows > (size_t)INT32_MAX ||
      rows > (size_t)LONG_MAX / channels)
    return c->fail(ULLIS_HIP_ERR_INVALID, "LayerNorm backward shape mismatch");
  if ((long)channels > kStaticMaxChannels)
    return c->fail(ULLIS_HIP_ERR_INVALID,
                   "layer_norm_backward_static: channels " + std::to_string(channels) +
                       " exceed the static scratch limit of " +
                       std::to_string(kStaticMaxChannels));
  if (!x || !gy || !weight || !gx)
    return c->fail(ULLIS_HIP_ERR_INVALID, "layer_norm_backward_static: x, gy, weight and gx "
                                          "must be non-NULL");
  if (!c->static_scratch)
    return c->fail(ULLIS_HIP_ERR_RUNTIME,
                   "layer_norm_backward_static: the static scratch address of this device is "
                   "unavailable: " + c->static_scratch_err);
  float* part = static_cast<float*>(c->static_scratch);
  int nb = 0;
  if (int rc = c->hip(layer_norm_backward_rows_capped(c->stream, x, gy, (long)rows, (long)channels,
                                                      weight, gx, part, &nb),
                      "layer_norm_backward_static"))
    return rc;
  if (nb <= 0 || nb > kStaticPartBlocks)
    return c->fail(ULLIS_HIP_ERR_RUNTIME, "layer_norm_backward_static: partial count");
  return c->hip(layer_norm_param_finish(c->stream, part, nb, (long)channels, gw, gb, 0.0f,
                                        nullptr, nullptr, nullptr, nullptr),
                "layer_norm_backward_static finish");
}
