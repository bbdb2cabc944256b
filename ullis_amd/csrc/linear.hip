// Packed +-1 BinaryConnect linear and FP16 linear on gfx950 MFMA: forward
// products and the parameter finishes (latent / weight steps, bit repack and
// transpose). The backward products are in linear_bwd.hip; the reference
// semantics are listed in linear_impl.hpp.
#include "linear_impl.hpp"

namespace ullis {

namespace {

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
      auto giant = [&](auto t) {
        using T = decltype(t);
        lds::OpMK<T::bm, T::bk, T::nw> a{static_cast<const half_t*>(x), in, (int)rows};
        lds::OpBitsX<T::bn, T::bk, T::nw> b{bits, in / 32, (int)out};
        return lds::launch_lds<T>(s, a, b, epi, rows, out, in, 1);
      };
      if (in % lds::LdsGiantBits::bk == 0) return giant(lds::LdsGiantBits{});
      return giant(lds::LdsGiant{});
    }
    if (x_dtype == kF16 && lds::mk_ok(x, in) &&
        lds::with_lds(rows, out, in, 1, &err, [&](auto t) {
          using T = decltype(t);
          lds::OpMK<T::bm, T::bk, T::nw> a{static_cast<const half_t*>(x), in, (int)rows};
          lds::OpBits<T::bn, T::bk, false, T::nw> b{bits, in / 32, (int)out, nullptr, 0};
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
        lds::Group<lds::OpMK<T::bm, T::bk, T::nw>, 3> a;
        lds::Group<lds::OpBits<T::bn, T::bk, false, T::nw>, 3> b;
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
  // very large products: 256x256 tiles (four waves; eight measured 343 -> 351
  // us at config 5's value forward)
  if (x_dtype == kF16 && lds::mk_ok(x, in) && lds::mk_ok(w, in) && lds::giant_ok(rows, out, in)) {
    using T = lds::LdsGiant;
    lds::OpMK<T::bm, T::bk, T::nw> a{static_cast<const half_t*>(x), in, (int)rows};
    lds::OpMK<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(w), in, (int)out};
    return lds::launch_lds<T>(s, a, b, epi, rows, out, in, 1);
  }
  if (x_dtype == kF16 && lds::mk_ok(x, in) && lds::mk_ok(w, in) &&
      lds::with_lds(rows, out, in, 1, &err, [&](auto t) {
        using T = decltype(t);
        lds::OpMK<T::bm, T::bk, T::nw> a{static_cast<const half_t*>(x), in, (int)rows};
        lds::OpMK<T::bn, T::bk, T::nw> b{reinterpret_cast<const half_t*>(w), in, (int)out};
        return lds::launch_lds<T>(s, a, b, epi, rows, out, in, 1);
        // one block per CU at heron sizes, reading an operand fresh from HBM:
        // the four-stage ring (measured 18.9 -> 15.2 us in the step)
      }, lds::LdsPolicy::kDeep))
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
