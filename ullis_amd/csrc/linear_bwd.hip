// Packed +-1 and FP16 linear on gfx950 MFMA: input-gradient and
// weight-gradient products, alone or paired in one launch (reference
// semantics in linear_impl.hpp).
#include "linear_impl.hpp"

namespace ullis {

// gx (+)= gy . (scale * S) over the window of PackedDxArgs.
hipError_t packed_dx(hipStream_t s, const PackedDxArgs& d) {
  if (d.col_part && (d.out_mul || d.accumulate || !d.sign_idx)) return hipErrorInvalidValue;
  hipError_t err = hipSuccess;
  if (packed_dx_lds(d, &err, launch_one(s))) return err;
  if (d.col_part) {
    // store gx, then the signed column sums over it
    PackedDxArgs st = d;
    st.col_part = nullptr;
    if ((err = packed_dx(s, st)) != hipSuccess) return err;
    return column_sum_partials(s, d.gx, d.sign_idx, d.rows, d.in, d.col_part, nullptr);
  }
  const long ldgy = ldgy_of(d), ldb = ldb_of(d);
  EpiStoreF32 epi{d.gx, d.gy32.amax, d.out_mul, d.accumulate};
  return with_tile(d.rows, d.in, [&](auto t) {
    using T = decltype(t);
    LoadBits<T::bn, T::bk, true> lb{d.bits_t, ldb, d.kofs, d.scale,
                                    bits_aligned(ldb, d.kofs, d.scale)};
    if (d.gy16) {
      LoadF16K<T::bm, T::bk> la{reinterpret_cast<const half_t*>(d.gy16), ldgy,
                                vec_ok_f16(d.gy16, ldgy)};
      return launch_gemm<T>(s, la, lb, epi, d.rows, d.in, d.out, 1);
    }
    LoadF32K<T::bm, T::bk> la{d.gy32.p, ldgy, vec_ok_f32(d.gy32.p, ldgy), d.gy32.amax, 1.0f};
    return launch_gemm<T>(s, la, lb, epi, d.rows, d.in, d.out, 1);
  });
}

hipError_t packed_backward_input(hipStream_t s, GradIn gy32, const uint16_t* gy16, long rows,
                                 long in, long out, const uint32_t* bits_t, const uint16_t* scale,
                                 float* gx, const float* out_mul, int accumulate) {
  return packed_dx(s, PackedDxArgs{gy32, gy16, rows, in, out, bits_t, scale, gx, out_mul,
                                   accumulate});
}

// Input gradient over a column window of the output features: contraction
// over k in [kofs, kofs + k_len) of a bits_t matrix with ldb bits per row, gy
// fp16 [rows][ldgy] holding only that window (unscaled), scale indexed kofs + k.
hipError_t packed_backward_input_ex(hipStream_t s, const uint16_t* gy16, long ldgy, long rows,
                                    long in, long k_len, const uint32_t* bits_t, long ldb,
                                    long kofs, const uint16_t* scale, float* gx,
                                    const float* out_mul, int accumulate) {
  return packed_dx(s, PackedDxArgs{GradIn{nullptr, nullptr}, gy16, rows, in, k_len, bits_t, scale,
                                   gx, out_mul, accumulate, ldgy, ldb, kofs});
}

hipError_t packed_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* gy16,
                                       const uint16_t* x16, long rows, long in, long out,
                                       int splits, float* part) {
  EpiPartial epi{part};
  hipError_t err = hipSuccess;
  if (weight_grad_lds(WeightGradArgs{gy32, gy16, x16, rows, in, out, splits, part}, &err,
                      launch_one(s)))
    return err;
  return with_tile(out, in, [&](auto t) {
    using T = decltype(t);
    LoadF16T<T::bn, T::bk> lb{reinterpret_cast<const half_t*>(x16), in, vec_ok_f16(x16, in)};
    if (gy16) {
      LoadF16T<T::bm, T::bk> la{reinterpret_cast<const half_t*>(gy16), out, vec_ok_f16(gy16, out)};
      return launch_gemm<T>(s, la, lb, epi, out, in, rows, splits);
    }
    LoadF32T<T::bm, T::bk> la{gy32.p, out, vec_ok_f32(gy32.p, out), gy32.amax, 1.0f};
    return launch_gemm<T>(s, la, lb, epi, out, in, rows, splits);
  });
}

hipError_t fp16_backward_input(hipStream_t s, GradIn gy32, long rows, long in, long out,
                               const uint16_t* w, float* gx, const uint16_t* key16,
                               uint16_t* gk16) {
  hipError_t err = hipSuccess;
  if (fp16_dx_lds(Fp16DxArgs{gy32, rows, in, out, w, gx, key16, gk16}, &err, launch_one(s)))
    return err;
  return with_tile(rows, in, [&](auto t) {
    using T = decltype(t);
    LoadF32K<T::bm, T::bk> la{gy32.p, out, vec_ok_f32(gy32.p, out), gy32.amax, 1.0f};
    LoadF16T<T::bn, T::bk> lb{reinterpret_cast<const half_t*>(w), in, vec_ok_f16(w, in)};
    if (gk16) {
      EpiRelu2Bwd epi{key16, gk16};
      return launch_gemm<T>(s, la, lb, epi, rows, in, out, 1);
    }
    EpiStoreF32 epi{gx, gy32.amax, nullptr, 0};
    return launch_gemm<T>(s, la, lb, epi, rows, in, out, 1);
  });
}

bool fp16_dx_wants_w_t(long rows, long in, long out) { return lds::giant_ok(rows, in, out); }

hipError_t fp16_weight_grad_partials(hipStream_t s, GradIn gy32, const uint16_t* x16, long rows,
                                     long in, long out, int splits, float* part) {
  return packed_weight_grad_partials(s, gy32, nullptr, x16, rows, in, out, splits, part);
}

// Both GEMMs of a backward in one launch when both take the streamed-LDS path
// (their blocks share the CUs); otherwise the two separate launches.
hipError_t packed_backward_pair(hipStream_t s, const PackedDxArgs& dx, const WeightGradArgs& dw) {
  hipError_t err = hipSuccess;
  bool dw_ok = false;
  if (packed_dx_lds(dx, &err, [&](const auto& p1) {
        hipError_t e2 = hipSuccess;
        dw_ok = weight_grad_lds(dw, &e2, [&](const auto& p2) {
          return lds::launch_lds_pair(s, p1, p2);
        });
        return dw_ok ? e2 : hipSuccess;
      }) &&
      dw_ok)
    return err;
  if ((err = packed_dx(s, dx)) != hipSuccess) return err;
  return packed_weight_grad_partials(s, dw.gy32, dw.gy16, dw.x16, dw.rows, dw.in, dw.out,
                                     dw.splits, dw.part);
}

hipError_t fp16_backward_pair(hipStream_t s, const Fp16DxArgs& dx, const WeightGradArgs& dw) {
  hipError_t err = hipSuccess;
  bool dw_ok = false;
  if (fp16_dx_lds(dx, &err, [&](const auto& p1) {
        hipError_t e2 = hipSuccess;
        dw_ok = weight_grad_lds(dw, &e2, [&](const auto& p2) {
          return lds::launch_lds_pair(s, p1, p2);
        });
        return dw_ok ? e2 : hipSuccess;
      }) &&
      dw_ok)
    return err;
  if ((err = fp16_backward_input(s, dx.gy32, dx.rows, dx.in, dx.out, dx.w, dx.gx, dx.key16,
                                 dx.gk16)) != hipSuccess)
    return err;
  return packed_weight_grad_partials(s, dw.gy32, dw.gy16, dw.x16, dw.rows, dw.in, dw.out,
                                     dw.splits, dw.part);
}

}  // namespace ullis
