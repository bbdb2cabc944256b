"""Pins the CPU oracle (oracle/cpu_ref.c) before it is trusted as the checker.

Each test checks an oracle function against something independent of it:
the reference's own known-answer tests and fixtures (cited file:line),
numpy's IEEE float16 conversion, float64 numpy re-derivations, finite
differences, or brute force on tiny shapes. None of these re-types the
oracle's own formula in float32.
"""
import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.synth import f16, pack_bits, unpack_bits

F16 = np.float16


def h2f(bits):
    return np.asarray(bits, np.uint16).view(F16).astype(np.float64)


# ----------------------------------------------------------------- a1 fp16
def test_f16_from_f32_matches_numpy_rne_on_stratified_patterns():
    rng = np.random.default_rng(1)
    pats = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    # dense coverage of the f16 range, the subnormal range and the halfway cases
    exps = rng.integers(100, 145, 500_000).astype(np.uint32)
    mant = rng.integers(0, 2**23, 500_000).astype(np.uint32)
    sign = rng.integers(0, 2, 500_000).astype(np.uint32) << 31
    dense = sign | (exps << 23) | mant
    halfway = sign | (exps << 23) | (mant & ~np.uint32(0x1FFF)) | np.uint32(0x1000)
    edges = np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x477FE000, 0x477FF000,
                      0x477FEFFF, 0x33000000, 0x33000001, 0x32FFFFFF, 0x387FC000, 0x38800000,
                      0x3F800000, 0xC0000000], dtype=np.uint32)
    allp = np.concatenate([pats, dense, halfway, edges])
    x = allp.view(np.float32)
    got = o.f16_from_f32(x)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(F16).view(np.uint16)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], want[~nan])
    # reference canonicalises NaN to sign | 0x7e00 (src/precision.rs:29-31)
    np.testing.assert_array_equal(got[nan], (allp[nan] >> 16 & 0x8000).astype(np.uint16) | 0x7E00)


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = o.f16_to_f32(bits)
    want = bits.view(F16).astype(np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_fp16_specials_reference_case():
    # src/precision.rs:219-228
    vals = np.array([0.0, -0.0, 1.0, -2.0, 0.5, 65504.0], np.float32)
    back = o.f16_to_f32(o.f16_from_f32(vals))
    np.testing.assert_array_equal(back.view(np.uint32), vals.view(np.uint32))
    assert np.isnan(o.f16_to_f32(o.f16_from_f32([np.nan]))[0])
    assert np.isinf(o.f16_to_f32(o.f16_from_f32([np.inf]))[0])


# ---------------------------------------------------------- a2 / a3 SGD
def numpy_clipped(p_bits, res, g, lr):
    """Independent float32 evaluation with numpy's own float16 rounding."""
    cur = np.asarray(p_bits, np.uint16).view(F16).astype(np.float32)
    upd = np.float32(lr) * np.clip(np.asarray(g, np.float32), np.float32(-1), np.float32(1))
    desired = (cur - upd) + np.asarray(res, np.float32)
    with np.errstate(invalid="ignore"):
        rounded = desired.astype(F16)
    bits = rounded.view(np.uint16).copy()
    # Fp16::from_f32 (src/precision.rs:29-31): any NaN -> sign | 0x7e00
    nan = np.isnan(desired)
    bits[nan] = ((desired[nan].view(np.uint32) >> 16) & 0x8000).astype(np.uint16) | 0x7E00
    return bits, desired - rounded.astype(np.float32)


def numpy_binaryconnect(p_bits, res, g, lr):
    p_bits = np.asarray(p_bits, np.uint16).copy()
    res = np.asarray(res, np.float32).copy()
    g = np.asarray(g, np.float32)
    live = np.isfinite(g) & (g != 0)
    cur = p_bits.view(F16).astype(np.float32)
    upd = np.float32(lr) * np.clip(g, np.float32(-1), np.float32(1))
    desired = np.clip((cur - upd) + res, np.float32(-1), np.float32(1))
    rounded = desired.astype(F16)
    p_bits[live] = rounded.view(np.uint16)[live]
    res[live] = (desired - rounded.astype(np.float32))[live]
    return p_bits, res


def test_clipped_sgd_metal_fixture_bit_exact():
    # inputs of clipped_sgd_fp16_matches_cpu_residual, src/metal.rs:4007-4023
    p = f16([0.25, -1.0, 2.0])
    g = np.array([0.001, 0.5, -0.25], np.float32)
    got_p, got_r = o.clipped_sgd(p, np.zeros(3, np.float32), g, 0.01)
    want_p, want_r = numpy_clipped(p, np.zeros(3, np.float32), g, 0.01)
    np.testing.assert_array_equal(got_p, want_p)
    np.testing.assert_array_equal(got_r.view(np.uint32), want_r.view(np.uint32))
    assert got_p[0] == f16([0.25])[0] and got_r[0] < 0  # sub-ULP step lands in the carry


def test_binaryconnect_metal_fixture_bit_exact():
    # inputs of binaryconnect_sgd_fp16_matches_cpu_magnitude_clip, src/metal.rs:4026-4042
    p = f16([0.0625, -0.0625, 0.9])
    g = np.array([1e-5, -1e-6, 2.0], np.float32)
    got_p, got_r = o.binaryconnect_sgd(p, np.zeros(3, np.float32), g, 0.1)
    want_p, want_r = numpy_binaryconnect(p, np.zeros(3, np.float32), g, 0.1)
    np.testing.assert_array_equal(got_p, want_p)
    np.testing.assert_array_equal(got_r.view(np.uint32), want_r.view(np.uint32))


@pytest.mark.parametrize("lr", [0.01, 0.1, 4.0])
def test_sgd_random_bit_exact_against_numpy(lr):
    rng = np.random.default_rng(int(lr * 100))
    n = 200_000
    p = f16(rng.uniform(-1.2, 1.2, n) * (10.0 ** rng.integers(-6, 1, n)))
    res = (rng.standard_normal(n) * 1e-5).astype(np.float32)
    g = (rng.standard_normal(n) * (10.0 ** rng.integers(-7, 2, n))).astype(np.float32)
    g[::97] = 0.0
    g[::101] = np.inf
    g[::103] = np.nan
    # non-finite gradients too: Inf clamps to +-1, NaN carries into value
    # (canonical sign | 0x7e00) and residual (src/precision.rs:29-31, 106-113)
    g[::107] = np.uint32(0xFFC00000).view(np.float32)
    g[::109] = np.uint32(0x7FA00001).view(np.float32)
    g[::113] = -np.inf
    gp, gr = o.clipped_sgd(p, res, g, lr)
    wp, wr = numpy_clipped(p, res, g, lr)
    np.testing.assert_array_equal(gp, wp)
    nan = np.isnan(g)
    assert np.isnan(gr[nan]).all() and ((gp[nan] & 0x7FFF) == 0x7E00).all()
    np.testing.assert_array_equal(gr[~nan].view(np.uint32), wr[~nan].view(np.uint32))
    gp, gr = o.binaryconnect_sgd(p, res, g, lr)
    wp, wr = numpy_binaryconnect(p, res, g, lr)
    np.testing.assert_array_equal(gp, wp)
    np.testing.assert_array_equal(gr.view(np.uint32), wr.view(np.uint32))


def test_precision_reference_unit_tests():
    # src/precision.rs:238-313 restated as known answers
    p, r = o.clipped_sgd(f16([0.25]), [0.0], [1.0], 0.01)
    assert h2f(p)[0] < 0.25
    p, r = f16([0.25]), np.zeros(1, np.float32)
    p, r = o.clipped_sgd(p, r, [0.001], 0.01)
    assert h2f(p)[0] == 0.25 and r[0] < 0
    for _ in range(64):
        p, r = o.clipped_sgd(p, r, [0.001], 0.01)
    assert h2f(p)[0] < 0.25
    p, r = o.binaryconnect_sgd(f16([0.5, 0.5]), np.zeros(2, np.float32), [1.0, 0.1], 0.1)
    assert abs(h2f(p)[0] - 0.4) < 1e-3 and abs(h2f(p)[1] - 0.49) < 1e-3
    p1, r1 = o.binaryconnect_sgd(p[:1], r[:1], [-1.0], 4.0)
    assert h2f(p1)[0] == 1.0
    p1, r1 = o.binaryconnect_sgd(p1, r1, [1.0], 4.0)
    assert h2f(p1)[0] == -1.0
    p, r = f16([0.25]), np.zeros(1, np.float32)
    p, r = o.binaryconnect_sgd(p, r, [0.001], 0.01)
    assert h2f(p)[0] == 0.25 and r[0] < 0
    for _ in range(64):
        p, r = o.binaryconnect_sgd(p, r, [0.001], 0.01)
    assert h2f(p)[0] < 0.25


# ---------------------------------------------------------------- a4 bits
def test_pack_bitplane_known_answer():
    # tests/rosa.rs:151-157
    x = np.array([1, 0, 1, 1, 0, 0, 0, 1], np.float32)
    assert o.sign_pack_bits(x)[0] == 1 | (1 << 2) | (1 << 3) | (1 << 7)


def test_latent_packing_treats_negative_zero_as_plus_and_matches_brute_force():
    rng = np.random.default_rng(3)
    lat = f16(rng.uniform(-1, 1, 1000))
    lat[:5] = [0x8000, 0x0000, 0x0001, 0x8001, 0x7E00]  # -0, +0, +tiny, -tiny, NaN
    got = o.pack_latent_bits(lat)
    plus = lat.view(F16).astype(np.float32) >= 0
    np.testing.assert_array_equal(got, pack_bits(plus))
    assert unpack_bits(got, 5).tolist() == [True, True, True, False, False]


def test_transpose_bits_brute_force():
    rng = np.random.default_rng(4)
    for out_f, in_f in [(18, 19), (64, 32), (5, 7)]:
        plus = rng.integers(0, 2, out_f * in_f).astype(bool)
        got = o.transpose_bits(pack_bits(plus), out_f, in_f)
        want = pack_bits(plus.reshape(out_f, in_f).T.ravel())
        np.testing.assert_array_equal(got, want)


# ------------------------------------------------------ a5 - a9 packed linear
def test_binary_linear_reference_closed_forms():
    # tests/binary_linear.rs:4-39
    bits = pack_bits([True, False])
    y = o.packed_forward([2.0, 3.0], 1, 2, 1, bits, f16([0.5]), f16([0.0]))
    assert abs(y[0] + 0.5) < 1e-6
    g = o.packed_backward_ste([2.0, 3.0], [1.0], 1, 2, 1, bits, f16([0.5]))
    np.testing.assert_allclose(g["weight_gradient"], [1.0, 1.5], atol=1e-6)
    np.testing.assert_allclose(g["input_gradient"], [0.5, -0.5], atol=1e-6)
    np.testing.assert_allclose(g["scale_gradient"], [-1.0], atol=1e-6)
    np.testing.assert_allclose(g["bias_gradient"], [1.0], atol=1e-6)


def metal_tiled_fixture():
    # tiled_linears_match_cpu_past_tile_boundary, src/metal.rs:3908-3974
    rows, inn, out = 17, 19, 18
    signs = np.array([[1 if (oo + i) % 2 == 0 else -1 for i in range(inn)] for oo in range(out)])
    weight = np.array([[((oo * 3 + i) % 7) * 0.25 - 0.5 for i in range(inn)] for oo in range(out)])
    x = np.array([[((r * 5 + i) % 11) * 0.125 - 0.5 for i in range(inn)] for r in range(rows)])
    gy = np.array([[((r + oo) % 5) * 0.2 - 0.4 for oo in range(out)] for r in range(rows)])
    return rows, inn, out, signs, weight, x, gy


def test_packed_linear_brute_force_float64_on_tiled_fixture():
    rows, inn, out, signs, _, x, gy = metal_tiled_fixture()
    bits = pack_bits((signs >= 0).ravel())
    scale = f16(np.full(out, 0.5))
    bias = f16(np.linspace(-0.1, 0.1, out))
    y = o.packed_forward(x.ravel(), rows, inn, out, bits, scale, bias)
    want = h2f(bias)[None, :] + h2f(scale)[None, :] * (x @ signs.T)
    np.testing.assert_allclose(y.reshape(rows, out), want, rtol=1e-6, atol=1e-6)
    g = o.packed_backward_ste(x.ravel(), gy.ravel(), rows, inn, out, bits, scale)
    sc = h2f(scale)
    np.testing.assert_allclose(g["input_gradient"].reshape(rows, inn), (gy * sc) @ signs,
                               rtol=1e-6, atol=1e-6)
    G = gy.T @ x
    np.testing.assert_allclose(g["weight_gradient"].reshape(out, inn), sc[:, None] * G, atol=1e-5)
    # identity used by the GPU: g_scale[o] = sum_i sign[o,i] * G[o,i]
    np.testing.assert_allclose(g["scale_gradient"], (signs * G).sum(1), atol=1e-5)
    np.testing.assert_allclose(g["bias_gradient"], gy.sum(0), atol=1e-6)


def test_packed_sgd_reference_behaviour():
    # tests/binary_linear.rs:42-88: the latent persists; the scale is learned
    bits = pack_bits([True])
    lat, lres = f16([0.5]), np.zeros(1, np.float32)
    sc, sres = f16([0.5]), np.zeros(1, np.float32)
    g = o.packed_backward_ste([1.0], [1.0], 1, 1, 1, bits, sc, want_gx=False, want_gb=False)
    lat, lres, sc, sres, _, _, bits = o.packed_apply_sgd(1, 1, lat, lres, sc, sres, None, None,
                                                         g["weight_gradient"], [0.0], None, 0.1, 1.0)
    after = h2f(lat)[0]
    assert abs(after - h2f(sc)[0] * 1.0) > 1e-3
    g = o.packed_backward_ste([1.0], [1.0], 1, 1, 1, bits, sc, want_gx=False, want_gb=False)
    lat2, *_ = o.packed_apply_sgd(1, 1, lat, lres, sc, sres, None, None, g["weight_gradient"],
                                  [0.0], None, 0.1, 1.0)
    assert h2f(lat2)[0] != after
    # scale_is_learned_not_mean_abs_latent
    bits = pack_bits([True, False])
    lat, sc = f16([0.5, -0.5]), f16([0.5])
    g = o.packed_backward_ste([1.0, 0.0], [1.0], 1, 2, 1, bits, sc, want_gx=False, want_gb=False)
    lat, _, sc, _, _, _, _ = o.packed_apply_sgd(2, 1, lat, np.zeros(2, np.float32), sc,
                                                np.zeros(1, np.float32), None, None,
                                                g["weight_gradient"], g["scale_gradient"], None,
                                                0.05, 1.0)
    assert abs(h2f(sc)[0] - 0.5 * np.abs(h2f(lat)).sum()) > 1e-4


def test_packed_sgd_composition_matches_independent_numpy():
    rng = np.random.default_rng(5)
    out_f, in_f = 7, 37
    lat = f16(rng.uniform(-0.01, 0.01, out_f * in_f))
    lres = (rng.standard_normal(out_f * in_f) * 1e-6).astype(np.float32)
    sc, sres = f16(rng.uniform(0.005, 0.02, out_f)), np.zeros(out_f, np.float32)
    bi, bres = f16(rng.normal(0, 0.01, out_f)), np.zeros(out_f, np.float32)
    gw = (rng.standard_normal(out_f * in_f) * 1e-3).astype(np.float32)
    gs = rng.standard_normal(out_f).astype(np.float32)
    gb = rng.standard_normal(out_f).astype(np.float32)
    l2, lr2, s2, sr2, b2, br2, bits = o.packed_apply_sgd(in_f, out_f, lat, lres, sc, sres, bi,
                                                         bres, gw, gs, gb, 0.01, 2047.0)
    wl, wlr = numpy_binaryconnect(lat, lres, gw * np.float32(2047.0), 0.01)
    ws, wsr = numpy_clipped(sc, sres, gs, 0.01)
    wb, wbr = numpy_clipped(bi, bres, gb, 0.01)
    np.testing.assert_array_equal(l2, wl)
    np.testing.assert_array_equal(lr2.view(np.uint32), wlr.view(np.uint32))
    np.testing.assert_array_equal(s2, ws)
    np.testing.assert_array_equal(b2, wb)
    np.testing.assert_array_equal(bits, pack_bits(wl.view(F16).astype(np.float32) >= 0))


# ------------------------------------------------------------ a10 / a11 LN
def test_layer_norm_population_moments_closed_form():
    # tests/cmix.rs:19-31
    y = o.layer_norm_forward([1.0, 2.0, 3.0], 1, 3, f16([1, 1, 1]), f16([0, 0, 0]))
    inv = 1.0 / np.sqrt(2.0 / 3.0 + 1e-5)
    np.testing.assert_allclose(y, (np.array([1, 2, 3]) - 2.0) * inv, atol=1e-5)


def np_layer_norm(x, w, b):
    mu = x.mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * w + b


def test_layer_norm_affine_metal_fixture_float64():
    # layer_norm_matches_cpu_affine_reference, src/metal.rs:3773-3788
    w, b = f16([1.25, 0.75, 1.0, 0.5]), f16([0.1, -0.2, 0.0, 0.05])
    x = np.array([1.0, 2.0, 3.0, 4.0, 0.5, -1.0, 0.0, 2.5])
    y = o.layer_norm_forward(x, 2, 4, w, b)
    np.testing.assert_allclose(y, np_layer_norm(x.reshape(2, 4), h2f(w), h2f(b)).ravel(), atol=1e-6)


def test_layer_norm_backward_finite_differences():
    rng = np.random.default_rng(6)
    rows, ch = 3, 10
    x = rng.standard_normal((rows, ch))
    gy = rng.standard_normal((rows, ch))
    w, b = f16(rng.uniform(0.5, 1.5, ch)), f16(rng.normal(0, 0.1, ch))
    gx, gw, gb = o.layer_norm_backward(x.ravel(), gy.ravel(), rows, ch, w)
    W, B = h2f(w), h2f(b)

    def loss(xx, ww, bb):
        return float((np_layer_norm(xx, ww, bb) * gy).sum())

    eps = 1e-6
    num = np.zeros_like(x)
    for i in range(rows):
        for j in range(ch):
            d = np.zeros_like(x)
            d[i, j] = eps
            num[i, j] = (loss(x + d, W, B) - loss(x - d, W, B)) / (2 * eps)
    np.testing.assert_allclose(gx.reshape(rows, ch), num, rtol=1e-3, atol=1e-4)
    numw = np.array([(loss(x, W + eps * np.eye(ch)[j], B) - loss(x, W - eps * np.eye(ch)[j], B))
                     / (2 * eps) for j in range(ch)])
    np.testing.assert_allclose(gw, numw, rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(gb, gy.sum(0), atol=1e-5)


# ------------------------------------------------------------- a12 / a13 CE
def test_ce_helpers_reference_cases():
    # src/model.rs:4510-4516: window-mean scale 1/(T-1)
    assert o.causal_ce_gradient_scale(5, 2048) == np.float32(1.0 / 2047.0)
    assert o.causal_ce_gradient_scale(0, 2048) == 0.0
    assert o.causal_ce_gradient_scale(3, 1) == 0.0
    t = [1, 3, 0, 7]
    assert [o.causal_ce_row_valid(r, 2, 1, t, 7) for r in range(4)] == [True, False, False, False]
    assert [o.causal_ce_row_valid(r, 4, 1, t, 99) for r in range(4)] == [True, True, True, False]


def test_head_ce_metal_fixture_float64_and_invariants():
    # streamed_cross_entropy_matches_cpu_oracle_without_materializing_on_gpu, src/metal.rs:4045-4085
    signs = np.array([1, -1, 1, -1, -1, 1, 1, 1]).reshape(4, 2)
    bits = pack_bits((signs >= 0).ravel())
    hidden = np.array([0.5, -0.25, 1.0, 0.0, -0.5, 0.75])
    tokens = np.array([1, 3, 0], np.uint32)
    scale = f16([0.5] * 4)
    bias = f16([0.1, -0.2, 0.0, 0.3])
    out = o.head_ce(hidden, 3, 3, 2, 4, bits, scale, bias, tokens, 0xFFFFFFFF)
    H = hidden.reshape(3, 2)
    logits = h2f(bias)[None] + 0.5 * H @ signs.T
    lse = np.log(np.exp(logits).sum(1))
    ce = lse - logits[np.arange(3), [3, 0, 0]]
    gscale = 1.0 / 2.0
    assert out["n_valid"] == 2 and out["row_loss"][2] == 0.0
    np.testing.assert_allclose(out["row_loss"][:2], ce[:2], atol=1e-6)
    np.testing.assert_allclose(out["mean_loss"], ce[:2].mean(), atol=1e-6)
    p = np.exp(logits - lse[:, None])
    gy = p.copy()
    gy[0, 3] -= 1
    gy[1, 0] -= 1
    gy[2] = 0
    gy *= gscale
    np.testing.assert_allclose(out["hidden_gradient"].reshape(3, 2), (gy * 0.5) @ signs, atol=1e-6)
    np.testing.assert_allclose(out["weight_gradient"].reshape(4, 2), 0.5 * gy.T @ H, atol=1e-6)
    np.testing.assert_allclose(out["scale_gradient"], (gy.T @ H * signs).sum(1), atol=1e-6)
    np.testing.assert_allclose(out["bias_gradient"], gy.sum(0), atol=1e-6)
    assert abs(out["bias_gradient"].sum()) < 1e-6  # sum_v gy = 0 per valid row


def test_head_ce_ignore_id_excludes_targets():
    rng = np.random.default_rng(8)
    rows, time, d, vocab = 8, 4, 3, 5
    plus = rng.integers(0, 2, vocab * d).astype(bool)
    t = np.array([1, 2, 4, 0, 3, 4, 4, 1], np.uint32)
    out = o.head_ce(rng.standard_normal(rows * d), rows, time, d, vocab, pack_bits(plus),
                    f16([0.3] * vocab), None, t, 4)
    valid = [r % time + 1 < time and t[r + 1] != 4 for r in range(rows)]
    assert out["n_valid"] == sum(valid)
    assert all(out["row_loss"][r] == 0.0 for r in range(rows) if not valid[r])


def test_head_ce_horizon_float64():
    # causal_ce_row_valid with horizon h (src/model.rs:27-39): row r is
    # scored against targets[r + h] while r % T + h < T
    rng = np.random.default_rng(13)
    rows, time, d, vocab = 12, 6, 4, 7
    plus = rng.integers(0, 2, vocab * d).astype(bool)
    signs = np.where(plus, 1.0, -1.0).reshape(vocab, d)
    hidden = rng.standard_normal(rows * d)
    t = rng.integers(0, vocab, rows).astype(np.uint32)
    for h in (1, 2, 3):
        out = o.head_ce(hidden, rows, time, d, vocab, pack_bits(plus), f16([0.4] * vocab), None,
                        t, 0xFFFFFFFF, horizon=h)
        H = hidden.astype(np.float32).astype(np.float64).reshape(rows, d)
        logits = h2f(f16([0.4]))[0] * H @ signs.T
        valid = np.array([r % time + h < time and r + h < rows for r in range(rows)])
        assert out["n_valid"] == valid.sum()
        lse = np.log(np.exp(logits).sum(1))
        want = np.where(valid, lse - logits[np.arange(rows), t[np.minimum(np.arange(rows) + h,
                                                                           rows - 1)]], 0.0)
        np.testing.assert_allclose(out["row_loss"], want, atol=2e-6)


# ------------------------------------------------- CausalLoss statistics
def test_causal_loss_statistics_float64():
    # rms / rms_fp16 / mean_abs / mean_abs_fp16 / mean_abs_delta_fp16,
    # src/model.rs:3293-3339, against float64 numpy
    rng = np.random.default_rng(21)
    v = rng.standard_normal(100_000).astype(np.float32) * 3
    h = f16(rng.standard_normal(50_000) * 0.2)
    h2 = f16(h.view(F16).astype(np.float64) + rng.standard_normal(50_000) * 1e-3)
    hv = h.view(F16).astype(np.float64)
    assert abs(o.rms(v) - np.sqrt(np.mean(v.astype(np.float64) ** 2))) <= 1e-4 * np.sqrt(
        np.mean(v.astype(np.float64) ** 2))
    assert abs(o.rms_fp16(h) - np.sqrt(np.mean(hv ** 2))) <= 1e-4 * np.sqrt(np.mean(hv ** 2))
    assert abs(o.mean_abs(v) - np.mean(np.abs(v))) <= 1e-4 * np.mean(np.abs(v))
    assert abs(o.mean_abs_fp16(h) - np.mean(np.abs(hv))) <= 1e-4 * np.mean(np.abs(hv))
    d = np.mean(np.abs(hv - h2.view(F16).astype(np.float64)))
    assert abs(o.mean_abs_delta_fp16(h, h2) - d) <= 1e-4 * d
    assert o.rms(np.zeros(0, np.float32)) == 0.0 and o.mean_abs_fp16(np.zeros(0, np.uint16)) == 0.0


def test_loss_percentiles_rank_rule():
    # loss_percentiles, src/model.rs:3341-3363: finite losses of valid rows,
    # total order, index min(round(p (n - 1)), n - 1) with f32 rounding half
    # away from zero
    rng = np.random.default_rng(22)
    rows, time = 2048, 512
    t = rng.integers(0, 50, rows).astype(np.uint32)
    t[::11] = 7  # ignore id below
    rl = (rng.standard_normal(rows) * 2 + 5).astype(np.float32)
    rl[::37] = np.nan
    rl[::41] = np.inf
    rl[5] = -0.0
    rl[6] = 0.0
    got = o.loss_percentiles(rl, time, t, 7)
    valid = [r for r in range(rows) if r % time + 1 < time and t[r + 1] != 7]
    vals = np.sort(np.array([rl[r] for r in valid if np.isfinite(rl[r])], np.float64))
    n = len(vals)
    for p, g in zip((0.10, 0.50, 0.90), got):
        x = np.float32(p) * np.float32(n - 1)
        at = min(int(np.floor(x + 0.5)), n - 1)  # half away from zero (x >= 0)
        assert g == vals[at], (p, g, vals[at])
    assert o.loss_percentiles(rl, time, np.full(rows, 7, np.uint32), 7) == (0.0, 0.0, 0.0)


def test_unigram_cross_entropy_float64():
    # unigram_cross_entropy, src/model.rs:3365-3390
    from collections import Counter

    rng = np.random.default_rng(23)
    rows, time = 1000, 100
    t = rng.integers(0, 40, rows).astype(np.uint32)
    t[::9] = 99
    valid = [r for r in range(rows) if r % time + 1 < time and t[r + 1] != 99]
    c = Counter(int(t[r + 1]) for r in valid)
    n = len(valid)
    want = -sum(k * np.log(k / n) for k in c.values()) / n
    ce, uniq = o.unigram_cross_entropy(t, time, 99)
    assert uniq == len(c)
    assert abs(ce - want) <= 1e-5 * want
    assert o.unigram_cross_entropy(np.full(10, 99, np.uint32), 5, 99) == (0.0, 0)


# -------------------------------------------------------- a14 FP16 linear
def test_fp16_linear_metal_fixture_float64():
    # fp16_linear_matches_cpu_forward_and_backward, src/metal.rs:3876-3905
    weight = f16([1.0, -0.5, 0.25, 2.0, 0.0, -1.0])
    x = np.array([0.5, 1.0, -1.0, 2.0, 0.0, 0.25])
    gy = np.array([1.0, -1.0, 0.5, 0.25])
    W = h2f(weight).reshape(2, 3)
    X = x.reshape(2, 3)
    np.testing.assert_allclose(o.fp16_forward(x, 2, 3, 2, weight), (X @ W.T).ravel(), atol=1e-6)
    gx, gw = o.fp16_backward(x, gy, 2, 3, 2, weight)
    G = gy.reshape(2, 2)
    np.testing.assert_allclose(gx, (G @ W).ravel(), atol=1e-6)
    np.testing.assert_allclose(gw, (G.T @ X).ravel(), atol=1e-6)


# ------------------------------------------------------------ a15 CMix
def cmix_forward(x, batch, time, d, f, x_k, key_bits, key_scale, value):
    xx = o.time_shift_delta(x, batch, time, d)
    shifted = (np.asarray(x, np.float32) + xx * np.tile(h2f(x_k).astype(np.float32), batch * time))
    k = o.packed_forward(shifted, batch * time, d, f, key_bits, key_scale, None)
    r = np.maximum(k, 0) ** 2
    return o.fp16_forward(r, batch * time, f, d, value)


def test_cmix_reference_closed_forms():
    # tests/cmix.rs:33-50: zero shift is relu^2 then value
    y = cmix_forward([1.0, 0.0, 0.0, 1.0], 1, 2, 2, 2, f16([0, 0]),
                     pack_bits([True, False, False, True]), f16([1, 1]), f16([1, 0, 0, 1]))
    np.testing.assert_allclose(y, [1, 0, 0, 1], atol=1e-5)
    # tests/cmix.rs:52-72: the shift uses the previous token
    y = cmix_forward([2.0, 0.0, 0.0, 0.0], 1, 2, 2, 1, f16([1, 0]), pack_bits([True, True]),
                     f16([1]), f16([1, 0]))
    np.testing.assert_allclose(y, [0, 0, 4, 0], atol=1e-4)


def test_time_shift_delta_batches_reset():
    x = np.arange(12, dtype=np.float32)
    xx = o.time_shift_delta(x, 2, 3, 2).reshape(2, 3, 2)
    X = x.reshape(2, 3, 2)
    want = np.concatenate([-X[:, :1], X[:, :-1] - X[:, 1:]], axis=1)
    np.testing.assert_array_equal(xx, want)


def test_lerp_shift_backward_finite_differences():
    rng = np.random.default_rng(9)
    batch, time, ch = 2, 5, 3
    x = rng.standard_normal(batch * time * ch)
    mix = f16(rng.uniform(0, 1, ch))
    gs = rng.standard_normal(batch * time * ch)
    M = h2f(mix)

    def shifted(xv, mv):
        X = xv.reshape(batch, time, ch)
        prev = np.concatenate([np.zeros((batch, 1, ch)), X[:, :-1]], axis=1)
        return (X + (prev - X) * mv).ravel()

    xx = o.time_shift_delta(x, batch, time, ch)
    g_x, g_mix = o.lerp_shift_backward(xx, mix, gs, batch, time, ch)
    eps = 1e-6
    num = np.array([((shifted(x + eps * e, M) - shifted(x - eps * e, M)) @ gs) / (2 * eps)
                    for e in np.eye(x.size)])
    np.testing.assert_allclose(g_x, num, atol=1e-5)
    numm = np.array([((shifted(x, M + eps * e) - shifted(x, M - eps * e)) @ gs) / (2 * eps)
                     for e in np.eye(ch)])
    np.testing.assert_allclose(g_mix, numm, atol=1e-4)


# ------------------------------------------------------------- a16 ROSA
def test_rosa_expand_and_e_grad_float64():
    rng = np.random.default_rng(10)
    rows, ch = 6, 4
    idx = rng.integers(0, 2, rows * ch).astype(np.uint8)
    e = f16(rng.normal(0, 0.1, ch))
    y = o.rosa_y_from_idx(idx, e, rows, ch)
    np.testing.assert_array_equal(y, ((2.0 * idx - 1.0).reshape(rows, ch) * h2f(e)).ravel().astype(np.float32))
    gy = rng.standard_normal(rows * ch)
    ge = o.rosa_e_grad(gy, idx, rows, ch)
    np.testing.assert_allclose(ge, (gy.reshape(rows, ch) * (2.0 * idx.reshape(rows, ch) - 1)).sum(0),
                               atol=1e-6)


def test_embedding_gather_and_scatter_sgd_against_numpy():
    # train_step_on's gather / scatter loops (src/model.rs:2866-2873, 2986-2993)
    rng = np.random.default_rng(12)
    vocab, d, rows = 9, 5, 40
    table = f16(rng.normal(0, 0.5, vocab * d))
    res = (rng.standard_normal(vocab * d) * 1e-4).astype(np.float32)
    tokens = rng.integers(0, vocab, rows).astype(np.uint32)  # many repeats
    x = o.embedding_gather(table, d, tokens)
    np.testing.assert_array_equal(x, h2f(table).reshape(vocab, d)[tokens].ravel())
    g = (rng.standard_normal(rows * d) * 0.7).astype(np.float32)
    lr = 0.05
    got_t, got_r = o.embedding_scatter_sgd(table, res, d, tokens, g, lr)
    want_t, want_r = table.copy(), res.copy()
    for r, tok in enumerate(tokens):  # one row at a time, in row order
        sl = slice(int(tok) * d, int(tok) * d + d)
        want_t[sl], want_r[sl] = numpy_clipped(want_t[sl], want_r[sl], g[r * d:(r + 1) * d], lr)
    np.testing.assert_array_equal(got_t, want_t)
    np.testing.assert_array_equal(got_r.view(np.uint32), want_r.view(np.uint32))
    # the order of repeated rows matters (f16 rounding between applications),
    # so a reordered loop fails this check
    rev_t, rev_r = table.copy(), res.copy()
    for r in reversed(range(rows)):
        sl = slice(int(tokens[r]) * d, int(tokens[r]) * d + d)
        rev_t[sl], rev_r[sl] = numpy_clipped(rev_t[sl], rev_r[sl], g[r * d:(r + 1) * d], lr)
    assert not (np.array_equal(rev_t, want_t) and np.array_equal(rev_r, want_r))
