"""GPU parity of the unit operations against the CPU oracle, through the C ABI.

Tolerances: bit-exact for sign packing and
the FP16 / BinaryConnect SGD updates on identical inputs; relative error
max|gpu - ref| / max|ref| <= 1e-3 per tensor for fp16 linear / LayerNorm
outputs and gradients (the GPU feeds fp16 operands to MFMA with fp32
accumulation; the oracle computes in fp32 on the same fp16-rounded inputs).
"""
import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.synth import f16, pack_bits

pytestmark = pytest.mark.gpu

REL = 1e-3


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    assert a.shape == r.shape
    assert np.isfinite(a).all()
    denom = max(float(np.max(np.abs(r))), 1e-30)
    return float(np.max(np.abs(a - r))) / denom


def h2f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def rand_case(rng, rows, in_f, out_f, bias=True):
    x16 = f16(rng.standard_normal(rows * in_f))
    lat = rng.uniform(-0.01, 0.01, out_f * in_f)
    bits = pack_bits(lat >= 0)
    scale = f16(rng.uniform(0.005, 0.02, out_f))
    b = f16(rng.normal(0, 0.01, out_f)) if bias else None
    return x16, bits, scale, b


# ------------------------------------------------------------ packed linear
def test_binary_linear_metal_fixture(rt):
    # binary_linear_matches_packed_cpu_forward_and_ste, src/metal.rs:3806-3844
    signs = [1, -1, -1, 1, 1, 1]
    bits = pack_bits(np.array(signs) >= 0)
    x = np.array([0.5, -1.0, 2.0, 1.0, 0.0, -0.5], np.float32)
    scale, bias = f16([0.5, 0.5]), f16([0.0, 0.0])
    y = rt.binary_linear(x, bits, scale, bias, 2, 3, 2)
    want = o.packed_forward(x, 2, 3, 2, bits, scale, bias)
    np.testing.assert_allclose(y, want, atol=2e-3)
    gy = np.array([1.0, -0.5, 0.25, 0.75], np.float32)
    g = rt.binary_linear_backward(f16(x), gy, bits, scale, True, 2, 3, 2)
    w = o.packed_backward_ste(x, gy, 2, 3, 2, bits, scale)
    for k in ["input_gradient", "weight_gradient", "scale_gradient", "bias_gradient"]:
        np.testing.assert_allclose(g[k], w[k], atol=2e-3, err_msg=k)


def test_binary_linear_tiled_fixture_past_tile_boundary(rt):
    # tiled_linears_match_cpu_past_tile_boundary, src/metal.rs:3908-3974 (rows 17, in 19, out 18)
    rows, inn, out = 17, 19, 18
    signs = np.array([[1 if (a + i) % 2 == 0 else -1 for i in range(inn)] for a in range(out)])
    x = np.array([[((r * 5 + i) % 11) * 0.125 - 0.5 for i in range(inn)] for r in range(rows)],
                 np.float32).ravel()
    gy = np.array([[((r + a) % 5) * 0.2 - 0.4 for a in range(out)] for r in range(rows)],
                  np.float32).ravel()
    bits = pack_bits((signs >= 0).ravel())
    scale, bias = f16([0.5] * out), f16([0.0] * out)
    y = rt.binary_linear(x, bits, scale, bias, rows, inn, out)
    np.testing.assert_allclose(y, o.packed_forward(x, rows, inn, out, bits, scale, bias), atol=3e-3)
    g = rt.binary_linear_backward(f16(x), gy, bits, scale, True, rows, inn, out)
    w = o.packed_backward_ste(x, gy, rows, inn, out, bits, scale)
    for k in ["input_gradient", "weight_gradient", "scale_gradient", "bias_gradient"]:
        np.testing.assert_allclose(g[k], w[k], atol=4e-3, err_msg=k)
    weight = f16(np.array([[((a * 3 + i) % 7) * 0.25 - 0.5 for i in range(inn)]
                           for a in range(out)]).ravel())
    np.testing.assert_allclose(rt.fp16_linear(x, weight, rows, inn, out),
                               o.fp16_forward(x, rows, inn, out, weight), atol=3e-3)
    gx, gw = rt.fp16_linear_backward(f16(x), gy, weight, rows, inn, out)
    wgx, wgw = o.fp16_backward(x, gy, rows, inn, out, weight)
    np.testing.assert_allclose(gx, wgx, atol=4e-3)
    np.testing.assert_allclose(gw, wgw, atol=4e-3)


SHAPES = [
    (2048, 256, 256),   # config 1 (TrainConfig::default layer)
    (2048, 512, 512),   # heron QKVO
    (2048, 512, 2048),  # heron CMix key
    (100, 96, 70),      # ragged, multi-tile
    (64, 40, 96),       # in not a multiple of 32 (unaligned sign rows)
]


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
def test_binary_linear_forward_parity(rt, rows, in_f, out_f):
    rng = np.random.default_rng(rows + in_f + out_f)
    x16, bits, scale, bias = rand_case(rng, rows, in_f, out_f)
    want = o.packed_forward(h2f32(x16), rows, in_f, out_f, bits, scale, bias)
    y32 = rt.binary_linear(x16, bits, scale, bias, rows, in_f, out_f)
    assert rel(y32, want) <= REL
    y16 = rt.binary_linear(x16, bits, scale, bias, rows, in_f, out_f, out_dtype=np.float16)
    assert rel(h2f32(y16), want) <= REL
    # fp32 activations accepted too (converted on load)
    yf = rt.binary_linear(h2f32(x16), bits, scale, None, rows, in_f, out_f, x_dtype=2)
    assert rel(yf, o.packed_forward(h2f32(x16), rows, in_f, out_f, bits, scale, None)) <= REL


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
def test_binary_linear_backward_parity(rt, rows, in_f, out_f):
    rng = np.random.default_rng(7 + rows + in_f + out_f)
    x16, bits, scale, _ = rand_case(rng, rows, in_f, out_f)
    gy = rng.normal(0, 1e-2, rows * out_f).astype(np.float32)
    g = rt.binary_linear_backward(x16, gy, bits, scale, True, rows, in_f, out_f)
    w = o.packed_backward_ste(h2f32(x16), gy, rows, in_f, out_f, bits, scale)
    for k in ["input_gradient", "weight_gradient", "scale_gradient", "bias_gradient"]:
        assert rel(g[k], w[k]) <= REL, k


# Weight gradients over >= 16384 rows whose [out, in] tiles by 256 run on
# 256x256 tiles split over the rows (context.hpp dw_giant), and packed input
# gradients with 512 or more 256x256 output tiles on 256x256 tiles over the
# scaled sign bits expanded in LDS (32768 rows here). The scalar oracle
# is too slow at these sizes, so the reference is the closed form in float64 on
# the same inputs, G = gy^T . x: the fp16 weight gradient is G
# (src/metal.rs:2829-2908); the packed one is scale[o] * G, with g_scale[o] =
# sum_i sign(o, i) G(o, i), g_bias = column sums of gy and gx = gy . (scale *
# sign) (the oracle's ucr_packed_backward_ste, src/model.rs:745-796).
@pytest.mark.parametrize("rows,in_f,out_f",
                         [(16384, 1024, 1024), (16384, 256, 4096), (32768, 1024, 1024),
                          # 4 row splits of 384 rows: the last split is empty
                          (1152, 256, 256)])
def test_weight_gradients_over_many_rows(rt, rows, in_f, out_f):
    rng = np.random.default_rng(rows + in_f + 3 * out_f)
    x16, bits, scale, _ = rand_case(rng, rows, in_f, out_f)
    gy = rng.normal(0, 1e-2, rows * out_f).astype(np.float32)
    x64 = h2f32(x16).reshape(rows, in_f).astype(np.float64)
    gy64 = gy.reshape(rows, out_f).astype(np.float64)
    G = gy64.T @ x64
    w = f16(rng.normal(0, 0.02, out_f * in_f))
    _, gw = rt.fp16_linear_backward(x16, gy, w, rows, in_f, out_f)
    assert rel(gw, G.ravel()) <= REL
    sc = h2f32(scale).astype(np.float64)
    lat = np.unpackbits(np.asarray(bits, np.uint32).view(np.uint8), bitorder="little")
    sign = np.where(lat[: out_f * in_f].reshape(out_f, in_f) != 0, 1.0, -1.0)
    g = rt.binary_linear_backward(x16, gy, bits, scale, True, rows, in_f, out_f)
    assert rel(g["weight_gradient"], (sc[:, None] * G).ravel()) <= REL
    assert rel(g["scale_gradient"], (sign * G).sum(axis=1)) <= REL
    assert rel(g["bias_gradient"], gy64.sum(axis=0)) <= REL
    assert rel(g["input_gradient"], (gy64 @ (sc[:, None] * sign)).ravel()) <= REL


def finite_rel_and_masks(a, r, name):
    """Non-finite entries must sit where the oracle's are (NaN where NaN, +-Inf
    where +-Inf); the finite ones within REL of the finite reference."""
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    np.testing.assert_array_equal(np.isnan(a), np.isnan(r), err_msg=name + " NaN mask")
    np.testing.assert_array_equal(np.isposinf(a), np.isposinf(r), err_msg=name + " +Inf mask")
    np.testing.assert_array_equal(np.isneginf(a), np.isneginf(r), err_msg=name + " -Inf mask")
    fin = np.isfinite(r)
    if fin.any():
        assert rel(a[fin], r[fin]) <= REL, name


@pytest.mark.parametrize("inject", ["nan", "inf"])
def test_binary_linear_backward_nonfinite_gradient(rt, inject):
    # A NaN or an Inf in the upstream gradient reaches the products as in the
    # reference's fp32 arithmetic: the gradient's fp16 operand keeps it (the
    # amax scale is taken over finite values only), so every output that sums
    # over it is NaN / Inf exactly where the oracle's is, and the rest keeps
    # the finite tolerance. One known divergence: for an Inf in column o the
    # reference forms g_scale[o] = sum_r gy[r,o] (sum_i sign x[r,i]) = +-Inf,
    # while here g_scale[o] = sum_i sign[o,i] G[o,i] adds +Inf and -Inf terms
    # of G's row o and gives NaN; both are non-finite.
    rows, in_f, out_f = 256, 128, 192
    rng = np.random.default_rng(99)
    x16, bits, scale, _ = rand_case(rng, rows, in_f, out_f)
    x16[(x16 & 0x7FFF) == 0] = f16([0.5])[0]  # no Inf * 0 in the products
    gy = rng.normal(0, 1e-2, rows * out_f).astype(np.float32)
    if inject == "nan":
        gy[17 * out_f + 5] = np.nan
        gy[30 * out_f + 77] = np.uint32(0xFFC00000).view(np.float32)
    else:
        gy[101 * out_f + 77] = np.inf
        gy[3 * out_f + 5] = -np.inf
    g = rt.binary_linear_backward(x16, gy, bits, scale, True, rows, in_f, out_f)
    w = o.packed_backward_ste(h2f32(x16), gy, rows, in_f, out_f, bits, scale)
    for k in ["input_gradient", "weight_gradient", "bias_gradient"]:
        finite_rel_and_masks(g[k], w[k], k)
    if inject == "nan":
        finite_rel_and_masks(g["scale_gradient"], w["scale_gradient"], "scale_gradient")
    else:
        np.testing.assert_array_equal(np.isfinite(g["scale_gradient"]),
                                      np.isfinite(w["scale_gradient"]))
        fin = np.isfinite(w["scale_gradient"])
        assert rel(g["scale_gradient"][fin], w["scale_gradient"][fin]) <= REL
    assert not np.isfinite(g["weight_gradient"][5 * in_f:6 * in_f]).any()
    assert not np.isfinite(g["weight_gradient"][77 * in_f:78 * in_f]).any()
    # the BinaryConnect step skips non-finite gradients (src/precision.rs:125-127)
    lat = f16(rng.uniform(-0.01, 0.01, out_f * in_f))
    res = np.zeros(out_f * in_f, np.float32)
    gl, gr, _, _ = rt.apply_latent_sgd(lat, res, g["weight_gradient"], out_f, in_f, 0.01, 63.0)
    bad = ~np.isfinite(g["weight_gradient"])
    np.testing.assert_array_equal(gl[bad], lat[bad])
    wl, wr = o.binaryconnect_sgd(lat, res, g["weight_gradient"], 0.01, 63.0)
    np.testing.assert_array_equal(gl, wl)
    np.testing.assert_array_equal(gr.view(np.uint32), wr.view(np.uint32))


@pytest.mark.parametrize("rows,in_f,out_f", [(2048, 2048, 512), (2048, 512, 2048), (50, 24, 40)])
def test_fp16_linear_parity(rt, rows, in_f, out_f):
    rng = np.random.default_rng(11 + rows + in_f)
    x16 = f16(np.maximum(rng.standard_normal(rows * in_f), 0) ** 2)
    w = f16(rng.normal(0, 0.02, out_f * in_f))
    want = o.fp16_forward(h2f32(x16), rows, in_f, out_f, w)
    assert rel(rt.fp16_linear(x16, w, rows, in_f, out_f), want) <= REL
    gy = rng.normal(0, 1e-2, rows * out_f).astype(np.float32)
    gx, gw = rt.fp16_linear_backward(x16, gy, w, rows, in_f, out_f)
    wgx, wgw = o.fp16_backward(h2f32(x16), gy, rows, in_f, out_f, w)
    assert rel(gx, wgx) <= REL
    assert rel(gw, wgw) <= REL


# -------------------------------------------------------------- LayerNorm
def test_layer_norm_metal_fixtures(rt):
    # src/metal.rs:3773-3803
    w, b = f16([1.25, 0.75, 1.0, 0.5]), f16([0.1, -0.2, 0.0, 0.05])
    x = np.array([1.0, 2.0, 3.0, 4.0, 0.5, -1.0, 0.0, 2.5], np.float32)
    np.testing.assert_allclose(rt.layer_norm(x, w, b, 2, 4), o.layer_norm_forward(x, 2, 4, w, b),
                               atol=2e-3)
    x = np.array([1.0, 2.0, 0.0, -1.0, 4.0, 1.0, -2.0, 0.5], np.float32)
    gy = np.array([0.2, -0.1, 0.3, 0.0, -0.4, 0.15, 0.05, -0.2], np.float32)
    wt = f16([1.0, 0.5, 1.5, 0.75])
    got = rt.layer_norm_backward(x, gy, wt, 2, 4)
    want = o.layer_norm_backward(x, gy, 2, 4, wt)
    for a, r in zip(got, want):
        np.testing.assert_allclose(a, r, atol=3e-3)


@pytest.mark.parametrize("rows,ch", [(2048, 256), (2048, 512), (4096, 1024), (37, 19), (5, 2000)])
def test_layer_norm_parity(rt, rows, ch):
    rng = np.random.default_rng(rows * 3 + ch)
    x = (rng.standard_normal(rows * ch) * 3 + 0.5).astype(np.float32)
    w, b = f16(rng.uniform(0.5, 1.5, ch)), f16(rng.normal(0, 0.1, ch))
    want = o.layer_norm_forward(x, rows, ch, w, b)
    assert rel(rt.layer_norm(x, w, b, rows, ch), want) <= REL
    assert rel(h2f32(rt.layer_norm(x, w, b, rows, ch, out_dtype=np.float16)), want) <= REL
    gy = rng.normal(0, 1e-2, rows * ch).astype(np.float32)
    got = rt.layer_norm_backward(x, gy, w, rows, ch)
    ref = o.layer_norm_backward(x, gy, rows, ch, w)
    for a, r, name in zip(got, ref, ["gx", "gw", "gb"]):
        assert rel(a, r) <= REL, name


# ---------------------------------------------------------- bit-exact ops
def test_sgd_metal_fixtures_bit_exact(rt):
    # src/metal.rs:4007-4042
    p, r = rt.clipped_sgd_fp16(f16([0.25, -1.0, 2.0]), np.zeros(3, np.float32),
                               np.array([0.001, 0.5, -0.25], np.float32), 0.01)
    wp, wr = o.clipped_sgd(f16([0.25, -1.0, 2.0]), np.zeros(3), [0.001, 0.5, -0.25], 0.01)
    np.testing.assert_array_equal(p, wp)
    np.testing.assert_array_equal(r.view(np.uint32), wr.view(np.uint32))
    p, r = rt.binaryconnect_sgd_fp16(f16([0.0625, -0.0625, 0.9]), np.zeros(3, np.float32),
                                     np.array([1e-5, -1e-6, 2.0], np.float32), 0.1)
    wp, wr = o.binaryconnect_sgd(f16([0.0625, -0.0625, 0.9]), np.zeros(3), [1e-5, -1e-6, 2.0], 0.1)
    np.testing.assert_array_equal(p, wp)
    np.testing.assert_array_equal(r.view(np.uint32), wr.view(np.uint32))


@pytest.mark.parametrize("lr", [0.01, 0.1])
def test_sgd_random_bit_exact(rt, lr):
    rng = np.random.default_rng(int(lr * 1000))
    n = 1 << 20
    p = f16(rng.uniform(-1.2, 1.2, n) * (10.0 ** rng.integers(-6, 1, n)))
    res = (rng.standard_normal(n) * 1e-5).astype(np.float32)
    g = (rng.standard_normal(n) * (10.0 ** rng.integers(-7, 2, n))).astype(np.float32)
    g[::97] = 0.0
    g[::101] = np.inf
    g[::103] = np.nan
    g[::107] = np.uint32(0xFFC00000).view(np.float32)  # negative quiet NaN
    g[::109] = np.uint32(0x7FA00001).view(np.float32)  # NaN with a payload
    g[::113] = -np.inf
    # clipped SGD takes non-finite gradients as the reference does: +-Inf
    # clamps to +-1 (bit-exact), NaN carries into the value as the canonical
    # quiet NaN 0x7e00 (src/precision.rs:29-31) and into the carry. IEEE 754
    # leaves the sign of a NaN result open (x86 and gfx950 differ in how a
    # subtraction treats it), so NaN values are compared up to the sign bit.
    a, b = rt.clipped_sgd_fp16(p, res, g, lr)
    wa, wb = o.clipped_sgd(p, res, g, lr)
    nan = np.isnan(g)
    np.testing.assert_array_equal(a[~nan], wa[~nan])
    np.testing.assert_array_equal(b[~nan].view(np.uint32), wb[~nan].view(np.uint32))
    assert ((a[nan] & 0x7FFF) == 0x7E00).all() and np.isnan(b[nan]).all()
    a, b = rt.binaryconnect_sgd_fp16(p, res, g, lr)
    wa, wb = o.binaryconnect_sgd(p, res, g, lr)
    np.testing.assert_array_equal(a, wa)
    np.testing.assert_array_equal(b.view(np.uint32), wb.view(np.uint32))


@pytest.mark.parametrize("out_f,in_f", [(512, 512), (2048, 512), (18, 19), (8192, 512)])
def test_apply_latent_sgd_bit_exact(rt, out_f, in_f):
    rng = np.random.default_rng(out_f + in_f)
    n = out_f * in_f
    lat = f16(rng.uniform(-0.01, 0.01, n))
    lat[:4] = [0x0000, 0x8000, 0x0001, 0x8001]
    res = np.zeros(n, np.float32)
    g = (rng.standard_normal(n) * 1e-5).astype(np.float32)
    g[5::7] = 0.0
    gl, gr, bits, bits_t = rt.apply_latent_sgd(lat, res, g, out_f, in_f, 0.01, 2047.0)
    wl, wr = o.binaryconnect_sgd(lat, res, g, 0.01, 2047.0)
    np.testing.assert_array_equal(gl, wl)
    np.testing.assert_array_equal(gr.view(np.uint32), wr.view(np.uint32))
    wbits = o.pack_latent_bits(wl)
    np.testing.assert_array_equal(bits, wbits)
    np.testing.assert_array_equal(bits_t, o.transpose_bits(wbits, out_f, in_f))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 2048 * 512])
def test_sign_pack_bits_bit_exact(rt, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    x[::13] = 0.0
    x[1::17] = -0.0
    np.testing.assert_array_equal(rt.sign_pack_bits(x), o.sign_pack_bits(x))


@pytest.mark.parametrize("out_f,in_f", [(512, 512), (8192, 512), (18, 19), (96, 40)])
def test_transpose_bits_bit_exact(rt, out_f, in_f):
    bits = pack_bits(np.random.default_rng(out_f).integers(0, 2, out_f * in_f).astype(bool))
    np.testing.assert_array_equal(rt.transpose_bits(bits, out_f, in_f),
                                  o.transpose_bits(bits, out_f, in_f))


# -------------------------------------------------------------- head + CE
def test_head_ce_metal_fixture(rt):
    # streamed_cross_entropy_matches_cpu_oracle_without_materializing_on_gpu, src/metal.rs:4045-4085
    signs = [1, -1, 1, -1, -1, 1, 1, 1]
    bits = pack_bits(np.array(signs) >= 0)
    hidden = np.array([0.5, -0.25, 1.0, 0.0, -0.5, 0.75], np.float32)
    tokens = np.array([1, 3, 0], np.uint32)
    scale = f16([0.5] * 4)
    lat = f16(np.where(np.array(signs) >= 0, 0.5, -0.5))
    got = rt.packed_head_train_sgd(f16(hidden), bits, scale, None, lat, np.zeros(8, np.float32),
                                   np.zeros(4, np.float32), None, tokens, 3, 3, 2, 4,
                                   0xFFFFFFFF, 0.0, 1.0, want_g_w=True)
    want = o.head_ce(hidden, 3, 3, 2, 4, bits, scale, None, tokens, 0xFFFFFFFF)
    assert abs(got["mean_loss"] - want["mean_loss"]) < 3e-3
    assert got["row_loss"][2] == 0.0
    np.testing.assert_allclose(got["hidden_gradient"], want["hidden_gradient"], atol=5e-3)
    np.testing.assert_allclose(got["scale_gradient"], want["scale_gradient"], atol=5e-3)
    np.testing.assert_allclose(got["weight_gradient"], want["weight_gradient"], atol=5e-3)


@pytest.mark.parametrize("rows,time,d,vocab,ignore", [
    (256, 64, 64, 1000, 0xFFFFFFFF),
    (512, 128, 128, 2500, 7),
    (256, 256, 512, 8192, 0xFFFFFFFF),  # config 3 widths (d 512, vocab 8192), 256 rows
    (2048, 2048, 512, 8192, 0xFFFFFFFF),  # config 3 at full size (T = 2048)
])
def test_head_ce_parity_and_update(rt, rows, time, d, vocab, ignore):
    rng = np.random.default_rng(rows + d + vocab)
    hidden16 = f16(rng.standard_normal(rows * d))
    lat = f16(rng.uniform(-0.01, 0.01, vocab * d))
    bits = pack_bits(h2f32(lat) >= 0)
    scale = f16(rng.uniform(0.005, 0.02, vocab))
    bias = f16(rng.normal(0, 0.01, vocab))
    targets = rng.integers(0, vocab, rows).astype(np.uint32)
    if ignore != 0xFFFFFFFF:
        targets[::5] = ignore
    lr, ste = 0.01, float(time - 1)
    got = rt.packed_head_train_sgd(hidden16, bits, scale, bias, lat, np.zeros(vocab * d, np.float32),
                                   np.zeros(vocab, np.float32), np.zeros(vocab, np.float32),
                                   targets, rows, time, d, vocab, ignore, lr, ste, want_g_w=True)
    want = o.head_ce(h2f32(hidden16), rows, time, d, vocab, bits, scale, bias, targets, ignore)
    assert got["n_valid"] == want["n_valid"]
    assert abs(got["mean_loss"] - want["mean_loss"]) <= 1e-4
    assert np.max(np.abs(got["row_loss"] - want["row_loss"])) <= 1e-4
    for k in ["hidden_gradient", "scale_gradient", "bias_gradient", "weight_gradient"]:
        assert rel(got[k], want[k]) <= REL, k
    # The update applied to the GPU's own gradients is bit-exact with the oracle's
    # update rules (head: latent step, scale at lr, bias at 8 lr; src/model.rs:3118-3193).
    wl, wlr = o.binaryconnect_sgd(lat, np.zeros(vocab * d), got["weight_gradient"], lr, ste)
    np.testing.assert_array_equal(got["next_latent"], wl)
    np.testing.assert_array_equal(got["next_residual"].view(np.uint32), wlr.view(np.uint32))
    ws, _ = o.clipped_sgd(scale, np.zeros(vocab), got["scale_gradient"], lr)
    np.testing.assert_array_equal(got["next_scale"], ws)
    wb, _ = o.clipped_sgd(bias, np.zeros(vocab), got["bias_gradient"], lr * 8.0)
    np.testing.assert_array_equal(got["next_bias"], wb)
    wbits = o.pack_latent_bits(wl)
    np.testing.assert_array_equal(got["next_bits"], wbits)
    np.testing.assert_array_equal(got["next_bits_t"], o.transpose_bits(wbits, vocab, d))


@pytest.mark.parametrize("horizon", [2, 5])
def test_head_ce_horizon_matches_oracle(rt, horizon):
    # packed_head_train_sgd's horizon (src/metal.rs:3300-3316; causal_ce_row_valid,
    # src/model.rs:27-39): row r is scored against targets[r + horizon]
    rows, time, d, vocab = 256, 64, 64, 1000
    rng = np.random.default_rng(40 + horizon)
    hidden16 = f16(rng.standard_normal(rows * d))
    lat = f16(rng.uniform(-0.01, 0.01, vocab * d))
    bits = pack_bits(h2f32(lat) >= 0)
    scale = f16(rng.uniform(0.005, 0.02, vocab))
    targets = rng.integers(0, vocab, rows).astype(np.uint32)
    targets[::9] = 3
    got = rt.packed_head_train_sgd(hidden16, bits, scale, None, lat, np.zeros(vocab * d, np.float32),
                                   np.zeros(vocab, np.float32), None, targets, rows, time, d,
                                   vocab, 3, 0.0, 1.0, want_g_w=True, horizon=horizon)
    want = o.head_ce(h2f32(hidden16), rows, time, d, vocab, bits, scale, None, targets, 3,
                     horizon=horizon)
    assert got["n_valid"] == want["n_valid"] < rows - rows // time
    assert got["invalid"] == 0
    assert np.max(np.abs(got["row_loss"] - want["row_loss"])) <= 1e-4
    for k in ["hidden_gradient", "scale_gradient", "weight_gradient"]:
        assert rel(got[k], want[k]) <= REL, k


def test_head_ce_labels_outside_vocab_are_counted_and_left_out(rt):
    # A label >= vocab (other than the ignore id) is refused by the reference's
    # train step (src/model.rs:2852-2861). The unit op counts it and leaves the
    # row out, which is the oracle's result with that label set to the ignore id.
    rows, time, d, vocab = 128, 64, 64, 500
    rng = np.random.default_rng(41)
    hidden16 = f16(rng.standard_normal(rows * d))
    lat = f16(rng.uniform(-0.01, 0.01, vocab * d))
    bits = pack_bits(h2f32(lat) >= 0)
    scale = f16(rng.uniform(0.005, 0.02, vocab))
    targets = rng.integers(0, vocab, rows).astype(np.uint32)
    targets[[10, 40, 0]] = [vocab, vocab + 7, 0xFFFFFFF0]
    got = rt.packed_head_train_sgd(hidden16, bits, scale, None, lat, np.zeros(vocab * d, np.float32),
                                   np.zeros(vocab, np.float32), None, targets, rows, time, d,
                                   vocab, 0xFFFFFFFF, 0.0, 1.0, want_g_w=True)
    assert got["invalid"] == 3
    clean = targets.copy()
    clean[[10, 40, 0]] = 0xFFFFFFFE
    want = o.head_ce(h2f32(hidden16), rows, time, d, vocab, bits, scale, None, clean, 0xFFFFFFFE)
    assert got["n_valid"] == want["n_valid"] == rows - 2 - 2
    assert got["row_loss"][9] == 0.0 and got["row_loss"][39] == 0.0
    assert np.max(np.abs(got["row_loss"] - want["row_loss"])) <= 1e-4
    for k in ["hidden_gradient", "scale_gradient", "weight_gradient"]:
        assert rel(got[k], want[k]) <= REL, k


# -------------------------------------------------------------- device copy
@pytest.mark.parametrize("dst_off,src_off,n", [(0, 0, 1 << 20), (3, 3, 4099), (1, 6, 777),
                                               (0, 0, 5), (16, 0, 4096 + 9)])
def test_device_copy_kernel(rt, dst_off, src_off, n):
    from ullis_amd.runtime import DeviceBuffer

    data = np.random.default_rng(n).integers(0, 256, src_off + n + 32).astype(np.uint8)
    src = rt.put(data)
    dst = DeviceBuffer(rt, dst_off + n + 32).upload(np.full(dst_off + n + 32, 0xAB, np.uint8))
    rt._check(rt.lib.ullis_hip_copy(rt.ctx, dst.ptr + dst_off, src.ptr + src_off, n), "copy")
    got = dst.download(np.uint8, dst_off + n + 32)
    np.testing.assert_array_equal(got[dst_off:dst_off + n], data[src_off:src_off + n])
    assert (got[:dst_off] == 0xAB).all() and (got[dst_off + n:] == 0xAB).all()
    src.free()
    dst.free()


# --------------------------------------------------------------- embedding
@pytest.mark.parametrize("vocab,d,rows,dist", [
    (8192, 512, 2048, "zipf"),   # config 4 widths, natural repeats
    (5, 7, 100, "uniform"),      # heavy collisions, d not a multiple of 4
    (1, 64, 300, "uniform"),     # one token: a 300-row chain across ballot chunks
    (50000, 256, 513, "uniform"),
    (3, 8, 40000, "uniform"),    # chains of ~13k rows across several 16384-row walk windows
    (32768, 1024, 32768, "uniform"),  # config 5 widths
    (40, 2100, 300, "uniform"),  # wider than one walk's 2048 register-held channels
])
def test_embedding_gather_scatter_sgd_bit_exact(rt, vocab, d, rows, dist):
    rng = np.random.default_rng(vocab + d + rows)
    table = f16(rng.normal(0, 0.5, vocab * d))
    res = (rng.standard_normal(vocab * d) * 1e-4).astype(np.float32)
    if dist == "zipf":
        tokens = (rng.zipf(1.3, rows) - 1) % vocab
    else:
        tokens = rng.integers(0, vocab, rows)
    tokens = tokens.astype(np.uint32)
    x = rt.embedding_gather(table, tokens, vocab, d)
    np.testing.assert_array_equal(x.view(np.uint32), o.embedding_gather(table, d, tokens).view(np.uint32))
    g = (rng.standard_normal(rows * d) * 0.7).astype(np.float32)
    for lr in (0.01, 0.3):
        got_t, got_r = rt.embedding_scatter_sgd(table, res, tokens, g, vocab, d, lr)
        want_t, want_r = o.embedding_scatter_sgd(table, res, d, tokens, g, lr)
        np.testing.assert_array_equal(got_t, want_t)
        np.testing.assert_array_equal(got_r.view(np.uint32), want_r.view(np.uint32))


def test_embedding_out_of_range_ids(rt):
    # the reference rejects ids >= vocab (src/model.rs:2850-2861); on the device
    # the gather zeroes and counts such rows and the scatter skips them
    from ullis_amd.runtime import HipError

    vocab, d = 16, 32
    rng = np.random.default_rng(3)
    table = f16(rng.normal(0, 0.5, vocab * d))
    res = np.zeros(vocab * d, np.float32)
    tokens = np.array([3, 16, 3, 0xFFFFFFFF, 7], np.uint32)
    with pytest.raises(HipError, match="2 token ids"):
        rt.embedding_gather(table, tokens, vocab, d)
    g = (rng.standard_normal(tokens.size * d)).astype(np.float32)
    got_t, got_r = rt.embedding_scatter_sgd(table, res, tokens, g, vocab, d, 0.1)
    keep = tokens < vocab
    gk = g.reshape(-1, d)[keep].ravel()
    want_t, want_r = o.embedding_scatter_sgd(table, res, d, tokens[keep], gk, 0.1)
    np.testing.assert_array_equal(got_t, want_t)
    np.testing.assert_array_equal(got_r.view(np.uint32), want_r.view(np.uint32))


# ------------------------------------------------------ few-row forward (GEMV)
GEMV_REL = 1e-5  # same fp16-rounded inputs, fp32 sums in another order


@pytest.mark.parametrize("rows", [1, 3, 8])
@pytest.mark.parametrize("in_f,out_f,bias", [(512, 2048, True), (1024, 32768, True),
                                             (96, 1000, False), (4096, 64, True),
                                             (128, 300, True), (256, 64, False),
                                             (384, 640, True), (640, 96, True)])
def test_packed_few_rows_matches_oracle(rt, rows, in_f, out_f, bias):
    # T = 1 decode shapes (batch <= 8): the few-row path of binary_linear
    rng = np.random.default_rng(rows * 7 + in_f + out_f)
    x16, bits, scale, b = rand_case(rng, rows, in_f, out_f, bias)
    want = o.packed_forward(h2f32(x16), rows, in_f, out_f, bits, scale, b)
    got = rt.binary_linear(x16, bits, scale, b, rows, in_f, out_f)
    assert rel(got, want) <= GEMV_REL
    got32 = rt.binary_linear(h2f32(x16), bits, scale, b, rows, in_f, out_f, x_dtype=2)
    assert rel(got32, want) <= GEMV_REL
    y16 = rt.binary_linear(x16, bits, scale, b, rows, in_f, out_f, out_dtype=np.float16)
    np.testing.assert_array_equal(y16, f16(got))


@pytest.mark.parametrize("rows", [1, 5, 8])
@pytest.mark.parametrize("in_f,out_f", [(4096, 1024), (2048, 512), (40, 17)])
def test_fp16_few_rows_matches_oracle(rt, rows, in_f, out_f):
    rng = np.random.default_rng(rows + in_f + out_f)
    x16 = f16(rng.standard_normal(rows * in_f))
    w = f16(rng.normal(0, 0.05, out_f * in_f))
    want = o.fp16_forward(h2f32(x16), rows, in_f, out_f, w)
    assert rel(rt.fp16_linear(x16, w, rows, in_f, out_f), want) <= GEMV_REL


# ------------------------------------------ tile configurations of large products
@pytest.mark.parametrize("rows,in_f,out_f,chunk", [
    (8192, 512, 8192, 1024),   # 1024 256x256 tiles: LdsGiant, sign bits expanded in LDS
    (8320, 512, 8192, 1040),   # 2080 128x256 tiles (rows not a multiple of 256): LdsHuge
    (4096, 512, 2048, 1024),   # 512 128x128 tiles: LdsBig
])
def test_large_products_match_small_tile_path(rt, rows, in_f, out_f, chunk):
    """A large product takes bigger tiles; every output element is still the
    same MFMA sequence over K, so the result equals the one computed in row
    chunks small enough for 64x64 tiles, bit for bit; and a row sample
    matches the oracle."""
    rng = np.random.default_rng(rows + out_f)
    x16, bits, scale, b = rand_case(rng, rows, in_f, out_f)
    whole = rt.binary_linear(x16, bits, scale, b, rows, in_f, out_f)
    parts = np.concatenate([
        rt.binary_linear(x16[r0 * in_f:(r0 + chunk) * in_f], bits, scale, b, chunk, in_f, out_f)
        for r0 in range(0, rows, chunk)])
    np.testing.assert_array_equal(whole.view(np.uint32), parts.view(np.uint32))
    sample = np.r_[0:16, rows - 16:rows]
    xs = h2f32(x16).reshape(rows, in_f)[sample]
    want = o.packed_forward(xs.ravel(), len(sample), in_f, out_f, bits, scale, b)
    assert rel(whole.reshape(rows, out_f)[sample].ravel(), want) <= REL


def test_large_backward_matches_small_tile_path(rt):
    # dX of 8192 x 1024 from K 4096 takes 128x128 tiles; in 1024-row chunks 64x64
    rows, in_f, out_f, chunk = 8192, 1024, 4096, 1024
    rng = np.random.default_rng(77)
    x16, bits, scale, _ = rand_case(rng, rows, in_f, out_f, bias=False)
    gy = (rng.standard_normal(rows * out_f) * 1e-2).astype(np.float32)
    whole = rt.binary_linear_backward(x16, gy, bits, scale, False, rows, in_f, out_f)
    gx = np.concatenate([
        rt.binary_linear_backward(x16[r0 * in_f:(r0 + chunk) * in_f],
                                  gy[r0 * out_f:(r0 + chunk) * out_f], bits, scale, False, chunk,
                                  in_f, out_f)["input_gradient"]
        for r0 in range(0, rows, chunk)])
    # the chunks scale their fp16 gradient operand by their own max |gy|
    assert rel(whole["input_gradient"], gx) <= 1e-5


def test_large_fp16_product_matches_small_tile_path(rt):
    # 16384 x 4096 from K 512: 1024 256x256 tiles; 1024-row chunks take the
    # 64x64 four-stage ring; the K order of the MFMAs is the same in both
    rows, in_f, out_f, chunk = 16384, 512, 4096, 1024
    rng = np.random.default_rng(91)
    x16 = f16(rng.standard_normal(rows * in_f))
    w = f16(rng.normal(0, 0.05, out_f * in_f))
    whole = rt.fp16_linear(x16, w, rows, in_f, out_f)
    parts = np.concatenate([rt.fp16_linear(x16[r0 * in_f:(r0 + chunk) * in_f], w, chunk, in_f, out_f)
                            for r0 in range(0, rows, chunk)])
    np.testing.assert_array_equal(whole.view(np.uint32), parts.view(np.uint32))
    sample = np.r_[0:8, rows - 8:rows]
    want = o.fp16_forward(h2f32(x16).reshape(rows, in_f)[sample].ravel(), len(sample), in_f, out_f, w)
    assert rel(whole.reshape(rows, out_f)[sample].ravel(), want) <= REL
