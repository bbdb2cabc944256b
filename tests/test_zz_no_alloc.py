"""ullis_hip_layer_norm_backward_static, the LayerNorm backward that allocates
nothing (its column partials live in a static device array), against the
allocating ullis_hip_layer_norm_backward on the same inputs, through the C
ABI: two calls in a row, the second on a smaller input, so the second reads
the array the first left behind."""
import numpy as np
import pytest

from ullis_amd.synth import f16

pytestmark = pytest.mark.gpu

REL = 1e-5  # the same per-row arithmetic; gw / gb sum the rows in other groups


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    assert a.shape == r.shape and np.isfinite(a).all()
    return float(np.max(np.abs(a - r))) / max(float(np.max(np.abs(r))), 1e-30)


def test_static_layer_norm_backward_matches_allocating_entry(rt):
    for rows, ch in ((4096, 1024), (300, 96)):
        rng = np.random.default_rng(rows + ch)
        x = (rng.standard_normal(rows * ch) * 2 + 0.3).astype(np.float32)
        gy = rng.normal(0, 1e-2, rows * ch).astype(np.float32)
        w = f16(rng.uniform(0.5, 1.5, ch))
        want = rt.layer_norm_backward(x, gy, w, rows, ch)
        dx, dg, dw = rt.put(x), rt.put(gy), rt.put(w)
        gx, gw, gb = rt.buffer(4 * rows * ch), rt.buffer(4 * ch), rt.buffer(4 * ch)
        rt.layer_norm_backward_static_dev(dx, dg, dw, rows, ch, gx, gw, gb)
        rt.sync()
        got = (gx.download(np.float32, rows * ch), gw.download(np.float32, ch),
               gb.download(np.float32, ch))
        for a, r, name in zip(got, want, ("gx", "gw", "gb")):
            assert rel(a, r) <= REL, (rows, ch, name, rel(a, r))


def test_static_layer_norm_backward_rejects_channels_beyond_its_scratch(rt):
    dx, dg, dw = rt.buffer(4 * 8 * 4100), rt.buffer(4 * 8 * 4100), rt.buffer(2 * 4100)
    gx = rt.buffer(4 * 8 * 4100)
    rc = rt.lib.ullis_hip_layer_norm_backward_static(rt.ctx, dx.ptr, dg.ptr, dw.ptr, 8, 4100,
                                                     gx.ptr, None, None)
    assert rc == -1
    assert b"static scratch limit" in rt.lib.ullis_hip_last_error(rt.ctx)
