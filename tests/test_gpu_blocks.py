"""GPU parity of the block-level methods (ullis_hip_cmix_block_*,
ullis_hip_rosa_*), through HipRuntime's MetalRuntime-shaped mirror, against
the oracle's CPU composition of the same block (the non-Metal branches of
src/model.rs:1018-1177 and 1354-1523), and of the block-by-block Heron step
(HeronBlockStep) against the fused device step (ullis_hip_heron_step),
which it must match bit for bit.

Bounds: a block chains GEMMs through fp16 operands where the oracle keeps
fp32 (the mixed input, ReLU^2, the scaled gradient), so composed outputs and
gradients are compared as max|gpu - ref| / max|ref| <= BLOCK_REL; updates are
compared as the change of the effective parameter (f16 value + fp32 carry),
which is -lr * clip(g), <= UPDATE_REL; sign bits as mismatch fractions (an
output or latent within rounding of zero may land on either side). Each case
writes its measured drift to block_drift/<case>.json under RESULTS; the maxima
over the cases were 9.1e-4 (the key scale gradient), 7.6e-4 (the key latent
step) and 5.8e-4 for everything else, and no updated weight sign bit
differed. The bounds are those maxima with a margin under 2x.
"""
import pathlib

import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.heron_blocks import HeronBlockStep
from ullis_amd.runtime import HeronShape, HeronTrainer
from ullis_amd.synth import f16, heron_arena, pack_bits, step_inputs, tensor_view, unpack_bits

# results folder of a GPU run (the one a remote run's outputs come back from)
RESULTS = pathlib.Path(__file__).resolve().parent.parent / "gpurun_out"

pytestmark = pytest.mark.gpu

NO_IGNORE = 0xFFFFFFFF
BLOCK_REL = 1.5e-3
UPDATE_REL = 1.5e-3
BITS_FRAC = 2e-3  # Q/K/V projection sign bit-planes


def h2f(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    assert a.shape == r.shape and np.isfinite(a).all()
    return float(np.max(np.abs(a - r))) / max(float(np.max(np.abs(r))), 1e-30)


def record_drift(case: str, drift: dict) -> None:
    """Writes one case's measured drift to RESULTS/block_drift/<case>.json
    (the figures the bounds above rest on)."""
    import json

    out = RESULTS / "block_drift"
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{case}.json").write_text(json.dumps(drift, indent=1, sort_keys=True))


def bit_frac(a, b, n):
    return float(np.mean(unpack_bits(a, n) != unpack_bits(b, n)))


def effective(values16, residual):
    return h2f(values16).astype(np.float64) + np.asarray(residual, np.float64)


def cm_to_rm(idx_cm, batch, time, ch):
    return np.ascontiguousarray(
        np.asarray(idx_cm, np.uint8).reshape(batch, ch, time).transpose(0, 2, 1)).reshape(-1)


def mixed(x, mix16, batch, time, ch):
    xx = o.time_shift_delta(x, batch, time, ch)
    return (x.reshape(-1, ch) + xx.reshape(-1, ch) * h2f(mix16)[None, :]).reshape(-1)


def cmix_case(rng, batch, time, d, f):
    rows = batch * time
    return dict(
        x16=f16(rng.standard_normal(rows * d)),
        mix=f16(rng.uniform(0.0, 1.0, d)),
        key_latent=f16(rng.uniform(-0.01, 0.01, f * d)),
        key_residual=rng.uniform(-1e-4, 1e-4, f * d).astype(np.float32),
        key_scale=f16(rng.uniform(0.02, 0.06, f)),
        value=f16(rng.normal(0, 0.05, d * f)),
        value_residual=rng.uniform(-1e-4, 1e-4, d * f).astype(np.float32),
        gy=(rng.standard_normal(rows * d) * 1e-3).astype(np.float32),
    )


@pytest.mark.parametrize("batch,time,d,f", [(1, 64, 64, 128), (2, 32, 64, 192), (1, 256, 128, 512),
                                            (2, 4, 64, 256)])  # 8 rows: the few-row forward
def test_cmix_block_forward_backward_match_oracle(rt, batch, time, d, f):
    rng = np.random.default_rng(11 + d + f)
    c = cmix_case(rng, batch, time, d, f)
    rows = batch * time
    key_bits = o.pack_latent_bits(c["key_latent"])
    fwd = rt.cmix_block_forward(c["x16"], c["mix"], key_bits, c["key_scale"], c["value"], batch,
                                time, d, f)
    # oracle: CMix forward_tape CPU branch (src/model.rs:1051-1061)
    x = h2f(c["x16"])
    shifted = mixed(x, c["mix"], batch, time, d)
    key = o.packed_forward(shifted, rows, d, f, key_bits, c["key_scale"])
    relu2 = np.maximum(key, 0.0) ** 2
    out = o.fp16_forward(relu2, rows, f, d, c["value"])
    assert rel(fwd["out"], out) <= BLOCK_REL

    lr, ste = 0.01, float(time - 1)
    bwd = rt.cmix_block_backward_sgd(fwd["gpu_tape"], c["gy"], c["mix"], key_bits, c["key_scale"],
                                     c["key_latent"], c["key_residual"], c["value"],
                                     c["value_residual"], batch, time, d, f, lr, ste)
    # oracle: CMix backward_update CPU branch (src/model.rs:1145-1177)
    g_relu2, g_value = o.fp16_backward(relu2, c["gy"], rows, f, d, c["value"])
    v_new, v_res = o.clipped_sgd(c["value"], c["value_residual"], g_value, lr)
    g_key = g_relu2 * 2.0 * np.maximum(key, 0.0)
    pb = o.packed_backward_ste(shifted, g_key, rows, d, f, key_bits, c["key_scale"], want_gb=False)
    lat, lat_res, _, _, _, _, bits_new = o.packed_apply_sgd(
        d, f, c["key_latent"], c["key_residual"], c["key_scale"], np.zeros(f, np.float32), None,
        None, pb["weight_gradient"], pb["scale_gradient"], None, lr, ste)
    g_x, g_mix = o.lerp_shift_backward(o.time_shift_delta(x, batch, time, d), c["mix"],
                                       pb["input_gradient"], batch, time, d)
    v0 = effective(c["value"], c["value_residual"])
    k0 = effective(c["key_latent"], c["key_residual"])
    drift = {
        "out": rel(fwd["out"], out),
        "g_x": rel(bwd["g_x"], g_x),
        "g_mix": rel(bwd["g_mix"], g_mix),
        "g_key_scale": rel(bwd["g_key_scale"], pb["scale_gradient"]),
        "value_step": rel(effective(bwd["next_value_weight"], bwd["next_value_residual"]) - v0,
                          effective(v_new, v_res) - v0),
        "key_step": rel(effective(bwd["next_key_latent"], bwd["next_key_residual"]) - k0,
                        effective(lat, lat_res) - k0),
        "key_bits_frac": bit_frac(bwd["next_key_bits"], bits_new, f * d),
    }
    record_drift(f"cmix_b{batch}t{time}d{d}f{f}", drift)
    assert drift["g_x"] <= BLOCK_REL
    assert drift["g_mix"] <= BLOCK_REL
    assert drift["g_key_scale"] <= BLOCK_REL
    assert drift["value_step"] <= UPDATE_REL
    assert drift["key_step"] <= UPDATE_REL
    # bits are the repack of the updated latent; bits_t their transpose
    np.testing.assert_array_equal(bwd["next_key_bits"], o.pack_latent_bits(bwd["next_key_latent"]))
    np.testing.assert_array_equal(bwd["next_key_bits_t"],
                                  o.transpose_bits(bwd["next_key_bits"], f, d))
    assert bit_frac(bwd["next_key_bits"], bits_new, f * d) <= BITS_FRAC


def test_cmix_block_backward_nonfinite_gradient_matches_oracle(rt):
    """A NaN and an Inf in the upstream gradient of a CMix block
    (src/model.rs:1145-1177): every gradient is NaN / Inf / finite where the
    oracle's is; the value weight's clipped SGD takes +-Inf as a +-1 step and
    NaN into the canonical quiet NaN (src/precision.rs:29-31, 106-113), bit
    for bit with the oracle on those elements; the key latent's BinaryConnect
    step leaves every weight with a non-finite gradient exactly as it was
    (src/precision.rs:125-127). The key scale gradient of an Inf row is
    non-finite on both sides (the reference's sum order gives +-Inf, the
    identity sum_i sign G gives NaN here)."""
    batch, time, d, f = 1, 64, 64, 128
    rows = batch * time
    lr, ste = 0.01, float(time - 1)
    # a seed whose keys in the two injected rows are clear of zero, so the
    # ReLU^2 zero pattern (Inf * 0 = NaN) is the same on both sides
    for seed in range(100, 200):
        rng = np.random.default_rng(seed)
        c = cmix_case(rng, batch, time, d, f)
        key_bits = o.pack_latent_bits(c["key_latent"])
        x = h2f(c["x16"])
        shifted = mixed(x, c["mix"], batch, time, d)
        key = o.packed_forward(shifted, rows, d, f, key_bits, c["key_scale"]).reshape(rows, f)
        w_row = c["value"].reshape(d, f)[20]  # the Inf's column meets this weight row
        if np.abs(key[[9, 40]]).min() > 5e-3 and ((w_row & 0x7FFF) != 0).all():
            break
    c["gy"][9 * d + 3] = np.nan
    c["gy"][40 * d + 20] = np.inf
    fwd = rt.cmix_block_forward(c["x16"], c["mix"], key_bits, c["key_scale"], c["value"], batch,
                                time, d, f)
    bwd = rt.cmix_block_backward_sgd(fwd["gpu_tape"], c["gy"], c["mix"], key_bits, c["key_scale"],
                                     c["key_latent"], c["key_residual"], c["value"],
                                     c["value_residual"], batch, time, d, f, lr, ste)
    relu2 = np.maximum(key.ravel(), 0.0) ** 2
    g_relu2, g_value = o.fp16_backward(relu2, c["gy"], rows, f, d, c["value"])
    v_new, v_res = o.clipped_sgd(c["value"], c["value_residual"], g_value, lr)
    g_key = np.where(key.ravel() > 0, g_relu2 * 2.0 * key.ravel(), 0.0).astype(np.float32)
    pb = o.packed_backward_ste(shifted, g_key, rows, d, f, key_bits, c["key_scale"], want_gb=False)
    lat, lat_res, _, _, _, _, _ = o.packed_apply_sgd(
        d, f, c["key_latent"], c["key_residual"], c["key_scale"], np.zeros(f, np.float32), None,
        None, pb["weight_gradient"], pb["scale_gradient"], None, lr, ste)
    g_x, g_mix = o.lerp_shift_backward(o.time_shift_delta(x, batch, time, d), c["mix"],
                                       pb["input_gradient"], batch, time, d)

    def masks_and_finite(a, r, name, tol=BLOCK_REL):
        a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
        for m in (np.isnan, np.isposinf, np.isneginf):
            np.testing.assert_array_equal(m(a), m(r), err_msg=f"{name} {m.__name__}")
        fin = np.isfinite(r)
        if fin.any():  # g_mix sums over every row: all of it is NaN here
            assert rel(a[fin], r[fin]) <= tol, name

    masks_and_finite(bwd["g_x"], g_x, "g_x")
    masks_and_finite(bwd["g_mix"], g_mix, "g_mix")
    np.testing.assert_array_equal(np.isfinite(bwd["g_key_scale"]),
                                  np.isfinite(pb["scale_gradient"]))
    assert not np.isfinite(bwd["g_key_scale"]).all()
    # value weight: non-finite gradients give the oracle's bits exactly
    gv = np.asarray(g_value)
    nan, inf = np.isnan(gv), np.isinf(gv)
    assert nan.any() and inf.any()
    nv = bwd["next_value_weight"]
    np.testing.assert_array_equal(nv[inf], v_new[inf])
    np.testing.assert_array_equal(bwd["next_value_residual"][inf].view(np.uint32),
                                  v_res[inf].view(np.uint32))
    assert ((nv[nan] & 0x7FFF) == 0x7E00).all() and np.isnan(bwd["next_value_residual"][nan]).all()
    fin = np.isfinite(gv)
    v0 = effective(c["value"], c["value_residual"])[fin]
    assert rel(effective(nv, bwd["next_value_residual"])[fin] - v0,
               effective(v_new, v_res)[fin] - v0) <= UPDATE_REL
    # key latent: weights with a non-finite gradient keep latent and carry
    gk = np.asarray(pb["weight_gradient"])
    skip = ~np.isfinite(gk)
    assert skip.any()
    np.testing.assert_array_equal(bwd["next_key_latent"][skip], c["key_latent"][skip])
    np.testing.assert_array_equal(bwd["next_key_residual"][skip].view(np.uint32),
                                  c["key_residual"][skip].view(np.uint32))
    np.testing.assert_array_equal(lat[skip], c["key_latent"][skip])
    k0 = effective(c["key_latent"], c["key_residual"])[~skip]
    assert rel(effective(bwd["next_key_latent"], bwd["next_key_residual"])[~skip] - k0,
               effective(lat, lat_res)[~skip] - k0) <= UPDATE_REL


def rosa_case(rng, batch, time, d):
    rows = batch * time

    def proj():
        return dict(bits=pack_bits(rng.uniform(-1, 1, d * d) >= 0),
                    scale=f16(rng.uniform(0.02, 0.06, d)), bias=f16(rng.normal(0, 0.01, d)))
    return dict(
        x16=f16(rng.standard_normal(rows * d)),
        mix=[f16(rng.uniform(0.0, 1.0, d)) for _ in range(3)],
        q=proj(), k=proj(), v=proj(), o=proj(),
        e=f16(rng.normal(0, 0.5, d)),
        idx=rng.integers(0, 2, rows * d, dtype=np.uint8),  # channel-major [B][D][T]
        latent=f16(rng.uniform(-0.01, 0.01, d * d)),
        residual=rng.uniform(-1e-4, 1e-4, d * d).astype(np.float32),
        gy=(rng.standard_normal(rows * d) * 1e-3).astype(np.float32),
    )


@pytest.mark.parametrize("batch,time,d", [(1, 64, 64), (2, 64, 96), (1, 128, 128), (1, 8, 64)])
def test_rosa_block_forward_and_o_stop_grad_match_oracle(rt, batch, time, d):
    rng = np.random.default_rng(5 + d + time)
    c = rosa_case(rng, batch, time, d)
    rows = batch * time
    seen = []

    def sam(qp, kp, vp):  # the suffix automaton's seat: hand back the fixed idx
        seen.append((qp, kp, vp))
        return c["idx"]

    q, k, v, op = c["q"], c["k"], c["v"], c["o"]
    fwd = rt.rosa_block_forward(c["x16"], *c["mix"], q["bits"], q["scale"], q["bias"], k["bits"],
                                k["scale"], k["bias"], v["bits"], v["scale"], v["bias"], c["e"],
                                op["bits"], op["scale"], op["bias"], batch, time, d, sam)
    assert len(seen) == 1
    # oracle: forward_tape CPU branch (src/model.rs:1412-1425) up to the planes
    x = h2f(c["x16"])
    words = (rows * d + 31) // 32
    for j, (p, m) in enumerate(zip((q, k, v), c["mix"])):
        y = o.packed_forward(mixed(x, m, batch, time, d), rows, d, d, p["bits"], p["scale"],
                             p["bias"])
        want = o.sign_pack_bits(y)
        assert fwd["planes"][j].shape == (words,)
        assert bit_frac(fwd["planes"][j], want, rows * d) <= BITS_FRAC, j
    idx_rm = cm_to_rm(c["idx"], batch, time, d)
    yv = o.rosa_y_from_idx(idx_rm, c["e"], rows, d)
    out = o.packed_forward(yv, rows, d, d, op["bits"], op["scale"], op["bias"])
    assert rel(fwd["out"], out) <= 1e-4  # y = +-e is exact in fp16

    lr, ste = 0.01, float(time - 1)
    bwd = rt.rosa_o_stop_grad_sgd(fwd["gpu_tape"], c["gy"], op["bits"], op["scale"], c["latent"],
                                  c["residual"], rows, d, lr, ste)
    # oracle: backward_stop_grad CPU branch (src/model.rs:1491-1522)
    pb = o.packed_backward_ste(yv, c["gy"], rows, d, d, op["bits"], op["scale"])
    g_e = o.rosa_e_grad(pb["input_gradient"], idx_rm, rows, d)
    lat, lat_res, _, _, _, _, bits_new = o.packed_apply_sgd(
        d, d, c["latent"], c["residual"], op["scale"], np.zeros(d, np.float32), None, None,
        pb["weight_gradient"], pb["scale_gradient"], None, lr, ste)
    l0 = effective(c["latent"], c["residual"])
    drift = {
        "out": rel(fwd["out"], out),
        "e_gradient": rel(bwd["e_gradient"], g_e),
        "scale_gradient": rel(bwd["scale_gradient"], pb["scale_gradient"]),
        "bias_gradient": rel(bwd["bias_gradient"], pb["bias_gradient"]),
        "o_step": rel(effective(bwd["next_latent"], bwd["next_residual"]) - l0,
                      effective(lat, lat_res) - l0),
        "o_bits_frac": bit_frac(bwd["next_bits"], bits_new, d * d),
    }
    record_drift(f"rosa_b{batch}t{time}d{d}", drift)
    assert drift["e_gradient"] <= BLOCK_REL
    assert drift["scale_gradient"] <= BLOCK_REL
    assert drift["bias_gradient"] <= 1e-5  # fp32 column sums
    assert drift["o_step"] <= UPDATE_REL
    np.testing.assert_array_equal(bwd["next_bits"], o.pack_latent_bits(bwd["next_latent"]))
    np.testing.assert_array_equal(bwd["next_bits_t"], o.transpose_bits(bwd["next_bits"], d, d))
    assert bit_frac(bwd["next_bits"], bits_new, d * d) <= BITS_FRAC


def test_block_methods_reject_bad_arguments(rt):
    lib = rt.lib
    d, f, b, t = 64, 128, 1, 64
    tape = rt.buffer(lib.ullis_hip_cmix_tape_bytes(b * t, d, f) + 256)
    x = rt.buffer(4 * b * t * d)
    small = rt.buffer(4096)
    args = [small.ptr] * 4
    # zero-sized shape, NULL tape, misaligned tape
    assert lib.ullis_hip_cmix_block_forward(rt.ctx, x.ptr, 2, *args, 0, t, d, f, x.ptr,
                                            tape.ptr) == -1
    assert lib.ullis_hip_cmix_block_forward(rt.ctx, x.ptr, 2, *args, b, t, d, f, x.ptr,
                                            None) == -1
    assert lib.ullis_hip_cmix_block_forward(rt.ctx, x.ptr, 2, *args, b, t, d, f, x.ptr,
                                            tape.ptr + 16) == -1
    assert b"aligned" in lib.ullis_hip_last_error(rt.ctx)
    assert lib.ullis_hip_cmix_block_forward(rt.ctx, x.ptr, 7, *args, b, t, d, f, x.ptr,
                                            tape.ptr) == -1
    assert lib.ullis_hip_rosa_o_stop_grad_sgd(rt.ctx, tape.ptr, x.ptr, small.ptr, None, small.ptr,
                                              small.ptr, small.ptr, t, d, -1.0, 1.0, small.ptr,
                                              small.ptr, small.ptr) == -1
    assert lib.ullis_hip_cmix_tape_bytes(0, d, f) == 0
    assert lib.ullis_hip_rosa_tape_bytes(t, 0) == 0


@pytest.mark.parametrize("d,layers,f,vocab,time,batch",
                         [(64, 2, 128, 256, 64, 1), (128, 3, 256, 512, 128, 1),
                          (512, 2, 2048, 8192, 2048, 1), (512, 1, 4096, 512, 8192, 1),
                          (64, 1, 128, 256, 4099, 3)])
def test_block_step_matches_fused_step(rt, d, layers, f, vocab, time, batch):
    """HeronBlockStep (block methods, host residual adds, the automaton
    handed the Q/K/V planes between the projections and O) against the fused
    step on the same arena and inputs: bit-identical, since both run the same
    kernels with the same reductions and the same update arithmetic (the
    third case has config 4's widths at two layers). In the last case the
    fused step's value input gradient reads its value^T cache (both operands
    k-contiguous) and the block path the value weight itself (a transposed
    operand): every output still sums the same products in the same order.
    The last case has three sequences of an odd length."""
    shape = HeronShape(d_model=d, n_layers=layers, dim_ffn=f, vocab=vocab, batch=batch, time=time)
    fused = HeronTrainer(rt, shape)
    blocks = HeronBlockStep(rt, shape)
    arena = heron_arena(fused.layout, fused.arena_bytes, shape.dims(), seed=3, random_ln=True)
    x, labels, idx = step_inputs(shape.rows, d, vocab, layers, batch, time, seed=3)
    nd = shape.rows * d
    words = (nd + 31) // 32

    fused.upload_arena(arena)
    dx, dl, di = rt.put(x), rt.put(labels), rt.put(idx)
    g = rt.zeros(np.float32, nd)
    rl = rt.zeros(np.float32, shape.rows)
    st = rt.zeros(np.float32, 4)
    qkv = rt.zeros(np.uint32, layers * 3 * words)
    fused.step(dx, dl, NO_IGNORE, 0.01, di, g, rl, st, qkv)
    rt.sync()
    fa, fg, frl = fused.download_arena(), g.download(np.float32), rl.download(np.float32)
    fst, fq = st.download(np.float32), qkv.download(np.uint32).reshape(layers, 3, words)

    blocks.upload_arena(arena)
    handed = []

    def sam(layer, qp, kp, vp):
        handed.append(layer)
        return idx[layer * nd:(layer + 1) * nd]

    out = blocks.step(x, labels, NO_IGNORE, 0.01, sam)
    ba = blocks.download_arena()
    assert handed == list(range(layers))
    for l in range(layers):
        for j in range(3):
            np.testing.assert_array_equal(out["qkv_planes"][l][j], fq[l, j], err_msg=f"{l}/{j}")
    np.testing.assert_array_equal(out["stats"][:3], fst[:3])
    np.testing.assert_array_equal(out["row_loss"].view(np.uint32), frl.view(np.uint32))
    np.testing.assert_array_equal(out["g_emb"].view(np.uint32), fg.view(np.uint32))
    for name, _dt, _count, _off, _derived in fused.layout:
        np.testing.assert_array_equal(tensor_view(ba, fused.layout, name),
                                      tensor_view(fa, fused.layout, name), err_msg=name)
    blocks.close()
    fused.close()


def stand_in_sam(batch, time, d):
    """A deterministic stand-in for the suffix automaton: its indices are a
    function of the sign bit-planes it is handed, as the automaton's are
    (rosa_qkv_batch_packed_channel_major, src/rosa.rs:486-513):
    idx[b, c, t] = q[t] xor k[t - 1] xor v[t - 2] of channel c (zero before
    the sequence's start), returned channel-major [batch][d][time]."""
    n = batch * time * d

    def sam(qp, kp, vp):
        q, k, v = (unpack_bits(p, n).reshape(batch, time, d).astype(np.uint8) for p in (qp, kp, vp))
        idx = q.copy()
        idx[:, 1:, :] ^= k[:, :-1, :]
        idx[:, 2:, :] ^= v[:, :-2, :]
        return np.ascontiguousarray(idx.transpose(0, 2, 1)).ravel()

    return sam


@pytest.mark.parametrize("d,layers,f,vocab,batch,time", [(64, 2, 128, 256, 2, 64),
                                                         (512, 2, 2048, 8192, 1, 512)])
def test_live_automaton_step_matches_block_path(rt, d, layers, f, vocab, batch, time):
    """ullis_hip_heron_step_sam (the fused step handing each layer's Q/K/V sign
    bit-planes to the caller's automaton and taking its indices back,
    src/metal.rs:1411-1511) against the block path (HeronBlockStep) driving the
    same stand-in automaton on its own planes: bit-identical arena, row losses,
    statistics and embedding gradient, and the automaton sees the same planes
    on both paths."""
    shape = HeronShape(d_model=d, n_layers=layers, dim_ffn=f, vocab=vocab, batch=batch, time=time)
    fused = HeronTrainer(rt, shape)
    blocks = HeronBlockStep(rt, shape)
    arena = heron_arena(fused.layout, fused.arena_bytes, shape.dims(), seed=6, random_ln=True)
    x, labels, _ = step_inputs(shape.rows, d, vocab, layers, batch, time, seed=6)
    nd = shape.rows * d
    words = (nd + 31) // 32
    automaton = stand_in_sam(batch, time, d)

    fused.upload_arena(arena)
    seen_fused = []

    def sam_fused(layer, planes):
        seen_fused.append((layer, planes.copy()))
        return automaton(planes[0], planes[1], planes[2])

    dx, dl = rt.put(x), rt.put(labels)
    g = rt.zeros(np.float32, nd)
    rl = rt.zeros(np.float32, shape.rows)
    st = rt.zeros(np.float32, 4)
    qkv = rt.zeros(np.uint32, layers * 3 * words)
    fused.step_sam(sam_fused, dx, dl, NO_IGNORE, 0.01, g, rl, st, qkv)
    rt.sync()
    fa, fg, frl = fused.download_arena(), g.download(np.float32), rl.download(np.float32)
    fst, fq = st.download(np.float32), qkv.download(np.uint32).reshape(layers, 3, words)

    blocks.upload_arena(arena)
    seen_blocks = []

    def sam_blocks(layer, qp, kp, vp):
        seen_blocks.append(layer)
        return automaton(qp, kp, vp)

    out = blocks.step(x, labels, NO_IGNORE, 0.01, sam_blocks)
    ba = blocks.download_arena()
    assert [l for l, _ in seen_fused] == seen_blocks == list(range(layers))
    for l, planes in seen_fused:
        for j in range(3):
            np.testing.assert_array_equal(planes[j], fq[l, j])
            np.testing.assert_array_equal(out["qkv_planes"][l][j], fq[l, j], err_msg=f"{l}/{j}")
    np.testing.assert_array_equal(out["stats"][:3], fst[:3])
    np.testing.assert_array_equal(out["row_loss"].view(np.uint32), frl.view(np.uint32))
    np.testing.assert_array_equal(out["g_emb"].view(np.uint32), fg.view(np.uint32))
    for name, _dt, _count, _off, _derived in fused.layout:
        np.testing.assert_array_equal(tensor_view(ba, fused.layout, name),
                                      tensor_view(fa, fused.layout, name), err_msg=name)
    blocks.close()
    fused.close()


def test_live_automaton_failure_aborts_before_any_update(rt):
    """An automaton that fails (non-zero from the callback, here at the second
    layer) ends the step with an error before any parameter changes."""
    shape = HeronShape(d_model=64, n_layers=3, dim_ffn=128, vocab=256, batch=1, time=32)
    tr = HeronTrainer(rt, shape)
    arena = heron_arena(tr.layout, tr.arena_bytes, shape.dims(), seed=8)
    x, labels, _ = step_inputs(shape.rows, 64, 256, 3, 1, 32, seed=8)
    tr.upload_arena(arena)
    before = tr.download_arena()
    automaton = stand_in_sam(1, 32, 64)

    def sam(layer, planes):
        if layer == 1:
            raise RuntimeError("automaton failed")
        return automaton(planes[0], planes[1], planes[2])

    g = rt.zeros(np.float32, shape.rows * 64)
    with pytest.raises(RuntimeError, match="automaton failed"):
        tr.step_sam(sam, rt.put(x), rt.put(labels), NO_IGNORE, 0.01, g)
    rt.sync()
    np.testing.assert_array_equal(tr.download_arena(), before)
    tr.close()
