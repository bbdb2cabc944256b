"""Pins the oracle's whole train step (ucr_heron_train_step) against an
independent float64 numpy re-derivation of UllisHeron::train_step_on
(src/model.rs:2827-3025, rosa_grad = stop_grad_bits) at tiny sizes.

The re-derivation below is written from the reference's Rust, not from
oracle/cpu_ref.c:
  forward      per block ln0 (block 0), ln3, time-shift mix, Q/K/V, y = (2 idx - 1) e,
               O + residual, ln2, CMix (mix, key, ReLU^2, value) + residual
               (src/model.rs:2874-2912, 1354-1440, 1018-1078), ln_out
  head         causal CE with the 1/(T-1) gradient scale (src/model.rs:27-55,
               3132-3274); latent/scale update via flip_after_gradients, then the
               bias at 8 x lr (src/model.rs:3118-3130)
  backward     ln_out bwd + step; per block in reverse: CMix backward_update (value dX
               with the pre-update value weight, value step, key STE with the
               pre-update bits, key latent/scale step, lerp_shift_backward, x_k step;
               src/model.rs:1080-1178, 1207-1240), ln2 bwd (+= into g_x), ROSA O
               stop-grad (O latent/scale/bias step, e step; src/model.rs:1442-1523),
               ln0 bwd at block 0 (src/model.rs:2940-2983)
Arithmetic is float64; parameters are rounded to f16 by numpy on update. The
oracle runs in float32, so FP16 parameters are compared as value + carry
(the update's `desired`, which is continuous in the gradient), within float32
rounding of the gradients.
"""
import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.synth import heron_arena, pack_bits, step_inputs, tensor_view, unpack_bits

NO_IGNORE = 0xFFFFFFFF


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


class Param:
    """FP16 storage + f32 carry (Fp16Storage, src/precision.rs:80-134) in float64."""

    def __init__(self, arena, layout, name):
        self.v = f16(tensor_view(arena, layout, name))
        self.r = tensor_view(arena, layout, name + ".residual").astype(np.float64)

    def clipped(self, g, lr):  # apply_clipped_sgd, src/precision.rs:106-113
        d = (self.v - lr * np.clip(g, -1.0, 1.0)) + self.r
        self.v = d.astype(np.float16).astype(np.float64)
        self.r = d - self.v

    def binaryconnect(self, g, lr):  # apply_binaryconnect_sgd, src/precision.rs:124-134
        live = np.isfinite(g) & (g != 0.0)
        d = np.clip((self.v - lr * np.clip(g, -1.0, 1.0)) + self.r, -1.0, 1.0)
        v = d.astype(np.float16).astype(np.float64)
        self.v = np.where(live, v, self.v)
        self.r = np.where(live, d - v, self.r)

    def desired(self):
        return self.v + self.r


class Packed:
    def __init__(self, arena, layout, p, out, inp, bias):
        self.out, self.inp = out, inp
        self.latent = Param(arena, layout, p + ".latent")
        self.scale = Param(arena, layout, p + ".scale")
        self.bias = Param(arena, layout, p + ".bias") if bias else None
        bits = tensor_view(arena, layout, p + ".bits")
        self.sign = np.where(unpack_bits(bits, out * inp), 1.0, -1.0).reshape(out, inp)

    def forward(self, x):  # PackedBinaryLinear::forward, src/model.rs:724-742
        y = (x @ self.sign.T) * self.scale.v
        return y + self.bias.v if self.bias is not None else y

    def backward(self, x, gy):  # backward_ste, src/model.rs:745-796
        gys = gy * self.scale.v
        g_w = gys.T @ x
        g_x = gys @ self.sign
        g_scale = (gy * (x @ self.sign.T)).sum(0)
        return g_w, g_x, g_scale, gy.sum(0)

    def flip(self, g_w, g_scale, g_bias, lr, ste):  # apply_packed_sgd, src/model.rs:808-884
        self.latent.binaryconnect((g_w * ste).ravel(), lr)
        self.scale.clipped(g_scale, lr)
        if g_bias is not None:
            self.bias.clipped(g_bias, lr)
        self.sign = np.where(self.latent.v >= 0.0, 1.0, -1.0).reshape(self.out, self.inp)


class Ln:
    def __init__(self, arena, layout, p):
        self.w = Param(arena, layout, p + ".weight")
        self.b = Param(arena, layout, p + ".bias")

    def forward(self, x):  # src/model.rs:259-276
        mean = x.mean(1, keepdims=True)
        var = ((x - mean) ** 2).mean(1, keepdims=True)
        return (x - mean) / np.sqrt(var + 1e-5) * self.w.v + self.b.v

    def backward(self, x, gy):  # src/model.rs:278-316
        n = x.shape[1]
        mean = x.mean(1, keepdims=True)
        inv = 1.0 / np.sqrt(((x - mean) ** 2).mean(1, keepdims=True) + 1e-5)
        xhat = (x - mean) * inv
        dxhat = gy * self.w.v
        gx = inv / n * (n * dxhat - dxhat.sum(1, keepdims=True)
                        - xhat * (dxhat * xhat).sum(1, keepdims=True))
        return gx, (gy * xhat).sum(0), gy.sum(0)

    def step(self, gw, gb, lr):
        self.w.clipped(gw, lr)
        self.b.clipped(gb, lr)


def time_shift(x, batch, time):  # time_shift_delta, src/model.rs:186-212
    x3 = x.reshape(batch, time, -1)
    xx = -x3.copy()
    xx[:, 1:] += x3[:, :-1]
    return xx.reshape(x.shape)


def lerp_shift_backward(xx, mix, g_shifted, batch, time):  # src/model.rs:1207-1240
    g_mix = (g_shifted * xx).sum(0)
    g_x = g_shifted.copy()
    g_xx = (g_shifted * mix).reshape(batch, time, -1)
    g3 = g_x.reshape(batch, time, -1)
    g3[:, :-1] += g_xx[:, 1:]
    g3 -= g_xx
    return g_x, g_mix


def numpy_step(dims, arena, layout, x_emb, labels, ignore, batch, time, lr, idx):
    D, L, F, V = dims.d_model, dims.n_layers, dims.dim_ffn, dims.vocab
    R = batch * time
    ste = float(time - 1)
    ln_out = Ln(arena, layout, "ln_out")
    head = Packed(arena, layout, "head", V, D, True)
    blocks = []
    for l in range(L):
        p = f"blocks.{l}"
        blk = {
            "ln0": Ln(arena, layout, p + ".ln0") if l == 0 else None,
            "ln2": Ln(arena, layout, p + ".ln2"), "ln3": Ln(arena, layout, p + ".ln3"),
            "x_q": Param(arena, layout, p + ".rosa.x_q"), "x_k": Param(arena, layout, p + ".rosa.x_k"),
            "x_v": Param(arena, layout, p + ".rosa.x_v"), "e": Param(arena, layout, p + ".rosa.e"),
            "q": Packed(arena, layout, p + ".rosa.q", D, D, True),
            "k": Packed(arena, layout, p + ".rosa.k", D, D, True),
            "v": Packed(arena, layout, p + ".rosa.v", D, D, True),
            "o": Packed(arena, layout, p + ".rosa.o", D, D, True),
            "cx_k": Param(arena, layout, p + ".ffn.x_k"),
            "key": Packed(arena, layout, p + ".ffn.key", F, D, False),
            "value": Param(arena, layout, p + ".ffn.value"),
        }
        blocks.append(blk)
    # forward (src/model.rs:2874-2912)
    x = np.asarray(x_emb, np.float64).reshape(R, D)
    idx = np.asarray(idx, np.uint8).reshape(L, batch, D, time)
    tapes, qkv_bits = [], []
    for l, b in enumerate(blocks):
        tape = {}
        if b["ln0"] is not None:
            tape["ln0_in"] = x
            x = b["ln0"].forward(x)
        rin = b["ln3"].forward(x)
        xx = time_shift(rin, batch, time)
        acts = []
        for j, mix in (("q", "x_q"), ("k", "x_k"), ("v", "x_v")):
            a = b[j].forward(rin + xx * b[mix].v)
            acts.append(a)
            qkv_bits.append(pack_bits((a > 0.0).ravel()))  # bit_from_activation, src/rosa.rs:372-374
        sgn = 2.0 * idx[l].transpose(0, 2, 1).reshape(R, D).astype(np.float64) - 1.0
        y = sgn * b["e"].v  # rosa_qkv_out_batched_channel_major, src/rosa.rs:614-639
        x = x + b["o"].forward(y)
        tape.update(y=y, sgn=sgn, after_rosa=x)
        ln2 = b["ln2"].forward(x)
        xx2 = time_shift(ln2, batch, time)
        shifted = ln2 + xx2 * b["cx_k"].v
        key = b["key"].forward(shifted)
        relu2 = np.maximum(key, 0.0) ** 2
        W = b["value"].v.reshape(D, F)
        x = x + relu2 @ W.T
        tape.update(xx2=xx2, shifted=shifted, key=key, relu2=relu2)
        tapes.append(tape)
    pre_ln_out = x
    hidden = ln_out.forward(x)
    # head + CE (src/model.rs:3132-3274)
    lab = np.asarray(labels, np.int64)
    valid = np.array([(r % time) + 1 < time and lab[r + 1] != ignore for r in range(R)])
    n_valid = int(valid.sum())
    loss_scale = 1.0 / (time - 1) if n_valid else 0.0
    logits = head.forward(hidden)
    m = logits.max(1, keepdims=True)
    ex = np.exp(logits - m)
    se = ex.sum(1, keepdims=True)
    tgt = np.where(valid, np.roll(lab, -1), 0)
    row_loss = np.where(valid, (m + np.log(se))[:, 0] - logits[np.arange(R), tgt], 0.0)
    onehot = np.zeros_like(logits)
    onehot[np.arange(R), tgt] = 1.0
    gy = np.where(valid[:, None], loss_scale * (ex / se - onehot), 0.0)
    g_w, g_x, g_scale, g_bias = head.backward(hidden, gy)
    head.flip(g_w, g_scale, None, lr, ste)
    head.bias.clipped(g_bias, lr * 8.0)
    mean_loss = row_loss.sum() / n_valid if n_valid else 0.0
    gi, gw, gb = ln_out.backward(pre_ln_out, g_x)
    ln_out.step(gw, gb, lr)
    g_x = gi
    # backward (src/model.rs:2940-2983)
    for l in reversed(range(L)):
        b, t = blocks[l], tapes[l]
        W = b["value"].v.reshape(D, F)
        g_relu2 = g_x @ W
        b["value"].clipped((g_x.T @ t["relu2"]).ravel(), lr)
        g_key = np.where(t["key"] > 0.0, 2.0 * t["key"] * g_relu2, 0.0)
        kw, g_shifted, ks, _ = b["key"].backward(t["shifted"], g_key)
        b["key"].flip(kw, ks, None, lr, ste)
        g_ln2_out, g_mix = lerp_shift_backward(t["xx2"], b["cx_k"].v, g_shifted, batch, time)
        b["cx_k"].clipped(g_mix, lr)
        gi, gw, gb = b["ln2"].backward(t["after_rosa"], g_ln2_out)
        b["ln2"].step(gw, gb, lr)
        g_x = g_x + gi
        ow, g_y, os_, ob = b["o"].backward(t["y"], g_x)
        b["o"].flip(ow, os_, ob, lr, ste)
        b["e"].clipped((g_y * t["sgn"]).sum(0), lr)  # rosa_e_grad, src/model.rs:1608-1634
        if b["ln0"] is not None:
            gi, gw, gb = b["ln0"].backward(t["ln0_in"], g_x)
            b["ln0"].step(gw, gb, lr)
            g_x = gi
    params = {"ln_out.weight": ln_out.w, "ln_out.bias": ln_out.b, "head.latent": head.latent,
              "head.scale": head.scale, "head.bias": head.bias}
    for l, b in enumerate(blocks):
        p = f"blocks.{l}"
        if b["ln0"] is not None:
            params[p + ".ln0.weight"], params[p + ".ln0.bias"] = b["ln0"].w, b["ln0"].b
        params[p + ".ln2.weight"], params[p + ".ln2.bias"] = b["ln2"].w, b["ln2"].b
        params[p + ".ln3.weight"], params[p + ".ln3.bias"] = b["ln3"].w, b["ln3"].b
        for n in ("x_q", "x_k", "x_v", "e"):
            params[f"{p}.rosa.{n}"] = b[n]
        for n in ("q", "k", "v", "o"):
            params[f"{p}.rosa.{n}.latent"] = b[n].latent
            params[f"{p}.rosa.{n}.scale"] = b[n].scale
            params[f"{p}.rosa.{n}.bias"] = b[n].bias
        params[p + ".ffn.x_k"] = b["cx_k"]
        params[p + ".ffn.key.latent"] = b["key"].latent
        params[p + ".ffn.key.scale"] = b["key"].scale
        params[p + ".ffn.value"] = b["value"]
    return {"g_emb": g_x.ravel(), "row_loss": row_loss, "mean_loss": mean_loss,
            "n_valid": n_valid, "params": params, "qkv_bits": np.concatenate(qkv_bits),
            "packed": {"head": head, **{f"blocks.{l}.rosa.o": blocks[l]["o"] for l in range(L)},
                       **{f"blocks.{l}.ffn.key": blocks[l]["key"] for l in range(L)}}}


def boost(arena, layout, seed):
    """Row scales ~U(0.5, 1.5) and value weights ~N(0, 0.5): gradients through
    every branch are then large enough that a step at a large learning rate
    moves each f16 parameter by many ulps."""
    rng = np.random.default_rng(seed)
    for name, dt, count, off, derived in layout:
        if name.endswith(".scale"):
            tensor_view(arena, layout, name)[:] = f16_bits(rng.uniform(0.5, 1.5, count))
        elif name.endswith(".value"):
            tensor_view(arena, layout, name)[:] = f16_bits(rng.normal(0.0, 0.5, count))


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


# lr 0.01 on the synthetic heron distributions is the heron setting. The
# boosted case at lr 10 makes every FP16 update move the f16 values
# themselves, so using a post-update weight anywhere in the backward, or a
# wrong learning-rate multiplier, changes g_emb or the parameters.
@pytest.mark.parametrize("d,layers,ffn,vocab,batch,time,ignore,lr,boosted", [
    (8, 2, 16, 32, 2, 6, NO_IGNORE, 0.01, False),
    (16, 3, 32, 48, 1, 9, 5, 0.01, False),
    (8, 2, 16, 32, 2, 6, 7, 10.0, True),
])
def test_oracle_heron_step_matches_float64_rederivation(d, layers, ffn, vocab, batch, time, ignore,
                                                        lr, boosted):
    dims = o.HeronDims(d, layers, ffn, vocab)
    layout, total = o.heron_layout(dims)
    arena = heron_arena(layout, total, dims, seed=11, random_ln=True, mix_range=(0.2, 0.8))
    if boosted:
        boost(arena, layout, 11)
    rows = batch * time
    x, labels, idx = step_inputs(rows, d, vocab, layers, batch, time, seed=11)
    if ignore != NO_IGNORE:
        labels[::3] = ignore
    ref_arena = arena.copy()
    want = numpy_step(dims, ref_arena, layout, x, labels, ignore, batch, time, lr, idx)
    got = o.heron_train_step(dims, arena, x, labels, ignore, batch, time, lr, idx)

    assert got["n_valid"] == want["n_valid"]
    assert abs(got["mean_loss"] - want["mean_loss"]) <= 1e-5
    np.testing.assert_allclose(got["row_loss"], want["row_loss"], atol=1e-5)
    np.testing.assert_allclose(got["g_emb"], want["g_emb"], rtol=0,
                               atol=2e-5 * np.max(np.abs(want["g_emb"])))
    np.testing.assert_array_equal(got["qkv_bits"], want["qkv_bits"])
    for name, p in want["params"].items():
        v = f16(tensor_view(arena, layout, name))
        r = tensor_view(arena, layout, name + ".residual").astype(np.float64)
        # value + carry is the update's `desired`: float32 vs float64 gradients
        # differ by float32 rounding, scaled by lr (and by the STE for latents).
        tol = 2e-6 * max(1.0, lr * (time - 1) if name.endswith(".latent") else lr)
        np.testing.assert_allclose(v + r, p.desired(), rtol=1e-5, atol=tol, err_msg=name)
    for name, pk in want["packed"].items():
        bits = tensor_view(arena, layout, name + ".bits")
        np.testing.assert_array_equal(bits, pack_bits((pk.sign > 0).ravel()), err_msg=name)



def test_oracle_decode_matches_the_train_forward_row_by_row():
    """ucr_heron_decode_step (generate_step, src/model.rs:2717-2753) fed the
    tokens of a sequence one at a time, with the automaton's indices of each
    position, reproduces the train step's forward: the CE of its logits at
    position t against label t + 1 equals the train step's row loss (the
    reference's generate_step_logits_match_one_shot_hidden, src/model.rs:
    4991-5043, states the same equivalence), and the Q/K/V sign bits it
    produces are the train step's bit-planes. The train step's forward is
    pinned by the float64 re-derivation above."""
    d, layers, ffn, vocab, batch, time = 64, 2, 128, 256, 2, 12
    dims = o.HeronDims(d, layers, ffn, vocab)
    layout, total = o.heron_layout(dims)
    arena = heron_arena(layout, total, dims, seed=21, random_ln=True, mix_range=(0.2, 0.8))
    rng = np.random.default_rng(21)
    table = rng.standard_normal(vocab * d).astype(np.float16).view(np.uint16)
    tokens = rng.integers(0, vocab, batch * time).astype(np.uint32)
    labels = np.roll(tokens, -1).astype(np.uint32)
    _, _, idx = step_inputs(batch * time, d, vocab, layers, batch, time, seed=21)
    x = o.embedding_gather(table, d, tokens)
    train = o.heron_train_step(dims, arena.copy(), x, labels, NO_IGNORE, batch, time, 1e-3, idx)
    # idx [L][B][D][T] channel-major -> per token [L][B][D]
    idx4 = idx.reshape(layers, batch, d, time)
    planes = unpack_bits(train["qkv_bits"], layers * 3 * ((batch * time * d + 31) // 32) * 32)
    words = (batch * time * d + 31) // 32
    planes = planes.reshape(layers, 3, words * 32)[:, :, :batch * time * d].reshape(
        layers, 3, batch, time, d)
    rp = np.zeros(layers * batch * d, np.float32)
    cp = np.zeros(layers * batch * d, np.float32)
    tok = tokens.reshape(batch, time)
    for t in range(time):
        logits, qkv = o.heron_decode_step(dims, arena, table, tok[:, t],
                                          np.ascontiguousarray(idx4[:, :, :, t]), rp, cp, t > 0)
        np.testing.assert_array_equal(qkv, planes[:, :, :, t, :], err_msg=f"bits at t={t}")
        if t + 1 >= time:
            continue
        lg = logits.astype(np.float64)
        for b in range(batch):
            m = lg[b].max()
            # the train step scores row r against labels[r + 1] (horizon 1)
            ce = m + np.log(np.exp(lg[b] - m).sum()) - lg[b, labels[b * time + t + 1]]
            assert abs(ce - train["row_loss"][b * time + t]) <= 1e-5, (t, b)
