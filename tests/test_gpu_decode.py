"""GPU T = 1 decode (ullis_hip_heron_decode_step) against the oracle's
generate_step (ucr_heron_decode_step, src/model.rs:2717-2753), which
test_oracle_heron.py pins to the train step's forward row by row.

Each case feeds a few tokens per sequence through both, carrying the
time-shift state across tokens, and compares the logits (max|gpu - ref| /
max|ref|, the north star's 1e-3), the Q/K/V sign bits the automaton would be
handed (as a mismatch fraction: a projection output within rounding of 0 may
land on either side) and the argmax. The product operands are fp16 on the GPU
(the few-row kernels round x to fp16, the train step's operand precision) and
fp32 in the oracle.
"""
import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.runtime import HeronShape, HeronTrainer
from ullis_amd.synth import heron_arena, unpack_bits

pytestmark = pytest.mark.gpu

LOGIT_REL = 1e-3   # max|gpu - ref| / max|ref| of a token's logits (north star)
BITS_FRAC = 7e-4   # Q/K/V sign bits, as for the train step's bit-planes

CASES = [
    # d, layers, ffn, vocab, batch, tokens
    (64, 2, 128, 256, 2, 6),
    (512, 12, 2048, 8192, 8, 3),
    (1024, 2, 4096, 32768, 1, 3),
]


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(a - r))) / max(float(np.max(np.abs(r))), 1e-30)


def make(rt, d, layers, ffn, vocab, batch, seed):
    shape = HeronShape(d, layers, ffn, vocab, 1, 2)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=seed,
                        random_ln=True, mix_range=(0.2, 0.8))
    trainer.upload_arena(arena)
    rng = np.random.default_rng(seed)
    table = rng.standard_normal(vocab * d).astype(np.float16).view(np.uint16)
    return trainer, trainer.download_arena(), table


def planes_to_bits(planes, batch, d):
    """[3, words] u32 planes (bit b*d + c) -> u8 [3, batch, d]."""
    bits = unpack_bits(planes.ravel(), planes.size * 32).reshape(3, -1)
    return bits[:, :batch * d].reshape(3, batch, d)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "d{}L{}F{}V{}B{}".format(*c[:5]))
def test_decode_matches_oracle(rt, case):
    d, layers, ffn, vocab, batch, steps = case
    trainer, arena, table = make(rt, d, layers, ffn, vocab, batch, seed=d + layers)
    dims = o.HeronDims(d, layers, ffn, vocab)
    rng = np.random.default_rng(5)
    tokens = rng.integers(0, vocab, (steps, batch)).astype(np.uint32)
    idx = (rng.random((steps, layers, batch, d)) < 0.5).astype(np.uint8)
    dtab = rt.put(table)
    dtok = rt.zeros(np.uint32, batch)
    logits = rt.zeros(np.float32, batch * vocab)
    nxt = rt.zeros(np.uint32, batch)
    inv = rt.zeros(np.uint32, 1)
    rp = np.zeros(layers * batch * d, np.float32)
    cp = np.zeros(layers * batch * d, np.float32)
    trainer.decode_init(batch)
    for t in range(steps):
        seen = {}

        def sam(layer, planes, t=t):
            seen[layer] = planes
            return idx[t, layer]

        dtok.upload(tokens[t])
        trainer.decode_step(dtab, dtok, logits, next_tokens=nxt, sam=sam, invalid=inv)
        rt.sync()
        gl = logits.download(np.float32).reshape(batch, vocab)
        gn = nxt.download(np.uint32)
        ref, qkv = o.heron_decode_step(dims, arena, table, tokens[t], idx[t], rp, cp, t > 0)
        r = rel(gl, ref)
        assert r <= LOGIT_REL, f"token {t}: logits rel {r:.3g}"
        assert sorted(seen) == list(range(layers))
        for layer in range(layers):
            got = planes_to_bits(seen[layer], batch, d)
            mism = int(np.count_nonzero(got != qkv[layer]))
            assert mism <= max(2, BITS_FRAC * got.size), (t, layer, mism)
        np.testing.assert_array_equal(gn, np.argmax(gl, axis=1))
        # the oracle's argmax wherever its top two logits are apart by more than the drift
        top2 = np.sort(ref.astype(np.float64), axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2 * LOGIT_REL * np.abs(ref).max()
        np.testing.assert_array_equal(gn[clear], np.argmax(ref, axis=1)[clear])
        assert int(inv.download(np.uint32)[0]) == 0


def test_decode_given_indices_equal_the_callback_path_and_init_restarts(rt):
    """The graph replay of the step with given indices (tokens 0 and 2 replay
    the parity-0 graph), the eager step, and the step whose indices come from
    the host callback give identical logits; decode_init restarts."""
    d, layers, ffn, vocab, batch = 128, 3, 256, 512, 4
    trainer, _, table = make(rt, d, layers, ffn, vocab, batch, seed=3)
    rng = np.random.default_rng(9)
    tokens = rng.integers(0, vocab, (3, batch)).astype(np.uint32)
    idx = (rng.random((3, layers, batch, d)) < 0.5).astype(np.uint8)
    dtab = rt.put(table)
    dtok = rt.zeros(np.uint32, batch)
    didx = rt.zeros(np.uint8, layers * batch * d)
    logits = rt.zeros(np.float32, batch * vocab)

    def run(via_callback, graph=True):
        trainer.decode_init(batch, graph=graph)
        out = []
        for t in range(3):
            dtok.upload(tokens[t])
            if via_callback:
                trainer.decode_step(dtab, dtok, logits, sam=lambda layer, planes, t=t: idx[t, layer])
            else:
                didx.upload(idx[t].ravel())
                trainer.decode_step(dtab, dtok, logits, rosa_idx=didx)
            rt.sync()
            out.append(logits.download(np.float32).copy())
        return out

    a = run(True)
    b = run(False)  # decode_init restarts the sequences: no previous token at t = 0
    c = run(False, graph=False)
    for t in range(3):
        np.testing.assert_array_equal(a[t], b[t], err_msg=f"token {t}")
        np.testing.assert_array_equal(a[t], c[t], err_msg=f"token {t}, eager")
    assert not np.array_equal(a[0], a[1])


def test_decode_token_outside_vocab_is_counted(rt):
    d, layers, ffn, vocab, batch = 64, 1, 128, 256, 2
    trainer, _, table = make(rt, d, layers, ffn, vocab, batch, seed=4)
    dtab = rt.put(table)
    dtok = rt.put(np.array([3, vocab + 5], np.uint32))
    didx = rt.zeros(np.uint8, layers * batch * d)
    logits = rt.zeros(np.float32, batch * vocab)
    inv = rt.zeros(np.uint32, 1)
    trainer.decode_init(batch)
    trainer.decode_step(dtab, dtok, logits, rosa_idx=didx, invalid=inv)
    rt.sync()
    assert int(inv.download(np.uint32)[0]) == 1


def test_decode_rejects_bad_arguments(rt):
    d, layers, ffn, vocab = 64, 1, 128, 256
    trainer, _, table = make(rt, d, layers, ffn, vocab, 1, seed=5)
    dtab = rt.put(table)
    dtok = rt.zeros(np.uint32, 1)
    didx = rt.zeros(np.uint8, layers * d)
    logits = rt.zeros(np.float32, vocab)
    with pytest.raises(Exception):
        trainer.decode_init(9)
    with pytest.raises(Exception):
        trainer.decode_init(0)
    trainer.decode_init(1)
    with pytest.raises(Exception):  # neither the indices nor the callback
        trainer.decode_step(dtab, dtok, logits)
    with pytest.raises(Exception):  # both
        trainer.decode_step(dtab, dtok, logits, rosa_idx=didx, sam=lambda l, p: didx)
    with pytest.raises(ValueError):  # the callback's failure surfaces
        trainer.decode_step(dtab, dtok, logits, sam=lambda l, p: np.zeros(3, np.uint8))
