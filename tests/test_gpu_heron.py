"""GPU Heron train step (ullis_hip_heron_step) against the oracle step
(ucr_heron_train_step, src/model.rs:2827-3025) on the same seeded inputs.

The GPU keeps GEMM operands in fp16 (LayerNorm outputs, CMix activations,
ROSA y) while the oracle carries fp32 activations, so composed outputs differ
by accumulated fp16 rounding. Per-op bounds are in test_gpu_ops.py; here each
output tensor is compared with max|gpu - ref| / max|ref| and the bounds below
(STEP_REL) are the measured composed drift with margin, stated per quantity.
Sign bits are compared as mismatch fractions: a latent within rounding of 0,
or a projection output within rounding of 0, may land on either side.
"""
import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.runtime import HeronShape, HeronTrainer
from ullis_amd.synth import heron_arena, step_inputs, tensor_view, unpack_bits

pytestmark = pytest.mark.gpu

NO_IGNORE = 0xFFFFFFFF
STEP_REL = 5e-3        # fp16 params / g_emb after one composed step
LOSS_ABS = 2e-3        # per-token CE after a composed forward (unit op bound is 1e-4)
BITS_FRAC = 2e-3       # allowed fraction of sign-bit disagreements


def h2f(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def rel(a, r):
    a = np.asarray(a, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(a - r))) / max(float(np.max(np.abs(r))), 1e-30)


def run_both(rt, shape: HeronShape, lr=0.01, ignore=NO_IGNORE, seed=7):
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=seed,
                        random_ln=True)
    x, labels, idx = step_inputs(shape.rows, shape.d_model, shape.vocab, shape.n_layers,
                                 shape.batch, shape.time, seed=seed)
    if ignore != NO_IGNORE:
        labels[::7] = ignore
    trainer.upload_arena(arena)
    ref_arena = trainer.download_arena()  # includes derived bits_t
    words = (shape.rows * shape.d_model + 31) // 32
    dx, dl, di = rt.put(x), rt.put(labels), rt.put(idx)
    g = rt.zeros(np.float32, shape.rows * shape.d_model)
    rl = rt.zeros(np.float32, shape.rows)
    st = rt.zeros(np.float32, 4)
    qkv = rt.zeros(np.uint32, shape.n_layers * 3 * words)
    trainer.step(dx, dl, ignore, lr, di, g, rl, st, qkv)
    rt.sync()
    gpu = {
        "arena": trainer.download_arena(),
        "g_emb": g.download(np.float32),
        "row_loss": rl.download(np.float32),
        "stats": st.download(np.float32),
        "qkv": qkv.download(np.uint32),
    }
    odims = o.HeronDims(shape.d_model, shape.n_layers, shape.dim_ffn, shape.vocab)
    cpu_arena = ref_arena.copy()
    cpu = o.heron_train_step(odims, cpu_arena, x, labels, ignore, shape.batch, shape.time, lr, idx)
    cpu["arena"] = cpu_arena
    return trainer, ref_arena, gpu, cpu


def compare(trainer, before, gpu, cpu, shape):
    lay = trainer.layout
    report = {}
    for name, dt, count, off, derived in lay:
        a = tensor_view(gpu["arena"], lay, name)
        r = tensor_view(cpu["arena"], lay, name)
        if name.endswith(".residual"):
            continue
        if dt == 3:  # bits
            if derived:
                continue  # checked against its own bits below
            n = count * 32
            mism = np.count_nonzero(unpack_bits(a, n) != unpack_bits(r, n))
            report[name] = ("bits", mism / max(n, 1))
        else:
            if name.endswith(".latent"):
                # compare the exact desired value: f16 payload + fp32 carry
                ra = tensor_view(gpu["arena"], lay, name + ".residual")
                rr = tensor_view(cpu["arena"], lay, name + ".residual")
                report[name] = ("rel", rel(h2f(a) + ra, h2f(r) + rr))
            else:
                report[name] = ("rel", rel(h2f(a), h2f(r)))
    return report


SMALL = [
    HeronShape(d_model=64, n_layers=2, dim_ffn=256, vocab=512, batch=2, time=32),
    HeronShape(d_model=96, n_layers=3, dim_ffn=160, vocab=300, batch=1, time=48),
    HeronShape(d_model=512, n_layers=2, dim_ffn=2048, vocab=8192, batch=1, time=64),
    HeronShape(d_model=64, n_layers=2, dim_ffn=128, vocab=256, batch=2, time=4),  # 8 rows
]


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: f"d{s.d_model}L{s.n_layers}T{s.time}")
def test_heron_step_matches_oracle(rt, shape):
    trainer, before, gpu, cpu = run_both(rt, shape)
    rows = shape.rows
    assert int(gpu["stats"][1]) == cpu["n_valid"] == rows - shape.batch
    assert abs(gpu["stats"][0] - cpu["mean_loss"]) <= LOSS_ABS
    assert np.max(np.abs(gpu["row_loss"] - cpu["row_loss"])) <= LOSS_ABS
    assert rel(gpu["g_emb"], cpu["g_emb"]) <= STEP_REL
    words = (rows * shape.d_model + 31) // 32
    n = rows * shape.d_model
    mism = np.count_nonzero(unpack_bits(gpu["qkv"], shape.n_layers * 3 * words * 32)
                            != unpack_bits(cpu["qkv_bits"], shape.n_layers * 3 * words * 32))
    assert mism / (shape.n_layers * 3 * n) <= BITS_FRAC
    report = compare(trainer, before, gpu, cpu, shape)
    bad = {k: v for k, v in report.items()
           if (v[0] == "rel" and v[1] > STEP_REL) or (v[0] == "bits" and v[1] > BITS_FRAC)}
    assert not bad, bad
    # bits_t caches agree with the updated bits on the GPU
    lay = trainer.layout
    for name, dt, count, off, derived in lay:
        if derived:
            prefix = name[: -len(".bits_t")]
            out_f, in_f = {"head": (shape.vocab, shape.d_model)}.get(
                prefix, (shape.dim_ffn, shape.d_model) if prefix.endswith("ffn.key")
                else (shape.d_model, shape.d_model))
            bits = tensor_view(gpu["arena"], lay, prefix + ".bits")
            np.testing.assert_array_equal(tensor_view(gpu["arena"], lay, name),
                                          o.transpose_bits(bits, out_f, in_f))


def test_heron_step_ignore_id_and_frozen_stop_grad_tensors(rt):
    shape = HeronShape(d_model=64, n_layers=2, dim_ffn=128, vocab=256, batch=2, time=16)
    trainer, before, gpu, cpu = run_both(rt, shape, ignore=5)
    assert int(gpu["stats"][1]) == cpu["n_valid"]
    lay = trainer.layout
    # stop_grad_bits freezes Q/K/V and ln3 (src/model.rs:4691-4719)
    for name, *_ in lay:
        if any(t in name for t in [".rosa.q.", ".rosa.k.", ".rosa.v.", ".ln3.", ".x_q", ".x_v",
                                   ".rosa.x_k"]):
            np.testing.assert_array_equal(tensor_view(gpu["arena"], lay, name),
                                          tensor_view(before, lay, name), err_msg=name)


def test_full_heron_step_properties(rt):
    """Config 4 at full size (D512 L12 T2048 V8192): no oracle run (minutes on a
    CPU); checks what the mathematics fixes instead."""
    shape = HeronShape(d_model=512, n_layers=12, dim_ffn=2048, vocab=8192, batch=1, time=2048)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=7)
    x, labels, idx = step_inputs(shape.rows, 512, 8192, 12, 1, 2048)
    dx, dl, di = rt.put(x), rt.put(labels), rt.put(idx)
    outs = []
    # same start state each time: bit-identical (deterministic reductions),
    # also with a launch probe armed (stamped GEMM launches, event-timed
    # LayerNorm launches)
    for probe in (None, None, "value_backward", "ln_backward"):
        trainer.upload_arena(arena)
        g = rt.zeros(np.float32, shape.rows * 512)
        rl = rt.zeros(np.float32, shape.rows)
        st = rt.zeros(np.float32, 4)
        if probe:
            trainer.probe_begin(probe)
        trainer.step(dx, dl, NO_IGNORE, 0.01, di, g, rl, st)
        rt.sync()
        if probe:
            k = trainer.probe_end(probe)
            assert k["count"] == 12, (probe, k)
            assert 1e-3 < k["total_ms"] / k["count"] < 5.0, (probe, k)
        outs.append((trainer.download_arena(), g.download(np.float32), rl.download(np.float32),
                     st.download(np.float32)))
    a0, g0, r0, s0 = outs[0]
    for a1, g1, r1, _ in outs[1:]:
        np.testing.assert_array_equal(a0, a1)
        np.testing.assert_array_equal(g0.view(np.uint32), g1.view(np.uint32))
        np.testing.assert_array_equal(r0.view(np.uint32), r1.view(np.uint32))
    assert s0[1] == 2047 and r0[2047] == 0.0
    # random init: logits are small, so the CE is close to ln(V)
    assert abs(s0[0] - np.log(8192)) < 0.05
    assert np.isfinite(g0).all() and np.abs(g0).max() > 0
    lay = trainer.layout
    for name, dt, count, off, derived in lay:
        if name.endswith(".bits") and not derived:
            lat = tensor_view(a0, lay, name[: -len(".bits")] + ".latent")
            np.testing.assert_array_equal(tensor_view(a0, lay, name), o.pack_latent_bits(lat),
                                          err_msg=name)


def test_graph_replay_matches_eager_steps(rt):
    """ullis_hip_heron_set_graph: steps replayed from the captured graph are
    bit-identical to eager steps, a new learning rate captures again, and
    turning the graph off returns to eager launches."""
    shape = HeronShape(d_model=256, n_layers=3, dim_ffn=1024, vocab=2048, batch=2, time=256)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=11)
    x, labels, idx = step_inputs(shape.rows, 256, 2048, 3, 2, 256, seed=11)
    dx, dl, di = rt.put(x), rt.put(labels), rt.put(idx)
    g = rt.zeros(np.float32, shape.rows * 256)
    rl = rt.zeros(np.float32, shape.rows)
    st = rt.zeros(np.float32, 4)
    lrs = (0.01, 0.01, 0.01, 0.02, 0.02)

    def run(graph):
        trainer.upload_arena(arena)
        trainer.set_graph(graph)
        outs = []
        for i, lr in enumerate(lrs):
            if graph and i == len(lrs) - 1:
                trainer.set_graph(False)
            trainer.step(dx, dl, NO_IGNORE, lr, di, g, rl, st)
            rt.sync()
            outs.append((trainer.download_arena(), g.download(np.float32),
                         rl.download(np.float32), st.download(np.float32)))
        return outs

    eager, graph = run(False), run(True)
    for i, (e, r) in enumerate(zip(eager, graph)):
        np.testing.assert_array_equal(e[0], r[0], err_msg=f"arena after step {i}")
        for a, b in zip(e[1:], r[1:]):
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32),
                                          err_msg=f"step {i}")
    assert not np.array_equal(eager[0][0], eager[1][0])  # the steps did move the state


def test_step_from_tokens_gathers_steps_and_scatters(rt):
    """HeronTrainer.step_tokens (gather, step, scatter-SGD on the device)
    against the same three stages run one at a time: the oracle's gather,
    the device step on its output, the oracle's scatter-SGD of the returned
    embedding gradient (all three bit-exact by construction)."""
    shape = HeronShape(d_model=64, n_layers=2, dim_ffn=128, vocab=300, batch=2, time=64)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=5)
    _, labels, idx = step_inputs(shape.rows, 64, 300, 2, 2, 64, seed=5)
    rng = np.random.default_rng(5)
    table = rng.standard_normal(300 * 64).astype(np.float16).view(np.uint16)
    table_res = (rng.standard_normal(300 * 64) * 1e-4).astype(np.float32)
    tokens = rng.integers(0, 40, shape.rows).astype(np.uint32)  # repeats
    nd = shape.rows * 64
    dl, di = rt.put(labels), rt.put(idx)

    trainer.upload_arena(arena)
    dt, dtr, dk = rt.put(table), rt.put(table_res), rt.put(tokens)
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    rl, st, bad = rt.zeros(np.float32, shape.rows), rt.zeros(np.float32, 4), rt.zeros(np.uint32, 1)
    trainer.step_tokens(dt, dtr, dk, dl, NO_IGNORE, 0.01, di, xe, g, rl, st, invalid=bad)
    rt.sync()
    assert bad.download(np.uint32)[0] == 0
    got = (trainer.download_arena(), dt.download(np.uint16), dtr.download(np.float32),
           rl.download(np.float32))

    trainer.upload_arena(arena)
    x = o.embedding_gather(table, 64, tokens)
    g2 = rt.zeros(np.float32, nd)
    rl2 = rt.zeros(np.float32, shape.rows)
    trainer.step(rt.put(x), dl, NO_IGNORE, 0.01, di, g2, rl2)
    rt.sync()
    want_t, want_r = o.embedding_scatter_sgd(table, table_res, 64, tokens, g2.download(np.float32),
                                             0.01)
    np.testing.assert_array_equal(got[0], trainer.download_arena())
    np.testing.assert_array_equal(got[1], want_t)
    np.testing.assert_array_equal(got[2].view(np.uint32), want_r.view(np.uint32))
    np.testing.assert_array_equal(got[3].view(np.uint32), rl2.download(np.float32).view(np.uint32))
    assert not np.array_equal(got[1], table)  # the table did move


def test_checkpoint_resume_continues_bit_identically(rt):
    """checkpoint_roundtrip_after_train_preserves_forward (src/model.rs:
    4888-4941) on the device: train a step, save checkpoint v2, load it into a
    second trainer, and the next step of both is bit-identical."""
    from ullis_amd.checkpoint import heron_config, load_checkpoint, save_checkpoint

    shape = HeronShape(d_model=64, n_layers=2, dim_ffn=128, vocab=256, batch=1, time=64)
    a, b = HeronTrainer(rt, shape), HeronTrainer(rt, shape)
    arena = heron_arena(a.layout, a.arena_bytes, shape.dims(), seed=4)
    _, labels, idx = step_inputs(shape.rows, 64, 256, 2, 1, 64, seed=4)
    rng = np.random.default_rng(4)
    table = rng.standard_normal(256 * 64).astype(np.float16).view(np.uint16)
    tokens = rt.put(rng.integers(0, 256, shape.rows).astype(np.uint32))
    nd = shape.rows * 64
    dl, di = rt.put(labels), rt.put(idx)
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    st = rt.zeros(np.float32, 4)
    a.upload_arena(arena)
    ta, tra = rt.put(table), rt.zeros(np.float32, table.size)
    a.step_tokens(ta, tra, tokens, dl, NO_IGNORE, 0.05, di, xe, g, stats=st)
    rt.sync()
    data = save_checkpoint(a.download_arena(), a.layout, ta.download(np.uint16),
                           tra.download(np.float32), heron_config(shape), step=17, loss_ema=4.5)
    arena2, emb, emb_res, meta = load_checkpoint(data, b.layout, b.arena_bytes, shape)
    assert meta["step"] == 17 and meta["loss_ema"] == 4.5
    b.upload_arena(arena2)  # rebuilds the derived bits_t
    tb, trb = rt.put(emb), rt.put(emb_res)
    np.testing.assert_array_equal(b.download_arena(), a.download_arena())
    outs = []
    for tr, t, r in ((a, ta, tra), (b, tb, trb)):
        rl = rt.zeros(np.float32, shape.rows)
        tr.step_tokens(t, r, tokens, dl, NO_IGNORE, 0.05, di, xe, g, rl)
        rt.sync()
        outs.append((tr.download_arena(), t.download(np.uint16), r.download(np.float32),
                     rl.download(np.float32)))
    for x, y in zip(*outs):
        np.testing.assert_array_equal(x, y)
