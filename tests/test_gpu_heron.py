"""GPU Heron train step (ullis_hip_heron_step) against the oracle step
(ucr_heron_train_step, src/model.rs:2827-3025) on the same seeded inputs.

The GPU keeps GEMM operands in fp16 (LayerNorm outputs, CMix activations,
ROSA y) while the oracle carries fp32 activations, so composed outputs differ
by accumulated fp16 rounding. Per-op bounds are in test_gpu_ops.py; here each
output tensor is compared with max|gpu - ref| / max|ref|. Every case writes
its measured drift to step_drift/<case>.json under RESULTS. Over the six cases
(up to config 4's full depth, L12, and config 5's widths, D1024 V32768) the
measured maxima were: mean CE 2.2e-5, any row's CE 2.5e-4, g_emb 3.5e-4,
updated f16 parameters 7.6e-4 (the ROSA O scales), Q/K/V sign bit-planes
3.3e-4 of the bits, updated weight sign bits 1e-6. The bounds below are the
north star's (1e-3 relative, 1e-4 per token for the mean CE) where the drift
stays inside them, and 2x the measured drift for the single-row CE and the
sign-bit fractions. Sign bits are compared as mismatch fractions: a latent
within rounding of 0, or a projection output within rounding of 0, may land
on either side.
"""
import ctypes as C
import json
import pathlib

import numpy as np
import pytest

from oracle import cpu_ref as o
from ullis_amd.runtime import HeronShape, HeronTrainer
from ullis_amd.synth import heron_arena, step_inputs, tensor_view, unpack_bits

pytestmark = pytest.mark.gpu

NO_IGNORE = 0xFFFFFFFF
STEP_REL = 1e-3        # fp16 params / g_emb after one composed step (north star)
LOSS_ABS = 1e-4        # mean CE over the valid rows (north star, per token)
ROW_LOSS_ABS = 5e-4    # the CE of any single row (2x the measured 2.5e-4)
BITS_FRAC = 7e-4       # Q/K/V sign bit-planes (2x the measured 3.3e-4)
WEIGHT_BITS_FRAC = 1e-5  # updated weight sign bits (measured 1e-6), at least 2 bits a tensor


def weight_bits_ok(mism: int, n: int) -> bool:
    return mism <= max(2, WEIGHT_BITS_FRAC * n)


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
            report[name] = ("bits", mism / max(n, 1), mism, n)
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
    # config 4's widths and full depth (D512 L12 F2048 V8192) on a 64-token window
    HeronShape(d_model=512, n_layers=12, dim_ffn=2048, vocab=8192, batch=1, time=64),
    # config 5's widths (D1024 F4096 V32768), two sequences of 16 tokens, two layers
    HeronShape(d_model=1024, n_layers=2, dim_ffn=4096, vocab=32768, batch=2, time=16),
]

ROOT = pathlib.Path(__file__).resolve().parent.parent
# results folder of a GPU run (the one a remote run's outputs come back from)
RESULTS = ROOT / "gpurun_out"


def record_drift(case: str, drift: dict) -> None:
    """Writes the measured composed drift of one case to
    RESULTS/step_drift/<case>.json (the figures the bounds above rest on)."""
    out = RESULTS / "step_drift"
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{case}.json").write_text(json.dumps(drift, indent=1, sort_keys=True))


def shape_id(s):
    return f"d{s.d_model}L{s.n_layers}F{s.dim_ffn}V{s.vocab}B{s.batch}T{s.time}"


@pytest.mark.parametrize("shape", SMALL, ids=shape_id)
def test_heron_step_matches_oracle(rt, shape):
    trainer, before, gpu, cpu = run_both(rt, shape)
    rows = shape.rows
    words = (rows * shape.d_model + 31) // 32
    n = rows * shape.d_model
    mism = np.count_nonzero(unpack_bits(gpu["qkv"], shape.n_layers * 3 * words * 32)
                            != unpack_bits(cpu["qkv_bits"], shape.n_layers * 3 * words * 32))
    report = compare(trainer, before, gpu, cpu, shape)
    drift = {
        "loss_abs": abs(float(gpu["stats"][0]) - cpu["mean_loss"]),
        "row_loss_abs": float(np.max(np.abs(gpu["row_loss"] - cpu["row_loss"]))),
        "g_emb_rel": rel(gpu["g_emb"], cpu["g_emb"]),
        "qkv_bits_frac": mism / (shape.n_layers * 3 * n),
        "param_rel_max": max([v[1] for v in report.values() if v[0] == "rel"], default=0.0),
        "bits_frac_max": max([v[1] for v in report.values() if v[0] == "bits"], default=0.0),
        "worst_param": max(((v[1], k) for k, v in report.items() if v[0] == "rel"),
                           default=(0.0, ""))[1],
    }
    record_drift(shape_id(shape), drift)
    assert int(gpu["stats"][1]) == cpu["n_valid"] == rows - shape.batch
    assert drift["loss_abs"] <= LOSS_ABS
    assert drift["row_loss_abs"] <= ROW_LOSS_ABS
    assert drift["g_emb_rel"] <= STEP_REL
    assert drift["qkv_bits_frac"] <= BITS_FRAC
    bad = {k: v for k, v in report.items()
           if (v[0] == "rel" and v[1] > STEP_REL) or (v[0] == "bits" and not weight_bits_ok(*v[2:]))}
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


def flips_by_class(before, after, lay):
    """bit_flip_count (src/model.rs:150-156) of every updated sign-bit tensor
    between two arenas, by CausalLoss class (head, CMix key, ROSA O)."""
    out = {"head": 0, "cmix": 0, "rosa_o": 0}
    for name, dt, count, off, derived in lay:
        if dt != 3 or derived:
            continue
        cls = ("head" if name == "head.bits" else "cmix" if name.endswith("ffn.key.bits")
               else "rosa_o" if name.endswith("rosa.o.bits") else None)
        diff = np.bitwise_xor(tensor_view(before, lay, name), tensor_view(after, lay, name))
        n = int(np.unpackbits(diff.view(np.uint8)).sum())
        if cls is None:
            assert n == 0, name  # Q/K/V are frozen under stop_grad_bits
        else:
            out[cls] += n
    return out


def test_full_stress_step_properties(rt):
    """Config 5 at full size (D1024 L24 F4096 V32768, batch 8 x T4096): no
    oracle run (hours on a CPU); what the mathematics fixes instead: two steps
    from one state are bit-identical, the CE of a random init is close to
    ln(V), every sign-bit tensor is the repack of its latent, the gradients are
    finite, and the step's CausalLoss flip counts are exactly the bits that
    changed between the arenas."""
    shape = HeronShape(d_model=1024, n_layers=24, dim_ffn=4096, vocab=32768, batch=8, time=4096)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=7)
    _, labels, idx = step_inputs(shape.rows, 1024, 32768, 24, 8, 4096, seed=7)
    rng = np.random.default_rng(7)
    table = rng.standard_normal(32768 * 1024).astype(np.float16).view(np.uint16)
    tokens = rt.put(rng.integers(0, 32768, shape.rows).astype(np.uint32))
    dl, di = rt.put(labels), rt.put(idx)
    nd = shape.rows * 1024
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    outs = []
    for _ in range(2):
        trainer.upload_arena(arena)
        dt, dtr = rt.put(table), rt.zeros(np.float32, table.size)
        rl, st, bad = rt.zeros(np.float32, shape.rows), rt.zeros(np.float32, 4), rt.zeros(
            np.uint32, 1)
        trainer.step_tokens(dt, dtr, tokens, dl, NO_IGNORE, 0.01, di, xe, g, rl, st, invalid=bad)
        cl = trainer.causal_loss(g, dl, NO_IGNORE, rl, dtr)
        rt.sync()
        outs.append((trainer.download_arena(), g.download(np.float32), rl.download(np.float32),
                     st.download(np.float32), bad.download(np.uint32)[0], cl))
    (a0, g0, r0, s0, b0, c0), (a1, g1, r1, _, _, c1) = outs
    np.testing.assert_array_equal(a0, a1)
    np.testing.assert_array_equal(g0.view(np.uint32), g1.view(np.uint32))
    np.testing.assert_array_equal(r0.view(np.uint32), r1.view(np.uint32))
    assert c0 == c1
    assert b0 == 0 and s0[1] == 8 * 4095
    # random init: CE ~ ln V + var(logit) / 2, var(logit) = scale^2 D E[h^2] ~ 0.17
    assert abs(s0[0] - np.log(32768)) < 0.25
    assert np.isfinite(g0).all() and np.abs(g0).max() > 0
    lay = trainer.layout
    for name, dt_, count, off, derived in lay:
        if name.endswith(".bits") and not derived:
            lat = tensor_view(a0, lay, name[: -len(".bits")] + ".latent")
            np.testing.assert_array_equal(tensor_view(a0, lay, name), o.pack_latent_bits(lat),
                                          err_msg=name)
    f = flips_by_class(arena, a0, lay)
    assert (c0["flips_head"], c0["flips_cmix"], c0["flips_rosa_o"]) == (
        f["head"], f["cmix"], f["rosa_o"])
    assert c0["binary_flip_count"] == sum(f.values()) > 0
    assert c0["next_token_count"] == 8 * 4095


def test_causal_loss_matches_oracle_and_host_statistics(rt):
    """ullis_hip_heron_causal_loss (CausalLoss, src/model.rs:2997-3024): exact
    against statistics taken on the host from the GPU's own outputs (flip
    counts from the arenas, percentiles and unigram CE from its row losses and
    labels), and against the oracle step within the composed-step bounds."""
    shape = HeronShape(d_model=64, n_layers=2, dim_ffn=256, vocab=512, batch=2, time=32)
    trainer, before, gpu, cpu = run_both(rt, shape)
    # run_both leaves the trainer after the step; take the diagnostics of it
    lay = trainer.layout
    x, labels, idx = step_inputs(shape.rows, shape.d_model, shape.vocab, shape.n_layers,
                                 shape.batch, shape.time, seed=7)
    dl = rt.put(labels)
    g = rt.put(gpu["g_emb"])
    rl = rt.put(gpu["row_loss"])
    cl = trainer.causal_loss(g, dl, NO_IGNORE, rl)
    f = flips_by_class(before, gpu["arena"], lay)
    assert (cl["flips_head"], cl["flips_cmix"], cl["flips_rosa_o"]) == (
        f["head"], f["cmix"], f["rosa_o"])
    assert cl["binary_flip_count"] == sum(f.values())
    assert (cl["loss_p10"], cl["loss_p50"], cl["loss_p90"]) == o.loss_percentiles(
        gpu["row_loss"], shape.time, labels, NO_IGNORE)
    uce, uniq = o.unigram_cross_entropy(labels, shape.time, NO_IGNORE)
    assert cl["unique_targets"] == uniq and abs(cl["unigram_ce"] - uce) <= 1e-6 * uce
    assert cl["next_token_count"] == cpu["n_valid"]
    assert cl["next_token"] == float(gpu["stats"][0])
    a = gpu["arena"]
    host = {
        "embed_grad_rms": o.rms(gpu["g_emb"]),
        "head_scale_rms": o.rms_fp16(tensor_view(a, lay, "head.scale")),
        "cmix_value_rms": o.rms_fp16(tensor_view(a, lay, "blocks.0.ffn.value")),
        "head_latent_abs_mean": o.mean_abs_fp16(tensor_view(a, lay, "head.latent")),
        "head_latent_step_abs": o.mean_abs_delta_fp16(tensor_view(before, lay, "head.latent"),
                                                      tensor_view(a, lay, "head.latent")),
        "head_bias_rms": o.rms_fp16(tensor_view(a, lay, "head.bias")),
    }
    for k, v in host.items():  # fixed-order sums against sequential ones
        assert abs(cl[k] - v) <= 1e-5 * abs(v) + 1e-30, (k, cl[k], v)
    assert cl["residual_abs_mean"] == 0.0  # no table carry given
    # against the oracle's own step
    for k in ["loss_p10", "loss_p50", "loss_p90"]:
        assert abs(cl[k] - cpu[k]) <= ROW_LOSS_ABS, k
    assert abs(cl["unigram_ce"] - cpu["unigram_ce"]) <= 1e-6 * cpu["unigram_ce"]
    for k in ["embed_grad_rms", "head_scale_grad_rms", "head_scale_rms", "cmix_value_rms",
              "head_latent_abs_mean", "head_latent_step_abs", "head_bias_rms"]:
        assert abs(cl[k] - cpu[k]) <= STEP_REL * abs(cpu[k]), (k, cl[k], cpu[k])
    weights = {"head": shape.vocab * shape.d_model,
               "cmix": shape.n_layers * shape.dim_ffn * shape.d_model,
               "rosa_o": shape.n_layers * shape.d_model * shape.d_model}
    for cls, key in (("head", "flips_head"), ("cmix", "flips_cmix"), ("rosa_o", "flips_rosa_o")):
        assert weight_bits_ok(abs(cl[key] - cpu[key]), weights[cls]), (cls, cl[key], cpu[key])


def test_step_with_labels_outside_vocab_changes_nothing(rt):
    """train_step_on refuses labels >= vocab (other than the ignore id) and
    token ids >= vocab before any update (src/model.rs:2852-2861). The device
    step counts them and every update launch leaves the parameters and the
    embedding table as they were."""
    shape = HeronShape(d_model=64, n_layers=2, dim_ffn=128, vocab=256, batch=2, time=32)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=9)
    x, labels, idx = step_inputs(shape.rows, 64, 256, 2, 2, 32, seed=9)
    rng = np.random.default_rng(9)
    table = rng.standard_normal(256 * 64).astype(np.float16).view(np.uint16)
    tokens = rng.integers(0, 256, shape.rows).astype(np.uint32)
    nd = shape.rows * 64
    di = rt.put(idx)
    cases = [("label", labels.copy(), tokens.copy()), ("token", labels.copy(), tokens.copy())]
    cases[0][1][5] = 256
    cases[1][2][9] = 300
    for what, lab, tok in cases:
        trainer.upload_arena(arena)
        before = trainer.download_arena()
        dt, dtr = rt.put(table), rt.zeros(np.float32, table.size)
        bad = rt.zeros(np.uint32, 1)
        xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
        trainer.step_tokens(dt, dtr, rt.put(tok), rt.put(lab), NO_IGNORE, 0.01, di, xe, g,
                            invalid=bad)
        rt.sync()
        assert bad.download(np.uint32)[0] == 1, what
        np.testing.assert_array_equal(trainer.download_arena(), before, err_msg=what)
        np.testing.assert_array_equal(dt.download(np.uint16), table, err_msg=what)
        assert not dtr.download(np.float32).any(), what
    # the same label through ullis_hip_heron_step
    trainer.upload_arena(arena)
    bad = rt.zeros(np.uint32, 1)
    g = rt.zeros(np.float32, nd)
    trainer.step(rt.put(x), rt.put(cases[0][1]), NO_IGNORE, 0.01, di, g, invalid=bad)
    rt.sync()
    assert bad.download(np.uint32)[0] == 1
    np.testing.assert_array_equal(trainer.download_arena(), before)
    # and a clean step does move the state
    trainer.step(rt.put(x), rt.put(labels), NO_IGNORE, 0.01, di, g, invalid=bad)
    rt.sync()
    assert bad.download(np.uint32)[0] == 0
    assert not np.array_equal(trainer.download_arena(), before)


def test_graph_replay_of_steps_from_tokens(rt):
    """Steps from token ids replayed from the step graph are bit-identical to
    eager steps, also across a change of learning rate (captured again)."""
    shape = HeronShape(d_model=128, n_layers=2, dim_ffn=512, vocab=1024, batch=2, time=128)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=12)
    _, labels, idx = step_inputs(shape.rows, 128, 1024, 2, 2, 128, seed=12)
    rng = np.random.default_rng(12)
    table = rng.standard_normal(1024 * 128).astype(np.float16).view(np.uint16)
    tokens = rt.put(rng.integers(0, 1024, shape.rows).astype(np.uint32))
    dl, di = rt.put(labels), rt.put(idx)
    nd = shape.rows * 128
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    rl, st = rt.zeros(np.float32, shape.rows), rt.zeros(np.float32, 4)

    def run(graph):
        trainer.upload_arena(arena)
        dt, dtr = rt.put(table), rt.zeros(np.float32, table.size)
        trainer.set_graph(graph)
        outs = []
        for lr in (0.01, 0.01, 0.02, 0.02):
            trainer.step_tokens(dt, dtr, tokens, dl, NO_IGNORE, lr, di, xe, g, rl, st)
            rt.sync()
            outs.append((trainer.download_arena(), dt.download(np.uint16),
                         dtr.download(np.float32).view(np.uint32),
                         rl.download(np.float32).view(np.uint32)))
        trainer.set_graph(False)
        return outs

    eager, graph = run(False), run(True)
    for i, (e, r) in enumerate(zip(eager, graph)):
        for a, b in zip(e, r):
            np.testing.assert_array_equal(a, b, err_msg=f"step {i}")


def test_step_phases_cover_the_step_and_change_nothing(rt):
    """ullis_hip_heron_phases (the reference's TrainStepProfile phases,
    src/model.rs:2864-2994): every phase of a step from token ids gets time,
    the phases add up to the step as events around it read it, and a phased
    step's results are bit-identical to an unphased one's."""
    shape = HeronShape(d_model=128, n_layers=2, dim_ffn=512, vocab=1024, batch=2, time=128)
    trainer = HeronTrainer(rt, shape)
    arena = heron_arena(trainer.layout, trainer.arena_bytes, shape.dims(), seed=13)
    _, labels, idx = step_inputs(shape.rows, 128, 1024, 2, 2, 128, seed=13)
    rng = np.random.default_rng(13)
    table = rng.standard_normal(1024 * 128).astype(np.float16).view(np.uint16)
    tokens = rt.put(rng.integers(0, 1024, shape.rows).astype(np.uint32))
    dl, di = rt.put(labels), rt.put(idx)
    nd = shape.rows * 128
    xe, g = rt.zeros(np.float32, nd), rt.zeros(np.float32, nd)
    rl = rt.zeros(np.float32, shape.rows)
    lib, ctx = rt.lib, rt.ctx

    def run(phased, steps=3):
        trainer.upload_arena(arena)
        dt, dtr = rt.put(table), rt.zeros(np.float32, table.size)
        if phased:
            trainer.phases_begin()
        rt.sync()
        rt._check(lib.ullis_hip_event_record(ctx, 0), "event")
        for _ in range(steps):
            trainer.step_tokens(dt, dtr, tokens, dl, NO_IGNORE, 0.01, di, xe, g, rl)
        rt._check(lib.ullis_hip_event_record(ctx, 1), "event")
        rt.sync()
        ms = C.c_float()
        rt._check(lib.ullis_hip_event_elapsed_ms(ctx, 0, 1, C.byref(ms)), "elapsed")
        ph = trainer.phases_end() if phased else None
        return (trainer.download_arena(), dt.download(np.uint16),
                rl.download(np.float32).view(np.uint32)), ms.value / steps, ph

    plain, _, _ = run(False)
    phased, step_ms, ph = run(True)
    for a, b in zip(plain, phased):
        np.testing.assert_array_equal(a, b)
    assert ph["steps"] == 3
    assert set(ph["phases_ms"]) == set(HeronTrainer.PHASES)
    assert all(v > 0.0 for v in ph["phases_ms"].values()), ph
    total = sum(ph["phases_ms"].values())
    # the phases run from the gather to the step's last launch; the events
    # around the steps also hold the launches between steps
    assert 0.8 * step_ms <= total <= 1.001 * step_ms, (total, step_ms)
