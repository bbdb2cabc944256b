"""Checkpoint v2 save/load of the train state (ullis_amd/checkpoint.py)
against the format the reference writes (ModelCheckpoint::to_safetensors_bytes,
src/model.rs:3426-3553): tensor names restated here from the reference's
push_* / carry_* functions (src/model.rs:3765-3797, 3878-3931), dtypes,
1-D shapes, metadata, and the round trip of its own test
(checkpoint_roundtrip_after_train_preserves_forward, src/model.rs:4888-4941:
step 17, loss_ema 4.5, latents present)."""
import json

import numpy as np
import pytest

from ullis_amd.checkpoint import heron_config, load_checkpoint, save_checkpoint
from ullis_amd.runtime import HeronShape, heron_layout
from ullis_amd.synth import heron_arena
from safetensors.numpy import load as st_load

SHAPE = HeronShape(d_model=64, n_layers=3, dim_ffn=128, vocab=200, batch=1, time=32)


def reference_names(layers: int) -> set:
    """The tensor names to_safetensors_bytes writes for a Heron model whose
    block 0 has ln0, restated from the reference's push / carry functions."""
    names = {"embedding", "ln_out.weight", "ln_out.bias", "embedding.residual"}

    def storage(n):  # an Fp16Storage: value + carry
        names.update({n, f"{n}.residual"})

    def packed(p, bias):  # push_packed + carry_packed
        names.update({f"{p}.bits", f"{p}.latent", f"{p}.latent.residual"})
        storage(f"{p}.scale")
        if bias:
            storage(f"{p}.bias")

    storage("ln_out.weight")
    storage("ln_out.bias")
    packed("head", True)
    for i in range(layers):
        b = f"blocks.{i}"
        lns = ["ln2", "ln3"] + (["ln0"] if i == 0 else [])
        for ln in lns:
            storage(f"{b}.{ln}.weight")
            storage(f"{b}.{ln}.bias")
        for v in ("x_q", "x_k", "x_v", "e"):
            storage(f"{b}.rosa.{v}")
        for p in ("q", "k", "v", "o"):
            packed(f"{b}.rosa.{p}", True)
        storage(f"{b}.ffn.x_k")
        packed(f"{b}.ffn.key", False)
        storage(f"{b}.ffn.value")
    return names


@pytest.fixture(scope="module")
def state():
    layout, nbytes = heron_layout(SHAPE.dims())
    arena = heron_arena(layout, nbytes, SHAPE.dims(), seed=9, random_ln=True)
    rng = np.random.default_rng(9)
    # residual carries non-zero, so the round trip checks them too
    for name, dt, count, off, derived in layout:
        if dt == 2:
            arena[off: off + 4 * count] = (rng.standard_normal(count) * 1e-4).astype(
                np.float32).view(np.uint8)
    emb = rng.standard_normal(SHAPE.vocab * SHAPE.d_model).astype(np.float16).view(np.uint16)
    emb_res = (rng.standard_normal(emb.size) * 1e-4).astype(np.float32)
    return layout, nbytes, arena, emb, emb_res


def test_names_dtypes_shapes_and_metadata_match_the_reference_format(state):
    layout, nbytes, arena, emb, emb_res = state
    cfg = heron_config(SHAPE)
    data = save_checkpoint(arena, layout, emb, emb_res, cfg, step=17, loss_ema=4.5)
    tensors = st_load(data)
    assert set(tensors) == reference_names(SHAPE.n_layers)
    for name, t in tensors.items():
        assert t.ndim == 1, name
        if name.endswith(".residual"):
            assert t.dtype == np.float32, name
        elif name.endswith(".bits"):
            assert t.dtype == np.uint32, name
        else:
            assert t.dtype == np.float16, name
    n = int.from_bytes(data[:8], "little")
    meta = json.loads(data[8: 8 + n])["__metadata__"]
    assert meta["format_version"] == "2" and meta["step"] == "17" and meta["loss_ema"] == "4.5"
    # serde_json::to_string of TrainConfig: compact, fields in struct order
    assert meta["config"].startswith('{"architecture":"heron","d_model":64,"n_layers":3,')
    assert json.loads(meta["config"]) == cfg
    # sizes follow the shape: head bits ceil(V*D/32) words, key latent F*D
    assert tensors["head.bits"].size == (SHAPE.vocab * SHAPE.d_model + 31) // 32
    assert tensors["blocks.1.ffn.key.latent"].size == SHAPE.dim_ffn * SHAPE.d_model
    assert tensors["blocks.2.ffn.value"].size == SHAPE.d_model * SHAPE.dim_ffn


def test_round_trip_is_exact(state):
    layout, nbytes, arena, emb, emb_res = state
    data = save_checkpoint(arena, layout, emb, emb_res, heron_config(SHAPE), step=17, loss_ema=4.5)
    a2, e2, r2, meta = load_checkpoint(data, layout, nbytes, SHAPE)
    assert meta["step"] == 17 and meta["loss_ema"] == 4.5 and meta["format_version"] == 2
    for name, dt, count, off, derived in layout:
        size = count * (2 if dt == 1 else 4)
        if derived:
            assert not a2[off: off + size].any(), name  # rebuilt after upload
        else:
            np.testing.assert_array_equal(a2[off: off + size], arena[off: off + size],
                                          err_msg=name)
    np.testing.assert_array_equal(e2, emb)
    np.testing.assert_array_equal(r2.view(np.uint32), emb_res.view(np.uint32))
    # saving the loaded state again gives the same header (as parsed: the
    # writer keeps metadata in a hash map, so its key order varies) and the
    # same tensor bytes
    again = save_checkpoint(a2, layout, e2, r2, meta["config"], step=17, loss_ema=4.5)
    n1, n2 = (int.from_bytes(b[:8], "little") for b in (data, again))
    assert json.loads(again[8: 8 + n2]) == json.loads(data[8: 8 + n1])
    assert again[8 + n2:] == data[8 + n1:]


def test_rejections_and_defaults(state):
    from safetensors.numpy import save as st_save

    layout, nbytes, arena, emb, emb_res = state
    good = st_load(save_checkpoint(arena, layout, emb, emb_res, heron_config(SHAPE)))
    meta = {"format_version": "2", "config": json.dumps(heron_config(SHAPE)), "step": "3"}
    # v1 (Hyena) and version-less files are rejected (require_v2, src/model.rs:2426-2431)
    with pytest.raises(ValueError, match="v1"):
        load_checkpoint(st_save(good, metadata=dict(meta, format_version="1")), layout, nbytes)
    with pytest.raises(ValueError, match="metadata"):
        load_checkpoint(st_save(good), layout, nbytes)
    with pytest.raises(ValueError, match="does not match"):
        load_checkpoint(st_save(good, metadata=dict(
            meta, config=json.dumps(heron_config(SHAPE, d_model=128)))), layout, nbytes, SHAPE)
    # a missing latent is an error; a missing carry loads as zeros
    no_lat = {k: v for k, v in good.items() if k != "head.latent"}
    with pytest.raises(ValueError, match="head.latent is missing"):
        load_checkpoint(st_save(no_lat, metadata=meta), layout, nbytes)
    no_res = {k: v for k, v in good.items() if k != "head.scale.residual"}
    a2, _, _, m2 = load_checkpoint(st_save(no_res, metadata=meta), layout, nbytes)
    assert m2["step"] == 3 and m2["loss_ema"] is None
    off = next(o for n, _, _, o, _ in layout if n == "head.scale.residual")
    assert not a2[off: off + 4 * SHAPE.vocab].any()
    # wrong dtype is an error
    bad = dict(good, **{"head.bits": good["head.bits"].view(np.float32)})
    with pytest.raises(ValueError, match="head.bits"):
        load_checkpoint(st_save(bad, metadata=meta), layout, nbytes)
