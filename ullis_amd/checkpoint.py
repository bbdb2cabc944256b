"""Checkpoint v2 (safetensors) of the device train state.

Writes and reads the format of `ModelCheckpoint::to_safetensors_bytes` /
`from_safetensors_bytes` (src/model.rs:3426-3553) for the Heron architecture:
- every tensor is 1-D (`push_f16` / `push_u32` / `push_f32`,
  src/model.rs:3688-3697, 3878-3898): parameters F16 (raw f16 bits), sign
  words U32, fp32 carries F32;
- parameter names are the checkpoint-v2 names, which the device arena uses
  too (include/ullis_heron_layout.h), plus `embedding`;
- the train carry (`fill_train_carry`, src/model.rs:3778-3797) is the
  `<packed>.latent` tensors and a `<name>.residual` for every f16 storage
  and latent;
- metadata `format_version` = "2", `config` (the TrainConfig JSON), `step`,
  and `loss_ema` when set.
Serialisation goes through the `safetensors` package, whose writer is the
same Rust crate at the same version (0.8.0) the reference links, so tensor
order and header layout are the crate's own.

A file written here loads in the reference and the other way round; the
derived `.bits_t` tensors of the arena are not part of the format and are
rebuilt after a load (`HeronTrainer.upload_arena`).
"""
from __future__ import annotations

import json

import numpy as np
from safetensors.numpy import load as st_load
from safetensors.numpy import save as st_save

FORMAT_VERSION = 2  # CHECKPOINT_FORMAT_VERSION, src/model.rs:21

# arena dtype codes (include/ullis_heron_layout.h) -> numpy dtype of the tensor
_NP = {1: np.float16, 2: np.float32, 3: np.uint32}
_BITS = {1: np.uint16, 2: np.float32, 3: np.uint32}


def heron_config(shape, seed: int = 7, **overrides) -> dict:
    """TrainConfig of a Heron run (src/config.rs:78-132) in serde field order,
    as `serde_json::to_string` writes it into the metadata."""
    cfg = {
        "architecture": "heron",
        "d_model": shape.d_model,
        "n_layers": shape.n_layers,
        "vocab_size": shape.vocab,
        "context_len": shape.time,
        "batch_size": shape.batch,
        "dim_ffn": shape.dim_ffn,
        "rosa_bits": 1,
        "rosa_grad": "stop_grad_bits",
        "head_size": 16,
        "tmix_lora_rank": 16,
        "seed": seed,
        "memory_budget_bytes": 4 * 1024 ** 3,
    }
    cfg.update(overrides)
    return cfg


def state_tensors(arena: np.ndarray, layout, embedding, embedding_residual) -> dict:
    """name -> 1-D numpy tensor of the checkpoint, from a downloaded arena."""
    out = {}
    for name, dt, count, off, derived in layout:
        if derived:
            continue
        raw = arena[off: off + count * np.dtype(_BITS[dt]).itemsize].view(_BITS[dt])
        out[name] = raw.view(_NP[dt]).copy()
    out["embedding"] = np.asarray(embedding, np.uint16).view(np.float16).copy()
    out["embedding.residual"] = np.asarray(embedding_residual, np.float32).copy()
    return out


def save_checkpoint(arena: np.ndarray, layout, embedding, embedding_residual, config: dict,
                    step: int = 0, loss_ema: float | None = None) -> bytes:
    """The checkpoint-v2 bytes of the train state (to_safetensors_bytes)."""
    meta = {
        "format_version": str(FORMAT_VERSION),
        "config": json.dumps(config, separators=(",", ":")),
        "step": str(int(step)),
    }
    if loss_ema is not None:  # f32 Display: shortest round-trip decimal, no exponent
        meta["loss_ema"] = np.format_float_positional(np.float32(loss_ema), unique=True,
                                                      trim="-")
    return st_save(state_tensors(arena, layout, embedding, embedding_residual), metadata=meta)


def _metadata(data: bytes) -> dict:
    n = int.from_bytes(data[:8], "little")
    header = json.loads(data[8: 8 + n])
    return header.get("__metadata__") or {}


def load_checkpoint(data: bytes, layout, arena_bytes: int, shape=None):
    """Parses checkpoint-v2 bytes (from_safetensors_bytes) into
    (arena uint8 with derived tensors zeroed, embedding f16 bits, embedding
    carry, metadata {"format_version", "config", "step", "loss_ema"}).
    Missing `.residual` carries load as zeros, as `install_storage` leaves
    them (src/model.rs:3799-3804); a missing latent is an error."""
    meta = _metadata(data)
    if not meta:
        raise ValueError("safetensors checkpoint is missing metadata")
    try:
        version = int(meta.get("format_version", "0"))
    except ValueError:
        version = 0
    if version != FORMAT_VERSION:
        raise ValueError(f"checkpoint format_version {version}: only v2 Heron checkpoints load "
                         "(Hyena checkpoints (v1) are not supported)")
    if "config" not in meta:
        raise ValueError("safetensors checkpoint is missing config")
    config = json.loads(meta["config"])
    if shape is not None:
        dim_ffn = config.get("dim_ffn", 0) or 4 * config["d_model"]
        got = (config["d_model"], config["n_layers"], dim_ffn, config["vocab_size"])
        want = (shape.d_model, shape.n_layers, shape.dim_ffn, shape.vocab)
        if got != want:
            raise ValueError(f"checkpoint config {got} does not match the trainer {want}")
    tensors = st_load(data)
    if any(n.startswith("hybrid_blocks.") for n in tensors):
        raise ValueError("hybrid (rosa_rwkv7) checkpoints do not load into a Heron trainer")
    arena = np.zeros(arena_bytes, np.uint8)
    for name, dt, count, off, derived in layout:
        if derived:
            continue
        t = tensors.get(name)
        if t is None:
            if name.endswith(".residual"):
                continue
            raise ValueError(f"checkpoint tensor {name} is missing")
        if t.dtype != _NP[dt] or t.ndim != 1 or t.size != count:
            raise ValueError(f"checkpoint tensor {name}: {t.dtype} {t.shape}, expected "
                             f"{np.dtype(_NP[dt])} ({count},)")
        arena[off: off + t.nbytes] = t.view(np.uint8)
    emb = tensors.get("embedding")
    if emb is None or emb.dtype != np.float16:
        raise ValueError("checkpoint tensor embedding is missing or not F16")
    emb_res = tensors.get("embedding.residual")
    if emb_res is None:
        emb_res = np.zeros(emb.size, np.float32)
    step = int(meta.get("step", "0"))
    loss_ema = float(meta["loss_ema"]) if "loss_ema" in meta else None
    return arena, emb.view(np.uint16), emb_res.astype(np.float32), {
        "format_version": version, "config": config, "step": step, "loss_ema": loss_ema}
