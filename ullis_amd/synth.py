"""Seeded synthetic parameters and inputs for the benchmark configurations.

Distributions follow the configs the benchmark is quoted on: BinaryConnect
latents ~U[-0.01, 0.01] with the sign bits derived from them (latent >= 0 is +1,
src/model.rs:878-884), FP16 row scales ~U[0.005, 0.02], biases ~N(0, 0.01),
CMix value weights ~N(0, 0.02), ROSA e ~N(0, 0.1), hidden / embedding rows
~N(0, 1), targets uniform over the vocabulary, ROSA indices Bernoulli(0.5).
LayerNorm gamma = 1, beta = 0 unless `random_ln`. Time-shift mixes ~U[0, 1]
(the reference initialises them to 0, which would hide the shift entirely).
Generator: numpy PCG64 seeded with the base seed (7) and a per-tensor salt.
"""
from __future__ import annotations

import zlib

import numpy as np

F16, F32, U32 = 1, 2, 3


def rng_for(seed: int, salt: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(salt.encode())])


def f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def pack_bits(plus: np.ndarray) -> np.ndarray:
    """LSB-first u32 words of a boolean vector (src/model.rs:158-166)."""
    plus = np.asarray(plus, dtype=bool).ravel()
    n_words = (plus.size + 31) // 32
    padded = np.zeros(n_words * 32, dtype=bool)
    padded[: plus.size] = plus
    return np.packbits(padded, bitorder="little").view("<u4").astype(np.uint32)


def unpack_bits(words: np.ndarray, n: int) -> np.ndarray:
    w = np.ascontiguousarray(words, dtype="<u4")
    return np.unpackbits(w.view(np.uint8), bitorder="little")[:n].astype(bool)


def latent_plus(latent_bits: np.ndarray) -> np.ndarray:
    return np.asarray(latent_bits, np.uint16).view(np.float16).astype(np.float32) >= 0.0


def heron_arena(layout, total: int, dims, seed: int = 7, random_ln: bool = False,
                mix_range=(0.0, 1.0)) -> np.ndarray:
    """Fills a parameter arena (uint8) described by `layout` rows of
    (name, dtype, count, offset, derived)."""
    arena = np.zeros(total, dtype=np.uint8)
    by_name = {row[0]: row for row in layout}

    def view(name):
        _, dt, count, off, _ = by_name[name]
        np_dt = {F16: np.uint16, F32: np.float32, U32: np.uint32}[dt]
        return arena[off: off + count * np.dtype(np_dt).itemsize].view(np_dt)

    for name, dt, count, off, derived in layout:
        if derived or name.endswith(".residual") or name.endswith(".bits"):
            continue
        r = rng_for(seed, name)
        v = view(name)
        if name.endswith(".latent"):
            v[:] = f16(r.uniform(-0.01, 0.01, count))
        elif name.endswith(".scale"):
            v[:] = f16(r.uniform(0.005, 0.02, count))
        elif name.endswith(".bias") and (".ln" in name or name.startswith("ln_out")):
            v[:] = f16(r.normal(0.0, 0.1, count) if random_ln else np.zeros(count))
        elif name.endswith(".weight"):
            v[:] = f16(r.uniform(0.5, 1.5, count) if random_ln else np.ones(count))
        elif name.endswith(".bias"):
            v[:] = f16(r.normal(0.0, 0.01, count))
        elif name.endswith(".e"):
            v[:] = f16(r.normal(0.0, 0.1, count))
        elif name.endswith(".value"):
            v[:] = f16(r.normal(0.0, 0.02, count))
        elif name.endswith((".x_q", ".x_k", ".x_v")):
            v[:] = f16(r.uniform(mix_range[0], mix_range[1], count))
        else:
            raise KeyError(f"no synthetic rule for {name}")
    # sign bits from latents; bits_t is derived on the device
    for name, dt, count, off, derived in layout:
        if name.endswith(".bits"):
            prefix = name[: -len(".bits")]
            view(name)[:] = pack_bits(latent_plus(view(prefix + ".latent")))
    return arena


def tensor_view(arena: np.ndarray, layout, name: str) -> np.ndarray:
    for n, dt, count, off, _ in layout:
        if n == name:
            np_dt = {F16: np.uint16, F32: np.float32, U32: np.uint32}[dt]
            return arena[off: off + count * np.dtype(np_dt).itemsize].view(np_dt)
    raise KeyError(name)


def step_inputs(rows: int, d: int, vocab: int, n_layers: int, batch: int, time: int,
                seed: int = 7):
    """x_emb fp32 [rows, d], labels u32 [rows], rosa_idx u8 [L][batch][d][time]."""
    x = rng_for(seed, "x_emb").standard_normal(rows * d).astype(np.float32)
    labels = rng_for(seed, "labels").integers(0, vocab, rows, dtype=np.uint32)
    idx = rng_for(seed, "rosa_idx").integers(0, 2, n_layers * batch * d * time, dtype=np.uint8)
    return x, labels, idx
