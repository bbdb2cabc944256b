"""CPU checks of the drop-in boundary: the C-ABI library builds, loads and
exports every symbol include/ullis_hip.h declares; its arena layout agrees
with the oracle's; argument validation fails loudly without touching a GPU."""
import ctypes as C
import subprocess

import numpy as np

from ullis_amd import _lib
from ullis_amd.runtime import heron_layout
from oracle import cpu_ref as o


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)
    assert lib.ullis_hip_version() == 1


def test_layout_matches_oracle_and_checkpoint_names():
    dims = _lib.HeronDims(64, 3, 256, 1000)
    lay, total = heron_layout(dims)
    odims = o.HeronDims(64, 3, 256, 1000)
    olay, ototal = o.heron_layout(odims)
    assert lay == olay and total == ototal
    names = {row[0] for row in lay}
    for n in ["ln_out.weight", "ln_out.bias.residual", "head.bits", "head.scale", "head.bias",
              "head.latent", "head.latent.residual", "head.scale.residual", "blocks.0.ln0.weight",
              "blocks.2.ln2.bias", "blocks.1.rosa.x_q", "blocks.1.rosa.e", "blocks.1.rosa.o.bits",
              "blocks.1.rosa.o.bias", "blocks.2.ffn.key.bits", "blocks.2.ffn.value",
              "blocks.2.ffn.value.residual"]:
        assert n in names, n
    assert "blocks.1.ln0.weight" not in names and "blocks.0.ffn.key.bias" not in names
    derived = {row[0] for row in lay if row[4]}
    assert derived == {"head.bits_t"} | {f"blocks.{i}.{p}.bits_t" for i in range(3)
                                         for p in ["rosa.o", "ffn.key"]}
    for name, dt, count, off, _ in lay:
        assert off % 256 == 0
        if name.endswith(".bits") or name.endswith(".bits_t"):
            assert dt == 3


def test_null_context_is_rejected_without_a_gpu():
    lib = _lib.load()
    rc = lib.ullis_hip_binary_linear(None, None, 1, None, None, None, 1, 1, 1, None, None)
    assert rc == -1
    assert lib.ullis_hip_sync(None) == -1
    assert lib.ullis_hip_heron_step(None, None, None, 0, 0.01, None, None, None, None, None,
                                    None) == -1
    assert lib.ullis_hip_heron_causal_loss(None, None, None, 0, None, None, 0, None) == -1


class _FakeLib:
    """Records the C-ABI calls of the runtime's object lifecycle (no GPU)."""

    def __init__(self):
        self.calls = []

    def ullis_hip_malloc(self, ctx, nbytes, out):
        out._obj.value = 4096
        self.calls.append(("malloc", ctx))
        return 0

    def ullis_hip_free(self, ctx, ptr):
        self.calls.append(("free", ctx, ptr))
        return 0

    def ullis_hip_heron_destroy(self, h):
        self.calls.append(("heron_destroy", h))

    def ullis_hip_destroy(self, ctx):
        self.calls.append(("destroy", ctx))


def test_runtime_close_frees_dependents_first_and_leaves_them_inert():
    """Objects that outlive HipRuntime.close (a traceback holding a trainer)
    must not call into the destroyed context."""
    import weakref

    from ullis_amd.runtime import DeviceBuffer, HeronTrainer, HipRuntime

    rt = HipRuntime.__new__(HipRuntime)
    rt.lib, rt.ctx, rt._owned = _FakeLib(), 77, weakref.WeakSet()
    buf = DeviceBuffer(rt, 64)
    tr = HeronTrainer.__new__(HeronTrainer)
    tr.rt, tr.h = rt, 99
    rt._own(tr)
    rt.close()
    assert rt.lib.calls[-1] == ("destroy", 77)
    assert ("free", 77, 4096) in rt.lib.calls and ("heron_destroy", 99) in rt.lib.calls
    n = len(rt.lib.calls)
    buf.free()
    tr.close()
    del buf, tr
    assert len(rt.lib.calls) == n
