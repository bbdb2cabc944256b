"""The Heron train step driven block by block through the C ABI, the way the
reference's model code drives its Metal runtime.

`UllisHeron::train_step_on` (src/model.rs:2827-3025) with
`Some(MetalTrainRuntime)` keeps the residual stream on the host, calls one
runtime method per block half (`rosa_block_forward`, `cmix_block_forward`,
`packed_head_train_sgd`, `cmix_block_backward_sgd`, `rosa_o_stop_grad_sgd`,
`layer_norm(_backward)`), adds the block outputs on the host, and steps the
small vectors (scales, biases, `e`, mixes, LayerNorm affine) from the
gradients those methods return. `HeronBlockStep` does the same over
libullis_hip's block entry points, with the parameters resident in one device
arena (the layout of include/ullis_heron_layout.h) and the suffix automaton
supplied by the caller between the Q/K/V projections and O (`sam`), as the
reference runs `rosa_qkv_batch_packed_channel_major` on the CPU there
(src/metal.rs:1484-1490).

The fused device step (`HeronTrainer`, ullis_hip_heron_step) computes the
same step in one call; this path exists for callers that need the per-block
boundary (the automaton hand-off) and as its cross-check.
"""
from __future__ import annotations

from typing import Callable

import numpy as np

from .runtime import F16, DeviceBuffer, HeronShape, HipRuntime, heron_layout

# sam(layer, q_plane, k_plane, v_plane) -> idx, u8 channel-major [batch][d][time]
Sam = Callable[[int, np.ndarray, np.ndarray, np.ndarray], np.ndarray]


class HeronBlockStep:
    """Per-block Heron train step over a device parameter arena."""

    def __init__(self, rt: HipRuntime, shape: HeronShape):
        self.rt = rt
        self.lib = rt.lib
        self.shape = shape
        self.layout, self.arena_bytes = heron_layout(shape.dims(), rt.lib)
        self.arena = rt.buffer(self.arena_bytes)
        self._addr = {name: (self.arena.ptr + off, count)
                      for name, _dt, count, off, _der in self.layout}
        r, d, f = shape.rows, shape.d_model, shape.dim_ffn
        self.cmix_tapes = [rt.buffer(self.lib.ullis_hip_cmix_tape_bytes(r, d, f))
                           for _ in range(shape.n_layers)]
        self.rosa_tapes = [rt.buffer(self.lib.ullis_hip_rosa_tape_bytes(r, d))
                           for _ in range(shape.n_layers)]

    # ------------------------------------------------------------- arena
    def upload_arena(self, arena: np.ndarray):
        a = np.ascontiguousarray(arena, dtype=np.uint8)
        assert a.nbytes == self.arena_bytes
        self.arena.upload(a)
        # derived [in, out] bit transposes from the uploaded bits
        for name, _dt, _count, _off, derived in self.layout:
            if derived:
                prefix = name[: -len(".bits_t")]
                out_f, in_f = self._shape_of(prefix)
                self._call("transpose_bits", self.lib.ullis_hip_transpose_bits(
                    self.rt.ctx, self.p(prefix + ".bits"), out_f, in_f, self.p(name)))

    def download_arena(self) -> np.ndarray:
        return self.arena.download(np.uint8, self.arena_bytes)

    def p(self, name: str) -> int:
        return self._addr[name][0]

    def has(self, name: str) -> bool:
        return name in self._addr

    def _shape_of(self, prefix: str):
        s = self.shape
        if prefix == "head":
            return s.vocab, s.d_model
        if prefix.endswith("ffn.key"):
            return s.dim_ffn, s.d_model
        return s.d_model, s.d_model

    def _call(self, what: str, rc: int):
        self.rt._check(rc, what)

    # ------------------------------------------------------- small steps
    def _clipped_sgd(self, name: str, grad: DeviceBuffer, n: int, lr: float):
        self._call("clipped_sgd_fp16", self.lib.ullis_hip_clipped_sgd_fp16(
            self.rt.ctx, self.p(name), self.p(name + ".residual"), grad.ptr, n, lr))

    def _ln_forward(self, prefix: str, x: DeviceBuffer, y32=None, y16=None):
        s = self.shape
        self._call("layer_norm", self.lib.ullis_hip_layer_norm(
            self.rt.ctx, x.ptr, self.p(prefix + ".weight"), self.p(prefix + ".bias"), s.rows,
            s.d_model, y32.ptr if y32 else None, y16.ptr if y16 else None))

    def _ln_backward_sgd(self, prefix: str, x: DeviceBuffer, gy: DeviceBuffer, lr: float):
        """LayerNorm::backward + apply_clipped_sgd (src/model.rs:278-332): the
        input gradient (device), with weight and bias stepped."""
        s, rt = self.shape, self.rt
        gx = rt.buffer(4 * s.rows * s.d_model)
        gw, gb = rt.buffer(4 * s.d_model), rt.buffer(4 * s.d_model)
        self._call("layer_norm_backward", self.lib.ullis_hip_layer_norm_backward(
            rt.ctx, x.ptr, gy.ptr, self.p(prefix + ".weight"), s.rows, s.d_model, gx.ptr, gw.ptr,
            gb.ptr))
        self._clipped_sgd(prefix + ".weight", gw, s.d_model, lr)
        self._clipped_sgd(prefix + ".bias", gb, s.d_model, lr)
        return gx

    def _host(self, buf: DeviceBuffer) -> np.ndarray:
        return buf.download(np.float32, self.shape.rows * self.shape.d_model)

    def _dev(self, a: np.ndarray) -> DeviceBuffer:
        return self.rt.put(np.ascontiguousarray(a, np.float32))

    # ------------------------------------------------------------- step
    def step(self, x_emb: np.ndarray, labels: np.ndarray, ignore_id: int, lr: float,
             sam: Sam) -> dict:
        """One train step from the gathered embedding rows (the embedding
        gather / scatter-SGD stay with the caller, src/model.rs:2866-2873,
        2986-2993). Returns the loss statistics, row losses, the embedding-row
        gradient and the Q/K/V sign bit-planes of each layer."""
        s, rt, lib = self.shape, self.rt, self.lib
        if not (lr > 0.0 and np.isfinite(lr)) or s.time < 2:
            raise ValueError("train step requires a positive learning rate and time >= 2")
        R, D, F, V, L, B, T = (s.rows, s.d_model, s.dim_ffn, s.vocab, s.n_layers, s.batch,
                               s.time)
        ste = float(T - 1)  # binaryconnect_ste_scale(time - 1), src/model.rs:554-556
        words = (R * D + 31) // 32
        x = np.ascontiguousarray(x_emb, np.float32).reshape(-1).copy()
        tapes, planes = [], []

        # ------------------------------------------------------- forward
        for l in range(L):
            blk = f"blocks.{l}"
            ln0_in = None
            if self.has(f"{blk}.ln0.weight"):
                ln0_in = self._dev(x)
                y = rt.buffer(4 * R * D)
                self._ln_forward(f"{blk}.ln0", ln0_in, y32=y)
                x = self._host(y)
            # ROSA block (RwkvRosaQkv1Bit::forward_tape, src/model.rs:1354-1410)
            xd = self._dev(x)
            rosa_in = rt.buffer(2 * R * D)
            self._ln_forward(f"{blk}.ln3", xd, y16=rosa_in)
            qp, kp, vp = (rt.buffer(4 * words) for _ in range(3))
            r = f"{blk}.rosa"
            self._call("rosa_qkv_forward", lib.ullis_hip_rosa_qkv_forward(
                rt.ctx, rosa_in.ptr, F16, self.p(f"{r}.x_q"), self.p(f"{r}.x_k"),
                self.p(f"{r}.x_v"), self.p(f"{r}.q.bits"), self.p(f"{r}.q.scale"),
                self.p(f"{r}.q.bias"), self.p(f"{r}.k.bits"), self.p(f"{r}.k.scale"),
                self.p(f"{r}.k.bias"), self.p(f"{r}.v.bits"), self.p(f"{r}.v.scale"),
                self.p(f"{r}.v.bias"), B, T, D, qp.ptr, kp.ptr, vp.ptr))
            pl = tuple(b.download(np.uint32, words) for b in (qp, kp, vp))
            planes.append(pl)
            idx = np.ascontiguousarray(sam(l, *pl), np.uint8)
            if idx.size != R * D:
                raise ValueError("sam returned idx of the wrong size")
            didx = rt.put(idx)
            out = rt.buffer(4 * R * D)
            self._call("rosa_out_forward", lib.ullis_hip_rosa_out_forward(
                rt.ctx, didx.ptr, self.p(f"{r}.e"), self.p(f"{r}.o.bits"), self.p(f"{r}.o.scale"),
                self.p(f"{r}.o.bias"), B, T, D, out.ptr, self.rosa_tapes[l].ptr))
            x = x + self._host(out)
            after_rosa = self._dev(x)
            # CMix block (src/model.rs:1018-1078)
            ln2 = rt.buffer(2 * R * D)
            self._ln_forward(f"{blk}.ln2", after_rosa, y16=ln2)
            out = rt.buffer(4 * R * D)
            c = f"{blk}.ffn"
            self._call("cmix_block_forward", lib.ullis_hip_cmix_block_forward(
                rt.ctx, ln2.ptr, F16, self.p(f"{c}.x_k"), self.p(f"{c}.key.bits"),
                self.p(f"{c}.key.scale"), self.p(f"{c}.value"), B, T, D, F, out.ptr,
                self.cmix_tapes[l].ptr))
            x = x + self._host(out)
            tapes.append((ln0_in, after_rosa))
        pre_ln_out = self._dev(x)
        hidden16 = rt.buffer(2 * R * D)
        self._ln_forward("ln_out", pre_ln_out, y16=hidden16)

        # ------------------------------------------------ head + CE (apply_head_ce)
        dl = rt.put(np.ascontiguousarray(labels, np.uint32))
        row_loss, stats = rt.buffer(4 * R), rt.buffer(16)
        g_hidden = rt.buffer(4 * R * D)
        g_scale, g_bias = rt.buffer(4 * V), rt.buffer(4 * V)
        self._call("packed_head_train_sgd", lib.ullis_hip_packed_head_train_sgd(
            rt.ctx, hidden16.ptr, self.p("head.bits"), self.p("head.bits_t"), self.p("head.scale"),
            self.p("head.bias"), self.p("head.latent"), self.p("head.latent.residual"),
            self.p("head.scale.residual"), self.p("head.bias.residual"), dl.ptr, R, T, D, V, 1,
            ignore_id, lr, ste, row_loss.ptr, stats.ptr, g_hidden.ptr, g_scale.ptr, g_bias.ptr,
            None, None))
        g_x = self._ln_backward_sgd("ln_out", pre_ln_out, g_hidden, lr)

        # ------------------------------------------------------ backward
        for l in reversed(range(L)):
            blk = f"blocks.{l}"
            ln0_in, after_rosa = tapes[l]
            c = f"{blk}.ffn"
            g_ln2_out = rt.buffer(4 * R * D)
            g_mix, g_key_scale = rt.buffer(4 * D), rt.buffer(4 * F)
            self._call("cmix_block_backward_sgd", lib.ullis_hip_cmix_block_backward_sgd(
                rt.ctx, self.cmix_tapes[l].ptr, g_x.ptr, self.p(f"{c}.x_k"),
                self.p(f"{c}.key.bits"), self.p(f"{c}.key.bits_t"), self.p(f"{c}.key.scale"),
                self.p(f"{c}.key.latent"), self.p(f"{c}.key.latent.residual"),
                self.p(f"{c}.value"), self.p(f"{c}.value.residual"), B, T, D, F, lr, ste,
                g_ln2_out.ptr, g_mix.ptr, g_key_scale.ptr))
            self._clipped_sgd(f"{c}.key.scale", g_key_scale, F, lr)
            self._clipped_sgd(f"{c}.x_k", g_mix, D, lr)
            g_ln2_in = self._ln_backward_sgd(f"{blk}.ln2", after_rosa, g_ln2_out, lr)
            g_x = self._dev(self._host(g_x) + self._host(g_ln2_in))
            r = f"{blk}.rosa"
            g_e, g_os, g_ob = rt.buffer(4 * D), rt.buffer(4 * D), rt.buffer(4 * D)
            self._call("rosa_o_stop_grad_sgd", lib.ullis_hip_rosa_o_stop_grad_sgd(
                rt.ctx, self.rosa_tapes[l].ptr, g_x.ptr, self.p(f"{r}.o.bits"),
                self.p(f"{r}.o.bits_t"), self.p(f"{r}.o.scale"), self.p(f"{r}.o.latent"),
                self.p(f"{r}.o.latent.residual"), R, D, lr, ste, g_e.ptr, g_os.ptr, g_ob.ptr))
            self._clipped_sgd(f"{r}.o.scale", g_os, D, lr)
            self._clipped_sgd(f"{r}.o.bias", g_ob, D, lr)
            self._clipped_sgd(f"{r}.e", g_e, D, lr)
            if ln0_in is not None:
                g_x = self._ln_backward_sgd(f"{blk}.ln0", ln0_in, g_x, lr)
        st = stats.download(np.float32, 4)
        return {
            "mean_loss": float(st[0]), "n_valid": int(st[1]), "gradient_scale": float(st[2]),
            "stats": st, "row_loss": row_loss.download(np.float32, R),
            "g_emb": self._host(g_x), "qkv_planes": planes,
        }

    def close(self):
        for b in [self.arena, *self.cmix_tapes, *self.rosa_tapes]:
            b.free()
