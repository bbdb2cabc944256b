"""Python convenience layer over the C ABI (tests, bench, smoke).

`HipRuntime` mirrors the host-slice methods of the reference's `MetalRuntime`
(src/metal.rs): numpy arrays in, numpy arrays out, one synchronous round trip
per call. It exists for parity tests and scripts; the device-resident API is
the C ABI itself (`DeviceBuffer` + `lib` calls), which is what `HeronTrainer`
and bench.py use. Shape rules and error texts come from the library.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from . import _lib

F16 = _lib.F16
F32 = _lib.F32


class HipError(RuntimeError):
    pass


class DeviceBuffer:
    """An owned device allocation."""

    def __init__(self, rt: "HipRuntime", nbytes: int):
        self.rt = rt
        self.nbytes = int(nbytes)
        ptr = C.c_void_p()
        rt._check(rt.lib.ullis_hip_malloc(rt.ctx, max(self.nbytes, 4), C.byref(ptr)), "malloc")
        self.ptr = ptr.value
        rt._own(self)

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        if a.nbytes > self.nbytes:
            raise ValueError("upload larger than buffer")
        self.rt._check(
            self.rt.lib.ullis_hip_upload(self.rt.ctx, self.ptr, a.ctypes.data, a.nbytes), "upload")
        return self

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            self.rt._check(self.rt.lib.ullis_hip_download(
                self.rt.ctx, out.ctypes.data, self.ptr + offset, out.nbytes), "download")
        return out

    def free(self):
        # after the runtime is closed the allocation is already gone
        if self.ptr and self.rt.ctx:
            self.rt.lib.ullis_hip_free(self.rt.ctx, self.ptr)
        self.ptr = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def f16_bits(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_values(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


class HipRuntime:
    """MetalRuntime-shaped host API over libullis_hip (src/metal.rs:466-3510)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        ctx = C.c_void_p()
        rc = self.lib.ullis_hip_create(device, C.byref(ctx))
        if rc != 0:
            raise HipError(f"ullis_hip_create failed ({rc}): no usable HIP device {device}")
        self.ctx = ctx.value
        self._owned = weakref.WeakSet()  # live buffers and trainers on this context

    def _own(self, obj):
        self._owned.add(obj)

    def close(self):
        """Frees every live buffer and trainer of this runtime, then the context;
        objects that outlive it (e.g. held by a traceback) become inert."""
        if self.ctx:
            for obj in list(self._owned):
                obj.close()
            self.lib.ullis_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str):
        if rc != 0:
            msg = self.lib.ullis_hip_last_error(self.ctx)
            raise HipError(f"{what}: {msg.decode() if msg else ''} (status {rc})")

    def sync(self):
        self._check(self.lib.ullis_hip_sync(self.ctx), "sync")

    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def put(self, arr) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return DeviceBuffer(self, a.nbytes).upload(a)

    def zeros(self, dtype, count: int) -> DeviceBuffer:
        return self.put(np.zeros(count, dtype=dtype))

    # ------------------------------------------------------------ unit ops
    def layer_norm(self, x, weight_bits, bias_bits, rows, channels, out_dtype=np.float32):
        dx = self.put(np.asarray(x, np.float32))
        dw = self.put(np.asarray(weight_bits, np.uint16))
        db = self.put(np.asarray(bias_bits, np.uint16))
        n = rows * channels
        if out_dtype == np.float16:
            y = self.buffer(2 * n)
            self._check(self.lib.ullis_hip_layer_norm(self.ctx, dx.ptr, dw.ptr, db.ptr, rows,
                                                      channels, None, y.ptr), "layer_norm")
            return y.download(np.uint16, n)
        y = self.buffer(4 * n)
        self._check(self.lib.ullis_hip_layer_norm(self.ctx, dx.ptr, dw.ptr, db.ptr, rows,
                                                  channels, y.ptr, None), "layer_norm")
        return y.download(np.float32, n)

    def layer_norm_backward(self, x, gy, weight_bits, rows, channels):
        dx = self.put(np.asarray(x, np.float32))
        dg = self.put(np.asarray(gy, np.float32))
        dw = self.put(np.asarray(weight_bits, np.uint16))
        gx, gw, gb = self.buffer(4 * rows * channels), self.buffer(4 * channels), self.buffer(4 * channels)
        self._check(self.lib.ullis_hip_layer_norm_backward(
            self.ctx, dx.ptr, dg.ptr, dw.ptr, rows, channels, gx.ptr, gw.ptr, gb.ptr),
            "layer_norm_backward")
        return (gx.download(np.float32, rows * channels), gw.download(np.float32, channels),
                gb.download(np.float32, channels))

    def layer_norm_backward_static_dev(self, x: DeviceBuffer, gy: DeviceBuffer,
                                       weight: DeviceBuffer, rows, channels, gx: DeviceBuffer,
                                       gw: DeviceBuffer | None, gb: DeviceBuffer | None):
        """ullis_hip_layer_norm_backward_static on device buffers (allocates nothing)."""
        self._check(self.lib.ullis_hip_layer_norm_backward_static(
            self.ctx, x.ptr, gy.ptr, weight.ptr, rows, channels, gx.ptr,
            gw.ptr if gw else None, gb.ptr if gb else None), "layer_norm_backward_static")

    def binary_linear(self, x, bits, scale_bits, bias_bits, rows, in_f, out_f, x_dtype=F16,
                      out_dtype=np.float32):
        xa = np.asarray(x)
        if x_dtype == F16:
            dx = self.put(xa.astype(np.uint16) if xa.dtype == np.uint16 else f16_bits(xa))
        else:
            dx = self.put(xa.astype(np.float32))
        db = self.put(np.asarray(bits, np.uint32))
        ds = self.put(np.asarray(scale_bits, np.uint16))
        dbias = self.put(np.asarray(bias_bits, np.uint16)) if bias_bits is not None else None
        n = rows * out_f
        y = self.buffer((2 if out_dtype == np.float16 else 4) * n)
        self._check(self.lib.ullis_hip_binary_linear(
            self.ctx, dx.ptr, x_dtype, db.ptr, ds.ptr, dbias.ptr if dbias else None, rows, in_f,
            out_f, None if out_dtype == np.float16 else y.ptr,
            y.ptr if out_dtype == np.float16 else None), "binary_linear")
        return y.download(np.uint16 if out_dtype == np.float16 else np.float32, n)

    def binary_linear_backward(self, x16_bits, gy, bits, scale_bits, has_bias, rows, in_f, out_f):
        dx = self.put(np.asarray(x16_bits, np.uint16))
        dg = self.put(np.asarray(gy, np.float32))
        db = self.put(np.asarray(bits, np.uint32))
        ds = self.put(np.asarray(scale_bits, np.uint16))
        gx = self.buffer(4 * rows * in_f)
        gw = self.buffer(4 * out_f * in_f)
        gs = self.buffer(4 * out_f)
        gb = self.buffer(4 * out_f)
        self._check(self.lib.ullis_hip_binary_linear_backward(
            self.ctx, dx.ptr, dg.ptr, db.ptr, ds.ptr, int(has_bias), rows, in_f, out_f, gx.ptr,
            gw.ptr, gs.ptr, gb.ptr), "binary_linear_backward")
        return {
            "input_gradient": gx.download(np.float32, rows * in_f),
            "weight_gradient": gw.download(np.float32, out_f * in_f),
            "scale_gradient": gs.download(np.float32, out_f),
            "bias_gradient": gb.download(np.float32, out_f) if has_bias else None,
        }

    def apply_latent_sgd(self, latent_bits, residual, gradient, out_f, in_f, lr, ste):
        dl = self.put(np.asarray(latent_bits, np.uint16))
        dr = self.put(np.asarray(residual, np.float32))
        dg = self.put(np.asarray(gradient, np.float32))
        words = (out_f * in_f + 31) // 32
        bits = self.buffer(4 * words)
        bits_t = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_apply_latent_sgd(
            self.ctx, dl.ptr, dr.ptr, dg.ptr, out_f, in_f, lr, ste, bits.ptr, bits_t.ptr),
            "apply_latent_sgd")
        n = out_f * in_f
        return (dl.download(np.uint16, n), dr.download(np.float32, n),
                bits.download(np.uint32, words), bits_t.download(np.uint32, words))

    def fp16_linear(self, x, w_bits, rows, in_f, out_f, x_dtype=F16):
        xa = np.asarray(x)
        dx = self.put(f16_bits(xa) if x_dtype == F16 and xa.dtype != np.uint16 else
                      (xa if x_dtype == F16 else xa.astype(np.float32)))
        dw = self.put(np.asarray(w_bits, np.uint16))
        y = self.buffer(4 * rows * out_f)
        self._check(self.lib.ullis_hip_fp16_linear(self.ctx, dx.ptr, x_dtype, dw.ptr, rows, in_f,
                                                   out_f, y.ptr, None), "fp16_linear")
        return y.download(np.float32, rows * out_f)

    def fp16_linear_backward(self, x16_bits, gy, w_bits, rows, in_f, out_f):
        dx = self.put(np.asarray(x16_bits, np.uint16))
        dg = self.put(np.asarray(gy, np.float32))
        dw = self.put(np.asarray(w_bits, np.uint16))
        gx = self.buffer(4 * rows * in_f)
        gw = self.buffer(4 * out_f * in_f)
        self._check(self.lib.ullis_hip_fp16_linear_backward(
            self.ctx, dx.ptr, dg.ptr, dw.ptr, rows, in_f, out_f, gx.ptr, gw.ptr),
            "fp16_linear_backward")
        return gx.download(np.float32, rows * in_f), gw.download(np.float32, out_f * in_f)

    def clipped_sgd_fp16(self, params, residual, gradient, lr):
        p, r, g = self.put(np.asarray(params, np.uint16)), self.put(np.asarray(residual, np.float32)), \
            self.put(np.asarray(gradient, np.float32))
        n = len(params)
        self._check(self.lib.ullis_hip_clipped_sgd_fp16(self.ctx, p.ptr, r.ptr, g.ptr, n, lr),
                    "clipped_sgd_fp16")
        return p.download(np.uint16, n), r.download(np.float32, n)

    def binaryconnect_sgd_fp16(self, params, residual, gradient, lr):
        p, r, g = self.put(np.asarray(params, np.uint16)), self.put(np.asarray(residual, np.float32)), \
            self.put(np.asarray(gradient, np.float32))
        n = len(params)
        self._check(self.lib.ullis_hip_binaryconnect_sgd_fp16(self.ctx, p.ptr, r.ptr, g.ptr, n, lr),
                    "binaryconnect_sgd_fp16")
        return p.download(np.uint16, n), r.download(np.float32, n)

    def sign_pack_bits(self, x):
        xa = np.asarray(x, np.float32)
        dx = self.put(xa)
        words = (xa.size + 31) // 32
        b = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_sign_pack_bits(self.ctx, dx.ptr, xa.size, b.ptr),
                    "sign_pack_bits")
        return b.download(np.uint32, words)

    def transpose_bits(self, bits, out_f, in_f):
        db = self.put(np.asarray(bits, np.uint32))
        words = (out_f * in_f + 31) // 32
        bt = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_transpose_bits(self.ctx, db.ptr, out_f, in_f, bt.ptr),
                    "transpose_bits")
        return bt.download(np.uint32, words)

    def packed_head_train_sgd(self, hidden16_bits, bits, scale_bits, bias_bits, latent_bits,
                              latent_res, scale_res, bias_res, targets, rows, time, d, vocab,
                              ignore_id, lr, ste, want_g_w=False, horizon=1):
        """Head + streamed CE (+ update when lr > 0). Returns a dict of host arrays;
        "invalid" counts targets >= vocab other than ignore_id (left out of the
        loss and the gradient)."""
        words = (vocab * d + 31) // 32
        dh = self.put(np.asarray(hidden16_bits, np.uint16))
        db = self.put(np.asarray(bits, np.uint32))
        dbt = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_transpose_bits(self.ctx, db.ptr, vocab, d, dbt.ptr),
                    "transpose_bits")
        ds = self.put(np.asarray(scale_bits, np.uint16))
        dbias = self.put(np.asarray(bias_bits, np.uint16)) if bias_bits is not None else None
        dl = self.put(np.asarray(latent_bits, np.uint16))
        dlr = self.put(np.asarray(latent_res, np.float32))
        dsr = self.put(np.asarray(scale_res, np.float32))
        dbr = self.put(np.asarray(bias_res, np.float32)) if bias_bits is not None else None
        dt = self.put(np.asarray(targets, np.uint32))
        row_loss = self.buffer(4 * rows)
        stats = self.buffer(16)
        g_hidden = self.buffer(4 * rows * d)
        g_scale = self.buffer(4 * vocab)
        g_bias = self.buffer(4 * vocab)
        g_w = self.buffer(4 * vocab * d) if want_g_w else None
        invalid = self.zeros(np.uint32, 1)
        self._check(self.lib.ullis_hip_packed_head_train_sgd(
            self.ctx, dh.ptr, db.ptr, dbt.ptr, ds.ptr, dbias.ptr if dbias else None, dl.ptr,
            dlr.ptr, dsr.ptr, dbr.ptr if dbr else None, dt.ptr, rows, time, d, vocab, horizon,
            ignore_id, lr, ste, row_loss.ptr, stats.ptr, g_hidden.ptr, g_scale.ptr, g_bias.ptr,
            g_w.ptr if g_w else None, invalid.ptr), "packed_head_train_sgd")
        st = stats.download(np.float32, 4)
        out = {
            "invalid": int(invalid.download(np.uint32, 1)[0]),
            "mean_loss": float(st[0]), "n_valid": int(st[1]), "gradient_scale": float(st[2]),
            "row_loss": row_loss.download(np.float32, rows),
            "hidden_gradient": g_hidden.download(np.float32, rows * d),
            "scale_gradient": g_scale.download(np.float32, vocab),
            "bias_gradient": g_bias.download(np.float32, vocab),
            "next_bits": db.download(np.uint32, words),
            "next_bits_t": dbt.download(np.uint32, words),
            "next_latent": dl.download(np.uint16, vocab * d),
            "next_residual": dlr.download(np.float32, vocab * d),
            "next_scale": ds.download(np.uint16, vocab),
            "next_scale_residual": dsr.download(np.float32, vocab),
        }
        if dbias is not None:
            out["next_bias"] = dbias.download(np.uint16, vocab)
            out["next_bias_residual"] = dbr.download(np.float32, vocab)
        if g_w is not None:
            out["weight_gradient"] = g_w.download(np.float32, vocab * d)
        return out

    # ------------------------------------------------------------ embedding
    def embedding_gather(self, table, tokens, vocab, d):
        """The gather of UllisHeron::train_step_on (src/model.rs:2866-2873): fp32
        rows of the f16 table. An id >= vocab raises, as the reference rejects
        it before the step (the library zeroes the row and counts it)."""
        tok = np.asarray(tokens, np.uint32)
        dt, dk = self.put(np.asarray(table, np.uint16)), self.put(tok)
        x = self.buffer(4 * tok.size * d)
        bad = self.zeros(np.uint32, 1)
        self._check(self.lib.ullis_hip_embedding_gather(self.ctx, dt.ptr, vocab, d, dk.ptr,
                                                        tok.size, x.ptr, bad.ptr),
                    "embedding_gather")
        n_bad = int(bad.download(np.uint32, 1)[0])
        if n_bad:
            raise HipError(f"embedding_gather: {n_bad} token ids >= vocab {vocab}")
        return x.download(np.float32, tok.size * d)

    def embedding_scatter_sgd(self, table, residual, tokens, g, vocab, d, lr):
        """The scatter-SGD of UllisHeron::train_step_on (src/model.rs:2986-2993).
        Returns the stepped (table, residual)."""
        tok = np.asarray(tokens, np.uint32)
        dt, dr = self.put(np.asarray(table, np.uint16)), self.put(np.asarray(residual, np.float32))
        dk, dg = self.put(tok), self.put(np.asarray(g, np.float32))
        self._check(self.lib.ullis_hip_embedding_scatter_sgd(self.ctx, dt.ptr, dr.ptr, vocab, d,
                                                             dk.ptr, tok.size, dg.ptr, lr),
                    "embedding_scatter_sgd")
        return dt.download(np.uint16, vocab * d), dr.download(np.float32, vocab * d)

    # --------------------------------------------------- block-level methods
    def _x16_or_f32(self, x):
        xa = np.asarray(x)
        if xa.dtype == np.uint16:
            return self.put(xa), F16
        return self.put(xa.astype(np.float32)), F32

    def cmix_block_forward(self, x, mix, key_bits, key_scale, value_weight, batch, time,
                           d_model, dim_ffn):
        """MetalRuntime::cmix_block_forward (src/metal.rs:1891). x: fp32 values or
        f16 bits (uint16). Returns {"out", "gpu_tape"}; the tape feeds
        cmix_block_backward_sgd."""
        dx, dt = self._x16_or_f32(x)
        rows = batch * time
        tape = self.buffer(self.lib.ullis_hip_cmix_tape_bytes(rows, d_model, dim_ffn))
        out = self.buffer(4 * rows * d_model)
        ptrs = [self.put(np.asarray(a, t)) for a, t in
                ((mix, np.uint16), (key_bits, np.uint32), (key_scale, np.uint16),
                 (value_weight, np.uint16))]
        self._check(self.lib.ullis_hip_cmix_block_forward(
            self.ctx, dx.ptr, dt, *(p.ptr for p in ptrs), batch, time, d_model, dim_ffn, out.ptr,
            tape.ptr), "cmix_block_forward")
        return {"out": out.download(np.float32, rows * d_model), "gpu_tape": tape}

    def cmix_block_backward_sgd(self, tape, gy, mix, key_bits, key_scale, key_latent,
                                key_residual, value_weight, value_residual, batch, time, d_model,
                                dim_ffn, learning_rate, ste_scale):
        """MetalRuntime::cmix_block_backward_sgd (src/metal.rs:2165); fields of
        CmixBlockBackwardSgd, plus next_key_bits_t."""
        rows = batch * time
        n_key, n_val = dim_ffn * d_model, d_model * dim_ffn
        words = (n_key + 31) // 32
        dg = self.put(np.asarray(gy, np.float32))
        dm = self.put(np.asarray(mix, np.uint16))
        db = self.put(np.asarray(key_bits, np.uint32))
        dbt = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_transpose_bits(self.ctx, db.ptr, dim_ffn, d_model, dbt.ptr),
                    "transpose_bits")
        ds = self.put(np.asarray(key_scale, np.uint16))
        dl = self.put(np.asarray(key_latent, np.uint16))
        dlr = self.put(np.asarray(key_residual, np.float32))
        dv = self.put(np.asarray(value_weight, np.uint16))
        dvr = self.put(np.asarray(value_residual, np.float32))
        g_x, g_mix, g_ks = (self.buffer(4 * rows * d_model), self.buffer(4 * d_model),
                            self.buffer(4 * dim_ffn))
        self._check(self.lib.ullis_hip_cmix_block_backward_sgd(
            self.ctx, tape.ptr, dg.ptr, dm.ptr, db.ptr, dbt.ptr, ds.ptr, dl.ptr, dlr.ptr, dv.ptr,
            dvr.ptr, batch, time, d_model, dim_ffn, learning_rate, ste_scale, g_x.ptr, g_mix.ptr,
            g_ks.ptr), "cmix_block_backward_sgd")
        return {
            "g_x": g_x.download(np.float32, rows * d_model),
            "g_mix": g_mix.download(np.float32, d_model),
            "g_key_scale": g_ks.download(np.float32, dim_ffn),
            "next_key_latent": dl.download(np.uint16, n_key),
            "next_key_residual": dlr.download(np.float32, n_key),
            "next_key_bits": db.download(np.uint32, words),
            "next_key_bits_t": dbt.download(np.uint32, words),
            "next_value_weight": dv.download(np.uint16, n_val),
            "next_value_residual": dvr.download(np.float32, n_val),
        }

    def rosa_block_forward(self, x, mix_q, mix_k, mix_v, q_bits, q_scale, q_bias, k_bits,
                           k_scale, k_bias, v_bits, v_scale, v_bias, e, o_bits, o_scale, o_bias,
                           batch, time, channels, sam):
        """MetalRuntime::rosa_block_forward (src/metal.rs:1334-1511). The suffix
        automaton stays with the caller: sam(q_plane, k_plane, v_plane) returns
        idx, u8 channel-major [batch][channels][time]
        (rosa_qkv_batch_packed_channel_major, src/rosa.rs:486-513). Returns
        {"out", "planes", "idx", "gpu_tape"}."""
        dx, dt = self._x16_or_f32(x)
        rows = batch * time
        words = (rows * channels + 31) // 32
        u16 = lambda a: self.put(np.asarray(a, np.uint16))
        u32 = lambda a: self.put(np.asarray(a, np.uint32))
        mq, mk, mv = u16(mix_q), u16(mix_k), u16(mix_v)
        qb, qs, qbi = u32(q_bits), u16(q_scale), u16(q_bias)
        kb, ks, kbi = u32(k_bits), u16(k_scale), u16(k_bias)
        vb, vs, vbi = u32(v_bits), u16(v_scale), u16(v_bias)
        planes = [self.buffer(4 * words) for _ in range(3)]
        self._check(self.lib.ullis_hip_rosa_qkv_forward(
            self.ctx, dx.ptr, dt, mq.ptr, mk.ptr, mv.ptr, qb.ptr, qs.ptr, qbi.ptr, kb.ptr, ks.ptr,
            kbi.ptr, vb.ptr, vs.ptr, vbi.ptr, batch, time, channels, *(p.ptr for p in planes)),
            "rosa_qkv_forward")
        host_planes = [p.download(np.uint32, words) for p in planes]
        idx = np.ascontiguousarray(sam(*host_planes), np.uint8)
        if idx.size != rows * channels:
            raise ValueError("ROSA idx length mismatch")
        di, de = self.put(idx), u16(e)
        ob, osc, obi = u32(o_bits), u16(o_scale), u16(o_bias)
        tape = self.buffer(self.lib.ullis_hip_rosa_tape_bytes(rows, channels))
        out = self.buffer(4 * rows * channels)
        self._check(self.lib.ullis_hip_rosa_out_forward(
            self.ctx, di.ptr, de.ptr, ob.ptr, osc.ptr, obi.ptr, batch, time, channels, out.ptr,
            tape.ptr), "rosa_out_forward")
        return {"out": out.download(np.float32, rows * channels), "planes": host_planes,
                "idx": idx, "gpu_tape": tape}

    def rosa_o_stop_grad_sgd(self, tape, gy, o_bits, o_scale, latent, residual, rows, channels,
                             learning_rate, ste_scale):
        """MetalRuntime::rosa_o_stop_grad_sgd (src/metal.rs:2409); fields of
        RosaOStopGradSgd, plus next_bits_t."""
        n = channels * channels
        words = (n + 31) // 32
        dg = self.put(np.asarray(gy, np.float32))
        db = self.put(np.asarray(o_bits, np.uint32))
        dbt = self.buffer(4 * words)
        self._check(self.lib.ullis_hip_transpose_bits(self.ctx, db.ptr, channels, channels,
                                                      dbt.ptr), "transpose_bits")
        ds = self.put(np.asarray(o_scale, np.uint16))
        dl = self.put(np.asarray(latent, np.uint16))
        dr = self.put(np.asarray(residual, np.float32))
        g_e, g_s, g_b = (self.buffer(4 * channels) for _ in range(3))
        self._check(self.lib.ullis_hip_rosa_o_stop_grad_sgd(
            self.ctx, tape.ptr, dg.ptr, db.ptr, dbt.ptr, ds.ptr, dl.ptr, dr.ptr, rows, channels,
            learning_rate, ste_scale, g_e.ptr, g_s.ptr, g_b.ptr), "rosa_o_stop_grad_sgd")
        return {
            "e_gradient": g_e.download(np.float32, channels),
            "scale_gradient": g_s.download(np.float32, channels),
            "bias_gradient": g_b.download(np.float32, channels),
            "next_latent": dl.download(np.uint16, n),
            "next_residual": dr.download(np.float32, n),
            "next_bits": db.download(np.uint32, words),
            "next_bits_t": dbt.download(np.uint32, words),
        }


@dataclass
class HeronShape:
    d_model: int
    n_layers: int
    dim_ffn: int
    vocab: int
    batch: int
    time: int

    @property
    def rows(self) -> int:
        return self.batch * self.time

    def dims(self) -> _lib.HeronDims:
        return _lib.HeronDims(self.d_model, self.n_layers, self.dim_ffn, self.vocab)


def heron_layout(dims: _lib.HeronDims, lib=None):
    """[(name, dtype, count, offset, derived)], total bytes - via the library export."""
    lib = lib or _lib.load()
    total = C.c_uint64()
    n = lib.ullis_hip_heron_layout(C.byref(dims), None, 0, C.byref(total))
    arr = (_lib.TensorDesc * n)()
    lib.ullis_hip_heron_layout(C.byref(dims), arr, n, C.byref(total))
    out = [(d.name.decode(), d.dtype, d.count, d.offset, d.derived) for d in arr]
    return out, total.value


class HeronTrainer:
    """Device-resident Heron train step (ullis_hip_heron_*)."""

    def __init__(self, rt: HipRuntime, shape: HeronShape):
        self.rt = rt
        self.shape = shape
        self._dims = shape.dims()
        h = C.c_void_p()
        rt._check(rt.lib.ullis_hip_heron_create(rt.ctx, C.byref(self._dims), shape.batch,
                                                shape.time, C.byref(h)), "heron_create")
        self.h = h.value
        ptr, nbytes = C.c_void_p(), C.c_uint64()
        rt._check(rt.lib.ullis_hip_heron_arena(self.h, C.byref(ptr), C.byref(nbytes)), "arena")
        self.arena_ptr, self.arena_bytes = ptr.value, nbytes.value
        self.layout, total = heron_layout(self._dims, rt.lib)
        assert total == self.arena_bytes
        rt._own(self)

    def close(self):
        if self.h and self.rt.ctx:
            self.rt.lib.ullis_hip_heron_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # probe name -> (id, roofline bound, algorithmic work per launch, kernel label)
    def probes(self):
        s = self.shape
        r, d, f, v = s.rows, s.d_model, s.dim_ffn, s.vocab
        return {
            "key_forward": (1, "mfma", 2.0 * r * d * f, "packed +-1 GEMM: CMix key fwd + ReLU^2"),
            "value_forward": (2, "mfma", 2.0 * r * f * d, "fp16 GEMM: CMix value fwd + residual"),
            "head_ce": (3, "mfma", 3 * 2.0 * r * d * v, "head + streamed CE (whole op)"),
            "value_backward": (4, "mfma", 2 * 2.0 * r * d * f,
                               "paired GEMMs: value dX + ReLU^2 bwd, value dW"),
            "key_backward": (5, "mfma", 2 * 2.0 * r * f * d, "paired GEMMs: packed key dX, key dW"),
            "o_backward": (6, "mfma", 2 * 2.0 * r * d * d, "paired GEMMs: packed O dX, O dW"),
            "ln_forward": (7, "hbm", r * d * (4 + 2 + 2) + 6.0 * d,
                           "LayerNorm fwd (ln2) + time-shift mix"),
            "ln_backward": (8, "hbm", r * d * (4 + 4 + 2 + 8) + 4.0 * d,
                            "mix bwd + LayerNorm bwd rows (ln2, += g_x)"),
        }

    PROBE_EVENTS = 0x100  # ULLIS_HIP_PROBE_EVENTS

    def probe_begin(self, name: str = "key_forward", events: bool = False) -> str:
        """Arms the probe for a launch class; events=True times its GEMM launches by
        kernel-timestamp events (what rocprofv3's kernel trace reports) instead of
        workgroup wall-clock stamps."""
        pid = self.probes()[name][0] | (self.PROBE_EVENTS if events else 0)
        self.rt._check(self.rt.lib.ullis_hip_heron_probe(self.h, pid), "probe")
        return name

    def probe_end(self, name: str) -> dict:
        total, count = C.c_float(), C.c_int()
        self.rt._check(self.rt.lib.ullis_hip_heron_probe_read(self.h, C.byref(total),
                                                              C.byref(count)), "probe read")
        self.rt._check(self.rt.lib.ullis_hip_heron_probe(self.h, 0), "probe off")
        pid, bound, work, label = self.probes()[name]
        return {"name": label, "probe": name, "bound": bound, "work": work,
                "total_ms": total.value, "count": count.value}

    def set_graph(self, enable: bool = True):
        """Replay the step's launches from a captured HIP graph while the
        step's pointers, ignore id and learning rate repeat."""
        self.rt._check(self.rt.lib.ullis_hip_heron_set_graph(self.h, 1 if enable else 0),
                       "set graph")

    def upload_arena(self, arena: np.ndarray):
        a = np.ascontiguousarray(arena, dtype=np.uint8)
        assert a.nbytes == self.arena_bytes
        self.rt._check(self.rt.lib.ullis_hip_upload(self.rt.ctx, self.arena_ptr, a.ctypes.data,
                                                    a.nbytes), "arena upload")
        self.rt._check(self.rt.lib.ullis_hip_heron_refresh_derived(self.h), "refresh derived")

    def download_arena(self) -> np.ndarray:
        out = np.empty(self.arena_bytes, dtype=np.uint8)
        self.rt._check(self.rt.lib.ullis_hip_download(self.rt.ctx, out.ctypes.data,
                                                      self.arena_ptr, out.nbytes), "arena download")
        return out

    def step(self, x_emb: DeviceBuffer, labels: DeviceBuffer, ignore_id: int, lr: float,
             rosa_idx: DeviceBuffer, g_emb: DeviceBuffer, row_loss: DeviceBuffer | None = None,
             stats: DeviceBuffer | None = None, qkv_bits: DeviceBuffer | None = None,
             invalid: DeviceBuffer | None = None):
        """ullis_hip_heron_step; invalid (optional u32) receives the count of labels
        >= vocab other than ignore_id (non-zero: the step changed no parameter)."""
        self.rt._check(self.rt.lib.ullis_hip_heron_step(
            self.h, x_emb.ptr, labels.ptr, ignore_id, lr, rosa_idx.ptr, g_emb.ptr,
            row_loss.ptr if row_loss else None, stats.ptr if stats else None,
            qkv_bits.ptr if qkv_bits else None, invalid.ptr if invalid else None), "heron_step")

    def step_sam(self, sam, x_emb: DeviceBuffer, labels: DeviceBuffer, ignore_id: int, lr: float,
                 g_emb: DeviceBuffer, row_loss: DeviceBuffer | None = None,
                 stats: DeviceBuffer | None = None, qkv_bits: DeviceBuffer | None = None,
                 invalid: DeviceBuffer | None = None, table: DeviceBuffer | None = None,
                 table_res: DeviceBuffer | None = None, tokens: DeviceBuffer | None = None):
        """ullis_hip_heron_step_sam: the step with the suffix automaton driven live.
        sam(layer, planes) gets the layer's Q/K/V sign bit-planes (uint32 [3, words])
        and returns its indices (uint8, channel-major [batch, d, time]). With table /
        table_res / tokens the step runs from token ids (x_emb is then written)."""
        s = self.shape
        words = (s.rows * s.d_model + 31) // 32
        n_idx = s.rows * s.d_model
        failure = []

        def cb(user, layer, planes_p, idx_p):
            try:
                planes = np.ctypeslib.as_array(planes_p, shape=(3 * words,)).reshape(3, words)
                idx = np.ascontiguousarray(sam(int(layer), planes.copy()), np.uint8).ravel()
                if idx.size != n_idx:
                    raise ValueError(f"automaton returned {idx.size} indices, want {n_idx}")
                C.memmove(idx_p, idx.ctypes.data, n_idx)
                return 0
            except Exception as e:  # reported after the call
                failure.append(e)
                return 1

        fn = _lib.SAM_FN(cb)
        rc = self.rt.lib.ullis_hip_heron_step_sam(
            self.h, table.ptr if table else None, table_res.ptr if table_res else None,
            s.vocab if table else 0, tokens.ptr if tokens else None, x_emb.ptr, labels.ptr,
            ignore_id, lr, fn, None, g_emb.ptr, row_loss.ptr if row_loss else None,
            stats.ptr if stats else None, qkv_bits.ptr if qkv_bits else None,
            invalid.ptr if invalid else None)
        if failure:
            raise failure[0]
        self.rt._check(rc, "heron_step_sam")

    PHASES = ("embed", "fwd_ln", "fwd_rosa", "fwd_cmix", "head", "bwd_ln", "bwd_cmix",
              "bwd_rosa", "embed_sgd")

    def phases_begin(self):
        """ullis_hip_heron_phases(h, 1): time the following steps by the
        reference's TrainStepProfile phases (main-stream segments)."""
        self.rt._check(self.rt.lib.ullis_hip_heron_phases(self.h, 1), "phases")

    def phases_end(self) -> dict:
        """The phases' milliseconds per step since phases_begin (averaged over
        the steps), as TrainStepProfile.phases_ms; stops the timing."""
        ms = (C.c_float * len(self.PHASES))()
        steps = C.c_int()
        self.rt._check(self.rt.lib.ullis_hip_heron_phases_read(self.h, ms, C.byref(steps)),
                       "phases read")
        self.rt._check(self.rt.lib.ullis_hip_heron_phases(self.h, 0), "phases")
        n = max(steps.value, 1)
        return {"steps": steps.value,
                "phases_ms": {k: ms[i] / n for i, k in enumerate(self.PHASES)}}

    def decode_init(self, batch: int, graph: bool = True):
        """ullis_hip_heron_decode_init: decode state for `batch` (1..8) new
        sequences; graph=False launches every token eagerly (no graph replay)."""
        self.rt._check(self.rt.lib.ullis_hip_heron_decode_init(self.h, batch, 0 if graph else 1),
                       "decode_init")
        self._decode_batch = batch

    def decode_step(self, table: DeviceBuffer, tokens: DeviceBuffer, logits: DeviceBuffer,
                    next_tokens: DeviceBuffer | None = None, rosa_idx: DeviceBuffer | None = None,
                    sam=None, invalid: DeviceBuffer | None = None):
        """ullis_hip_heron_decode_step: one token per sequence (generate_step). The
        automaton's indices come from rosa_idx (device u8 [n_layers][batch][d]) or
        from sam(layer, planes) -> idx u8 [batch, d] (planes: uint32 [3, words])."""
        s = self.shape
        batch = self._decode_batch
        words = (batch * s.d_model + 31) // 32
        failure = []
        fn = _lib.SAM_FN()  # NULL unless a callback is given
        if sam is not None:
            n_idx = batch * s.d_model

            def cb(user, layer, planes_p, idx_p):
                try:
                    planes = np.ctypeslib.as_array(planes_p, shape=(3 * words,)).reshape(3, words)
                    idx = np.ascontiguousarray(sam(int(layer), planes.copy()), np.uint8).ravel()
                    if idx.size != n_idx:
                        raise ValueError(f"automaton returned {idx.size} indices, want {n_idx}")
                    C.memmove(idx_p, idx.ctypes.data, n_idx)
                    return 0
                except Exception as e:
                    failure.append(e)
                    return 1

            fn = _lib.SAM_FN(cb)
        rc = self.rt.lib.ullis_hip_heron_decode_step(
            self.h, table.ptr, s.vocab, tokens.ptr, rosa_idx.ptr if rosa_idx else None, fn, None,
            logits.ptr, next_tokens.ptr if next_tokens else None,
            invalid.ptr if invalid else None)
        if failure:
            raise failure[0]
        self.rt._check(rc, "decode_step")

    def causal_loss(self, g_emb: DeviceBuffer, labels: DeviceBuffer, ignore_id: int,
                    row_loss: DeviceBuffer | None = None, table_res: DeviceBuffer | None = None
                    ) -> dict:
        """CausalLoss of the last step (src/model.rs:58-80, train_step_on's return
        value): ullis_hip_heron_causal_loss into a device struct, downloaded."""
        out = self.rt.zeros(np.uint8, C.sizeof(_lib.CausalLoss))
        n = self.shape.vocab * self.shape.d_model if table_res is not None else 0
        self.rt._check(self.rt.lib.ullis_hip_heron_causal_loss(
            self.h, g_emb.ptr, labels.ptr, ignore_id, row_loss.ptr if row_loss else None,
            table_res.ptr if table_res is not None else None, n, out.ptr), "heron_causal_loss")
        cl = _lib.CausalLoss.from_buffer_copy(out.download(np.uint8).tobytes())
        return cl.as_dict()

    def step_tokens(self, table: DeviceBuffer, table_res: DeviceBuffer, tokens: DeviceBuffer,
                    labels: DeviceBuffer, ignore_id: int, lr: float, rosa_idx: DeviceBuffer,
                    x_emb: DeviceBuffer, g_emb: DeviceBuffer, row_loss: DeviceBuffer | None = None,
                    stats: DeviceBuffer | None = None, qkv_bits: DeviceBuffer | None = None,
                    invalid: DeviceBuffer | None = None):
        """UllisHeron::train_step_on from token ids (src/model.rs:2827-3025): the
        embedding gather, the step and the embedding scatter-SGD, all
        stream-ordered on the device. table / table_res: f16 [vocab, d] and its
        fp32 carry; x_emb / g_emb: fp32 [rows, d] work buffers; invalid
        (optional u32) receives the count of token ids >= vocab and labels >=
        vocab other than ignore_id (non-zero: the step changed nothing)."""
        self.rt._check(self.rt.lib.ullis_hip_heron_step_tokens(
            self.h, table.ptr, table_res.ptr, self.shape.vocab, tokens.ptr, labels.ptr, ignore_id,
            lr, rosa_idx.ptr, x_emb.ptr, g_emb.ptr, row_loss.ptr if row_loss else None,
            stats.ptr if stats else None, qkv_bits.ptr if qkv_bits else None,
            invalid.ptr if invalid else None), "heron_step_tokens")
