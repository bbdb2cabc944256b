"""ctypes binding of the CPU oracle (oracle/libullis_cpu_ref.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load this module, as the checker or the CPU baseline. The
product path (ullis_amd/) never imports it.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libullis_cpu_ref.so"


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


class HeronDims(C.Structure):
    _fields_ = [("d_model", C.c_uint32), ("n_layers", C.c_uint32), ("dim_ffn", C.c_uint32),
                ("vocab", C.c_uint32)]


class TensorDesc(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("dtype", C.c_int32), ("derived", C.c_int32),
                ("count", C.c_uint64), ("offset", C.c_uint64)]


class StepStats(C.Structure):
    _fields_ = [("mean_loss", C.c_float), ("n_valid", C.c_uint64), ("flips_head", C.c_uint64),
                ("flips_cmix", C.c_uint64), ("flips_rosa_o", C.c_uint64),
                ("loss_p10", C.c_float), ("loss_p50", C.c_float), ("loss_p90", C.c_float),
                ("unigram_ce", C.c_float), ("unique_targets", C.c_uint64),
                ("embed_grad_rms", C.c_float), ("head_scale_grad_rms", C.c_float),
                ("head_scale_rms", C.c_float), ("cmix_value_rms", C.c_float),
                ("head_latent_abs_mean", C.c_float), ("head_latent_step_abs", C.c_float),
                ("head_bias_rms", C.c_float)]


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        _LIB = C.CDLL(str(LIB_PATH))
        _LIB.ucr_f16_from_f32.restype = C.c_uint16
        _LIB.ucr_f16_from_f32.argtypes = [C.c_float]
        _LIB.ucr_f16_to_f32.restype = C.c_float
        _LIB.ucr_f16_to_f32.argtypes = [C.c_uint16]
        _LIB.ucr_causal_ce_gradient_scale.restype = C.c_float
        _LIB.ucr_causal_ce_gradient_scale.argtypes = [C.c_size_t, C.c_size_t]
        _LIB.ucr_causal_ce_row_valid.restype = C.c_int
        _LIB.ucr_causal_ce_row_valid.argtypes = [C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p,
                                                 C.c_size_t, C.c_uint32]
        _LIB.ucr_bit_flip_count.restype = C.c_size_t
        for name in ["ucr_rms", "ucr_rms_fp16", "ucr_mean_abs", "ucr_mean_abs_fp16",
                     "ucr_mean_abs_delta_fp16", "ucr_unigram_cross_entropy"]:
            getattr(_LIB, name).restype = C.c_float
        _LIB.ucr_head_ce_horizon.restype = C.c_int
        _LIB.ucr_heron_decode_step.restype = C.c_int
        _LIB.ucr_heron_layout.restype = C.c_size_t
        _LIB.ucr_heron_layout.argtypes = [C.POINTER(HeronDims), C.POINTER(TensorDesc), C.c_size_t,
                                          C.POINTER(C.c_uint64)]
        for name in ["ucr_clipped_sgd", "ucr_binaryconnect_sgd", "ucr_packed_forward",
                     "ucr_packed_backward_ste", "ucr_packed_apply_sgd", "ucr_layer_norm_forward",
                     "ucr_layer_norm_backward", "ucr_head_ce", "ucr_fp16_forward",
                     "ucr_fp16_backward", "ucr_time_shift_delta", "ucr_lerp_shift_backward",
                     "ucr_rosa_y_from_idx", "ucr_rosa_e_grad", "ucr_heron_train_step",
                     "ucr_embedding_gather", "ucr_embedding_scatter_sgd"]:
            getattr(_LIB, name).restype = C.c_int
    return _LIB


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _sz(v):
    return C.c_size_t(int(v))


# ------------------------------------------------------------------ a1 - a4
def f16_from_f32(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.empty(x.size, np.uint16)
    lib().ucr_f16_from_f32_array(_p(x), _p(out), _sz(x.size))
    return out


def f16_to_f32(bits) -> np.ndarray:
    b = _u16(bits).ravel()
    out = np.empty(b.size, np.float32)
    lib().ucr_f16_to_f32_array(_p(b), _p(out), _sz(b.size))
    return out


def clipped_sgd(values, residual, gradient, lr):
    v, r, g = _u16(values).copy(), _f32(residual).copy(), _f32(gradient)
    lib().ucr_clipped_sgd(_p(v), _p(r), _p(g), _sz(v.size), C.c_float(lr))
    return v, r


def binaryconnect_sgd(values, residual, gradient, lr, gradient_scale=1.0):
    v, r, g = _u16(values).copy(), _f32(residual).copy(), _f32(gradient)
    lib().ucr_binaryconnect_sgd(_p(v), _p(r), _p(g), _sz(v.size), C.c_float(lr),
                                C.c_float(gradient_scale))
    return v, r


def words(n):
    return (int(n) + 31) // 32


def pack_latent_bits(latent):
    l = _u16(latent).ravel()
    out = np.zeros(words(l.size), np.uint32)
    lib().ucr_pack_latent_bits(_p(l), _sz(l.size), _p(out))
    return out


def sign_pack_bits(x):
    x = _f32(x).ravel()
    out = np.zeros(words(x.size), np.uint32)
    lib().ucr_sign_pack_bits(_p(x), _sz(x.size), _p(out))
    return out


def transpose_bits(bits, out_f, in_f):
    b = _u32(bits)
    out = np.zeros(words(out_f * in_f), np.uint32)
    lib().ucr_transpose_bits(_p(b), _sz(out_f), _sz(in_f), _p(out))
    return out


# ------------------------------------------------------------------ a5 - a9
def packed_forward(x, rows, in_f, out_f, bits, scale, bias=None):
    x, b, s = _f32(x), _u32(bits), _u16(scale)
    bb = None if bias is None else _u16(bias)
    y = np.empty(rows * out_f, np.float32)
    lib().ucr_packed_forward(_p(x), _sz(rows), _sz(in_f), _sz(out_f), _p(b), _p(s), _p(bb), _p(y))
    return y


def packed_backward_ste(x, gy, rows, in_f, out_f, bits, scale, want_gx=True, want_gb=True):
    x, gy, b, s = _f32(x), _f32(gy), _u32(bits), _u16(scale)
    g_w = np.zeros(out_f * in_f, np.float32)
    g_x = np.zeros(rows * in_f, np.float32) if want_gx else None
    g_s = np.zeros(out_f, np.float32)
    g_b = np.zeros(out_f, np.float32) if want_gb else None
    lib().ucr_packed_backward_ste(_p(x), _p(gy), _sz(rows), _sz(in_f), _sz(out_f), _p(b), _p(s),
                                  _p(g_w), _p(g_x), _p(g_s), _p(g_b))
    return {"weight_gradient": g_w, "input_gradient": g_x, "scale_gradient": g_s,
            "bias_gradient": g_b}


def packed_apply_sgd(in_f, out_f, latent, latent_res, scale, scale_res, bias, bias_res, g_w,
                     g_scale, g_bias, lr, ste):
    latent, latent_res = _u16(latent).copy(), _f32(latent_res).copy()
    scale, scale_res = _u16(scale).copy(), _f32(scale_res).copy()
    if bias is not None:
        bias, bias_res = _u16(bias).copy(), _f32(bias_res).copy()
    bits = np.zeros(words(in_f * out_f), np.uint32)
    lib().ucr_packed_apply_sgd(_sz(in_f), _sz(out_f), _p(latent), _p(latent_res), _p(scale),
                               _p(scale_res), _p(bias), _p(bias_res), _p(bits), _p(_f32(g_w)),
                               _p(_f32(g_scale)), _p(None if g_bias is None else _f32(g_bias)),
                               C.c_float(lr), C.c_float(ste))
    return latent, latent_res, scale, scale_res, bias, bias_res, bits


# ---------------------------------------------------------------- a10 / a11
def layer_norm_forward(x, rows, ch, weight, bias):
    x, w, b = _f32(x), _u16(weight), _u16(bias)
    y = np.empty(rows * ch, np.float32)
    lib().ucr_layer_norm_forward(_p(x), _sz(rows), _sz(ch), _p(w), _p(b), _p(y))
    return y


def layer_norm_backward(x, gy, rows, ch, weight):
    x, gy, w = _f32(x), _f32(gy), _u16(weight)
    gx = np.empty(rows * ch, np.float32)
    gw = np.empty(ch, np.float32)
    gb = np.empty(ch, np.float32)
    lib().ucr_layer_norm_backward(_p(x), _p(gy), _sz(rows), _sz(ch), _p(w), _p(gx), _p(gw), _p(gb))
    return gx, gw, gb


# --------------------------------------------------------------- a12 / a13
def causal_ce_row_valid(row, time, horizon, targets, ignore_id):
    t = _u32(targets)
    return bool(lib().ucr_causal_ce_row_valid(row, time, horizon, _p(t), t.size, ignore_id))


def causal_ce_gradient_scale(n_valid, time):
    return lib().ucr_causal_ce_gradient_scale(n_valid, time)


def head_ce(hidden, rows, time, d, vocab, bits, scale, bias, targets, ignore_id, horizon=1):
    h, b, s, t = _f32(hidden), _u32(bits), _u16(scale), _u32(targets)
    bb = None if bias is None else _u16(bias)
    mean = C.c_float()
    nv = C.c_size_t()
    row_loss = np.zeros(rows, np.float32)
    g_h = np.zeros(rows * d, np.float32)
    g_w = np.zeros(vocab * d, np.float32)
    g_s = np.zeros(vocab, np.float32)
    g_b = np.zeros(vocab, np.float32) if bias is not None else None
    rc = lib().ucr_head_ce_horizon(_p(h), _sz(rows), _sz(time), _sz(horizon), _sz(d), _sz(vocab),
                                   _p(b), _p(s), _p(bb), _p(t), C.c_uint32(ignore_id),
                                   C.byref(mean), C.byref(nv), _p(row_loss), _p(g_h), _p(g_w),
                                   _p(g_s), _p(g_b))
    assert rc == 0
    return {"mean_loss": mean.value, "n_valid": nv.value, "row_loss": row_loss,
            "hidden_gradient": g_h, "weight_gradient": g_w, "scale_gradient": g_s,
            "bias_gradient": g_b}


# ------------------------------------------------------------ T = 1 decode
def heron_decode_step(dims: HeronDims, arena: np.ndarray, table, tokens, idx, rosa_prev,
                      cmix_prev, has_prev: bool):
    """generate_step for len(tokens) sequences with the automaton's indices given
    ([n_layers][batch][d] u8). rosa_prev / cmix_prev (float32 [n_layers*batch*d])
    are updated in place. Returns (logits [batch, vocab], qkv_bits u8
    [n_layers, 3, batch, d])."""
    t = _u32(tokens)
    batch = t.size
    assert rosa_prev.dtype == np.float32 and cmix_prev.dtype == np.float32
    logits = np.zeros(batch * dims.vocab, np.float32)
    qkv = np.zeros(dims.n_layers * 3 * batch * dims.d_model, np.uint8)
    rc = lib().ucr_heron_decode_step(C.byref(dims), _p(arena), _p(_u16(table)), _p(t),
                                     _sz(batch), _p(np.ascontiguousarray(idx, np.uint8)),
                                     _p(rosa_prev), _p(cmix_prev), C.c_int(int(has_prev)),
                                     _p(logits), _p(qkv))
    if rc != 0:
        raise RuntimeError(f"ucr_heron_decode_step failed: {rc}")
    return (logits.reshape(batch, dims.vocab),
            qkv.reshape(dims.n_layers, 3, batch, dims.d_model))


# ---------------------------------------------------- CausalLoss statistics
def rms(v) -> float:
    v = _f32(v).ravel()
    return lib().ucr_rms(_p(v), _sz(v.size))


def rms_fp16(bits) -> float:
    b = _u16(bits).ravel()
    return lib().ucr_rms_fp16(_p(b), _sz(b.size))


def mean_abs(v) -> float:
    v = _f32(v).ravel()
    return lib().ucr_mean_abs(_p(v), _sz(v.size))


def mean_abs_fp16(bits) -> float:
    b = _u16(bits).ravel()
    return lib().ucr_mean_abs_fp16(_p(b), _sz(b.size))


def mean_abs_delta_fp16(before, after) -> float:
    a, b = _u16(before).ravel(), _u16(after).ravel()
    assert a.size == b.size
    return lib().ucr_mean_abs_delta_fp16(_p(a), _p(b), _sz(a.size))


def loss_percentiles(row_loss, time, targets, ignore_id):
    rl, t = _f32(row_loss).ravel(), _u32(targets).ravel()
    out = np.zeros(3, np.float32)
    lib().ucr_loss_percentiles(_p(rl), _sz(rl.size), _sz(time), _p(t), C.c_uint32(ignore_id),
                               _p(out))
    return tuple(float(x) for x in out)


def unigram_cross_entropy(targets, time, ignore_id):
    t = _u32(targets).ravel()
    u = C.c_size_t()
    ce = lib().ucr_unigram_cross_entropy(_p(t), _sz(t.size), _sz(time), C.c_uint32(ignore_id),
                                         C.byref(u))
    return float(ce), int(u.value)


# ---------------------------------------------------------------- a14 - a16
def fp16_forward(x, rows, in_f, out_f, w):
    x, w = _f32(x), _u16(w)
    y = np.empty(rows * out_f, np.float32)
    lib().ucr_fp16_forward(_p(x), _sz(rows), _sz(in_f), _sz(out_f), _p(w), _p(y))
    return y


def fp16_backward(x, gy, rows, in_f, out_f, w):
    x, gy, w = _f32(x), _f32(gy), _u16(w)
    gx = np.empty(rows * in_f, np.float32)
    gw = np.empty(out_f * in_f, np.float32)
    lib().ucr_fp16_backward(_p(x), _p(gy), _sz(rows), _sz(in_f), _sz(out_f), _p(w), _p(gx), _p(gw))
    return gx, gw


def time_shift_delta(x, batch, time, ch):
    x = _f32(x)
    xx = np.empty(x.size, np.float32)
    lib().ucr_time_shift_delta(_p(x), _sz(batch), _sz(time), _sz(ch), _p(xx))
    return xx


def lerp_shift_backward(xx, mix, g_shifted, batch, time, ch):
    xx, m, gs = _f32(xx), _u16(mix), _f32(g_shifted)
    g_x = np.zeros(xx.size, np.float32)
    g_mix = np.zeros(ch, np.float32)
    lib().ucr_lerp_shift_backward(_p(xx), _p(m), _p(gs), _sz(batch), _sz(time), _sz(ch), _p(g_x),
                                  _p(g_mix))
    return g_x, g_mix


def rosa_y_from_idx(idx, e, rows, ch):
    i, e = np.ascontiguousarray(idx, np.uint8), _u16(e)
    y = np.empty(rows * ch, np.float32)
    lib().ucr_rosa_y_from_idx(_p(i), _p(e), _sz(rows), _sz(ch), _p(y))
    return y


def rosa_e_grad(g_y, idx, rows, ch):
    g, i = _f32(g_y), np.ascontiguousarray(idx, np.uint8)
    out = np.empty(ch, np.float32)
    lib().ucr_rosa_e_grad(_p(g), _p(i), _sz(rows), _sz(ch), _p(out))
    return out


def embedding_gather(table, d, tokens):
    t, k = _u16(table), _u32(tokens)
    x = np.empty(k.size * d, np.float32)
    lib().ucr_embedding_gather(_p(t), _sz(d), _p(k), _sz(k.size), _p(x))
    return x


def embedding_scatter_sgd(table, residual, d, tokens, g_x, lr):
    t, r, k, g = _u16(table).copy(), _f32(residual).copy(), _u32(tokens), _f32(g_x)
    lib().ucr_embedding_scatter_sgd(_p(t), _p(r), _sz(d), _p(k), _sz(k.size), _p(g), C.c_float(lr))
    return t, r


# -------------------------------------------------------------------- a17
def heron_layout(dims: HeronDims):
    total = C.c_uint64()
    n = lib().ucr_heron_layout(C.byref(dims), None, 0, C.byref(total))
    arr = (TensorDesc * n)()
    lib().ucr_heron_layout(C.byref(dims), arr, n, C.byref(total))
    return [(d.name.decode(), d.dtype, d.count, d.offset, d.derived) for d in arr], total.value


def heron_train_step(dims: HeronDims, arena: np.ndarray, x_emb, labels, ignore_id, batch, time,
                     lr, rosa_idx, want_qkv=True):
    """Runs one oracle step IN PLACE on `arena` (uint8). Returns outputs."""
    rows = batch * time
    d = dims.d_model
    assert arena.dtype == np.uint8 and arena.flags.c_contiguous
    x, lab = _f32(x_emb), _u32(labels)
    idx = np.ascontiguousarray(rosa_idx, np.uint8)
    g_emb = np.empty(rows * d, np.float32)
    row_loss = np.zeros(rows, np.float32)
    w = words(rows * d)
    qkv = np.zeros(dims.n_layers * 3 * w, np.uint32) if want_qkv else None
    st = StepStats()
    rc = lib().ucr_heron_train_step(C.byref(dims), _p(arena), _p(x), _p(lab), C.c_uint32(ignore_id),
                                    _sz(batch), _sz(time), C.c_float(lr), _p(idx), _p(g_emb),
                                    _p(row_loss), _p(qkv), C.byref(st))
    if rc != 0:
        raise RuntimeError(f"ucr_heron_train_step failed: {rc}")
    out = {"g_emb": g_emb, "row_loss": row_loss, "qkv_bits": qkv}
    out.update({name: getattr(st, name) for name, _ in StepStats._fields_})
    return out
