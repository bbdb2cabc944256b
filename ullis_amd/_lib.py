"""ctypes binding of libullis_hip.so (include/ullis_hip.h).

The library is loaded from this package directory only; there is no fallback.
If it is missing the import raises, so a GPU run can never silently use
another code path.
"""
from __future__ import annotations

import ctypes as C
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libullis_hip.so"

F16 = 1
F32 = 2

vp = C.c_void_p
sz = C.c_size_t
i32 = C.c_int
u32 = C.c_uint32
f32 = C.c_float


class TensorDesc(C.Structure):
    _fields_ = [
        ("name", C.c_char * 64),
        ("dtype", C.c_int32),
        ("derived", C.c_int32),
        ("count", C.c_uint64),
        ("offset", C.c_uint64),
    ]


class HeronDims(C.Structure):
    _fields_ = [
        ("d_model", C.c_uint32),
        ("n_layers", C.c_uint32),
        ("dim_ffn", C.c_uint32),
        ("vocab", C.c_uint32),
    ]


class CausalLoss(C.Structure):
    """ullis_hip_causal_loss: CausalLoss of src/model.rs:58-80 (counts as u32)."""
    _fields_ = [
        ("next_token", C.c_float),
        ("next_token_count", C.c_uint32),
        ("binary_flip_count", C.c_uint32),
        ("loss_p10", C.c_float),
        ("loss_p50", C.c_float),
        ("loss_p90", C.c_float),
        ("unigram_ce", C.c_float),
        ("unique_targets", C.c_uint32),
        ("flips_head", C.c_uint32),
        ("flips_cmix", C.c_uint32),
        ("flips_rosa_o", C.c_uint32),
        ("embed_grad_rms", C.c_float),
        ("head_scale_grad_rms", C.c_float),
        ("head_scale_rms", C.c_float),
        ("residual_abs_mean", C.c_float),
        ("cmix_value_rms", C.c_float),
        ("head_latent_abs_mean", C.c_float),
        ("head_latent_step_abs", C.c_float),
        ("head_bias_rms", C.c_float),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


# ullis_hip_sam_fn: int (*)(void* user, size_t layer, const uint32_t* planes, uint8_t* idx)
SAM_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32),
                     C.POINTER(C.c_uint8))

# name -> (restype, argtypes)
SIGNATURES = {
    "ullis_hip_version": (i32, []),
    "ullis_hip_device_count": (i32, [C.POINTER(i32)]),
    "ullis_hip_create": (i32, [i32, C.POINTER(vp)]),
    "ullis_hip_destroy": (None, [vp]),
    "ullis_hip_last_error": (C.c_char_p, [vp]),
    "ullis_hip_sync": (i32, [vp]),
    "ullis_hip_malloc": (i32, [vp, sz, C.POINTER(vp)]),
    "ullis_hip_free": (i32, [vp, vp]),
    "ullis_hip_upload": (i32, [vp, vp, vp, sz]),
    "ullis_hip_download": (i32, [vp, vp, vp, sz]),
    "ullis_hip_copy": (i32, [vp, vp, vp, sz]),
    "ullis_hip_event_record": (i32, [vp, i32]),
    "ullis_hip_event_elapsed_ms": (i32, [vp, i32, i32, C.POINTER(f32)]),
    "ullis_hip_time_next_launch": (i32, [vp, i32, i32]),
    "ullis_hip_layer_norm": (i32, [vp, vp, vp, vp, sz, sz, vp, vp]),
    "ullis_hip_layer_norm_backward": (i32, [vp, vp, vp, vp, sz, sz, vp, vp, vp]),
    "ullis_hip_layer_norm_backward_static": (i32, [vp, vp, vp, vp, sz, sz, vp, vp, vp]),
    "ullis_hip_binary_linear": (i32, [vp, vp, i32, vp, vp, vp, sz, sz, sz, vp, vp]),
    "ullis_hip_binary_linear_backward": (
        i32, [vp, vp, vp, vp, vp, i32, sz, sz, sz, vp, vp, vp, vp]),
    "ullis_hip_apply_latent_sgd": (i32, [vp, vp, vp, vp, sz, sz, f32, f32, vp, vp]),
    "ullis_hip_fp16_linear": (i32, [vp, vp, i32, vp, sz, sz, sz, vp, vp]),
    "ullis_hip_fp16_linear_backward": (i32, [vp, vp, vp, vp, sz, sz, sz, vp, vp]),
    "ullis_hip_clipped_sgd_fp16": (i32, [vp, vp, vp, vp, sz, f32]),
    "ullis_hip_binaryconnect_sgd_fp16": (i32, [vp, vp, vp, vp, sz, f32]),
    "ullis_hip_sign_pack_bits": (i32, [vp, vp, sz, vp]),
    "ullis_hip_transpose_bits": (i32, [vp, vp, sz, sz, vp]),
    "ullis_hip_packed_head_train_sgd": (
        i32,
        [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, u32, f32, f32,
         vp, vp, vp, vp, vp, vp, vp]),
    "ullis_hip_embedding_gather": (i32, [vp, vp, sz, sz, vp, sz, vp, vp]),
    "ullis_hip_embedding_scatter_sgd": (i32, [vp, vp, vp, sz, sz, vp, sz, vp, f32]),
    "ullis_hip_cmix_tape_bytes": (sz, [sz, sz, sz]),
    "ullis_hip_rosa_tape_bytes": (sz, [sz, sz]),
    "ullis_hip_cmix_block_forward": (i32, [vp, vp, i32, vp, vp, vp, vp, sz, sz, sz, sz, vp, vp]),
    "ullis_hip_cmix_block_backward_sgd": (
        i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, f32, f32, vp, vp, vp]),
    "ullis_hip_rosa_qkv_forward": (
        i32, [vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, vp, vp,
              vp]),
    "ullis_hip_rosa_out_forward": (i32, [vp, vp, vp, vp, vp, vp, sz, sz, sz, vp, vp]),
    "ullis_hip_rosa_o_stop_grad_sgd": (
        i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, f32, f32, vp, vp, vp]),
    "ullis_hip_heron_layout": (sz, [C.POINTER(HeronDims), C.POINTER(TensorDesc), sz,
                                    C.POINTER(C.c_uint64)]),
    "ullis_hip_heron_create": (i32, [vp, C.POINTER(HeronDims), sz, sz, C.POINTER(vp)]),
    "ullis_hip_heron_destroy": (None, [vp]),
    "ullis_hip_heron_arena": (i32, [vp, C.POINTER(vp), C.POINTER(C.c_uint64)]),
    "ullis_hip_heron_refresh_derived": (i32, [vp]),
    "ullis_hip_heron_step": (i32, [vp, vp, vp, u32, f32, vp, vp, vp, vp, vp, vp]),
    "ullis_hip_heron_causal_loss": (i32, [vp, vp, vp, u32, vp, vp, sz, vp]),
    "ullis_hip_heron_phases": (i32, [vp, i32]),
    "ullis_hip_heron_phases_read": (i32, [vp, vp, vp]),
    "ullis_hip_heron_decode_init": (i32, [vp, sz, i32]),
    "ullis_hip_heron_decode_step": (i32, [vp, vp, sz, vp, vp, SAM_FN, vp, vp, vp, vp]),
    "ullis_hip_heron_step_sam": (i32, [vp, vp, vp, sz, vp, vp, vp, u32, f32, SAM_FN, vp, vp, vp,
                                      vp, vp, vp]),
    "ullis_hip_heron_step_tokens": (i32, [vp, vp, vp, sz, vp, vp, u32, f32, vp, vp, vp, vp, vp,
                                         vp, vp]),
    "ullis_hip_heron_set_graph": (i32, [vp, i32]),
    "ullis_hip_heron_probe": (i32, [vp, i32]),
    "ullis_hip_heron_probe_read": (i32, [vp, C.POINTER(f32), C.POINTER(i32)]),
}


def header_symbols() -> list[str]:
    """Function names declared in include/ullis_hip.h."""
    import re

    text = (HERE.parent / "include" / "ullis_hip.h").read_text()
    return sorted(set(re.findall(r"\b(ullis_hip_[a-z0-9_]+)\s*\(", text)))


_LIB = None


def load() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ullis_amd.build`"
            )
        lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB
