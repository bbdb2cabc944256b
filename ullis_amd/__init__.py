"""ullis_amd: MI355X (gfx950) backend for the Ullis packed +-1 linear / LayerNorm /
streamed cross-entropy training hot path, behind the C ABI in include/ullis_hip.h."""
from ._lib import F16, F32, LIB_PATH, load  # noqa: F401

__all__ = ["F16", "F32", "LIB_PATH", "load"]
