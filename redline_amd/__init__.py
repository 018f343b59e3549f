"""redline_amd — MI355X (gfx950) fused per-layer kernels of the Redline engine.

Embedding gather, fused residual-add + RMSNorm, RoPE fused with the paged
KV-cache write (FP16, INT8 with per-token/per-head scales) and SwiGLU, as
hand-written HIP kernels behind a C ABI (include/redline_amd/rlk.h) and the
reference's C++ launch signatures (include/redline_amd/kernels.h).
"""
from ._lib import Error, KVLayerView, LIB_PATH, lib  # noqa: F401
from .host import (BatchBuilder, LogitsMode, float_to_half_bits, half_bits_to_float,  # noqa: F401
                   meta_layout, rope_cos_sin_tables, rope_inv_freq)

__version__ = "0.1.0"


def __getattr__(name):
    # The torch-facing launchers import torch lazily so host-only users
    # (metadata, tables) do not pay for it.
    if name == "kernels":
        import importlib
        return importlib.import_module(".kernels", __name__)
    raise AttributeError(name)
