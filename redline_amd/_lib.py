"""ctypes binding of librlk.so (the C ABI declared in include/redline_amd/rlk.h).

The library is the product: there is no Python or CPU fallback.  Loading fails
loudly when librlk.so has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("RLK_LIBRARY", Path(__file__).resolve().parent / "librlk.so"))

RLK_OK = 0
RLK_EINVAL = -1
RLK_EUNSUPPORTED = -2
RLK_KV_FP16 = 0
RLK_KV_INT8 = 1
RLK_LOGITS_NONE, RLK_LOGITS_LAST, RLK_LOGITS_ALL = 0, 1, 2


class Error(RuntimeError):
    """Raised for a non-zero rlk status (the reference throws redline::Error)."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class KVLayerView(C.Structure):
    """Mirror of rlk_kv_layer_view / redline::KVLayerView (kernels.h:18-27)."""

    _fields_ = [
        ("k", C.c_void_p),
        ("v", C.c_void_p),
        ("k_scale", C.c_void_p),
        ("v_scale", C.c_void_p),
        ("block_size", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("dtype", C.c_int),
    ]


RLK_SCALE_F32, RLK_SCALE_F16 = 0, 1


class RopeKVOptions(C.Structure):
    """Mirror of rlk_rope_kv_options (extension of rope_and_write_kv)."""

    _fields_ = [("qkv_bias", C.c_void_p), ("scale_dtype", C.c_int)]


class AttentionOptions(C.Structure):
    """Mirror of rlk_attention_options (extension of paged_attention_decode)."""

    _fields_ = [("scale_dtype", C.c_int)]


RLK_DECODE_PARTITION_SIZE = 256
RLK_GEMV_W4_MAX_M = 32


class AttentionParams(C.Structure):
    """Mirror of rlk_attention_params / kernels::AttentionParams (kernels.h:91-101)."""

    _fields_ = [("q", C.c_void_p), ("q_stride", C.c_int), ("out", C.c_void_p),
                ("num_heads", C.c_int), ("scale", C.c_float), ("kv", KVLayerView),
                ("block_tables", C.c_void_p), ("max_blocks_per_seq", C.c_int),
                ("positions", C.c_void_p)]


class DecodeAttentionWork(C.Structure):
    """Mirror of rlk_decode_attention_work / kernels::DecodeAttentionWork."""

    _fields_ = [("item_token", C.c_void_p), ("item_seq", C.c_void_p), ("num_items", C.c_int),
                ("max_partitions", C.c_int), ("ws_out", C.c_void_p), ("ws_max", C.c_void_p),
                ("ws_sum", C.c_void_p)]


class PrefillAttentionWork(C.Structure):
    """Mirror of rlk_prefill_attention_work / kernels::PrefillAttentionWork."""

    _fields_ = [("seq_ids", C.c_void_p), ("q_start", C.c_void_p), ("q_len", C.c_void_p),
                ("ctx_len", C.c_void_p), ("num_seqs", C.c_int), ("max_q_tiles", C.c_int)]


class BatchShape(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "num_tokens", "num_seqs", "num_logit_rows", "num_decode_items",
        "num_prefill_seqs", "max_prefill_q_tiles", "max_context")]


META_FIELDS = ("input_ids", "input_src", "positions", "slot_mapping", "seq_q_start",
               "seq_q_len", "seq_ctx_len", "block_tables", "decode_token", "decode_seq",
               "prefill_seq", "logit_token", "param_row", "temperature", "top_k", "top_p",
               "seed_lo", "seed_hi", "total_words")


class MetaLayout(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in META_FIELDS]


_P = C.c_void_p
_I = C.c_int
_SIGNATURES = {
    "rlk_last_error": (C.c_char_p, []),
    "rlk_version": (C.c_char_p, []),
    "rlk_set_tune_knob": (_I, [C.c_char_p, _I, _I]),
    "rlk_get_tune_knob": (_I, [C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "rlk_embedding_lookup": (_I, [_P, _P, _I, _I, _P, _P]),
    "rlk_fused_add_rmsnorm": (_I, [_P, _P, _P, _I, _I, C.c_float, _P, _P]),
    "rlk_embedding_rmsnorm": (_I, [_P, _P, _I, _I, _P, C.c_float, _P, _P, _P]),
    "rlk_silu_and_mul": (_I, [_P, _I, _I, _P, _P]),
    "rlk_silu_and_mul_interleaved": (_I, [_P, _I, _I, _P, _P]),
    "rlk_gather_rows": (_I, [_P, _P, _I, _I, _P, _P]),
    "rlk_resolve_input_ids": (_I, [_P, _P, _P, _I, _P]),
    "rlk_rope_and_write_kv": (_I, [_P, _P, _P, _I, _I, _P, _P, C.POINTER(KVLayerView), _P]),
    "rlk_rope_and_write_kv_ex": (_I, [_P, _P, _P, _I, _I, _P, _P, C.POINTER(KVLayerView),
                                      C.POINTER(RopeKVOptions), _P]),
    "rlk_paged_attention_decode": (_I, [C.POINTER(AttentionParams),
                                        C.POINTER(DecodeAttentionWork), _P]),
    "rlk_paged_attention_decode_noalloc": (_I, [C.POINTER(AttentionParams),
                                                C.POINTER(DecodeAttentionWork), _P]),
    "rlk_paged_attention_decode_ex": (_I, [C.POINTER(AttentionParams),
                                           C.POINTER(DecodeAttentionWork),
                                           C.POINTER(AttentionOptions), _P]),
    "rlk_paged_attention_prefill": (_I, [C.POINTER(AttentionParams),
                                         C.POINTER(PrefillAttentionWork), _P]),
    "rlk_paged_attention_prefill_ex": (_I, [C.POINTER(AttentionParams),
                                            C.POINTER(PrefillAttentionWork),
                                            C.POINTER(AttentionOptions), _P]),
    "rlk_gemv_w8a16": (_I, [_P, _I, _P, _P, _P, _I, _I, _P, _I, _P]),
    "rlk_gemv_w4a16": (_I, [_P, _I, _P, _P, _P, _I, _P, _I, _I, _P, _I, _P]),
    "rlk_gemv_w4a16_swiglu": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _P, _P]),
    "rlk_float_to_half_bits": (C.c_uint16, [C.c_float]),
    "rlk_half_bits_to_float": (C.c_float, [C.c_uint16]),
    "rlk_rope_inv_freq": (_I, [C.c_double, _I, _I, C.c_double, C.c_double, C.c_double, _I, _P]),
    "rlk_rope_cos_sin_tables": (_I, [C.c_double, _I, _I, C.c_double, C.c_double, C.c_double,
                                     _I, _I, _P, _P]),
    "rlk_meta_layout_make": (_I, [C.POINTER(BatchShape), _I, C.POINTER(MetaLayout)]),
    "rlk_batch_builder_create": (_P, [_I, _I, _I, _I, _I, _I]),
    "rlk_batch_builder_destroy": (None, [_P]),
    "rlk_batch_builder_reset": (None, [_P]),
    "rlk_batch_builder_max_meta_words": (C.c_size_t, [_P]),
    "rlk_batch_builder_add": (_I, [_P, _P, _I, _I, _P, _P, _I, C.c_float, _I, C.c_float,
                                   C.c_uint64, _I, C.POINTER(C.c_int)]),
    "rlk_batch_builder_pad_decode_to": (_I, [_P, _I]),
    "rlk_batch_builder_shape": (_I, [_P, C.POINTER(BatchShape)]),
    "rlk_batch_builder_write": (_I, [_P, _P, C.POINTER(BatchShape)]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded librlk.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m redline_amd.build` "
                "(there is no fallback implementation)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def set_tune_knob(name: str, value: int | None) -> None:
    """Sets (or, with None, clears) a launch-policy override RLK_TUNE_*.
    The library reads the environment once per process; tuning runs and the
    tests that cover every launch policy change the knobs through this."""
    check(lib().rlk_set_tune_knob(name.encode(), 0 if value is None else int(value),
                                  0 if value is None else 1))


def get_tune_knob(name: str) -> int | None:
    """The current value of launch-policy override `name`, None when unset."""
    value, is_set = C.c_int(0), C.c_int(0)
    check(lib().rlk_get_tune_knob(name.encode(), C.byref(value), C.byref(is_set)))
    return value.value if is_set.value else None


class tune_knob:
    """Context manager: the knob set to `value` inside the block, restored to
    its previous value (or cleared, if it was unset) after.  Knobs are
    process-wide: use it only while no other thread launches kernels."""

    def __init__(self, name: str, value: int | None):
        self.name, self.value = name, value
        self.prev = None

    def __enter__(self):
        self.prev = get_tune_knob(self.name)
        set_tune_knob(self.name, self.value)
        return self

    def __exit__(self, *exc):
        set_tune_knob(self.name, self.prev)
        return False


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int) -> None:
    if status != RLK_OK:
        raise Error(status, lib().rlk_last_error().decode())
