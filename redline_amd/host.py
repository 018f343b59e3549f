"""Host-side helpers over the C ABI: fp16 bits, RoPE tables, BatchBuilder.

Mirrors the reference host core the kernels are driven by:
rope_inv_freq / rope_cos_sin_tables (src/core/model_config.cpp:126-169),
float_to_half_bits / half_bits_to_float (src/core/common.cpp:37-89) and
BatchBuilder / MetaLayout (src/core/batch_builder.cpp).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (RLK_LOGITS_ALL, RLK_LOGITS_LAST, RLK_LOGITS_NONE, BatchShape, Error,
                   META_FIELDS, MetaLayout, check, lib)

SCALING = {"none": 0, "default": 0, "linear": 1, "llama3": 2}


def float_to_half_bits(f: float) -> int:
    return int(lib().rlk_float_to_half_bits(float(f)))


def half_bits_to_float(h: int) -> float:
    return float(lib().rlk_half_bits_to_float(int(h)))


def _np_ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def rope_inv_freq(theta, head_dim, scaling="none", factor=1.0, low_freq_factor=1.0,
                  high_freq_factor=4.0, original_max_position_embeddings=8192) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float64)
    check(lib().rlk_rope_inv_freq(theta, head_dim, SCALING[scaling], factor, low_freq_factor,
                                  high_freq_factor, original_max_position_embeddings, _np_ptr(out)))
    return out


def rope_cos_sin_tables(theta, head_dim, max_pos, scaling="none", factor=1.0,
                        low_freq_factor=1.0, high_freq_factor=4.0,
                        original_max_position_embeddings=8192):
    """fp32 cos, sin tables of shape [max_pos, head_dim // 2] (numpy)."""
    cos = np.empty((max_pos, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    check(lib().rlk_rope_cos_sin_tables(theta, head_dim, SCALING[scaling], factor, low_freq_factor,
                                        high_freq_factor, original_max_position_embeddings,
                                        max_pos, _np_ptr(cos), _np_ptr(sin)))
    return cos, sin


def meta_layout(shape: BatchShape, max_blocks_per_seq: int) -> dict:
    m = MetaLayout()
    check(lib().rlk_meta_layout_make(C.byref(shape), max_blocks_per_seq, C.byref(m)))
    return {f: getattr(m, f) for f in META_FIELDS}


class LogitsMode:
    kNone, kLast, kAll = RLK_LOGITS_NONE, RLK_LOGITS_LAST, RLK_LOGITS_ALL


class BatchBuilder:
    """Per-step batch metadata in one int32 buffer (redline::BatchBuilder)."""

    def __init__(self, max_tokens, max_seqs, max_logit_rows, max_blocks_per_seq, block_size,
                 decode_query_threshold):
        self._h = lib().rlk_batch_builder_create(max_tokens, max_seqs, max_logit_rows,
                                                 max_blocks_per_seq, block_size,
                                                 decode_query_threshold)
        if not self._h:
            raise Error(-1, lib().rlk_last_error().decode())
        self.max_blocks_per_seq = max_blocks_per_seq

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            lib().rlk_batch_builder_destroy(h)

    def reset(self):
        lib().rlk_batch_builder_reset(self._h)

    def max_meta_words(self) -> int:
        return int(lib().rlk_batch_builder_max_meta_words(self._h))

    def add(self, tokens, start_pos, n, src_rows, blocks, temperature=0.0, top_k=0, top_p=1.0,
            seed=0, mode=LogitsMode.kNone) -> int:
        tok = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
        src = None if src_rows is None else np.ascontiguousarray(src_rows, np.int32)
        blk = np.ascontiguousarray(blocks, np.int32)
        first = C.c_int(-1)
        check(lib().rlk_batch_builder_add(
            self._h, None if tok is None else _np_ptr(tok), start_pos, n,
            None if src is None else _np_ptr(src), _np_ptr(blk), len(blk), temperature, top_k,
            top_p, seed, mode, C.byref(first)))
        return first.value

    def pad_decode_to(self, num_seqs):
        check(lib().rlk_batch_builder_pad_decode_to(self._h, num_seqs))

    def shape(self) -> BatchShape:
        s = BatchShape()
        check(lib().rlk_batch_builder_shape(self._h, C.byref(s)))
        return s

    def write(self, dst: np.ndarray | None = None):
        """Serializes into an int32 buffer; returns (buffer, shape, layout dict)."""
        if dst is None:
            dst = np.zeros(self.max_meta_words(), np.int32)
        assert dst.dtype == np.int32 and dst.size >= self.max_meta_words()
        s = BatchShape()
        check(lib().rlk_batch_builder_write(self._h, _np_ptr(dst), C.byref(s)))
        return dst, s, meta_layout(s, self.max_blocks_per_seq)
