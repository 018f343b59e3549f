"""numpy front end of the CPU oracle (oracle.c).  TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, always as the checker — never as the thing measured or shipped.
`ref()` exposes the compiled reference host core (oracle/_ref), present only
in the container that has /root/reference.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libredline_ref_core.so"

_P = C.c_void_p
_I = C.c_int
_o = None
_r = None


def build(ref: bool = False) -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> C.CDLL:
    global _o
    if _o is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        L.orc_f2h.restype, L.orc_f2h.argtypes = C.c_uint16, [C.c_float]
        L.orc_h2f.restype, L.orc_h2f.argtypes = C.c_float, [C.c_uint16]
        L.orc_rope_cos_sin_tables.argtypes = [C.c_double, _I, _I, C.c_double, C.c_double,
                                              C.c_double, _I, _I, _P, _P]
        L.orc_embedding_lookup.argtypes = [_P, _P, _I, _I, _P]
        L.orc_gather_rows.argtypes = [_P, _P, _I, _I, _P]
        L.orc_resolve_input_ids.argtypes = [_P, _P, _P, _I]
        L.orc_fused_add_rmsnorm.argtypes = [_P, _P, _P, _I, _I, C.c_float, _P]
        L.orc_silu_and_mul.argtypes = [_P, _I, _I, _P]
        L.orc_silu_and_mul_interleaved.argtypes = [_P, _I, _I, _P]
        L.orc_rope_and_write_kv.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P,
                                            _I, _I]
        L.orc_rope_and_write_kv_ex.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P,
                                               _P, _I, _I, _P, _I]
        L.orc_paged_attention_decode.argtypes = [_P, _I, _P, _I, C.c_float, _P, _P, _P, _P, _I,
                                                 _I, _I, _I, _P, _I, _P, _P, _P, _I]
        L.orc_paged_attention_prefill.argtypes = [_P, _I, _P, _I, C.c_float, _P, _P, _P, _P, _I, _I,
                                                  _I, _I, _P, _I, _P, _P, _P, _P, _I]
        L.orc_gemv_w8a16.argtypes = [_P, _I, _P, _P, _P, _I, _I, _P]
        L.orc_gemv_w4a16.argtypes = [_P, _I, _P, _P, _P, _I, _P, _I, _I, _P]
        L.orc_gemv_w4a16_swiglu.argtypes = [_P, _I, _P, _P, _P, _I, _I, _I, _P]
        L.orc_layer_step.argtypes = [_P, _P, _I, _I, _P, _P, _P, _P, C.c_float, _P, _P, _P, _P,
                                     _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _P, _I, _P]
        _o = L
    return _o


CPUSTEP_LIB = HERE / "libcpustep.so"
_c = None


def cpu_step_lib() -> C.CDLL:
    """The multi-threaded CPU port of the layer step (cpu_step.cpp), used as
    bench.py's CPU baseline; same step arguments as orc_layer_step after the
    pool handle."""
    global _c
    if _c is None:
        if not CPUSTEP_LIB.exists():
            build()
        L = C.CDLL(str(CPUSTEP_LIB))
        L.cps_affinity_cores.restype, L.cps_affinity_cores.argtypes = _I, []
        L.cps_create.restype, L.cps_create.argtypes = _P, [_I]
        L.cps_destroy.restype, L.cps_destroy.argtypes = None, [_P]
        L.cps_layer_step.restype = None
        L.cps_layer_step.argtypes = [_P] + list(lib().orc_layer_step.argtypes)
        L.cps_layer_step_timed.restype = None
        L.cps_layer_step_timed.argtypes = [_P] + list(lib().orc_layer_step.argtypes) + [_P]
        _c = L
    return _c


def has_ref() -> bool:
    return REF_LIB.exists()


def ref() -> C.CDLL:
    """The reference's own host core (float_to_half_bits, rope tables, BatchBuilder)."""
    global _r
    if _r is None:
        L = C.CDLL(str(REF_LIB))
        L.ref_float_to_half_bits.restype, L.ref_float_to_half_bits.argtypes = C.c_uint16, [C.c_float]
        L.ref_half_bits_to_float.restype, L.ref_half_bits_to_float.argtypes = C.c_float, [C.c_uint16]
        L.ref_float_to_half_many.argtypes = [_P, C.c_size_t, _P]
        L.ref_quantize_int8_rows.argtypes = [_P, _I, _I, _P, _P]
        L.ref_model_config_json.restype = _I
        L.ref_model_config_json.argtypes = [_I, _I, _I, _I, _I, _I, _I, C.c_double, C.c_double,
                                            _I, C.c_char_p, _I]
        L.ref_model_forward.restype = _I
        L.ref_model_forward.argtypes = [C.c_char_p, _P, _I, _P]
        L.ref_quantize_int4_groups.argtypes = [_P, _I, _I, _I, _P, _P, _P]
        L.ref_rope_inv_freq.argtypes = [C.c_double, _I, _I, C.c_double, C.c_double, C.c_double, _I, _P]
        L.ref_rope_cos_sin_tables.argtypes = [C.c_double, _I, _I, C.c_double, C.c_double,
                                              C.c_double, _I, _I, _P, _P]
        L.ref_bb_create.restype, L.ref_bb_create.argtypes = _P, [_I] * 6
        L.ref_bb_destroy.argtypes = [_P]
        L.ref_bb_max_meta_words.restype, L.ref_bb_max_meta_words.argtypes = C.c_size_t, [_P]
        L.ref_bb_add.restype = _I
        L.ref_bb_add.argtypes = [_P, _P, _I, _I, _P, _P, _I, C.c_float, _I, C.c_float, C.c_uint64, _I]
        L.ref_bb_pad_decode_to.argtypes = [_P, _I]
        L.ref_bb_write.argtypes = [_P, _P, _P]
        L.ref_meta_layout.argtypes = [_P, _I, _P]
        _r = L
    return _r


def p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ wrappers

def f2h(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bit patterns through the oracle's own conversion."""
    f = lib().orc_f2h
    flat = np.asarray(x, np.float32).ravel()
    return np.fromiter((f(float(v)) for v in flat), np.uint16, flat.size).reshape(np.shape(x))


def rope_cos_sin_tables(theta, head_dim, max_pos, scaling=0, factor=1.0, lo=1.0, hi=4.0,
                        old_ctx=8192):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_cos_sin_tables(theta, head_dim, scaling, factor, lo, hi, old_ctx, max_pos,
                                  p(c), p(s))
    return c, s


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16
    return a


def embedding_lookup(ids, table, hidden):
    ids = np.ascontiguousarray(ids, np.int32)
    table = _u16(table)
    out = np.empty((ids.size, hidden), np.uint16)
    lib().orc_embedding_lookup(p(ids), p(table), ids.size, hidden, p(out))
    return out.view(np.float16)


def gather_rows(src, idx, cols):
    idx = np.ascontiguousarray(idx, np.int32)
    out = np.empty((idx.size, cols), np.uint16)
    lib().orc_gather_rows(p(_u16(src)), p(idx), idx.size, cols, p(out))
    return out.view(np.float16)


def resolve_input_ids(ids, src, prev):
    ids = np.array(ids, np.int32)
    lib().orc_resolve_input_ids(p(ids), p(np.ascontiguousarray(src, np.int32)),
                                p(np.ascontiguousarray(prev, np.int32)), ids.size)
    return ids


def fused_add_rmsnorm(residual, delta, weight, eps):
    """Returns (new residual, out) as float16 arrays [rows, hidden]."""
    res = np.array(_u16(residual), copy=True)
    rows, hidden = res.shape
    out = np.empty_like(res)
    d = None if delta is None else _u16(delta)
    lib().orc_fused_add_rmsnorm(p(res), p(d), p(_u16(weight)), rows, hidden, eps, p(out))
    return res.view(np.float16), out.view(np.float16)


def silu_and_mul(gate_up, inter, interleaved=False):
    gu = _u16(gate_up)
    rows = gu.size // (2 * inter)
    out = np.empty((rows, inter), np.uint16)
    fn = lib().orc_silu_and_mul_interleaved if interleaved else lib().orc_silu_and_mul
    fn(p(gu), rows, inter, p(out))
    return out.view(np.float16)


def paged_attention_prefill(q, q_stride, num_heads, scale, k_cache, v_cache, k_scale, v_scale,
                            block_tables, seq_ids, q_start, q_len, ctx_len, num_tokens, int8=False):
    """Returns out fp16 [num_tokens, num_heads * D]; rows of tokens outside the
    prefill sequences are zero.  Caches are [num_blocks, Hkv, bs, D]."""
    nb, hkv, bs, D = k_cache.shape
    out = np.zeros((num_tokens, num_heads * D), np.uint16)
    kc = k_cache.view(np.uint16) if k_cache.dtype == np.float16 else np.ascontiguousarray(k_cache)
    vc = v_cache.view(np.uint16) if v_cache.dtype == np.float16 else np.ascontiguousarray(v_cache)
    bt = np.ascontiguousarray(block_tables, np.int32)
    sid = np.ascontiguousarray(seq_ids, np.int32)
    i32 = lambda a: np.ascontiguousarray(a, np.int32)  # noqa: E731
    lib().orc_paged_attention_prefill(
        p(_u16(q)), q_stride, p(out), num_heads, scale, p(kc), p(vc),
        p(None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)),
        p(None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)), bs, hkv, D,
        int(int8), p(bt), bt.shape[1], p(sid), p(i32(q_start)), p(i32(q_len)), p(i32(ctx_len)),
        sid.size)
    return out.view(np.float16)


def gemv_w8a16(x, w, scales, bias=None):
    """float64 y [m, n] of x [m, k] fp16 times the INT8 W [n, k] with per-row fp16 scales."""
    x = _u16(x)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.int8)
    n = w.shape[0]
    assert w.shape[1] == k
    y = np.empty((m, n), np.float64)
    lib().orc_gemv_w8a16(p(x), m, p(w), p(_u16(scales)), p(None if bias is None else _u16(bias)),
                         n, k, p(y))
    return y


def gemv_w4a16(x, w, scales, offsets, group_size, bias=None):
    """float64 y [m, n] of x [m, k] fp16 times the group-dequantised INT4 W [n, k/2]."""
    x = _u16(x)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.uint8)
    n = w.shape[0]
    assert w.shape[1] * 2 == k
    y = np.empty((m, n), np.float64)
    lib().orc_gemv_w4a16(p(x), m, p(w), p(_u16(scales)), p(_u16(offsets)), group_size,
                         p(None if bias is None else _u16(bias)), n, k, p(y))
    return y


def gemv_w4a16_swiglu(x, w, scales, offsets, group_size):
    """fp16 [m, n/2]: SwiGLU of the interleaved (gate, up) rows of the INT4 GEMV."""
    x = _u16(x)
    m, k = x.shape
    w = np.ascontiguousarray(w, np.uint8)
    n = w.shape[0]
    out = np.empty((m, n // 2), np.uint16)
    lib().orc_gemv_w4a16_swiglu(p(x), m, p(w), p(_u16(scales)), p(_u16(offsets)), group_size, n,
                                k, p(out))
    return out.view(np.float16)


def rope_and_write_kv(qkv, positions, slots, hq, hkv, d, cos_t, sin_t, k_cache, v_cache,
                      k_scale=None, v_scale=None, block_size=16, int8=False, bias=None,
                      scale16=False):
    """Updates qkv (fp16 [T, (hq+2hkv)*d]) and the caches in place.  `bias`
    (fp16 [(hq+2hkv)*d]) and `scale16` select the extension semantics."""
    q = _u16(qkv)
    assert q.flags.c_contiguous
    positions = np.ascontiguousarray(positions, np.int32)
    slots = np.ascontiguousarray(slots, np.int32)
    T = positions.size
    kc = k_cache.view(np.uint16) if k_cache.dtype == np.float16 else k_cache
    vc = v_cache.view(np.uint16) if v_cache.dtype == np.float16 else v_cache
    b = None if bias is None else _u16(bias)
    lib().orc_rope_and_write_kv_ex(p(q), p(positions), p(slots), T, hq, hkv, d,
                                   p(np.ascontiguousarray(cos_t, np.float32)),
                                   p(np.ascontiguousarray(sin_t, np.float32)), p(kc), p(vc),
                                   p(k_scale), p(v_scale), block_size, int(int8), p(b),
                                   int(scale16))


def paged_attention_decode(q, q_stride, num_heads, scale, k_cache, v_cache, k_scale, v_scale,
                           block_tables, positions, item_token, item_seq, num_tokens,
                           int8=False):
    """Returns out fp16 [num_tokens, num_heads * D]; rows of tokens that are not
    decode items are zero.  Caches are [num_blocks, Hkv, bs, D]."""
    nb, hkv, bs, D = k_cache.shape
    out = np.zeros((num_tokens, num_heads * D), np.uint16)
    kc = k_cache.view(np.uint16) if k_cache.dtype == np.float16 else np.ascontiguousarray(k_cache)
    vc = v_cache.view(np.uint16) if v_cache.dtype == np.float16 else np.ascontiguousarray(v_cache)
    bt = np.ascontiguousarray(block_tables, np.int32)
    it = np.ascontiguousarray(item_token, np.int32)
    lib().orc_paged_attention_decode(
        p(_u16(q)), q_stride, p(out), num_heads, scale, p(kc), p(vc),
        p(None if k_scale is None else np.ascontiguousarray(k_scale, np.float32)),
        p(None if v_scale is None else np.ascontiguousarray(v_scale, np.float32)), bs, hkv, D,
        int(int8), p(bt), bt.shape[1], p(np.ascontiguousarray(positions, np.int32)), p(it),
        p(np.ascontiguousarray(item_seq, np.int32)), it.size)
    return out.view(np.float16)
