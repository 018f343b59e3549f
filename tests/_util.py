"""Shared helpers for the parity tests."""
from __future__ import annotations

import sys

import numpy as np

# Tolerances for fp16 outputs (fp32 accumulation): elementwise
# |a - b| <= ATOL + RTOL * |b|, plus the reference's own metric
# max|a - b| / max|b| <= REL_MAX (tests/cuda/cuda_test_utils.h:83-90).
ATOL = 2e-3
RTOL = 1e-2
REL_MAX = 2e-3


def say(*msg):
    """Names the case on stdout before a GPU step (flushed, survives a crash)."""
    print(*msg, flush=True)
    sys.stdout.flush()


def randn_f16(rng: np.random.Generator, shape, std=1.0, mean=0.0) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * std + mean).astype(np.float16)


def rel_max_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-12)) if a.size else 0.0


def assert_close_f16(got, want, atol=ATOL, rtol=RTOL, rel_max=REL_MAX, what=""):
    g = np.asarray(got, np.float32)
    w = np.asarray(want, np.float32)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    assert np.all(np.isfinite(g) == np.isfinite(w)), f"{what}: finiteness differs"
    fin = np.isfinite(w)
    diff = np.abs(g[fin] - w[fin])
    bound = atol + rtol * np.abs(w[fin])
    bad = diff > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements out of tolerance; worst "
                           f"diff {float(diff.max()):.3g}")
    assert rel_max_err(g[fin], w[fin]) <= rel_max, f"{what}: rel max err {rel_max_err(g[fin], w[fin])}"


def assert_bits_equal(got, want, what=""):
    g = np.ascontiguousarray(got)
    w = np.ascontiguousarray(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    gv, wv = g.view(np.uint8), w.view(np.uint8)
    if not np.array_equal(gv, wv):
        n = int(np.sum(g.reshape(-1) != w.reshape(-1)))
        raise AssertionError(f"{what}: {n} elements differ bitwise")


def int8_linear(rng: np.random.Generator, n: int, k: int, std: float = 0.05):
    """A per-row INT8 weight in the reference's GEMV layout, quantised the way
    quantize_int8_rows does it (src/cpu/random_model.cpp:99-115): scale =
    fp16(amax / 127), codes = clamp(rint(w / scale), -127, 127) against the stored
    scale.  Returns (codes int8 [n, k], scales fp16 [n], float64 W = codes * scale)."""
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    q, s = int8_quantize_rows(w)
    return q, s, q.astype(np.float64) * s.astype(np.float64)[:, None]


def int8_quantize_rows(w: np.ndarray):
    """quantize_int8_rows (src/cpu/random_model.cpp:99-115) in numpy: fp32 w
    [n, k] -> (codes int8 [n, k], scales fp16 [n])."""
    w = np.asarray(w, np.float32)
    amax = np.abs(w).max(axis=1)
    s = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float16)
    q = np.clip(np.rint(w / s.astype(np.float32)[:, None]), -127, 127).astype(np.int8)
    return q, s


def int4_quantize_groups(w: np.ndarray, group_size: int):
    """quantize_int4_groups (src/cpu/random_model.cpp:118-140) in numpy: per
    group scale = fp16((hi - lo) / 15) (1 when hi == lo), offset = fp16(lo),
    code = clamp(rint((x - offset) / scale), 0, 15) against the stored fp16
    values, two codes per byte with the even column in the low nibble.
    Returns (packed uint8 [n, k/2], scales fp16 [n, k/g], offsets fp16 [n, k/g])."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    x = w.reshape(n, k // group_size, group_size)
    lo, hi = x.min(axis=2), x.max(axis=2)
    s = np.where(hi > lo, (hi - lo) / np.float32(15), np.float32(1)).astype(np.float16)
    o = lo.astype(np.float16)
    q = np.clip(np.rint((x - o.astype(np.float32)[..., None]) / s.astype(np.float32)[..., None]),
                0, 15).astype(np.uint8).reshape(n, k)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8), s, o


def int4_linear(rng: np.random.Generator, n: int, k: int, group_size: int, dense: bool = True):
    """A group-quantised INT4 weight in the reference's GEMV layout.

    Returns (packed uint8 [n, k/2], scales fp16 [n, k/g], offsets fp16 [n, k/g],
    float64 dequantised W [n, k], or None when not `dense`).  W is built from the codes before they are
    packed (W = q * s + o), so it checks the packing rather than restating it.
    Scales and offsets have the magnitudes a min/max quantiser gives a weight
    of std ~0.05 (offset ~ -7.5 scale: W is roughly zero-mean)."""
    groups = k // group_size
    q = rng.integers(0, 16, (n, k), dtype=np.uint8)
    s = rng.uniform(0.004, 0.02, (n, groups)).astype(np.float16)
    o = (-7.5 * s.astype(np.float64) * rng.uniform(0.9, 1.1, (n, groups))).astype(np.float16)
    w = None
    if dense:
        s64 = np.repeat(s.astype(np.float64), group_size, axis=1)
        o64 = np.repeat(o.astype(np.float64), group_size, axis=1)
        w = q * s64 + o64
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, s, o, w


def interleave_rows(a: np.ndarray) -> np.ndarray:
    """[gate; up] rows -> (gate_0, up_0, gate_1, up_1, ...), the loader's INT4
    gate_up layout (src/cuda/model/weights.cpp:157-167)."""
    half = a.shape[0] // 2
    out = np.empty_like(a)
    out[0::2] = a[:half]
    out[1::2] = a[half:]
    return out


# A tiny Llama model for the end-to-end parity test: the reference's
# tiny_test_config (src/cpu/random_model.cpp:148-166) with smaller dims.
TINY_MODEL = dict(vocab=512, hidden=128, inter=256, layers=2, heads=2, kv_heads=1, head_dim=64,
                  theta=1e4, eps=1e-5)


TINY_INT4_GROUP = 64  # the reference's tiny_test_config group size


def tiny_model_weights(seed: int = 7, cfg: dict = TINY_MODEL, int4: bool = False) -> dict:
    """Weights of a random model under the reference's tensor names and
    layouts (src/cpu/random_model.cpp:62-85): embeddings ~N(0, 1), linear rows
    ~N(0, gain^2 / k) with gain 4 for lm_head, norm weights U[0.8, 1.2], wqkv
    rows q heads then k heads then v heads, w_gate_up rows gate then up; all
    fp16, or with int4 the four layer projections as the reference's INT4
    format (prefix.weight packed codes, .scales, .offsets: its
    quantize_int4_groups, restated by int4_quantize_groups, group 64)."""
    rng = np.random.default_rng(seed)
    V, H, I, D = cfg["vocab"], cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv = cfg["heads"], cfg["kv_heads"]

    def lin32(n, k, gain=1.0):
        return (rng.standard_normal((n, k)) * (gain / np.sqrt(k))).astype(np.float32)

    def norm_w():
        return rng.uniform(0.8, 1.2, H).astype(np.float16)

    def add_linear(name, n, k):
        v = lin32(n, k)
        if int4:
            packed, s, o = int4_quantize_groups(v, TINY_INT4_GROUP)
            w[name + ".weight"], w[name + ".scales"], w[name + ".offsets"] = packed, s, o
        else:
            w[name + ".weight"] = v.astype(np.float16)

    w = {"tok_embeddings.weight": rng.standard_normal((V, H)).astype(np.float16)}
    for layer in range(cfg["layers"]):
        p = f"layers.{layer}."
        w[p + "attn_norm.weight"] = norm_w()
        add_linear(p + "wqkv", (hq + 2 * hkv) * D, H)
        add_linear(p + "wo", H, hq * D)
        w[p + "ffn_norm.weight"] = norm_w()
        add_linear(p + "w_gate_up", 2 * I, H)
        add_linear(p + "w_down", H, I)
    w["norm.weight"] = norm_w()
    w["lm_head.weight"] = lin32(V, H, 4.0).astype(np.float16)
    return w


def int4_dequantize(packed: np.ndarray, s: np.ndarray, o: np.ndarray, group_size: int) -> np.ndarray:
    """float32 W = q * scale + offset per group (the reference's
    dequantize_linear for INT4, src/cpu/reference_model.cpp:70-85)."""
    q = np.empty((packed.shape[0], packed.shape[1] * 2), np.float32)
    q[:, 0::2] = packed & 15
    q[:, 1::2] = packed >> 4
    sg = np.repeat(s.astype(np.float32), group_size, axis=1)
    og = np.repeat(o.astype(np.float32), group_size, axis=1)
    return q * sg + og


def tiny_model_tokens(n: int = 150) -> np.ndarray:
    """The token pattern of the reference's engine scoring test
    (tests/cuda/test_engine.cpp:104-105)."""
    return np.array([3 + (i * 37) % 500 for i in range(n)], np.int32)


def next_token_logprobs(logits: np.ndarray, tokens: np.ndarray) -> np.ndarray:
    """log p(tokens[i + 1] | prefix) from logits rows 0 .. n-2 (float64)."""
    x = np.asarray(logits, np.float64)[:-1]
    mx = x.max(axis=1, keepdims=True)
    lse = mx[:, 0] + np.log(np.exp(x - mx).sum(axis=1))
    return x[np.arange(x.shape[0]), tokens[1:]] - lse
