"""Writes the golden vectors under tests/golden/ from the reference's own host
core, compiled from /root/reference/src/core by `make -C oracle ref`
(oracle/_ref/libredline_ref_core.so).  Run in the container that has the
reference:  python tests/golden/make_golden.py

Fixtures (inputs and the reference's outputs only):
  half_f2h.npz       float32 inputs -> reference float_to_half_bits
  rope_tables.npz    inv_freq and cos/sin rows at selected positions for the
                     theta / head_dim / scaling cases of the workloads
  quantize.npz       weights -> reference quantize_int8_rows / quantize_int4_groups
                     (src/cpu/random_model.cpp:99-140)
  batch_meta.npz     BatchBuilder metadata for the KAT case of
                     tests/cpp/test_core.cpp:334-386, the graph-padding case
                     (:388-404), and the C2 / C3 workload batches (per-token
                     arrays in full, the whole buffer as a SHA-256)
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from oracle import p  # noqa: E402

OUT = Path(__file__).resolve().parent

# (theta, head_dim, scaling, factor, low_freq_factor, high_freq_factor, old_ctx)
ROPE_CASES = [
    (1e4, 64, 0, 1.0, 1.0, 4.0, 8192),      # TinyLlama, tiny test config
    (5e5, 128, 0, 1.0, 1.0, 4.0, 8192),     # Llama-3.1-8B shape (unscaled)
    (5e5, 128, 2, 8.0, 1.0, 4.0, 8192),     # Llama-3.1 llama3 scaling
    (1e6, 128, 0, 1.0, 1.0, 4.0, 8192),     # Qwen2-7B
    (5e5, 32, 2, 8.0, 1.0, 4.0, 8192),      # test_core.cpp:134-171 config
    (1e4, 64, 1, 4.0, 1.0, 4.0, 8192),      # linear scaling
]
ROPE_POSITIONS = np.array([0, 1, 2, 3, 5, 17, 100, 1000, 2047, 3071, 4095, 8191, 12345, 16383],
                          np.int32)


def half_fixture(R):
    rng = np.random.default_rng(1234)
    bits = rng.integers(0, 2**32, 40000, dtype=np.uint64).astype(np.uint32)
    grid = np.arange(0, 0x7C00, 7, dtype=np.uint32)
    hf = np.array([R.ref_half_bits_to_float(int(h)) for h in grid], np.float32)
    allh = np.array([R.ref_half_bits_to_float(int(h)) for h in range(0x7C01)], np.float64)
    mids = ((allh[:-1] + allh[1:]) / 2)[::5].astype(np.float32)  # exact ties
    special = np.array([0.0, -0.0, 1.0, -2.0, 1e6, 1.0009765625, 1.00048828125, 65504, 65519.996,
                        65520, 6.1035156e-05, 5.9604645e-08, 2.0**-25, 2.0**-26, 3 * 2.0**-26,
                        np.inf, -np.inf, 0.1, 1e-3], np.float32)
    x = np.concatenate([bits.view(np.float32), hf, mids, -mids, special])
    x = x[~np.isnan(x)]
    y = np.empty(x.size, np.uint16)
    R.ref_float_to_half_many(p(x), x.size, p(y))
    np.savez_compressed(OUT / "half_f2h.npz", x=x, y=y)


def rope_fixture(R):
    arrays = {"cases": np.array(ROPE_CASES, np.float64), "positions": ROPE_POSITIONS}
    for i, (theta, D, sc, f, lo, hi, old) in enumerate(ROPE_CASES):
        inv = np.empty(D // 2, np.float64)
        R.ref_rope_inv_freq(theta, D, sc, f, lo, hi, old, p(inv))
        max_pos = int(ROPE_POSITIONS.max()) + 1
        c = np.empty((max_pos, D // 2), np.float32)
        s = np.empty_like(c)
        R.ref_rope_cos_sin_tables(theta, D, sc, f, lo, hi, old, max_pos, p(c), p(s))
        arrays[f"inv_{i}"] = inv
        arrays[f"cos_{i}"] = c[ROPE_POSITIONS]
        arrays[f"sin_{i}"] = s[ROPE_POSITIONS]
    np.savez_compressed(OUT / "rope_tables.npz", **arrays)


class RefBuilder:
    def __init__(self, R, *args):
        self.R, self.h, self.max_blocks = R, R.ref_bb_create(*args), args[3]

    def add(self, tokens, start, n, src, blocks, temp=0.0, top_k=0, top_p=1.0, seed=0, mode=0):
        tok = None if tokens is None else np.asarray(tokens, np.int32)
        sr = None if src is None else np.asarray(src, np.int32)
        blk = np.asarray(blocks, np.int32)
        return self.R.ref_bb_add(self.h, p(tok), start, n, p(sr), p(blk), blk.size, temp, top_k,
                                 top_p, seed, mode)

    def write(self):
        buf = np.full(self.R.ref_bb_max_meta_words(self.h), -7, np.int32)
        shape = np.zeros(7, np.int32)
        self.R.ref_bb_write(self.h, p(buf), p(shape))
        layout = np.zeros(19, np.uint64)
        self.R.ref_meta_layout(p(shape), self.max_blocks, p(layout))
        return buf, shape, layout


def kat_case(R):
    # tests/cpp/test_core.cpp:334-386 (block size 4, decode threshold 2).
    b = RefBuilder(R, 64, 8, 16, 4, 4, 2)
    rows = [b.add(None, 9, 1, [5], [11, 12, 13], mode=1),
            b.add([40, 41, 42, 43, 44, 45], 3, 6, None, [20, 21, 22], 0.5, 7, 1.0,
                  (3 << 32) | 9, 0),
            b.add([7, 0], 0, 2, [-1, 2], [30], mode=2),
            b.add([40, 41, 42, 43, 44, 45], 10, 6, None, [1, 2], mode=0)]  # too few blocks
    buf, shape, layout = b.write()
    return dict(kat_rows=np.array(rows, np.int32), kat_buf=buf, kat_shape=shape,
                kat_layout=layout)


def pad_case(R):
    # tests/cpp/test_core.cpp:388-404.
    b = RefBuilder(R, 64, 8, 16, 4, 16, 1)
    b.add([5], 20, 1, None, [3, 4], mode=1)
    R.ref_bb_pad_decode_to(b.h, 4)
    buf, shape, layout = b.write()
    return dict(pad_buf=buf, pad_shape=shape, pad_layout=layout)


def workload_case(R, key):
    from redline_amd.configs import block_tables, make_workload
    w = make_workload(key, seed=0)
    rng = np.random.default_rng(w.seed + 1)
    tables = block_tables(w, rng)
    b = RefBuilder(R, w.num_tokens, len(w.segments), len(w.segments), max(map(len, tables)),
                   w.block_size, 1)
    for s, t in zip(w.segments, tables):
        b.add(np.zeros(s.n, np.int32), s.start, s.n, None, t, mode=1)
    buf, shape, layout = b.write()
    T = w.num_tokens
    lay = dict(zip(("input_ids", "input_src", "positions", "slot_mapping"), layout[:4]))
    tab_hash = hashlib.sha256(b"".join(t.tobytes() for t in tables)).hexdigest()
    return {
        f"{key}_shape": shape, f"{key}_layout": layout,
        f"{key}_positions": buf[int(lay["positions"]):int(lay["positions"]) + T],
        f"{key}_slot_mapping": buf[int(lay["slot_mapping"]):int(lay["slot_mapping"]) + T],
        f"{key}_sha256": np.array(hashlib.sha256(buf[:int(layout[18])].tobytes()).hexdigest()),
        f"{key}_tables_sha256": np.array(tab_hash),
    }


def batch_fixture(R):
    arrays = {}
    arrays.update(kat_case(R))
    arrays.update(pad_case(R))
    for key in ("C1", "C2", "C3", "C5"):
        arrays.update(workload_case(R, key))
    np.savez_compressed(OUT / "batch_meta.npz", **arrays)


def quantize_fixture(R):
    """The reference's weight quantisers on seeded weights, including rows and
    groups that are constant (amax 0 / hi == lo) and values on exact .5 code
    ties, for the GEMV tests' weight builders."""
    rng = np.random.default_rng(99)
    arrays = {}
    w8 = (rng.standard_normal((37, 200)) * 0.05).astype(np.float32)
    w8[3] = 0.0
    w8[4, :] = 0.25
    w8[5, :8] = np.float32(127.0) * np.array([1, -1, 0.5, -0.5, 1.5, -2.5, 0, 126.5], np.float32) / 127
    q8 = np.empty(w8.shape, np.int8)
    s8 = np.empty(w8.shape[0], np.uint16)
    R.ref_quantize_int8_rows(p(w8), *w8.shape, p(q8), p(s8))
    arrays.update(w8=w8, q8=q8, s8=s8)
    for g in (32, 64, 128):
        w4 = (rng.standard_normal((20, 256)) * 0.05).astype(np.float32)
        w4[2, :g] = 0.125  # hi == lo
        w4[3, :g] = np.linspace(0, 15, g).astype(np.float32)  # ties at x.5 codes
        n, k = w4.shape
        packed = np.empty((n, k // 2), np.uint8)
        s4 = np.empty((n, k // g), np.uint16)
        o4 = np.empty_like(s4)
        R.ref_quantize_int4_groups(p(w4), n, k, g, p(packed), p(s4), p(o4))
        arrays.update({f"w4_{g}": w4, f"packed_{g}": packed, f"s4_{g}": s4, f"o4_{g}": o4})
    np.savez_compressed(OUT / "quantize.npz", **arrays)


def main():
    oracle.build(ref=True)
    R = oracle.ref()
    if sys.argv[1:] == ["quantize"]:  # only the quantiser fixture
        quantize_fixture(R)
        return
    half_fixture(R)
    rope_fixture(R)
    batch_fixture(R)
    quantize_fixture(R)
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
