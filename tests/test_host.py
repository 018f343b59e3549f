"""Host-side checks (no GPU): the C ABI library loads and exports what
include/redline_amd/rlk.h declares; argument errors are reported before any
launch; fp16 conversion, RoPE tables and BatchBuilder metadata match the
reference's own host core bit for bit (golden vectors from
tests/golden/make_golden.py) and the KATs of tests/cpp/test_core.cpp."""
import ctypes as C
import hashlib
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import redline_amd as ra
from redline_amd import _lib
from redline_amd.configs import block_tables, build_batch, make_workload

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "redline_amd" / "rlk.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(rlk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = ra.lib()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), f"librlk.so does not export {n}"
    assert set(names) <= set(_lib.exported_symbols()) | set(names)
    assert b"gfx950" in L.rlk_version()


def test_binding_covers_header():
    assert set(declared_symbols()) == set(_lib.exported_symbols())


# ------------------------------------------------------------- error paths

def _call(name, *args):
    return getattr(ra.lib(), name)(*args)


def test_shape_errors_fail_before_launch():
    L = ra.lib()
    assert L.rlk_embedding_lookup(None, None, 4, 12, None, None) == _lib.RLK_EINVAL
    assert b"multiple of 8" in L.rlk_last_error()
    assert L.rlk_fused_add_rmsnorm(None, None, None, 3, 100, 1e-5, None, None) == _lib.RLK_EINVAL
    assert L.rlk_silu_and_mul(None, 2, 12, None, None) == _lib.RLK_EINVAL
    assert L.rlk_gather_rows(None, None, 2, 4, None, None) == _lib.RLK_EINVAL
    kv = _lib.KVLayerView(None, None, None, None, 16, 2, 96, 0)
    assert L.rlk_rope_and_write_kv(None, None, None, 1, 4, None, None, C.byref(kv), None) == \
        _lib.RLK_EUNSUPPORTED
    assert b"head_dim 96" in L.rlk_last_error()
    kv.head_dim, kv.dtype = 128, 7
    assert L.rlk_rope_and_write_kv(None, None, None, 1, 4, None, None, C.byref(kv), None) == \
        _lib.RLK_EINVAL


def test_null_pointers_fail_before_launch():
    """Required device pointers are checked before anything is launched
    (optional ones -- delta, the gather index, prev_sampled, bias -- may be
    null)."""
    L = ra.lib()
    d = C.c_void_p(16)  # a non-null stand-in: nothing is launched
    assert L.rlk_embedding_lookup(d, None, 4, 16, d, None) == _lib.RLK_EINVAL
    assert b"null pointer" in L.rlk_last_error()
    assert L.rlk_gather_rows(None, None, 2, 8, d, None) == _lib.RLK_EINVAL
    assert L.rlk_fused_add_rmsnorm(d, None, None, 3, 64, 1e-5, d, None) == _lib.RLK_EINVAL
    assert L.rlk_silu_and_mul(d, 2, 16, None, None) == _lib.RLK_EINVAL
    assert L.rlk_silu_and_mul_interleaved(None, 2, 3, d, None) == _lib.RLK_EINVAL
    assert L.rlk_resolve_input_ids(d, None, d, 4, None) == _lib.RLK_EINVAL
    kv = _lib.KVLayerView(d, d, None, None, 16, 2, 128, 1)  # INT8 without scales
    assert L.rlk_rope_and_write_kv(d, d, d, 1, 4, d, d, C.byref(kv), None) == _lib.RLK_EINVAL
    assert b"null pointer" in L.rlk_last_error()
    kv = _lib.KVLayerView(d, d, None, None, 16, 2, 128, 0)
    prm = _lib.AttentionParams(d, 384, d, 4, 0.1, kv, None, 4, d)
    wk = _lib.DecodeAttentionWork(d, d, 2, 1, None, None, None)
    assert L.rlk_paged_attention_decode(C.byref(prm), C.byref(wk), None) == _lib.RLK_EINVAL
    assert b"null pointer" in L.rlk_last_error()
    prm = _lib.AttentionParams(d, 100, d, 4, 0.1, kv, d, 4, d)
    assert L.rlk_paged_attention_decode(C.byref(prm), C.byref(wk), None) == _lib.RLK_EINVAL
    assert b"16-byte aligned" in L.rlk_last_error()


def test_empty_batches_are_noops():
    L = ra.lib()
    assert L.rlk_embedding_lookup(None, None, 0, 12, None, None) == 0  # checked after n <= 0
    assert L.rlk_fused_add_rmsnorm(None, None, None, 0, 4096, 1e-5, None, None) == 0
    assert L.rlk_silu_and_mul(None, -1, 14336, None, None) == 0
    assert L.rlk_silu_and_mul_interleaved(None, 0, 3, None, None) == 0
    assert L.rlk_gather_rows(None, None, 0, 8, None, None) == 0
    assert L.rlk_resolve_input_ids(None, None, None, 0, None) == 0
    kv = _lib.KVLayerView(None, None, None, None, 16, 8, 96, 0)
    assert L.rlk_rope_and_write_kv(None, None, None, 0, 32, None, None, C.byref(kv), None) == 0


def test_cpp_header_throws_redline_error(tmp_path):
    """The C++ interface (same names as redline::kernels) throws redline::Error."""
    src = ROOT / "tests" / "cpp" / "boundary_main.cpp"
    exe = tmp_path / "boundary"
    subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", f"-I{ROOT / 'include'}", str(src),
                    "-o", str(exe), f"-L{ROOT / 'redline_amd'}", "-lrlk",
                    f"-Wl,-rpath,{ROOT / 'redline_amd'}"], check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert "PASS" in out, out


# ------------------------------------------------------------ fp16 bits

def test_half_conversion_matches_reference(golden):
    g = golden("half_f2h.npz")
    f = ra.lib().rlk_float_to_half_bits
    got = np.fromiter((f(float(v)) for v in g["x"]), np.uint16, g["x"].size)
    assert np.array_equal(got, g["y"])


def test_half_conversion_kats():
    # tests/cpp/test_core.cpp:97-112
    assert ra.float_to_half_bits(1.0) == 0x3C00
    assert ra.float_to_half_bits(-2.0) == 0xC000
    assert ra.float_to_half_bits(1e6) == 0x7C00
    assert ra.float_to_half_bits(1.0009765625) == 0x3C01
    assert ra.float_to_half_bits(1.00048828125) == 0x3C00
    for h in range(0, 0x7C00, 7):
        assert ra.float_to_half_bits(ra.half_bits_to_float(h)) == h
    # exhaustive decode against numpy's binary16
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([ra.half_bits_to_float(int(h)) for h in allh], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


# ------------------------------------------------------------ RoPE tables

def test_rope_tables_match_reference(golden):
    g = golden("rope_tables.npz")
    pos = g["positions"]
    for i, (theta, D, sc, f, lo, hi, old) in enumerate(g["cases"]):
        D, sc, old = int(D), int(sc), int(old)
        scaling = {0: "none", 1: "linear", 2: "llama3"}[sc]
        inv = ra.rope_inv_freq(theta, D, scaling, f, lo, hi, old)
        assert np.array_equal(inv, g[f"inv_{i}"]), i
        c, s = ra.rope_cos_sin_tables(theta, D, int(pos.max()) + 1, scaling, f, lo, hi, old)
        assert np.array_equal(c[pos].view(np.uint32), g[f"cos_{i}"].view(np.uint32)), i
        assert np.array_equal(s[pos].view(np.uint32), g[f"sin_{i}"].view(np.uint32)), i


def test_rope_table_kats():
    # tests/cpp/test_core.cpp:160-170: llama3 endpoints, cos[0] = 1, sin(3).
    plain = ra.rope_inv_freq(5e5, 32)
    scaled = ra.rope_inv_freq(5e5, 32, "llama3", 8.0, 1.0, 4.0, 8192)
    assert abs(scaled[0] - plain[0]) <= 1e-12
    assert abs(scaled[-1] - plain[-1] / 8.0) <= 1e-15
    c, s = ra.rope_cos_sin_tables(5e5, 32, 16)
    assert c[0, 0] == 1.0
    assert abs(s[3, 0] - np.sin(3.0)) <= 1e-6


# -------------------------------------------------------- batch metadata

def _kat_builder():
    b = ra.BatchBuilder(64, 8, 16, 4, 4, 2)
    rows = [b.add(None, 9, 1, [5], [11, 12, 13], mode=ra.LogitsMode.kLast),
            b.add([40, 41, 42, 43, 44, 45], 3, 6, None, [20, 21, 22], 0.5, 7, 1.0,
                  (3 << 32) | 9, ra.LogitsMode.kNone),
            b.add([7, 0], 0, 2, [-1, 2], [30], mode=ra.LogitsMode.kAll)]
    return b, rows


def test_batch_builder_kats():
    # tests/cpp/test_core.cpp:334-386
    b, rows = _kat_builder()
    assert rows == [0, -1, 1]
    with pytest.raises(ra.Error, match="too few KV blocks"):
        b.add([40, 41, 42, 43, 44, 45], 10, 6, None, [1, 2])
    buf = np.full(b.max_meta_words(), -7, np.int32)
    buf, s, m = b.write(buf)
    assert (s.num_tokens, s.num_seqs, s.num_logit_rows, s.num_decode_items,
            s.num_prefill_seqs, s.max_prefill_q_tiles, s.max_context) == (9, 3, 3, 3, 1, 1, 10)
    assert buf[m["input_src"]] == 5 and buf[m["input_ids"] + 1] == 40
    assert buf[m["input_src"] + 8] == 2 and buf[m["positions"]] == 9
    assert buf[m["slot_mapping"]] == 13 * 4 + 1
    assert buf[m["slot_mapping"] + 1] == 20 * 4 + 3
    assert buf[m["slot_mapping"] + 6] == 22 * 4 + 0
    assert buf[m["seq_q_start"] + 2] == 7 and buf[m["seq_ctx_len"] + 1] == 9
    assert buf[m["block_tables"] + 6] == 22 and buf[m["block_tables"] + 9] == 0
    assert buf[m["decode_token"] + 1] == 7 and buf[m["decode_seq"] + 2] == 2
    assert buf[m["prefill_seq"]] == 1
    assert buf[m["logit_token"]] == 0 and buf[m["logit_token"] + 2] == 8
    assert buf[m["param_row"] + 2] == 2 and buf[m["top_k"] + 1] == 7
    assert buf[m["seed_lo"] + 1] == 9 and buf[m["seed_hi"] + 1] == 3
    assert buf[m["temperature"] + 1:m["temperature"] + 2].view(np.float32)[0] == 0.5
    assert m["total_words"] <= b.max_meta_words()


def test_batch_builder_matches_reference_buffer(golden):
    g = golden("batch_meta.npz")
    b, rows = _kat_builder()
    try:
        b.add([40, 41, 42, 43, 44, 45], 10, 6, None, [1, 2])
    except ra.Error:
        rows.append(-2)
    assert rows == list(g["kat_rows"])
    buf = np.full(b.max_meta_words(), -7, np.int32)
    buf, s, m = b.write(buf)
    assert np.array_equal(buf, g["kat_buf"])
    assert [getattr(s, f[0]) for f in _lib.BatchShape._fields_] == list(g["kat_shape"])
    assert [m[f] for f in _lib.META_FIELDS] == [int(x) for x in g["kat_layout"]]


def test_batch_builder_graph_padding(golden):
    # tests/cpp/test_core.cpp:388-404: padded rows write the scratch block 0.
    g = golden("batch_meta.npz")
    b = ra.BatchBuilder(64, 8, 16, 4, 16, 1)
    b.add([5], 20, 1, None, [3, 4], mode=ra.LogitsMode.kLast)
    b.pad_decode_to(4)
    buf, s, m = b.write(np.full(b.max_meta_words(), -7, np.int32))
    assert buf[m["slot_mapping"] + 3] == 0
    assert np.array_equal(buf, g["pad_buf"])
    d = ra.BatchBuilder(64, 8, 16, 4, 16, 1)
    d.pad_decode_to(4)
    assert d.shape().num_tokens == s.num_tokens
    assert d.shape().num_decode_items == s.num_decode_items


@pytest.mark.parametrize("key", ["C1", "C2", "C3", "C5"])
def test_workload_metadata_matches_reference(golden, key):
    g = golden("batch_meta.npz")
    w = make_workload(key, seed=0)
    tables = block_tables(w, np.random.default_rng(w.seed + 1))
    tab_hash = hashlib.sha256(b"".join(t.tobytes() for t in tables)).hexdigest()
    assert tab_hash == str(g[f"{key}_tables_sha256"]), "numpy generator drift"
    meta, s, m, _ = build_batch(w)
    T = w.num_tokens
    assert np.array_equal(meta[m["positions"]:m["positions"] + T], g[f"{key}_positions"])
    assert np.array_equal(meta[m["slot_mapping"]:m["slot_mapping"] + T], g[f"{key}_slot_mapping"])
    assert hashlib.sha256(meta[:m["total_words"]].tobytes()).hexdigest() == str(g[f"{key}_sha256"])
    # every KV cell written in the step is distinct (no write races)
    slots = meta[m["slot_mapping"]:m["slot_mapping"] + T]
    assert np.unique(slots).size == T


def test_batch_builder_limits():
    b = ra.BatchBuilder(4, 2, 2, 2, 16, 1)
    with pytest.raises(ra.Error, match="max tokens"):
        b.add(np.zeros(5, np.int32), 0, 5, None, [1])
    with pytest.raises(ra.Error, match="empty"):
        b.add(None, 0, 0, None, [1])
    with pytest.raises(ra.Error, match="no source"):
        b.add(None, 0, 1, None, [1])
    b.add([1], 0, 1, None, [1], mode=ra.LogitsMode.kLast)
    b.add([1], 0, 1, None, [1], mode=ra.LogitsMode.kLast)
    with pytest.raises(ra.Error, match="max sequences"):
        b.add([1], 0, 1, None, [1])


def test_batch_builder_null_block_table():
    L = ra.lib()
    b = L.rlk_batch_builder_create(4, 2, 2, 2, 16, 1)
    try:
        toks = (C.c_int32 * 1)(5)
        st = L.rlk_batch_builder_add(b, toks, 0, 1, None, None, 1, 1.0, 0, 1.0, 0, 0, None)
        assert st == _lib.RLK_EINVAL
        assert b"null block table" in L.rlk_last_error()
    finally:
        L.rlk_batch_builder_destroy(b)


def test_prefill_argument_errors():
    """The prefill launcher validates the KV dtype, the options' scale dtype and
    the grid limits before launching, as the decode launcher does."""
    L = ra.lib()
    d = C.c_void_p(16)  # non-null stand-in: nothing is launched
    kv = _lib.KVLayerView(d, d, d, d, 16, 2, 128, 5)
    prm = _lib.AttentionParams(d, 1024, d, 4, 0.1, kv, d, 4, d)
    wk = _lib.PrefillAttentionWork(d, d, d, d, 2, 1)
    assert L.rlk_paged_attention_prefill(C.byref(prm), C.byref(wk), None) == _lib.RLK_EINVAL
    assert b"unknown KV dtype" in L.rlk_last_error()
    prm.kv.dtype = 0
    opt = _lib.AttentionOptions(7)
    assert L.rlk_paged_attention_prefill_ex(C.byref(prm), C.byref(wk), C.byref(opt), None) == \
        _lib.RLK_EINVAL
    assert b"unknown scale dtype" in L.rlk_last_error()
    wk.num_seqs = 70000
    assert L.rlk_paged_attention_prefill(C.byref(prm), C.byref(wk), None) == _lib.RLK_EINVAL
    assert b"split the call" in L.rlk_last_error()


def test_tune_knobs_set_and_clear():
    """Launch-policy overrides change only through rlk_set_tune_knob once the
    library has started; unknown names are rejected."""
    L = ra.lib()
    assert L.rlk_set_tune_knob(b"RLK_TUNE_ROPE_WPT", 3, 1) == 0
    assert L.rlk_set_tune_knob(b"RLK_TUNE_ROPE_WPT", 0, 0) == 0
    assert L.rlk_set_tune_knob(b"RLK_TUNE_NOPE", 1, 1) == _lib.RLK_EINVAL
    assert b"unknown knob" in L.rlk_last_error()
    assert _lib.get_tune_knob("RLK_TUNE_ROPE_WPT") is None
    with _lib.tune_knob("RLK_TUNE_W4_CFG", 2):
        assert _lib.get_tune_knob("RLK_TUNE_W4_CFG") == 2
    assert _lib.get_tune_knob("RLK_TUNE_W4_CFG") is None
    # a nested override restores the outer value, not "unset"
    with _lib.tune_knob("RLK_TUNE_W8_CFG", 1):
        with _lib.tune_knob("RLK_TUNE_W8_CFG", 3):
            assert _lib.get_tune_knob("RLK_TUNE_W8_CFG") == 3
        assert _lib.get_tune_knob("RLK_TUNE_W8_CFG") == 1
    assert _lib.get_tune_knob("RLK_TUNE_W8_CFG") is None
    v, st = C.c_int(7), C.c_int(7)
    assert L.rlk_get_tune_knob(b"RLK_TUNE_NOPE", C.byref(v), C.byref(st)) == _lib.RLK_EINVAL


def test_embedding_rmsnorm_argument_errors():
    L = ra.lib()
    d = C.c_void_p(16)
    assert L.rlk_embedding_rmsnorm(d, d, 0, 12, d, 1e-5, d, d, None) == 0  # n <= 0: no-op
    assert L.rlk_embedding_rmsnorm(d, d, 4, 12, d, 1e-5, d, d, None) == _lib.RLK_EINVAL
    assert b"multiple of 8" in L.rlk_last_error()
    assert L.rlk_embedding_rmsnorm(d, None, 4, 16, d, 1e-5, d, d, None) == _lib.RLK_EINVAL
    assert b"null pointer" in L.rlk_last_error()


def test_gemv_w8_weight_over_2gib_refused():
    # checked before any launch: the pointers are never dereferenced
    L = ra.lib()
    fake = C.c_void_p(1 << 20)  # 16-byte aligned, never read
    y = C.c_void_p(2 << 20)
    assert L.rlk_gemv_w8a16(fake, 1, fake, fake, None, 65536, 65536, y, 0, None) == \
        _lib.RLK_EUNSUPPORTED
    assert b"exceeds 2 GiB" in L.rlk_last_error()
