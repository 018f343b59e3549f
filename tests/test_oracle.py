"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something it does not share code or
formula with: the reference's own outputs (golden vectors written by the
compiled reference host core), the KATs of the reference's tests, closed forms
and invariants, and float64 mathematics.  Rounding points are pinned by
"tie-masked exactness": the float64 value of each fp16 rounding step is
computed independently and, wherever it is not within a sliver of an fp16
rounding tie (where fp32 evaluation order may legitimately decide), the oracle
must agree bit for bit — so a dropped or extra rounding, a wrong sign, a
swapped operand or a different rounding rule fails.
"""
import numpy as np
import pytest

import oracle
from tests._util import randn_f16

F16_ULP_TOL = 2e-3  # fraction of an fp16 ulp around a tie that is masked


def f16_tie_distance(x):
    """Distance (in fp16 ulps) of float64 values to the nearest fp16 rounding tie."""
    x = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -14)))
    ulp = 2.0 ** (e - 10)
    q = x / ulp
    return np.abs(q - np.floor(q) - 0.5)


def safe(*xs):
    m = np.ones(np.shape(xs[0]), bool)
    for x in xs:
        m &= f16_tie_distance(x) > F16_ULP_TOL
    return m


def to16(x64):
    return np.asarray(x64, np.float64).astype(np.float16)


# ------------------------------------------------------------------ fp16 bits

def test_f2h_matches_reference_outputs(golden):
    g = golden("half_f2h.npz")
    got = oracle.f2h(g["x"])
    assert np.array_equal(got, g["y"])


def test_f2h_kats_and_numpy():
    # tests/cpp/test_core.cpp:97-112
    assert oracle.f2h(np.array([1.0, -2.0, 1e6, 1.0009765625, 1.00048828125], np.float32)).tolist() \
        == [0x3C00, 0xC000, 0x7C00, 0x3C01, 0x3C00]
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-20, 12, 20000))).astype(np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.f2h(x), x.astype(np.float16).view(np.uint16))


def test_h2f_exhaustive():
    h = oracle.lib().orc_h2f
    allh = np.arange(65536, dtype=np.uint16)
    want = allh.view(np.float16).astype(np.float32)
    got = np.array([h(int(v)) for v in allh], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


@pytest.mark.skipif(not oracle.has_ref(), reason="compiled reference core not present")
def test_f2h_exhaustive_against_compiled_reference():
    R = oracle.ref()
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    want = np.empty(x.size, np.uint16)
    R.ref_float_to_half_many(oracle.p(x), x.size, oracle.p(want))
    assert np.array_equal(oracle.f2h(x), want)


# --------------------------------------------------------------- RoPE tables

def test_rope_tables_match_reference(golden):
    g = golden("rope_tables.npz")
    pos = g["positions"]
    for i, (theta, D, sc, f, lo, hi, old) in enumerate(g["cases"]):
        c, s = oracle.rope_cos_sin_tables(theta, int(D), int(pos.max()) + 1, int(sc), f, lo, hi,
                                          int(old))
        assert np.array_equal(c[pos].view(np.uint32), g[f"cos_{i}"].view(np.uint32)), i
        assert np.array_equal(s[pos].view(np.uint32), g[f"sin_{i}"].view(np.uint32)), i


def test_rope_tables_closed_form():
    c, s = oracle.rope_cos_sin_tables(1e4, 64, 100)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    inv = 1.0 / 1e4 ** (np.arange(32) * 2 / 64)
    ang = np.arange(100)[:, None] * inv[None, :]
    assert np.max(np.abs(c - np.cos(ang))) < 2e-5  # fp32 angle at p <= 99
    assert np.max(np.abs(s - np.sin(ang))) < 2e-5


# ----------------------------------------------------------------- embedding

def test_embedding_is_a_row_copy():
    rng = np.random.default_rng(2)
    table = rng.integers(-2048, 2048, (300, 64)).astype(np.float16)  # exact integers
    ids = rng.integers(0, 300, 77).astype(np.int32)
    assert np.array_equal(oracle.embedding_lookup(ids, table, 64), table[ids])
    assert np.array_equal(oracle.gather_rows(table, ids, 64), table[ids])
    prev = rng.integers(0, 1000, 8).astype(np.int32)
    src = np.array([-1, 0, 7, -1, 3], np.int32)
    ids5 = np.array([5, 6, 7, 8, 9], np.int32)
    assert oracle.resolve_input_ids(ids5, src, prev).tolist() == [5, prev[0], prev[7], 8, prev[3]]


# -------------------------------------------------------------- RMSNorm

def test_rmsnorm_rounding_points_float64():
    """out = fp16(fp16(r * inv) * w), r = fp16(res + delta), inv from the
    float64 mean square (elementwise.cu:45,52,61; test_kernels.cu:26-39)."""
    rng = np.random.default_rng(3)
    rows, H = 64, 512
    res, d = randn_f16(rng, (rows, H)), randn_f16(rng, (rows, H))
    w = (1 + 0.2 * rng.standard_normal(H)).astype(np.float16)
    new_res, out = oracle.fused_add_rmsnorm(res, d, w, 1e-5)
    r64 = res.astype(np.float64) + d.astype(np.float64)
    m = safe(r64)
    assert np.array_equal(new_res[m], to16(r64)[m])
    r = new_res.astype(np.float64)
    inv = 1.0 / np.sqrt((r * r).mean(1, keepdims=True) + 1e-5)
    t = r * inv
    y = to16(t).astype(np.float64) * w.astype(np.float64)
    m = safe(t, y)
    assert m.mean() > 0.98
    assert np.array_equal(out[m], to16(y)[m])
    # dropping the intermediate rounding would change many results
    assert np.mean(to16(t * w) != to16(y)) > 0.01


def test_rmsnorm_null_delta_and_constant_rows():
    rng = np.random.default_rng(4)
    res = randn_f16(rng, (3, 256))
    w = np.full(256, 2.0, np.float16)
    r1, out1 = oracle.fused_add_rmsnorm(res, None, w, 1e-5)
    assert np.array_equal(r1, res)  # residual untouched
    z = np.zeros_like(res)
    _, out0 = oracle.fused_add_rmsnorm(res, z, w, 1e-5)
    assert np.array_equal(out1, out0)  # adding zero == no delta
    c = np.repeat(np.array([[0.5], [-3.0], [100.0]], np.float16), 256, 1)
    _, oc = oracle.fused_add_rmsnorm(c, None, w, 1e-5)
    cf = np.array([0.5, -3.0, 100.0])
    want = to16(to16(cf / np.sqrt(cf * cf + 1e-5)).astype(np.float64) * 2.0)
    assert np.array_equal(oc, np.repeat(want[:, None], 256, 1))


# ----------------------------------------------------------------- SwiGLU

def test_swiglu_rounding_points_float64():
    """out = fp16(fp16(silu(g)) * u) (elementwise.cu:66-82), silu from float64."""
    rng = np.random.default_rng(5)
    rows, I = 16, 1024
    gu = randn_f16(rng, (rows, 2 * I), 2.0)
    out = oracle.silu_and_mul(gu, I)
    g, u = gu[:, :I].astype(np.float64), gu[:, I:].astype(np.float64)
    s = g / (1 + np.exp(-g))
    y = to16(s).astype(np.float64) * u
    m = safe(s, y)
    assert m.mean() > 0.98
    assert np.array_equal(out[m], to16(y)[m])
    # interleaved layout of the same numbers gives the same outputs
    inter = np.empty_like(gu)
    inter[:, 0::2], inter[:, 1::2] = gu[:, :I], gu[:, I:]
    assert np.array_equal(oracle.silu_and_mul(inter, I, interleaved=True), out)


def test_swiglu_special_values():
    g = np.array([0, 30, -30, -100, 1, -1], np.float16)
    u = np.array([3, 1, 1, 1, 2, 2], np.float16)
    out = oracle.silu_and_mul(np.concatenate([g, u])[None], 6)[0].astype(np.float64)
    assert out[0] == 0 and out[1] == 30 and abs(out[2]) < 1e-6 and out[3] == 0
    assert out[4] == float(to16(to16(1 / (1 + np.exp(-1.0))) * 2.0))


# ---------------------------------------------------------------- RoPE + KV

def _rope(qkv, pos, slots, hq, hkv, D, nblocks, int8, theta=1e4, bs=16):
    cos, sin = oracle.rope_cos_sin_tables(theta, D, int(pos.max()) + 1)
    kc = np.zeros((nblocks, hkv, bs, D), np.int8 if int8 else np.float16)
    vc = np.zeros_like(kc)
    ks = np.zeros((nblocks, hkv, bs), np.float32) if int8 else None
    vs = np.zeros_like(ks) if int8 else None
    out = qkv.copy()
    oracle.rope_and_write_kv(out, pos, slots, hq, hkv, D, cos, sin, kc, vc, ks, vs, bs, int8)
    return out, kc, vc, ks, vs, cos, sin


def _rotate64(x, pos, cos, sin):
    """float64 rotate-half on [..., D] with the fp32 table values."""
    h = x.shape[-1] // 2
    c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
    x0, x1 = x[..., :h], x[..., h:]
    return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], -1)


def test_rope_fp16_against_float64_rotation():
    rng = np.random.default_rng(6)
    T, hq, hkv, D = 40, 4, 2, 128
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    pos = rng.integers(0, 500, T).astype(np.int32)
    slots = rng.permutation(np.arange(16, 16 * 8)).astype(np.int32)[:T]
    out, kc, vc, _, _, cos, sin = _rope(qkv, pos, slots, hq, hkv, D, 8, False)
    heads = qkv.reshape(T, -1, D).astype(np.float64)
    rot = np.stack([_rotate64(heads[t], pos[t], cos, sin) for t in range(T)])
    o = out.reshape(T, -1, D)
    m = safe(rot[:, :hq])
    assert np.array_equal(o[:, :hq][m], to16(rot[:, :hq])[m])          # q roped in place
    assert np.array_equal(o[:, hq:], qkv.reshape(T, -1, D)[:, hq:])    # k, v sections untouched
    blk, off = slots // 16, slots % 16
    for t in range(T):
        for h in range(hkv):
            kk = kc[blk[t], h, off[t]]
            m = safe(rot[t, hq + h])
            assert np.array_equal(kk[m], to16(rot[t, hq + h])[m])
            assert np.array_equal(vc[blk[t], h, off[t]], heads[t, hq + hkv + h].astype(np.float16))
    # untouched cells stay zero
    written = np.zeros((8, 16), bool)
    written[blk, off] = True
    assert not np.any(kc.transpose(0, 2, 1, 3)[~written])


def test_rope_slot_kats_and_skip():
    # tests/cpp/test_core.cpp:365-367: slots 13*4+1, 20*4+3, 22*4+0 at block size 4
    rng = np.random.default_rng(7)
    hq, hkv, D = 2, 1, 64
    qkv = randn_f16(rng, (4, (hq + 2 * hkv) * D))
    pos = np.array([9, 3, 8, 0], np.int32)
    slots = np.array([13 * 4 + 1, 20 * 4 + 3, 22 * 4 + 0, -1], np.int32)
    out, kc, vc, _, _, _, _ = _rope(qkv, pos, slots, hq, hkv, D, 24, False, bs=4)
    for t, (b, o) in enumerate([(13, 1), (20, 3), (22, 0)]):
        assert np.array_equal(vc[b, 0, o], qkv[t, (hq + hkv) * D:].astype(np.float16))
    nz = {(b, o) for b, o in zip(*np.nonzero(np.any(vc[:, 0] != 0, -1)))}
    assert nz == {(13, 1), (20, 3), (22, 0)}  # slot -1 wrote nothing
    # position 0 is the identity rotation
    assert np.array_equal(out[3], qkv[3])


def test_rope_int8_codes_and_scales():
    """INT8 (rope_kv.cu:71-85): scale = amax/127 over the fp16-rounded head,
    codes = round-half-even(x / scale) clamped to +/-127; checked against
    float64 wherever x/scale is not within a sliver of a .5 tie; the
    reference test bound |code * scale - x| <= 0.51 scale; amax 0 -> scale 1."""
    rng = np.random.default_rng(8)
    T, hq, hkv, D = 64, 2, 2, 128
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    qkv.reshape(T, -1, D)[:, hq:, 5] *= 8  # per-head outlier channel
    qkv.reshape(T, -1, D)[3, hq + 1] = 0   # an all-zero k head
    pos = rng.integers(0, 300, T).astype(np.int32)
    slots = (np.arange(T) + 16).astype(np.int32)
    out16, kc16, vc16, _, _, _, _ = _rope(qkv, pos, slots, hq, hkv, D, 6, False)
    out8, kc8, vc8, ks, vs, _, _ = _rope(qkv, pos, slots, hq, hkv, D, 6, True)
    assert np.array_equal(out16, out8)
    blk, off = slots // 16, slots % 16
    for cache16, cache8, scales in ((kc16, kc8, ks), (vc16, vc8, vs)):
        x = cache16[blk, :, off].astype(np.float64)            # [T, hkv, D] fp16 values
        q = cache8[blk, :, off].astype(np.float64)
        sc = scales[blk, :, off].astype(np.float64)[..., None]
        amax = np.abs(x).max(-1, keepdims=True)
        want_sc = np.where(amax > 0, (amax.astype(np.float32) / np.float32(127)), 1.0)
        assert np.array_equal(sc, want_sc)
        assert np.all(np.abs(q * sc - x) <= 0.51 * sc)
        r = x / sc
        far = np.abs(np.abs(r - np.floor(r)) - 0.5) > 1e-4
        assert np.array_equal(q[far], np.clip(np.rint(r[far]), -127, 127))
        assert np.all(np.abs(q).max(-1)[amax[..., 0] > 0] == 127)
    assert ks[blk[3], 1, off[3]] == 1.0 and not np.any(kc8[blk[3], 1, off[3]])


def test_rope_int8_ties_round_half_even():
    """A V head (no rotation) with amax = 127/64 has scale exactly 2^-6, so
    values (n + 0.5)/64 sit exactly on ties: __float2int_rn rounds them to
    even (rope_kv.cu:80,82)."""
    hq, hkv, D = 1, 1, 128
    n = np.arange(D) % 126
    v = ((n + 0.5) / 64).astype(np.float16)
    v[0] = np.float16(127 / 64)
    v[1::2] *= -1
    qkv = np.zeros((1, (hq + 2 * hkv) * D), np.float16)
    qkv[0, (hq + hkv) * D:] = v
    _, _, vc, _, vs, _, _ = _rope(qkv, np.array([0], np.int32), np.array([16], np.int32),
                                  hq, hkv, D, 2, True)
    assert vs[1, 0, 0] == np.float32(2.0 ** -6)
    want = np.rint(v.astype(np.float64) * 64)  # numpy rint: half to even
    assert np.array_equal(vc[1, 0, 0].astype(np.float64), want)
    assert np.any(np.abs(v.astype(np.float64) * 64 % 1) == 0.5)


def test_rope_bias_extension_equivalence():
    """With a QKV bias the result equals the plain function applied to
    fp16(qkv + bias) (the reference adds the bias in its QKV GEMM epilogue,
    linear.cpp:108), except that qkv's k/v sections stay unbiased."""
    rng = np.random.default_rng(9)
    T, hq, hkv, D = 20, 4, 2, 128
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    bias = randn_f16(rng, ((hq + 2 * hkv) * D,), 0.02)
    pos = rng.integers(0, 200, T).astype(np.int32)
    slots = (np.arange(T) + 16).astype(np.int32)
    cos, sin = oracle.rope_cos_sin_tables(1e6, D, 200)
    kc_a, vc_a = np.zeros((4, hkv, 16, D), np.float16), np.zeros((4, hkv, 16, D), np.float16)
    a = qkv.copy()
    oracle.rope_and_write_kv(a, pos, slots, hq, hkv, D, cos, sin, kc_a, vc_a, bias=bias)
    biased = (qkv.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    kc_b, vc_b = np.zeros_like(kc_a), np.zeros_like(vc_a)
    b = biased.copy()
    oracle.rope_and_write_kv(b, pos, slots, hq, hkv, D, cos, sin, kc_b, vc_b)
    assert np.array_equal(a[:, :hq * D], b[:, :hq * D])
    assert np.array_equal(a[:, hq * D:], qkv[:, hq * D:])
    assert np.array_equal(kc_a, kc_b) and np.array_equal(vc_a, vc_b)


def test_rope_fp16_scale_extension():
    """scale16 = fp16(amax/127); codes = rint(x / scale16) (tie-masked float64),
    within 1 of the fp32-scale codes; |code*scale16 - x| <= 0.51*scale16 +
    the clamp at 127 when rounding the scale down pushes amax/scale16 > 127."""
    rng = np.random.default_rng(10)
    T, hq, hkv, D = 48, 2, 2, 128
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    pos = rng.integers(0, 100, T).astype(np.int32)
    slots = (np.arange(T) + 16).astype(np.int32)
    cos, sin = oracle.rope_cos_sin_tables(1e4, D, 100)
    shape = (5, hkv, 16, D)
    k16 = np.zeros(shape, np.float16)
    v16 = np.zeros_like(k16)
    oracle.rope_and_write_kv(qkv.copy(), pos, slots, hq, hkv, D, cos, sin, k16, v16)
    k8, v8 = np.zeros(shape, np.int8), np.zeros(shape, np.int8)
    ks, vs = np.zeros(shape[:3], np.uint16), np.zeros(shape[:3], np.uint16)
    oracle.rope_and_write_kv(qkv.copy(), pos, slots, hq, hkv, D, cos, sin, k8, v8, ks, vs,
                             int8=True, scale16=True)
    k8f, v8f = np.zeros(shape, np.int8), np.zeros(shape, np.int8)
    ksf, vsf = np.zeros(shape[:3], np.float32), np.zeros(shape[:3], np.float32)
    oracle.rope_and_write_kv(qkv.copy(), pos, slots, hq, hkv, D, cos, sin, k8f, v8f, ksf, vsf,
                             int8=True)
    blk, off = slots // 16, slots % 16
    for c16, c8, sc, c8f in ((k16, k8, ks, k8f), (v16, v8, vs, v8f)):
        x = c16[blk, :, off].astype(np.float64)
        q = c8[blk, :, off].astype(np.float64)
        s = sc[blk, :, off].view(np.float16).astype(np.float64)[..., None]
        amax = np.abs(x).max(-1, keepdims=True)
        assert np.array_equal(s, to16(np.float32(amax) / np.float32(127)).astype(np.float64))
        r = x / s
        far = np.abs(np.abs(r - np.floor(r)) - 0.5) > 1e-4
        assert np.array_equal(q[far], np.clip(np.rint(r[far]), -127, 127))
        assert np.max(np.abs(q - c8f[blk, :, off])) <= 1


# ------------------------------------------------------- paged decode attention

def _attn_case(rng, lens, hq, hkv, D, bs=16, int8=False):
    """Random paged caches for sequences of the given context lengths; one
    decode item per sequence at its last position."""
    nblk = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblk)).astype(np.int32)
    maxb = max((L + bs - 1) // bs for L in lens)
    tables = np.zeros((len(lens), maxb), np.int32)
    nxt = 0
    for i, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        tables[i, :nb] = ids[nxt:nxt + nb]
        nxt += nb
    shape = (nblk, hkv, bs, D)
    if int8:
        kc = rng.integers(-127, 128, shape).astype(np.int8)
        vc = rng.integers(-127, 128, shape).astype(np.int8)
        ks = (rng.random(shape[:3]) * 0.02 + 0.001).astype(np.float32)
        vs = (rng.random(shape[:3]) * 0.02 + 0.001).astype(np.float32)
    else:
        kc, vc = randn_f16(rng, shape), randn_f16(rng, shape)
        ks = vs = None
    T = len(lens)
    q = randn_f16(rng, (T, hq * D))
    pos = np.array([L - 1 for L in lens], np.int32)
    return q, kc, vc, ks, vs, tables, pos


def _dequant(c, s):
    return c.astype(np.float64) if s is None else c.astype(np.float64) * s[..., None]


def _attn_numpy(q, kc, vc, ks, vs, tables, pos, hq, hkv, D, scale, bs=16):
    from scipy.special import softmax
    G = hq // hkv
    K, V = _dequant(kc, ks), _dequant(vc, vs)
    out = np.zeros((len(pos), hq * D))
    for i, p_ in enumerate(pos):
        js = np.arange(p_ + 1)
        blk = tables[i, js // bs]
        for h in range(hq):
            k = K[blk, h // G, js % bs]
            v = V[blk, h // G, js % bs]
            s = (q[i, h * D:(h + 1) * D].astype(np.float64) * np.float64(np.float32(scale))) @ k.T
            out[i, h * D:(h + 1) * D] = softmax(s) @ v
    return out


@pytest.mark.parametrize("int8", [False, True])
def test_attention_against_scipy_softmax(int8):
    rng = np.random.default_rng(20)
    hq, hkv, D = 8, 2, 64
    lens = [1, 37, 300, 16]
    q, kc, vc, ks, vs, tables, pos = _attn_case(rng, lens, hq, hkv, D, int8=int8)
    scale = 1 / np.sqrt(D)
    got = oracle.paged_attention_decode(q, hq * D, hq, scale, kc, vc, ks, vs, tables, pos,
                                        np.arange(4), np.arange(4), 4, int8)
    want = _attn_numpy(q, kc, vc, ks, vs, tables, pos, hq, hkv, D, scale)
    m = safe(want)
    assert np.array_equal(got[m], to16(want)[m])


def test_attention_closed_forms_and_paging_invariance():
    rng = np.random.default_rng(21)
    hq, hkv, D = 4, 1, 128
    q, kc, vc, ks, vs, tables, pos = _attn_case(rng, [50, 200], hq, hkv, D)
    # q = 0: uniform weights, the output is the mean of the V rows
    z = np.zeros_like(q)
    out = oracle.paged_attention_decode(z, hq * D, hq, 0.1, kc, vc, None, None, tables, pos,
                                        np.arange(2), np.arange(2), 2)
    for i, L in enumerate([50, 200]):
        js = np.arange(L)
        mean = vc[tables[i, js // 16], 0, js % 16].astype(np.float64).mean(0)
        for h in range(hq):
            assert np.array_equal(out[i, h * D:(h + 1) * D], to16(mean))
    # a key aligned with q and a large scale: the output is that key's V row
    k_pos = 33
    blk, off = tables[1, k_pos // 16], k_pos % 16
    kc2 = kc.copy()
    kc2[blk, 0, off] = q[1, :D]
    out = oracle.paged_attention_decode(q, hq * D, hq, 50.0, kc2, vc, None, None, tables, pos,
                                        np.arange(2), np.arange(2), 2)
    assert np.array_equal(out[1, :D], vc[blk, 0, off])
    # moving every block to another physical slot (and fixing the tables)
    # leaves the result unchanged
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    a = oracle.paged_attention_decode(q, hq * D, hq, 0.09, kc, vc, None, None, tables, pos,
                                      np.arange(2), np.arange(2), 2)
    b = oracle.paged_attention_decode(q, hq * D, hq, 0.09, kc[perm], vc[perm], None, None,
                                      inv[tables].astype(np.int32), pos, np.arange(2),
                                      np.arange(2), 2)
    assert np.array_equal(a, b)


def test_attention_int8_equals_dequantised_fp64():
    """INT8 attention equals the attention of the dequantised cache (codes x scale)."""
    rng = np.random.default_rng(22)
    hq, hkv, D = 4, 2, 64
    q, kc, vc, ks, vs, tables, pos = _attn_case(rng, [90], hq, hkv, D, int8=True)
    got = oracle.paged_attention_decode(q, hq * D, hq, 0.125, kc, vc, ks, vs, tables, pos,
                                        np.arange(1), np.arange(1), 1, True)
    want = _attn_numpy(q, kc, vc, ks, vs, tables, pos, hq, hkv, D, 0.125)
    m = safe(want)
    assert m.mean() > 0.98 and np.array_equal(got[m], to16(want)[m])


# ------------------------------------------------------------- prefill attention

def _prefill_case(rng, chunks, hq, hkv, D, bs=16, int8=False):
    """Sequences given as (past, q_len): random paged caches holding past + q_len
    positions each; the new tokens' q rows are packed one sequence after the other."""
    lens = [a + b for a, b in chunks]
    q, kc, vc, ks, vs, tables, _ = _attn_case(rng, lens, hq, hkv, D, bs, int8)
    q_len = np.array([b for _, b in chunks], np.int32)
    q_start = np.concatenate([[0], np.cumsum(q_len)[:-1]]).astype(np.int32)
    T = int(q_len.sum())
    q = randn_f16(rng, (T, hq * D))
    return q, kc, vc, ks, vs, tables, q_start, q_len, np.array(lens, np.int32), T


def _prefill_numpy(q, kc, vc, ks, vs, tables, q_start, q_len, ctx, hq, hkv, D, scale, bs=16):
    """float64 causal attention; INT8 dequantised through fp16 as the reference's tile loader does."""
    from scipy.special import softmax
    G = hq // hkv
    if ks is None:
        K, V = kc.astype(np.float64), vc.astype(np.float64)
    else:
        K = (kc.astype(np.float32) * ks[..., None]).astype(np.float16).astype(np.float64)
        V = (vc.astype(np.float32) * vs[..., None]).astype(np.float16).astype(np.float64)
    out = np.zeros((q.shape[0], hq * D))
    for s_ in range(len(q_len)):
        past = ctx[s_] - q_len[s_]
        for i in range(q_len[s_]):
            js = np.arange(past + i + 1)
            blk = tables[s_, js // bs]
            row = q_start[s_] + i
            for h in range(hq):
                k, v = K[blk, h // G, js % bs], V[blk, h // G, js % bs]
                sc = (q[row, h * D:(h + 1) * D].astype(np.float64) @ k.T) * np.float64(np.float32(scale))
                out[row, h * D:(h + 1) * D] = softmax(sc) @ v
    return out


@pytest.mark.parametrize("int8", [False, True])
def test_prefill_attention_against_scipy_softmax(int8):
    rng = np.random.default_rng(30 + int8)
    hq, hkv, D = 4, 2, 64
    chunks = [(0, 37), (50, 20), (0, 1), (16, 16)]
    q, kc, vc, ks, vs, tables, q_start, q_len, ctx, T = _prefill_case(rng, chunks, hq, hkv, D, int8=int8)
    scale = 1 / np.sqrt(D)
    sid = np.arange(len(chunks))
    got = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc, vc, ks, vs, tables, sid, q_start,
                                         q_len, ctx, T, int8)
    want = _prefill_numpy(q, kc, vc, ks, vs, tables, q_start, q_len, ctx, hq, hkv, D, scale)
    m = safe(want)
    assert m.mean() > 0.98 and np.array_equal(got[m], to16(want)[m])


def test_prefill_attention_closed_forms_and_decode_equivalence():
    """A one-token chunk at position p equals decode attention at p (FP16
    cache); the first token of an empty context returns its own V row; moving
    blocks to other physical slots (and the table with them) changes nothing;
    only the rows of the listed sequences are written."""
    rng = np.random.default_rng(31)
    hq, hkv, D, bs = 8, 2, 128, 16
    chunks = [(40, 1), (0, 5), (100, 1)]
    q, kc, vc, ks, vs, tables, q_start, q_len, ctx, T = _prefill_case(rng, chunks, hq, hkv, D, bs)
    scale = 0.125
    sid = np.arange(3)
    got = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc, vc, None, None, tables, sid,
                                         q_start, q_len, ctx, T)
    for s_, row in ((0, 0), (2, 6)):
        dec = oracle.paged_attention_decode(q, hq * D, hq, scale, kc, vc, None, None, tables,
                                            np.array([ctx[s_] - 1] * T, np.int32),
                                            np.array([row]), np.array([s_]), T)
        np.testing.assert_array_equal(got[row].view(np.uint16), dec[row].view(np.uint16))
    blk0 = tables[1, 0]
    for h in range(hq):
        np.testing.assert_array_equal(got[1, h * D:(h + 1) * D].view(np.uint16),
                                      vc[blk0, h // (hq // hkv), 0].view(np.uint16))
    # physical moves: permute every block id and the cache rows with them
    perm = np.concatenate([[0], rng.permutation(np.arange(1, kc.shape[0]))])
    kc2, vc2 = np.empty_like(kc), np.empty_like(vc)
    kc2[perm], vc2[perm] = kc, vc
    moved = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc2, vc2, None, None, perm[tables],
                                           sid, q_start, q_len, ctx, T)
    np.testing.assert_array_equal(moved.view(np.uint16), got.view(np.uint16))
    only = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc, vc, None, None, tables,
                                          np.array([1]), q_start, q_len, ctx, T)
    assert not only[[0, 6]].view(np.uint16).any()
    np.testing.assert_array_equal(only[1:6].view(np.uint16), got[1:6].view(np.uint16))


# ------------------------------------------------------------- INT8 GEMV

def test_gemv_w8_code_kat():
    """Codes are two's complement bytes (int8), one fp16 scale per row applied to
    the sum, then the bias (gemv_weight_only.cu:64-93, :19-44)."""
    k = 32
    w = np.zeros((2, k), np.int8)
    w[0, :5] = [-128, -1, 0, 1, 127]
    w[1, 7] = -7
    s = np.array([0.5, 2.0], np.float16)
    b = np.array([0.25, -1.0], np.float16)
    x = np.zeros((6, k), np.float16)
    for i in range(5):
        x[i, i] = 1
    x[5, 7] = 3
    y = oracle.gemv_w8a16(x, w, s, b)
    np.testing.assert_array_equal(y[:5, 0], [-64 + 0.25, -0.5 + 0.25, 0.25, 0.5 + 0.25, 63.5 + 0.25])
    assert y[5, 1] == -7 * 3 * 2.0 - 1.0 and y[5, 0] == 0.25


def test_gemv_w8_against_float64_matmul():
    from tests._util import int8_linear
    rng = np.random.default_rng(8)
    n, k, m = 41, 272, 6
    q, s, w = int8_linear(rng, n, k)
    x = randn_f16(rng, (m, k))
    bias = randn_f16(rng, (n,), 0.1)
    want = x.astype(np.float64) @ w.T + bias.astype(np.float64)
    np.testing.assert_allclose(oracle.gemv_w8a16(x, q, s, bias), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.gemv_w8a16(x, q, s), want - bias.astype(np.float64),
                               rtol=1e-12, atol=1e-12)


def test_gemv_w8_closed_forms():
    """Zero weight -> bias; one-hot x -> the scaled column; doubling the scale
    doubles y - bias."""
    rng = np.random.default_rng(9)
    n, k = 12, 64
    q = rng.integers(-128, 128, (n, k), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, n).astype(np.float16)
    b = randn_f16(rng, (n,), 0.1)
    x = randn_f16(rng, (3, k))
    np.testing.assert_array_equal(oracle.gemv_w8a16(x, np.zeros_like(q), s, b),
                                  np.broadcast_to(b.astype(np.float64), (3, n)))
    for c in (0, 31, 63):
        e = np.zeros((1, k), np.float16)
        e[0, c] = 1
        np.testing.assert_array_equal(oracle.gemv_w8a16(e, q, s)[0],
                                      q[:, c].astype(np.float64) * s.astype(np.float64))
    y1 = oracle.gemv_w8a16(x, q, s, b) - b.astype(np.float64)
    y2 = oracle.gemv_w8a16(x, q, (2 * s.astype(np.float32)).astype(np.float16), b) - b.astype(np.float64)
    np.testing.assert_allclose(y2, 2 * y1, rtol=1e-14, atol=0)


def test_int8_linear_matches_the_reference_quantiser_rules():
    """The test weights follow quantize_int8_rows: |code| <= 127, the row's
    absmax maps to +-127, codes round half to even against the fp16 scale."""
    from tests._util import int8_linear
    q, s, w = int8_linear(np.random.default_rng(3), 16, 96)
    assert np.abs(q.astype(int)).max() <= 127
    assert np.all(np.abs(q.astype(int)).max(axis=1) >= 126)
    assert w.shape == (16, 96) and s.dtype == np.float16


# ------------------------------------------------------------- INT4 GEMV

def test_gemv_w4_nibble_order_kat():
    """Byte c/2 holds code c, low nibble for even c (tests/cuda/test_gemm.cu:40-45)."""
    k, g = 64, 32
    w = np.zeros((2, k // 2), np.uint8)
    w[0, 0] = 0x21          # codes 1 (c = 0) and 2 (c = 1)
    w[1, 5] = 0xF0          # code 15 at c = 11, code 0 at c = 10
    s = np.ones((2, 2), np.float16)
    o = np.zeros((2, 2), np.float16)
    o[1, 0] = -0.5
    x = np.zeros((3, k), np.float16)
    x[0, 0], x[1, 1], x[2, 11] = 1, 1, 1
    y = oracle.gemv_w4a16(x, w, s, o, g)
    assert y[0, 0] == 1 and y[1, 0] == 2 and y[2, 0] == 0
    assert y[2, 1] == 14.5 and y[0, 1] == -0.5 and y[1, 1] == -0.5


@pytest.mark.parametrize("g", [32, 64, 128])
def test_gemv_w4_against_float64_matmul(g):
    from tests._util import int4_linear
    rng = np.random.default_rng(g)
    n, k, m = 37, 256, 5
    packed, s, o, w = int4_linear(rng, n, k, g)
    x = randn_f16(rng, (m, k))
    bias = randn_f16(rng, (n,), 0.1)
    want = x.astype(np.float64) @ w.T + bias.astype(np.float64)
    got = oracle.gemv_w4a16(x, packed, s, o, g, bias)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_gemv_w4_closed_forms():
    """q = 0 -> offset * sum(x); one-hot x picks the dequantised column."""
    rng = np.random.default_rng(1)
    n, k, g = 8, 128, 32
    s = rng.uniform(0.01, 0.1, (n, k // g)).astype(np.float16)
    o = rng.uniform(-1, 1, (n, k // g)).astype(np.float16)
    x = randn_f16(rng, (2, k))
    y = oracle.gemv_w4a16(x, np.zeros((n, k // 2), np.uint8), s, o, g)
    xs = x.astype(np.float64).reshape(2, k // g, g).sum(-1)
    np.testing.assert_allclose(y, xs @ o.astype(np.float64).T, rtol=1e-12, atol=1e-12)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    for c in (0, 1, 63, 64, 127):
        e = np.zeros((1, k), np.float16)
        e[0, c] = 1
        q = (packed[:, c // 2] >> (4 * (c & 1))) & 15
        col = q * s[:, c // g].astype(np.float64) + o[:, c // g].astype(np.float64)
        np.testing.assert_array_equal(oracle.gemv_w4a16(e, packed, s, o, g)[0], col)


def test_gemv_w4_swiglu_is_interleaved_silu_of_fp16_outputs():
    """The fused epilogue equals the unfused path: fp16 GEMV output, then
    silu_and_mul_interleaved (pinned above), except where float64 -> fp16
    sits on a rounding tie."""
    from tests._util import int4_linear, interleave_rows
    rng = np.random.default_rng(2)
    inter, k, g = 96, 256, 64
    packed, s, o, _ = int4_linear(rng, 2 * inter, k, g)
    packed, s, o = interleave_rows(packed), interleave_rows(s), interleave_rows(o)
    x = randn_f16(rng, (4, k))
    y = oracle.gemv_w4a16(x, packed, s, o, g)
    unfused = oracle.silu_and_mul(to16(y), inter, interleaved=True)
    fused = oracle.gemv_w4a16_swiglu(x, packed, s, o, g)
    ok = safe(y[:, 0::2]) & safe(y[:, 1::2])
    assert ok.mean() > 0.99
    np.testing.assert_array_equal(fused.view(np.uint16)[ok], unfused.view(np.uint16)[ok])


# ------------------------------------------------- GEMV weight quantisers

def test_weight_quantisers_match_reference(golden):
    """The GEMV tests' weight builders (tests/_util.py) quantise exactly as the
    reference's quantize_int8_rows / quantize_int4_groups
    (src/cpu/random_model.cpp:99-140): codes, packing and fp16 scales/offsets
    bit for bit, on the reference's own output (tests/golden/quantize.npz)."""
    from tests._util import int4_quantize_groups, int8_quantize_rows
    z = golden("quantize.npz")
    q, s = int8_quantize_rows(z["w8"])
    assert np.array_equal(q, z["q8"])
    assert np.array_equal(s.view(np.uint16), z["s8"])
    for g in (32, 64, 128):
        packed, s4, o4 = int4_quantize_groups(z[f"w4_{g}"], g)
        assert np.array_equal(packed, z[f"packed_{g}"]), g
        assert np.array_equal(s4.view(np.uint16), z[f"s4_{g}"]), g
        assert np.array_equal(o4.view(np.uint16), z[f"o4_{g}"]), g


@pytest.mark.skipif(not oracle.has_ref(), reason="compiled reference core not present")
def test_weight_quantisers_match_compiled_reference_random():
    from tests._util import int4_quantize_groups, int8_quantize_rows
    R = oracle.ref()
    rng = np.random.default_rng(5)
    for n, k, g in ((64, 512, 128), (9, 96, 32), (33, 1024, 256)):
        w = (rng.standard_normal((n, k)) * rng.uniform(0.01, 1.0)).astype(np.float32)
        q8, s8 = np.empty((n, k), np.int8), np.empty(n, np.uint16)
        R.ref_quantize_int8_rows(oracle.p(w), n, k, oracle.p(q8), oracle.p(s8))
        q, s = int8_quantize_rows(w)
        assert np.array_equal(q, q8) and np.array_equal(s.view(np.uint16), s8)
        pk, s4, o4 = (np.empty((n, k // 2), np.uint8), np.empty((n, k // g), np.uint16),
                      np.empty((n, k // g), np.uint16))
        R.ref_quantize_int4_groups(oracle.p(w), n, k, g, oracle.p(pk), oracle.p(s4), oracle.p(o4))
        a, b, c = int4_quantize_groups(w, g)
        assert np.array_equal(a, pk) and np.array_equal(b.view(np.uint16), s4)
        assert np.array_equal(c.view(np.uint16), o4)
