"""The multi-threaded CPU port of the layer step (oracle/cpu_step.cpp, the
bench's CPU baseline) against the oracle on the same seeded inputs: the
gather, the residual, the RoPE'd q and the KV cells (FP16 and INT8 codes and
scales) bit for bit; the normed output and SwiGLU within the fp16 tolerance
(max abs 2e-3, rel 1e-2).  1 and 3 threads, so row ranges split unevenly."""
import numpy as np
import pytest

import oracle


def _step(fn, pool, a, extra=()):
    p = oracle.p
    args = (p(a["ids"]), p(a["table"]), a["T"], a["H"], p(a["emb"]), p(a["res"]), p(a["delta"]),
            p(a["w"]), np.float32(a["eps"]).item(), p(a["normed"]), p(a["qkv"]), p(a["pos"]),
            p(a["slot"]), a["hq"], a["hkv"], a["D"], p(a["cos"]), p(a["sin"]), p(a["kc"]),
            p(a["vc"]), p(a["ks"]), p(a["vs"]), 16, int(a["int8"]), p(a["gu"]), a["I"],
            p(a["act"])) + tuple(extra)
    fn(*((pool,) + args if pool is not None else args))


def _inputs(rng, int8, D):
    T, H, I, hq, hkv, V, nblk = 7, 64, 40, 4, 2, 50, 8
    f16 = lambda *s: rng.standard_normal(s).astype(np.float16).view(np.uint16)  # noqa: E731
    cos, sin = oracle.rope_cos_sin_tables(1e4, D, 64)
    slots = rng.permutation(nblk * 16)[:T].astype(np.int32)
    slots[2] = -1
    cdt = np.int8 if int8 else np.uint16
    return dict(
        T=T, H=H, I=I, hq=hq, hkv=hkv, D=D, eps=1e-5, int8=int8,
        ids=rng.integers(0, V, T).astype(np.int32), table=f16(V, H), emb=np.zeros((T, H), np.uint16),
        res=f16(T, H), delta=f16(T, H), w=(1 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16),
        normed=np.zeros((T, H), np.uint16), qkv=f16(T, (hq + 2 * hkv) * D),
        pos=rng.integers(0, 64, T).astype(np.int32), slot=slots, cos=cos, sin=sin,
        kc=np.zeros((nblk, hkv, 16, D), cdt), vc=np.zeros((nblk, hkv, 16, D), cdt),
        ks=np.zeros((nblk, hkv, 16), np.float32), vs=np.zeros((nblk, hkv, 16), np.float32),
        gu=f16(T, 2 * I), act=np.zeros((T, I), np.uint16))


@pytest.mark.parametrize("threads", [1, 3])
@pytest.mark.parametrize("int8,D", [(False, 128), (True, 128), (False, 64)])
def test_cpu_step_matches_oracle(threads, int8, D):
    rng = np.random.default_rng(threads * 10 + D + int8)
    a = _inputs(rng, int8, D)
    b = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in a.items()}
    _step(oracle.lib().orc_layer_step, None, a)
    L = oracle.cpu_step_lib()
    pool = L.cps_create(threads)
    if not pool:
        pytest.skip("CPU lacks AVX2/F16C")
    try:
        _step(L.cps_layer_step, pool, b)
    finally:
        L.cps_destroy(pool)
    for k in ("emb", "res", "qkv", "kc", "vc", "ks", "vs"):
        assert np.array_equal(a[k], b[k]), k
    for k in ("normed", "act"):
        x, y = a[k].view(np.float16).astype(np.float64), b[k].view(np.float16).astype(np.float64)
        assert np.all(np.abs(x - y) <= 2e-3 + 1e-2 * np.abs(x)), k


def test_affinity_cores():
    assert oracle.cpu_step_lib().cps_affinity_cores() >= 1


def test_cpu_step_timed_same_results_and_op_times():
    """cps_layer_step_timed: the same outputs as cps_layer_step on the same
    inputs, and each of the five ops' wall times added to its slot (the
    bench's per-kernel CPU figures)."""
    rng = np.random.default_rng(5)
    a = _inputs(rng, False, 128)
    b = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in a.items()}
    L = oracle.cpu_step_lib()
    pool = L.cps_create(2)
    if not pool:
        pytest.skip("CPU lacks AVX2/F16C")
    t = np.zeros(5, np.float64)
    try:
        _step(L.cps_layer_step, pool, a)
        _step(L.cps_layer_step_timed, pool, b, (oracle.p(t),))
    finally:
        L.cps_destroy(pool)
    for k in ("emb", "res", "normed", "qkv", "kc", "vc", "act"):
        assert np.array_equal(a[k], b[k]), k
    assert np.all(t > 0) and t.sum() < 10.0


def test_cpu_step_swiglu_wide_gate():
    """The port's vectorised exp over gates from -100 to 100 (its clamps at
    -87.3 and 88.7 included): SwiGLU within the fp16 tolerance of the oracle."""
    rng = np.random.default_rng(11)
    a = _inputs(rng, False, 64)
    g = np.linspace(-100, 100, a["T"] * a["I"]).reshape(a["T"], a["I"]).astype(np.float16)
    u = rng.uniform(-2, 2, (a["T"], a["I"])).astype(np.float16)
    a["gu"] = np.ascontiguousarray(np.concatenate([g, u], axis=1)).view(np.uint16)
    b = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in a.items()}
    _step(oracle.lib().orc_layer_step, None, a)
    L = oracle.cpu_step_lib()
    pool = L.cps_create(2)
    if not pool:
        pytest.skip("CPU lacks AVX2/F16C")
    try:
        _step(L.cps_layer_step, pool, b)
    finally:
        L.cps_destroy(pool)
    x, y = a["act"].view(np.float16).astype(np.float64), b["act"].view(np.float16).astype(np.float64)
    assert np.all(np.abs(x - y) <= 2e-3 + 1e-2 * np.abs(x))
