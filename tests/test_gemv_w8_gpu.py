"""Parity of the INT8 weight-only GEMV (through the C ABI) with the CPU oracle.

The oracle evaluates (x . codes^T) * scale + bias in float64 (pinned in
tests/test_oracle.py against a numpy matmul, a two's-complement code KAT and
closed forms).  The kernel sums in fp32 on the matrix cores, so fp32 outputs
are compared with the reference test's own bound (relative max error 1e-4,
tests/cuda/test_gemm.cu:134-160) and fp16 outputs at fp16 tolerance.
Geometries: the reference test's (n = 97, k = 512, m in 1, 3, 8, 13, 16, with a
bias), K that is not a multiple of the 128-K chunk pair (16 .. 1040), m up to 32
(two activation tiles), Llama-3.1-8B projections (gate: n = 14336, k = 4096;
down: n = 4096, k = 14336, where x is staged in several passes) and every
launch policy."""

import numpy as np
import pytest

import oracle
import redline_amd as ra
from redline_amd._lib import tune_knob
from tests._util import assert_close_f16, int8_linear, randn_f16, rel_max_err, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_w8(torch, x, q, s, bias=None, f32=False):
    from redline_amd import kernels as K
    m, k = x.shape
    n = q.shape[0]
    y = torch.empty((m, n), dtype=torch.float32 if f32 else torch.float16, device="cuda")
    K.gemv_w8a16(dev(torch, x), m, dev(torch, q), dev(torch, s),
                 None if bias is None else dev(torch, bias), n, k, y, f32)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("f32", [True, False])
@pytest.mark.parametrize("m", [1, 3, 8, 13, 16, 20, 32])
def test_gemv_w8_reference_geometry(torch_cuda, m, f32):
    """tests/cuda/test_gemm.cu:134-160: n = 97 (odd: the row tail), k = 512, bias."""
    say(f"gemv_w8 reference geometry m={m} f32={f32}")
    rng = np.random.default_rng(100 + m)
    n, k = 97, 512
    q, s, _ = int8_linear(rng, n, k)
    bias = randn_f16(rng, (n,), 0.02)
    x = randn_f16(rng, (m, k))
    want = oracle.gemv_w8a16(x, q, s, bias)
    got = run_w8(torch_cuda, x, q, s, bias, f32)
    if f32:
        assert rel_max_err(got, want) <= 1e-4
    else:
        assert_close_f16(got, want, what="w8 f16")


@pytest.mark.parametrize("k", [16, 80, 144, 528, 1040])
@pytest.mark.parametrize("m", [1, 5, 17])
def test_gemv_w8_k_not_a_whole_chunk_pair(torch_cuda, k, m):
    """K % 128 != 0: the staged x is zero past k and code loads past a row's end
    are clamped to the row."""
    say(f"gemv_w8 k={k} m={m}")
    rng = np.random.default_rng(k + m)
    n = 50
    q = rng.integers(-128, 128, (n, k), dtype=np.int8)  # the full int8 range, -128 included
    s = rng.uniform(0.001, 0.01, n).astype(np.float16)
    x = randn_f16(rng, (m, k))
    want = oracle.gemv_w8a16(x, q, s)
    assert rel_max_err(run_w8(torch_cuda, x, q, s, None, True), want) <= 1e-4


@pytest.mark.parametrize("n,k,m", [(14336, 4096, 1), (14336, 4096, 16), (4096, 14336, 4),
                                   (4096, 14336, 32)])
def test_gemv_w8_llama_projections(torch_cuda, n, k, m):
    """Llama-3.1-8B gate (n = 14336, k = 4096) and down (n = 4096, k = 14336;
    x of 4 rows and more is staged in several passes)."""
    say(f"gemv_w8 llama n={n} k={k} m={m}")
    rng = np.random.default_rng(n + m)
    q, s, _ = int8_linear(rng, n, k, 0.02)
    x = randn_f16(rng, (m, k))
    want = oracle.gemv_w8a16(x, q, s)
    got = run_w8(torch_cuda, x, q, s, None, False)
    assert_close_f16(got, want, what="llama w8")


@pytest.mark.parametrize("cfg", range(7))
def test_gemv_w8_launch_policies_agree(torch_cuda, cfg):
    say(f"gemv_w8 cfg={cfg}")
    rng = np.random.default_rng(cfg)
    n, k = 200, 1040
    q, s, _ = int8_linear(rng, n, k)
    for m in (1, 9, 24):
        x = randn_f16(rng, (m, k))
        want = oracle.gemv_w8a16(x, q, s)
        with tune_knob("RLK_TUNE_W8_CFG", cfg):
            got = run_w8(torch_cuda, x, q, s, None, True)
        assert rel_max_err(got, want) <= 1e-4, m


@pytest.mark.parametrize("cfg", [4, 5, 6])
@pytest.mark.parametrize("n,k", [(592, 1024), (12368, 512), (160, 2048), (14336, 4096)])
@pytest.mark.parametrize("m", [1, 9, 17, 32])
def test_gemv_w8_kslice_shapes(torch_cuda, cfg, n, k, m):
    """The INT8 K-slice kernel (each wave one K slice of 512 or 256 codes of
    every tile of its workgroup, codes biased by 1152 and taken out through
    the slice's sum of x) on the shapes it takes: rows in whole 16-row tiles,
    K a whole number of slices (the others fall back to the pair kernel);
    one tile per workgroup and several, the last workgroup partial.  fp32
    with a bias at the reference's bound, and fp16."""
    say(f"gemv_w8 kslice cfg={cfg} n={n} k={k} m={m}")
    rng = np.random.default_rng(cfg * 1000 + m + k)
    q = rng.integers(-128, 128, (n, k), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, n).astype(np.float16)
    bias = randn_f16(rng, (n,), 0.02)
    x = randn_f16(rng, (m, k))
    want = oracle.gemv_w8a16(x, q, s, bias)
    with tune_knob("RLK_TUNE_W8_CFG", cfg):
        got = run_w8(torch_cuda, x, q, s, bias, True)
        got16 = run_w8(torch_cuda, x, q, s, bias, False)
    assert rel_max_err(got, want) <= 1e-4
    assert_close_f16(got16, want, what="w8 kslice f16")


def test_gemv_w8_deterministic_and_errors(torch_cuda):
    torch = torch_cuda
    from redline_amd import kernels as K
    say("gemv_w8 determinism/errors")
    rng = np.random.default_rng(4)
    n, k, m = 64, 256, 5
    q, s, _ = int8_linear(rng, n, k)
    x = randn_f16(rng, (m, k))
    a = run_w8(torch, x, q, s, None, True)
    b = run_w8(torch, x, q, s, None, True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    dx, dq, ds = dev(torch, x), dev(torch, q), dev(torch, s)
    y = torch.zeros((40, n), dtype=torch.float16, device="cuda")
    with pytest.raises(ra.Error, match="K % 16"):
        K.gemv_w8a16(dx, m, dq, ds, None, n, 250, y)
    with pytest.raises(ra.Error, match="unsupported m"):
        K.gemv_w8a16(torch.zeros((33, k), dtype=torch.float16, device="cuda"), 33, dq, ds, None, n, k,
                     y)
    with pytest.raises(ra.Error, match="16-byte aligned"):
        K.gemv_w8a16(dx.view(-1)[4:], 1, dq, ds, None, n, k, y)
    K.gemv_w8a16(dx, 0, dq, ds, None, n, k, y)  # m = 0: no-op
    torch.cuda.synchronize()
    assert not y.any()
