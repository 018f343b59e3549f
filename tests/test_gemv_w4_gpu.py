"""Parity of the INT4 weight-only GEMV and its fused SwiGLU epilogue (through
the C ABI) with the CPU oracle.

The oracle evaluates x . dequant(W)^T in float64 (pinned in tests/test_oracle.py
against a matmul over the weight built before packing, the reference's nibble
order KAT and closed forms).  The kernel sums in fp32 on the matrix cores, so
fp32 outputs are compared with the reference test's own bound (relative max
error 1e-4, tests/cuda/test_gemm.cu:147-154), fp16 outputs at fp16 tolerance,
and the SwiGLU output additionally with the reference's 6e-3 bound
(test_gemm.cu:258-292).  Geometries: the reference test's (n = 97, k = 512,
g = 64, m in 1, 3, 8, 13, 16; inter = 192, k = 256, g = 64), the 128-K chunk
path (g a multiple of 128), m up to 32 (two activation tiles) and the
Llama-3.1-8B gate_up projection (n = 2 x 14336, k = 4096, g = 128)."""

import numpy as np
import pytest

import oracle
import redline_amd as ra
from redline_amd._lib import tune_knob
from tests._util import (assert_close_f16, int4_linear, interleave_rows, randn_f16, rel_max_err,
                         say)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_gemv(torch, x, packed, s, o, g, bias=None, f32=False):
    from redline_amd import kernels as K
    m, k = x.shape
    n = packed.shape[0]
    y = torch.empty((m, n), dtype=torch.float32 if f32 else torch.float16, device="cuda")
    K.gemv_w4a16(dev(torch, x), m, dev(torch, packed), dev(torch, s), dev(torch, o), g,
                 None if bias is None else dev(torch, bias), n, k, y, f32)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def run_swiglu(torch, x, packed, s, o, g):
    from redline_amd import kernels as K
    m, k = x.shape
    n = packed.shape[0]
    y = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
    K.gemv_w4a16_swiglu(dev(torch, x), m, dev(torch, packed), dev(torch, s), dev(torch, o), g, n,
                        k, y)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("g", [64, 128, 256])
@pytest.mark.parametrize("m", [1, 3, 8, 13, 16, 20, 32])
def test_gemv_w4_reference_geometry(torch_cuda, g, m):
    """gemv_weight_only_matches_cpu: odd n exercises the row tail; bias; fp32 and fp16 out."""
    torch = torch_cuda
    say(f"gemv_w4 n=97 k=512 g={g} m={m}")
    rng = np.random.default_rng(100 * g + m)
    n, k = 97, 512
    packed, s, o, _ = int4_linear(rng, n, k, g)
    x = randn_f16(rng, (m, k))
    bias = randn_f16(rng, (n,), 0.1)
    want = oracle.gemv_w4a16(x, packed, s, o, g, bias)
    got32 = run_gemv(torch, x, packed, s, o, g, bias, f32=True)
    assert rel_max_err(got32, want) <= 1e-4
    np.testing.assert_allclose(got32, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
    got16 = run_gemv(torch, x, packed, s, o, g, bias, f32=False)
    assert_close_f16(got16, want.astype(np.float16), what="gemv fp16")


@pytest.mark.parametrize("g,k", [(64, 256), (128, 512), (32, 96), (128, 640)])
@pytest.mark.parametrize("m", [1, 3, 8, 16, 20, 32])
def test_gemv_w4_swiglu_interleaved_rows(torch_cuda, g, k, m):
    """gemv_w4a16_swiglu_interleaved_rows: [gate; up] quantised, rows interleaved
    as the loader stores them; compared with the oracle's fused epilogue and
    with silu(gate) * up of the float64 projection (the reference's bound)."""
    torch = torch_cuda
    say(f"gemv_w4_swiglu inter=192 k={k} g={g} m={m}")
    rng = np.random.default_rng(1200 + m + g)
    inter = 192
    packed, s, o, w = int4_linear(rng, 2 * inter, k, g)
    pi, si, oi = interleave_rows(packed), interleave_rows(s), interleave_rows(o)
    x = randn_f16(rng, (m, k))
    got = run_swiglu(torch, x, pi, si, oi, g)
    want = oracle.gemv_w4a16_swiglu(x, pi, si, oi, g)
    assert_close_f16(got, want, what="swiglu")
    y = x.astype(np.float64) @ w.T
    gate, up = y[:, :inter], y[:, inter:]
    exact = gate / (1 + np.exp(-gate)) * up
    assert rel_max_err(got, exact) <= 6e-3


@pytest.mark.parametrize("m", [1, 8, 32])
def test_gemv_w4_swiglu_llama_gate_up(torch_cuda, m):
    """Llama-3.1-8B gate_up at decode: n = 28672 interleaved rows, k = 4096, g = 128."""
    torch = torch_cuda
    say(f"gemv_w4_swiglu llama m={m}")
    rng = np.random.default_rng(7 + m)
    n, k, g = 2 * 14336, 4096, 128
    packed, s, o, _ = int4_linear(rng, n, k, g, dense=False)
    x = randn_f16(rng, (m, k))
    got = run_swiglu(torch, x, packed, s, o, g)
    want = oracle.gemv_w4a16_swiglu(x, packed, s, o, g)
    assert_close_f16(got, want, what="llama swiglu")


@pytest.mark.parametrize("cfg", range(16))
def test_gemv_w4_launch_policies_agree(torch_cuda, cfg):
    """Every selectable launch policy gives the same result as the default
    (bit-identical is not required: split-K order differs)."""
    torch = torch_cuda
    say(f"gemv_w4 cfg={cfg}")
    rng = np.random.default_rng(cfg)
    n, k, g, m = 200, 1024, 128, 9
    packed, s, o, _ = int4_linear(rng, n, k, g)
    x = randn_f16(rng, (m, k))
    want = oracle.gemv_w4a16(x, packed, s, o, g)
    with tune_knob("RLK_TUNE_W4_CFG", cfg):
        got = run_gemv(torch, x, packed, s, o, g, f32=True)
    assert rel_max_err(got, want) <= 1e-4


@pytest.mark.parametrize("cfg", [12, 13, 14, 15])
@pytest.mark.parametrize("n,k,g", [(592, 1024, 128), (592, 1024, 256), (12368, 512, 128),
                                   (160, 2048, 512)])
@pytest.mark.parametrize("m", [1, 9, 17, 32])
def test_gemv_w4_kslice_shapes(torch_cuda, cfg, n, k, g, m):
    """The K-slice kernel (each wave one K slice of every tile of its
    workgroup, x in registers, partials added in LDS) on the shapes it takes:
    rows in whole 16-row tiles, K a whole number of slices; one tile per
    workgroup (n = 592: 37 tiles) and several, with the last workgroup
    partial (n = 12368: 773 tiles); groups of 1, 2 and 4 chunks.  fp32 out
    against the float64 oracle at the reference's bound, and the SwiGLU
    epilogue at fp16 tolerance."""
    torch = torch_cuda
    say(f"gemv_w4 kslice cfg={cfg} n={n} k={k} g={g} m={m}")
    rng = np.random.default_rng(cfg * 1000 + m + k)
    packed, s, o, _ = int4_linear(rng, n, k, g, dense=False)
    x = randn_f16(rng, (m, k))
    bias = randn_f16(rng, (n,), 0.1)
    want = oracle.gemv_w4a16(x, packed, s, o, g, bias)
    with tune_knob("RLK_TUNE_W4_CFG", cfg):
        got = run_gemv(torch, x, packed, s, o, g, bias, f32=True)
        got_sw = run_swiglu(torch, x, packed, s, o, g)
    assert rel_max_err(got, want) <= 1e-4
    assert_close_f16(got_sw, oracle.gemv_w4a16_swiglu(x, packed, s, o, g), what="kslice swiglu")


@pytest.mark.parametrize("cfg", [12, 13])
@pytest.mark.parametrize("m", [1, 16, 32])
def test_gemv_w4_kslice_llama_gate_up(torch_cuda, cfg, m):
    torch = torch_cuda
    say(f"gemv_w4_swiglu kslice cfg={cfg} llama m={m}")
    rng = np.random.default_rng(70 + m)
    n, k, g = 2 * 14336, 4096, 128
    packed, s, o, _ = int4_linear(rng, n, k, g, dense=False)
    x = randn_f16(rng, (m, k))
    with tune_knob("RLK_TUNE_W4_CFG", cfg):
        got = run_swiglu(torch, x, packed, s, o, g)
    assert_close_f16(got, oracle.gemv_w4a16_swiglu(x, packed, s, o, g), what="llama kslice")


@pytest.mark.parametrize("m", [9, 32])
def test_gemv_w4_kslice_fp32_k4096_row_scales(torch_cuda, m):
    """fp32 output of the default kernel above m = 8 at k = 4096 (the
    Llama-3.1-8B hidden size), activation rows scaled from 1e-3 to 1e3: its
    codes carry a bias of 1024 on half the elements, which the per-chunk
    sum(x * bias) takes out again in fp32, so each row's error stays relative
    to that row.  Every row within the reference's 1e-4 of its own largest
    output."""
    torch = torch_cuda
    say(f"gemv_w4 kslice fp32 k=4096 row scales m={m}")
    rng = np.random.default_rng(500 + m)
    n, k, g = 1024, 4096, 128
    packed, s, o, _ = int4_linear(rng, n, k, g, dense=False)
    scales = np.logspace(-3, 3, m).astype(np.float32)
    x = (randn_f16(rng, (m, k)).astype(np.float32) * scales[:, None]).astype(np.float16)
    want = oracle.gemv_w4a16(x, packed, s, o, g)
    got = run_gemv(torch, x, packed, s, o, g, f32=True)
    for r in range(m):
        assert rel_max_err(got[r], want[r]) <= 1e-4, (r, rel_max_err(got[r], want[r]))


@pytest.mark.parametrize("m", [9, 17])
def test_gemv_w4_kslice_tiles_cut_to_lds(torch_cuda, m):
    """The default (K-slice) kernel above m = 8 at a shape whose partial sums
    for one workgroup per CU would overflow LDS (n = 40960: 2560 tiles, 10 per
    workgroup; at two activation tiles that is 160 KiB of partials), so the
    launcher gives each workgroup fewer tiles.  Checked on 1024 sampled
    (gate, up) column pairs against the oracle."""
    torch = torch_cuda
    say(f"gemv_w4_swiglu kslice lds-cut n=40960 m={m}")
    rng = np.random.default_rng(4096 + m)
    n, k, g = 40960, 4096, 128
    packed, s, o, _ = int4_linear(rng, n, k, g, dense=False)
    x = randn_f16(rng, (m, k))
    got = run_swiglu(torch, x, packed, s, o, g)
    cols = np.sort(rng.choice(n // 2, 1024, replace=False))
    rows = np.stack([2 * cols, 2 * cols + 1], axis=1).reshape(-1)
    want = oracle.gemv_w4a16_swiglu(x, packed[rows], s[rows], o[rows], g)
    assert_close_f16(got[:, cols], want, what="kslice lds-cut")


def test_gemv_w4_deterministic_and_errors(torch_cuda):
    torch = torch_cuda
    from redline_amd import kernels as K
    say("gemv_w4 determinism/errors")
    rng = np.random.default_rng(3)
    n, k, g, m = 64, 256, 64, 5
    packed, s, o, _ = int4_linear(rng, n, k, g)
    x = randn_f16(rng, (m, k))
    a = run_gemv(torch, x, packed, s, o, g, f32=True)
    b = run_gemv(torch, x, packed, s, o, g, f32=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    dx, dw, ds, do = (dev(torch, v) for v in (x, packed, s, o))
    y = torch.zeros((40, n), dtype=torch.float16, device="cuda")
    with pytest.raises(ra.Error, match="multiples of 32"):
        K.gemv_w4a16(dx, m, dw, ds, do, 48, None, n, k, y)
    with pytest.raises(ra.Error, match="multiples of 32"):
        K.gemv_w4a16(dx, m, dw, ds, do, 64, None, n, 250, y)
    with pytest.raises(ra.Error, match="unsupported m"):
        K.gemv_w4a16(torch.zeros((33, k), dtype=torch.float16, device="cuda"), 33, dw, ds, do, g,
                     None, n, k, y)
    with pytest.raises(ra.Error, match="even"):
        K.gemv_w4a16_swiglu(dx, m, dw, ds, do, g, n - 1, k, y)
    with pytest.raises(ra.Error, match="16-byte aligned"):
        K.gemv_w4a16(dx.view(-1)[4:], 1, dw, ds, do, g, None, n, k, y)
    K.gemv_w4a16(dx, 0, dw, ds, do, g, None, n, k, y)  # m = 0: no-op
    torch.cuda.synchronize()
    assert not y.any()
