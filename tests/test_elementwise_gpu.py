"""Parity of the elementwise HIP kernels (through the C ABI) with the CPU
oracle: embedding gather / gather_rows / resolve_input_ids bit-exact; fused
add + RMSNorm residual bit-exact and output within fp16 tolerance; SwiGLU
within fp16 tolerance.  Cases follow tests/cuda/test_kernels.cu:18-69 and the
workload shapes (Llama-3.1-8B decode b32 and mixed prefill, Qwen2-7B 16k)."""
import numpy as np
import pytest

import oracle
from tests._util import assert_bits_equal, assert_close_f16, randn_f16, rel_max_err, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401  (fails loudly without librlk.so)
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


# ---------------------------------------------------------------- embedding

@pytest.mark.parametrize("vocab,hidden,n", [(50, 64, 4), (32000, 2048, 1), (1000, 4096, 32),
                                            (997, 3584, 300), (64, 8, 5), (300, 4104, 2049)])
def test_embedding_bit_exact(torch_cuda, vocab, hidden, n):
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"embedding vocab={vocab} hidden={hidden} n={n}")
    rng = np.random.default_rng(vocab + hidden + n)
    table = randn_f16(rng, (vocab, hidden), 0.02)
    ids = rng.integers(0, vocab, n, dtype=np.int32)
    ids[0], ids[-1] = vocab - 1, 0
    out = torch.empty((n, hidden), dtype=torch.float16, device="cuda")
    K.embedding_lookup(dev(torch, ids), dev(torch, table), n, hidden, out)
    assert_bits_equal(host(out), oracle.embedding_lookup(ids, table, hidden), "embedding")


@pytest.mark.parametrize("bs,nt", [(64, 1), (256, 1), (128, 0)])
def test_embedding_launch_policies(torch_cuda, bs, nt):
    """The gather under each block width and cache policy (launch-policy
    knobs) is bit-exact, including a ragged final workgroup."""
    torch = torch_cuda
    from redline_amd import kernels as K
    from redline_amd._lib import tune_knob
    say(f"embedding policy bs={bs} nt={nt}")
    rng = np.random.default_rng(bs + nt)
    for vocab, hidden, n in ((1000, 4096, 37), (64, 8, 5), (300, 4104, 129)):
        table = randn_f16(rng, (vocab, hidden), 0.02)
        ids = rng.integers(0, vocab, n, dtype=np.int32)
        out = torch.empty((n, hidden), dtype=torch.float16, device="cuda")
        with tune_knob("RLK_TUNE_GATHER_BS", bs), tune_knob("RLK_TUNE_GATHER_NT", nt):
            K.embedding_lookup(dev(torch, ids), dev(torch, table), n, hidden, out)
        assert_bits_equal(host(out), oracle.embedding_lookup(ids, table, hidden), "embedding")


def test_embedding_full_vocab_zipf(torch_cuda):
    """Qwen2-7B-shaped gather (152064 x 3584) with Zipf(1.1) ids: every row
    equals the table row it names (size-independent check on the device)."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say("embedding qwen2 full table zipf")
    g = torch.Generator(device="cuda").manual_seed(5)
    table = (torch.randn((152064, 3584), generator=g, device="cuda") * 0.02).half()
    rng = np.random.default_rng(7)
    ids = ((rng.zipf(1.1, 16384) - 1) % 152064).astype(np.int32)
    d_ids = dev(torch, ids)
    out = torch.empty((16384, 3584), dtype=torch.float16, device="cuda")
    K.embedding_lookup(d_ids, table, 16384, 3584, out)
    want = table.index_select(0, d_ids.long())
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("vocab,hidden,n,eps", [(50, 64, 4, 1e-5), (4096, 4096, 32, 1e-5),
                                                (997, 3584, 300, 1e-6), (64, 8, 5, 1e-5),
                                                (300, 4104, 33, 1e-5), (40, 73728, 3, 1e-5)])
def test_embedding_rmsnorm_matches_two_calls(torch_cuda, vocab, hidden, n, eps):
    """The fused extension equals embedding_lookup + fused_add_rmsnorm(delta =
    None) bit for bit (the same kernel arithmetic), and the oracle's composition
    of the two: residual bit-exact, out within fp16 tolerance.  Covers H = 4096
    (C2's shape and table), the Qwen2 width, H = 8, a ragged 513-vector row and
    the two-pass width (73728)."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"embedding_rmsnorm vocab={vocab} hidden={hidden} n={n}")
    rng = np.random.default_rng(vocab + hidden + n)
    table = randn_f16(rng, (vocab, hidden), 0.02)
    w = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)
    ids = rng.integers(0, vocab, n, dtype=np.int32)
    ids[0], ids[-1] = vocab - 1, 0
    d_ids, d_table, d_w = dev(torch, ids), dev(torch, table), dev(torch, w)
    res = torch.empty((n, hidden), dtype=torch.float16, device="cuda")
    out = torch.empty_like(res)
    K.embedding_rmsnorm(d_ids, d_table, n, hidden, d_w, eps, res, out)
    res2, out2 = torch.empty_like(res), torch.empty_like(res)
    K.embedding_lookup(d_ids, d_table, n, hidden, res2)
    K.fused_add_rmsnorm(res2, None, d_w, n, hidden, eps, out2)
    assert torch.equal(res.view(torch.int16), res2.view(torch.int16))
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    want_res = oracle.embedding_lookup(ids, table, hidden)
    _, want = oracle.fused_add_rmsnorm(want_res, None, w, eps)
    assert_bits_equal(host(res), want_res, "residual")
    assert_close_f16(host(out), want, what="out")


def test_gather_rows_and_resolve(torch_cuda):
    torch = torch_cuda
    from redline_amd import kernels as K
    say("gather_rows / resolve_input_ids")
    rng = np.random.default_rng(3)
    src = randn_f16(rng, (77, 1024))
    cols = src.shape[1]
    idx = rng.integers(0, 77, 40, dtype=np.int32)
    out = torch.empty((40, cols), dtype=torch.float16, device="cuda")
    K.gather_rows(dev(torch, src), dev(torch, idx), 40, cols, out)
    assert_bits_equal(host(out), oracle.gather_rows(src, idx, cols), "gather_rows")

    ids = rng.integers(0, 1000, 600, dtype=np.int32)
    srcr = rng.integers(-1, 64, 600, dtype=np.int32)
    prev = rng.integers(0, 1000, 64, dtype=np.int32)
    d_ids = dev(torch, ids)
    K.resolve_input_ids(d_ids, dev(torch, srcr), dev(torch, prev), 600)
    assert np.array_equal(host(d_ids), oracle.resolve_input_ids(ids, srcr, prev))


# -------------------------------------------------------------- add + RMSNorm

def _norm_case(torch, rows, hidden, eps, seed, delta=True, outliers=0.0, tpr=None, monkeypatch=None):
    from redline_amd import kernels as K
    rng = np.random.default_rng(seed)
    res = randn_f16(rng, (rows, hidden))
    d = randn_f16(rng, (rows, hidden)) if delta else None
    if outliers:
        m = rng.random((rows, hidden)) < outliers
        res = np.where(m, (res.astype(np.float32) * 20).astype(np.float16), res)
    w = (1.0 + rng.standard_normal(hidden, dtype=np.float32) * 0.1).astype(np.float16)
    d_res = dev(torch, res)
    out = torch.empty_like(d_res)
    K.fused_add_rmsnorm(d_res, None if d is None else dev(torch, d), dev(torch, w), rows, hidden,
                        eps, out)
    want_res, want_out = oracle.fused_add_rmsnorm(res, d, w, eps)
    assert_bits_equal(host(d_res), want_res, "residual")
    assert_close_f16(host(out), want_out, what="rmsnorm out")
    return host(out), want_res, w


def test_rmsnorm_reference_case(torch_cuda):
    """tests/cuda/test_kernels.cu:18-46 (rows 5, H 512, w = 1 + N(0, 0.2)),
    then delta == nullptr reduces to plain RMSNorm of the updated residual."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say("rmsnorm reference case")
    rng = np.random.default_rng(1)
    res = randn_f16(rng, (5, 512))
    d = randn_f16(rng, (5, 512))
    w = (1.0 + rng.standard_normal(512, dtype=np.float32) * 0.2).astype(np.float16)
    d_res, d_w = dev(torch, res), dev(torch, w)
    out = torch.empty_like(d_res)
    K.fused_add_rmsnorm(d_res, dev(torch, d), d_w, 5, 512, 1e-5, out)
    want_res, want_out = oracle.fused_add_rmsnorm(res, d, w, 1e-5)
    assert rel_max_err(host(d_res), want_res) <= 1e-3
    assert rel_max_err(host(out), want_out) <= 2e-3
    K.fused_add_rmsnorm(d_res, None, d_w, 5, 512, 1e-5, out)
    assert rel_max_err(host(out), want_out) <= 2e-3
    # torch fp32 reference (unrounded HF formula) of the same op
    r = torch.from_numpy(want_res.astype(np.float32))
    ref = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + 1e-5) * torch.from_numpy(w.astype(np.float32))
    assert rel_max_err(host(out), ref.numpy()) <= 2e-3


@pytest.mark.parametrize("rows,hidden", [(32, 4096), (1, 2048), (7, 8), (3, 520), (2049, 4096),
                                         (33, 3584), (300, 8192), (5, 16384), (2, 40960), (1, 73728),
                                         (4100, 64), (2050, 3584)])
@pytest.mark.parametrize("delta", [True, False])
def test_rmsnorm_shapes(torch_cuda, rows, hidden, delta):
    say(f"rmsnorm rows={rows} hidden={hidden} delta={delta}")
    _norm_case(torch_cuda, rows, hidden, 1e-5, rows * 7 + hidden, delta)


def test_rmsnorm_mixed_prefill_outliers(torch_cuda):
    """C3: 4096 rows x 4096, 1% of activations x20."""
    say("rmsnorm C3 outliers")
    _norm_case(torch_cuda, 4096, 4096, 1e-5, 33, True, outliers=0.01)


def test_rmsnorm_qwen2_16k(torch_cuda):
    """C5: 16384 rows x 3584, eps 1e-6."""
    say("rmsnorm C5")
    _norm_case(torch_cuda, 16384, 3584, 1e-6, 55, True)


def test_rmsnorm_constant_row_closed_form(torch_cuda):
    """A row of constant c normalises to fp16(c / sqrt(c^2 + eps)) * w."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say("rmsnorm constant rows")
    H = 4096
    c = np.array([0.5, -3.0, 1e-3, 100.0], np.float16)
    res = np.repeat(c[:, None], H, 1)
    w = np.full(H, 1.5, np.float16)
    d_res = dev(torch, res)
    out = torch.empty_like(d_res)
    K.fused_add_rmsnorm(d_res, None, dev(torch, w), 4, H, 1e-5, out)
    cf = c.astype(np.float64)
    want = (cf / np.sqrt(cf * cf + 1e-5)).astype(np.float16).astype(np.float32) * 1.5
    for r in range(4):
        assert_close_f16(host(out)[r], np.full(H, want[r], np.float32), what=f"row {r}")


# -------------------------------------------------------------------- SwiGLU

@pytest.mark.parametrize("rows,inter", [(3, 256), (1, 5632), (32, 14336), (4096, 14336),
                                        (5, 8), (2, 18944), (2100, 520)])
@pytest.mark.parametrize("interleaved", [False, True])
def test_swiglu(torch_cuda, rows, inter, interleaved):
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"swiglu rows={rows} inter={inter} interleaved={interleaved}")
    rng = np.random.default_rng(rows + inter)
    gu = randn_f16(rng, (rows, 2 * inter), 2.0 if rows == 3 else 1.0)
    out = torch.empty((rows, inter), dtype=torch.float16, device="cuda")
    fn = K.silu_and_mul_interleaved if interleaved else K.silu_and_mul
    fn(dev(torch, gu), rows, inter, out)
    want = oracle.silu_and_mul(gu, inter, interleaved)
    assert_close_f16(host(out), want, what="swiglu")
    if rows == 3 and not interleaved:
        # tests/cuda/test_kernels.cu:48-59: fp32 unrounded reference, 3e-3.
        g = torch.from_numpy(gu[:, :inter].astype(np.float32))
        u = torch.from_numpy(gu[:, inter:].astype(np.float32))
        ref = torch.nn.functional.silu(g) * u
        assert rel_max_err(host(out), ref.numpy()) <= 3e-3


@pytest.mark.parametrize("inter", [1, 3, 100, 1001])
def test_swiglu_interleaved_any_width(torch_cuda, inter):
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"swiglu interleaved inter={inter}")
    rng = np.random.default_rng(inter)
    gu = randn_f16(rng, (9, 2 * inter))
    out = torch.empty((9, inter), dtype=torch.float16, device="cuda")
    K.silu_and_mul_interleaved(dev(torch, gu), 9, inter, out)
    assert_close_f16(host(out), oracle.silu_and_mul(gu, inter, True), what="swiglu interleaved")


def test_swiglu_special_values(torch_cuda):
    """silu(0) = 0; silu(g) -> g for large g; -> -0 for very negative g; inf up stays inf."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say("swiglu special values")
    g = np.array([0, 20, -20, -100, 60000, 1, -1, 0.5], np.float16)
    u = np.array([5, 1, 1, 1, 1, 0, 2, -3], np.float16)
    gu = np.concatenate([g, u])[None, :]
    out = torch.empty((1, 8), dtype=torch.float16, device="cuda")
    K.silu_and_mul(dev(torch, gu), 1, 8, out)
    got = host(out)[0].astype(np.float32)
    want = oracle.silu_and_mul(gu, 8)[0].astype(np.float32)
    assert_close_f16(got, want, what="special")
    assert got[0] == 0 and got[1] == 20 and abs(got[2]) < 1e-6 and got[3] == 0


def test_swiglu_qwen2_16k_sampled_rows(torch_cuda):
    """C5 shape (16384 x 18944): full launch, oracle on every 64th row."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say("swiglu C5")
    rows, inter = 16384, 18944
    g = torch.Generator(device="cuda").manual_seed(9)
    gu = torch.randn((rows, 2 * inter), generator=g, device="cuda").half()
    out = torch.empty((rows, inter), dtype=torch.float16, device="cuda")
    K.silu_and_mul(gu, rows, inter, out)
    sel = torch.arange(0, rows, 64, device="cuda")
    want = oracle.silu_and_mul(host(gu.index_select(0, sel)), inter)
    assert_close_f16(host(out.index_select(0, sel)), want, what="swiglu C5 rows")
