"""End-to-end parity with the reference's own CPU model: the tiny random model
of tests/_util.py run through the reference's CpuReferenceModel::forward
(src/cpu/reference_model.cpp:157-238; fixture tests/golden/tiny_model_logits.npz
from tests/golden/make_model_fixture.py) against the forward pass composed from
this library's layer kernels (tests/_tiny_model.py).  The bar is the
reference's own for its fp16 engine against that CPU model
(tests/cuda/test_engine.cpp:99-124): per-token next-token log-probability
error mean < 0.03, max < 0.3.  The CPU test composes the oracle's functions
(pins the oracle end to end); the GPU tests the HIP kernels, as a 150-token
prefill and as a prefill of 149 tokens plus one decode step."""
import numpy as np
import pytest

import oracle
from tests._tiny_model import GpuModel, forward_oracle
from tests._util import next_token_logprobs, say, tiny_model_tokens, tiny_model_weights


def _check(lp, want, what):
    err = np.abs(lp - want)
    say(f"{what}: logprob error mean {err.mean():.4f} max {err.max():.4f}")
    assert err.mean() < 0.03 and err.max() < 0.3, (what, err.mean(), err.max())


def test_fixture_matches_reference_model():
    """The committed fixture is what the compiled reference computes for these
    weights (where the reference tree exists)."""
    if not oracle.has_ref():
        pytest.skip("compiled reference core not present")
    from tests.golden.make_model_fixture import SEED, reference_logits
    z = np.load("tests/golden/tiny_model_logits.npz")
    tokens = tiny_model_tokens()
    logits = reference_logits(tiny_model_weights(SEED), tokens)
    assert np.array_equal(z["tokens"], tokens)
    np.testing.assert_allclose(next_token_logprobs(logits, tokens), z["logprobs"], atol=1e-6)


def test_oracle_model_matches_reference(golden):
    z = golden("tiny_model_logits.npz")
    tokens = z["tokens"]
    logits = forward_oracle(tiny_model_weights(int(z["seed"])), tokens)
    _check(next_token_logprobs(logits, tokens), z["logprobs"], "oracle composition")
    assert (logits.argmax(axis=1) == z["argmax"]).mean() > 0.95


@pytest.mark.gpu
def test_gpu_model_prefill_matches_reference(golden):
    import torch
    z = golden("tiny_model_logits.npz")
    tokens = z["tokens"]
    say("tiny model e2e: prefill of 150 tokens")
    m = GpuModel(torch, tiny_model_weights(int(z["seed"])), tokens.size)
    logits = m.step(tokens, 0, tokens.size)
    _check(next_token_logprobs(logits, tokens), z["logprobs"], "HIP kernels, prefill")
    assert (logits.argmax(axis=1) == z["argmax"]).mean() > 0.95


@pytest.mark.gpu
def test_gpu_model_decode_step_matches_reference(golden):
    """Prefill of the first 149 tokens, then the last token as a decode step
    attending to the cache the prefill wrote: its logits row against the
    reference's last row."""
    import torch
    z = golden("tiny_model_logits.npz")
    tokens = z["tokens"]
    n = tokens.size
    say("tiny model e2e: prefill 149 + decode 1")
    m = GpuModel(torch, tiny_model_weights(int(z["seed"])), n)
    pre = m.step(tokens[:-1], 0, n)
    _check(next_token_logprobs(pre, tokens[:-1]), z["logprobs"][:-1], "HIP kernels, prefill of 149")
    last = m.step(tokens[-1:], n - 1, n)[0].astype(np.float64)
    want = z["last_logits"].astype(np.float64)
    ls = lambda v: v - v.max() - np.log(np.exp(v - v.max()).sum())  # noqa: E731
    err = np.abs(ls(last) - ls(want))
    say(f"decode step: log-softmax error over the vocabulary max {err.max():.4f}")
    assert err.max() < 0.3 and int(last.argmax()) == int(z["argmax"][-1])


def test_oracle_int4_model_matches_reference(golden):
    """The same with the four layer projections in the reference's INT4
    format (the oracle composition multiplies by the dequantized weights)."""
    z = golden("tiny_model_int4_logits.npz")
    tokens = z["tokens"]
    logits = forward_oracle(tiny_model_weights(int(z["seed"]), int4=True), tokens)
    _check(next_token_logprobs(logits, tokens), z["logprobs"], "oracle composition, INT4 weights")


@pytest.mark.gpu
def test_gpu_int4_model_decode_steps_match_reference(golden):
    """INT4 weights: prefill of the first 146 tokens (dequantized weights, as
    the reference engine's prefill GEMM), then the last 4 tokens as decode
    steps whose projections run on the INT4 GEMV kernels, gate_up on the fused
    SwiGLU epilogue: each step's next-token log-probability, and the last
    step's whole row, against the reference's INT4 model."""
    import torch
    z = golden("tiny_model_int4_logits.npz")
    tokens = z["tokens"]
    n = tokens.size
    say("tiny INT4 model e2e: prefill 146 + 4 decode steps")
    m = GpuModel(torch, tiny_model_weights(int(z["seed"]), int4=True), n)
    pre = m.step(tokens[:n - 4], 0, n)
    _check(next_token_logprobs(pre, tokens[:n - 4]), z["logprobs"][:n - 5], "INT4 prefill")
    rows = [pre[-1]]
    for t in range(n - 4, n):
        rows.append(m.step(tokens[t:t + 1], t, n)[0])
    logits = np.stack(rows)  # predictions after tokens n-5 .. n-1
    lp = next_token_logprobs(logits, tokens[n - 5:])  # rows after tokens n-5 .. n-2
    _check(lp, z["logprobs"][n - 5:], "INT4 decode steps (GEMV kernels)")
    ls = lambda v: v - v.max() - np.log(np.exp(v - v.max()).sum())  # noqa: E731
    err = np.abs(ls(logits[-1].astype(np.float64)) - ls(z["last_logits"].astype(np.float64)))
    say(f"INT4 last decode row: log-softmax error max {err.max():.4f}")
    assert err.max() < 0.3
