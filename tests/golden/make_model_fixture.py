"""Writes tests/golden/tiny_model_logits.npz: the reference's own fp32 CPU
model (CpuReferenceModel::forward, src/cpu/reference_model.cpp:157-238, built
by `make -C oracle ref`) run on the tiny random model of tests/_util.py
(tiny_model_weights, saved in the reference's safetensors model format with
its model-config metadata from ModelConfig::to_json), over the token pattern
of the reference's engine scoring test, with FP16 weights and with the four
layer projections in the reference's INT4 format (tiny_model_int4_logits.npz).
Only outputs are stored: the
next-token log-probabilities, the argmax of every row and the last row's
logits; the weights are regenerated from their seed by the test.

Run in the container that has the reference:  python tests/golden/make_model_fixture.py
"""
from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from tests._util import (TINY_MODEL, next_token_logprobs, tiny_model_tokens,  # noqa: E402
                         tiny_model_weights)

OUT = {False: Path(__file__).resolve().parent / "tiny_model_logits.npz",
       True: Path(__file__).resolve().parent / "tiny_model_int4_logits.npz"}
SEED = 7


def reference_logits(weights, tokens, int4=False, cfg=TINY_MODEL):
    import safetensors.numpy as st
    import ctypes as C
    R = oracle.ref()
    cbuf = C.create_string_buffer(4096)
    n = R.ref_model_config_json(cfg["vocab"], cfg["hidden"], cfg["inter"], cfg["layers"],
                                cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["theta"],
                                cfg["eps"], int(int4), cbuf, 4096)
    assert n > 0, "the reference rejected the config"
    config_json = cbuf.value.decode()
    with tempfile.TemporaryDirectory() as d:
        path = str(Path(d) / "tiny.rlm")
        st.save_file(weights, path, metadata={"format": "redline", "redline_config": config_json})
        logits = np.empty((tokens.size, cfg["vocab"]), np.float32)
        rc = R.ref_model_forward(path.encode(), oracle.p(tokens), tokens.size, oracle.p(logits))
        assert rc == 0, "the reference model failed"
    return logits


def main():
    oracle.build(ref=True)
    tokens = tiny_model_tokens()
    for int4 in (False, True):
        logits = reference_logits(tiny_model_weights(SEED, int4=int4), tokens, int4)
        np.savez_compressed(OUT[int4], tokens=tokens, seed=np.array(SEED),
                            logprobs=next_token_logprobs(logits, tokens),
                            argmax=logits.argmax(axis=1).astype(np.int32), last_logits=logits[-1])
        print(f"wrote {OUT[int4]} ({OUT[int4].stat().st_size} bytes)")


if __name__ == "__main__":
    main()
