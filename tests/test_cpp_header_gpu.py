"""The kernels launched through the C++ drop-in header (redline::kernels,
include/redline_amd/kernels.h) by a compiled program, as the reference's own
kernel tests call them (tests/cuda/test_kernels.cu:18-69,90-148,289-322 in
Neil456/Redline): embedding (and the embedding_rmsnorm extension), add+RMSNorm
with and without delta, SwiGLU
split and interleaved, RoPE + FP16 paged-KV write, decode attention over that
cache, and the INT8 KV write with scales, against the oracle's fixtures in
tests/golden/kernels_cpp.bin (bit-exact for the gather, residual, q, cells,
codes and scales; fp16 tolerance 2e-3 abs + 1e-2 rel for norm, SwiGLU and
attention).  The program is built by build() into tests/cpp/bin/."""
import subprocess
from pathlib import Path

import pytest

from tests._util import say

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "bin" / "kernels_gpu"
FIXTURE = ROOT / "tests" / "golden" / "kernels_cpp.bin"


@pytest.mark.gpu
def test_cpp_header_kernels_on_gpu():
    assert EXE.exists(), f"{EXE} is missing: run __graft_entry__.build() first"
    say("C++ header program tests/cpp/bin/kernels_gpu")
    r = subprocess.run([str(EXE), str(FIXTURE)], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("PASS"), r.stdout + r.stderr
