"""The five benchmark/parity workloads of the fused per-layer kernels and the
batch metadata that drives them.

Model shapes (hidden H, intermediate I, query heads Hq, KV heads Hkv, head_dim
D, RoPE theta, vocab V, RMSNorm eps) and row counts T:

  C1  TinyLlama-1.1B decode, batch 1            T = 1      (CPU-reference case)
  C2  Llama-3.1-8B decode, batch 32             T = 32     (headline workload)
  C3  Llama-3.1-8B chunked prefill, mixed rows  T = 4096   (2x1024 prefill + 2048 decode)
  C4  Llama-3.1-8B INT8 KV write                T = 16384
  C5  Qwen2-7B prefill                          T = 16384  (4 x 4096, positions 0..16383)

Batch metadata is produced by the BatchBuilder (host C ABI), exactly as the
engine would produce it: positions and slot_mapping per token, block tables
per sequence.  Block tables are drawn from a pool of `num_blocks` blocks
(block 0 reserved as scratch) such that every KV cell written in the step is
distinct: the blocks holding a step's new positions are taken without
replacement from a random permutation of the pool; the older blocks of a
table (read only by attention) are random pool blocks.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .host import BatchBuilder, LogitsMode


@dataclass(frozen=True)
class ModelShape:
    name: str
    hidden: int
    inter: int
    hq: int
    hkv: int
    head_dim: int
    theta: float
    vocab: int
    eps: float

    @property
    def qkv_cols(self) -> int:
        return (self.hq + 2 * self.hkv) * self.head_dim


TINYLLAMA = ModelShape("TinyLlama-1.1B", 2048, 5632, 32, 4, 64, 1e4, 32000, 1e-5)
LLAMA31_8B = ModelShape("Llama-3.1-8B", 4096, 14336, 32, 8, 128, 5e5, 128256, 1e-5)
QWEN2_7B = ModelShape("Qwen2-7B", 3584, 18944, 28, 4, 128, 1e6, 152064, 1e-6)


@dataclass(frozen=True)
class Segment:
    """One sequence's contribution to the step: positions [start, start + n)."""
    start: int
    n: int


@dataclass
class Workload:
    key: str
    model: ModelShape
    segments: list = field(default_factory=list)
    num_blocks: int = 16384
    max_pos: int = 8192          # RoPE table rows
    kv_int8: bool = False
    outlier_frac: float = 0.0    # fraction of activations scaled x20 (C3)
    kv_outlier_dims: int = 0     # per-head channels with N(0, 8) (C4)
    zipf: float = 0.0            # Zipf exponent of token ids (C5), 0 = uniform
    qkv_bias: bool = False       # Qwen2 QKV bias (applied before RoPE)
    kv_scale_f16: bool = False   # INT8 KV scales stored as fp16 (C4)
    block_size: int = 16
    seed: int = 0

    @property
    def num_tokens(self) -> int:
        return sum(s.n for s in self.segments)


def make_workload(key: str, seed: int = 0) -> Workload:
    rng = np.random.default_rng(seed)
    key = key.upper()
    if key == "C1":
        return Workload("C1", TINYLLAMA, [Segment(int(rng.integers(0, 2048)), 1)],
                        num_blocks=129, max_pos=2048, seed=seed)
    if key == "C2":
        segs = [Segment(int(p), 1) for p in rng.integers(0, 8192, 32)]
        return Workload("C2", LLAMA31_8B, segs, seed=seed)
    if key == "C3":
        segs = [Segment(0, 1024), Segment(3072, 1024)]
        segs += [Segment(int(p), 1) for p in rng.integers(0, 8192, 2048)]
        return Workload("C3", LLAMA31_8B, segs, outlier_frac=0.01, seed=seed)
    if key == "C4":
        segs = [Segment(0, 4096) for _ in range(4)]
        return Workload("C4", LLAMA31_8B, segs, kv_int8=True, kv_outlier_dims=2, kv_scale_f16=True,
                        seed=seed)
    if key == "C5":
        segs = [Segment(4096 * i, 4096) for i in range(4)]
        return Workload("C5", QWEN2_7B, segs, num_blocks=16384, max_pos=16384, zipf=1.1,
                        qkv_bias=True, seed=seed)
    raise ValueError(f"unknown workload {key}")


def block_tables(w: Workload, rng: np.random.Generator) -> list[np.ndarray]:
    """Per-segment block tables; the blocks written in this step are distinct."""
    bs = w.block_size
    pool = rng.permutation(np.arange(1, w.num_blocks, dtype=np.int32))
    nxt = 0
    tables = []
    for s in w.segments:
        nblk = (s.start + s.n + bs - 1) // bs
        first_new = s.start // bs
        t = rng.integers(1, w.num_blocks, nblk, dtype=np.int32)  # history blocks
        k = nblk - first_new
        if nxt + k > pool.size:
            raise ValueError("KV pool too small for the step's writes")
        t[first_new:] = pool[nxt:nxt + k]
        nxt += k
        tables.append(t)
    return tables


def build_batch(w: Workload, rng: np.random.Generator | None = None,
                decode_query_threshold: int = 1):
    """BatchBuilder metadata for the workload.

    Returns (meta int32 buffer, shape, layout dict, tables)."""
    rng = rng if rng is not None else np.random.default_rng(w.seed + 1)
    tables = block_tables(w, rng)
    max_blocks = max(len(t) for t in tables)
    bb = BatchBuilder(w.num_tokens, len(w.segments), len(w.segments), max_blocks, w.block_size,
                      decode_query_threshold)
    for s, t in zip(w.segments, tables):
        tok = np.zeros(s.n, np.int32)
        bb.add(tok, s.start, s.n, None, t, mode=LogitsMode.kLast)
    meta, shape, layout = bb.write()
    return meta, shape, layout, tables


def token_ids(w: Workload, rng: np.random.Generator) -> np.ndarray:
    """Token ids: uniform over the vocab, or Zipf(w.zipf) ranks folded into it."""
    T, V = w.num_tokens, w.model.vocab
    if w.zipf > 0:
        return ((rng.zipf(w.zipf, T) - 1) % V).astype(np.int32)
    return rng.integers(0, V, T, dtype=np.int32)


# Algorithmic HBM bytes per call (each tensor element counted once, read or written).
def bytes_embedding(T, H):
    return T * (4 + 2 * H) + T * 2 * H


def bytes_add_rmsnorm(T, H, delta=True):
    return T * (8 * H if delta else 4 * H) + 2 * H


def bytes_embedding_rmsnorm(T, H):
    """ids and table rows read, residual and normed rows written, weight once."""
    return T * (4 + 6 * H) + 2 * H


def bytes_swiglu(T, I):
    return T * 6 * I


def bytes_rope_kv(T, hq, hkv, D, int8=False, scale16=False, bias=False):
    """qkv read, q written back, K/V cells (and INT8 scales) written, cos/sin
    rows and position/slot read per token; the QKV bias vector once."""
    qkv_read = 2 * (hq + 2 * hkv) * D
    q_write = 2 * hq * D
    kv_write = (2 * hkv * D + (4 if scale16 else 8) * hkv) if int8 else 4 * hkv * D
    return T * (qkv_read + q_write + kv_write + 4 * D + 8) + (qkv_read if bias else 0)


def bytes_decode_attention(contexts, hq, hkv, D, int8=False):
    """K and V rows of every attended key (plus their scales for INT8), the
    query heads read and the output written; split-K partials are workspace
    traffic and not counted."""
    ctx = int(np.sum(contexts))
    elem = 1 if int8 else 2
    kv = ctx * hkv * (2 * D * elem + (8 if int8 else 0))
    return kv + len(contexts) * hq * D * 2 * 2 + ctx // 16 * 4
