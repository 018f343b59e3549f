"""Writes tests/golden/kernels_cpp.bin: inputs and expected outputs for
tests/cpp/kernels_gpu_main.cpp, the GPU test that drives the kernels through
the C++ drop-in header (redline::kernels).  The expected outputs come from the
CPU oracle (oracle/), itself pinned by tests/test_oracle.py.

Cases mirror the reference's kernel tests (tests/cuda/test_kernels.cu in
Neil456/Redline), plus the embedding_rmsnorm extension over the embedding case:
fused_add_rmsnorm 5 x 512 with and without delta (:18-47),
silu_and_mul and embedding_lookup (:48-69), rope_and_write_kv FP16 over a
shuffled paged pool and decode attention over the cache it wrote (:90-148,
geometry hq 8, hkv 1, D 64, lengths 48 and 17: :285), and the INT8 KV write
with scales (:289-322: hq 2, hkv 1, D 64, pos 5, slot bs + 3).

Format: b"RLKFIX01", uint32 count, then per array: uint32 name length, name,
uint64 byte count, raw little-endian bytes.  Run: python tests/golden/make_cpp_fixtures.py
"""
from __future__ import annotations

import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "kernels_cpp.bin"


def f16(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def main():
    rng = np.random.default_rng(2024)
    arrs: dict[str, np.ndarray] = {}

    # embedding_lookup: V 64, H 256, 7 ids
    table = f16(rng, 64, 256, scale=0.02)
    ids = rng.integers(0, 64, 7).astype(np.int32)
    emb = oracle.embedding_lookup(ids, table, 256)
    arrs.update(emb_table=table, emb_ids=ids, emb_out=emb)
    # embedding_rmsnorm (extension): the gathered rows, then RMSNorm without delta
    wn = (1 + 0.1 * rng.standard_normal(256)).astype(np.float16)
    arrs.update(embnorm_w=wn, embnorm_out=oracle.fused_add_rmsnorm(emb, None, wn, 1e-5)[1])

    # fused_add_rmsnorm: 5 x 512, eps 1e-5, with delta and without
    res, delta = f16(rng, 5, 512), f16(rng, 5, 512)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(np.float16)
    r1, o1 = oracle.fused_add_rmsnorm(res, delta, w, 1e-5)
    _, o2 = oracle.fused_add_rmsnorm(res, None, w, 1e-5)
    arrs.update(norm_res=res, norm_delta=delta, norm_w=w, norm_res_out=r1, norm_out=o1,
                norm_nodelta_out=o2)

    # silu_and_mul (split and interleaved): 3 rows, inter 256
    gu = f16(rng, 3, 512)
    arrs.update(swiglu_gu=gu, swiglu_out=oracle.silu_and_mul(gu, 256),
                swiglu_il_out=oracle.silu_and_mul(gu, 256, interleaved=True))

    # rope_and_write_kv FP16 + decode attention: hq 8, hkv 1, D 64, lengths 48, 17
    hq, hkv, D, bs, lens = 8, 1, 64, 16, [48, 17]
    stride = (hq + 2 * hkv) * D
    T = sum(lens)
    cos, sin = oracle.rope_cos_sin_tables(1e4, D, max(lens))
    nblk = 1 + sum((n + bs - 1) // bs for n in lens)
    perm = rng.permutation(np.arange(1, nblk)).astype(np.int32)
    max_blocks = (max(lens) + bs - 1) // bs
    tables = np.zeros((len(lens), max_blocks), np.int32)
    pos, slots, nxt = [], [], 0
    for s, n in enumerate(lens):
        nb = (n + bs - 1) // bs
        tables[s, :nb] = perm[nxt:nxt + nb]
        nxt += nb
        for p in range(n):
            pos.append(p)
            slots.append(tables[s, p // bs] * bs + p % bs)
    pos, slots = np.array(pos, np.int32), np.array(slots, np.int32)
    qkv = f16(rng, T, stride)
    q_out = qkv.copy()
    kc = np.zeros((nblk, hkv, bs, D), np.float16)
    vc = np.zeros_like(kc)
    oracle.rope_and_write_kv(q_out, pos, slots, hq, hkv, D, cos, sin, kc, vc)
    items = np.array([lens[0] - 1, T - 1], np.int32)
    seqs = np.array([0, 1], np.int32)
    att = oracle.paged_attention_decode(q_out, stride, hq, D ** -0.5, kc, vc, None, None, tables,
                                        pos, items, seqs, T)
    arrs.update(rope_dims=np.array([T, hq, hkv, D, bs, nblk, len(lens), max_blocks], np.int32),
                rope_qkv=qkv, rope_pos=pos, rope_slots=slots, rope_cos=cos, rope_sin=sin,
                rope_tables=tables, rope_qkv_out=q_out, rope_k_out=kc, rope_v_out=vc,
                att_items=items, att_seqs=seqs, att_out=att[items])

    # INT8 KV write: hq 2, hkv 1, D 64, one token at position 5 into slot bs + 3
    hq8, D8 = 2, 64
    qkv8 = f16(rng, 1, (hq8 + 2) * D8)
    cos8, sin8 = oracle.rope_cos_sin_tables(1e4, D8, 8)
    q8 = qkv8.copy()
    k8 = np.zeros((2, 1, bs, D8), np.int8)
    v8 = np.zeros_like(k8)
    ks8 = np.zeros((2, 1, bs), np.float32)
    vs8 = np.zeros_like(ks8)
    oracle.rope_and_write_kv(q8, np.array([5], np.int32), np.array([bs + 3], np.int32), hq8, 1, D8,
                             cos8, sin8, k8, v8, ks8, vs8, bs, int8=True)
    arrs.update(int8_qkv=qkv8, int8_cos=cos8, int8_sin=sin8, int8_qkv_out=q8, int8_k_out=k8,
                int8_v_out=v8, int8_ks_out=ks8, int8_vs_out=vs8)

    with open(OUT, "wb") as f:
        f.write(b"RLKFIX01")
        f.write(struct.pack("<I", len(arrs)))
        for name, a in arrs.items():
            b = np.ascontiguousarray(a).tobytes()
            f.write(struct.pack("<I", len(name)) + name.encode())
            f.write(struct.pack("<Q", len(b)) + b)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrs)} arrays)")


if __name__ == "__main__":
    main()
