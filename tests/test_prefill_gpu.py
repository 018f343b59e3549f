"""Parity of paged prefill attention (through the C ABI) with the CPU oracle.

The oracle evaluates causal softmax attention in float64 over the same cache
contents, with INT8 dequantised through fp16 as the reference's tile loader
does (pinned in tests/test_oracle.py against scipy's softmax, the decode
oracle, closed forms and paging invariance).  The kernel accumulates in fp32
and rounds the output to fp16, so outputs are compared at the fp16 tolerance;
for INT8 the reference test's own bound against unquantised attention (3e-2,
tests/cuda/test_kernels.cu:195) is checked too.

Cases follow the reference's run_attention_case (test_kernels.cu:90-280): the
cache is written by this build's rope_and_write_kv from BatchBuilder metadata,
then (1) every sequence is prefilled from position 0, and (2) chunked prefill:
the second half of each sequence attends to the cached first half, with its q
rows gathered into a compact buffer.  Larger cases cover several 64-row query
tiles and 64-key tiles, contexts that are not multiples of either, fp16-stored
INT8 scales, and the Llama-3.1-8B C3 chunks at full size (sampled rows).

Prefill attention has two kernels: one that copies tiles to LDS with load-to-LDS
instructions (the default when the block table fits its LDS copy) and one that
stages them through registers (RLK_TUNE_PREFILL_DMA=0).  At D = 128 the first
gives each wave 32 query rows, or 16 for small grids (RLK_TUNE_PREFILL_QS=1).
Each test runs under the three settings."""
import numpy as np
import pytest

import oracle
import redline_amd as ra
from tests._util import assert_close_f16, randn_f16, rel_max_err, say

pytestmark = pytest.mark.gpu

REF_CASES = [(8, 2, 128, False, [37, 300, 5]), (4, 4, 64, False, [64, 129, 1]),
             (6, 2, 128, False, [700]), (8, 1, 64, False, [48, 17]),
             (8, 2, 128, True, [33, 280]), (4, 2, 64, True, [520])]


@pytest.fixture(autouse=True, params=["dma", "dma16", "reg"])
def kernel_path(request):
    from redline_amd._lib import tune_knob
    with tune_knob("RLK_TUNE_PREFILL_DMA", 0 if request.param == "reg" else 1), \
            tune_knob("RLK_TUNE_PREFILL_QS", 1 if request.param == "dma16" else 2):
        yield request.param


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_prefill(torch, K, d_q, q_stride, hq, scale, layer, d_tables, max_blocks, d_pos, d_meta, lay,
                shape, num_rows, D, scale16=False):
    out = torch.zeros((num_rows, hq * D), dtype=torch.float16, device="cuda")
    p = K.attention_params(d_q, q_stride, out, hq, scale, layer, d_tables, max_blocks, d_pos)
    sl = lambda name: d_meta[lay[name]:]  # noqa: E731
    w = K.prefill_work(sl("prefill_seq"), sl("seq_q_start"), sl("seq_q_len"), sl("seq_ctx_len"),
                       shape.num_prefill_seqs, shape.max_prefill_q_tiles)
    if scale16:
        K.paged_attention_prefill_ex(p, w, K.SCALE_F16)
    else:
        K.paged_attention_prefill(p, w)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def meta_arrays(meta, lay, shape, S):
    g = lambda name, n: meta[lay[name]:lay[name] + n]  # noqa: E731
    return (g("prefill_seq", shape.num_prefill_seqs), g("seq_q_start", S), g("seq_q_len", S),
            g("seq_ctx_len", S))


@pytest.mark.parametrize("hq,hkv,D,int8,lens", REF_CASES)
def test_prefill_attention_reference_geometries(torch_cuda, hq, hkv, D, int8, lens):
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"prefill hq={hq} hkv={hkv} D={D} int8={int8} lens={lens}")
    bs = 16
    rng = np.random.default_rng(hq * 11 + D + sum(lens))
    S, T, max_len = len(lens), sum(lens), max(lens)
    nblocks = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblocks, dtype=np.int32))
    max_blocks = (max_len + bs - 1) // bs
    tables_l, nxt = [], 0
    for L in lens:
        nb = (L + bs - 1) // bs
        tables_l.append(ids[nxt:nxt + nb])
        nxt += nb

    def build(chunk_start):
        b = ra.BatchBuilder(T, S, S, max_blocks, bs, 0)  # every sequence a prefill sequence
        for L, tb in zip(lens, tables_l):
            start = min(chunk_start, L - 1)
            b.add(np.zeros(L - start, np.int32), start, L - start, None, tb)
        return b.write()

    meta, shape, lay = build(0)
    assert shape.num_prefill_seqs == S
    stride = (hq + 2 * hkv) * D
    qkv = randn_f16(rng, (T, stride))
    cos, sin = ra.rope_cos_sin_tables(1e4, D, max_len)
    cache = K.KVCache(1, nblocks, hkv, D, bs, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    d_meta, d_qkv = dev(torch, meta), dev(torch, qkv)
    sl = lambda name, n: d_meta[lay[name]:lay[name] + n]  # noqa: E731
    K.rope_and_write_kv(d_qkv, sl("positions", T), sl("slot_mapping", T), T, hq, dev(torch, cos),
                        dev(torch, sin), cache.layer(0))
    scale = 1 / np.sqrt(D)
    d_tables = d_meta[lay["block_tables"]:]
    got = run_prefill(torch, K, d_qkv, stride, hq, scale, cache.layer(0), d_tables, max_blocks,
                      sl("positions", T), d_meta, lay, shape, T, D)

    # oracle: the same rope into CPU caches, then float64 causal attention
    pos = meta[lay["positions"]:lay["positions"] + T]
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T]
    shape4 = (nblocks, hkv, bs, D)
    kc = np.zeros(shape4, np.int8 if int8 else np.float16)
    vc = np.zeros_like(kc)
    ks = np.zeros(shape4[:3], np.float32) if int8 else None
    vs = np.zeros_like(ks) if int8 else None
    roped = qkv.copy()
    oracle.rope_and_write_kv(roped, pos, slots, hq, hkv, D, cos, sin, kc, vc, ks, vs, bs, int8)
    tables = meta[lay["block_tables"]:lay["block_tables"] + S * max_blocks].reshape(S, max_blocks)
    sid, q_start, q_len, ctx = meta_arrays(meta, lay, shape, S)
    want = oracle.paged_attention_prefill(roped, stride, hq, scale, kc, vc, ks, vs, tables, sid,
                                          q_start, q_len, ctx, T, int8)
    assert_close_f16(got, want, what="prefill")
    if int8:  # the reference test's bound against unquantised attention
        kf, vf = np.zeros(shape4, np.float16), np.zeros(shape4, np.float16)
        r2 = qkv.copy()
        oracle.rope_and_write_kv(r2, pos, slots, hq, hkv, D, cos, sin, kf, vf, block_size=bs)
        exact = oracle.paged_attention_prefill(r2, stride, hq, scale, kf, vf, None, None, tables,
                                               sid, q_start, q_len, ctx, T)
        assert rel_max_err(got, exact) <= 3e-2

    # (2) chunked prefill: the second half attends to the cached first half
    split = max_len // 2
    meta3, shape3, lay3 = build(split)
    starts = [min(split, L - 1) for L in lens]
    rows = np.concatenate([np.arange(sum(lens[:s]) + starts[s], sum(lens[:s + 1]))
                           for s in range(S)])
    d_cq, d_meta3 = dev(torch, roped[rows]), dev(torch, meta3)
    got3 = run_prefill(torch, K, d_cq, stride, hq, scale, cache.layer(0),
                       d_meta3[lay3["block_tables"]:], max_blocks,
                       d_meta3[lay3["positions"]:], d_meta3, lay3, shape3, len(rows), D)
    assert_close_f16(got3, want[rows], what="chunked prefill")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kv", ["fp16", "int8", "int8_f16scale"])
@pytest.mark.parametrize("bs,pad", [(16, 0), (7, 0), (16, 4100)])
def test_prefill_attention_random_cache_many_tiles(torch_cuda, D, kv, bs, pad, kernel_path):
    """Several query and key tiles per sequence, GQA 4, random cache contents,
    chunks with and without cached context (lengths not multiples of 64).
    Block size 7 puts block boundaries at odd keys inside a tile; a block
    table padded past 4096 columns exceeds the load-to-LDS kernel's LDS copy
    of it (the register-staged kernel runs)."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"prefill random D={D} kv={kv} bs={bs} pad={pad} path={kernel_path}")
    rng = np.random.default_rng(D + len(kv) + bs)
    hq, hkv = 8, 2
    int8 = kv != "fp16"
    chunks = [(0, 190), (333, 75), (64, 64), (0, 1), (1000, 130)]
    lens = [a + b for a, b in chunks]
    S = len(chunks)
    nblk = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblk)).astype(np.int32)
    maxb = max((L + bs - 1) // bs for L in lens) + pad
    tables = np.zeros((S, maxb), np.int32)
    nxt = 0
    for i, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        tables[i, :nb] = ids[nxt:nxt + nb]
        nxt += nb
    shape4 = (nblk, hkv, bs, D)
    if int8:
        kc = rng.integers(-127, 128, shape4).astype(np.int8)
        vc = rng.integers(-127, 128, shape4).astype(np.int8)
        kscl = (rng.random(shape4[:3]) * 0.02 + 0.001).astype(np.float32)
        vscl = (rng.random(shape4[:3]) * 0.02 + 0.001).astype(np.float32)
        if kv == "int8_f16scale":  # the values the fp16 cells hold
            kscl = kscl.astype(np.float16).astype(np.float32)
            vscl = vscl.astype(np.float16).astype(np.float32)
    else:
        kc, vc = randn_f16(rng, shape4), randn_f16(rng, shape4)
        kscl = vscl = None
    q_len = np.array([b for _, b in chunks], np.int32)
    q_start = np.concatenate([[0], np.cumsum(q_len)[:-1]]).astype(np.int32)
    ctx = np.array(lens, np.int32)
    T = int(q_len.sum())
    q = randn_f16(rng, (T, hq * D))
    scale = 1 / np.sqrt(D)
    sid = np.arange(S, dtype=np.int32)
    want = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc, vc, kscl, vscl, tables, sid,
                                          q_start, q_len, ctx, T, int8)

    cache = K.KVCache(1, nblk, hkv, D, bs, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ksc, vsc = cache.tensors(0)
    k.copy_(dev(torch, kc))
    v.copy_(dev(torch, vc))
    if int8:
        if kv == "int8_f16scale":
            ksc.view(-1).view(torch.float16)[:kscl.size].copy_(dev(torch, kscl.astype(np.float16).ravel()))
            vsc.view(-1).view(torch.float16)[:vscl.size].copy_(dev(torch, vscl.astype(np.float16).ravel()))
        else:
            ksc.copy_(dev(torch, kscl))
            vsc.copy_(dev(torch, vscl))
    out = torch.zeros((T, hq * D), dtype=torch.float16, device="cuda")
    # the parameter structs hold raw pointers: keep every device array alive
    d = {name: dev(torch, a) for name, a in (("q", q), ("tables", tables), ("pos", np.zeros(T, np.int32)),
                                            ("sid", sid), ("q_start", q_start), ("q_len", q_len),
                                            ("ctx", ctx))}
    p = K.attention_params(d["q"], hq * D, out, hq, scale, cache.layer(0), d["tables"], maxb, d["pos"])
    w = K.prefill_work(d["sid"], d["q_start"], d["q_len"], d["ctx"], S, int((q_len.max() + 31) // 32))
    if kv == "int8_f16scale":
        K.paged_attention_prefill_ex(p, w, K.SCALE_F16)
    else:
        K.paged_attention_prefill(p, w)
    torch.cuda.synchronize()
    assert_close_f16(out.cpu().numpy(), want, what=f"prefill {kv}")


def test_prefill_attention_llama_c3_chunks(torch_cuda):
    """C3's two prefill chunks at full size (Llama-3.1-8B: 32 heads, 8 kv heads,
    D = 128): 1024 new tokens at offset 0 and 1024 at offset 3072 (after 3072
    cached tokens), random FP16 cache; 24 sampled (row, head) pairs against a
    float64 numpy evaluation."""
    torch = torch_cuda
    from redline_amd import kernels as K
    from scipy.special import softmax
    say("prefill C3 chunks")
    rng = np.random.default_rng(3)
    hq, hkv, D, bs = 32, 8, 128, 16
    chunks = [(0, 1024), (3072, 1024)]
    lens = [a + b for a, b in chunks]
    nblk = 1 + sum(L // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblk)).astype(np.int32)
    maxb = max(lens) // bs
    tables = np.zeros((2, maxb), np.int32)
    tables[0, :lens[0] // bs] = ids[:lens[0] // bs]
    tables[1, :lens[1] // bs] = ids[lens[0] // bs:]
    cache = K.KVCache(1, nblk, hkv, D, bs, K.KVDType.kFP16)
    k, v, _, _ = cache.tensors(0)
    k.copy_(torch.randn(k.shape, device="cuda").half())
    v.copy_(torch.randn(v.shape, device="cuda").half())
    T = 2048
    q = torch.randn((T, hq * D), device="cuda").half()
    out = torch.zeros((T, hq * D), dtype=torch.float16, device="cuda")
    q_len = np.array([1024, 1024], np.int32)
    d = {name: dev(torch, a) for name, a in (
        ("tables", tables), ("pos", np.zeros(T, np.int32)), ("sid", np.arange(2, dtype=np.int32)),
        ("q_start", np.array([0, 1024], np.int32)), ("q_len", q_len), ("ctx", np.array(lens, np.int32)))}
    p = K.attention_params(q, hq * D, out, hq, 1 / np.sqrt(D), cache.layer(0), d["tables"], maxb,
                           d["pos"])
    w = K.prefill_work(d["sid"], d["q_start"], d["q_len"], d["ctx"], 2, 32)
    K.paged_attention_prefill(p, w)
    torch.cuda.synchronize()
    got, qh = out.cpu().numpy(), q.cpu().numpy()
    kh, vh = k.cpu().numpy().astype(np.float64), v.cpu().numpy().astype(np.float64)
    for s_, row, h in [(0, 0, 0), (0, 63, 5), (0, 64, 31), (0, 1023, 7)] + \
            [(int(a), int(b), int(c)) for a, b, c in zip(rng.integers(0, 2, 20),
                                                        rng.integers(0, 1024, 20),
                                                        rng.integers(0, hq, 20))]:
        past = chunks[s_][0]
        js = np.arange(past + row + 1)
        blk = tables[s_, js // bs]
        kk, vv = kh[blk, h // 4, js % bs], vh[blk, h // 4, js % bs]
        r = 1024 * s_ + row
        sc = (qh[r, h * D:(h + 1) * D].astype(np.float64) @ kk.T) * np.float64(np.float32(1 / np.sqrt(D)))
        want = softmax(sc) @ vv
        assert_close_f16(got[r, h * D:(h + 1) * D], want, what=f"C3 s={s_} row={row} h={h}")
    assert not out[:, :].isnan().any()


def test_prefill_attention_errors(torch_cuda):
    torch = torch_cuda
    from redline_amd import kernels as K
    cache = K.KVCache(1, 4, 2, 64, 16, K.KVDType.kFP16)
    q = torch.zeros((4, 4 * 64), dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    z = dev(torch, np.zeros(4, np.int32))
    p = K.attention_params(q, 4 * 64, out, 4, 0.125, cache.layer(0), z, 1, z)
    K.paged_attention_prefill(p, K.prefill_work(z, z, z, z, 0, 1))  # no sequences: no-op
    p.num_heads = 3
    with pytest.raises(ra.Error, match="multiple of num_kv_heads"):
        K.paged_attention_prefill(p, K.prefill_work(z, z, z, z, 1, 1))
    p.num_heads = 4
    p.q_stride = 4 * 64 - 4
    with pytest.raises(ra.Error, match="16-byte aligned"):
        K.paged_attention_prefill(p, K.prefill_work(z, z, z, z, 1, 1))
    torch.cuda.synchronize()
    assert not out.any()


@pytest.mark.parametrize("D", [64, 128])
def test_prefill_attention_rising_scores(torch_cuda, D, kernel_path):
    """Scores that rise with the key position by about 40 (natural units) over
    the context, plus noise: the running max of every row moves again and
    again, past and within the kernel's rescale threshold."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"prefill rising scores D={D} path={kernel_path}")
    rng = np.random.default_rng(77 + D)
    hq, hkv, bs = 4, 2, 16
    past, ql = 700, 300
    L = past + ql
    nblk = 1 + (L + bs - 1) // bs
    tables = rng.permutation(np.arange(1, nblk)).astype(np.int32)[None, :]
    u = np.zeros(D, np.float32)
    u[:8] = 1 / np.sqrt(8)
    scale = 1 / np.sqrt(D)
    drift = 40.0 / scale / 4.0  # q . k grows by 40 / scale over the context
    kc = np.zeros((nblk, hkv, bs, D), np.float16)
    vc = randn_f16(rng, (nblk, hkv, bs, D))
    for pos in range(L):
        b, o = tables[0, pos // bs], pos % bs
        kc[b, :, o] = (rng.standard_normal((hkv, D)) * 0.5 + (pos / L) * drift * u).astype(np.float16)
    q = (rng.standard_normal((ql, hq * D)) * 0.5).astype(np.float32)
    for h in range(hq):
        q[:, h * D:(h + 1) * D] += 4.0 * u
    q = q.astype(np.float16)
    sid = np.zeros(1, np.int32)
    q_start, q_len, ctx = np.zeros(1, np.int32), np.array([ql], np.int32), np.array([L], np.int32)
    want = oracle.paged_attention_prefill(q, hq * D, hq, scale, kc, vc, None, None, tables, sid,
                                          q_start, q_len, ctx, ql, False)
    cache = K.KVCache(1, nblk, hkv, D, bs, K.KVDType.kFP16)
    k, v, _, _ = cache.tensors(0)
    k.copy_(dev(torch, kc))
    v.copy_(dev(torch, vc))
    out = torch.zeros((ql, hq * D), dtype=torch.float16, device="cuda")
    d = {name: dev(torch, a) for name, a in (("q", q), ("tables", tables), ("pos", np.zeros(ql, np.int32)),
                                            ("sid", sid), ("q_start", q_start), ("q_len", q_len),
                                            ("ctx", ctx))}
    p = K.attention_params(d["q"], hq * D, out, hq, scale, cache.layer(0), d["tables"], tables.shape[1],
                           d["pos"])
    w = K.prefill_work(d["sid"], d["q_start"], d["q_len"], d["ctx"], 1, (ql + 31) // 32)
    K.paged_attention_prefill(p, w)
    torch.cuda.synchronize()
    assert_close_f16(out.cpu().numpy(), want, what="prefill rising scores")
