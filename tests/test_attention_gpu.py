"""Parity of paged decode attention (through the C ABI) with the CPU oracle.

The oracle evaluates the softmax attention in float64 over the same cache
contents (pinned in tests/test_oracle.py against scipy's softmax, closed forms
and paging invariance); the kernel accumulates in fp32 and rounds the output
to fp16, so outputs are compared at the fp16 tolerance.  The caches are
written by this build's own rope_and_write_kv from BatchBuilder metadata, as in
the reference's test (tests/cuda/test_kernels.cu:90-280), or filled at random
at the Llama-3.1-8B decode shape (C2)."""
import numpy as np
import pytest

import oracle
import redline_amd as ra
from tests._util import assert_close_f16, randn_f16, rel_max_err, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_attention(torch, K, d_q, q_stride, hq, scale, cache, d_tables, max_blocks, d_pos,
                  d_items, d_seqs, num_items, num_tokens, max_parts):
    D = cache.head_dim
    out = torch.zeros((num_tokens, hq * D), dtype=torch.float16, device="cuda")
    ws = K.DecodeWorkspace(max(num_items, 1), hq, max_parts, D) if max_parts > 1 else None
    p = K.attention_params(d_q, q_stride, out, hq, scale, cache.layer(0), d_tables, max_blocks,
                           d_pos)
    w = K.decode_work(d_items, d_seqs, num_items, max_parts, ws)
    K.paged_attention_decode(p, w)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.fixture(params=["default", "grid", "persistent", "grid-dot2", "persistent-dot2"])
def attention_form(request):
    """The launcher's two kernel forms -- one workgroup per (partition, kv
    head, item), or persistent workgroups over the in-context units only
    (RLK_TUNE_ATTN_PERSIST = 0 or workgroups per CU) -- each with P . V on
    the matrix cores (the default) or on v_dot2 (RLK_TUNE_ATTN_PV = 0)."""
    from redline_amd._lib import tune_knob
    form = request.param.split("-")[0]
    pv = 0 if request.param.endswith("dot2") else None
    with tune_knob("RLK_TUNE_ATTN_PERSIST", {"grid": 0, "persistent": 2}.get(form)), \
            tune_knob("RLK_TUNE_ATTN_PV", pv):
        yield request.param


REF_CASES = [(8, 2, 128, False, [37, 300, 5]), (4, 4, 64, False, [64, 129, 1]),
             (6, 2, 128, False, [700]), (8, 1, 64, False, [48, 17]),
             (8, 2, 128, True, [33, 280]), (4, 2, 64, True, [520]),
             # G = 8 at D = 128: the largest LDS footprint of either form
             (8, 1, 128, False, [300, 40]), (8, 1, 128, True, [260]),
             # G = 5 and 7; sequences ending on a partition boundary
             (8, 2, 128, True, [256, 512]), (10, 2, 128, False, [257, 1]),
             (7, 1, 64, True, [300, 17])]


@pytest.mark.parametrize("hq,hkv,D,int8,lens", REF_CASES)
@pytest.mark.parametrize("static_parts", [False, True])
def test_decode_attention_reference_geometries(torch_cuda, hq, hkv, D, int8, lens, static_parts,
                                               attention_form):
    """Every token of every sequence is a decode item attending to its causal
    prefix, over a cache written by rope_and_write_kv (shuffled blocks)."""
    say(f"attention hq={hq} hkv={hkv} D={D} int8={int8} lens={lens} static={static_parts} "
        f"form={attention_form}")
    _causal_prefix_case(torch_cuda, hq, hkv, D, int8, lens, static_parts, 16)


@pytest.mark.parametrize("bs", [8, 32])
@pytest.mark.parametrize("hq,hkv,D,int8,lens", [(8, 2, 128, False, [300, 17]),
                                                (8, 2, 128, True, [270]),
                                                (4, 2, 64, True, [140, 33])])
def test_decode_attention_other_block_sizes(torch_cuda, hq, hkv, D, int8, lens, bs,
                                            attention_form):
    """Cache blocks of 8 and 32 keys (the reference uses 16): a 256-key
    partition then spans 32 or 8 blocks."""
    say(f"attention bs={bs} hq={hq} hkv={hkv} D={D} int8={int8} lens={lens} form={attention_form}")
    _causal_prefix_case(torch_cuda, hq, hkv, D, int8, lens, False, bs)


def _causal_prefix_case(torch, hq, hkv, D, int8, lens, static_parts, bs):
    from redline_amd import kernels as K
    rng = np.random.default_rng(hq * 7 + D + sum(lens))
    S, T, max_len = len(lens), sum(lens), max(lens)
    nblocks = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblocks, dtype=np.int32))
    max_blocks = (max_len + bs - 1) // bs
    b = ra.BatchBuilder(T, S, S, max_blocks, bs, 1 << 30)  # every token a decode item
    nxt = 0
    for L in lens:
        nb = (L + bs - 1) // bs
        b.add(np.zeros(L, np.int32), 0, L, None, ids[nxt:nxt + nb])
        nxt += nb
    meta, shape, lay = b.write()
    assert shape.num_decode_items == T
    stride = (hq + 2 * hkv) * D
    qkv = randn_f16(rng, (T, stride))
    cos, sin = ra.rope_cos_sin_tables(1e4, D, max_len)
    cache = K.KVCache(1, nblocks, hkv, D, bs, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    d_meta, d_qkv = dev(torch, meta), dev(torch, qkv)
    sl = lambda name, n: d_meta[lay[name]:lay[name] + n]  # noqa: E731
    K.rope_and_write_kv(d_qkv, sl("positions", T), sl("slot_mapping", T), T, hq, dev(torch, cos),
                        dev(torch, sin), cache.layer(0))
    max_parts = ((max_len if static_parts else shape.max_context) + 255) // 256
    scale = 1 / np.sqrt(D)
    got = run_attention(torch, K, d_qkv, stride, hq, scale, cache,
                        d_meta[lay["block_tables"]:], max_blocks, sl("positions", T),
                        sl("decode_token", T), sl("decode_seq", T), T, T, max_parts)

    # oracle: the same rope into CPU caches, then float64 attention
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
    want = oracle.paged_attention_decode(roped, stride, hq, scale, kc, vc, ks, vs, tables, pos,
                                         meta[lay["decode_token"]:lay["decode_token"] + T],
                                         meta[lay["decode_seq"]:lay["decode_seq"] + T], T, int8)
    assert_close_f16(got, want, what="attention")
    # the reference test's own bound against unquantised attention
    # (test_kernels.cu:195): 5e-3 FP16 KV, 3e-2 INT8 KV
    if int8:
        kf = np.zeros(shape4, np.float16)
        vf = np.zeros_like(kf)
        r2 = qkv.copy()
        oracle.rope_and_write_kv(r2, pos, slots, hq, hkv, D, cos, sin, kf, vf, block_size=bs)
        exact = oracle.paged_attention_decode(r2, stride, hq, scale, kf, vf, None, None, tables,
                                              pos, meta[lay["decode_token"]:lay["decode_token"] + T],
                                              meta[lay["decode_seq"]:lay["decode_seq"] + T], T)
        assert rel_max_err(got, exact) <= 3e-2


@pytest.mark.parametrize("int8", [False, True])
def test_decode_attention_llama_b32(torch_cuda, int8, attention_form):
    """C2: Llama-3.1-8B decode at batch 32, contexts up to 8192 over a
    16384-block pool (random cache contents); only the decode items' rows of
    `out` are written."""
    torch = torch_cuda
    from redline_amd import kernels as K
    from redline_amd.configs import build_batch, make_workload
    say(f"attention C2 int8={int8} form={attention_form}")
    w = make_workload("C2")
    m = w.model
    meta, shape, lay, tables_list = build_batch(w)
    T, S = w.num_tokens, len(w.segments)
    D, hq, hkv = m.head_dim, m.hq, m.hkv
    cache = K.KVCache(1, w.num_blocks, hkv, D, 16, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ks, vs = cache.tensors(0)
    g = torch.Generator(device="cuda").manual_seed(3)
    if int8:
        k.copy_(torch.randint(-127, 128, k.shape, generator=g, device="cuda", dtype=torch.int8))
        v.copy_(torch.randint(-127, 128, v.shape, generator=g, device="cuda", dtype=torch.int8))
        ks.copy_(torch.rand(ks.shape, generator=g, device="cuda") * 0.02 + 1e-3)
        vs.copy_(torch.rand(vs.shape, generator=g, device="cuda") * 0.02 + 1e-3)
    else:
        k.copy_(torch.randn(k.shape, generator=g, device="cuda").half())
        v.copy_(torch.randn(v.shape, generator=g, device="cuda").half())
    rng = np.random.default_rng(5)
    qkv = randn_f16(rng, (T, m.qkv_cols))
    d_meta = dev(torch, meta)
    sl = lambda name, n: d_meta[lay[name]:lay[name] + n]  # noqa: E731
    max_blocks = max(len(t) for t in tables_list)
    max_parts = (shape.max_context + 255) // 256
    nd = shape.num_decode_items
    got = run_attention(torch, K, dev(torch, qkv), m.qkv_cols, hq, 1 / np.sqrt(D), cache,
                        d_meta[lay["block_tables"]:], max_blocks, sl("positions", T),
                        sl("decode_token", nd), sl("decode_seq", nd), nd, T, max_parts)
    tables = meta[lay["block_tables"]:lay["block_tables"] + S * max_blocks].reshape(S, max_blocks)
    want = oracle.paged_attention_decode(
        qkv, m.qkv_cols, hq, 1 / np.sqrt(D), k.cpu().numpy(), v.cpu().numpy(),
        None if ks is None else ks.cpu().numpy(), None if vs is None else vs.cpu().numpy(), tables,
        meta[lay["positions"]:lay["positions"] + T], meta[lay["decode_token"]:lay["decode_token"] + nd],
        meta[lay["decode_seq"]:lay["decode_seq"] + nd], T, int8)
    assert_close_f16(got, want, what="attention C2")


LONG_CASES = {
    # past 32 partitions (the merge's batched rows, then its loop) and past D
    # partitions (its statistics loop): 157 / 36 / 33 / 2 partitions
    "few": [40000, 9000, 8200, 257],
    # enough units that a persistent workgroup runs through several
    # consecutive partitions of one (item, kv head), its range boundaries
    # splitting items: 2 to 157 partitions per item
    "runs": [40000, 9000, 300, 25000, 513, 17000, 4097, 30001, 257, 12000, 33000, 768,
             21000, 6000, 39000, 1100],
}


@pytest.mark.parametrize("lens,D", [("few", 64), ("few", 128), ("runs", 64), ("runs", 128)])
@pytest.mark.parametrize("int8", [False, True])
def test_decode_attention_long_contexts(torch_cuda, D, int8, lens, attention_form):
    """Long contexts (LONG_CASES), random cache contents."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"attention long contexts {lens} D={D} int8={int8} form={attention_form}")
    hq, hkv, bs = 8, 2, 16
    ctx = np.array(LONG_CASES[lens])
    n = len(ctx)
    nb = (ctx + bs - 1) // bs
    max_blocks = int(nb.max())
    rng = np.random.default_rng(17 + D + int8)
    pool = rng.permutation(np.arange(1, 1 + int(nb.sum()), dtype=np.int32))
    tables = np.zeros((n, max_blocks), np.int32)  # rows padded with block 0
    off = 0
    for i, b in enumerate(nb):
        tables[i, :b] = pool[off:off + b]
        off += b
    cache = K.KVCache(1, 1 + int(nb.sum()), hkv, D, bs, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ks, vs = cache.tensors(0)
    g = torch.Generator(device="cuda").manual_seed(7)
    if int8:
        k.copy_(torch.randint(-127, 128, k.shape, generator=g, device="cuda", dtype=torch.int8))
        v.copy_(torch.randint(-127, 128, v.shape, generator=g, device="cuda", dtype=torch.int8))
        ks.copy_(torch.rand(ks.shape, generator=g, device="cuda") * 0.02 + 1e-3)
        vs.copy_(torch.rand(vs.shape, generator=g, device="cuda") * 0.02 + 1e-3)
    else:
        k.copy_(torch.randn(k.shape, generator=g, device="cuda").half())
        v.copy_(torch.randn(v.shape, generator=g, device="cuda").half())
    stride = (hq + 2 * hkv) * D
    qkv = randn_f16(rng, (n, stride))
    pos = (ctx - 1).astype(np.int32)
    ids = np.arange(n, dtype=np.int32)
    max_parts = int((ctx.max() + 255) // 256)
    got = run_attention(torch, K, dev(torch, qkv), stride, hq, 1 / np.sqrt(D), cache,
                        dev(torch, tables), max_blocks, dev(torch, pos), dev(torch, ids),
                        dev(torch, ids), n, n, max_parts)
    want = oracle.paged_attention_decode(
        qkv, stride, hq, 1 / np.sqrt(D), k.cpu().numpy(), v.cpu().numpy(),
        None if ks is None else ks.cpu().numpy(), None if vs is None else vs.cpu().numpy(), tables,
        pos, ids, ids, n, int8)
    assert_close_f16(got, want, what="attention long contexts")


@pytest.mark.parametrize("hq,hkv,D,lens", [(8, 2, 128, [33, 280]), (4, 2, 64, [520]),
                                           (32, 8, 128, [300, 17])])
def test_decode_attention_int8_fp16_scales(torch_cuda, hq, hkv, D, lens, attention_form):
    """Extension: an INT8 cache whose scales rope_and_write_kv_ex stored as
    fp16 (C4's scale format), attended by paged_attention_decode_ex; the
    oracle dequantises with the same fp16 scales.  Bad scale dtypes are
    rejected."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"attention fp16 scales hq={hq} hkv={hkv} D={D} lens={lens} form={attention_form}")
    bs = 16
    rng = np.random.default_rng(11 * hq + D + sum(lens))
    S, T, max_len = len(lens), sum(lens), max(lens)
    nblocks = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblocks, dtype=np.int32))
    max_blocks = (max_len + bs - 1) // bs
    b = ra.BatchBuilder(T, S, S, max_blocks, bs, 1 << 30)
    nxt = 0
    for L in lens:
        nb = (L + bs - 1) // bs
        b.add(np.zeros(L, np.int32), 0, L, None, ids[nxt:nxt + nb])
        nxt += nb
    meta, shape, lay = b.write()
    stride = (hq + 2 * hkv) * D
    qkv = randn_f16(rng, (T, stride))
    cos, sin = ra.rope_cos_sin_tables(1e4, D, max_len)
    cache = K.KVCache(1, nblocks, hkv, D, bs, K.KVDType.kINT8, scale_dtype=K.SCALE_F16)
    d_meta, d_qkv = dev(torch, meta), dev(torch, qkv)
    sl = lambda name, n: d_meta[lay[name]:lay[name] + n]  # noqa: E731
    K.rope_and_write_kv_ex(d_qkv, sl("positions", T), sl("slot_mapping", T), T, hq,
                           dev(torch, cos), dev(torch, sin), cache.layer(0),
                           scale_dtype=K.SCALE_F16)
    max_parts = (shape.max_context + 255) // 256
    out = torch.zeros((T, hq * D), dtype=torch.float16, device="cuda")
    ws = K.DecodeWorkspace(T, hq, max_parts, D) if max_parts > 1 else None
    prm = K.attention_params(d_qkv, stride, out, hq, 1 / np.sqrt(D), cache.layer(0),
                             d_meta[lay["block_tables"]:], max_blocks, sl("positions", T))
    wk = K.decode_work(sl("decode_token", T), sl("decode_seq", T), T, max_parts, ws)
    K.paged_attention_decode_ex(prm, wk, K.SCALE_F16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()

    pos = meta[lay["positions"]:lay["positions"] + T]
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T]
    shape4 = (nblocks, hkv, bs, D)
    kc = np.zeros(shape4, np.int8)
    vc = np.zeros_like(kc)
    ks16 = np.zeros(shape4[:3], np.uint16)
    vs16 = np.zeros_like(ks16)
    roped = qkv.copy()
    oracle.rope_and_write_kv(roped, pos, slots, hq, hkv, D, cos, sin, kc, vc, ks16, vs16, bs, True,
                             scale16=True)
    tables = meta[lay["block_tables"]:lay["block_tables"] + S * max_blocks].reshape(S, max_blocks)
    want = oracle.paged_attention_decode(
        roped, stride, hq, 1 / np.sqrt(D), kc, vc, ks16.view(np.float16).astype(np.float32),
        vs16.view(np.float16).astype(np.float32), tables, pos,
        meta[lay["decode_token"]:lay["decode_token"] + T],
        meta[lay["decode_seq"]:lay["decode_seq"] + T], T, True)
    assert_close_f16(got, want, what="attention fp16 scales")
    with pytest.raises(ra.Error, match="scale dtype"):
        K.paged_attention_decode_ex(prm, wk, 7)


def test_decode_attention_items_subset_and_errors(torch_cuda):
    """Only decode items' rows are written (mixed prefill/decode batch), and
    argument errors are reported before launch."""
    torch = torch_cuda
    from redline_amd import _lib, kernels as K
    say("attention subset/errors")
    rng = np.random.default_rng(6)
    hq, hkv, D, bs = 4, 2, 64, 16
    cache = K.KVCache(1, 8, hkv, D, bs)
    k, v, _, _ = cache.tensors(0)
    k.copy_(torch.randn(k.shape, device="cuda").half())
    v.copy_(torch.randn(v.shape, device="cuda").half())
    T = 6
    q = randn_f16(rng, (T, hq * D))
    pos = np.array([3, 4, 5, 6, 7, 20], np.int32)
    tables = np.array([[1, 2], [3, 4]], np.int32)
    items, seqs = np.array([1, 5], np.int32), np.array([0, 1], np.int32)
    got = run_attention(torch, K, dev(torch, q), hq * D, hq, 0.125, cache, dev(torch, tables), 2,
                        dev(torch, pos), dev(torch, items), dev(torch, seqs), 2, T, 1)
    assert not np.any(got[[0, 2, 3, 4]])
    want = oracle.paged_attention_decode(q, hq * D, hq, 0.125, k.cpu().numpy(), v.cpu().numpy(),
                                         None, None, tables, pos, items, seqs, T)
    assert_close_f16(got, want, what="subset")
    out = torch.zeros((T, hq * D), dtype=torch.float16, device="cuda")
    p = K.attention_params(dev(torch, q), hq * D, out, 3, 0.1, cache.layer(0), dev(torch, tables), 2,
                           dev(torch, pos))
    with pytest.raises(ra.Error, match="multiple of num_kv_heads"):
        K.paged_attention_decode(p, K.decode_work(dev(torch, items), dev(torch, seqs), 2, 1))
    p.num_heads = 4
    with pytest.raises(ra.Error, match="workspace"):
        K.paged_attention_decode(p, K.decode_work(dev(torch, items), dev(torch, seqs), 2, 2))
    K.paged_attention_decode(p, K.decode_work(dev(torch, items), dev(torch, seqs), 0, 1))  # no-op
    assert _lib.RLK_DECODE_PARTITION_SIZE == K.kDecodePartitionSize == 256


@pytest.mark.parametrize("max_parts", [1, 2])
def test_decode_attention_short_workspace_truncates(torch_cuda, max_parts, attention_form):
    """A max_partitions smaller than a context needs (a caller error the
    reference leaves undefined) attends the first max_partitions * 256 keys
    and never writes past the workspace -- with max_partitions == 1 no
    workspace is passed at all."""
    torch = torch_cuda
    from redline_amd import kernels as K
    say(f"attention short workspace max_parts={max_parts} form={attention_form}")
    rng = np.random.default_rng(11)
    hq, hkv, D, bs = 4, 2, 64, 16
    nb = 50
    cache = K.KVCache(1, nb, hkv, D, bs)
    k, v, _, _ = cache.tensors(0)
    k.copy_(torch.randn(k.shape, device="cuda").half())
    v.copy_(torch.randn(v.shape, device="cuda").half())
    T = 2
    q = randn_f16(rng, (T, hq * D))
    pos = np.array([699, 100], np.int32)
    tables = rng.integers(1, nb, (2, 44), dtype=np.int32)  # read only: blocks may repeat
    items, seqs = np.array([0, 1], np.int32), np.array([0, 1], np.int32)
    got = run_attention(torch, K, dev(torch, q), hq * D, hq, 0.125, cache, dev(torch, tables), 44,
                        dev(torch, pos), dev(torch, items), dev(torch, seqs), 2, T, max_parts)
    cut = np.minimum(pos, max_parts * K.kDecodePartitionSize - 1)
    want = oracle.paged_attention_decode(q, hq * D, hq, 0.125, k.cpu().numpy(), v.cpu().numpy(),
                                         None, None, tables, cut, items, seqs, T)
    assert_close_f16(got, want, what="truncated")
