"""rlk_paged_attention_decode_noalloc (split-K partials in the library's
device scratch array, no allocation) against rlk_paged_attention_decode with a
caller workspace, through the C ABI: the same kernels over the same partials,
so the outputs must be identical bit for bit.  Two calls in a row on one GPU,
the second smaller (the scratch keeps the first call's contents), then the
size limit."""
import ctypes as C

import numpy as np
import pytest

from redline_amd import _lib
from tests._util import say


def _case(torch, K, rng, items, hq, hkv, D, max_ctx, int8):
    bs = 16
    max_blocks = (max_ctx + bs - 1) // bs
    nblk = 1 + items * max_blocks
    cache = K.KVCache(1, nblk, hkv, D, bs, K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ks, vs = cache.tensors(0)
    g = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 30)))
    if int8:
        k.copy_(torch.randint(-127, 128, k.shape, generator=g, device="cuda", dtype=torch.int8))
        v.copy_(torch.randint(-127, 128, v.shape, generator=g, device="cuda", dtype=torch.int8))
        ks.uniform_(0.005, 0.02, generator=g)
        vs.uniform_(0.005, 0.02, generator=g)
    else:
        k.normal_(generator=g)
        v.normal_(generator=g)
    tables = rng.permutation(np.arange(1, nblk, dtype=np.int32)).reshape(items, max_blocks)
    ctx = rng.integers(1, max_ctx + 1, items)
    ctx[0] = max_ctx
    stride = (hq + 2 * hkv) * D
    q = torch.randn((items, stride), generator=g, device="cuda").half()
    pos = torch.from_numpy((ctx - 1).astype(np.int32)).cuda()
    ids = torch.arange(items, dtype=torch.int32, device="cuda")
    parts = (max_ctx + 255) // 256
    return cache, q, stride, torch.from_numpy(tables).cuda(), max_blocks, pos, ids, parts


def _run(torch, K, case, hq, noalloc):
    cache, q, stride, tables, max_blocks, pos, ids, parts = case
    items, D = q.shape[0], cache.head_dim
    out = torch.zeros((items, hq * D), dtype=torch.float16, device="cuda")
    ws = None if noalloc else K.DecodeWorkspace(items, hq, parts, D)
    p = K.attention_params(q, stride, out, hq, D ** -0.5, cache.layer(0), tables, max_blocks, pos)
    w = K.decode_work(ids, ids, items, parts, ws)
    L = _lib.lib()
    fn = L.rlk_paged_attention_decode_noalloc if noalloc else L.rlk_paged_attention_decode
    _lib.check(fn(C.byref(p), C.byref(w), C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    return out


@pytest.mark.gpu
def test_decode_noalloc_matches_workspace_entry():
    import torch
    from redline_amd import kernels as K
    rng = np.random.default_rng(11)
    # C2 shape (32 items, 32 heads / 8 kv heads, D 128, contexts to 8192: 32
    # partitions, 17 MB of partials), then a smaller INT8 call at D 64, then a
    # single-partition call (contexts <= 256: no split-K scratch is used)
    for items, hq, hkv, D, max_ctx, int8 in ((32, 32, 8, 128, 8192, False),
                                             (5, 8, 2, 64, 700, True),
                                             (3, 8, 2, 128, 200, False)):
        say(f"noalloc decode items={items} hq={hq} hkv={hkv} D={D} ctx={max_ctx} int8={int8}")
        case = _case(torch, K, rng, items, hq, hkv, D, max_ctx, int8)
        want = _run(torch, K, case, hq, noalloc=False)
        got = _run(torch, K, case, hq, noalloc=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        assert torch.isfinite(got.float()).all()


def test_decode_noalloc_rejects_oversized_calls():
    """Beyond RLK_DECODE_SCRATCH_BYTES the entry point fails before touching
    the device."""
    L = _lib.lib()
    d = C.c_void_p(16)
    kv = _lib.KVLayerView(d, d, None, None, 16, 8, 128, 0)
    p = _lib.AttentionParams(d, 6144, d, 32, 0.1, kv, d, 1024, d)
    w = _lib.DecodeAttentionWork(d, d, 256, 64, None, None, None)  # 256 x 32 x 64 x 130 x 4 B
    assert L.rlk_paged_attention_decode_noalloc(C.byref(p), C.byref(w), None) == _lib.RLK_EINVAL
    assert b"split-K scratch" in L.rlk_last_error()
