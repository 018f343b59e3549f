"""Parity of rope_and_write_kv (through the C ABI) with the CPU oracle.

The rotation is evaluated without FMA contraction on both sides, so the roped
q (written back in place), the FP16 cache cells, the INT8 codes and their fp32
scales are all compared bit for bit; KV slot / cell addressing is checked by
reading back exactly the cells the batch metadata names and by checking that
every other cell of the (zeroed) cache is untouched.  Metadata comes from the
BatchBuilder, uploaded to the GPU as one int32 buffer, as the engine drives the
kernel.  Cases follow tests/cuda/test_kernels.cu:80-148, 282-322 and the
workload shapes."""
import numpy as np
import pytest

import oracle
import redline_amd as ra
from redline_amd.configs import build_batch, make_workload
from tests._util import assert_bits_equal, assert_close_f16, randn_f16, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    import redline_amd.kernels  # noqa: F401
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_case(torch, qkv, positions, slots, hq, hkv, D, num_blocks, int8, theta=1e4, bs=16,
             max_pos=None, meta=None, layout=None, bias=None, scale16=False):
    """Runs GPU and oracle on the same inputs; returns the GPU cache tensors.
    With a QKV bias or fp16 INT8 scales the extension entry point runs."""
    from redline_amd import kernels as K
    T = positions.size
    max_pos = max_pos or int(positions.max()) + 1
    cos, sin = ra.rope_cos_sin_tables(theta, D, max_pos)
    dtype = K.KVDType.kINT8 if int8 else K.KVDType.kFP16
    sdt = K.SCALE_F16 if scale16 else K.SCALE_F32
    cache = K.KVCache(1, num_blocks, hkv, D, bs, dtype, scale_dtype=sdt)
    d_qkv = dev(torch, qkv)
    if meta is not None:  # the engine's single metadata buffer
        d_meta = dev(torch, meta)
        d_pos = d_meta[layout["positions"]:layout["positions"] + T]
        d_slot = d_meta[layout["slot_mapping"]:layout["slot_mapping"] + T]
    else:
        d_pos, d_slot = dev(torch, positions), dev(torch, slots)
    if bias is None and not scale16:
        K.rope_and_write_kv(d_qkv, d_pos, d_slot, T, hq, dev(torch, cos), dev(torch, sin),
                            cache.layer(0))
    else:
        K.rope_and_write_kv_ex(d_qkv, d_pos, d_slot, T, hq, dev(torch, cos), dev(torch, sin),
                               cache.layer(0), None if bias is None else dev(torch, bias), sdt)
    torch.cuda.synchronize()

    # oracle on a cache of the same geometry (zero pages are not materialised)
    shape = (num_blocks, hkv, bs, D)
    kc = np.zeros(shape, np.int8 if int8 else np.float16)
    vc = np.zeros_like(kc)
    sc_np = np.uint16 if scale16 else np.float32
    ks = np.zeros(shape[:3], sc_np) if int8 else None
    vs = np.zeros(shape[:3], sc_np) if int8 else None
    want_qkv = np.array(qkv, copy=True)
    oracle.rope_and_write_kv(want_qkv, positions, slots, hq, hkv, D, cos, sin, kc, vc, ks, vs,
                             bs, int8, bias=bias, scale16=scale16)
    assert_bits_equal(d_qkv.cpu().numpy(), want_qkv, "qkv (q roped in place, k/v untouched)")

    # the written cells, bit for bit
    valid = slots >= 0
    blk, off = slots[valid] // bs, slots[valid] % bs
    cells = ((blk[:, None] * hkv + np.arange(hkv)[None, :]) * bs + off[:, None]).reshape(-1)
    k, v, k_s, v_s = cache.tensors(0)
    d_cells = dev(torch, cells.astype(np.int64))
    for name, gpu, cpu in (("k", k, kc), ("v", v, vc)):
        got = gpu.reshape(-1, D).index_select(0, d_cells).cpu().numpy()
        assert_bits_equal(got, cpu.reshape(-1, D)[cells], f"{name} cache cells")
        # nothing else written: the nonzero count of the whole cache equals
        # the nonzero count of the named cells
        total_nz = int((gpu.view(torch.uint8) != 0).sum().item())
        cells_nz = int((got.view(np.uint8) != 0).sum())
        assert total_nz == cells_nz, f"{name}: writes outside the named cells"
    if int8:
        for name, gpu, cpu in (("k_scale", k_s, ks), ("v_scale", v_s, vs)):
            got = gpu.reshape(-1).index_select(0, d_cells).cpu().numpy()
            if scale16:
                got = got.view(np.uint16)
            assert_bits_equal(got, cpu.reshape(-1)[cells], name)
            assert int((gpu != 0).sum().item()) == int((got != 0).sum())
    return cache, want_qkv, cells


# Reference attention-test geometries (tests/cuda/test_kernels.cu:282-287).
REF_CASES = [(8, 2, 128, False, [37, 300, 5]), (4, 4, 64, False, [64, 129, 1]),
             (6, 2, 128, False, [700]), (8, 1, 64, False, [48, 17]),
             (8, 2, 128, True, [33, 280]), (4, 2, 64, True, [520])]


@pytest.mark.parametrize("hq,hkv,D,int8,lens", REF_CASES)
def test_rope_kv_reference_geometries(torch_cuda, hq, hkv, D, int8, lens):
    say(f"rope hq={hq} hkv={hkv} D={D} int8={int8} lens={lens}")
    bs = 16
    rng = np.random.default_rng(hq * 100 + D + sum(lens))
    nblocks = 1 + sum((L + bs - 1) // bs for L in lens)
    ids = rng.permutation(np.arange(1, nblocks, dtype=np.int32))
    b = ra.BatchBuilder(sum(lens), len(lens), len(lens), (max(lens) + bs - 1) // bs, bs, 0)
    nxt = 0
    for L in lens:
        nb = (L + bs - 1) // bs
        b.add(np.zeros(L, np.int32), 0, L, None, ids[nxt:nxt + nb])
        nxt += nb
    meta, shape, lay = b.write()
    T = sum(lens)
    pos = meta[lay["positions"]:lay["positions"] + T].copy()
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T].copy()
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    run_case(torch_cuda, qkv, pos, slots, hq, hkv, D, nblocks, int8, meta=meta, layout=lay)


def test_rope_int8_scale_kat(torch_cuda):
    """tests/cuda/test_kernels.cu:289-322: scale == amax/127 and
    |code * scale - k| <= 0.51 * scale against the fp32 rotation."""
    torch = torch_cuda
    say("rope int8 scale KAT")
    hq, hkv, D, bs = 2, 1, 64, 16
    rng = np.random.default_rng(21)
    qkv = randn_f16(rng, (1, (hq + 2 * hkv) * D))
    cache, _, cells = run_case(torch, qkv, np.array([5], np.int32), np.array([bs + 3], np.int32),
                               hq, hkv, D, 2, True, max_pos=8)
    cos, sin = ra.rope_cos_sin_tables(1e4, D, 8)
    k = qkv[0, hq * D:(hq + 1) * D].astype(np.float32)
    x0, x1 = k[:32], k[32:]
    roped = np.concatenate([x0 * cos[5] - x1 * sin[5], x1 * cos[5] + x0 * sin[5]])
    roped = roped.astype(np.float16).astype(np.float32)
    kt, _, kst, _ = cache.tensors(0)
    codes = kt[1, 0, 3].cpu().numpy().astype(np.float32)
    scale = float(kst[1, 0, 3].item())
    assert abs(scale - np.abs(roped).max() / 127) <= 1e-6
    assert np.all(np.abs(codes * scale - roped) <= 0.51 * scale)


def test_rope_position_zero_identity_and_skip(torch_cuda):
    """pos 0 rotates by angle 0 (q, k unchanged); slot < 0 writes no KV."""
    torch = torch_cuda
    say("rope pos0 / negative slots")
    hq, hkv, D = 4, 2, 128
    rng = np.random.default_rng(4)
    qkv = randn_f16(rng, (6, (hq + 2 * hkv) * D))
    pos = np.array([0, 0, 7, 0, 9, 3], np.int32)
    slots = np.array([17, -1, 40, -1, 63, 16], np.int32)
    cache, want, _ = run_case(torch, qkv, pos, slots, hq, hkv, D, 4, False)
    assert_bits_equal(want[[0, 1, 3]], qkv[[0, 1, 3]], "pos 0 identity")
    k, v, _, _ = cache.tensors(0)
    # token 0 (slot 17 = block 1, off 1): k equals the unrotated k head
    got_k = k[1, :, 1].cpu().numpy().reshape(-1)
    assert_bits_equal(got_k, qkv[0, hq * D:(hq + hkv) * D], "k at pos 0")


def test_rope_matches_fp32_rotation(torch_cuda):
    """Roped q against a float64 rotation (rotate-half convention): within
    one fp16 rounding."""
    torch = torch_cuda
    say("rope vs float64 rotation")
    hq, hkv, D = 32, 8, 128
    rng = np.random.default_rng(8)
    T = 64
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    pos = rng.integers(0, 8192, T).astype(np.int32)
    slots = (np.arange(T) + 16).astype(np.int32)
    _, got, _ = run_case(torch, qkv, pos, slots, hq, hkv, D, 1 + T // 16 + 1, False, theta=5e5,
                         max_pos=8192)
    inv = 1.0 / 5e5 ** (np.arange(64) * 2 / 128)
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    q = qkv[:, :hq * D].astype(np.float64).reshape(T, hq, D)
    ref = np.concatenate([q[..., :64] * c - q[..., 64:] * s, q[..., 64:] * c + q[..., :64] * s], -1)
    assert_close_f16(got[:, :hq * D].reshape(T, hq, D), ref, what="q vs float64 rotation")


@pytest.mark.parametrize("key", ["C1", "C2", "C3", "C5"])
def test_rope_kv_workloads_fp16(torch_cuda, key):
    torch = torch_cuda
    w = make_workload(key)
    m = w.model
    say(f"rope workload {key} T={w.num_tokens}")
    meta, shape, lay, _ = build_batch(w)
    T = w.num_tokens
    pos = meta[lay["positions"]:lay["positions"] + T].copy()
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T].copy()
    rng = np.random.default_rng(11)
    qkv = randn_f16(rng, (T, m.qkv_cols))
    if w.qkv_bias:  # Qwen2: the bias arrives in the activations (GEMM epilogue)
        bias = randn_f16(rng, (m.qkv_cols,), 0.02)
        qkv = (qkv.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    run_case(torch, qkv, pos, slots, m.hq, m.hkv, m.head_dim, w.num_blocks, False, theta=m.theta,
             max_pos=w.max_pos, meta=meta, layout=lay)


def test_rope_kv_workload_c5_bias_in_kernel(torch_cuda):
    """C5 (Qwen2-7B, 16384 tokens): the QKV bias ~N(0, 0.02) added before RoPE
    by the extension entry point, bit-exact against the oracle's extension."""
    torch = torch_cuda
    w = make_workload("C5")
    m = w.model
    say("rope workload C5 bias in kernel")
    meta, shape, lay, _ = build_batch(w)
    T = w.num_tokens
    pos = meta[lay["positions"]:lay["positions"] + T].copy()
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T].copy()
    rng = np.random.default_rng(13)
    qkv = randn_f16(rng, (T, m.qkv_cols))
    bias = randn_f16(rng, (m.qkv_cols,), 0.02)
    run_case(torch, qkv, pos, slots, m.hq, m.hkv, m.head_dim, w.num_blocks, False, theta=m.theta,
             max_pos=w.max_pos, meta=meta, layout=lay, bias=bias)


@pytest.mark.parametrize("scale16", [False, True])
def test_rope_kv_int8_16k_outliers(torch_cuda, scale16):
    """C4: 16384 tokens, INT8 KV, K/V ~ N(0,1) with 2 of 128 channels per head
    ~ N(0, 8): codes and scales bit-exact; dequantised cache within 0.51 scale
    of the fp16 cache written by the FP16 path on the same inputs.  The config
    stores the scales as fp16 (extension entry point); fp32 is the reference's
    own format."""
    torch = torch_cuda
    w = make_workload("C4")
    m = w.model
    say(f"rope workload C4 int8 scale16={scale16}")
    meta, shape, lay, _ = build_batch(w)
    T = w.num_tokens
    pos = meta[lay["positions"]:lay["positions"] + T].copy()
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T].copy()
    rng = np.random.default_rng(12)
    qkv = randn_f16(rng, (T, m.qkv_cols)).reshape(T, -1, m.head_dim)
    dims = rng.choice(m.head_dim, 2, replace=False)
    qkv[:, m.hq:, dims] = randn_f16(rng, (T, 2 * m.hkv, 2), 8.0)
    qkv = qkv.reshape(T, -1)
    c8, _, cells = run_case(torch, qkv, pos, slots, m.hq, m.hkv, m.head_dim, w.num_blocks, True,
                            theta=m.theta, max_pos=w.max_pos, meta=meta, layout=lay,
                            scale16=scale16)
    c16, _, _ = run_case(torch, qkv, pos, slots, m.hq, m.hkv, m.head_dim, w.num_blocks, False,
                         theta=m.theta, max_pos=w.max_pos, meta=meta, layout=lay)
    d_cells = dev(torch, cells.astype(np.int64))
    k8, v8, ks, vs = c8.tensors(0)
    k16, v16, _, _ = c16.tensors(0)
    D = m.head_dim
    for q8, sc, f16 in ((k8, ks, k16), (v8, vs, v16)):
        codes = q8.reshape(-1, D).index_select(0, d_cells).float()
        scale = sc.reshape(-1).index_select(0, d_cells).float()[:, None]
        ref = f16.reshape(-1, D).index_select(0, d_cells).float()
        assert bool((codes.abs() <= 127).all())
        if scale16:  # the scale is fp16(amax/127): amax/scale may round just past 127 (clamped)
            assert bool(((codes * scale - ref).abs() <= 0.51 * scale + 2e-3 * ref.abs()).all())
            assert bool((codes.abs().amax(1) >= 126).all())
        else:
            assert bool(((codes * scale - ref).abs() <= 0.51 * scale).all())
            assert bool((codes.abs().amax(1) == 127).all())  # the absmax element maps to +/-127


def test_rope_int8_zero_head_scale_one(torch_cuda):
    """amax == 0 -> scale 1 and all-zero codes (rope_kv.cu:77)."""
    torch = torch_cuda
    say("rope int8 zero head")
    hq, hkv, D = 2, 2, 128
    qkv = np.zeros((3, (hq + 2 * hkv) * D), np.float16)
    cache, _, _ = run_case(torch, qkv, np.array([1, 2, 3], np.int32),
                           np.array([16, 17, 18], np.int32), hq, hkv, D, 2, True)
    _, _, ks, vs = cache.tensors(0)
    assert bool((ks[1, :, :3] == 1.0).all()) and bool((vs[1, :, :3] == 1.0).all())


@pytest.mark.parametrize("bs", [8, 32])
def test_rope_other_block_sizes(torch_cuda, bs):
    torch = torch_cuda
    say(f"rope block size {bs}")
    hq, hkv, D = 8, 2, 64
    rng = np.random.default_rng(bs)
    T = 100
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    pos = rng.integers(0, 512, T).astype(np.int32)
    slots = rng.permutation(np.arange(bs, 40 * bs)).astype(np.int32)[:T]
    run_case(torch, qkv, pos, slots, hq, hkv, D, 40, True, bs=bs, max_pos=512)
    run_case(torch, qkv, pos, slots, hq, hkv, D, 40, False, bs=bs, max_pos=512)


def test_rope_int8_exact_ties(torch_cuda):
    """Values exactly on .5 code ties (scale 2^-6) round half to even, as the
    oracle (pinned against numpy's rint) does."""
    say("rope int8 exact ties")
    hq, hkv, D = 1, 1, 128
    n = np.arange(D) % 126
    v = ((n + 0.5) / 64).astype(np.float16)
    v[0] = np.float16(127 / 64)
    v[1::2] *= -1
    qkv = np.zeros((1, (hq + 2 * hkv) * D), np.float16)
    qkv[0, (hq + hkv) * D:] = v
    cache, _, _ = run_case(torch_cuda, qkv, np.array([0], np.int32), np.array([16], np.int32),
                           hq, hkv, D, 2, True)
    _, vq, _, vs = cache.tensors(0)
    assert np.array_equal(vq[1, 0, 0].cpu().numpy().astype(np.float64), np.rint(v.astype(np.float64) * 64))


@pytest.mark.parametrize("int8,scale16", [(False, False), (True, False), (True, True)])
def test_rope_extension_bias_and_fp16_scale(torch_cuda, int8, scale16):
    """rlk_rope_and_write_kv_ex on the Qwen2-7B workload (C5, bias before
    RoPE): bit-exact with the oracle's extension, including fp16 scales."""
    torch = torch_cuda
    from redline_amd import kernels as K
    w = make_workload("C5")
    m = w.model
    say(f"rope ex C5 int8={int8} scale16={scale16}")
    meta, shape, lay, _ = build_batch(w)
    T = w.num_tokens
    pos = meta[lay["positions"]:lay["positions"] + T].copy()
    slots = meta[lay["slot_mapping"]:lay["slot_mapping"] + T].copy()
    rng = np.random.default_rng(13)
    qkv = randn_f16(rng, (T, m.qkv_cols))
    bias = randn_f16(rng, (m.qkv_cols,), 0.02)
    D = m.head_dim
    cos, sin = ra.rope_cos_sin_tables(m.theta, D, w.max_pos)
    sdt = K.SCALE_F16 if scale16 else K.SCALE_F32
    cache = K.KVCache(1, w.num_blocks, m.hkv, D, 16, K.KVDType.kINT8 if int8 else K.KVDType.kFP16,
                      scale_dtype=sdt)
    d_qkv, d_meta = dev(torch, qkv), dev(torch, meta)
    K.rope_and_write_kv_ex(d_qkv, d_meta[lay["positions"]:], d_meta[lay["slot_mapping"]:], T, m.hq,
                           dev(torch, cos), dev(torch, sin), cache.layer(0), dev(torch, bias), sdt)
    shape4 = (w.num_blocks, m.hkv, 16, D)
    kc = np.zeros(shape4, np.int8 if int8 else np.float16)
    vc = np.zeros_like(kc)
    ks = np.zeros(shape4[:3], np.uint16 if scale16 else np.float32) if int8 else None
    vs = np.zeros_like(ks) if int8 else None
    want = qkv.copy()
    oracle.rope_and_write_kv(want, pos, slots, m.hq, m.hkv, D, cos, sin, kc, vc, ks, vs, 16, int8,
                             bias=bias, scale16=scale16)
    assert_bits_equal(d_qkv.cpu().numpy(), want, "qkv")
    blk, off = slots // 16, slots % 16
    cells = ((blk[:, None] * m.hkv + np.arange(m.hkv)[None, :]) * 16 + off[:, None]).reshape(-1)
    d_cells = dev(torch, cells.astype(np.int64))
    k, v, k_s, v_s = cache.tensors(0)
    for gpu, cpu in ((k, kc), (v, vc)):
        assert_bits_equal(gpu.reshape(-1, D).index_select(0, d_cells).cpu().numpy(),
                          cpu.reshape(-1, D)[cells], "cache")
    if int8:
        for gpu, cpu in ((k_s, ks), (v_s, vs)):
            got = gpu.reshape(-1).index_select(0, d_cells).cpu().numpy()
            assert_bits_equal(got.view(cpu.dtype), cpu.reshape(-1)[cells], "scales")


@pytest.mark.parametrize("tok", [0, 1, 2])
@pytest.mark.parametrize("hq,hkv,D,int8", [(28, 4, 128, False), (28, 4, 128, True), (32, 4, 64, False),
                                           (64, 8, 64, True)])
def test_rope_bias_token_policies(torch_cuda, tok, hq, hkv, D, int8):
    """The QKV bias through each launch form (RLK_TUNE_ROPE_BIAS_TOK: 0 the
    general kernel, 1 and 2 tokens per workgroup with the bias kept in
    registers), on an odd token count (the last workgroup of the two-token
    form holds one token) with a skipped slot; bits against the oracle."""
    from redline_amd._lib import tune_knob
    say(f"rope bias tok={tok} hq={hq} hkv={hkv} D={D} int8={int8}")
    bs = 16
    rng = np.random.default_rng(tok * 7 + hq + D)
    T = 37
    nblocks = 2 + T // bs + 2
    slots = rng.permutation(np.arange(bs, nblocks * bs, dtype=np.int32))[:T]
    slots[5] = -1
    pos = rng.integers(0, 4096, T).astype(np.int32)
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    bias = randn_f16(rng, ((hq + 2 * hkv) * D,), 0.02)
    with tune_knob("RLK_TUNE_ROPE_BIAS_TOK", tok):
        run_case(torch_cuda, qkv, pos, slots, hq, hkv, D, nblocks, int8, theta=1e6, bias=bias)


def test_rope_extension_null_options_is_plain(torch_cuda):
    torch = torch_cuda
    import ctypes as C
    from redline_amd import _lib, kernels as K
    say("rope ex null options")
    rng = np.random.default_rng(14)
    hq, hkv, D = 4, 2, 64
    qkv = randn_f16(rng, (5, (hq + 2 * hkv) * D))
    pos = np.arange(5, dtype=np.int32)
    slots = np.arange(16, 21, dtype=np.int32)
    cos, sin = ra.rope_cos_sin_tables(1e4, D, 8)
    outs = []
    for use_ex in (False, True):
        cache = K.KVCache(1, 2, hkv, D)
        # keep every device tensor referenced until the kernel has run (a
        # temporary freed after .data_ptr() can be handed to the next one)
        d, d_pos, d_slots = dev(torch, qkv), dev(torch, pos), dev(torch, slots)
        d_cos, d_sin = dev(torch, cos), dev(torch, sin)
        args = (d.data_ptr(), d_pos.data_ptr(), d_slots.data_ptr(), 5, hq, d_cos.data_ptr(),
                d_sin.data_ptr(), C.byref(cache.layer(0)))
        stream = torch.cuda.current_stream().cuda_stream
        st = (_lib.lib().rlk_rope_and_write_kv_ex(*args, None, stream) if use_ex
              else _lib.lib().rlk_rope_and_write_kv(*args, stream))
        assert st == 0
        torch.cuda.synchronize()
        outs.append((d.cpu().numpy(), cache.tensors(0)[0].cpu().numpy()))
    assert_bits_equal(outs[0][0], outs[1][0], "qkv")
    assert_bits_equal(outs[0][1], outs[1][1], "k cache")


@pytest.mark.parametrize("wpt", [1, 2, 3, 8])
@pytest.mark.parametrize("hq,hkv,D,int8,lens", [REF_CASES[0], REF_CASES[1], REF_CASES[4],
                                                (32, 8, 128, False, [200, 57]),
                                                (32, 8, 128, True, [130]), (28, 4, 128, False, [90])])
def test_rope_kv_launch_policies(torch_cuda, wpt, hq, hkv, D, int8, lens):
    """Every launch policy (waves per token) gives the same bits: the
    Llama-3.1-8B and Qwen2-7B head counts leave partial head sweeps at every
    setting."""
    from redline_amd._lib import tune_knob
    say(f"rope policy wpt={wpt} hq={hq} hkv={hkv} D={D} int8={int8}")
    bs = 16
    rng = np.random.default_rng(hq + hkv + D + wpt)
    T = sum(lens)
    nblocks = 2 + T // bs + len(lens)
    slots = rng.permutation(np.arange(bs, nblocks * bs, dtype=np.int32))[:T]
    slots[rng.integers(0, T)] = -1
    pos = rng.integers(0, 4096, T).astype(np.int32)
    qkv = randn_f16(rng, (T, (hq + 2 * hkv) * D))
    with tune_knob("RLK_TUNE_ROPE_WPT", wpt):
        run_case(torch_cuda, qkv, pos, slots, hq, hkv, D, nblocks, int8, theta=5e5)
