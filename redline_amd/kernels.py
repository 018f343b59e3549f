"""Python launch interface over the C ABI, mirroring redline::kernels.

Names, parameter order and meaning follow the reference's launchers
(src/cuda/kernels/kernels.h:64-88 in Neil456/Redline).  Arguments are torch
tensors on the GPU (device memory and streams come from PyTorch; the compute
is the HIP code in librlk.so).  Errors raise redline_amd.Error before anything
is launched, as the reference's RL_CHECK throws.  Every launcher is
asynchronous on `stream` (default: torch's current stream).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import KVLayerView, check, lib

__all__ = [
    "embedding_lookup", "embedding_rmsnorm", "fused_add_rmsnorm", "silu_and_mul", "silu_and_mul_interleaved",
    "gather_rows", "resolve_input_ids", "rope_and_write_kv", "rope_and_write_kv_ex", "KVDType",
    "KVCache", "SCALE_F32", "SCALE_F16", "paged_attention_decode", "paged_attention_decode_ex",
    "attention_params",
    "decode_work", "prefill_work", "paged_attention_prefill", "paged_attention_prefill_ex",
    "DecodeWorkspace", "kDecodePartitionSize", "gemv_w8a16", "gemv_w4a16", "gemv_w4a16_swiglu",
    "kGemvW4MaxM",
]

kDecodePartitionSize = _lib.RLK_DECODE_PARTITION_SIZE
kGemvW4MaxM = _lib.RLK_GEMV_W4_MAX_M

SCALE_F32 = _lib.RLK_SCALE_F32
SCALE_F16 = _lib.RLK_SCALE_F16


class KVDType:
    kFP16 = _lib.RLK_KV_FP16
    kINT8 = _lib.RLK_KV_INT8


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _ptr(t, dtype, what, allow_none=False):
    if t is None:
        if allow_none:
            return None
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} must not be None")
    if not isinstance(t, torch.Tensor):
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} must be a torch.Tensor")
    if t.dtype != dtype:
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} must be a GPU tensor")
    if not t.is_contiguous():
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} must be contiguous")
    return t.data_ptr()


def _need(t, n, what):
    if t is not None and t.numel() < n:
        raise _lib.Error(_lib.RLK_EINVAL, f"{what} holds {t.numel()} elements, needs {n}")


def embedding_lookup(ids, table, n, hidden, out, stream=None):
    """out[t, :] = table[ids[t], :] for t < n (kernels::embedding_lookup)."""
    if n > 0:
        _need(ids, n, "ids"); _need(out, n * hidden, "out")
    check(lib().rlk_embedding_lookup(_ptr(ids, torch.int32, "ids"), _ptr(table, torch.float16, "table"),
                                     n, hidden, _ptr(out, torch.float16, "out"), _stream(stream)))


def fused_add_rmsnorm(residual, delta, weight, rows, hidden, eps, out, stream=None):
    """residual += delta (unless None); out = rmsnorm(residual) * weight."""
    if rows > 0:
        for t, w in ((residual, "residual"), (delta, "delta"), (out, "out")):
            _need(t, rows * hidden, w)
        _need(weight, hidden, "weight")
    check(lib().rlk_fused_add_rmsnorm(
        _ptr(residual, torch.float16, "residual"), _ptr(delta, torch.float16, "delta", True),
        _ptr(weight, torch.float16, "weight"), rows, hidden, float(eps),
        _ptr(out, torch.float16, "out"), _stream(stream)))


def embedding_rmsnorm(ids, table, n, hidden, weight, eps, residual, out, stream=None):
    """Extension: residual[t, :] = table[ids[t], :]; out = rmsnorm(residual) *
    weight, in one launch -- the reference's embedding_lookup followed by
    fused_add_rmsnorm(delta=None) (llama.cpp:79-80), same results."""
    if n > 0:
        _need(ids, n, "ids"); _need(residual, n * hidden, "residual"); _need(out, n * hidden, "out")
        _need(weight, hidden, "weight")
    check(lib().rlk_embedding_rmsnorm(
        _ptr(ids, torch.int32, "ids"), _ptr(table, torch.float16, "table"), n, hidden,
        _ptr(weight, torch.float16, "weight"), float(eps), _ptr(residual, torch.float16, "residual"),
        _ptr(out, torch.float16, "out"), _stream(stream)))


def silu_and_mul(gate_up, rows, inter, out, stream=None):
    """out[r, i] = silu(gate_up[r, i]) * gate_up[r, inter + i]."""
    if rows > 0:
        _need(gate_up, rows * 2 * inter, "gate_up"); _need(out, rows * inter, "out")
    check(lib().rlk_silu_and_mul(_ptr(gate_up, torch.float16, "gate_up"), rows, inter,
                                 _ptr(out, torch.float16, "out"), _stream(stream)))


def silu_and_mul_interleaved(gate_up, rows, inter, out, stream=None):
    """Same with (gate_i, up_i) interleaved columns."""
    if rows > 0:
        _need(gate_up, rows * 2 * inter, "gate_up"); _need(out, rows * inter, "out")
    check(lib().rlk_silu_and_mul_interleaved(_ptr(gate_up, torch.float16, "gate_up"), rows, inter,
                                             _ptr(out, torch.float16, "out"), _stream(stream)))


def gemv_w8a16(x, m, w, scales, bias, n, k, y, y_fp32=False, stream=None):
    """y[m, n] = (x[m, k] . w^T) * scales (+ bias): INT8 weight [n, k] with one
    fp16 scale per row; y fp16, or fp32 with y_fp32."""
    if m > 0 and n > 0 and k > 0:
        _need(x, m * k, "x"); _need(w, n * k, "w"); _need(scales, n, "scales"); _need(y, m * n, "y")
        if bias is not None:
            _need(bias, n, "bias")
    check(lib().rlk_gemv_w8a16(
        _ptr(x, torch.float16, "x"), m, _ptr(w, torch.int8, "w"), _ptr(scales, torch.float16, "scales"),
        _ptr(bias, torch.float16, "bias", True), n, k,
        _ptr(y, torch.float32 if y_fp32 else torch.float16, "y"), int(bool(y_fp32)), _stream(stream)))


def _gemv_w4_need(x, m, w, scales, offsets, group_size, n, k):
    if m > 0 and k > 0 and group_size > 0 and k % group_size == 0:
        _need(x, m * k, "x"); _need(w, n * k // 2, "w")
        _need(scales, n * (k // group_size), "scales"); _need(offsets, n * (k // group_size), "offsets")


def gemv_w4a16(x, m, w, scales, offsets, group_size, bias, n, k, y, y_fp32=False, stream=None):
    """y[m, n] = x[m, k] . dequant(w)^T (+ bias): INT4 weight [n, k/2] uint8 with
    fp16 scales/offsets [n, k/group_size]; y fp16, or fp32 with y_fp32."""
    _gemv_w4_need(x, m, w, scales, offsets, group_size, n, k)
    if m > 0:
        _need(y, m * n, "y")
    check(lib().rlk_gemv_w4a16(
        _ptr(x, torch.float16, "x"), m, _ptr(w, torch.uint8, "w"),
        _ptr(scales, torch.float16, "scales"), _ptr(offsets, torch.float16, "offsets"), group_size,
        _ptr(bias, torch.float16, "bias", True), n, k,
        _ptr(y, torch.float32 if y_fp32 else torch.float16, "y"), int(bool(y_fp32)),
        _stream(stream)))


def gemv_w4a16_swiglu(x, m, w, scales, offsets, group_size, n, k, y, stream=None):
    """y[m, n/2] = silu(gate) * up from an INT4 weight whose rows are interleaved
    (gate_i, up_i), in the GEMV epilogue."""
    _gemv_w4_need(x, m, w, scales, offsets, group_size, n, k)
    if m > 0:
        _need(y, m * (n // 2), "y")
    check(lib().rlk_gemv_w4a16_swiglu(
        _ptr(x, torch.float16, "x"), m, _ptr(w, torch.uint8, "w"),
        _ptr(scales, torch.float16, "scales"), _ptr(offsets, torch.float16, "offsets"), group_size,
        n, k, _ptr(y, torch.float16, "y"), _stream(stream)))


def gather_rows(src, idx, n, cols, dst, stream=None):
    """dst[i, :] = src[idx[i], :] (idx None: dst[i, :] = src[i, :])."""
    if n > 0:
        if idx is not None:
            _need(idx, n, "idx")
        _need(dst, n * cols, "dst")
    check(lib().rlk_gather_rows(_ptr(src, torch.float16, "src"), _ptr(idx, torch.int32, "idx", True), n, cols,
                                _ptr(dst, torch.float16, "dst"), _stream(stream)))


def resolve_input_ids(input_ids, src, prev_sampled, n, stream=None):
    """input_ids[i] = prev_sampled[src[i]] where src[i] >= 0."""
    if n > 0:
        _need(input_ids, n, "input_ids"); _need(src, n, "src")
    check(lib().rlk_resolve_input_ids(_ptr(input_ids, torch.int32, "input_ids"),
                                      _ptr(src, torch.int32, "src"),
                                      _ptr(prev_sampled, torch.int32, "prev_sampled"), n,
                                      _stream(stream)))


def rope_and_write_kv(qkv, positions, slot_mapping, num_tokens, num_heads, cos_table, sin_table,
                      kv: KVLayerView, stream=None):
    """RoPE on q/k heads (q in place) and paged KV write at slot_mapping[t]."""
    if num_tokens > 0:
        _need(positions, num_tokens, "positions"); _need(slot_mapping, num_tokens, "slot_mapping")
        _need(qkv, num_tokens * (num_heads + 2 * kv.num_kv_heads) * kv.head_dim, "qkv")
    check(lib().rlk_rope_and_write_kv(
        _ptr(qkv, torch.float16, "qkv"), _ptr(positions, torch.int32, "positions"),
        _ptr(slot_mapping, torch.int32, "slot_mapping"), num_tokens, num_heads,
        _ptr(cos_table, torch.float32, "cos_table"), _ptr(sin_table, torch.float32, "sin_table"),
        C.byref(kv), _stream(stream)))


def rope_and_write_kv_ex(qkv, positions, slot_mapping, num_tokens, num_heads, cos_table, sin_table,
                         kv: KVLayerView, qkv_bias=None, scale_dtype=SCALE_F32, stream=None):
    """Extension: optional QKV bias added before RoPE, optional fp16 INT8 scales."""
    if num_tokens > 0:
        _need(positions, num_tokens, "positions"); _need(slot_mapping, num_tokens, "slot_mapping")
        _need(qkv, num_tokens * (num_heads + 2 * kv.num_kv_heads) * kv.head_dim, "qkv")
        _need(qkv_bias, (num_heads + 2 * kv.num_kv_heads) * kv.head_dim, "qkv_bias")
    opt = _lib.RopeKVOptions(_ptr(qkv_bias, torch.float16, "qkv_bias", True), scale_dtype)
    check(lib().rlk_rope_and_write_kv_ex(
        _ptr(qkv, torch.float16, "qkv"), _ptr(positions, torch.int32, "positions"),
        _ptr(slot_mapping, torch.int32, "slot_mapping"), num_tokens, num_heads,
        _ptr(cos_table, torch.float32, "cos_table"), _ptr(sin_table, torch.float32, "sin_table"),
        C.byref(kv), C.byref(opt), _stream(stream)))


def attention_params(q, q_stride, out, num_heads, scale, kv: KVLayerView, block_tables,
                     max_blocks_per_seq, positions) -> _lib.AttentionParams:
    """kernels::AttentionParams from torch tensors (q may be a view into qkv)."""
    return _lib.AttentionParams(
        _ptr(q, torch.float16, "q"), q_stride, _ptr(out, torch.float16, "out"), num_heads,
        float(scale), kv, _ptr(block_tables, torch.int32, "block_tables"), max_blocks_per_seq,
        _ptr(positions, torch.int32, "positions"))


def decode_work(item_token, item_seq, num_items, max_partitions, workspace=None):
    """kernels::DecodeAttentionWork; `workspace` is a DecodeWorkspace (needed
    when max_partitions > 1)."""
    ws = workspace
    return _lib.DecodeAttentionWork(
        _ptr(item_token, torch.int32, "item_token"), _ptr(item_seq, torch.int32, "item_seq"),
        num_items, max_partitions,
        None if ws is None else ws.out.data_ptr(), None if ws is None else ws.max.data_ptr(),
        None if ws is None else ws.sum.data_ptr())


def prefill_work(seq_ids, q_start, q_len, ctx_len, num_seqs, max_q_tiles):
    """kernels::PrefillAttentionWork (max_q_tiles in 32-row tiles, as BatchBuilder writes it)."""
    return _lib.PrefillAttentionWork(
        _ptr(seq_ids, torch.int32, "seq_ids"), _ptr(q_start, torch.int32, "q_start"),
        _ptr(q_len, torch.int32, "q_len"), _ptr(ctx_len, torch.int32, "ctx_len"), num_seqs,
        max_q_tiles)


def paged_attention_prefill(params: _lib.AttentionParams, work: _lib.PrefillAttentionWork,
                            stream=None):
    """Causal paged prefill attention (kernels::paged_attention_prefill)."""
    check(lib().rlk_paged_attention_prefill(C.byref(params), C.byref(work), _stream(stream)))


def paged_attention_prefill_ex(params: _lib.AttentionParams, work: _lib.PrefillAttentionWork,
                               scale_dtype=SCALE_F32, stream=None):
    """Extension: prefill attention over an INT8 cache with fp16 scales."""
    opt = _lib.AttentionOptions(scale_dtype)
    check(lib().rlk_paged_attention_prefill_ex(C.byref(params), C.byref(work), C.byref(opt),
                                               _stream(stream)))


class DecodeWorkspace:
    """Split-K partials of the decode attention, sized like the reference
    model's workspace (src/cuda/model/llama.cpp:37-40)."""

    def __init__(self, max_items, num_heads, max_partitions, head_dim, device="cuda"):
        rows = max_items * num_heads * max_partitions
        self.out = torch.empty(rows * head_dim, dtype=torch.float32, device=device)
        self.max = torch.empty(rows, dtype=torch.float32, device=device)
        self.sum = torch.empty(rows, dtype=torch.float32, device=device)


def paged_attention_decode(params: _lib.AttentionParams, work: _lib.DecodeAttentionWork,
                           stream=None):
    """Flash-decoding paged attention (kernels::paged_attention_decode)."""
    check(lib().rlk_paged_attention_decode(C.byref(params), C.byref(work), _stream(stream)))


def paged_attention_decode_ex(params: _lib.AttentionParams, work: _lib.DecodeAttentionWork,
                              scale_dtype=SCALE_F32, stream=None):
    """Extension: decode attention over an INT8 cache with fp16 scales
    (written by rope_and_write_kv_ex with SCALE_F16)."""
    opt = _lib.AttentionOptions(scale_dtype)
    check(lib().rlk_paged_attention_decode_ex(C.byref(params), C.byref(work), C.byref(opt),
                                              _stream(stream)))


class KVCache:
    """Paged KV cache in one zeroed device allocation, laid out per layer as
    K, V (then k_scale, v_scale for INT8), each [num_blocks, Hkv, bs, D]
    (scales [num_blocks, Hkv, bs] fp32) — the layout of the reference's
    KVCache (src/cuda/model/kv_cache.cpp:25-52).  Block 0 is the scratch block
    that padded rows write into."""

    def __init__(self, num_layers, num_blocks, num_kv_heads, head_dim, block_size=16,
                 dtype=KVDType.kFP16, device="cuda", scale_dtype=SCALE_F32):
        if num_blocks <= 1 or block_size <= 0 or num_layers <= 0:
            raise _lib.Error(_lib.RLK_EINVAL, "bad KV cache config")
        self.num_layers, self.num_blocks = num_layers, num_blocks
        self.num_kv_heads, self.head_dim, self.block_size, self.dtype = (
            num_kv_heads, head_dim, block_size, dtype)
        cells = num_blocks * num_kv_heads * block_size
        elem = 2 if dtype == KVDType.kFP16 else 1
        sbytes = 2 if scale_dtype == SCALE_F16 else 4
        sdt = torch.float16 if scale_dtype == SCALE_F16 else torch.float32
        per_layer = 2 * cells * head_dim * elem + (2 * cells * sbytes if dtype == KVDType.kINT8 else 0)
        self.storage = torch.zeros(per_layer * num_layers, dtype=torch.uint8, device=device)
        self._views, self._tensors = [], []
        shape = (num_blocks, num_kv_heads, block_size, head_dim)
        tdt = torch.float16 if dtype == KVDType.kFP16 else torch.int8
        off = 0
        for _ in range(num_layers):
            kb = cells * head_dim * elem
            k = self.storage[off:off + kb].view(tdt).view(shape); off += kb
            v = self.storage[off:off + kb].view(tdt).view(shape); off += kb
            ks = vs = None
            if dtype == KVDType.kINT8:
                ks = self.storage[off:off + cells * sbytes].view(sdt).view(shape[:3]); off += cells * sbytes
                vs = self.storage[off:off + cells * sbytes].view(sdt).view(shape[:3]); off += cells * sbytes
            view = KVLayerView(k.data_ptr(), v.data_ptr(), ks.data_ptr() if ks is not None else None,
                               vs.data_ptr() if vs is not None else None, block_size, num_kv_heads,
                               head_dim, dtype)
            self._views.append(view)
            self._tensors.append((k, v, ks, vs))

    def layer(self, i) -> KVLayerView:
        return self._views[i]

    def tensors(self, i):
        """(k, v, k_scale, v_scale) torch views of layer i (scales None for FP16)."""
        return self._tensors[i]
