"""Forward pass of the tiny random model of tests/_util.py composed from this
library's layer kernels, in the reference engine's order
(src/cuda/model/llama.cpp:79-150): embedding + RMSNorm, then per layer the QKV
projection, RoPE + paged-KV write, paged attention, the output projection,
residual add + RMSNorm, the gate/up projection, SwiGLU, the down projection,
residual add + RMSNorm; then the LM head.  The projections are plain matmuls
(fp32 accumulation, fp16 outputs, as the engine's fp16 GEMMs): they are not
part of the path under test.  Two backends: the HIP kernels through the C ABI
(GPU), and the CPU oracle's functions (CPU)."""
from __future__ import annotations

import numpy as np

import redline_amd as ra
from tests._util import TINY_INT4_GROUP, TINY_MODEL, int4_dequantize, interleave_rows

PROJ = ("wqkv", "wo", "w_gate_up", "w_down")


def dense_weights(w):
    """float32 projection weights (INT4 ones dequantized as the reference's
    CPU model does)."""
    out = {}
    for name, v in w.items():
        if name.endswith(".scales") or name.endswith(".offsets"):
            continue
        base = name[:-len(".weight")]
        if base + ".scales" in w:
            out[name] = int4_dequantize(v, w[base + ".scales"], w[base + ".offsets"], TINY_INT4_GROUP)
        else:
            out[name] = v.astype(np.float32)
    return out

BS = 16


def batch(n, start=0, seed=3, decode=False, total=None):
    """Metadata of one sequence: n new tokens at positions start.., its block
    table a permutation of blocks 1.. of a pool sized for `total` tokens."""
    total = total or start + n
    nblk = (total + BS - 1) // BS
    blocks = np.random.default_rng(seed).permutation(np.arange(1, nblk + 1, dtype=np.int32))
    b = ra.BatchBuilder(n, 1, 1, nblk, BS, 1 if decode else 0)
    b.add(np.zeros(n, np.int32), start, n, None, blocks)
    meta, shape, lay = b.write()
    return meta, shape, lay, nblk + 1


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def forward_oracle(w, tokens, cfg=TINY_MODEL):
    """CPU: the oracle's restatements of the kernels; logits fp32 [T, V]."""
    import oracle
    T, H, I, D = tokens.size, cfg["hidden"], cfg["inter"], cfg["head_dim"]
    hq, hkv, eps = cfg["heads"], cfg["kv_heads"], cfg["eps"]
    w32 = dense_weights(w)
    meta, shape, lay, nblk = batch(T)
    g = lambda name, n: meta[lay[name]:lay[name] + n]  # noqa: E731
    pos, slots = g("positions", T), g("slot_mapping", T)
    tables = g("block_tables", nblk - 1).reshape(1, nblk - 1)
    cos, sin = oracle.rope_cos_sin_tables(cfg["theta"], D, T)
    mm = lambda x, name: _f16(np.asarray(x, np.float32) @ w32[name].T)  # noqa: E731
    res = oracle.embedding_lookup(tokens, w["tok_embeddings.weight"], H)
    _, x = oracle.fused_add_rmsnorm(res, None, w["layers.0.attn_norm.weight"], eps)
    for layer in range(cfg["layers"]):
        p = f"layers.{layer}."
        qkv = mm(x, p + "wqkv.weight")
        kc = np.zeros((nblk, hkv, BS, D), np.float16)
        vc = np.zeros_like(kc)
        oracle.rope_and_write_kv(qkv, pos, slots, hq, hkv, D, cos, sin, kc, vc)
        att = oracle.paged_attention_prefill(qkv, qkv.shape[1], hq, D ** -0.5, kc, vc, None, None,
                                             tables, g("prefill_seq", 1), g("seq_q_start", 1),
                                             g("seq_q_len", 1), g("seq_ctx_len", 1), T)
        res, x = oracle.fused_add_rmsnorm(res, mm(att, p + "wo.weight"), w[p + "ffn_norm.weight"], eps)
        act = oracle.silu_and_mul(mm(x, p + "w_gate_up.weight"), I)
        nxt = f"layers.{layer + 1}.attn_norm.weight" if layer + 1 < cfg["layers"] else "norm.weight"
        res, x = oracle.fused_add_rmsnorm(res, mm(act, p + "w_down.weight"), w[nxt], eps)
    return np.asarray(x, np.float32) @ w["lm_head.weight"].astype(np.float32).T


class GpuModel:
    """The weights on the GPU, one paged KV cache per layer, and the forward
    pass through the HIP kernels (C ABI).  With INT4 projections, steps of at
    most 32 tokens run them on the INT4 GEMV kernels (gate_up on the fused
    SwiGLU epilogue over its rows interleaved as the reference's loader does,
    src/cuda/model/weights.cpp:157-167); longer steps, where the reference
    engine runs a GEMM, multiply by the dequantized weights."""

    def __init__(self, torch, w, total_tokens, cfg=TINY_MODEL):
        from redline_amd import kernels as K
        self.torch, self.K, self.cfg = torch, K, cfg
        self.int4 = any(k.endswith(".scales") for k in w)
        # fp16 tensors as stored; INT4 projections also dequantized to fp32
        self.w = {k: torch.from_numpy(v).cuda() for k, v in w.items() if v.dtype == np.float16}
        self.w32 = {k: torch.from_numpy(v).cuda() for k, v in dense_weights(w).items()
                    if k not in self.w}
        self.q = {}
        if self.int4:
            for k, v in w.items():
                self.q[k] = torch.from_numpy(np.ascontiguousarray(v)).cuda()
                if "w_gate_up" in k:  # (gate_i, up_i) rows for the fused epilogue
                    self.q[k + ".il"] = torch.from_numpy(np.ascontiguousarray(interleave_rows(v))).cuda()
        D = cfg["head_dim"]
        self.nblk = (total_tokens + BS - 1) // BS + 1
        self.caches = [K.KVCache(1, self.nblk, cfg["kv_heads"], D, BS) for _ in range(cfg["layers"])]
        cos, sin = ra.rope_cos_sin_tables(cfg["theta"], D, total_tokens)
        self.cos, self.sin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()

    def mm(self, x, name):
        torch, K = self.torch, self.K
        base = name[:-len(".weight")]
        if self.int4 and base + ".scales" in self.q and x.shape[0] <= K.kGemvW4MaxM:
            n, k = self.q[name].shape[0], x.shape[1]
            y = torch.empty((x.shape[0], n), dtype=torch.float16, device="cuda")
            K.gemv_w4a16(x.contiguous(), x.shape[0], self.q[name], self.q[base + ".scales"],
                         self.q[base + ".offsets"], TINY_INT4_GROUP, None, n, k, y)
            return y
        if self.int4 and base + ".scales" in self.q:
            return torch.matmul(x.float(), self.w32[name].t()).half()
        return torch.matmul(x, self.w[name].t())

    def gate_up_swiglu(self, x, name):
        """silu(gate) * up of the gate/up projection: the fused INT4 GEMV
        epilogue where it applies, else the projection then silu_and_mul."""
        torch, K, I = self.torch, self.K, self.cfg["inter"]
        n = x.shape[0]
        act = torch.empty((n, I), dtype=torch.float16, device="cuda")
        base = name[:-len(".weight")]
        if self.int4 and n <= K.kGemvW4MaxM:
            K.gemv_w4a16_swiglu(x.contiguous(), n, self.q[name + ".il"],
                                self.q[base + ".scales.il"], self.q[base + ".offsets.il"],
                                TINY_INT4_GROUP, 2 * I, x.shape[1], act)
        else:
            K.silu_and_mul(self.mm(x, name).contiguous(), n, I, act)
        return act

    def step(self, tokens, start, total):
        """New tokens at positions start..: returns fp32 logits [n, V] (the
        tokens' K/V stay in the caches for later steps)."""
        torch, K, cfg = self.torch, self.K, self.cfg
        n, H, I, D = tokens.size, cfg["hidden"], cfg["inter"], cfg["head_dim"]
        hq, hkv, eps = cfg["heads"], cfg["kv_heads"], cfg["eps"]
        decode = n == 1
        meta, shape, lay, _ = batch(n, start, decode=decode, total=total)
        d_meta = torch.from_numpy(meta).cuda()
        sl = lambda name: d_meta[lay[name]:]  # noqa: E731
        ids = torch.from_numpy(tokens).cuda()
        res = torch.empty((n, H), dtype=torch.float16, device="cuda")
        x = torch.empty_like(res)
        K.embedding_rmsnorm(ids, self.w["tok_embeddings.weight"], n, H,
                            self.w["layers.0.attn_norm.weight"], eps, res, x)
        stride = (hq + 2 * hkv) * D
        max_blocks = self.nblk - 1
        for layer in range(cfg["layers"]):
            p = f"layers.{layer}."
            qkv = self.mm(x, p + "wqkv.weight").contiguous()
            kv = self.caches[layer].layer(0)
            K.rope_and_write_kv(qkv, sl("positions"), sl("slot_mapping"), n, hq, self.cos, self.sin, kv)
            att = torch.zeros((n, hq * D), dtype=torch.float16, device="cuda")
            prm = K.attention_params(qkv, stride, att, hq, D ** -0.5, kv, sl("block_tables"),
                                     max_blocks, sl("positions"))
            if decode:
                parts = (start + 1 + K.kDecodePartitionSize - 1) // K.kDecodePartitionSize
                ws = K.DecodeWorkspace(1, hq, parts, D) if parts > 1 else None
                K.paged_attention_decode(prm, K.decode_work(sl("decode_token"), sl("decode_seq"),
                                                            shape.num_decode_items, parts, ws))
            else:
                K.paged_attention_prefill(prm, K.prefill_work(
                    sl("prefill_seq"), sl("seq_q_start"), sl("seq_q_len"), sl("seq_ctx_len"),
                    shape.num_prefill_seqs, shape.max_prefill_q_tiles))
            K.fused_add_rmsnorm(res, self.mm(att, p + "wo.weight").contiguous(),
                                self.w[p + "ffn_norm.weight"], n, H, eps, x)
            act = self.gate_up_swiglu(x, p + "w_gate_up.weight")
            nxt = f"layers.{layer + 1}.attn_norm.weight" if layer + 1 < cfg["layers"] else "norm.weight"
            K.fused_add_rmsnorm(res, self.mm(act, p + "w_down.weight").contiguous(), self.w[nxt],
                                n, H, eps, x)
        logits = torch.matmul(x.float(), self.w["lm_head.weight"].float().t())
        torch.cuda.synchronize()
        return logits.cpu().numpy()
