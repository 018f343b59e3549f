#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernels on one MI355X.

A step is one pass of the layer hot path over one batch of the workload, in
engine order: embedding gather, residual-add + RMSNorm, RoPE + paged-KV write,
residual-add + RMSNorm, SwiGLU.  Default workload: Llama-3.1-8B decode at
batch 32 (C2), the configuration the headline metric is quoted on.

Every step is a replay of a HIP graph holding the five launches for one of R
rotating input sets (R sets > 512 MB, so the 256 MB Infinity Cache cannot serve
the "HBM" traffic); K steps are timed between HIP events on the launch stream.
Per-kernel figures time R back-to-back launches of one kernel in a graph.  The
prefill-sized workloads (C3 mixed 4096 rows, C4 INT8 KV 16k tokens, C5 Qwen2
16k) are timed per kernel as well, since only they can approach the HBM
roofline.  `value` = algorithmic bytes of a step / time of a step (GB/s).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C2]
                       [--no-cpu] [--no-extra] [--only KERNEL] [--reps N]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 640 << 20  # > 2 x Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class LayerData:
    """Device buffers of one workload: R rotating activation sets, the shared
    embedding table / norm weight / RoPE tables / KV cache."""

    def __init__(self, torch, K, w, rotations=None, seed=0):
        from redline_amd.configs import build_batch, token_ids
        import redline_amd as ra
        self.torch, self.K, self.w = torch, K, w
        m = w.model
        self.T = T = w.num_tokens
        dev = "cuda"
        g = torch.Generator(device=dev).manual_seed(seed)
        self.table = (torch.randn((m.vocab, m.hidden), generator=g, device=dev) * 0.02).half()
        self.weight = (1 + 0.1 * torch.randn(m.hidden, generator=g, device=dev)).half()
        cos, sin = ra.rope_cos_sin_tables(m.theta, m.head_dim, w.max_pos)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        dtype = K.KVDType.kINT8 if w.kv_int8 else K.KVDType.kFP16
        self.scale_dtype = K.SCALE_F16 if w.kv_scale_f16 else K.SCALE_F32
        self.cache = K.KVCache(1, w.num_blocks, m.hkv, m.head_dim, w.block_size, dtype,
                               scale_dtype=self.scale_dtype)
        # Qwen2's QKV bias ~N(0, 0.02), added before RoPE by the extension entry point
        self.bias = ((torch.randn(m.qkv_cols, generator=g, device=dev) * 0.02).half()
                     if w.qkv_bias else None)
        # enough sets that every kernel's own footprint over the rotation
        # exceeds twice the Infinity Cache
        smallest = min(self.bytes().values())
        self.R = rotations or max(2, min(1024, -(-ROTATE_BYTES // smallest)))
        rng = np.random.default_rng(seed + 17)
        self.sets = []
        for r in range(self.R):
            meta, shape, lay, _ = build_batch(w, np.random.default_rng(seed * 1000 + r + 1))
            d_meta = torch.from_numpy(meta[:lay["total_words"]]).to(dev)
            s = {
                "ids": torch.from_numpy(token_ids(w, rng)).to(dev),
                "pos": d_meta[lay["positions"]:lay["positions"] + T],
                "slot": d_meta[lay["slot_mapping"]:lay["slot_mapping"] + T],
                "meta": d_meta,
                "emb": torch.empty((T, m.hidden), dtype=torch.float16, device=dev),
                "res": torch.randn((T, m.hidden), generator=g, device=dev).half(),
                "delta": torch.randn((T, m.hidden), generator=g, device=dev).half(),
                "normed": torch.empty((T, m.hidden), dtype=torch.float16, device=dev),
                "qkv": torch.randn((T, m.qkv_cols), generator=g, device=dev).half(),
                "gu": torch.randn((T, 2 * m.inter), generator=g, device=dev).half(),
                "act": torch.empty((T, m.inter), dtype=torch.float16, device=dev),
            }
            self.sets.append(s)
        torch.cuda.synchronize()

    # individual launches on set r (stream = torch's current stream)
    def embedding(self, r):
        s, m = self.sets[r], self.w.model
        self.K.embedding_lookup(s["ids"], self.table, self.T, m.hidden, s["emb"])

    def norm(self, r):
        s, m = self.sets[r], self.w.model
        self.K.fused_add_rmsnorm(s["res"], s["delta"], self.weight, self.T, m.hidden, m.eps,
                                 s["normed"])

    def rope(self, r):
        s, m = self.sets[r], self.w.model
        if self.bias is None and self.scale_dtype == self.K.SCALE_F32:
            self.K.rope_and_write_kv(s["qkv"], s["pos"], s["slot"], self.T, m.hq, self.cos,
                                     self.sin, self.cache.layer(0))
        else:  # C4 (fp16 INT8 scales), C5 (QKV bias)
            self.K.rope_and_write_kv_ex(s["qkv"], s["pos"], s["slot"], self.T, m.hq, self.cos,
                                        self.sin, self.cache.layer(0), self.bias, self.scale_dtype)

    def swiglu(self, r):
        s, m = self.sets[r], self.w.model
        self.K.silu_and_mul(s["gu"], self.T, m.inter, s["act"])

    def stream_copy(self, r):
        """Yardstick: a plain contiguous copy of T hidden rows (the identity
        gather_rows), the embedding gather's bytes without the random rows."""
        s, m = self.sets[r], self.w.model
        self.K.gather_rows(s["res"], None, self.T, m.hidden, s["normed"])

    def norm_first(self, r):
        """The layer's first norm: fused_add_rmsnorm(delta=None) on the
        residual the embedding gather just wrote (llama.cpp:79-80)."""
        s, m = self.sets[r], self.w.model
        self.K.fused_add_rmsnorm(s["emb"], None, self.weight, self.T, m.hidden, m.eps, s["normed"])

    def embedding_norm(self, r):
        """Extension: the gather and the first norm in one launch."""
        s, m = self.sets[r], self.w.model
        self.K.embedding_rmsnorm(s["ids"], self.table, self.T, m.hidden, self.weight, m.eps,
                                 s["emb"], s["normed"])

    def step_plain(self, r):
        """The reference's launches in its forward-pass order (llama.cpp:79-80,
        122, 131, 139 with silu_and_mul for the gated projection's epilogue):
        embedding_lookup, fused_add_rmsnorm(delta=None), rope_and_write_kv,
        fused_add_rmsnorm(delta), silu_and_mul."""
        self.embedding(r)
        self.norm_first(r)
        self.rope(r)
        self.norm(r)
        self.swiglu(r)

    def step(self, r):
        """The same layer step with the first two launches fused
        (embedding_rmsnorm): four launches."""
        self.embedding_norm(r)
        self.rope(r)
        self.norm(r)
        self.swiglu(r)

    def bytes(self):
        from redline_amd import configs as C
        m, T = self.w.model, self.T
        return {
            "embedding_lookup": C.bytes_embedding(T, m.hidden),
            "embedding_rmsnorm": C.bytes_embedding_rmsnorm(T, m.hidden),
            "stream_copy": 4 * T * m.hidden,
            "fused_add_rmsnorm_nodelta": C.bytes_add_rmsnorm(T, m.hidden, delta=False),
            "fused_add_rmsnorm": C.bytes_add_rmsnorm(T, m.hidden),
            "rope_and_write_kv": C.bytes_rope_kv(T, m.hq, m.hkv, m.head_dim, self.w.kv_int8,
                                                 self.w.kv_scale_f16, self.w.qkv_bias),
            "silu_and_mul": C.bytes_swiglu(T, m.inter),
        }


def measured_traffic(workload, kernel_prefix):
    """HBM bytes per launch of a kernel as measured by the rocprofv3 FETCH_SIZE
    / WRITE_SIZE runs summarised in profiles/hbm_traffic_C2_C5.md (None when
    that summary has no row for it)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_C2_C5.md")
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == workload and cells[1].startswith("`" + kernel_prefix):
            return round(float(cells[4]) * 1e6)
    return None


def trace_average_us(workload, kernel_prefix, name):
    """Average dispatch duration (us) of kernel `name` (symbol prefix
    kernel_prefix) in the committed rocprofv3 kernel-trace summary
    profiles/kernel_trace_C2_C5.md (None when absent)."""
    path = os.path.join(ROOT, "profiles", "kernel_trace_C2_C5.md")
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if (len(cells) == 10 and cells[0] == workload and cells[1].startswith("`" + kernel_prefix)
                and cells[2] == name):
            return float(cells[4])
    return None


KERNEL_SYMBOL = {"embedding_lookup": "gather_rows_kernel", "fused_add_rmsnorm": "add_rmsnorm_kernel",
                 "rope_and_write_kv": "rope_kv_kernel", "silu_and_mul": "silu_and_mul_kernel"}


def copy_baseline(torch, nbytes=1 << 30, reps=20):
    """A plain device-to-device copy (torch) of `nbytes`: the practical
    streaming ceiling, read + write bytes counted."""
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").normal_()
    dst = torch.empty_like(src)
    g = capture(torch, lambda: dst.copy_(src))
    ms = time_graph(torch, g, reps)
    del g, src, dst
    return round(2 * nbytes / (ms * 1e-3) / 1e9, 1)


def launch_floor_us(torch, K, calls=1000):
    """Per-launch time of a one-workgroup kernel (resolve_input_ids on one
    id) replayed back to back in a graph: the dispatch floor every call pays."""
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    src = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    g = capture(torch, lambda: [K.resolve_input_ids(ids, src, ids, 1) for _ in range(calls)])
    ms = time_graph(torch, g, 5) / calls
    del g
    return round(ms * 1e3, 3)


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def time_graph(torch, graph, reps, warm_ms=20.0):
    """Median ms per replay over `reps` (at least 20) replays, each between its
    own pair of HIP events on the replay stream, after at least `warm_ms` of
    untimed replays (a single warm-up replay left the first of several
    back-to-back timings of one kernel up to 10% slow)."""
    reps = max(reps, 20)
    t0 = time.perf_counter()
    while True:
        graph.replay()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= warm_ms:
            break
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        graph.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return float(np.median([ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]))


KERNELS = ("embedding_lookup", "fused_add_rmsnorm", "rope_and_write_kv", "silu_and_mul")
# the launches of the decode step that are not in KERNELS
STEP_EXTRA = ("embedding_rmsnorm", "fused_add_rmsnorm_nodelta")


def kernel_fns(data):
    return {"embedding_lookup": data.embedding, "fused_add_rmsnorm": data.norm,
            "rope_and_write_kv": data.rope, "silu_and_mul": data.swiglu,
            "embedding_rmsnorm": data.embedding_norm, "fused_add_rmsnorm_nodelta": data.norm_first,
            "stream_copy": data.stream_copy}


# Launches per timed graph at least: with fewer, the per-replay overhead of
# the graph itself (about 1 us) would be charged to each launch (at C4/C5 the
# rotation holds only R = 3 input sets).
MIN_GRAPH_LAUNCHES = 24


def per_kernel(torch, data, reps, only=None, names=KERNELS, warm=True):
    """Per-call time of each kernel: a graph of back-to-back launches cycling
    through the R rotating input sets (so the inputs come from HBM: the cold
    figure the roofline uses), at least MIN_GRAPH_LAUNCHES of them, replayed
    `reps` times between HIP events on the launch stream; with `warm`, also
    as many launches on input set 0 (the warm figure: inputs left in the
    caches by the previous launch where they fit)."""
    fns = kernel_fns(data)
    nbytes = data.bytes()
    out = {}
    n = data.R * -(-MIN_GRAPH_LAUNCHES // data.R)
    for name in names:
        if only and name != only:
            continue
        f = fns[name]
        g = capture(torch, lambda: [f(i % data.R) for i in range(n)])
        ms = time_graph(torch, g, reps) / n
        del g
        gbs = nbytes[name] / (ms * 1e-3) / 1e9
        out[name] = {"us_per_call": round(ms * 1e3, 3), "gb_per_s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                     "bytes_per_call": nbytes[name]}
        msg = (f"  {data.w.key} {name:20s} {ms * 1e3:9.2f} us  {gbs:8.1f} GB/s "
               f"({100 * gbs / HBM_PEAK_GBS:5.1f}% of peak)  R={data.R}, {n} per graph")
        if warm:
            g = capture(torch, lambda: [f(0) for _ in range(n)])
            ms_w = time_graph(torch, g, reps) / n
            del g
            out[name]["us_per_call_warm"] = round(ms_w * 1e3, 3)
            msg += f"; warm {ms_w * 1e3:9.2f} us"
        log(msg)
    return out


SWEEP_KNOBS = {
    "embedding_lookup": {"RLK_TUNE_GATHER_BS": [64, 128, 256], "RLK_TUNE_GATHER_NT": [0, 1]},
    "fused_add_rmsnorm": {"RLK_TUNE_NORM_TPR": [64, 128, 256, 512], "RLK_TUNE_NORM_NT": [0, 1]},
    "silu_and_mul": {"RLK_TUNE_SWIGLU_BS": [64, 128, 256], "RLK_TUNE_SWIGLU_NT": [0, 1]},
    "rope_and_write_kv": {"RLK_TUNE_ROPE_WPT": [1, 2, 3, 4, 5, 6, 8]},
}



def sweep(torch, data, reps, only=None):
    """Times each kernel under every combination of its launch-policy knobs
    (the RLK_TUNE_* overrides, set through rlk_set_tune_knob)."""
    import itertools
    from redline_amd._lib import set_tune_knob
    for key, knobs in SWEEP_KNOBS.items():
        kern = key
        if only and kern != only:
            continue
        names = list(knobs)
        for vals in itertools.product(*knobs.values()):
            for n, v in zip(names, vals):
                set_tune_knob(n, v)
            r = per_kernel(torch, data, reps, kern, names=(kern,), warm=False)[kern]
            print(json.dumps({"workload": data.w.key, "kernel": kern, "knobs": dict(zip(names, vals)),
                              "us_per_call": r["us_per_call"], "gb_per_s": r["gb_per_s"]}),
                  flush=True)
        for n in names:
            set_tune_knob(n, None)


def attention_bench(torch, K, w, int8, reps, rotations=3, seed=0, eager_calls=0):
    """Decode attention over the workload's decode items: per-call time and
    GB/s (K/V rows read once per GQA group), rotating over `rotations`
    batches drawn from one KV pool filled at random."""
    from redline_amd.configs import build_batch, bytes_decode_attention
    m = w.model
    D = m.head_dim
    cache = K.KVCache(1, w.num_blocks, m.hkv, D, w.block_size,
                      K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ks, vs = cache.tensors(0)
    g = torch.Generator(device="cuda").manual_seed(seed)
    if int8:
        k.copy_(torch.randint(-127, 128, k.shape, generator=g, device="cuda", dtype=torch.int8))
        v.copy_(torch.randint(-127, 128, v.shape, generator=g, device="cuda", dtype=torch.int8))
        ks.fill_(0.01)
        vs.fill_(0.01)
    else:
        k.normal_(generator=g)
        v.normal_(generator=g)
    calls, nbytes = [], 0
    for r in range(rotations):
        meta, shape, lay, tables = build_batch(w, np.random.default_rng(seed * 100 + r + 7))
        T, nd = w.num_tokens, shape.num_decode_items
        d_meta = torch.from_numpy(meta[:lay["total_words"]]).cuda()
        qkv = torch.randn((T, m.qkv_cols), generator=g, device="cuda").half()
        out = torch.empty((T, m.hq * D), dtype=torch.float16, device="cuda")
        parts = (shape.max_context + K.kDecodePartitionSize - 1) // K.kDecodePartitionSize
        ws = K.DecodeWorkspace(nd, m.hq, parts, D)
        sl = lambda name, n: d_meta[lay[name]:lay[name] + n]  # noqa: E731
        p = K.attention_params(qkv, m.qkv_cols, out, m.hq, D ** -0.5, cache.layer(0),
                               d_meta[lay["block_tables"]:], max(len(t) for t in tables),
                               sl("positions", T))
        wk = K.decode_work(sl("decode_token", nd), sl("decode_seq", nd), nd, parts, ws)
        pos = meta[lay["positions"]:lay["positions"] + T]
        toks = meta[lay["decode_token"]:lay["decode_token"] + nd]
        nbytes += bytes_decode_attention(pos[toks] + 1, m.hq, m.hkv, D, int8)
        calls.append((p, wk, qkv, out, ws, d_meta))
    if eager_calls:  # counter-collection mode: plain launches, no timing
        for i in range(eager_calls):
            K.paged_attention_decode(calls[i % rotations][0], calls[i % rotations][1])
        torch.cuda.synchronize()
        return None
    gph = capture(torch, lambda: [K.paged_attention_decode(c[0], c[1]) for c in calls])
    ms = time_graph(torch, gph, reps) / rotations
    del gph
    gbs = nbytes / rotations / (ms * 1e-3) / 1e9
    log(f"  {w.key} paged_attention_decode {'INT8' if int8 else 'FP16'} KV: {ms * 1e3:8.2f} us "
        f"{gbs:8.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:5.1f}% of peak)")
    return {"us_per_call": round(ms * 1e3, 3), "gb_per_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_call": int(nbytes / rotations)}


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix-core peak


def prefill_flops(w):
    """Algorithmic flops of the workload's prefill attention: every causal
    (query, key) pair costs 2 D for q . k and 2 D for p . v, per query head."""
    m = w.model
    pairs = sum(s.n * s.start + s.n * (s.n + 1) // 2 for s in w.segments if s.n > 1)
    return 4 * m.head_dim * m.hq * pairs


def prefill_attention_bench(torch, K, w, reps, rotations=2, seed=0, eager_calls=0):
    """Prefill attention over the workload's prefill sequences (q_len > 1) in
    the workload's cache format, rotating over `rotations` batches drawn from
    one KV pool filled at random; reported against the fp16 MFMA peak."""
    from redline_amd.configs import build_batch
    m = w.model
    D = m.head_dim
    int8 = w.kv_int8
    sdt = K.SCALE_F16 if (int8 and w.kv_scale_f16) else K.SCALE_F32
    cache = K.KVCache(1, w.num_blocks, m.hkv, D, w.block_size,
                      K.KVDType.kINT8 if int8 else K.KVDType.kFP16)
    k, v, ks, vs = cache.tensors(0)
    g = torch.Generator(device="cuda").manual_seed(seed)
    if int8:
        k.copy_(torch.randint(-127, 128, k.shape, generator=g, device="cuda", dtype=torch.int8))
        v.copy_(torch.randint(-127, 128, v.shape, generator=g, device="cuda", dtype=torch.int8))
        if sdt == K.SCALE_F16:
            ks.view(torch.float16).fill_(0.01)
            vs.view(torch.float16).fill_(0.01)
        else:
            ks.fill_(0.01)
            vs.fill_(0.01)
    else:
        k.normal_(generator=g)
        v.normal_(generator=g)
    calls = []
    for r in range(rotations):
        meta, shape, lay, tables = build_batch(w, np.random.default_rng(seed * 100 + r + 11))
        T = w.num_tokens
        d_meta = torch.from_numpy(meta[:lay["total_words"]]).cuda()
        qkv = torch.randn((T, m.qkv_cols), generator=g, device="cuda").half()
        out = torch.empty((T, m.hq * D), dtype=torch.float16, device="cuda")
        sl = lambda name: d_meta[lay[name]:]  # noqa: E731
        p = K.attention_params(qkv, m.qkv_cols, out, m.hq, D ** -0.5, cache.layer(0),
                               sl("block_tables"), max(len(t) for t in tables), sl("positions"))
        wk = K.prefill_work(sl("prefill_seq"), sl("seq_q_start"), sl("seq_q_len"), sl("seq_ctx_len"),
                            shape.num_prefill_seqs, shape.max_prefill_q_tiles)
        calls.append((p, wk, qkv, out, d_meta))
    run = lambda c: K.paged_attention_prefill_ex(c[0], c[1], sdt)  # noqa: E731
    if eager_calls:
        for i in range(eager_calls):
            run(calls[i % rotations])
        torch.cuda.synchronize()
        return None
    gph = capture(torch, lambda: [run(c) for c in calls])
    ms = time_graph(torch, gph, reps) / rotations
    del gph
    fl = prefill_flops(w)
    tfs = fl / (ms * 1e-3) / 1e12
    log(f"  {w.key} paged_attention_prefill {'INT8' if int8 else 'FP16'} KV: {ms * 1e3:9.1f} us "
        f"{tfs:7.1f} TFLOP/s ({100 * tfs / MFMA_F16_PEAK_TFLOPS:5.1f}% of the fp16 MFMA peak)")
    return {"us_per_call": round(ms * 1e3, 2), "tflop_per_s": round(tfs, 1),
            "frac_of_mfma_f16_peak": round(tfs / MFMA_F16_PEAK_TFLOPS, 4), "flops_per_call": fl,
            "kv": "int8" + ("_f16scale" if sdt == K.SCALE_F16 else "") if int8 else "fp16"}


def gemv_bytes(m, n, k, g):
    """Algorithmic bytes of one INT4 GEMV with SwiGLU epilogue: codes, fp16
    scales and offsets, activations read once, fp16 [m, n/2] written."""
    return n * k // 2 + 2 * n * (k // g) * 2 + m * k * 2 + m * (n // 2) * 2


def gemv_bench(torch, K, m, reps, n=2 * 14336, k=4096, g=128, unfused=True, eager_calls=0):
    """INT4 gate_up projection of Llama-3.1-8B (rows interleaved) at decode
    batch m with the fused SwiGLU epilogue, rotating over enough weight sets to
    exceed 2x the Infinity Cache; with `unfused`, also the reference's path for
    a weight without the fused epilogue: GEMV to fp16 [m, n] + silu_and_mul_interleaved."""
    nb = gemv_bytes(m, n, k, g)
    R = max(2, -(-(640 << 20) // nb))
    gen = torch.Generator(device="cuda").manual_seed(m)
    sets = []
    for _ in range(R):
        w = torch.randint(0, 256, (n, k // 2), generator=gen, device="cuda", dtype=torch.uint8)
        sc = (torch.rand((n, k // g), generator=gen, device="cuda") * 0.016 + 0.004).half()
        of = (-7.5 * sc.float()).half()
        x = torch.randn((m, k), generator=gen, device="cuda").half()
        sets.append((x, w, sc, of, torch.empty((m, n // 2), dtype=torch.float16, device="cuda")))
    fused = lambda c: K.gemv_w4a16_swiglu(c[0], m, c[1], c[2], c[3], g, n, k, c[4])  # noqa: E731
    if eager_calls:
        for i in range(eager_calls):
            fused(sets[i % R])
        torch.cuda.synchronize()
        return None
    gph = capture(torch, lambda: [fused(c) for c in sets])
    ms = time_graph(torch, gph, reps) / R
    del gph
    gbs = nb / (ms * 1e-3) / 1e9
    out = {"m": m, "n": n, "k": k, "group_size": g, "us_per_call": round(ms * 1e3, 3),
           "gb_per_s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "bytes_per_call": nb, "rotating_input_sets": R}
    msg = f"  gemv_w4a16_swiglu m={m:2d}: {ms * 1e3:8.2f} us {gbs:8.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:5.1f}%)"
    if unfused:
        scratch = torch.empty((m, n), dtype=torch.float16, device="cuda")

        def two(c):
            K.gemv_w4a16(c[0], m, c[1], c[2], c[3], g, None, n, k, scratch)
            K.silu_and_mul_interleaved(scratch, m, n // 2, c[4])
        gph = capture(torch, lambda: [two(c) for c in sets])
        ms2 = time_graph(torch, gph, reps) / R
        del gph
        out["unfused_us_per_call"] = round(ms2 * 1e3, 3)
        msg += f"; unfused gemv + silu_and_mul_interleaved {ms2 * 1e3:8.2f} us"
    log(msg)
    del sets
    return out


def w8_bytes(m, n, k):
    """Algorithmic bytes of one INT8 GEMV: codes, fp16 row scales, activations
    read once, fp16 [m, n] written."""
    return n * k + 2 * n + m * k * 2 + m * n * 2


def w8_bench(torch, K, m, reps, n=2 * 14336, k=4096, eager_calls=0):
    """INT8 weight-only GEMV (gemv_w8a16) at the Llama-3.1-8B gate_up shape
    (n = 28672, k = 4096, 117 MB of codes), fp16 out, rotating over enough
    weight sets to exceed 2x the Infinity Cache."""
    nb = w8_bytes(m, n, k)
    R = max(2, -(-(640 << 20) // nb))
    gen = torch.Generator(device="cuda").manual_seed(100 + m)
    sets = []
    for _ in range(R):
        w = torch.randint(-128, 128, (n, k), generator=gen, device="cuda", dtype=torch.int8)
        sc = (torch.rand((n,), generator=gen, device="cuda") * 0.004 + 0.001).half()
        x = torch.randn((m, k), generator=gen, device="cuda").half()
        sets.append((x, w, sc, torch.empty((m, n), dtype=torch.float16, device="cuda")))
    call = lambda c: K.gemv_w8a16(c[0], m, c[1], c[2], None, n, k, c[3])  # noqa: E731
    if eager_calls:
        for i in range(eager_calls):
            call(sets[i % R])
        torch.cuda.synchronize()
        return None
    gph = capture(torch, lambda: [call(c) for c in sets])
    ms = time_graph(torch, gph, reps) / R
    del gph, sets
    gbs = nb / (ms * 1e-3) / 1e9
    log(f"  gemv_w8a16 m={m:2d}: {ms * 1e3:8.2f} us {gbs:8.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:5.1f}%)")
    return {"m": m, "n": n, "k": k, "us_per_call": round(ms * 1e3, 3), "gb_per_s": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_call": nb,
            "rotating_input_sets": R}


def cpu_baseline(torch, data, seconds=8.0, max_threads=16):
    """The CPU port of the layer step (oracle/cpu_step.cpp: F16C conversions,
    rows split over a persistent std::thread pool pinned to the affinity
    mask's cores) on the same step, timed on this box's host cores: once on
    one thread and once on min(affinity cores, max_threads) threads, each for
    a bounded `seconds` of full steps over one input set copied to host."""
    import oracle
    L = oracle.cpu_step_lib()
    w, m, T = data.w, data.w.model, data.T
    s = data.sets[0]
    h = lambda t: np.ascontiguousarray(t.cpu().numpy())  # noqa: E731
    table, ids = h(data.table).view(np.uint16), h(s["ids"])
    emb = np.empty((T, m.hidden), np.uint16)
    res, delta, wgt = h(s["res"]).view(np.uint16), h(s["delta"]).view(np.uint16), h(data.weight).view(np.uint16)
    normed = np.empty_like(res)
    qkv = h(s["qkv"]).view(np.uint16)
    pos, slot = h(s["pos"]), h(s["slot"])
    cos, sin = h(data.cos), h(data.sin)
    shape = (w.num_blocks, m.hkv, w.block_size, m.head_dim)
    kc = np.zeros(shape, np.int8 if w.kv_int8 else np.uint16)
    vc = np.zeros_like(kc)
    ks = np.zeros(shape[:3], np.float32) if w.kv_int8 else None
    vs = np.zeros(shape[:3], np.float32) if w.kv_int8 else None
    gu, act = h(s["gu"]).view(np.uint16), np.empty((T, m.inter), np.uint16)
    p = oracle.p
    import ctypes as C
    args = (p(ids), p(table), T, m.hidden, p(emb), p(res), p(delta), p(wgt), C.c_float(m.eps),
            p(normed), p(qkv), p(pos), p(slot), m.hq, m.hkv, m.head_dim, p(cos), p(sin), p(kc),
            p(vc), p(ks), p(vs), w.block_size, int(w.kv_int8), p(gu), m.inter, p(act))
    nb = data.bytes()
    step_bytes = (nb["embedding_lookup"] + nb["fused_add_rmsnorm_nodelta"] + nb["rope_and_write_kv"] +
                  nb["fused_add_rmsnorm"] + nb["silu_and_mul"])
    affinity = L.cps_affinity_cores()

    ops = ("embedding_lookup", "fused_add_rmsnorm_nodelta", "rope_and_write_kv", "fused_add_rmsnorm",
           "silu_and_mul")

    def run(threads):
        """Steps for `seconds`; returns (steps, seconds, each op's seconds)."""
        pool = L.cps_create(threads)
        if not pool:
            raise RuntimeError("CPU baseline needs AVX2 and F16C")
        op_s = np.zeros(len(ops), np.float64)
        try:
            for _ in range(3):
                L.cps_layer_step(pool, *args)  # warm: page in the table rows and the cache
            n, t0 = 0, time.perf_counter()
            while True:
                L.cps_layer_step_timed(pool, *args, p(op_s))
                n += 1
                dt = time.perf_counter() - t0
                if dt >= seconds:
                    break
        finally:
            L.cps_destroy(pool)
        return n, dt, op_s

    def per_op(n, op_s):
        return {k: {"us_per_call": round(op_s[i] / n * 1e6, 2),
                    "gb_per_s": round(nb[k] / (op_s[i] / n) / 1e9, 3)} for i, k in enumerate(ops)}

    n1, dt1, op1 = run(1)
    threads = max(1, min(affinity, max_threads))
    nm, dtm, opm = run(threads)
    gbs = lambda n, dt: round(step_bytes * n / dt / 1e9, 3)  # noqa: E731
    return {"value": gbs(nm, dtm), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": round(dtm / nm * 1e3, 4), "per_kernel": per_op(nm, opm),
            "single_thread": {"value": gbs(n1, dt1), "ms_per_step": round(dt1 / n1 * 1e3, 4),
                              "per_kernel": per_op(n1, op1)},
            "affinity_cores": affinity,
            "sample": f"{w.key} layer steps (embedding, RMSNorm, RoPE+KV, add+RMSNorm, SwiGLU: the "
                      f"reference's five launches) on one "
                      f"input set: {nm} steps in {dtm:.1f} s on {threads} threads, {n1} steps in "
                      f"{dt1:.1f} s on 1 thread; oracle/cpu_step.cpp (F16C, std::thread rows)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="C2")
    ap.add_argument("--reps", type=int, default=20, help="graph replays per kernel timing (their median is reported; at least 20)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the C3-C5 per-kernel figures")
    ap.add_argument("--no-attention", action="store_true", help="skip the decode-attention figures")
    ap.add_argument("--no-gemv", action="store_true", help="skip the INT4 GEMV + SwiGLU figures")
    ap.add_argument("--only", default=None,
                    help="time only this kernel (profiling runs); with --profile-calls, "
                         "'elementwise' selects the layer kernels only")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="seconds of CPU steps per thread count (single and multi)")
    ap.add_argument("--rotations", type=int, default=None,
                    help="rotating input sets (default: enough to exceed 2x the Infinity Cache)")
    ap.add_argument("--sweep", action="store_true",
                    help="launch-policy sweep: time every kernel under each setting of its "
                         "RLK_TUNE_* overrides on the workload, one JSON line per setting")
    ap.add_argument("--profile-calls", type=int, default=0,
                    help="counter-collection mode: N eager calls of each kernel (rotating sets) "
                         "plus N copies of 256 MiB for calibration, then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the fused per-layer kernels are row-independent "
              "(rows or heads would shard across GPUs with no exchange) and this build has no "
              "multi-GPU path.", file=sys.stderr)
        sys.exit(2)

    import torch
    from redline_amd import kernels as K
    from redline_amd.configs import make_workload
    torch.cuda.set_device(0)

    if args.only == "paged_attention_decode" and not args.profile_calls and not args.sweep:
        w = make_workload(args.workload)
        for int8 in (False, True):
            r = attention_bench(torch, K, w, int8, args.reps)
            print(json.dumps({"workload": w.key, "int8_kv": int8, **r}), flush=True)
        return

    if args.only == "paged_attention_prefill" and not args.profile_calls:
        for key in ("C3", "C4", "C5"):
            r = prefill_attention_bench(torch, K, make_workload(key), max(3, args.reps // 4))
            print(json.dumps({"workload": key, **r}), flush=True)
            torch.cuda.empty_cache()
        return

    if args.only == "gemv_w8a16" and not args.profile_calls:
        for m in (1, 8, 16, 32):
            print(json.dumps(w8_bench(torch, K, m, args.reps)), flush=True)
        return

    if args.only == "gemv_w4a16_swiglu" and not args.profile_calls:
        res = []
        for m in (1, 8, 16, 32):
            for cfg in ((0, 9, 11, 12, 13, 14, 15) if args.sweep else [None]):
                if cfg is not None:
                    from redline_amd._lib import set_tune_knob
                    set_tune_knob("RLK_TUNE_W4_CFG", cfg)
                r = gemv_bench(torch, K, m, args.reps, unfused=not args.sweep)
                r["cfg"] = cfg
                print(json.dumps(r), flush=True)
                res.append(r)
        return

    w = make_workload(args.workload)
    log(f"setting up {w.key} ({w.model.name}, T={w.num_tokens})")
    data = LayerData(torch, K, w, rotations=args.rotations)
    nb = data.bytes()
    step_bytes = nb["embedding_rmsnorm"] + nb["rope_and_write_kv"] + nb["fused_add_rmsnorm"] + nb["silu_and_mul"]
    plain_bytes = (nb["embedding_lookup"] + nb["fused_add_rmsnorm_nodelta"] + nb["rope_and_write_kv"] +
                   nb["fused_add_rmsnorm"] + nb["silu_and_mul"])

    if args.sweep:
        sweep(torch, data, args.reps, args.only)
        return

    if args.profile_calls:
        fns = kernel_fns(data)
        for name in KERNELS + STEP_EXTRA + ("stream_copy",):
            if args.only and args.only not in (name, "elementwise"):
                continue
            if name == "stream_copy" and args.only != name:
                continue  # the yardstick shares gather_rows_kernel's symbol: only on request
            for i in range(args.profile_calls):
                fns[name](i % data.R)
        if args.only in (None, "paged_attention_decode"):
            for int8 in (False, True):
                attention_bench(torch, K, w, int8, 0, eager_calls=args.profile_calls)
        if args.only in (None, "gemv_w4a16_swiglu"):
            for m in (1, 8, 16, 32):
                gemv_bench(torch, K, m, 0, eager_calls=args.profile_calls)
        if args.only in (None, "gemv_w8a16"):
            for m in (1, 8, 16, 32):
                w8_bench(torch, K, m, 0, eager_calls=args.profile_calls)
        if args.only in (None, "paged_attention_prefill"):
            for key in ("C3", "C4", "C5"):
                prefill_attention_bench(torch, K, make_workload(key), 0, eager_calls=2)
        src = torch.empty(128 << 20, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.profile_calls):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_calls": args.profile_calls, "workload": w.key,
                          "bytes_per_call": nb, "copy_bytes": 2 * src.numel() * 2,
                          "rotating_input_sets": data.R}))
        return

    def time_steps(step, data, steps=None, warmup=None):
        """K timed steps after W warmup steps, every step on its own rotating
        input set.  The warm-up takes the last W % R sets of the rotation (and
        W // R full rotations before them); the timed steps start at set 0 and
        walk the rotation in order, so no timed step reads a set the warm-up
        touched less than R - W % R sets earlier (R sets > 2x the Infinity
        Cache).  Replays of graphs of R (or fewer) steps, between HIP events on
        the launch stream."""
        steps = args.steps if steps is None else steps
        warmup = args.warmup if warmup is None else warmup
        R = data.R
        full = capture(torch, lambda: [step(r) for r in range(R)])
        rem = capture(torch, lambda: [step(r) for r in range(steps % R)]) if steps % R else None
        wrem = (capture(torch, lambda: [step(r) for r in range(R - warmup % R, R)])
                if warmup % R else None)
        for _ in range(warmup // R):
            full.replay()
        if wrem is not None:
            wrem.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps // R):
            full.replay()
        if rem is not None:
            rem.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        del full, rem, wrem
        return ms
    result = {}
    if args.only is None:
        ms_step = time_steps(data.step, data)
        value = step_bytes / (ms_step * 1e-3) / 1e9
        log(f"{w.key} step (4 launches, embedding_rmsnorm): {ms_step * 1e3:.2f} us, {value:.1f} GB/s")
        result.update(ms_per_step=round(ms_step, 5), value=round(value, 2))
        ms_plain = time_steps(data.step_plain, data)
        log(f"{w.key} step of the reference's 5 launches: {ms_plain * 1e3:.2f} us, "
            f"{plain_bytes / (ms_plain * 1e-3) / 1e9:.1f} GB/s")
        result["step_plain"] = {"us_per_step": round(ms_plain * 1e3, 3),
                                "gb_per_s": round(plain_bytes / (ms_plain * 1e-3) / 1e9, 1),
                                "bytes_per_step": plain_bytes,
                                "launches": "embedding_lookup, fused_add_rmsnorm(delta=None), "
                                            "rope_and_write_kv, fused_add_rmsnorm, silu_and_mul"}

    kern = per_kernel(torch, data, args.reps, args.only,
                      KERNELS + (STEP_EXTRA if args.only is None or args.only in STEP_EXTRA else ()))
    rot = data.R
    del data
    torch.cuda.empty_cache()
    if args.only is not None:
        print(json.dumps({"only": args.only, "workload": w.key, "kernels": kern}))
        return

    # The dominant kernel (most bytes per launch) at its per-call time in a
    # graph of back-to-back launches (HIP events on the launch stream); beside
    # it, the same bytes over the average dispatch duration of the committed
    # rocprofv3 kernel trace of this command (profiles/kernel_trace_C2_C5.md).
    dominant = max(KERNELS, key=lambda k: nb[k])
    dk = kern[dominant]
    trace_us = trace_average_us(w.key, KERNEL_SYMBOL[dominant], dominant)
    roofline = {"bound": "hbm", "kernel": dominant, "achieved": dk["gb_per_s"],
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dk["frac_of_hbm_peak"],
                "us_per_launch": dk["us_per_call"],
                "trace_us_per_dispatch": trace_us,
                "trace_frac": (round(nb[dominant] / (trace_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                               if trace_us else None),
                "trace_source": "profiles/kernel_trace_C2_C5.md (rocprofv3 --kernel-trace "
                                "--stats of this command; the profiler's per-dispatch "
                                "signalling serialises launches and adds ~0.4 us to each "
                                "2-3 us C2 dispatch, so us_per_launch is the kernel's own "
                                "figure)",
                "traffic": measured_traffic(w.key, KERNEL_SYMBOL[dominant]),
                "traffic_source": "profiles/hbm_traffic_C2_C5.md (rocprofv3 FETCH_SIZE and "
                                  "WRITE_SIZE, each scaled by its reading for a 256 MiB copy)",
                "bytes_per_launch": nb[dominant]}

    extra = {}
    if not args.no_extra:
        for key in ("C3", "C4", "C5"):
            wx = make_workload(key)
            log(f"setting up {key} ({wx.model.name}, T={wx.num_tokens})")
            dx = LayerData(torch, K, wx)
            extra[key] = per_kernel(torch, dx, max(3, args.reps // 4),
                                    names=KERNELS + STEP_EXTRA + ("stream_copy",))
            if key == "C3":
                # the layer step at the prefill shape, in both launch orders:
                # 2 x R steps after R warm-up steps (every set cold)
                nbx = dx.bytes()
                for name, fn, nbytes in (
                        ("step", dx.step, nbx["embedding_rmsnorm"] + nbx["rope_and_write_kv"] +
                         nbx["fused_add_rmsnorm"] + nbx["silu_and_mul"]),
                        ("step_plain", dx.step_plain, nbx["embedding_lookup"] +
                         nbx["fused_add_rmsnorm_nodelta"] + nbx["rope_and_write_kv"] +
                         nbx["fused_add_rmsnorm"] + nbx["silu_and_mul"])):
                    ms = time_steps(fn, dx, steps=2 * dx.R * 4, warmup=dx.R)
                    gbs = nbytes / (ms * 1e-3) / 1e9
                    extra[key][name] = {"us_per_step": round(ms * 1e3, 3), "gb_per_s": round(gbs, 1),
                                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                        "bytes_per_step": nbytes}
                    log(f"  {key} {name:20s} {ms * 1e3:9.2f} us  {gbs:8.1f} GB/s "
                        f"({100 * gbs / HBM_PEAK_GBS:5.1f}% of peak)")
            del dx
            torch.cuda.empty_cache()

    gemv, w8 = [], []
    if not args.no_gemv:
        for m in (1, 8, 16, 32):
            gemv.append(gemv_bench(torch, K, m, args.reps))
            torch.cuda.empty_cache()
        for m in (1, 8, 16, 32):
            w8.append(w8_bench(torch, K, m, args.reps))
            torch.cuda.empty_cache()

    prefill = {}
    if not args.no_attention:
        for key in ("C3", "C4", "C5"):
            prefill[key] = prefill_attention_bench(torch, K, make_workload(key), max(3, args.reps // 4))
            torch.cuda.empty_cache()
    attention = {}
    if not args.no_attention:
        for int8 in (False, True):
            attention["int8_kv" if int8 else "fp16_kv"] = attention_bench(torch, K, w, int8, args.reps)
            torch.cuda.empty_cache()

    copy = copy_baseline(torch)
    floor = launch_floor_us(torch, K)
    log(f"device copy baseline: {copy} GB/s; one-workgroup launch floor {floor} us")

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle/cpu_step.cpp, 1 and N threads) ...")
        dcpu = LayerData(torch, K, w, rotations=1)
        cpu = cpu_baseline(torch, dcpu, args.cpu_seconds)
        del dcpu
        log(f"CPU: {cpu['value']} GB/s, {cpu['ms_per_step']} ms/step on {cpu['cores']} threads; "
            f"1 thread {cpu['single_thread']['value']} GB/s")

    line = {
        "metric": "achieved HBM GB/s (% of peak) and us/call per fused layer kernel, 8B decode b32",
        "value": result["value"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": result["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"{w.key}: {w.model.name}-shaped decode, batch {w.num_tokens}"
                               if w.key == "C2" else f"{w.key}: {w.model.name}, T={w.num_tokens}",
                   "step": "embedding_rmsnorm (embedding_lookup + fused_add_rmsnorm(delta=None) "
                           "in one launch), rope_and_write_kv (FP16 KV), fused_add_rmsnorm, "
                           "silu_and_mul",
                   "global_batch": w.num_tokens, "rotating_input_sets": rot,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kern,
        "step_plain": result.get("step_plain"),
        "prefill": extra,
        "decode_attention": attention,
        "prefill_attention": prefill,
        "gemv_w4a16_swiglu": gemv,
        "gemv_w8a16": w8,
        "copy_baseline_gb_per_s": copy,
        "launch_floor_us": floor,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
