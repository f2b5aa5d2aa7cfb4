#!/usr/bin/env python3
"""Benchmark of the MI355X DSA sparse-attention hot path on one GPU.

Headline (BASELINE.json metric "sparse MLA decode us/layer @180k ctx (HBM
GB/s); indexer prefill TFLOPS @64k"):

* step = one decode step of the model's DSA attention: sparse MLA decode
  for a batch of 4 tokens (64 heads, qk 576 / v 512, top-2048 keys, 180k
  context, fp8_ds_mla paged cache) through `--layers` layers (default 78,
  GLM-5.1's depth), each layer with its own queries and top-k indices so the
  gathered rows do not stay resident in the 256 MB MALL.  The layer calls are
  captured once in a HIP graph and replayed; `value` is microseconds per
  layer (lower is better).
* extra records: indexer prefill logits TFLOPS over a 64k-token causal
  prefill (the caller's 128-row sub-chunks, causal-triangle FLOPs only), a
  context-flatness sweep of the decode, the roofline of the decode kernel
  and the CPU baseline (the oracle's PyTorch restatement on the host cores),
  one whole DSA decode layer step (cache writes, indexer, top-k, the two
  head projections and the attention) at the same shape, and the dense MLA
  decode (sm70_mla_decode) at 4k / 32k / 131k context, and the dense varlen
  MLA prefill attention on one causal 16k-token sequence, and the key-shard
  indexer merge (tp=4, 4096 rows).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L]
Only one GPU is supported: --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

METRIC = ("sparse MLA decode µs/layer @180k ctx (HBM GB/s); "
          "indexer prefill TFLOPS @64k")
HBM_PEAK_GBPS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3
# The reference's own published kernel figures (NVIDIA V100, other shapes;
# reference README.md:42-44, sm70_mla_decode.cu:483-484 and :1805-1806,
# sm70_attn_fp8.cu:10-12), quoted beside the matching extra records.
V100_PUBLISHED = {
    "indexer_prefill_tflops": 44.0,   # packed-Q logits, key spans 8k-49k, B=128
    "sparse_prefill_tflops": 15.73,   # warp-specialised fp8 prefill, B=1024, ctx 48k
    "fp8_gemv_m1_gbps": 630.0,        # weight-only GEMV, M=1
}
# algorithmic bytes of one C3 decode layer at B=4 (gathered 656-B rows,
# q, o, lse, idx and the block-table entries read)
DECODE_BYTES = 5_997_568
DECODE_FLOPS = 4 * 64 * 2048 * (576 + 512) * 2


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "sparse_mla_decode_c3_pmc.md")


def measured_traffic():
    """HBM bytes per decode layer from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE of both kernels, scaled by the copy-kernel
    calibration); None when the summary is absent."""
    try:
        for ln in open(TRAFFIC_PROFILE):
            if ln.startswith("traffic_bytes_per_layer:"):
                return int(ln.split(":")[1])
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=78)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extra", action="store_true", help="only the headline decode")
    p.add_argument("--no-kernel-times", action="store_true",
                   help="skip the per-kernel device times (torch.profiler) of the headline")
    p.add_argument("--extra", default="all",
                   help="comma list of extra records: sweep, indexer_prefill, sparse_prefill, "
                        "indexer_decode, gemv, k_store (default all)")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--calib-copy-mib", type=int, default=0,
                   help="run one device copy of this many MiB first (a known-size "
                        "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return p.parse_args()


def time_graph(torch, graph, steps, warmup):
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)  # ms


def capture(torch, fn):
    fn()  # eager run: first-launch attribute setup happens outside capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def cache_copies(cache_bytes, layers, pool_bytes=3 << 30):
    """Distinct latent caches the timed decode graph rotates over: enough that
    their total (at least 3 GB, and at least 8 caches) dwarfs the 256 MB MALL,
    so a layer's gathered rows were last touched several GB of traffic ago."""
    return max(1, min(layers, max(8, -(-pool_bytes // cache_bytes))))


def kernel_times(torch, graph, replays=2):
    """Average device duration (us) of each kernel of `graph` over `replays`
    replays, from torch.profiler's device timestamps; {} if the profiler is
    unavailable here (e.g. under another tracer)."""
    try:
        from torch.profiler import profile, ProfilerActivity
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            for _ in range(replays):
                graph.replay()
            torch.cuda.synchronize()
        agg = {}
        for e in prof.events():
            if e.device_type != torch.autograd.DeviceType.CUDA:
                continue
            name = e.name.split("(")[0].replace("mi355dsa::", "")
            for k in ("sparse_mla_decode_dma_kernel", "sparse_mla_merge_kernel"):
                if k in name:
                    name = k
            agg.setdefault(name, []).append(e.device_time_total)
        return {k: (sum(v) / len(v), len(v)) for k, v in agg.items()}
    except Exception as exc:  # profiler absent or refused: report nothing
        log(f"kernel times unavailable: {exc}")
        return {}


def bench_decode(torch, pkg, dev, ctx, layers, steps, warmup, seed=3, per_kernel=False):
    """C3 decode: `layers` layers with their own q and idx, layer l reading
    cache copy l % n (cache_copies), replayed from one HIP graph.  With
    per_kernel, d["kernel_us"] holds each kernel's average device time over
    two more replays of the same graph."""
    S = pkg.synthetic
    ops = pkg._sm70_ops
    d = S.decode_inputs(B=4, H=64, ctx=ctx, topk=2048, fp8=True, device=dev, seed=seed)
    n_kv = cache_copies(d["kv"].numel(), layers)
    kvs = [d["kv"]] + [d["kv"].clone() for _ in range(n_kv - 1)]
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 100)
    idxs = [S.sorted_unique_positions(4, 2048, ctx, g, dev) for _ in range(layers)]
    qs = [(torch.randn(4, 64, 576, generator=g, device=dev) / 24.0).to(torch.float16)
          for _ in range(layers)]
    outs = [torch.empty(4, 64, 512, dtype=torch.float16, device=dev) for _ in range(layers)]
    lses = [torch.empty(4, 64, device=dev) for _ in range(layers)]
    d["n_caches"] = n_kv

    def run():
        for l in range(layers):
            ops.sm70_sparse_mla_decode(outs[l], lses[l], qs[l], kvs[l % n_kv], idxs[l], d["bt"],
                                       d["seq"], d["scale"])

    graph = capture(torch, run)
    ms = time_graph(torch, graph, steps, warmup)
    assert all(torch.isfinite(o).all() for o in outs[:2])
    if per_kernel:
        d["kernel_us"] = kernel_times(torch, graph)
    del graph, kvs[1:]
    return ms, d, idxs, qs


def bench_decode_batch(torch, pkg, dev, B, layers, steps, warmup, ctx=184320, seed=11):
    """C3's decode at batch B (64 heads, topk 2048, 180k context per token,
    fp8_ds_mla): the tokens' block tables draw pages from one shared pool of
    at most 8 GB, so every layer's gathered rows come from HBM; `layers`
    layers with their own q and idx are replayed from one HIP graph."""
    S = pkg.synthetic
    ops = pkg._sm70_ops
    page = 64
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    bps = ctx // page
    pool = min(B * bps, (8 << 30) // (656 * page))
    kv = S.latent_cache(pool * page, True, g, dev)
    bt = torch.randint(0, pool, (B, bps), generator=g, device=dev, dtype=torch.int32)
    seq = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    idxs = [S.sorted_unique_positions(B, 2048, ctx, g, dev) for _ in range(layers)]
    qs = [(torch.randn(B, 64, 576, generator=g, device=dev) / 24.0).to(torch.float16)
          for _ in range(layers)]
    o = torch.empty(B, 64, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(B, 64, device=dev)

    def run():
        for l in range(layers):
            ops.sm70_sparse_mla_decode(o, lse, qs[l], kv, idxs[l], bt, seq, 576 ** -0.5)

    graph = capture(torch, run)
    ms = time_graph(torch, graph, steps, warmup)
    del graph
    us = ms * 1000.0 / (steps * layers)
    nbytes = B * 2048 * 656 + B * 64 * (576 + 512) * 2 + B * 64 * 4 + B * 2048 * 8
    gbps = nbytes / (us * 1e-6) / 1e9
    flops = B * 64 * 2048 * (576 + 512) * 2
    return {"us_per_layer": round(us, 2), "gbps": round(gbps, 1),
            "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
            "tflops": round(flops / (us * 1e-6) / 1e12, 1),
            "frac_fp16_peak": round(flops / (us * 1e-6) / 1e12 / FP16_PEAK_TFLOPS, 4),
            "layers": layers}


def decode_splits(pkg, B, H=64, topk=2048):
    """Split count the library runs for a decode batch (from its workspace
    size: B * H * splits * (512 fp16 + 2 fp32) bytes; 1 when none)."""
    ws = pkg._lib.lib().mi355_dsa_sparse_mla_workspace_size(B, H, topk)
    return max(1, ws // (B * H * 1032))


def bench_indexer_prefill(torch, pkg, dev, T=65536, sub=128, steps=3, warmup=1):
    """Config C4 indexer: packed-Q logits over a causal 64k prefill, in the
    caller's sub-chunks (reference/sparse_attn_indexer.py:764-881)."""
    ops = pkg._sm70_ops
    page = 64
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    npg = (T + page - 1) // page
    kc = torch.randn(npg, page, 128, generator=g, device=dev).to(torch.float16)
    bt_row = torch.randperm(npg, generator=g, device=dev).to(torch.int32)
    bt = bt_row[None].expand(sub, npg).contiguous()
    q = torch.randn(T, 32, 128, generator=g, device=dev).to(torch.float16)
    w = (torch.randn(T, 32, generator=g, device=dev) / 32 ** 0.5).to(torch.float16)
    score_buf = torch.empty(sub * T, device=dev)
    chunks = []
    for lo in range(0, T, sub):
        n = min(sub, T - lo)
        qs = q[lo:lo + n]
        n16 = (n + 15) // 16 * 16
        if n16 != n:
            qs = torch.nn.functional.pad(qs, (0, 0, 0, 0, 0, n16 - n))
        qp = qs.reshape(n16 // 16, 16, 32, 8, 16).permute(2, 0, 3, 1, 4).contiguous()
        max_kv = min(npg * page, (lo + n + 63) // 64 * 64)
        seq = torch.arange(lo + 1, lo + n + 1, dtype=torch.int32, device=dev)
        chunks.append((qp, w[lo:lo + n].contiguous(), seq, n, max_kv))
    del q

    def run():
        for qp, wc, seq, n, max_kv in chunks:
            score = score_buf[: n * max_kv].view(n, max_kv)
            ops.sm70_indexer_logits_packed(score, qp, kc, wc, bt[:n], seq)

    graph = capture(torch, run)
    ms = time_graph(torch, graph, steps, warmup) / steps
    flops = 8192.0 * T * (T + 1) / 2
    del graph
    return ms, flops


SPARSE_PREFILL_T = 65536
EXTRAS = ("sweep", "batch_sweep", "indexer_prefill", "sparse_prefill", "indexer_decode", "gemv", "k_store",
          "dsa_layer", "dense_decode", "varlen_prefill", "shard_merge", "c1", "prefill_topk",
          "dsa_layer_prefill")


def sparse_prefill_flops(T=SPARSE_PREFILL_T, topk=2048, heads=64):
    keys = sum(min(t + 1, topk) for t in range(T))
    return keys * heads * (576 + 512) * 2, keys


def bench_sparse_prefill(torch, pkg, dev, fp8=True, T=SPARSE_PREFILL_T, sub=4096, steps=2):
    """Config C4 sparse MLA prefill: one 64k-token causal sequence, 64 heads,
    top-2048 keys per token (causally masked: token t selects min(t+1, 2048)
    distinct positions < t+1), latent cache of the sequence (MALL-resident),
    run in 4096-token launches of the op (B = 4096 takes the 64-head prefill
    configuration).  FLOPs count only the selected keys."""
    S = pkg.synthetic
    ops = pkg._sm70_ops
    page = 64
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    npg = T // page
    kv = S.latent_cache(T, fp8, g, dev)
    bt_row = torch.randperm(npg, generator=g, device=dev).to(torch.int32)
    bt = bt_row[None].expand(sub, npg).contiguous()
    q = (torch.randn(sub, 64, 576, generator=g, device=dev) / 24.0).to(torch.float16)
    j = torch.arange(2048, device=dev, dtype=torch.float64)
    chunks = []
    for lo in range(0, T, sub):
        t = torch.arange(lo, lo + sub, device=dev, dtype=torch.float64)
        n = t + 1
        u = torch.rand(sub, 1, generator=g, device=dev, dtype=torch.float64)
        spread = torch.floor((j[None] + u) * n[:, None] / 2048.0)
        idx = torch.where(n[:, None] <= 2048, torch.where(j[None] < n[:, None], j[None], -1.0), spread)
        chunks.append((idx.to(torch.int32), (t + 1).to(torch.int32)))
    o = torch.empty(sub, 64, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(sub, 64, device=dev)
    scale = 576 ** -0.5

    def run():
        for idx, seq in chunks:
            ops.sm70_sparse_mla_decode(o, lse, q, kv, idx, bt, seq, scale)

    run()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        run()
    e1.record(st)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    ms = e0.elapsed_time(e1) / steps
    flops, keys = sparse_prefill_flops(T)
    tf = flops / (ms * 1e-3) / 1e12
    return {"tflops": round(tf, 2), "ms": round(ms, 3), "flops": flops, "selected_keys": keys,
            "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4),
            "workload": ("65536-token causal prefill, 64 heads, qk 576 / v 512, top-2048 per "
                         "token, %s latent cache, 4096-token launches, selected-key FLOPs only"
                         % ("fp8_ds_mla" if fp8 else "fp16"))}


def graph_time_per_call(torch, fn, n_calls, steps=10, warmup=2):
    """Captures fn (n_calls launches) in a graph; returns microseconds per call."""
    graph = capture(torch, fn)
    ms = time_graph(torch, graph, steps, warmup)
    del graph
    return ms * 1000.0 / (steps * n_calls)


def bench_indexer_decode(torch, pkg, dev, copies=5):
    """Config C2: indexer logits (fused histogram) + decode top-k, B=4 x 64k
    keys, fp16 indexer-K cache; `copies` distinct caches (> 256 MB MALL).
    Also the logits alone on the 132-byte fp8 indexer-K cache the reference
    offers beside fp16 rows (glue.patch:2952-2966)."""
    ops = pkg._sm70_ops
    ins = [pkg.synthetic.indexer_decode_inputs(device=dev, seed=20 + i, fp8=True)
           for i in range(copies)]
    B, max_kv = 4, ins[0]["max_kv"]
    score = torch.empty(B, max_kv, device=dev)
    hist = torch.zeros(B, 4096, dtype=torch.int32, device=dev)
    idx = torch.empty(B, 2048, dtype=torch.int32, device=dev)

    def logits_only():
        for d in ins:
            ops.sm70_indexer_logits(score, d["q"], d["kc"], d["w"], d["bt"], d["seq"], None)

    def full():
        for d in ins:
            hist.zero_()
            ops.sm70_indexer_logits(score, d["q"], d["kc"], d["w"], d["bt"], d["seq"], hist)
            ops.sm70_decode_topk(idx, score, d["seq"], hist, 2048)

    def logits_fp8():
        for d in ins:
            ops.sm70_indexer_logits(score, d["q"], d["kc8"], d["w"], d["bt"], d["seq"], None)

    us_logits = graph_time_per_call(torch, logits_only, copies)
    us_full = graph_time_per_call(torch, full, copies)
    us_fp8 = graph_time_per_call(torch, logits_fp8, copies)
    nbytes = 4 * 65536 * 256 + 4 * 65536 * 4 + 4 * 4096 * 4 + 4 * (32 * 128 + 32) * 2
    nbytes8 = nbytes - 4 * 65536 * (256 - 132)
    return {
        "logits_us": round(us_logits, 2),
        "logits_gbps": round(nbytes / (us_logits * 1e-6) / 1e9, 1),
        "logits_frac_hbm": round(nbytes / (us_logits * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "logits_plus_topk_us": round(us_full, 2),
        "logits_fp8_index_k_us": round(us_fp8, 2),
        "logits_fp8_index_k_gbps": round(nbytes8 / (us_fp8 * 1e-6) / 1e9, 1),
        "workload": "C2: B=4, 65536 keys each, 32 heads x 128, fp16 indexer-K, top-2048",
    }


def bench_gemv(torch, pkg, dev):
    """Config C5a: fp8 weight-only GEMV at the three projection shapes, M=1
    and 4, rotating weight copies past the 256 MB MALL."""
    ops = pkg._sm70_ops
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    for (N, K) in ((24576, 6144), (6144, 24576), (2112, 6144)):
        copies = max(2, (600 << 20) // (N * K))
        ws = [torch.randint(0, 0x7E, (N, K), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
              for _ in range(copies)]
        ss = [torch.rand((N + 127) // 128, (K + 127) // 128, generator=g, device=dev) * 1e-3
              for _ in range(copies)]
        for M in (1, 4):
            x = torch.randn(M, K, generator=g, device=dev).to(torch.float16)
            y = torch.empty(M, N, dtype=torch.float16, device=dev)

            def fn():
                for w, s in zip(ws, ss):
                    ops.sm70_attn_fp8_gemv(y, x, w, s)

            us = graph_time_per_call(torch, fn, copies)
            nbytes = N * K + 4 * ((N + 127) // 128) * ((K + 127) // 128) + 2 * M * K + 2 * M * N
            gbps = nbytes / (us * 1e-6) / 1e9
            out[f"{N}x{K}_M{M}"] = {"us": round(us, 2), "gbps": round(gbps, 1),
                                    "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        del ws, ss
        torch.cuda.empty_cache()
    return out


def bench_k_store(torch, pkg, dev, n_tok=65536, copies=8):
    """Config C5b: indexer-K scatter of 64k tokens into random unique slots, and
    the fp8_ds_mla latent-cache writer on 64k tokens."""
    ops = pkg._sm70_ops
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    out = {}
    for fp8 in (False, True):
        ks = [torch.randn(n_tok, 128, generator=g, device=dev).to(torch.float16) for _ in range(copies)]
        slots = [torch.randperm(n_tok, generator=g, device=dev).to(torch.int32) for _ in range(copies)]
        caches = [torch.zeros(n_tok // 64, 64, 132 if fp8 else 128,
                              dtype=torch.uint8 if fp8 else torch.float16, device=dev)
                  for _ in range(copies)]

        def fn():
            for k, sl, c in zip(ks, slots, caches):
                ops.sm70_indexer_k_store(c, k, sl)

        us = graph_time_per_call(torch, fn, copies)
        nbytes = n_tok * (256 + (132 if fp8 else 256) + 4)
        gbps = nbytes / (us * 1e-6) / 1e9
        out["fp8" if fp8 else "fp16"] = {"us": round(us, 2), "gbps": round(gbps, 1),
                                         "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        del ks, slots, caches
    # latent-cache writer (concat_and_cache_mla, fp8_ds_mla): the same 64k
    # tokens as kv_c [T, 512] + k_pe [T, 64] fp16 into 656-byte rows
    cops = pkg._cache_ops
    kvs = [torch.randn(n_tok, 576, generator=g, device=dev).to(torch.float16)
           for _ in range(copies)]
    slots = [torch.randperm(n_tok, generator=g, device=dev) for _ in range(copies)]
    caches = [torch.zeros(n_tok // 64, 64, 656, dtype=torch.uint8, device=dev)
              for _ in range(copies)]
    one = torch.ones((), device=dev)

    def fn2():
        for kv, sl, c in zip(kvs, slots, caches):
            cops.concat_and_cache_mla(kv[:, :512], kv[:, 512:], c, sl, "fp8_ds_mla", one)

    us = graph_time_per_call(torch, fn2, copies)
    nbytes = n_tok * (1152 + 8 + 656)
    gbps = nbytes / (us * 1e-6) / 1e9
    out["latent_fp8_ds_mla"] = {"us": round(us, 2), "gbps": round(gbps, 1),
                                "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
    del kvs, slots, caches
    return out


def bench_dsa_layer(torch, pkg, dev, ctx=184320, copies=3, P=128, V=128, idx_fp8=False):
    """One whole DSA decode layer step at the C3 shape (B=4 tokens at ctx,
    64 heads, top-2048): the step's cache writes (latent + indexer-K), the
    indexer logits with the fused histogram over the full context, decode
    top-k, the q_nope -> latent bmm, sparse MLA decode + merge and the W_UV
    bmm.  `copies` layers with their own caches and weights (> 256 MB MALL)
    are captured in one graph.  Also reports the indexer + top-k, the
    attention with both projections (the layer's fused merge + W_UV
    launch, and the same work as sparse MLA decode + merge then a separate
    W_UV projection) and the two projections alone, from graphs of their
    own.  idx_fp8 runs the layer on the 132-byte fp8
    indexer-K cache instead of fp16 rows (the reference offers both,
    glue.patch:2952-2966)."""
    m = pkg.dsa_layer
    B, H, page = 4, 64, 64
    layers, steps = [], []
    for i in range(copies):
        d = pkg.synthetic.decode_inputs(B=B, H=H, ctx=ctx, device=dev, seed=60 + i)
        ix = pkg.synthetic.indexer_decode_inputs(B=B, ctx=ctx, dup_frac=0.0, device=dev,
                                                 seed=70 + i, fp8=idx_fp8)
        if idx_fp8:
            ix["kc"] = ix.pop("kc8")
        del ix["k"]
        g = torch.Generator(device=dev)
        g.manual_seed(80 + i)
        w = m.DsaLayerWeights(
            (torch.randn(H, P, 512, generator=g, device=dev) / P ** 0.5).to(torch.float16),
            (torch.randn(H, 512, V, generator=g, device=dev) / 512 ** 0.5).to(torch.float16),
            (P + 64) ** -0.5)
        # both caches share the latent cache's block table
        layer = m.DsaLayer(w, d["kv"], ix["kc"])
        bt, seq = d["bt"], d["seq"]
        pos = (seq.long() - 1)
        # int32 slots: the indexer-K store takes int32 (sm70_mla_decode.cu:2919),
        # and the latent writer accepts them too
        slot = (bt.long().gather(1, (pos // page).view(B, 1)).view(B) * page
                + pos % page).to(torch.int32)
        steps.append(dict(
            layer=layer, bt=bt, seq=seq, slot=slot,
            q=(torch.randn(B, H, P + 64, generator=g, device=dev) / 8).to(torch.float16),
            idx_q=ix["q"], idx_w=ix["w"],
            kv_c=(torch.randn(B, 512, generator=g, device=dev) / 24).to(torch.float16),
            k_pe=(torch.randn(B, 64, generator=g, device=dev) / 24).to(torch.float16),
            idx_k=torch.randn(B, 128, generator=g, device=dev).to(torch.float16)))
        del d, ix

    def full():
        for s in steps:
            s["layer"].decode(s["q"], s["idx_q"], s["idx_w"], s["bt"], s["seq"],
                              s["kv_c"], s["k_pe"], s["idx_k"], s["slot"])

    def topk_only():
        for s in steps:
            s["layer"].decode_topk(s["idx_q"], s["idx_w"], s["bt"], s["seq"])

    def attn_only():
        for s in steps:
            L = s["layer"]
            ql = m.q_latent(s["q"], L.w)
            L._attention(ql, L.last_idx, s["bt"], s["seq"])

    def attn_two_calls():
        ops = pkg._sm70_ops
        for s in steps:
            L = s["layer"]
            ql = m.q_latent(s["q"], L.w)
            o = torch.empty(B, H, 512, dtype=torch.float16, device=dev)
            lse = torch.empty(B, H, device=dev)
            ops.sm70_sparse_mla_decode(o, lse, ql, L.latent_cache, L.last_idx, s["bt"],
                                       s["seq"], L.w.scale)
            m.v_up(o, L.w)

    def proj_only():
        for s in steps:
            L = s["layer"]
            m.q_latent(s["q"], L.w)
            m.v_up(L.last_o, L.w)

    us = graph_time_per_call(torch, full, copies)
    us_topk = graph_time_per_call(torch, topk_only, copies)
    us_attn = graph_time_per_call(torch, attn_only, copies)
    us_attn2 = graph_time_per_call(torch, attn_two_calls, copies)
    us_proj = graph_time_per_call(torch, proj_only, copies)
    # weight bytes of the two projections (each read once per call)
    proj_bytes = 2 * H * 512 * (P + V)
    del steps
    return {
        "us_per_layer": round(us, 2),
        "indexer_topk_us": round(us_topk, 2),
        "attention_us": round(us_attn, 2),
        "attention_two_calls_us": round(us_attn2, 2),
        "projections_us": round(us_proj, 2),
        "projections_gbps": round(proj_bytes / (us_proj * 1e-6) / 1e9, 1),
        "workload": (f"one DSA decode layer: B=4 tokens at {ctx} ctx, 64 heads (q_nope {P}, "
                     f"v {V}), cache writes + indexer 32x128 {'fp8' if idx_fp8 else 'fp16'} K "
                     "over the full context + "
                     "top-2048 + q_latent bmm + sparse MLA (fp8_ds_mla) + W_UV bmm; "
                     f"{copies} layers per graph"),
    }


def bench_dense_decode(torch, pkg, dev):
    """Dense MLA decode (sm70_mla_decode) over an fp16 latent cache, B=4
    tokens x 64 heads, at three context lengths; enough distinct caches per
    graph that the rows stream from HBM.  Algorithmic bytes: the B x ctx
    rows of 1152 B, each read once."""
    ops = pkg._sm70_ops
    out = {}
    for ctx in (4096, 32768, 131072):
        copies = max(2, min(8, (1200 << 20) // (4 * ctx * 1152)))
        ins = [pkg.synthetic.decode_inputs(B=4, H=64, ctx=ctx, fp8=False, device=dev,
                                           seed=90 + i) for i in range(copies)]
        o = torch.empty(4, 64, 512, dtype=torch.float16, device=dev)
        lse = torch.empty(4, 64, device=dev)

        def fn():
            for d in ins:
                ops.sm70_mla_decode(o, lse, d["q"], d["kv"], d["bt"], d["seq"], d["scale"])

        us = graph_time_per_call(torch, fn, copies)
        nbytes = 4 * ctx * 1152
        gbps = nbytes / (us * 1e-6) / 1e9
        out[str(ctx)] = {"us": round(us, 2), "gbps": round(gbps, 1),
                         "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        del ins
        torch.cuda.empty_cache()
    return out


def bench_varlen_prefill(torch, pkg, dev, L=16384, H=64, dqk=192, dv=128):
    """Dense varlen MLA prefill attention (the reference's _varlen_attention):
    one causal sequence of L new tokens, H heads, qk 192 / v 128, fp16 and
    bf16 (fp16 / bf16 MFMA), and fp32 (fp32 MFMA, whose peak is 157.3
    TFLOP/s).  FLOPs count the unmasked (causal) scores only."""
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    cu = torch.tensor([0, L], dtype=torch.int32, device=dev)
    flops = H * (L * (L + 1) / 2) * (dqk + dv) * 2
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        q = torch.randn(L, H, dqk, generator=g, device=dev).to(dtype)
        k = torch.randn(L, H, dqk, generator=g, device=dev).to(dtype)
        v = torch.randn(L, H, dv, generator=g, device=dev).to(dtype)

        def fn():
            pkg.mla_prefill.varlen_attention(q, k, v, cu, cu, dqk ** -0.5, True, True,
                                             max_seqlen_q=L)

        us = graph_time_per_call(torch, fn, 1, steps=5, warmup=1)
        tf = flops / (us * 1e-6) / 1e12
        if dtype == torch.float32:
            out["fp32"] = {"ms": round(us / 1000, 3), "tflops": round(tf, 1),
                           "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
        else:
            out["fp16" if dtype == torch.float16 else "bf16"] = {
                "ms": round(us / 1000, 3), "tflops": round(tf, 1),
                "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)}
        del q, k, v
    out["workload"] = (f"one causal sequence of {L} tokens, {H} heads, qk {dqk} / v {dv}, "
                       "causal FLOPs only")
    return out


def bench_shard_merge(torch, pkg, dev, R=4096, tp=4, K=2048):
    """Key-shard indexer merge (sm70_indexer_shard_merge) of an all-gathered
    payload [tp, R, 2K] as a 64k-context prefill produces it: shard s scored
    positions [16384 s, +16384) and kept K of them.  HBM-bound, algorithmic
    bytes = the payload read once + the [R, K] int32 output."""
    ops = pkg._sm70_ops
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    copies = 2
    allfs = []
    for _ in range(copies):
        vals = torch.randn(tp, R, K, generator=g, device=dev)
        span = 65536 // tp
        pos = (torch.rand(tp, R, span, generator=g, device=dev).argsort(dim=2)[:, :, :K]
               + span * torch.arange(tp, device=dev).view(tp, 1, 1)).to(torch.int32)
        allfs.append(torch.cat([vals, pos.view(torch.float32)], dim=2).contiguous())
        del vals, pos
    out = torch.empty(R, K, dtype=torch.int32, device=dev)
    e = torch.empty(0, dtype=torch.int32, device=dev)

    def fn():
        for a in allfs:
            ops.sm70_indexer_shard_merge(out, a, e, 0, K)

    us = graph_time_per_call(torch, fn, copies)
    nbytes = tp * R * 2 * K * 4 + R * K * 4
    gbps = nbytes / (us * 1e-6) / 1e9
    del allfs
    return {"us": round(us, 2), "gbps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
            "workload": f"tp={tp}, R={R} rows, K={K}"}


def bench_c1(torch, pkg, dev, cpu_seconds=5.0, copies=16):
    """Config C1, the reference's CPU-runnable case, as one pipeline: indexer
    logits (with the top-k histogram) -> decode top-2048 -> sparse MLA decode,
    B=1, 64 heads, 4096-token context, fp16 latent and indexer-K caches
    (page 64, random block table), on the GPU (`copies` pipelines with their
    own inputs per graph) and, beside it, the oracle's fp32 PyTorch
    restatement of the same pipeline on the host cores."""
    sys.path.insert(0, ROOT)
    from oracle import dsa_oracle as O

    ops = pkg._sm70_ops
    ctx, page, H = 4096, 64, 64
    nblk = ctx // page
    g = torch.Generator()
    g.manual_seed(1)
    ins = []
    for _ in range(copies):
        ins.append(dict(
            q=(torch.randn(1, H, 576, generator=g) / 24.0).to(torch.float16),
            kv=(torch.randn(nblk, page, 576, generator=g) / 24.0).to(torch.float16),
            iq=torch.randn(1, 32, 128, generator=g).to(torch.float16),
            ik=torch.randn(nblk, page, 128, generator=g).to(torch.float16),
            w=(torch.randn(1, 32, generator=g) / 32 ** 0.5).to(torch.float16),
            bt=torch.randperm(nblk, generator=g).to(torch.int32)[None].contiguous(),
            seq=torch.tensor([ctx], dtype=torch.int32)))
    scale = 576 ** -0.5
    gins = [{k: v.to(dev) for k, v in d.items()} for d in ins]
    score = torch.empty(1, ctx, device=dev)
    hist = torch.zeros(1, 4096, dtype=torch.int32, device=dev)
    idx = torch.empty(1, 2048, dtype=torch.int32, device=dev)
    o = torch.empty(1, H, 512, dtype=torch.float16, device=dev)
    lse = torch.empty(1, H, device=dev)

    def fn():
        for d in gins:
            hist.zero_()
            ops.sm70_indexer_logits(score, d["iq"], d["ik"], d["w"], d["bt"], d["seq"], hist)
            ops.sm70_decode_topk(idx, score, d["seq"], hist, 2048)
            ops.sm70_sparse_mla_decode(o, lse, d["q"], d["kv"], idx, d["bt"], d["seq"], scale)

    us = graph_time_per_call(torch, fn, copies)
    n, t0 = 0, time.perf_counter()
    while True:
        d = ins[n % copies]
        sc, _ = O.indexer_logits(d["iq"], d["ik"], d["w"], d["bt"], d["seq"], ctx,
                                 dtype=torch.float32)
        ix = O.topk_rows(sc, d["seq"], 2048)
        O.sparse_mla(d["q"], d["kv"], ix, d["bt"], d["seq"], scale, dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= cpu_seconds or n >= 50:
            break
    cpu_us = el / n * 1e6
    return {"gpu_us": round(us, 2), "cpu_us": round(cpu_us, 1), "cpu_threads": torch.get_num_threads(),
            "cpu_pipelines": n, "gpu_over_cpu": round(cpu_us / us, 1),
            "workload": ("C1: B=1, 64 heads, ctx 4096, topk 2048, fp16 caches; indexer logits + "
                         "decode top-k + sparse MLA decode per pipeline; CPU = the oracle's fp32 "
                         "restatement of the same pipeline")}


def bench_prefill_topk(torch, pkg, dev, T=65536, sub=1024, K=2048):
    """Row a4 at C4: persistent_topk over every sub-chunk of a 64k-token
    causal prefill (row t keeps the top-2048 of its t + 1 scores), as the
    layer harness calls it: each sub-chunk's scores are a contiguous
    [1024, width] fp32 buffer (width = the chunk's reach rounded up to 64
    keys), carved from two alternating 256 MB random buffers.  Algorithmic
    bytes: the causal scores read once plus the int32 indices written."""
    ops = pkg._sm70_ops
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    bufs = [torch.randn(sub, T, generator=g, device=dev) for _ in range(2)]
    out = torch.empty(sub, K, dtype=torch.int32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    chunks = []
    for i, lo in enumerate(range(0, T, sub)):
        lens = torch.arange(lo + 1, lo + sub + 1, dtype=torch.int32, device=dev).view(sub, 1)
        width = min(T, (lo + sub + 63) // 64 * 64)
        sc = bufs[i & 1].view(-1)[:sub * width].view(sub, width)
        chunks.append((sc, lens, width))

    def fn():
        for sc, lens, width in chunks:
            ops.persistent_topk(sc, lens, out, ws, K, width)

    ms = graph_time_per_call(torch, fn, 1, steps=3, warmup=1) / 1000.0
    nbytes = 4 * T * (T + 1) / 2 + 4 * T * K
    gbps = nbytes / (ms * 1e-3) / 1e9
    del bufs
    return {"ms": round(ms, 3), "gbps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4),
            "workload": f"64k causal rows in {sub}-row sub-chunks, top-{K} per row"}


def bench_dsa_layer_prefill(torch, pkg, dev, T=65536, P=128, V=128, sub=1024, steps=2):
    """One DSA prefill layer step at the C4 shape through the layer harness:
    one causal request of 64k tokens, 64 heads, top-2048.  Per 1024-row
    sub-chunk the packed indexer logits and persistent_topk, then the
    q_nope -> latent projection, sparse MLA prefill on the fp8_ds_mla cache
    and the W_UV projection.  The step has host-side control flow (the
    sub-chunk loop, the token -> request map), so it runs eagerly, timed
    with events on the current stream after one untimed call."""
    S = pkg.synthetic
    m = pkg.dsa_layer
    H, page = 64, 64
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    npg = T // page
    kv = S.latent_cache(T, True, g, dev)
    kc = torch.randn(npg, page, 128, generator=g, device=dev).to(torch.float16)
    bt = torch.randperm(npg, generator=g, device=dev).to(torch.int32)[None]
    w = m.DsaLayerWeights(
        (torch.randn(H, P, 512, generator=g, device=dev) / P ** 0.5).to(torch.float16),
        (torch.randn(H, 512, V, generator=g, device=dev) / 512 ** 0.5).to(torch.float16),
        (P + 64) ** -0.5)
    layer = m.DsaLayer(w, kv, kc)
    q = (torch.randn(T, H, P + 64, generator=g, device=dev) / 8).to(torch.float16)
    iq = torch.randn(T, 32, 128, generator=g, device=dev).to(torch.float16)
    iw = (torch.randn(T, 32, generator=g, device=dev) / 32 ** 0.5).to(torch.float16)
    causal = torch.arange(1, T + 1, dtype=torch.int32, device=dev)
    reach = [min(T, lo + sub) for lo in range(0, T, sub)]

    def run():
        return layer.prefill(q, iq, iw, [0, T], bt, causal, sub_rows=sub, reach=reach)

    run()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        run()
    e1.record(st)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = (8192.0 * T * (T + 1) / 2 + sparse_prefill_flops(T)[0]
             + 2.0 * T * H * 512 * (P + V))
    del layer, kv, kc, q, iq, iw
    return {"ms": round(ms, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "workload": f"one DSA prefill layer: one causal request of {T} tokens, {H} heads "
                        f"(q_nope {P}, v {V}), indexer in {sub}-row sub-chunks + persistent_topk "
                        "+ q_latent + sparse MLA prefill (fp8_ds_mla) + W_UV; eager, host "
                        "control flow included"}


def cpu_baseline(torch, d, idxs, qs, budget_s):
    """The oracle's PyTorch restatement (fp32) of the same decode layers on
    the host cores: gather -> dequant -> QK -> softmax -> PV."""
    sys.path.insert(0, ROOT)
    from oracle import dsa_oracle as O

    kv = d["kv"].cpu()
    bt = d["bt"].cpu()
    seq = d["seq"].cpu()
    n, t0 = 0, time.perf_counter()
    while True:
        O.sparse_mla(qs[n % len(qs)].cpu(), kv, idxs[n % len(idxs)].cpu(), bt, seq,
                     d["scale"], dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return el / n * 1e6, n


def cpu_threads():
    """Host threads for the CPU legs: the cores this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when the box sets it (its
    CPU share for one GPU)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    n = min(aff, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else aff
    return n, aff


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, budget_s, max_n):
    """Runs fn() until budget_s seconds or max_n calls; returns (s/call, n)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn(n)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= max_n:
            return el / n, n


def cpu_baselines(torch, pkg, budget_s, gpu):
    """The oracle's fp32 PyTorch restatement of configs C2, C4 and C5 on the
    host cores, each on a bounded sample of the GPU workload (stated per
    record), beside the GPU figure of the same config (`gpu`: the bench's
    own records, None when that record was not run)."""
    sys.path.insert(0, ROOT)
    from oracle import dsa_oracle as O

    S = pkg.synthetic
    out = {}
    # C2: indexer logits (+ histogram) and exact top-2048, B=4 x 64k keys
    d = S.indexer_decode_inputs(device="cpu", seed=20)
    B, max_kv = 4, d["max_kv"]

    def c2(_):
        sc, _h = O.indexer_logits(d["q"], d["kc"], d["w"], d["bt"], d["seq"], max_kv,
                                  dtype=torch.float32, with_hist=True)
        O.topk_rows(sc, d["seq"], 2048)

    t, n = _timed(c2, budget_s, 20)
    out["c2_logits_topk"] = {"value": round(t * 1e6, 1), "unit": "us/step", "kind": "port",
                             "sample": f"{n} whole C2 steps (B=4 x 65536 keys, top-2048)",
                             "gpu_value": gpu.get("c2")}
    del d
    # C4 indexer: rows of the last 1024-row sub-chunk of the 64k causal prefill
    # (full reach), extrapolated to the causal triangle by FLOP ratio
    T, page, R = 65536, 64, 1024
    g = torch.Generator().manual_seed(4)
    npg = T // page
    kc = torch.randn(npg, page, 128, generator=g).to(torch.float16)
    bt = torch.randperm(npg, generator=g).to(torch.int32)[None]
    q = torch.randn(R, 32, 128, generator=g).to(torch.float16)
    w = (torch.randn(R, 32, generator=g) / 32 ** 0.5).to(torch.float16)
    rows_per_call = 8
    done = [0, 0.0]

    def c4i(i):
        lo = (i * rows_per_call) % R
        seq = torch.arange(T - R + lo + 1, T - R + lo + rows_per_call + 1, dtype=torch.int32)
        O.indexer_logits(q[lo:lo + rows_per_call], kc, w[lo:lo + rows_per_call],
                         bt.expand(rows_per_call, npg), seq, T, dtype=torch.float32)
        done[0] += rows_per_call
        done[1] += 8192.0 * float(seq.double().sum())

    t, n = _timed(c4i, budget_s, R // rows_per_call)
    rate = done[1] / (t * n)  # FLOP/s
    total = 8192.0 * T * (T + 1) / 2
    out["c4_indexer_prefill"] = {
        "value": round(total / rate * 1e3, 1), "unit": "ms (extrapolated)", "kind": "port",
        "tflops": round(rate / 1e12, 4),
        "sample": (f"{done[0]} rows of the last 1024-row sub-chunk (full 64k reach), "
                   "extrapolated to the 64k causal triangle by FLOP ratio"),
        "gpu_value": gpu.get("c4_indexer")}
    del kc, q, w
    # C4 sparse attention: tokens of the last 1024 of the prefill, 2048 keys each
    nrow = T
    kv = S.latent_cache(nrow, True, torch.Generator().manual_seed(6), "cpu")
    btp = torch.randperm(npg, generator=g).to(torch.int32)[None]
    qa = (torch.randn(64, 64, 576, generator=g) / 24.0).to(torch.float16)
    idx = torch.stack([torch.randperm(T - 1024 + i, generator=g)[:2048].sort().values
                       for i in range(64)]).to(torch.int32)
    seqa = torch.arange(T - 1024 + 1, T - 1024 + 65, dtype=torch.int32)
    tok = 4

    def c4s(i):
        lo = (i * tok) % 64
        O.sparse_mla(qa[lo:lo + tok], kv, idx[lo:lo + tok], btp.expand(tok, npg),
                     seqa[lo:lo + tok], 576 ** -0.5, dtype=torch.float32)

    t, n = _timed(c4s, budget_s, 16)
    flops_tok = 2048 * 64 * (576 + 512) * 2
    rate = flops_tok * tok / t
    sp_flops, _ = sparse_prefill_flops()
    out["c4_sparse_prefill_fp8"] = {
        "value": round(sp_flops / rate * 1e3, 1), "unit": "ms (extrapolated)", "kind": "port",
        "tflops": round(rate / 1e12, 4),
        "sample": (f"{n * tok} tokens of the last 1024 of the 64k prefill (2048 selected keys, "
                   "64 heads, fp8_ds_mla), extrapolated by FLOP ratio to the selected-key total"),
        "gpu_value": gpu.get("c4_sparse")}
    del kv, qa, idx
    # C5a: fp8 GEMV at M=1 on each shape (dequantise in fp32, then x @ W^T)
    gemv = {}
    for (N, K) in ((24576, 6144), (6144, 24576), (2112, 6144)):
        wq = torch.randint(0, 0x7E, (N, K), generator=g, dtype=torch.int32).to(torch.uint8)
        sc = torch.rand((N + 127) // 128, (K + 127) // 128, generator=g) * 1e-3
        x = torch.randn(1, K, generator=g).to(torch.float16)

        def c5(_):
            deq = O.e4m3_decode(wq) * O.expand_block_scale(sc, N, K)
            (x.float() @ deq.T).to(torch.float16)

        t, n = _timed(c5, budget_s / 3, 5)
        gemv[f"{N}x{K}_M1"] = {"us": round(t * 1e6, 1), "calls": n}
        del wq
    out["c5a_fp8_gemv"] = {"value": gemv, "unit": "us/call", "kind": "port",
                           "sample": "1-5 calls per shape at M=1", "gpu_value": gpu.get("c5a")}
    # C5b: indexer-K scatter of 64k tokens, fp8 rows
    n_tok = 65536
    k = torch.randn(n_tok, 128, generator=g).to(torch.float16)
    slot = torch.randperm(n_tok, generator=g).to(torch.int32)
    cache = torch.zeros(n_tok // 64, 64, 132, dtype=torch.uint8)
    t, n = _timed(lambda _: O.indexer_k_store(cache, k, slot), budget_s / 2, 5)
    out["c5b_k_store_fp8"] = {"value": round(t * 1e6, 1), "unit": "us/call", "kind": "port",
                              "sample": f"{n} scatters of 65536 tokens into fp8 132-byte rows",
                              "gpu_value": gpu.get("c5b")}
    return out


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the hot path on one GPU only; multi-GPU runs are "
              "not part of this build (--gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch

    sys.path.insert(0, ROOT)
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device: {torch.cuda.get_device_name(dev)}")
    if args.calib_copy_mib:
        n = args.calib_copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {n} bytes read, {n} bytes written")
        del src, dst

    # ---- headline: C3 decode at 180k ----
    L = args.layers
    torch.cuda.synchronize()
    ms, d, idxs, qs = bench_decode(torch, pkg, dev, 184320, L, args.steps, args.warmup,
                                   per_kernel=not args.no_kernel_times)
    ms_per_step = ms / args.steps
    us_layer = ms_per_step * 1000.0 / L
    gbps = DECODE_BYTES / (us_layer * 1e-6) / 1e9
    tflops = DECODE_FLOPS / (us_layer * 1e-6) / 1e12
    log(f"decode C3: {us_layer:.2f} us/layer, {gbps:.0f} GB/s, {tflops:.1f} TFLOPS")

    line = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": ("C3 sparse MLA decode: B=4 tokens, 64 heads, qk 576 / v 512, "
                         "topk 2048, ctx 184320, fp8_ds_mla paged cache (page 64, "
                         "11520 pages), one step = %d layers replayed from a HIP graph, "
                         "layer l reading cache copy l %% %d (distinct %d MB caches, so the "
                         "gathered rows come from HBM, not the 256 MB MALL)"
                         % (L, d["n_caches"], d["kv"].numel() >> 20)),
            "batch": 4, "heads": 64, "topk": 2048, "ctx": 184320, "kv": "fp8_ds_mla",
            "layers_per_step": L,
            "distinct_caches": d["n_caches"],
            # the library's split count at this shape (BASELINE C3 names 8; results
            # are split-invariant, tested); each split is one 128-key workgroup
            "splits": decode_splits(pkg, 4),
        },
        "hbm_gbps": round(gbps, 1),
        "tflops": round(tflops, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, profiles/sparse_mla_decode_c3_pmc.md",
            "kernel": "sparse_mla_decode_dma_kernel + sparse_mla_merge_kernel",
            "bytes_per_launch": DECODE_BYTES,
        },
    }
    # the dominant kernel alone: the layer's algorithmic bytes over the split
    # decode kernel's own device time (torch.profiler timestamps of two more
    # replays of the timed graph), beside the whole-layer figure above
    kt = d.get("kernel_us", {})
    if "sparse_mla_decode_dma_kernel" in kt:
        us_k, n_k = kt["sparse_mla_decode_dma_kernel"]
        gb_k = DECODE_BYTES / (us_k * 1e-6) / 1e9
        line["roofline"]["dominant_kernel"] = {
            "name": "sparse_mla_decode_dma_kernel",
            "avg_us": round(us_k, 3),
            "launches": n_k,
            "achieved": round(gb_k, 1),
            "frac": round(gb_k / HBM_PEAK_GBPS, 4),
            "source": "torch.profiler device timestamps, 2 replays of the timed graph",
        }
        if "sparse_mla_merge_kernel" in kt:
            line["roofline"]["merge_kernel_avg_us"] = round(kt["sparse_mla_merge_kernel"][0], 3)
        log(f"decode kernels: {kt}")

    extras = set(EXTRAS if args.extra == "all" else args.extra.split(","))
    if args.no_extra:
        extras = set()
    if "sweep" in extras:
        sweep = {}
        for ctx in (4096, 16384, 65536):
            ms_c, *_ = bench_decode(torch, pkg, dev, ctx, L, max(args.steps // 2, 3),
                                    2, seed=7)
            sweep[str(ctx)] = round(ms_c / max(args.steps // 2, 3) * 1000.0 / L, 3)
            torch.cuda.empty_cache()
        sweep["184320"] = line["value"]
        line["ctx_sweep_us_per_layer"] = sweep
        log(f"ctx sweep: {sweep}")
    if "batch_sweep" in extras:
        bs = {}
        for B, layers in ((4, 78), (16, 40), (64, 12), (128, 6), (256, 4)):
            r = bench_decode_batch(torch, pkg, dev, B, layers, max(args.steps // 2, 4), 2)
            r["splits"] = decode_splits(pkg, B)
            bs[str(B)] = r
            torch.cuda.empty_cache()
            log(f"decode batch {B}: {r}")
        line["decode_batch_sweep"] = bs
    if "indexer_prefill" in extras:
        pms, pflops = bench_indexer_prefill(torch, pkg, dev)
        ptf = pflops / (pms * 1e-3) / 1e12
        line["indexer_prefill"] = {
            "tflops": round(ptf, 2),
            "ms": round(pms, 3),
            "flops": pflops,
            "frac_fp16_peak": round(ptf / FP16_PEAK_TFLOPS, 4),
            "workload": ("65536-token causal prefill, indexer 32 heads x 128, fp16 "
                         "K cache, 128-row sub-chunks, causal-triangle FLOPs only"),
            "reference_v100_published_tflops": V100_PUBLISHED["indexer_prefill_tflops"],
        }
        log(f"indexer prefill: {ptf:.1f} TFLOPS ({pms:.2f} ms)")
        torch.cuda.empty_cache()
        # the same prefill in 1024-row sub-chunks: the caller's 128-row split
        # bounds the fp32 score buffer for a 32 GB card; at 1024 rows the
        # buffer is 256 MB and every launch fills the chip
        pms, pflops = bench_indexer_prefill(torch, pkg, dev, sub=1024)
        ptf = pflops / (pms * 1e-3) / 1e12
        line["indexer_prefill_sub1024"] = {
            "tflops": round(ptf, 2),
            "ms": round(pms, 3),
            "frac_fp16_peak": round(ptf / FP16_PEAK_TFLOPS, 4),
            "workload": "as indexer_prefill, 1024-row sub-chunks (256 MB score buffer)",
        }
        log(f"indexer prefill, 1024-row sub-chunks: {ptf:.1f} TFLOPS ({pms:.2f} ms)")
        torch.cuda.empty_cache()
    if "sparse_prefill" in extras:
        for fp8 in (True, False):
            key = "sparse_prefill_fp8" if fp8 else "sparse_prefill_fp16"
            line[key] = bench_sparse_prefill(torch, pkg, dev, fp8=fp8)
            if fp8:
                line[key]["reference_v100_published_tflops"] = V100_PUBLISHED["sparse_prefill_tflops"]
            log(f"sparse prefill ({key}): {line[key]['tflops']} TFLOPS ({line[key]['ms']} ms)")
            torch.cuda.empty_cache()
    if "indexer_decode" in extras:
        line["indexer_decode_topk"] = bench_indexer_decode(torch, pkg, dev)
        log(f"indexer decode: {line['indexer_decode_topk']}")
        torch.cuda.empty_cache()
    if "gemv" in extras:
        line["fp8_gemv"] = bench_gemv(torch, pkg, dev)
        line["fp8_gemv"]["reference_v100_published_m1_gbps"] = V100_PUBLISHED["fp8_gemv_m1_gbps"]
        log(f"fp8 gemv: {line['fp8_gemv']}")
    if "k_store" in extras:
        line["k_store"] = bench_k_store(torch, pkg, dev)
        log(f"k store: {line['k_store']}")
        torch.cuda.empty_cache()
    if "dense_decode" in extras:
        line["dense_mla_decode"] = bench_dense_decode(torch, pkg, dev)
        log(f"dense mla decode: {line['dense_mla_decode']}")
    if "varlen_prefill" in extras:
        line["dense_varlen_prefill"] = bench_varlen_prefill(torch, pkg, dev)
        log(f"dense varlen prefill: {line['dense_varlen_prefill']}")
        torch.cuda.empty_cache()
    if "shard_merge" in extras:
        line["indexer_shard_merge"] = bench_shard_merge(torch, pkg, dev)
        log(f"indexer shard merge: {line['indexer_shard_merge']}")
        torch.cuda.empty_cache()
    if "prefill_topk" in extras:
        line["prefill_topk"] = bench_prefill_topk(torch, pkg, dev)
        log(f"prefill top-k: {line['prefill_topk']}")
        torch.cuda.empty_cache()
    if "dsa_layer_prefill" in extras:
        line["dsa_layer_prefill"] = bench_dsa_layer_prefill(torch, pkg, dev)
        log(f"dsa layer prefill: {line['dsa_layer_prefill']}")
        torch.cuda.empty_cache()
    if "c1" in extras:
        line["c1_pipeline"] = bench_c1(torch, pkg, dev)
        log(f"C1 pipeline: {line['c1_pipeline']}")
    if "dsa_layer" in extras:
        line["dsa_layer_decode"] = bench_dsa_layer(torch, pkg, dev)
        log(f"dsa layer decode: {line['dsa_layer_decode']}")
        line["dsa_layer_decode_fp8_index_k"] = bench_dsa_layer(torch, pkg, dev, idx_fp8=True)
        log(f"dsa layer decode, fp8 indexer K: {line['dsa_layer_decode_fp8_index_k']}")
        torch.cuda.empty_cache()

    if not args.no_cpu:
        cores, aff = cpu_threads()
        torch.set_num_threads(cores)
        model = cpu_model()
        cpu_us, n = cpu_baseline(torch, d, idxs, qs, args.cpu_seconds)
        line["cpu_baseline"] = {
            "value": round(cpu_us, 1),
            "unit": "us/layer",
            "cores": cores,
            "kind": "port",
            "sample": (f"{n} C3 decode layers (B=4, 64 heads, topk 2048, fp8_ds_mla) "
                       "through the oracle's fp32 PyTorch restatement on the host CPU"),
            "cpu_model": model,
            "affinity_cores": aff,
        }
        log(f"cpu baseline: {cpu_us:.0f} us/layer on {cores} threads ({n} layers), {model}")
        if not args.no_extra:
            gpu = {
                "c2": line.get("indexer_decode_topk", {}).get("logits_plus_topk_us"),
                "c4_indexer": line.get("indexer_prefill", {}).get("ms"),
                "c4_sparse": line.get("sparse_prefill_fp8", {}).get("ms"),
                "c5a": {k: v["us"] for k, v in line.get("fp8_gemv", {}).items()
                        if isinstance(v, dict) and k.endswith("_M1")} or None,
                "c5b": line.get("k_store", {}).get("fp8", {}).get("us"),
            }
            line["cpu_baselines"] = cpu_baselines(torch, pkg, args.cpu_seconds / 2, gpu)
            for k2, v2 in line["cpu_baselines"].items():
                v2["cores"] = cores
            log(f"cpu baselines: {line['cpu_baselines']}")

    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
