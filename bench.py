"""Benchmark of the MI355X attention path at the Llama-3.2-3B shape.

One step = one decode token through all 28 attention layers at batch 1:
per layer, RoPE of q/k from the resident table, split-K f32 decode against
that layer's 8192-token HBM cache, and the in-place append of the new K/V.
Each layer has its own cache (1.9 GB in total, far above the 256 MB
Infinity Cache), inputs are resident in HBM before timing, and the step is
replayed from a HIP graph so host launch cost is not measured.

Printed JSON (one line): value = whole-step decode HBM GB/s (algorithmic
bytes: each KV head's visible K/V rows once, q/out, append); extra fields give
µs/layer, the batch-16 decode, the 4096-token causal prefill in TFLOP/s,
`roofline` of the dominant decode kernel (event-timed back-to-back launches),
and `cpu_baseline` (the oracle on this host's cores over a bounded sample).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--decode-only] [--skip-workloads]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, spec
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, spec

LAYERS, HQ, HKV, D, CTX, THETA = 28, 24, 8, 128, 8192, 500000.0
PREFILL_S = 4096
BATCH = 16


def decode_bytes(key_len: int, hq=HQ, hkv=HKV, d=D) -> int:
    """Algorithmic HBM bytes of one decode layer for one sequence."""
    return key_len * hkv * d * 4 * 2 + hq * d * 4 * 2 + 2 * hkv * d * 4


def prefill_flops(s: int, hq=HQ, d=D) -> float:
    return 4.0 * d * hq * s * (s + 1) / 2


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_b1_hbm_traffic.md"


# Plan fields a traffic profile records for the launch it measured.
TRAFFIC_PLAN_FIELDS = ("heads_per_block", "head_blocks", "keys_per_split", "splits", "token_split", "workgroups")


def decode_plan() -> dict:
    """The launch geometry of the batch-1 decode at 8192 cached keys, as the
    library plans it (spissa_plan_attention, host arithmetic only)."""
    from spissa_amd.device import plan_attention
    from spissa_amd.rotary import KvAttentionConfig

    plan = plan_attention(KvAttentionConfig(1, HQ, HKV, D, True), [CTX])
    return {k: plan[k] for k in TRAFFIC_PLAN_FIELDS}


def measured_traffic(plan=None) -> dict:
    """HBM bytes per decode launch from the committed calibrated counter
    summary, with the plan it was measured on. The bytes are withheld (None)
    when that plan differs from the launch the library plans now: the counts
    would belong to kernels that no longer run."""
    out = {"bytes": None, "profile_plan": None, "stale": None}
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return out
    nbytes, recorded = None, {}
    for line in text.splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            nbytes = int(line.split(":", 1)[1])
        elif line.startswith("plan:"):
            for item in line.split(":", 1)[1].split():
                k, _, v = item.partition("=")
                recorded[k] = int(v)
    out["profile_plan"] = recorded or None
    if plan is not None:
        out["stale"] = recorded != plan
    out["bytes"] = nbytes if (plan is None or not out["stale"]) else None
    return out


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def derived_peaks() -> dict:
    """Peaks re-derived from the device's own attributes (HIP runtime): dense
    bf16 MFMA = CUs x 4 SIMDs x 1024 flop/clk (one 32x32x16 MFMA per 32
    clocks) x peak engine clock; HBM = memory clock x bus width x 4 (HBM3E
    moves 4 bits per pin per reported memory clock: 8 Gb/s at 2000 MHz).
    Reported next to the spec peaks the roofline uses."""
    import ctypes

    try:
        hip = ctypes.CDLL("libamdhip64.so")
    except OSError:
        return {}

    def attr(code: int) -> int:
        v = ctypes.c_int(0)
        return v.value if hip.hipDeviceGetAttribute(ctypes.byref(v), code, 0) == 0 else 0

    # hipDeviceAttribute_t values of the ROCm 7 headers
    clock_khz, mem_khz, bus_bits, cus = attr(5), attr(60), attr(59), attr(63)
    out = {"sclk_max_MHz": clock_khz / 1e3, "mclk_MHz": mem_khz / 1e3, "mem_bus_bits": bus_bits}
    if cus and clock_khz:
        out["derived_bf16_dense_TFLOPs"] = round(cus * 4 * 1024 * clock_khz * 1e3 / 1e12, 1)
    if mem_khz and bus_bits:
        out["derived_hbm_GBps"] = round(mem_khz * 1e3 * 4 * bus_bits / 8 / 1e9, 1)
    return out


def read_ceiling(sess, stream, dev) -> dict:
    """The library's streaming-read kernel (spissa_hbm_read_probe_device: every
    byte once, 16-byte non-temporal loads) at the decode working-set sizes:
    one layer's K/V (67,149,824 bytes at 8192 keys) over 28 distinct buffers
    back to back in a graph, as the decode step reads its 28 layers, and a
    1 GiB read. Event-timed on the session stream."""
    import torch

    per = decode_bytes(CTX + 1) // 16 * 16
    big = torch.ones(LAYERS * per // 4, dtype=torch.float32, device=dev)
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    views = [big[l * per // 4:(l + 1) * per // 4] for l in range(LAYERS)]
    gib = big[:(1 << 30) // 4]
    out = {}

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for v in views:
            sess.hbm_read_probe(v, sink)
    ms = timed(g.replay, 20) / LAYERS
    out["layer_67MB"] = {"bytes": per, "us": round(ms * 1e3, 3), "GBps": round(per / (ms * 1e-3) / 1e9, 1)}
    ms = timed(lambda: sess.hbm_read_probe(gib, sink), 20)
    out["read_1GiB"] = {"bytes": 1 << 30, "us": round(ms * 1e3, 2), "GBps": round((1 << 30) / (ms * 1e-3) / 1e9, 1)}
    del g, big, views, gib
    sess.sync()
    return out


def mfma_ceiling(sess, stream, dev) -> dict:
    """The library's dense-MFMA kernel (spissa_mfma_rate_probe_device: eight
    waves per CU issuing independent v_mfma_f32_32x32x16_bf16 from registers,
    no memory traffic), about 1 ms per launch; event-timed over 10 launches on
    the session stream after one warm-up. The rate it sustains, with the
    chip's clock and power limits, is the achievable bound of the prefill
    kernels beside the 2.5 PFLOP/s spec."""
    import torch

    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    rounds = 4096
    flop = sess.mfma_rate_probe(rounds, sink)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(10):
        sess.mfma_rate_probe(rounds, sink)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / 10
    tf = flop / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 2), "flop": flop, "TFLOPs": round(tf, 1), "frac_of_spec": round(tf / BF16_PEAK_TFLOPS, 4)}


def gpu_bench(args) -> dict:
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    torch.cuda.init()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    sess = Session(0, stream=stream)
    res = {}
    props = torch.cuda.get_device_properties(0)
    res["device"] = {"name": props.name, "cus": props.multi_processor_count,
                     "gcn_arch": getattr(props, "gcnArchName", "")}
    res["device"].update(derived_peaks())

    with torch.cuda.stream(stream):
        res["hbm_read_ceiling"] = read_ceiling(sess, stream, dev)
        res["mfma_ceiling"] = mfma_ceiling(sess, stream, dev)

        # ---- decode, batch 1 ----
        log("filling 28 layer caches (8192 tokens each)")
        gen = torch.Generator(device=dev)
        caches, qs, ks, vs, outs = [], [], [], [], []
        w = HKV * D
        for l in range(LAYERS):
            gen.manual_seed(1000 + l)
            c = sess.kv_cache(HKV, D, CTX + 1)
            kk = torch.randn(CTX * w, generator=gen, device=dev)
            vv = torch.randn(CTX * w, generator=gen, device=dev)
            sess.append(c, kk, vv, CTX)
            caches.append(c)
            qs.append(torch.randn(HQ * D, generator=gen, device=dev))
            ks.append(torch.randn(w, generator=gen, device=dev))
            vs.append(torch.randn(w, generator=gen, device=dev))
            outs.append(torch.empty(HQ * D, device=dev))
        sess.sync()
        table = sess.rope_table(_ffi.ROPE_LLAMA, D, THETA, max_positions=CTX + 64)
        cfg1 = KvAttentionConfig(1, HQ, HKV, D, True)

        def decode_step():
            # rope(q, k) -> attention -> append(k, v) per layer, fused in two launches
            for l in range(LAYERS):
                sess.decode_step(table, qs[l], ks[l], vs[l], [caches[l]], cfg1, outs[l])

        def reset_lengths():
            for c in caches:
                c.truncate(CTX)

        def attn_only():
            for l in range(LAYERS):
                sess.attention(qs[l], ks[l], vs[l], caches[l], cfg1, outs[l])

        decode_step()  # sizes the workspace before capture
        sess.sync()
        reset_lengths()
        g_step = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_step, stream=stream):
            decode_step()
        reset_lengths()
        g_attn = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_attn, stream=stream):
            attn_only()

        def time_graph(g, reps, warm):
            for _ in range(warm):
                g.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            sess.sync()
            return a.elapsed_time(b) / reps

        log("timing decode step")
        ms_step = time_graph(g_step, args.steps, args.warmup)
        ms_attn = time_graph(g_attn, args.steps, args.warmup)
        per_layer_bytes = decode_bytes(CTX + 1)
        res["decode_b1"] = {
            "ms_per_step": ms_step,
            "us_per_layer": ms_step * 1e3 / LAYERS,
            "GBps": LAYERS * per_layer_bytes / (ms_step * 1e-3) / 1e9,
            "tokens_per_s": 1e3 / ms_step,
            "attn_kernel_us": ms_attn * 1e3 / LAYERS,
            "attn_kernel_GBps": LAYERS * per_layer_bytes / (ms_attn * 1e-3) / 1e9,
            "bytes_per_layer": per_layer_bytes,
        }
        del g_step, g_attn

        # ---- the whole attention sublayer at decode, batch 1 ----
        if not args.decode_only:
            log("timing the decode attention sublayer")
            res["sublayer_b1"] = sublayer_bench(sess, stream, dev, gen, caches, table, reset_lengths,
                                                time_graph, args)

        if args.copy_probe:
            # A plain copy of known size: 256 MiB read + 256 MiB written per launch.
            src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst

        # ---- decode, batch 16 ----
        if not args.decode_only:
            log("filling batch-16 caches")
            bcaches = []
            for l in range(LAYERS):
                row = []
                for b in range(BATCH):
                    gen.manual_seed(50000 + l * BATCH + b)
                    c = sess.kv_cache(HKV, D, CTX + 1)
                    sess.append(c, torch.randn(CTX * w, generator=gen, device=dev),
                                torch.randn(CTX * w, generator=gen, device=dev), CTX)
                    row.append(c)
                bcaches.append(row)
            sess.sync()
            bq = [torch.randn(BATCH * HQ * D, generator=gen, device=dev) for _ in range(LAYERS)]
            bk = [torch.randn(BATCH * w, generator=gen, device=dev) for _ in range(LAYERS)]
            bv = [torch.randn(BATCH * w, generator=gen, device=dev) for _ in range(LAYERS)]
            bo = [torch.empty(BATCH * HQ * D, device=dev) for _ in range(LAYERS)]

            def batch_step():
                for l in range(LAYERS):
                    sess.decode_step(table, bq[l], bk[l], bv[l], bcaches[l], cfg1, bo[l])

            def reset_batch():
                for row in bcaches:
                    for c in row:
                        c.truncate(CTX)

            batch_step()
            sess.sync()
            reset_batch()
            g_b = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g_b, stream=stream):
                batch_step()
            reset_batch()
            ms_b = time_graph(g_b, max(3, args.steps // 2), 2)
            res["decode_b16"] = {
                "ms_per_step": ms_b,
                "us_per_layer": ms_b * 1e3 / LAYERS,
                "GBps": LAYERS * BATCH * decode_bytes(CTX + 1) / (ms_b * 1e-3) / 1e9,
                "tokens_per_s": BATCH * 1e3 / ms_b,
            }
            del g_b, bcaches, bq, bk, bv, bo
            torch.cuda.empty_cache()

        # ---- causal prefill, 4096 tokens, no cache ----
        if not args.decode_only:
            res.update(prefill_bench(sess, stream, gen, dev, args, time_graph))

        # ---- the projections either side (q/k/v fused, bf16 weights) ----
        if not args.decode_only:
            log("timing projections")
            res["projections"] = projection_bench(sess, stream, gen, dev, args, time_graph)
            log("timing the LM head")
            res["lm_head"] = lm_head_bench(sess, stream, gen, dev, args, time_graph)
            log("timing the other BASELINE configs")
            res["configs"] = configs_bench(sess, stream, gen, dev, args, time_graph)
            if not args.skip_workloads:
                log("timing the Gemma workloads")
                res["workloads"] = workloads_bench(sess, stream, gen, dev, args, time_graph)
    return res


def sublayer_bench(sess, stream, dev, gen, caches, table, reset_lengths, time_graph, args) -> dict:
    """One Llama-3.2-3B attention sublayer per layer at decode batch 1, over
    the 8192-token caches: input RMSNorm, q/k/v projections (bf16 weights),
    RoPE + attention + append (the fused decode step), o projection."""
    import numpy as np
    import torch

    from spissa_amd.device import AttentionLayer
    from spissa_amd.linear import DTYPE_BF16

    hid = HQ * D
    rng = np.random.default_rng(12)

    def bits(n):
        return ((rng.standard_normal(n).astype(np.float32) * 0.02).view(np.uint32) >> 16).astype(np.uint16)

    hq, hkv, ho = bits(hid * hid), bits(HKV * D * hid), bits(hid * hid)
    layers = []
    for l in range(LAYERS):
        wq = sess.linear_weight(hq, DTYPE_BF16, hid, hid)
        wk = sess.linear_weight(hkv, DTYPE_BF16, HKV * D, hid)
        wv = sess.linear_weight(hkv, DTYPE_BF16, HKV * D, hid)
        wo = sess.linear_weight(ho, DTYPE_BF16, hid, hid)
        with torch.cuda.stream(stream):
            norm = 1.0 + 0.1 * torch.randn(hid, generator=gen, device=dev)
        layers.append(AttentionLayer(hid, HQ, HKV, D, wq, wk, wv, wo, input_norm=norm, eps=1e-5, rope=table))
    with torch.cuda.stream(stream):
        xs = [torch.randn(hid, generator=gen, device=dev) for _ in range(LAYERS)]
        ys = [torch.empty(hid, device=dev) for _ in range(LAYERS)]

    def step():
        for l in range(LAYERS):
            sess.attention_sublayer(layers[l], xs[l], 1, caches[l], ys[l])

    reset_lengths()
    step()  # sizes the workspace before capture
    sess.sync()
    reset_lengths()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    reset_lengths()
    ms = time_graph(g, args.steps, args.warmup)
    wbytes = 2 * (2 * hid * hid + 2 * HKV * D * hid)
    per_layer = wbytes + decode_bytes(CTX + 1)
    del g, layers
    return {"us_per_layer": ms * 1e3 / LAYERS, "bytes_per_layer": per_layer,
            "GBps": LAYERS * per_layer / (ms * 1e-3) / 1e9, "tokens_per_s": 1e3 / ms}


def projection_bench(sess, stream, gen, dev, args, time_graph) -> dict:
    """Llama-3.2-3B fused q/k/v projection (5120 x 3072 bf16 weight, one per
    layer) at decode batch 1 and 16 and at the 4096-token prefill."""
    import numpy as np
    import torch

    from spissa_amd.linear import DTYPE_BF16

    hid, qkv = HQ * D, (HQ + 2 * HKV) * D
    host = (np.random.default_rng(11).standard_normal(qkv * hid).astype(np.float32) * 0.02)
    host = (host.view(np.uint32) >> 16).astype(np.uint16)  # bf16 bits (truncated: data only)
    weights = [sess.linear_weight(host, DTYPE_BF16, qkv, hid) for _ in range(LAYERS)]
    out = {}
    for batch, layers in ((1, LAYERS), (16, LAYERS), (PREFILL_S, 4)):
        with torch.cuda.stream(stream):
            x = torch.randn(batch * hid, generator=gen, device=dev)
            y = torch.empty(batch * qkv, device=dev)

        def step():
            for l in range(layers):
                sess.linear(weights[l], x, None, batch, y)

        step()
        sess.sync()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step()
        ms = time_graph(g, max(3, args.steps // 2), 2)
        us = ms * 1e3 / layers
        wbytes = qkv * hid * 2
        rec = {"us_per_layer": round(us, 3), "weight_GBps": round(wbytes / (us * 1e-6) / 1e9, 1),
               "TFLOPs": round(2.0 * batch * qkv * hid / (us * 1e-6) / 1e12, 2)}
        if batch == 1:
            rec["hbm_frac"] = round(rec["weight_GBps"] / HBM_PEAK_GBS, 4)
        if batch == PREFILL_S:
            # the split activations double the MFMA work
            rec["mfma_TFLOPs"] = round(2 * rec["TFLOPs"], 2)
            rec["mfma_frac"] = round(2 * rec["TFLOPs"] / BF16_PEAK_TFLOPS, 4)
        out[f"qkv_b{batch}"] = rec
        del g, x, y
    del weights
    torch.cuda.empty_cache()
    return out


# Tied LM heads (vocab, hidden) timed by lm_head_bench.
LM_HEADS = {"llama32_3b": (128256, 3072), "gemma3_1b": (262144, 1152)}


def lm_head_bench(sess, stream, gen, dev, args, time_graph) -> dict:
    """The greedy decode tail: logits = table x hidden over the bf16 tied
    embedding, then the argmax token, per generated token. Two copies of each
    table alternate so that no replay finds the previous one in the 256 MB
    last-level cache."""
    import torch

    from spissa_amd.linear import DTYPE_BF16

    out = {}
    for name, (vocab, hid) in LM_HEADS.items():
        with torch.cuda.stream(stream):
            bits = (torch.randn(vocab * hid, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            tables = [sess.linear_weight(bits, DTYPE_BF16, vocab, hid) for _ in range(2)]
        del bits
        with torch.cuda.stream(stream):
            x = torch.randn(hid, generator=gen, device=dev)
            logits = torch.empty(vocab, device=dev)
            tok = torch.zeros(1, dtype=torch.int32, device=dev)
        reps = 8
        rec = {}
        for part in ("token", "logits", "argmax"):
            def step():
                for r in range(reps):
                    if part == "argmax":
                        sess.argmax(logits, vocab, tok)
                    else:
                        sess.lm_head(tables[r % 2], x, logits, tok if part == "token" else None)

            step()
            sess.sync()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
            rec[f"{part}_us"] = round(time_graph(g, max(3, args.steps // 2), 2) * 1e3 / reps, 3)
            del g
        tbytes = vocab * hid * 2
        # table + hidden read, logits written by the GEMV and read by the argmax
        step_bytes = tbytes + hid * 4 + 2 * vocab * 4
        rec["GBps"] = round(step_bytes / (rec["token_us"] * 1e-6) / 1e9, 1)
        rec["hbm_frac"] = round(rec["GBps"] / HBM_PEAK_GBS, 4)
        rec["logits_GBps"] = round((tbytes + hid * 4 + vocab * 4) / (rec["logits_us"] * 1e-6) / 1e9, 1)
        rec["tokens_per_s"] = round(1e6 / rec["token_us"], 1)
        rec["table_bytes"] = tbytes
        out[name] = rec
        del tables, x, logits, tok
        torch.cuda.empty_cache()
    return out


# The attention layers of the other BASELINE configs, each measured over
# `layers` distinct caches (more than the 256 MB last-level cache holds, where
# the reads are large enough to matter):
# (name, index i of BASELINE.json configs[i], layers, Hq, Hkv, d, query rows S, cached rows P, window,
#  llama RoPE)
CONFIG_CASES = [
    ("llama32_1b_decode_512", 0, 16, 32, 8, 64, 1, 512, 0, True),
    ("llama32_1b_prefill_2048", 1, 16, 32, 8, 64, 2048, 0, 0, False),
    ("llama32_1b_decode_2048", 1, 16, 32, 8, 64, 1, 2048, 0, True),
    ("gemma3_1b_prefill_4096_global", 3, 4, 4, 1, 256, 4096, 0, 0, False),
    ("gemma3_1b_prefill_4096_local_w512", 3, 8, 4, 1, 256, 4096, 0, 512, False),
    ("gemma3_1b_decode_32768_global", 3, 8, 4, 1, 256, 1, 32768, 0, False),
    ("gemma3_1b_decode_32768_local_w512", 3, 8, 4, 1, 256, 1, 32768, 512, False),
    ("gemma3_4b_chunk_128_on_16384_global", 4, 5, 8, 4, 256, 128, 16384, 0, False),
    ("gemma3_4b_chunk_128_on_16384_local_w1024", 4, 8, 8, 4, 256, 128, 16384, 1024, False),
    ("gemma3_4b_decode_16512_global", 4, 5, 8, 4, 256, 1, 16512, 0, False),
    ("gemma3_4b_decode_16512_local_w1024", 4, 8, 8, 4, 256, 1, 16512, 1024, False),
    # one GPU's share of config 2 split 8 ways by KV head (one KV head and its
    # three query heads per GPU): the kernels at that real shape
    ("llama32_3b_decode_8192_tp8_share", 2, 28, 3, 1, 128, 1, 8192, 0, True),
    ("llama32_3b_prefill_4096_tp8_share", 2, 28, 3, 1, 128, 4096, 0, 0, False),
]


# Gemma 3 layer schedule (models/gemma/model.rs:46-51): global iff (layer + 1) % 6 == 0.
GEMMA_PATTERN = 6
# Decode tokens per captured graph of the Gemma-3-4B turn.
TURN_GRAPH_TOKENS = 16
GEMMA_WORKLOADS = {  # BASELINE configs 3 and 4: heads, head_dim, layers, local window
    "gemma3_1b": {"config": 3, "hq": 4, "hkv": 1, "d": 256, "layers": 26, "window": 512},
    "gemma3_4b": {"config": 4, "hq": 8, "hkv": 4, "d": 256, "layers": 34, "window": 1024},
}


def workloads_bench(sess, stream, gen, dev, args, time_graph) -> dict:
    """BASELINE configs 3 and 4 as whole workloads through every layer, in the
    reference's per-layer order (models/gemma/generate.rs:232-295): the QK-norm
    + Gemma RoPE + prescale prologue of the layer's new q and k rows, the
    attention over the cache and the new rows, the append. Prefill chunks run
    spissa_gemma_prefill_step_device (1/rms pass, append with the norm and
    RoPE folded in, attention); a decode token runs
    spissa_gemma_decode_step_device, which does all of it in two launches. Local layers use the sliding window with RoPE base
    1e4; global layers ((l + 1) % 6 == 0) see every key, RoPE base 1e6 with
    position divisor 8. Each workload is one graph per phase set; the phases
    are the reference's buckets (session.rs:14-32): rotary (the prologue),
    attention and kv_append (the fused step's append pass, where it is a
    launch of its own). The buckets are timed on the unfused sequence
    (prologue launch, then the prefill or decode step), which is also
    reported whole beside the fused steps."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.rotary import KvAttentionConfig

    out = {}

    def layer_kinds(L):
        return [(l + 1) % GEMMA_PATTERN == 0 for l in range(L)]

    def tables(d, positions, W):
        return {True: sess.rope_table(_ffi.ROPE_GEMMA, d, 1000000.0, position_divisor=8.0, max_positions=positions),
                False: sess.rope_table(_ffi.ROPE_GEMMA, d, 10000.0, max_positions=positions)}

    def captured(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        return g

    # ---- Gemma-3-1B: prefill 4096, then decode at 32768 ----
    w1 = GEMMA_WORKLOADS["gemma3_1b"]
    hq, hkv, d, L, W = w1["hq"], w1["hkv"], w1["d"], w1["layers"], w1["window"]
    kinds = layer_kinds(L)
    S = 4096
    with torch.cuda.stream(stream):
        tab = tables(d, 32768 + 64, W)
        qn = [torch.randn(d, generator=gen, device=dev) * 0.1 + 1.0 for _ in range(L)]
        kn = [torch.randn(d, generator=gen, device=dev) * 0.1 + 1.0 for _ in range(L)]
        q = [torch.randn(S * hq * d, generator=gen, device=dev) for _ in range(L)]
        k = [torch.randn(S * hkv * d, generator=gen, device=dev) for _ in range(L)]
        v = [torch.randn(S * hkv * d, generator=gen, device=dev) for _ in range(L)]
        o = [torch.empty(S * hq * d, device=dev) for _ in range(L)]
        caches = [sess.kv_cache(hkv, d, S) for _ in range(L)]
    cfgs = [KvAttentionConfig(S, hq, hkv, d, True, 0 if g else W) for g in kinds]

    def prologue():
        for l in range(L):
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], S, hq, hkv, d, qn[l], kn[l], 1e-6, 0, 1.0)

    def steps():
        for l in range(L):
            sess.prefill_step(None, q[l], k[l], v[l], caches[l], cfgs[l], o[l])

    def attention():
        for l in range(L):
            sess.attention_cached(q[l], caches[l], cfgs[l], o[l])

    def layers():
        for l in range(L):
            sess.gemma_prefill_step(tab[kinds[l]], q[l], k[l], v[l], caches[l], cfgs[l], qn[l], kn[l], 1e-6, 1.0,
                                    o[l])

    def unfused():
        for l in range(L):
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], S, hq, hkv, d, qn[l], kn[l], 1e-6, 0, 1.0)
            sess.prefill_step(None, q[l], k[l], v[l], caches[l], cfgs[l], o[l])

    def reset():
        for c in caches:
            c.truncate(0)

    steps()
    sess.sync()
    reset()
    layers()
    sess.sync()
    reset()
    g_all = captured(layers)
    reset()
    g_unf, g_pro = captured(unfused), captured(prologue)
    reset()
    g_step = captured(steps)
    g_att = captured(attention)  # the caches hold the prompt after the step's capture
    reps = max(3, args.steps // 4)
    ms = {n: time_graph(g, reps, 2) for n, g in (("all", g_all), ("unfused", g_unf), ("rotary", g_pro),
                                                  ("step", g_step), ("attention", g_att))}
    rec = {"layers": L, "global_layers": [l for l in range(L) if kinds[l]],
           "prefill_4096": {"ms": round(ms["all"], 3), "tokens_per_s": round(S / (ms["all"] * 1e-3), 1),
                            "us_per_layer": round(ms["all"] * 1e3 / L, 2),
                            "unfused_ms": round(ms["unfused"], 3),
                            "unfused_phases_ms": {"rotary": round(ms["rotary"], 3),
                                                  "attention": round(ms["attention"], 3),
                                                  "kv_append": round(ms["step"] - ms["attention"], 3)}}}
    del g_all, g_unf, g_pro, g_step, g_att, q, k, v, o, caches
    torch.cuda.empty_cache()

    P = 32768
    with torch.cuda.stream(stream):
        caches = []
        for l in range(L):
            c = sess.kv_cache(hkv, d, P + 1)
            sess.append(c, torch.randn(P * hkv * d, generator=gen, device=dev),
                        torch.randn(P * hkv * d, generator=gen, device=dev), P)
            caches.append(c)
        q = [torch.randn(hq * d, generator=gen, device=dev) for _ in range(L)]
        k = [torch.randn(hkv * d, generator=gen, device=dev) for _ in range(L)]
        v = [torch.randn(hkv * d, generator=gen, device=dev) for _ in range(L)]
        o = [torch.empty(hq * d, device=dev) for _ in range(L)]
    dcfgs = [KvAttentionConfig(1, hq, hkv, d, True, 0 if g else W) for g in kinds]

    def d_prologue():
        for l in range(L):
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], 1, hq, hkv, d, qn[l], kn[l], 1e-6, P, 1.0)

    def d_steps():
        for l in range(L):
            sess.decode_step(None, q[l], k[l], v[l], [caches[l]], dcfgs[l], o[l])

    def d_unfused():
        for l in range(L):
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], 1, hq, hkv, d, qn[l], kn[l], 1e-6, P, 1.0)
            sess.decode_step(None, q[l], k[l], v[l], [caches[l]], dcfgs[l], o[l])

    def d_layers():
        for l in range(L):
            sess.gemma_decode_step(tab[kinds[l]], q[l], k[l], v[l], [caches[l]], dcfgs[l], qn[l], kn[l], 1e-6, 1.0,
                                   o[l])

    def reset():
        for c in caches:
            c.truncate(P)

    d_steps()
    sess.sync()
    reset()
    d_layers()
    sess.sync()
    reset()
    graphs = {}
    for n, fn in (("all", d_layers), ("unfused", d_unfused), ("rotary", d_prologue), ("step", d_steps)):
        graphs[n] = captured(fn)
        reset()
    ms = {n: time_graph(g, max(5, args.steps), 3) for n, g in graphs.items()}
    rec["decode_32768"] = {"ms_per_token": round(ms["all"], 4), "tokens_per_s": round(1e3 / ms["all"], 1),
                           "us_per_layer": round(ms["all"] * 1e3 / L, 3),
                           "unfused_ms_per_token": round(ms["unfused"], 4),
                           "unfused_phases_ms": {"rotary": round(ms["rotary"], 4),
                                                 "attention_and_kv_append": round(ms["step"], 4)}}
    out["gemma3_1b"] = rec
    del graphs, caches, q, k, v, o
    torch.cuda.empty_cache()

    # ---- Gemma-3-4B turn: 16384 cached tokens, a 128-token chunk, 256 decode steps ----
    w4 = GEMMA_WORKLOADS["gemma3_4b"]
    hq, hkv, d, L, W = w4["hq"], w4["hkv"], w4["d"], w4["layers"], w4["window"]
    kinds = layer_kinds(L)
    P, S, T = 16384, 128, 256
    with torch.cuda.stream(stream):
        tab = tables(d, P + S + T + 64, W)
        qn = [torch.randn(d, generator=gen, device=dev) * 0.1 + 1.0 for _ in range(L)]
        kn = [torch.randn(d, generator=gen, device=dev) * 0.1 + 1.0 for _ in range(L)]
        caches = []
        for l in range(L):
            c = sess.kv_cache(hkv, d, P + S + T)
            sess.append(c, torch.randn(P * hkv * d, generator=gen, device=dev),
                        torch.randn(P * hkv * d, generator=gen, device=dev), P)
            caches.append(c)
        cq = [torch.randn(S * hq * d, generator=gen, device=dev) for _ in range(L)]
        ck = [torch.randn(S * hkv * d, generator=gen, device=dev) for _ in range(L)]
        cv = [torch.randn(S * hkv * d, generator=gen, device=dev) for _ in range(L)]
        co = [torch.empty(S * hq * d, device=dev) for _ in range(L)]
        q = [torch.randn(hq * d, generator=gen, device=dev) for _ in range(L)]
        k = [torch.randn(hkv * d, generator=gen, device=dev) for _ in range(L)]
        v = [torch.randn(hkv * d, generator=gen, device=dev) for _ in range(L)]
        o = [torch.empty(hq * d, device=dev) for _ in range(L)]
    ccfg = [KvAttentionConfig(S, hq, hkv, d, True, 0 if g else W) for g in kinds]
    dcfg = [KvAttentionConfig(1, hq, hkv, d, True, 0 if g else W) for g in kinds]

    def chunk():
        for l in range(L):
            sess.gemma_prefill_step(tab[kinds[l]], cq[l], ck[l], cv[l], caches[l], ccfg[l], qn[l], kn[l], 1e-6, 1.0,
                                    co[l])

    def decode_token():
        for l in range(L):
            sess.gemma_decode_step(tab[kinds[l]], q[l], k[l], v[l], [caches[l]], dcfg[l], qn[l], kn[l], 1e-6, 1.0,
                                   o[l])

    def decode_token_unfused():
        for l in range(L):
            pos = caches[l].len()
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], 1, hq, hkv, d, qn[l], kn[l], 1e-6, pos, 1.0)
            sess.decode_step(None, q[l], k[l], v[l], [caches[l]], dcfg[l], o[l])

    def reset():
        for c in caches:
            c.truncate(P)

    chunk()  # sizes every workspace and creates the caches' bf16 operands
    for _ in range(T):
        decode_token()
    sess.sync()
    reset()
    # The turn as one graph for the chunk and one per TURN_GRAPH_TOKENS decode
    # tokens (each token's launches carry its own cache position), replayed back
    # to back: no graph holds more than 16 x 34 x 2 = 1088 dispatches.
    g_turn = [captured(chunk)]
    for _ in range(T // TURN_GRAPH_TOKENS):
        g_turn.append(captured(lambda: [decode_token() for _ in range(TURN_GRAPH_TOKENS)]))
    reset()
    g_chunk = captured(chunk)  # then one decode token right after the chunk, with its phases
    g_tok = captured(decode_token)
    for c in caches:
        c.truncate(P + S)
    g_tok_unf = captured(decode_token_unfused)
    for c in caches:
        c.truncate(P + S)

    def tok_prologue():
        for l in range(L):
            sess.gemma_qk_prologue(tab[kinds[l]], q[l], k[l], 1, hq, hkv, d, qn[l], kn[l], 1e-6, P + S, 1.0)

    def tok_steps():
        for l in range(L):
            sess.decode_step(None, q[l], k[l], v[l], [caches[l]], dcfg[l], o[l])

    g_tok_rot = captured(tok_prologue)
    g_tok_step = captured(tok_steps)
    reset()
    ms_turn = time_graphs(g_turn, 3, 1)
    sess.sync()
    ms_chunk = time_graph(g_chunk, reps, 2)
    ms_tok = time_graph(g_tok, max(5, args.steps), 3)
    ms_unf = time_graph(g_tok_unf, max(5, args.steps), 3)
    ms_rot = time_graph(g_tok_rot, max(5, args.steps), 3)
    ms_st = time_graph(g_tok_step, max(5, args.steps), 3)
    decode_ms = ms_turn - ms_chunk
    out["gemma3_4b"] = {
        "layers": L, "global_layers": [l for l in range(L) if kinds[l]],
        "turn": {"ms": round(ms_turn, 3), "cached_tokens": P, "chunk_tokens": S, "decode_tokens": T,
                 "tokens_per_s": round((S + T) / (ms_turn * 1e-3), 1),
                 "chunk_ms": round(ms_chunk, 3), "chunk_us_per_layer": round(ms_chunk * 1e3 / L, 2),
                 "decode_ms": round(decode_ms, 3), "decode_tokens_per_s": round(T / (decode_ms * 1e-3), 1)},
        "decode_token_after_chunk": {"ms": round(ms_tok, 4), "us_per_layer": round(ms_tok * 1e3 / L, 3),
                                     "unfused_ms": round(ms_unf, 4),
                                     "unfused_phases_ms": {"rotary": round(ms_rot, 4),
                                                           "attention_and_kv_append": round(ms_st, 4)}},
    }
    del g_turn, g_chunk, g_tok, g_tok_unf, g_tok_rot, g_tok_step, caches
    torch.cuda.empty_cache()
    return out


def time_graphs(graphs, reps, warm) -> float:
    """ms per replay of a sequence of graphs launched back to back on the
    current stream (event-timed around reps sequences)."""
    import torch

    for _ in range(warm):
        for g in graphs:
            g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        for g in graphs:
            g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def visible_pairs(S: int, P: int, window: int) -> int:
    """Unmasked (query, key) pairs of a causal chunk of S rows after P cached rows."""
    total = 0
    for i in range(S):
        k = P + i + 1
        total += min(k, window) if window > 0 else k
    return total


def configs_bench(sess, stream, gen, dev, args, time_graph) -> dict:
    """One record per case of CONFIG_CASES: decode layers as the fused step
    (RoPE for the Llama shapes, attention, append), prefill and chunk layers
    as the attention call. Work is credited by the algorithmic figures: decode
    bytes of the visible keys, prefill FLOP of the unmasked pairs; chunks also
    report the bytes of their visible f32 K/V."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.rotary import KvAttentionConfig

    out = {}
    only = set(args.configs.split(",")) if getattr(args, "configs", None) else None
    for name, cfg_id, L, hq, hkv, d, S, P, W, rope in CONFIG_CASES:
        if only is not None and name not in only:
            continue
        w = hkv * d
        with torch.cuda.stream(stream):
            caches = []
            for l in range(L):
                gen.manual_seed(5000 + 100 * cfg_id + l)
                c = sess.kv_cache(hkv, d, P + S) if P > 0 or S == 1 else None
                if P > 0:
                    sess.append(c, torch.randn(P * w, generator=gen, device=dev),
                                torch.randn(P * w, generator=gen, device=dev), P)
                caches.append(c)
            q = [torch.randn(S * hq * d, generator=gen, device=dev) for _ in range(L)]
            k = [torch.randn(S * w, generator=gen, device=dev) for _ in range(L)]
            v = [torch.randn(S * w, generator=gen, device=dev) for _ in range(L)]
            o = [torch.empty(S * hq * d, device=dev) for _ in range(L)]
        table = sess.rope_table(_ffi.ROPE_LLAMA, d, THETA, max_positions=P + S + 64) if rope else None
        cfg = KvAttentionConfig(S, hq, hkv, d, True, W)
        decode = S == 1

        def step():
            for l in range(L):
                if decode:
                    sess.decode_step(table, q[l], k[l], v[l], [caches[l]], cfg, o[l])
                else:
                    sess.attention(q[l], k[l], v[l], caches[l], cfg, o[l])

        def reset():
            if decode:
                for c in caches:
                    c.truncate(P)

        step()
        sess.sync()
        reset()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step()
        reset()
        ms = time_graph(g, max(3, args.steps // 4), 2)
        us = ms * 1e3 / L
        rec = {"config": cfg_id, "layers": L, "us_per_layer": round(us, 3)}
        if decode:
            keys = min(P + 1, W) if W > 0 else P + 1
            nbytes = decode_bytes(keys, hq, hkv, d)
            rec.update(GBps=round(nbytes / (us * 1e-6) / 1e9, 1),
                       hbm_frac=round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), bytes_per_layer=nbytes)
        else:
            fl = 4.0 * d * hq * visible_pairs(S, P, W)
            rec.update(TFLOPs=round(fl / (us * 1e-6) / 1e12, 2),
                       mfma_frac=round(fl / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4), flop_per_layer=fl)
            if P > 0:
                keys = min(P + S, W + S) if W > 0 else P + S
                nbytes = keys * w * 8 + 2 * S * hq * d * 4
                rec.update(GBps=round(nbytes / (us * 1e-6) / 1e9, 1),
                           hbm_frac=round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
        out[name] = rec
        del g, caches, q, k, v, o, table
        torch.cuda.empty_cache()
    return out


def prefill_bench(sess, stream, gen, dev, args, time_graph) -> dict:
    """The 4096-token causal prefill of config 2a over 28 layers, three forms:
    prefill_4096 = the attention call in the reference's order (the prompt's
    f32 q/k/v passed in, no cache; the bf16 K/V operands are made inside the
    call, rotary.rs:335-415); prefill_step_4096 = the fused prefill step (RoPE,
    append of the f32 rows and bf16 operands, staged q, then attention);
    prefill_attention_4096 = the attention call over a cache that already
    holds the prompt (spissa_attention_cached_device: one launch, f32 q
    rounded to bf16 in the kernel, K/V from each layer's bf16 shadow; the
    dominant kernel's MFMA rate). Inside the fused step the same kernel reads
    q already staged in bf16 and K/V the append just wrote, and runs faster."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.rotary import KvAttentionConfig

    res = {}
    w = HKV * D
    log("timing prefill")
    pq = [torch.randn(PREFILL_S * HQ * D, generator=gen, device=dev) for _ in range(LAYERS)]
    pk = [torch.randn(PREFILL_S * w, generator=gen, device=dev) for _ in range(LAYERS)]
    pv = [torch.randn(PREFILL_S * w, generator=gen, device=dev) for _ in range(LAYERS)]
    po = [torch.empty(PREFILL_S * HQ * D, device=dev) for _ in range(LAYERS)]
    cfgp = KvAttentionConfig(PREFILL_S, HQ, HKV, D, True)

    ptable = sess.rope_table(_ffi.ROPE_LLAMA, D, THETA, max_positions=PREFILL_S + 64)
    pcaches = [sess.kv_cache(HKV, D, PREFILL_S) for _ in range(LAYERS)]

    def call_order():
        # the reference's attention call: f32 K/V of the prompt passed in
        # (converted to the bf16 operands inside the call), no cache
        for l in range(LAYERS):
            sess.attention(pq[l], pk[l], pv[l], None, cfgp, po[l])

    def fused_step():
        # RoPE + append (f32 rows and bf16 operands) + staged q, then attention
        for l in range(LAYERS):
            sess.prefill_step(ptable, pq[l], pk[l], pv[l], pcaches[l], cfgp, po[l])

    def attention_phase():
        # the attention call alone: the prompt is already in the cache
        for l in range(LAYERS):
            sess.attention_cached(pq[l], pcaches[l], cfgp, po[l])

    call_order()
    fused_step()
    sess.sync()
    for c in pcaches:
        c.truncate(0)
    graphs = {}
    for name, fn in (("call", call_order), ("step", fused_step), ("attn", attention_phase)):
        graphs[name] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[name], stream=stream):
            fn()  # the step's capture appends the prompt, so the attention phase sees it
    fl = prefill_flops(PREFILL_S)
    ms = {name: time_graph(g, max(3, args.steps // 4), 2) for name, g in graphs.items()}

    def rec(m):
        return {"ms_per_step": m, "us_per_layer": m * 1e3 / LAYERS,
                "TFLOPs": LAYERS * fl / (m * 1e-3) / 1e12, "tokens_per_s": PREFILL_S * 1e3 / m,
                "flop_per_layer": fl}

    res["prefill_4096"] = rec(ms["call"])
    res["prefill_step_4096"] = rec(ms["step"])
    res["prefill_step_4096"]["rope_append_us_per_layer"] = (ms["step"] - ms["attn"]) * 1e3 / LAYERS
    res["prefill_attention_4096"] = rec(ms["attn"])
    del graphs, pq, pk, pv, po, pcaches
    torch.cuda.empty_cache()
    return res


def configs_only(args) -> dict:
    """The records of the CONFIG_CASES named in --configs, nothing else."""
    import torch

    from spissa_amd.device import Session

    torch.cuda.init()
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    sess = Session(0, stream=stream)
    gen = torch.Generator(device=dev)

    def time_graph(g, reps, warm):
        for _ in range(warm):
            g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        sess.sync()
        return a.elapsed_time(b) / reps

    names = args.configs.split(",")
    with torch.cuda.stream(stream):
        out = configs_bench(sess, stream, gen, dev, args, time_graph)
        if "projections" in names:
            out["projections"] = projection_bench(sess, stream, gen, dev, args, time_graph)
        if "prefill_4096" in names:
            out.update(prefill_bench(sess, stream, gen, dev, args, time_graph))
        if "workloads" in names:
            out["workloads"] = workloads_bench(sess, stream, gen, dev, args, time_graph)
    return out


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# CPU-baseline workloads: (name, BASELINE.json config index, Hq, Hkv, d, new rows S, cached rows P,
# window, rows sampled for a prefill or chunk (0: the whole call)).
CPU_CASES = [
    ("llama32_1b_decode_512", 0, 32, 8, 64, 1, 512, 0, 0),
    ("llama32_1b_prefill_2048", 1, 32, 8, 64, 2048, 0, 0, 32),
    ("llama32_1b_decode_2048", 1, 32, 8, 64, 1, 2048, 0, 0),
    ("llama32_3b_prefill_4096", 2, 24, 8, 128, 4096, 0, 0, 32),
    ("llama32_3b_decode_8192", 2, 24, 8, 128, 1, 8192, 0, 0),
    ("gemma3_1b_prefill_4096_global", 3, 4, 1, 256, 4096, 0, 0, 32),
    ("gemma3_1b_prefill_4096_local_w512", 3, 4, 1, 256, 4096, 0, 512, 32),
    ("gemma3_1b_decode_32768_global", 3, 4, 1, 256, 1, 32768, 0, 0),
    ("gemma3_1b_decode_32768_local_w512", 3, 4, 1, 256, 1, 32768, 512, 0),
    ("gemma3_4b_chunk_128_on_16384_global", 4, 8, 4, 256, 128, 16384, 0, 16),
    ("gemma3_4b_chunk_128_on_16384_local_w1024", 4, 8, 4, 256, 128, 16384, 1024, 16),
    ("gemma3_4b_decode_16512_global", 4, 8, 4, 256, 1, 16512, 0, 0),
    ("gemma3_4b_decode_16512_local_w1024", 4, 8, 4, 256, 1, 16512, 1024, 0),
]


def cpu_baseline(args) -> dict:
    """The oracle (the C restatement of rotary.rs:335-415) on this host's cores,
    over a bounded sample of every BASELINE config. Single-thread figures are
    the reference's own behaviour (its attention is single-threaded per call);
    the n-thread figure runs independent decode layers on `threads` POSIX
    threads (harness parallelism). Prefill and chunk layers time their last
    rows as one chunked call (the same keys and loop order as the whole call)
    and scale by the oracle's operation count: per query row, QK over its
    visible keys plus PV over every key of the call (rotary.rs:389-410)."""
    import numpy as np

    import oracle
    from spissa_amd.synth import normal_f32, seed_for

    # the GPU box grants 16 cores per GPU, whatever the host reports
    threads = min(16, os.cpu_count() or 1)
    configs = {}
    decode_units = []
    for name, cfg_id, hq, hkv, d, S, P, W, sample in CPU_CASES:
        w = hkv * d
        rows = S if sample == 0 else sample
        first = S - rows  # rows of the call before the timed ones sit in the cache
        q = normal_f32(seed_for(100 + cfg_id, 0, 0, "q"), rows * hq * d)
        kk = normal_f32(seed_for(100 + cfg_id, 0, 0, "k"), (P + S) * w)
        vv = normal_f32(seed_for(100 + cfg_id, 0, 0, "v"), (P + S) * w)
        cached = P + first
        c = oracle.KvCache(hkv, d, P + S)
        if cached:
            c.append(kk[:cached * w].copy(), vv[:cached * w].copy(), cached)
        k_cur, v_cur = kk[cached * w:].copy(), vv[cached * w:].copy()
        reps = 3 if S == 1 else 1
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            oracle.sdpa_with_cache(q, k_cur, v_cur, c, rows, hq, hkv, d, True, W)
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        rec = {"config": cfg_id, "cores": 1}
        if S == 1:
            keys = min(P + 1, W) if W else P + 1
            nbytes = decode_bytes(keys, hq, hkv, d)
            rec.update(us_per_layer=round(t * 1e6, 1), GBps=round(nbytes / t / 1e9, 3),
                       sample=f"one decode layer call, median of {reps}")
            decode_units.append((name, (q, k_cur, v_cur, c), (1, hq, hkv, d, 1, W), nbytes))
        else:
            key_len = P + S

            def cost(r):
                vis = min(P + r + 1, W) if W else P + r + 1
                return vis + key_len
            scale = sum(cost(r) for r in range(S)) / sum(cost(r) for r in range(first, S))
            t_layer = t * scale
            fl = 4.0 * d * hq * visible_pairs(S, P, W)
            rec.update(us_per_layer=round(t_layer * 1e6, 1), TFLOPs=fl / t_layer / 1e12,
                       sample=f"last {rows} of {S} query rows as one chunked call ({t * 1e3:.0f} ms), "
                              f"x{scale:.1f} by operation count")
        configs[name] = rec
    # n-thread throughput of the decode layers: 2 x threads independent units
    nthread = {}
    for name, unit, cfg_t, nbytes in decode_units:
        many = [unit] * (2 * threads)
        t0 = time.perf_counter()
        oracle.sdpa_many(many, cfg_t, threads)
        tn = time.perf_counter() - t0
        nthread[name] = {"GBps": round(len(many) * nbytes / tn / 1e9, 3), "us_per_layer": round(tn / len(many) * 1e6, 1)}
    main_rec = configs["llama32_3b_decode_8192"]
    out = {
        "value": main_rec["GBps"], "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": "oracle decode, Llama-3.2-3B heads, 8192-token cache, median of 3 single-thread layer calls "
                  f"({main_rec['us_per_layer']:.0f} us/layer)",
        "us_per_layer": main_rec["us_per_layer"],
        "cpu_model": cpu_model(), "host_cpus": os.cpu_count(), "threads_used": threads,
        "threads_note": "one GPU's share of the box's cores (16); RLLM_THREADS does not reach the reference's "
                        "attention, which is single-threaded per call (rotary.rs:354-412)",
        "configs": configs,
        "nthread": {"cores": threads, "note": "harness parallelism: independent decode layer calls on POSIX "
                                              "threads", "layers": nthread},
    }
    if not args.decode_only:
        p4 = configs["llama32_3b_prefill_4096"]
        out["prefill"] = {"TFLOPs": p4["TFLOPs"], "us_per_layer": p4["us_per_layer"], "cores": 1,
                          "sample": p4["sample"]}
        # The fused q/k/v projection at decode batch 1 (ops.rs linear over the
        # bf16 weight): 5120 x 3072 multiply-adds, single thread.
        hid, qkv = HQ * D, (HQ + 2 * HKV) * D
        wbits = (normal_f32(seed_for(3, 0, 2, "k"), qkv * hid, 0.0, 0.02).view(np.uint32) >> 16).astype(np.uint16)
        x = normal_f32(seed_for(3, 0, 2, "q"), hid)
        lt = []
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.linear(x, wbits, oracle.DTYPE_BF16, None, 1, hid, qkv)
            lt.append(time.perf_counter() - t0)
        tl = statistics.median(lt)
        out["projection_b1"] = {
            "value": qkv * hid * 2 / tl / 1e9, "unit": "GB/s of weights", "us_per_layer": tl * 1e6, "cores": 1,
            "sample": "oracle linear, Llama-3.2-3B fused q/k/v weight (5120 x 3072 bf16), batch 1, median of 3"}
        # The LM head over the Llama-3.2-3B tied table (128256 x 3072 bf16) and the
        # argmax (the reference's serial lm_head_logits_rows_bf16 + sample_argmax).
        vocab, hid = LM_HEADS["llama32_3b"]
        import torch

        g = torch.Generator(device="cuda").manual_seed(13)  # synthetic data only: drawn on the device
        tb = (torch.randn(vocab * hid, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        tbits = tb.view(torch.int16).cpu().numpy().view(np.uint16)
        del tb
        x = normal_f32(seed_for(3, 0, 3, "q"), hid)
        t0 = time.perf_counter()
        lg = oracle.lm_head_logits(x, tbits, oracle.DTYPE_BF16, vocab, hid)
        oracle.sample_argmax(lg)
        th = time.perf_counter() - t0
        out["lm_head_b1"] = {
            "value": vocab * hid * 2 / th / 1e9, "unit": "GB/s of table", "us_per_token": th * 1e6, "cores": 1,
            "sample": "oracle LM head + argmax, Llama-3.2-3B tied table (128256 x 3072 bf16), one token"}
    return out


def headline(res: dict, cpu) -> dict:
    """The figures the north star names, compactly, for the end of the line."""
    def r(v, n=3):
        return None if v is None else round(v, n)

    d1 = res["decode_b1"]
    h = {"decode_b1_us_per_layer": r(d1["us_per_layer"]), "decode_b1_GBps": r(d1["GBps"], 1),
         "decode_b1_hbm_frac": r(d1["GBps"] / HBM_PEAK_GBS, 4),
         "decode_b1_attn_kernel_us": r(d1["attn_kernel_us"]),
         "decode_b1_attn_kernel_hbm_frac": r(d1["attn_kernel_GBps"] / HBM_PEAK_GBS, 4)}
    if "decode_b16" in res:
        b = res["decode_b16"]
        h.update(decode_b16_us_per_layer=r(b["us_per_layer"]), decode_b16_hbm_frac=r(b["GBps"] / HBM_PEAK_GBS, 4))
    for key, short in (("prefill_4096", "prefill_call"), ("prefill_step_4096", "prefill_step"),
                       ("prefill_attention_4096", "prefill_attention")):
        if key in res:
            p = res[key]
            h[f"{short}_us_per_layer"] = r(p["us_per_layer"])
            h[f"{short}_TFLOPs"] = r(p["TFLOPs"], 1)
            h[f"{short}_mfma_frac"] = r(p["TFLOPs"] / BF16_PEAK_TFLOPS, 4)
    ceil = res.get("hbm_read_ceiling") or {}
    if "layer_67MB" in ceil:
        h["hbm_read_ceiling_GBps"] = ceil["layer_67MB"]["GBps"]
    if res.get("mfma_ceiling"):
        h["mfma_ceiling_TFLOPs"] = res["mfma_ceiling"]["TFLOPs"]
    wl = res.get("workloads") or {}
    if "gemma3_1b" in wl:
        h["gemma3_1b_prefill_4096_ms"] = wl["gemma3_1b"]["prefill_4096"]["ms"]
        h["gemma3_1b_decode_32768_ms_per_token"] = wl["gemma3_1b"]["decode_32768"]["ms_per_token"]
    if "gemma3_4b" in wl:
        h["gemma3_4b_turn_ms"] = wl["gemma3_4b"]["turn"]["ms"]
        h["gemma3_4b_decode_token_ms"] = wl["gemma3_4b"]["decode_token_after_chunk"]["ms"]
    if cpu is not None:
        h["cpu_decode_b1_us_per_layer"] = cpu["us_per_layer"]
        if "prefill" in cpu:
            h["cpu_prefill_4096_us_per_layer"] = round(cpu["prefill"]["us_per_layer"], 1)
    return h


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true")
    ap.add_argument("--skip-workloads", action="store_true",
                    help="leave out the Gemma workloads (for counter passes: three whole-bench rocprofv3 --pmc "
                         "runs ended in a SIGSEGV in the profiler's threads while these graphs replayed)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 256 MiB device copy (HBM-counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--configs", default="",
                    help="only time these comma-separated cases of CONFIG_CASES (and 'projections': the "
                         "q/k/v projection at batch 1, 16 and 4096; 'prefill_4096': config 2a's prefill; 'workloads': "
                         "the whole Gemma workloads) and print their records; the benchmark line is not printed")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's attention path has no multi-GPU leg "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    if args.configs:
        print(json.dumps(configs_only(args)), flush=True)
        return 0
    t0 = time.time()
    res = gpu_bench(args)
    log(f"gpu part done in {time.time() - t0:.1f}s")
    cpu = None if args.no_cpu else cpu_baseline(args)
    d1 = res["decode_b1"]
    plan = decode_plan()
    traffic = measured_traffic(plan)
    line = {
        "metric": "decode-attn HBM GB/s + us/layer; prefill-attn TFLOP/s (Llama-3.2-3B shape)",
        "value": round(d1["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch.randn N(0,1) K/V/Q resident in HBM)",
        "config": {"workload": "llama-3.2-3B attention decode, 8192-token KV cache, batch 1, 28 layers "
                               "(RoPE + split-K decode + KV append per layer, fused in two launches)",
                   "heads": f"{HQ}q/{HKV}kv", "head_dim": D, "context": CTX, "layers": LAYERS},
        "us_per_layer": round(d1["us_per_layer"], 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(d1["attn_kernel_GBps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(d1["attn_kernel_GBps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"],
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, calibrated on copies of known size "
                              "(profiles/decode_b1_hbm_traffic.md), withheld when the profile's plan differs "
                              "from the current launch",
            "traffic_plan": traffic["profile_plan"],
            "plan": plan,
            "kernel": "one decode attention launch = decode_split_kernel<128,3,3> + "
                      "decode_combine_kernel<128,3,16,256>; event-timed average over 28 back-to-back launches "
                      "per graph replay",
        },
        "device": res.get("device"),
    }
    # Detail blocks first; the headline figures close the line (its tail is
    # what a log keeps).
    if "sublayer_b1" in res:
        line["sublayer_b1"] = {"workload": "llama-3.2-3B attention sublayer at decode, batch 1, 8192-token "
                                           "cache: input RMSNorm, q/k/v projections (bf16), RoPE + attention "
                                           "+ append, o projection",
                               **{k: round(v, 3) for k, v in res["sublayer_b1"].items()}}
    if "projections" in res:
        line["projections"] = {"workload": "llama-3.2-3B fused q/k/v projection, 5120 x 3072 bf16 weight "
                                           "resident in HBM, f32 activations and output",
                               **res["projections"]}
    if "lm_head" in res:
        line["lm_head"] = {"workload": "greedy decode tail per token: tied-embedding LM head over the bf16 "
                                       "table (logits GEMV) + argmax token; token_us = both, logits_us = GEMV "
                                       "only, argmax_us = argmax only",
                           **res["lm_head"]}
    if "configs" in res:
        line["configs"] = {"workload": "attention layers of the other BASELINE configs (index into "
                                       "BASELINE.json configs): decode = fused RoPE/attention/append step, "
                                       "prefill and chunk = the attention call; GB/s and TFLOP/s from the "
                                       "algorithmic bytes and unmasked pairs",
                           **res["configs"]}
    if "workloads" in res:
        line["workloads"] = {"workload": "BASELINE configs 3 and 4 through every layer: the Gemma prefill and "
                                         "decode steps (QK-norm, RoPE, attention, append fused; unfused_* = the "
                                         "prologue launch, then the prefill or decode step); 5 local (sliding "
                                         "window) : 1 global layers; phases are the reference's rotary / "
                                         "attention / kv_append buckets, timed on the unfused sequence",
                             **res["workloads"]}
    if cpu is not None:
        line["cpu_baseline"] = cpu
    line["hbm_read_ceiling"] = res.get("hbm_read_ceiling")
    line["mfma_ceiling"] = res.get("mfma_ceiling")
    line["decode_b1"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in d1.items()}
    if "decode_b16" in res:
        line["decode_b16"] = {k: round(v, 3) for k, v in res["decode_b16"].items()}
    phases = {
        "prefill_4096": "the attention call in the reference's order (f32 q/k/v of the prompt, no cache; the "
                        "bf16 K/V operands are made inside the call)",
        "prefill_step_4096": "fused prefill step: RoPE + append of f32 rows and bf16 operands + staged q, then "
                             "attention",
        "prefill_attention_4096": "the attention call over a cache already holding the prompt (one launch; f32 q, "
                                  "K/V from the cache's bf16 shadow)",
    }
    for key, phase in phases.items():
        if key in res:
            line[key] = {"phase": phase, **{k: round(v, 3) for k, v in res[key].items()}}
    if "prefill_attention_4096" in res:
        p = res["prefill_attention_4096"]
        line["roofline_prefill"] = {"bound": "mfma", "kernel": "prefill_kernel<128,1,4,64,1,1> (the attention "
                                                                "launch of prefill_attention_4096)",
                                    "achieved": round(p["TFLOPs"], 2), "peak": BF16_PEAK_TFLOPS,
                                    "unit": "TFLOP/s", "frac": round(p["TFLOPs"] / BF16_PEAK_TFLOPS, 4),
                                    "dtype": "bf16 MFMA, f32 accumulate"}
        if res.get("mfma_ceiling"):
            line["roofline_prefill"]["frac_of_measured_ceiling"] = round(
                p["TFLOPs"] / res["mfma_ceiling"]["TFLOPs"], 4)
    line["headline"] = headline(res, cpu)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
