"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (`value`): Q4_0X4 GEMV at the Qwen3-1.7B FFN up-proj shape
(6144 x 2048, fp32 x), HBM GB/s of algorithmic bytes, weights rotating over
> 512 MB of copies so every launch streams from HBM (the 256 MB Infinity
Cache cannot hold the set).  A step is one GEMV launch; steps are replayed
from a HIP graph so that host launch cost is not timed.

Also reported: batch-1 greedy decode tok/s of a random-init
Qwen3-1.7B-shaped model (128-token prompt, then 256 tokens), the same prompt
through the batched int8-MFMA prefill (Q8_0 activations), and the CPU
baseline (the oracle's AVX-512 restatement of the reference kernels on the
host cores, pinned threads, same rotating working set).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-decode] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Q4_0 GEMV HBM GB/s (% of peak); bs1 decode tok/s, Qwen3-1.7B-shape, 1 GPU"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
ROWS, K = 6144, 2048
# W (6144 x 2048 Q4_0 = 7,077,888 B) + x fp32 (8,192 B) + y fp32 (24,576 B)
GEMV_BYTES = ROWS * (K // 32) * 18 + 4 * K + 4 * ROWS
ROTATE_BYTES = 512 << 20
# HBM bytes per launch of the GEMV kernel, from rocprofv3 --pmc FETCH_SIZE
# (3,508 KiB x 2.00) and WRITE_SIZE (32 KiB x 1.00) over the eager `--profile
# c1` launches; the factors come from the same counters read on an
# elementwise kernel that reads and writes 256 MiB (`--profile copy`).
# 1.01 x GEMV_BYTES: the weights are read exactly once.
GEMV_TRAFFIC_BYTES = 7_216_029


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Launches per captured graph, at least: a replay's own start costs a few
# microseconds (the 6144x2048 GEMV: 3.45 us per launch with one pass over
# its 77 rotating copies per graph, 3.38 us with eight), which is the graph
# API's, not the kernel's.
MIN_GRAPH_LAUNCHES = 1024


def _graph_time(launch, n_launch: int, steps: int, warmup: int):
    """Mean device time per launch of `launch(i % n_launch)`, i = 0, 1, ...,
    whole passes over the n_launch launches (at least MIN_GRAPH_LAUNCHES)
    captured once into a graph on a side stream and replayed; HIP events on
    that stream bracket the timed replays."""
    import torch

    stream = torch.cuda.Stream()
    st = stream.cuda_stream
    with torch.cuda.stream(stream):
        for i in range(n_launch):  # eager warm-up outside capture
            launch(i, st)
    torch.cuda.synchronize()
    n_launch_all = n_launch * max(1, math.ceil(MIN_GRAPH_LAUNCHES / n_launch))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(n_launch_all):
            launch(i % n_launch, st)
    n_launch = n_launch_all
    reps = max(1, math.ceil(steps / n_launch))
    wreps = max(1, math.ceil(warmup / n_launch))
    with torch.cuda.stream(stream):
        for _ in range(wreps):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    del g
    return ms / (reps * n_launch), reps * n_launch, wreps * n_launch


def _copies(nbytes: int) -> int:
    return math.ceil(ROTATE_BYTES / nbytes) + 1


def bench_gemv(ctx, steps: int, warmup: int):
    import numpy as np
    import torch

    from zero_amd import synth

    rng = np.random.default_rng(0)
    w_host = synth.weight(rng, synth.Q4_0, ROWS, K, 4)
    copies = _copies(w_host.nbytes)
    w0 = torch.from_numpy(w_host).cuda()
    w_dev = [w0] + [w0.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(synth.activations(rng, K)).cuda()
    y = torch.empty(ROWS, dtype=torch.float32, device="cuda")

    def launch(i, st):
        ctx.linear_dev(x, w_dev[i], y, K, ROWS, synth.Q4_0, 4, stream=st)

    per, n, nw = _graph_time(launch, copies, steps, warmup)
    gbs = GEMV_BYTES / (per * 1e-3) / 1e9
    return {"launches": n, "warmup": nw, "copies": copies, "ms_per_gemv": per, "gbs": gbs,
            "w_host": w_host, "x_host": x.cpu().numpy()}


def _row(name, per_ms, nbytes, n, copies, **extra):
    gbs = nbytes / (per_ms * 1e-3) / 1e9
    d = {"workload": name, "us_per_launch": round(per_ms * 1e3, 3), "launches": n, "rotating_copies": copies,
         "bytes_per_launch": nbytes, "GB_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    d.update(extra)
    log(f"{name}: {per_ms * 1e3:.2f} us, {gbs:.0f} GB/s")
    return d


def bench_rows(ctx, steps: int, cpu=None):
    """The other hot-path workloads, each timed like the headline GEMV:
    fused Q|K|V Q8_0X4, LM head Q8_0X4 + argmax, Q4_K and Q6_K GEMVs at
    Llama-3-8B FFN shapes (Q4_K also through the Q8_K integer path), and the
    M=512 int8-MFMA prefill GEMM.  With `cpu`, every row also carries the
    same workload on the host cores (cpu_baseline)."""
    import numpy as np
    import torch

    from zero_amd import synth

    rng = np.random.default_rng(7)
    out = {}
    H = 2048

    def rotating(w_host):
        c = _copies(w_host.nbytes)
        w0 = torch.from_numpy(w_host).cuda()
        return [w0] + [w0.clone() for _ in range(c - 1)], c

    # fused Q|K|V, Q8_0X4, 2048 + 1024 + 1024 rows x 2048
    segs = [(2048, synth.weight(rng, synth.Q8_0, 2048, H, 4)), (1024, synth.weight(rng, synth.Q8_0, 1024, H, 4)),
            (1024, synth.weight(rng, synth.Q8_0, 1024, H, 4))]
    per_copy = sum(w.nbytes for _, w in segs)
    c = _copies(per_copy)
    sd = [[torch.from_numpy(w).cuda() for _, w in segs]]
    sd += [[t.clone() for t in sd[0]] for _ in range(c - 1)]
    x_host = synth.activations(rng, H)
    x = torch.from_numpy(x_host).cuda()
    ys = [torch.empty(n, device="cuda") for n, _ in segs]

    def qkv(i, st):
        ctx.linear_fused_dev(x, [(sd[i][j], ys[j], segs[j][0], synth.Q8_0, 4) for j in range(3)], H, stream=st)

    per, n, _ = _graph_time(qkv, c, steps, steps // 10)
    out["fused_qkv_q8_0x4"] = _row("fused Q|K|V Q8_0X4 (2048+1024+1024)x2048", per, per_copy + 4 * H + 4 * 4096, n, c)
    del sd
    if cpu:
        out["fused_qkv_q8_0x4"]["cpu_baseline"] = cpu.fused(
            "Q|K|V Q8_0X4 (2048+1024+1024)x2048", [(r, w, synth.Q8_0, 4) for r, w in segs], x_host, H,
            per_copy + 4 * H + 4 * 4096)

    # LM head Q8_0X4 151936 x 2048 + argmax, logits written
    V = 151_936
    wl = synth.weight(rng, synth.Q8_0, V, H, 4)
    wd, c = rotating(wl)
    logits = torch.empty(V, device="cuda")
    best = torch.zeros(1, dtype=torch.int64, device="cuda")

    def head(i, st):
        ctx.lm_head_dev(x, wd[i], logits, H, V, synth.Q8_0, 4, best, stream=st)

    per, n, _ = _graph_time(head, c, max(20, steps // 40), 4)
    out["lm_head_q8_0x4_argmax"] = _row("LM head Q8_0X4 151936x2048 + argmax", per, wl.nbytes + 4 * H + 4 * V, n, c)
    del wd
    if cpu:
        out["lm_head_q8_0x4_argmax"]["cpu_baseline"] = cpu.lm_head("LM head Q8_0X4 151936x2048", wl, x_host, H, V,
                                                                   synth.Q8_0, 4, wl.nbytes + 4 * H + 4 * V)
    del wl

    # the headline GEMV with x encoded to Q8_0 first (the integer block dots):
    # the GEMV alone on a resident Q8_0 row, and quantize + GEMV
    wh = synth.weight(rng, synth.Q4_0, 6144, H, 4)
    wd, c = rotating(wh)
    xf = torch.from_numpy(synth.activations(rng, H)).cuda()
    xq = torch.empty(H // 32 * 34, dtype=torch.uint8, device="cuda")
    yq = torch.empty(6144, device="cuda")
    ctx.quantize_q8_0_dev(xf, xq, 1, H)

    def g8(i, st):
        ctx.linear_q8act_dev(xq, wd[i], yq, H, 6144, synth.Q4_0, 4, stream=st)

    def g8q(i, st):
        ctx.quantize_q8_0_dev(xf, xq, 1, H, stream=st)
        ctx.linear_q8act_dev(xq, wd[i], yq, H, 6144, synth.Q4_0, 4, stream=st)

    nbytes = wh.nbytes + H // 32 * 34 + 4 * 6144
    per, n, _ = _graph_time(g8, c, max(200, steps // 4), 40)
    out["q4_0x4_q8act_6144x2048"] = _row("Q4_0X4 6144x2048, x as Q8_0 (integer dots)", per, nbytes, n, c)
    per, n, _ = _graph_time(g8q, c, max(200, steps // 4), 40)
    out["q4_0x4_quant_q8act_6144x2048"] = _row("Q4_0X4 6144x2048, quantize x to Q8_0 + GEMV", per,
                                               nbytes + 4 * H + H // 32 * 34, n, c)
    del wd
    if cpu:
        # the reference has no Q8_0-activation GEMV: its CPU path for these
        # weights is the fp32-x Q4_0X4 kernel
        cb = cpu.gemv("Q4_0X4 6144x2048 (fp32 x: the reference's kernel for these weights)", wh,
                      xf.cpu().numpy(), H, 6144, synth.Q4_0, 4, wh.nbytes + 4 * H + 4 * 6144)
        out["q4_0x4_q8act_6144x2048"]["cpu_baseline"] = cb
        out["q4_0x4_quant_q8act_6144x2048"]["cpu_baseline"] = cb

    # plain (GGUF, .smodel-v1) row-major Q4_0: the headline shape and a Kimi K2
    # expert projection (the DeepSeek2 path's bulk layer weights)
    for name, key, rows, k in (("Q4_0 plain 6144x2048", "q4_0_plain_6144x2048", 6144, 2048),
                               ("Q4_0 plain 2048x7168 (Kimi K2 expert gate/up)", "q4_0_plain_2048x7168", 2048, 7168)):
        wh = synth.weight(rng, synth.Q4_0, rows, k, 1)
        wd, c = rotating(wh)
        xk_host = synth.activations(rng, k)
        xk = torch.from_numpy(xk_host).cuda()
        yk = torch.empty(rows, device="cuda")

        def pl(i, st, wd=wd, xk=xk, yk=yk, rows=rows, k=k):
            ctx.linear_dev(xk, wd[i], yk, k, rows, synth.Q4_0, 1, stream=st)

        per, n, _ = _graph_time(pl, c, max(200, steps // 4), 40)
        out[key] = _row(name, per, wh.nbytes + 4 * k + 4 * rows, n, c)
        del wd
        if cpu:
            out[key]["cpu_baseline"] = cpu.gemv(name, wh, xk_host, k, rows, synth.Q4_0, 1,
                                                wh.nbytes + 4 * k + 4 * rows)

    # the headline GEMV on taller Q4_0X4 matrices (8x the headline rows, and
    # the LM head's height) with more bytes per launch: the strip kernel's
    # batch loop at 49152 rows, the LDS-staged streaming kernel at 151936
    for name, key, rows in (("Q4_0X4 49152x2048 (8x the headline rows)", "q4_0x4_49152x2048", 49152),
                            ("Q4_0X4 151936x2048 (LM-head height)", "q4_0x4_151936x2048", 151_936)):
        wh = synth.weight(rng, synth.Q4_0, rows, H, 4)
        wd, c = rotating(wh)
        yk = torch.empty(rows, device="cuda")

        def tall(i, st, wd=wd, yk=yk, rows=rows):
            ctx.linear_dev(x, wd[i], yk, H, rows, synth.Q4_0, 4, stream=st)

        per, n, _ = _graph_time(tall, c, max(40, steps // 20), 8)
        out[key] = _row(name, per, wh.nbytes + 4 * H + 4 * rows, n, c)
        del wd
        if cpu:
            out[key]["cpu_baseline"] = cpu.gemv(name, wh, x_host, H, rows, synth.Q4_0, 4, wh.nbytes + 4 * H + 4 * rows)
        del wh

    # the headline GEMV through the code-object route: zg_kernels.hsaco loaded
    # with hipModuleLoad, each launch a hipModuleLaunchKernel (captured into
    # the graph like the library's launches)
    from zero_amd import module as zmod

    km = zmod.KernelModule()
    wh = synth.weight(rng, synth.Q4_0, ROWS, H, 4)
    wd, c = rotating(wh)
    yk = torch.empty(ROWS, device="cuda")

    def modl(i, st, wd=wd, yk=yk):
        km.gemv_x4(wd[i].data_ptr(), x.data_ptr(), yk.data_ptr(), ROWS, H, synth.Q4_0, stream=st)

    per, n, _ = _graph_time(modl, c, steps // 4, 40)
    out["module_q4_0x4_6144x2048"] = _row("Q4_0X4 6144x2048 through zg_kernels.hsaco (hipModuleLaunchKernel)", per,
                                          wh.nbytes + 4 * H + 4 * ROWS, n, c,
                                          entry=zmod.plan(synth.Q4_0, ROWS, H, km.cu_count).entry)
    del wd, wh
    km.close()

    # the same weights in the model's split-scale X4 device layout
    # (interleave 5: each group's quants, then its scales): the headline shape
    # and the LM-head height, the same strip kernel with one 16-byte quant load
    # and one contiguous scale load per lane
    for name, key, rows in (("Q4_0 split-scale X4 6144x2048 (the model's layout of the headline weights)",
                             "q4_0_split_6144x2048", 6144),
                            ("Q4_0 split-scale X4 151936x2048", "q4_0_split_151936x2048", 151_936)):
        wh = synth.x4_split(synth.weight(rng, synth.Q4_0, rows, H, 4), rows, H, synth.Q4_0)
        wd, c = rotating(wh)
        yk = torch.empty(rows, device="cuda")

        def spl(i, st, wd=wd, yk=yk, rows=rows):
            ctx.linear_dev(x, wd[i], yk, H, rows, synth.Q4_0, 5, stream=st)

        per, n, _ = _graph_time(spl, c, max(40, steps // (4 if rows < 16384 else 20)), 8 if rows > 16384 else 40)
        out[key] = _row(name, per, wh.nbytes + 4 * H + 4 * rows, n, c)
        del wd, wh

    # k-quants at Llama-3-8B FFN shapes
    for name, qt, rows, k in (("Q4_K 14336x4096 (gate/up)", synth.Q4K, 14336, 4096),
                              ("Q6_K 4096x14336 (down)", synth.Q6K, 4096, 14336)):
        wh = synth.weight(rng, qt, rows, k, 1)
        wd, c = rotating(wh)
        xk_host = synth.activations(rng, k)
        xk = torch.from_numpy(xk_host).cuda()
        yk = torch.empty(rows, device="cuda")

        def kq(i, st, wd=wd, xk=xk, yk=yk, qt=qt, rows=rows, k=k):
            ctx.linear_dev(xk, wd[i], yk, k, rows, qt, 1, stream=st)

        per, n, _ = _graph_time(kq, c, max(40, steps // 10), 20)
        key = "q4_k_14336x4096" if qt == synth.Q4K else "q6_k_4096x14336"
        out[key] = _row(name, per, wh.nbytes + 4 * k + 4 * rows, n, c)
        if cpu:
            out[key]["cpu_baseline"] = cpu.gemv(name, wh, xk_host, k, rows, qt, 1, wh.nbytes + 4 * k + 4 * rows)
        if qt == synth.Q4K:
            # the same weights through the Q8_K integer path: quantize_row_q8k
            # of x, then the integer GEMV (two launches per call)
            q8 = torch.empty(k // 256 * 292, dtype=torch.uint8, device="cuda")

            def kq8(i, st, wd=wd, xk=xk, yk=yk, rows=rows, k=k, q8=q8):
                ctx.quantize_q8k_dev(xk, q8, k, stream=st)
                ctx.linear_q4k_q8k_dev(q8, wd[i], yk, k, rows, stream=st)

            per8, n8, _ = _graph_time(kq8, c, max(40, steps // 10), 20)
            out["q4_k_q8_k_14336x4096"] = _row("Q4_K x Q8_K integer path 14336x4096 (quantize + GEMV)", per8,
                                               wh.nbytes + 4 * k + k // 256 * 292 + 4 * rows, n8, c)
            if cpu:
                # the reference's default Q4_K kernel (its VNNI path is
                # feature-gated off by default)
                out["q4_k_q8_k_14336x4096"]["cpu_baseline"] = out[key]["cpu_baseline"]
        del wd

    # prefill GEMM, M = 512, both FFN shapes, Q4_0X4 weights, Q8_0 activations
    M = 512
    for name, n_out, k in (("up", 6144, 2048), ("down", 2048, 6144)):
        wh = synth.weight(rng, synth.Q4_0, n_out, k, 4)
        wd = torch.from_numpy(wh).cuda()
        xm_host = synth.activations(rng, M, k)
        xm = torch.from_numpy(xm_host).cuda()
        qs = torch.empty((M, k), dtype=torch.int8, device="cuda")
        dd = torch.empty((M, k // 32), dtype=torch.int16, device="cuda")
        ym = torch.empty((M, n_out), device="cuda")
        ctx.quantize_q8_0_split_dev(xm, qs, dd, M, k)

        def gemm(i, st, wd=wd, qs=qs, dd=dd, ym=ym, n_out=n_out, k=k):
            ctx.gemm_q8act_dev(qs, dd, wd, ym, M, n_out, k, synth.Q4_0, 4, stream=st)

        def quant(i, st, xm=xm, qs=qs, dd=dd, k=k):
            ctx.quantize_q8_0_split_dev(xm, qs, dd, M, k, stream=st)

        # 16 launches per graph replay, so that the replay's own cost is
        # spread over them (operands stay resident: the GEMM is MFMA-bound)
        per, n, _ = _graph_time(gemm, 16, max(64, steps // 20), 16)
        perq, _, _ = _graph_time(quant, 16, max(64, steps // 20), 16)
        ops = 2 * M * n_out * k
        tops = ops / (per * 1e-3) / 1e12
        nbytes = wh.nbytes + M * k + M * (k // 32) * 2 + 4 * M * n_out
        out[f"prefill_gemm_{name}"] = {
            "workload": f"prefill GEMM M=512 x {n_out}x{k} Q4_0X4, Q8_0 activations, int8 MFMA",
            "us_per_launch": round(per * 1e3, 2), "int8_TOPS": round(tops, 1),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4), "ops_per_launch": ops, "bytes_per_launch": nbytes,
            "quantize_us": round(perq * 1e3, 2)}
        log(f"prefill GEMM {name}: {per * 1e3:.1f} us, {tops:.0f} TOPS; quantize {perq * 1e3:.1f} us")
        if cpu:
            out[f"prefill_gemm_{name}"]["cpu_baseline"] = cpu.prefill(f"{n_out}x{k} Q4_0X4 (fp32 x rows)", wh,
                                                                      xm_host, k, n_out, synth.Q4_0, 4, M)
        del wd

    # K-quant prefill GEMM, M = 512, the Qwen3-1.7B Q4_K_M FFN shapes: Q4_K
    # gate / up 6144x2048 and Q6_K down 2048x6144, Q8_K activations
    for name, qt, n_out, k in (("q4k_up", synth.Q4K, 6144, 2048), ("q6k_down", synth.Q6K, 2048, 6144)):
        wh = synth.weight(rng, qt, n_out, k, 1)
        wd = torch.from_numpy(wh).cuda()
        xm_host = synth.activations(rng, M, k)
        xm = torch.from_numpy(xm_host).cuda()
        qs = torch.empty((M, k), dtype=torch.int8, device="cuda")
        d8 = torch.empty((M, k // 256), dtype=torch.float32, device="cuda")
        bs = torch.empty((M, k // 32), dtype=torch.int16, device="cuda")
        ym = torch.empty((M, n_out), device="cuda")
        ctx.quantize_q8k_split_dev(xm, qs, d8, bs, M, k)

        def kgemm(i, st, wd=wd, qs=qs, d8=d8, bs=bs, ym=ym, qt=qt, n_out=n_out, k=k):
            ctx.gemm_q8k_dev(qs, d8, bs, wd, ym, M, n_out, k, qt, stream=st)

        def kquant(i, st, xm=xm, qs=qs, d8=d8, bs=bs, k=k):
            ctx.quantize_q8k_split_dev(xm, qs, d8, bs, M, k, stream=st)

        per, n, _ = _graph_time(kgemm, 16, max(64, steps // 20), 16)
        perq, _, _ = _graph_time(kquant, 16, max(64, steps // 20), 16)
        ops = 2 * M * n_out * k
        tops = ops / (per * 1e-3) / 1e12
        nbytes = wh.nbytes + M * k + M * (k // 256) * 4 + M * (k // 32) * 2 + 4 * M * n_out
        tname = "Q4_K" if qt == synth.Q4K else "Q6_K"
        out[f"prefill_gemm_{name}"] = {
            "workload": f"prefill GEMM M=512 x {n_out}x{k} {tname}, Q8_K activations, int8 MFMA",
            "us_per_launch": round(per * 1e3, 2), "int8_TOPS": round(tops, 1),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4), "ops_per_launch": ops, "bytes_per_launch": nbytes,
            "quantize_us": round(perq * 1e3, 2)}
        log(f"prefill GEMM {name}: {per * 1e3:.1f} us, {tops:.0f} TOPS; Q8_K quantize {perq * 1e3:.1f} us")
        if cpu:
            out[f"prefill_gemm_{name}"]["cpu_baseline"] = cpu.prefill(f"{n_out}x{k} {tname} (fp32 x rows)", wh,
                                                                      xm_host, k, n_out, qt, 1, M)
        del wd
    return out


def bench_read_floor(ctx, steps: int):
    """The floor the GEMVs are measured against: one launch that streams the
    same number of weight bytes and computes nothing (zg_read_floor_dev),
    graph-replayed over rotating copies like the headline.  Each size is
    timed with 1, 2, 4 and 8 128-bit loads per thread; the fastest is the
    floor.  Then the Q4_0X4 strip GEMV's load pattern without its decode
    (zg_strip_loads_dev) at the C1 and LM-head heights."""
    import torch

    out = {}
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for key, nbytes, what in (("read_floor_7077888B", 7_077_888, "the C1 Q4_0X4 6144x2048 weights"),
                              ("read_floor_33030144B", 33_030_144, "Q4_K 14336x4096 weights"),
                              ("read_floor_48168960B", 48_168_960, "Q6_K 4096x14336 weights"),
                              ("read_floor_175646208B", 175_646_208, "Q4_0X4 151936x2048 weights")):
        c = _copies(nbytes)
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i & 0x7F) for i in range(c)]
        per_u = {}
        for u in (1, 2, 4, 8):
            def rd(i, st, u=u):
                ctx.read_floor_dev(bufs[i], nbytes, u, sink, stream=st)

            per, n, _ = _graph_time(rd, c, max(40, steps // (4 if nbytes < 1 << 24 else 40)), c)
            per_u[u] = per
        best_u = min(per_u, key=per_u.get)
        out[key] = _row(f"read floor: {nbytes} B ({what}), best of 1/2/4/8 loads per thread", per_u[best_u],
                        nbytes, n, c, loads_per_thread=best_u,
                        us_by_loads_per_thread={u: round(v * 1e3, 3) for u, v in per_u.items()})
        del bufs
    # the strip GEMV's load pattern alone (zg_strip_loads_dev): the one-batch
    # form at C1's 6144 rows and the batch-loop form at 151,936 rows, weights
    # only and with each lane's x quarters
    import numpy as np

    from zero_amd import synth

    x = torch.from_numpy(synth.activations(np.random.default_rng(5), 2048)).cuda()
    for key, rows, what in (("strip_loads_6144x2048", 6144, "C1 form: one batch of 3 groups per workgroup"),
                            ("strip_loads_151936x2048", 151_936, "tall form: 4-group batches, two in flight")):
        nbytes = rows * 2048 // 32 * 18
        c = _copies(nbytes)
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i & 0x7F) for i in range(c)]
        per_x = {}
        for with_x in (False, True):
            def ld(i, st, with_x=with_x):
                ctx.strip_loads_dev(bufs[i], rows, x if with_x else None, sink, stream=st)

            per, n, _ = _graph_time(ld, c, max(40, steps // (4 if nbytes < 1 << 24 else 40)), c)
            per_x[with_x] = per
        out[key] = _row(f"Q4_0X4 strip GEMV loads without the decode, {rows}x2048 ({what}), weights only",
                        per_x[False], nbytes, n, c, us_with_x_quarters=round(per_x[True] * 1e3, 3))
        log(f"  with the x quarters: {per_x[True] * 1e3:.2f} us")
        del bufs
    return out


def _profile_workloads(ctx, names, reps: int):
    """Eager launches (no graph) of named workloads, for rocprofv3 counter
    passes: each dispatch of a kernel gets its own counters.  Weights rotate
    over copies larger than the Infinity Cache, as in the timed rows."""
    import numpy as np
    import torch

    from zero_amd import synth

    rng = np.random.default_rng(11)
    H = 2048
    x = torch.from_numpy(synth.activations(rng, 16384)).cuda()

    def rotating(w_host):
        c = _copies(w_host.nbytes)
        w0 = torch.from_numpy(w_host).cuda()
        return [w0] + [w0.clone() for _ in range(c - 1)]

    def run(name, launch, n_rot):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(reps):
            launch(i % n_rot)
        torch.cuda.synchronize()
        log(f"profile {name}: {reps} eager launches, {(time.perf_counter() - t0) / reps * 1e6:.1f} us wall each")

    for name in names:
        if name == "copy":  # known-size reference for FETCH_SIZE / WRITE_SIZE: 256 MiB read, 256 MiB written
            src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
            dst = torch.empty_like(src)
            run(name, lambda i: torch.add(src, 1, out=dst), 1)
            del src, dst
        elif name in ("c1", "tall"):
            rows = 6144 if name == "c1" else 151_936
            wd = rotating(synth.weight(rng, synth.Q4_0, rows, H, 4))
            y = torch.empty(rows, device="cuda")
            run(name, lambda i: ctx.linear_dev(x, wd[i], y, H, rows, synth.Q4_0, 4), len(wd))
            del wd
        elif name in ("floor_c1", "floor_tall"):
            nbytes = 7_077_888 if name == "floor_c1" else 175_646_208
            bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i & 0x7F)
                    for i in range(_copies(nbytes))]
            sink = torch.zeros(1, dtype=torch.int32, device="cuda")
            for u in (1, 2, 4, 8):
                run(f"{name} x{u}", lambda i, u=u: ctx.read_floor_dev(bufs[i], nbytes, u, sink), len(bufs))
            del bufs
        elif name == "lmhead":
            V = 151_936
            wd = rotating(synth.weight(rng, synth.Q8_0, V, H, 4))
            logits = torch.empty(V, device="cuda")
            best = torch.zeros(1, dtype=torch.int64, device="cuda")
            run(name, lambda i: ctx.lm_head_dev(x, wd[i], logits, H, V, synth.Q8_0, 4, best), len(wd))
            del wd
        elif name == "qkv":
            segs = [(2048, synth.weight(rng, synth.Q8_0, 2048, H, 4)), (1024, synth.weight(rng, synth.Q8_0, 1024, H, 4)),
                    (1024, synth.weight(rng, synth.Q8_0, 1024, H, 4))]
            c = _copies(sum(w.nbytes for _, w in segs))
            sd = [[torch.from_numpy(w).cuda() for _, w in segs]]
            sd += [[t.clone() for t in sd[0]] for _ in range(c - 1)]
            ys = [torch.empty(n, device="cuda") for n, _ in segs]
            run(name, lambda i: ctx.linear_fused_dev(
                x, [(sd[i][j], ys[j], segs[j][0], synth.Q8_0, 4) for j in range(3)], H), c)
            del sd
        elif name in ("q4k", "q6k"):
            qt, rows, k = (synth.Q4K, 14336, 4096) if name == "q4k" else (synth.Q6K, 4096, 14336)
            wd = rotating(synth.weight(rng, qt, rows, k, 1))
            y = torch.empty(rows, device="cuda")
            run(name, lambda i: ctx.linear_dev(x, wd[i], y, k, rows, qt, 1), len(wd))
            del wd
        elif name in ("gemm_up", "gemm_down"):
            M = 512
            n_out, k = (6144, 2048) if name == "gemm_up" else (2048, 6144)
            wd = torch.from_numpy(synth.weight(rng, synth.Q4_0, n_out, k, 4)).cuda()
            xm = torch.from_numpy(synth.activations(rng, M, k)).cuda()
            qs = torch.empty((M, k), dtype=torch.int8, device="cuda")
            dd = torch.empty((M, k // 32), dtype=torch.int16, device="cuda")
            ym = torch.empty((M, n_out), device="cuda")
            ctx.quantize_q8_0_split_dev(xm, qs, dd, M, k)
            run(name, lambda i: ctx.gemm_q8act_dev(qs, dd, wd, ym, M, n_out, k, synth.Q4_0, 4), 1)
        elif name in ("kgemm_up", "kgemm_down"):
            M = 512
            qt, n_out, k = (synth.Q4K, 6144, 2048) if name == "kgemm_up" else (synth.Q6K, 2048, 6144)
            wd = torch.from_numpy(synth.weight(rng, qt, n_out, k, 1)).cuda()
            xm = torch.from_numpy(synth.activations(rng, M, k)).cuda()
            qs = torch.empty((M, k), dtype=torch.int8, device="cuda")
            d8 = torch.empty((M, k // 256), dtype=torch.float32, device="cuda")
            bs = torch.empty((M, k // 32), dtype=torch.int16, device="cuda")
            ym = torch.empty((M, n_out), device="cuda")
            ctx.quantize_q8k_split_dev(xm, qs, d8, bs, M, k)
            run(name, lambda i: ctx.gemm_q8k_dev(qs, d8, bs, wd, ym, M, n_out, k, qt), 1)
        elif name == "decode":
            # the decode bench's model and lengths, with the step's kernels
            # launched directly (no graph replay under the profiler); reps
            # does not apply
            from zero_amd.model import GpuModel
            n_prompt, n_gen = 128, 256
            cfg = synth.ModelConfig(max_ctx=n_prompt + n_gen)
            model = synth.random_model(cfg, seed=0)
            gm = GpuModel(ctx, model)
            prompt = synth.prompt(1, n_prompt, cfg.vocab_real)
            t0 = time.perf_counter()
            gm.generate(prompt, n_gen, eager=True)
            log(f"profile decode: {n_prompt}-token prompt + {n_gen} tokens eager in {time.perf_counter() - t0:.1f} s")
            gm.close()
            ctx.clear()
        else:
            raise SystemExit(f"unknown profile workload {name!r}")


def _plain_copy(model):
    """The model with plain row-major layer linears and LM head."""
    import dataclasses

    from zero_amd import synth

    c = model.cfg
    shapes = {"attn_q": (c.q_dim, c.hidden), "attn_k": (c.kv_dim, c.hidden), "attn_v": (c.kv_dim, c.hidden),
              "attn_o": (c.hidden, c.q_dim), "ffn_gate": (c.ffn, c.hidden), "ffn_up": (c.ffn, c.hidden),
              "ffn_down": (c.hidden, c.ffn)}
    out = synth.RandomModel(dataclasses.replace(c, lin_interleave=1, head_interleave=1),
                            token_embd=model.token_embd.copy(), output_norm=model.output_norm,
                            lm_head=synth.deinterleave_x4(model.lm_head, c.vocab_padded, c.hidden, c.head_type))
    for L in model.layers:
        out.layers.append(dataclasses.replace(
            L, **{k: synth.deinterleave_x4(getattr(L, k), r, kk, c.lin_type) for k, (r, kk) in shapes.items()}))
    return out


def bench_decode(ctx, n_prompt=128, n_gen=256, seed=0):
    import numpy as np

    from zero_amd import synth
    from zero_amd.model import GpuModel

    cfg = synth.ModelConfig(max_ctx=n_prompt + n_gen)
    t0 = time.time()
    model = synth.random_model(cfg, seed)
    log(f"decode: random-init Qwen3-1.7B-shape model generated in {time.time() - t0:.1f}s")
    gm = GpuModel(ctx, model)
    prompt = synth.prompt(seed + 1, n_prompt, cfg.vocab_real)
    gm.generate(prompt, 8)  # warm-up (first graph launches)
    toks, t_pre, t_gen = gm.generate(prompt, n_gen)
    tok_s = (n_gen - 1) / t_gen
    # the same prompt through the batched int8-MFMA prefill (Q8_0 activations)
    gm.generate(prompt, 8, batched_prefill=True)  # warm-up (row buffers, first launches)
    toks_b, t_pre_b, t_gen_b = gm.generate(prompt, n_gen, batched_prefill=True)
    agree = int(np.argmin(np.concatenate([toks_b == toks, [False]])))
    # mean algorithmic bytes per decode step over contexts t = n_prompt+1 .. n_prompt+n_gen-1
    kv_per_pos = 2 * cfg.n_layers * cfg.kv_dim * 4
    norms = (2 * cfg.n_layers * cfg.hidden + 2 * cfg.n_layers * cfg.head_dim + cfg.hidden) * 4
    ctxs = np.arange(n_prompt + 1, n_prompt + n_gen)
    per_tok = cfg.weight_bytes_per_token() + norms + float(np.mean(ctxs)) * kv_per_pos + kv_per_pos
    gm.close()
    # the same weights in the packer's default v1 layout (plain rows for the
    # layer linears and the LM head)
    plain = _plain_copy(model)
    gp = GpuModel(ctx, plain)
    gp.generate(prompt, 8)
    toks_p, _, t_gen_p = gp.generate(prompt, n_gen)
    agree_p = int(np.argmin(np.concatenate([toks_p == toks, [False]])))
    gp.close()
    del plain
    # the reference's default dispatch (GGUF Q4_K_M pattern): Q4_K
    # projections with Q6_K attn_v / ffn_down on 14 of the 28 layers, Q4_K
    # token embedding, Q6_K LM head
    kcfg = synth.ModelConfig(max_ctx=n_prompt + n_gen, embd_type=synth.Q4K, head_type=synth.Q6K, head_interleave=1,
                             layer_quants=synth.q4_k_m_layers(cfg.n_layers))
    kmodel = synth.random_model(kcfg, seed)
    gk = GpuModel(ctx, kmodel)
    gk.generate(prompt, 8)
    toks_k, t_pre_k, t_gen_k = gk.generate(prompt, n_gen)
    # the same prompt through the batched prefill (Q8_K rows, K-quant GEMMs)
    gk.generate(prompt, 8, batched_prefill=True)
    toks_kb, t_pre_kb, _ = gk.generate(prompt, 8, batched_prefill=True)
    gk.close()
    k_bytes = kcfg.weight_bytes_per_token() + norms + float(np.mean(ctxs)) * kv_per_pos + kv_per_pos
    del kmodel
    return {"tok_s": tok_s, "ms_per_token": 1e3 / tok_s, "prefill_tok_s": n_prompt / t_pre,
            "batched_prefill": {"prefill_tok_s": n_prompt / t_pre_b, "prefill_ms": t_pre_b * 1e3,
                                "decode_tok_s": (n_gen - 1) / t_gen_b, "tokens_equal_to_token_by_token": agree},
            "plain_layout": {"decode_tok_s": (n_gen - 1) / t_gen_p, "tokens_equal_to_x4": agree_p},
            "q4_k_m": {"decode_tok_s": (n_gen - 1) / t_gen_k, "bytes_per_token": int(k_bytes),
                       "gbs": k_bytes * (n_gen - 1) / t_gen_k / 1e9, "prefill_tok_s": n_prompt / t_pre_k,
                       "batched_prefill_tok_s": n_prompt / t_pre_kb, "batched_prefill_ms": t_pre_kb * 1e3,
                       "batched_first_token_equal": bool(toks_kb[0] == toks_k[0])},
            "n_prompt": n_prompt,
            "n_gen": n_gen, "bytes_per_token": int(per_tok), "gbs": per_tok * tok_s / 1e9,
            "first_tokens": [int(t) for t in toks[:8]], "model": model, "prompt": prompt}


CPU_ROTATE_BYTES = 1 << 30  # host copies per CPU leg: above any host last-level cache


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class CpuBaseline:
    """The reference's CPU path on this host: the AVX-512 intrinsics
    restatement of its range kernels (oracle/zg_avx512.c), split with
    row_range_for(align = interleave) over one pinned worker per core of the
    process's CPU share, as the reference's SMP dispatch splits rows over
    every active core (smp.rs:1282-1296, 1567-1712).  The share is the
    affinity mask, capped by OMP_NUM_THREADS where the host sets it (the GPU
    host grants 16 cores per GPU).  Each leg rotates over host copies of its
    weights totalling >= 1 GiB, so every call streams from DRAM."""

    def __init__(self, seconds: float = 2.0):
        from oracle import zo

        self.zo = zo
        self.seconds = seconds
        aff = len(os.sched_getaffinity(0))
        share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        self.affinity = aff
        self.threads = min(aff, share) if share > 0 else aff
        self.model = _cpu_model()
        self.pool = zo.Pool(self.threads)
        self.simd = zo.set_simd(True)
        self.kind = "port"

    def close(self):
        self.zo.set_simd(False)
        self.zo.load().zo_pool_stop()

    def _desc(self):
        kern = "AVX-512 intrinsics" if self.simd else "scalar lane-order C (no AVX-512F on this host)"
        return (f"{kern} restatement of the reference range kernels, row_range_for split over {self.pool.n} "
                f"pinned threads of a {self.affinity}-CPU affinity mask, {self.model}")

    def _result(self, value, unit, sample):
        return {"value": value, "unit": unit, "cores": self.pool.n, "kind": self.kind,
                "cpu_model": self.model, "sample": f"{sample}; {self._desc()}"}

    def _timed(self, call, n_copies):
        call(0)  # first touch of the pool and the first copy
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < self.seconds:
            call(n % n_copies)
            n += 1
        return n, time.perf_counter() - t0

    @staticmethod
    def _copies(w_host):
        c = max(2, math.ceil(CPU_ROTATE_BYTES / w_host.nbytes))
        return [w_host] + [w_host.copy() for _ in range(c - 1)]

    def gemv(self, name, w_host, x, k, rows, quant, il, nbytes):
        """GB/s of algorithmic bytes for the same GEMV as a GPU row."""
        import numpy as np

        ws = self._copies(w_host)
        out = np.empty(rows, np.float32)
        n, dt = self._timed(lambda i: self.zo.linear_parallel(x, ws[i], k, rows, quant, il, out=out), len(ws))
        return self._result(nbytes * n / dt / 1e9, "GB/s",
                            f"{n} {name} GEMVs over {len(ws)} rotating copies "
                            f"({len(ws) * w_host.nbytes >> 20} MiB) in {dt:.1f}s")

    def fused(self, name, segs, x, k, nbytes):
        import numpy as np

        n_c = max(2, math.ceil(CPU_ROTATE_BYTES / sum(w.nbytes for _, w, _, _ in segs)))
        sets = [[(w if c == 0 else w.copy(), r, q, il) for r, w, q, il in segs] for c in range(n_c)]
        outs = [np.empty(r, np.float32) for r, _, _, _ in segs]
        n, dt = self._timed(lambda i: self.zo.linear_fused_parallel(
            x, [(w, r, q, il) for w, r, q, il in sets[i]], k, outs), n_c)
        return self._result(nbytes * n / dt / 1e9, "GB/s",
                            f"{n} {name} fused dispatches over {n_c} rotating copies in {dt:.1f}s")

    def lm_head(self, name, w_host, x, k, rows, quant, il, nbytes):
        import numpy as np

        ws = self._copies(w_host)
        logits = np.empty(rows, np.float32)
        n, dt = self._timed(lambda i: self.zo.lm_head_parallel(x, ws[i], k, rows, quant, il, logits), len(ws))
        return self._result(nbytes * n / dt / 1e9, "GB/s",
                            f"{n} {name} GEMV + argmax calls over {len(ws)} rotating copies in {dt:.1f}s")

    def prefill(self, name, w_host, xm, k, rows, quant, il, m):
        """The reference prefills token by token: one GEMV per prompt row.
        Rate = 2*m*rows*k ops over the time of m GEMVs (fp32 FMAs, in the
        GPU GEMM's unit), on a bounded sample of rows."""
        import numpy as np

        ws = self._copies(w_host)
        out = np.empty(rows, np.float32)
        n, dt = self._timed(lambda i: self.zo.linear_parallel(xm[i % m], ws[i], k, rows, quant, il, out=out),
                            len(ws))
        per_gemv = dt / n
        tops = 2.0 * rows * k / per_gemv / 1e12
        return self._result(tops, "TOPS (2*M*N*K fp32 ops)",
                            f"{n} of the M={m} per-row GEMVs {name} in {dt:.1f}s over {len(ws)} rotating copies "
                            f"(M GEMVs per GEMM: {m * per_gemv * 1e3:.1f} ms)")

    def decode(self, model, prompt, n_gen, max_gen_seconds=20.0):
        """forward_single_token over the same random-init model: the prompt
        token by token (as the reference prefills), then greedy tokens until
        n_gen or the time bound; tok/s over the generated steps."""
        zo = self.zo
        om = zo.OracleModel(model)
        t0 = time.perf_counter()
        for i, t in enumerate(prompt):
            om.forward(int(t), i)
        rc, tok, _, _ = om.lm_head()
        t1 = time.perf_counter()
        pos, steps = len(prompt), 0
        while steps < n_gen - 1 and time.perf_counter() - t1 < max_gen_seconds:
            om.forward(tok, pos)
            pos += 1
            steps += 1
            rc, tok, _, _ = om.lm_head()
        t2 = time.perf_counter()
        om.close()
        return self._result(steps / (t2 - t1), "tok/s",
                            f"{len(prompt)}-token prompt token by token ({len(prompt) / (t1 - t0):.1f} tok/s, "
                            f"{t1 - t0:.1f}s), then {steps} greedy steps in {t2 - t1:.1f}s "
                            f"(cap {n_gen - 1} steps or {max_gen_seconds:.0f}s), same random-init Qwen3-1.7B-shape "
                            f"model")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-rows", action="store_true", help="skip the fused-QKV, LM-head, k-quant and GEMM lines")
    ap.add_argument("--profile", default="",
                    help="comma list of workloads to launch eagerly (no graph) for rocprofv3 counter passes, "
                         "then exit: c1, tall, floor_c1, floor_tall, lmhead, qkv, q4k, q6k, gemm_up, gemm_down, kgemm_up, "
                         "kgemm_down, copy")
    ap.add_argument("--profile-reps", type=int, default=30)
    ap.add_argument("--pmc-calib", action="store_true",
                    help="first run one elementwise kernel that reads 256 MiB and writes 256 MiB, the "
                         "known-size reference for FETCH_SIZE/WRITE_SIZE counter scaling")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import zero_amd

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    ctx = zero_amd.Context(0)
    torch.cuda.synchronize()
    if args.profile:
        _profile_workloads(ctx, [n for n in args.profile.split(",") if n], args.profile_reps)
        ctx.close()
        return
    if args.pmc_calib:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.add(src, 1, out=dst)  # one kernel: reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst
    g = bench_gemv(ctx, args.steps, args.warmup)
    log(f"gemv: {g['launches']} launches, {g['ms_per_gemv'] * 1e3:.2f} us/GEMV, {g['gbs']:.0f} GB/s")
    out = {
        "metric": METRIC,
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["launches"],
        "warmup": g["warmup"],
        "ms_per_step": g["ms_per_gemv"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Q4_0X4 GEMV 6144x2048 (Qwen3-1.7B FFN up-proj), x fp32, y fp32",
                   "rotating_weight_copies": g["copies"], "bytes_per_step": GEMV_BYTES},
        "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": GEMV_TRAFFIC_BYTES},
    }
    cpu = None if args.no_cpu else CpuBaseline()
    if cpu:
        out["cpu_baseline"] = cpu.gemv("Q4_0X4 6144x2048", g["w_host"], g["x_host"], K, ROWS, 2, 4, GEMV_BYTES)
        log(f"cpu: {out['cpu_baseline']['value']:.1f} GB/s on {cpu.pool.n} threads ({cpu.model})")
    if not args.no_rows:
        out["rows"] = bench_rows(ctx, args.steps, cpu)
        out["rows"].update(bench_read_floor(ctx, args.steps))
    dec = None
    if not args.no_decode:
        dec = bench_decode(ctx)
        log(f"decode: {dec['tok_s']:.1f} tok/s ({dec['gbs']:.0f} GB/s effective)")
        bp = dec["batched_prefill"]
        log(f"batched prefill: {bp['prefill_ms']:.2f} ms for {dec['n_prompt']} tokens "
            f"({bp['prefill_tok_s']:.0f} tok/s; token by token {dec['prefill_tok_s']:.0f} tok/s)")
        log(f"decode, plain v1 layout: {dec['plain_layout']['decode_tok_s']:.1f} tok/s")
        log(f"decode, Q4_K_M pattern: {dec['q4_k_m']['decode_tok_s']:.1f} tok/s ({dec['q4_k_m']['gbs']:.0f} GB/s); "
            f"batched prefill {dec['q4_k_m']['batched_prefill_ms']:.2f} ms "
            f"({dec['q4_k_m']['batched_prefill_tok_s']:.0f} tok/s; token by token "
            f"{dec['q4_k_m']['prefill_tok_s']:.0f} tok/s)")
        out["decode"] = {"tok_s": round(dec["tok_s"], 2), "ms_per_token": dec["ms_per_token"],
                         "prefill_tok_s": round(dec["prefill_tok_s"], 2),
                         "batched_prefill": {k: (round(v, 2) if isinstance(v, float) else v)
                                             for k, v in dec["batched_prefill"].items()},
                         "plain_layout": {k: (round(v, 2) if isinstance(v, float) else v)
                                          for k, v in dec["plain_layout"].items()},
                         "q4_k_m": {k: (round(v, 2) if isinstance(v, float) else v)
                                    for k, v in dec["q4_k_m"].items()},
                         "workload": "random-init Qwen3-1.7B shape, Q4_0X4 linears, Q8_0X4 LM head, "
                                     f"{dec['n_prompt']}-token prompt then {dec['n_gen']} greedy tokens",
                         "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1), "peak": HBM_PEAK_GBS,
                                      "unit": "GB/s", "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                                      "bytes_per_token": dec["bytes_per_token"]}}
        if cpu:
            cd = cpu.decode(dec["model"], dec["prompt"], dec["n_gen"])
            log(f"cpu decode: {cd['value']:.1f} tok/s")
            out["decode"]["cpu_baseline"] = cd
    if cpu:
        cpu.close()
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
