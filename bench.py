"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (`value`): Q4_0X4 GEMV at the Qwen3-1.7B FFN up-proj shape
(6144 x 2048, fp32 x), HBM GB/s of algorithmic bytes, weights rotating over
> 512 MB of copies so every launch streams from HBM (the 256 MB Infinity
Cache cannot hold the set).  A step is one GEMV launch; steps are replayed
from a HIP graph so that host launch cost is not timed.

Also reported: batch-1 greedy decode tok/s of a random-init
Qwen3-1.7B-shaped model (128-token prompt, then 256 tokens), and the CPU
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
ROWS, K = 6144, 2048
# W (6144 x 2048 Q4_0 = 7,077,888 B) + x fp32 (8,192 B) + y fp32 (24,576 B)
GEMV_BYTES = ROWS * (K // 32) * 18 + 4 * K + 4 * ROWS
ROTATE_BYTES = 512 << 20
# HBM bytes per launch of the GEMV kernel, from rocprofv3 --pmc FETCH_SIZE
# (3,538.5 KiB x 2.00) and WRITE_SIZE (24.0 KiB x 1.00); the factors come from
# the same counters read on an elementwise kernel that reads and writes 256 MiB
# (--pmc-calib).  1.02 x GEMV_BYTES: the weights are read exactly once.
GEMV_TRAFFIC_BYTES = 7_271_424


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def bench_gemv(ctx, steps: int, warmup: int):
    import numpy as np
    import torch

    from zero_amd import synth

    rng = np.random.default_rng(0)
    w_host = synth.weight(rng, synth.Q4_0, ROWS, K, 4)
    copies = math.ceil(ROTATE_BYTES / w_host.nbytes) + 1
    w_dev = [torch.from_numpy(w_host).cuda() for _ in range(copies)]
    x = torch.from_numpy(synth.activations(rng, K)).cuda()
    y = torch.empty(ROWS, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    # all GEMVs run on one side stream: it is captured into a graph, and the
    # timing events are recorded on it
    stream = torch.cuda.Stream()
    st = stream.cuda_stream

    def launch_all():
        for w in w_dev:
            ctx.linear_dev(x, w, y, K, ROWS, synth.Q4_0, 4, stream=st)

    with torch.cuda.stream(stream):
        launch_all()  # eager warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        launch_all()
    reps = max(1, math.ceil(steps / copies))
    wreps = max(1, math.ceil(warmup / copies))
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
    n = reps * copies
    per = ms / n
    gbs = GEMV_BYTES / (per * 1e-3) / 1e9
    del g
    return {"launches": n, "warmup": wreps * copies, "copies": copies, "ms_per_gemv": per, "gbs": gbs,
            "w_host": w_host, "x_host": x.cpu().numpy()}


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
    # mean algorithmic bytes per decode step over contexts t = n_prompt+1 .. n_prompt+n_gen-1
    kv_per_pos = 2 * cfg.n_layers * cfg.kv_dim * 4
    norms = (2 * cfg.n_layers * cfg.hidden + 2 * cfg.n_layers * cfg.head_dim + cfg.hidden) * 4
    ctxs = np.arange(n_prompt + 1, n_prompt + n_gen)
    per_tok = cfg.weight_bytes_per_token() + norms + float(np.mean(ctxs)) * kv_per_pos + kv_per_pos
    gm.close()
    return {"tok_s": tok_s, "ms_per_token": 1e3 / tok_s, "prefill_tok_s": n_prompt / t_pre, "n_prompt": n_prompt,
            "n_gen": n_gen, "bytes_per_token": int(per_tok), "gbs": per_tok * tok_s / 1e9,
            "first_tokens": [int(t) for t in toks[:8]], "model": model, "prompt": prompt}


def cpu_gemv(w_host, x, seconds=5.0):
    import numpy as np

    from oracle import zo

    copies = math.ceil(ROTATE_BYTES / w_host.nbytes) + 1
    ws = [w_host.copy() for _ in range(copies)]
    threads = min(16, os.cpu_count() or 1)
    n = 0
    with zo.Pool(threads) as pool:
        zo.linear_parallel(x, ws[0], K, ROWS, 2, 4)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            zo.linear_parallel(x, ws[n % copies], K, ROWS, 2, 4)
            n += 1
        dt = time.perf_counter() - t0
        used = pool.n
    return {"value": GEMV_BYTES * n / dt / 1e9, "unit": "GB/s", "cores": used, "kind": "port",
            "sample": f"{n} Q4_0X4 6144x2048 GEMVs over {copies} rotating copies ({copies * w_host.nbytes >> 20} MiB), "
                      f"{dt:.1f}s wall, row_range_for split align 4 over {used} pinned threads"}


def cpu_decode(model, n_prompt=16, n_gen=32):
    from oracle import zo

    threads = min(16, os.cpu_count() or 1)
    with zo.Pool(threads) as pool:
        om = zo.OracleModel(model)
        prompt = model_prompt = list(range(1, n_prompt + 1))
        t0 = time.perf_counter()
        for i, t in enumerate(prompt):
            om.forward(t, i)
        rc, tok, _, _ = om.lm_head()
        t1 = time.perf_counter()
        pos = n_prompt
        for _ in range(n_gen - 1):
            om.forward(tok, pos)
            pos += 1
            rc, tok, _, _ = om.lm_head()
        t2 = time.perf_counter()
        om.close()
        used = pool.n
    del model_prompt
    return {"value": (n_gen - 1) / (t2 - t1), "unit": "tok/s", "cores": used, "kind": "port",
            "sample": f"{n_prompt}-token prompt ({t1 - t0:.1f}s) then {n_gen} greedy tokens, tok/s over the "
                      f"{n_gen - 1} decode steps ({t2 - t1:.1f}s), same random-init Qwen3-1.7B-shape model"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
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
    dec = None
    if not args.no_decode:
        dec = bench_decode(ctx)
        log(f"decode: {dec['tok_s']:.1f} tok/s ({dec['gbs']:.0f} GB/s effective)")
        out["decode"] = {"tok_s": round(dec["tok_s"], 2), "ms_per_token": dec["ms_per_token"],
                         "prefill_tok_s": round(dec["prefill_tok_s"], 2),
                         "workload": "random-init Qwen3-1.7B shape, Q4_0X4 linears, Q8_0X4 LM head, "
                                     f"{dec['n_prompt']}-token prompt then {dec['n_gen']} greedy tokens",
                         "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1), "peak": HBM_PEAK_GBS,
                                      "unit": "GB/s", "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                                      "bytes_per_token": dec["bytes_per_token"]}}
    if not args.no_cpu:
        cb = cpu_gemv(g["w_host"], g["x_host"])
        log(f"cpu: {cb['value']:.1f} GB/s on {cb['cores']} threads")
        out["cpu_baseline"] = cb
        if dec is not None:
            cd = cpu_decode(dec["model"])
            log(f"cpu decode: {cd['value']:.1f} tok/s")
            out["decode"]["cpu_baseline"] = cd
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
