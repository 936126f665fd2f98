"""Benchmark of the MI355X int4 GPTQ decode hot path (one GPU).

Workloads
  gemv    the per-layer int4 GEMV sweep at M=1 with act-order (QKV 4096x6144,
          O 4096x4096, gate_up 4096x24576, down 12288x4096, group 128); one step
          = the four GEMVs of one layer.  Weight copies are rotated so that more
          than 640 MB of distinct weights stream per cycle (MI355X's 256 MB
          Infinity Cache cannot serve repeats).
Prints ONE JSON line (rank 0).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode steps/s at bs=1; int4 GEMV HBM GB/s as % of ~8 TB/s peak"
HBM_PEAK_GBS = 8000.0
GEMV_SHAPES = (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576),
               ("down", 12288, 4096))
GROUP = 128


def algo_bytes(m: int, k: int, n: int, g: int, act_order: bool) -> int:
    """Algorithmic HBM bytes of one int4 GEMM launch (AutoGPTQ layout)."""
    return (n * k // 2 + 2 * n * k // g + n * k // (2 * g) + (4 * k if act_order else 0)
            + 2 * m * k + 2 * m * n)


def make_gptq_weights(torch, dev, k, n, g, seed, act_order=True):
    """Random AutoGPTQ weights of the benchmark distribution, generated on the device."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    qweight = torch.randint(-2**31, 2**31 - 1, (k // 8, n), dtype=torch.int32, device=dev,
                            generator=gen)
    scales = (torch.rand(k // g, n, device=dev, generator=gen) * 0.018 + 0.002).half()
    z = torch.randint(6, 10, (k // g, n), dtype=torch.int32, device=dev, generator=gen)
    zw = torch.zeros(k // g, n // 8, dtype=torch.int64, device=dev)
    for j in range(8):
        zw |= (z[:, j::8].long() & 0xF) << (4 * j)
    qzeros = (((zw + 2**31) % 2**32) - 2**31).to(torch.int32)
    g_idx = None
    if act_order:
        perm = torch.randperm(k, device=dev, generator=gen)
        g_idx = torch.empty(k, dtype=torch.int32, device=dev)
        g_idx[perm] = (torch.arange(k, device=dev) // g).int()
    return qweight, qzeros, scales, g_idx


def bench_gemv(args, torch, pkg):
    from moss_tts_lite_amd import _native as N
    from moss_tts_lite_amd import ops

    dev = torch.device("cuda:0")
    shapes = []
    for name, k, n in GEMV_SHAPES:
        per_copy = algo_bytes(1, k, n, GROUP, True)
        copies = max(2, math.ceil(640e6 / per_copy))
        ws = []
        for c in range(copies):
            qw, qz, sc, g_idx = make_gptq_weights(torch, dev, k, n, GROUP, seed=1234 + 97 * c + k + n)
            qws, perm = ops.actorder_prepare(qw, g_idx, GROUP)
            del qw
            ws.append((qws, qz, sc, perm))
        x = torch.randn(1, k, device=dev, generator=torch.Generator(device=dev).manual_seed(7)).bfloat16()
        y = torch.empty(1, n, dtype=torch.bfloat16, device=dev)
        ops.reserve_workspace(dev, ops.gemm_workspace_bytes(1, k, n, GROUP))
        shapes.append(dict(name=name, k=k, n=n, copies=ws, x=x, y=y, bytes=per_copy))
    torch.cuda.synchronize()

    def launch(s, i):
        qws, qz, sc, perm = s["copies"][i % len(s["copies"])]
        ops.w4_gemm(s["x"], qws, N.META_GPTQ, sc, qz, perm, s["n"], GROUP, out=s["y"])

    for i in range(args.warmup):
        for s in shapes:
            launch(s, i)
    torch.cuda.synchronize()

    # The step loop replays a hipGraph of `cycle` steps (one per weight copy of the
    # deepest rotation), so host launch overhead is out of the timed region.
    cycle = max(len(s["copies"]) for s in shapes)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(cycle):
            for s in shapes:
                launch(s, i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(cycle):
            for s in shapes:
                launch(s, i)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(args.steps / cycle))
    steps = reps * cycle
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / steps

    # Per-kernel durations: event pairs around single launches on the launch stream,
    # queued behind a GPU spin so the host never starves the queue.
    per = {}
    for s in shapes:
        nrep = max(20, 4 * len(s["copies"]))
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(nrep)]
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2e8))
        for i, (a, b) in enumerate(evs):
            a.record()
            launch(s, i)
            b.record()
        torch.cuda.synchronize()
        us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
        mean_us = sum(us) / len(us)
        per[s["name"]] = dict(us=round(mean_us, 3), median_us=round(us[len(us) // 2], 3),
                              gbs=round(s["bytes"] / mean_us / 1e3, 1),
                              frac=round(s["bytes"] / mean_us / 1e3 / HBM_PEAK_GBS, 4),
                              copies=len(s["copies"]))
    step_bytes = sum(s["bytes"] for s in shapes)
    gu = per["gate_up"]
    return dict(
        value=round(step_bytes / (ms_step * 1e-3) / 1e9, 1), unit="GB/s", ms_per_step=ms_step,
        steps=steps,
        dtype="int4 weights, bf16 x, fp32 accumulate",
        config={"workload": "int4 GEMV sweep M=1 act-order g128: qkv 4096x6144, o 4096x4096, "
                            "gate_up 4096x24576, down 12288x4096 (one step = one layer's 4 GEMVs)",
                "per_kernel": per, "step_bytes": step_bytes},
        roofline={"bound": "hbm", "achieved": gu["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": gu["frac"], "traffic": None,
                  "kernel": "w4_gemm_kernel<1,16,GPTQ,perm> gate_up 4096x24576 M=1"},
    )


def cpu_baseline_gemv(budget_s: float = 12.0):
    """The oracle's port of the reference CPU path on the gate_up shape: dequantise
    (effective weight) then an fp32 x @ W, timed on this host's cores."""
    import numpy as np

    from oracle import synth

    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        threads = 1
    k, n = 4096, 24576
    case = synth.gptq_case(k=k, n=n, m=1, group=GROUP, act_order=True, seed=1234, with_ref=False)
    x = case["x_bits"].astype(np.uint32) << 16
    x = x.view(np.float32)
    times = []
    t_end = time.time() + budget_s
    while time.time() < t_end or not times:
        t = time.perf_counter()
        synth.chunked_gptq_gemm(x, case["qweight"], case["qzeros"], case["scales"], case["g_idx"],
                                GROUP, chunk=4096)
        times.append(time.perf_counter() - t)
    best = sorted(times)[len(times) // 2]
    gbs = algo_bytes(1, k, n, GROUP, True) / best / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"gate_up 4096x24576 M=1 act-order, {len(times)} calls, median "
                      f"{best * 1e3:.0f} ms/call (numpy dequant + BLAS matmul)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gemv", choices=["gemv"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__

    pkg = __graft_entry__.import_package()
    res = bench_gemv(args, torch, pkg)
    cpu = None if args.no_cpu_baseline else cpu_baseline_gemv()
    line = {
        "metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": res["steps"], "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"],
        "data": "synthetic (seeded random codes/scales/zeros, act-order permutation)",
        "config": res["config"], "roofline": res["roofline"], "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
