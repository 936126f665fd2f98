"""Benchmark of the MI355X int4 GPTQ decode hot path (one GPU).

Workloads
  decode  (default) the full random-init 36-layer Qwen3-8B-shaped int4 backbone
          (hidden 4096, 32/8 heads, head_dim 128, SwiGLU 12288, act-order g128 GPTQ
          projections) plus a bf16 head 151936x4096: prefill 256 random token ids,
          then hipGraph-replayed greedy decode steps, the KV cache growing to 1280
          (W warmup + K timed steps = 1024 by default); one step = one token.
  gemv    the per-layer int4 GEMV sweep at M=1 with act-order (QKV 4096x6144,
          O 4096x4096, gate_up 4096x24576, down 12288x4096, group 128); one step
          = the four GEMVs of one layer.  Weight copies are rotated so that more
          than 640 MB of distinct weights stream per cycle (MI355X's 256 MB
          Infinity Cache cannot serve repeats).
  skinny  the skinny-batch int4 GEMM on gate_up 4096x24576 and down 12288x4096 (group 128,
          no act-order) at M = 1, 2, 4, 8, 16 rows: the full-K strip GEMM and the split-K
          GEMM, mean us per launch over rotated weight copies (gate_up is also part of the
          gemv workload's line).
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
# decode positions of the benchmark workload: prefill 256, then 1024 steps (KV 257 -> 1280)
CONFIG4_POSITIONS = (256, 1279)
GEMV_SHAPES = (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576),
               ("down", 12288, 4096))
GROUP = 128


COPY_BYTES = 256 << 20


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


def module_gemv_sweep(torch, dev, steps: int, warmup: int, with_split_k: bool = False) -> dict:
    """The GPTQ module at one row (GPTQLinear.forward, M = 1, act-order g128) on the four
    decode shapes, weight copies rotated so no launch finds its weights in the caches:
    the full-K strip GEMV over the strip copy with x gathered through the act-order index
    while staging.  The sweep (one layer's four GEMVs per step) replays a hipGraph of
    module calls, so host overhead is out of the timed region; per-shape durations replay
    a hipGraph of that shape's calls alone, back to back over its weight copies (as the
    decode workload times its GEMVs).  ``with_split_k`` also times the split-K GEMM over
    the AutoGPTQ layout on every shape (event pairs around single launches)."""
    from moss_tts_lite_amd import _native as N
    from moss_tts_lite_amd import ops
    from moss_tts_lite_amd.gptq import GPTQLinear

    shapes = []
    for name, k, n in GEMV_SHAPES:
        per_copy = algo_bytes(1, k, n, GROUP, True)
        copies = max(2, math.ceil(640e6 / per_copy))
        mods = []
        for c in range(copies):
            qw, qz, sc, g_idx = make_gptq_weights(torch, dev, k, n, GROUP, seed=1234 + 97 * c + k + n)
            lin = GPTQLinear.from_buffers(qw, qz, sc, g_idx, GROUP).post_init()
            if with_split_k:
                lin.drop_original()
            else:
                lin.keep_strip_only()
            mods.append(lin)
        x = torch.randn(1, k, device=dev, generator=torch.Generator(device=dev).manual_seed(7)).bfloat16()
        ops.reserve_workspace(dev, ops.gemm_workspace_bytes(1, k, n, GROUP))
        shapes.append(dict(name=name, k=k, n=n, mods=mods, x=x, bytes=per_copy))
    torch.cuda.synchronize()

    def launch(s, i):
        s["mods"][i % len(s["mods"])](s["x"])

    def launch_split_k(s, i):
        qws, qz, sc, perm = s["mods"][i % len(s["mods"])].kernel_args()
        ops.w4_gemm(s["x"], qws, N.META_GPTQ, sc, qz, perm, s["n"], GROUP)

    for i in range(warmup):
        for s in shapes:
            launch(s, i)
    torch.cuda.synchronize()
    cycle = max(len(s["mods"]) for s in shapes)
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
    reps = max(1, math.ceil(steps / cycle))
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    sweep_us = t0.elapsed_time(t1) * 1e3 / (reps * cycle)

    def event_us(s, fn):
        nrep = max(20, 4 * len(s["mods"]))
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(nrep)]
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2e8))
        for i, (a, b) in enumerate(evs):
            a.record()
            fn(s, i)
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) * 1e3 for a, b in evs)

    def back_to_back_us(s):
        calls = len(s["mods"]) * max(1, math.ceil(64 / len(s["mods"])))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(calls):
                launch(s, i)
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(4):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (4 * calls)

    per = {}
    for s in shapes:
        us = back_to_back_us(s)
        per[s["name"]] = dict(us=round(us, 3), gbs=round(s["bytes"] / us / 1e3, 1),
                              frac=round(s["bytes"] / us / 1e3 / HBM_PEAK_GBS, 4),
                              copies=len(s["mods"]))
        if with_split_k:
            sk = event_us(s, launch_split_k)
            per[s["name"]]["split_k_us"] = round(sum(sk) / len(sk), 3)
    step_bytes = sum(s["bytes"] for s in shapes)
    return {"workload": "GPTQ module forward at one row (GPTQLinear, act-order g128): qkv "
                        "4096x6144, o 4096x4096, gate_up 4096x24576, down 12288x4096 on the "
                        "full-K strip GEMV with the act-order gather while staging",
            "sweep_us": round(sweep_us, 3), "sweep_gbs": round(step_bytes / sweep_us / 1e3, 1),
            "per_shape": per, "step_bytes": step_bytes}


def bench_gemv(args, torch, pkg):
    dev = torch.device("cuda:0")
    sweep = module_gemv_sweep(torch, dev, args.steps, args.warmup, with_split_k=True)
    skinny = bench_skinny(args, torch, dev)
    gu = sweep["per_shape"]["gate_up"]
    ms_step = sweep["sweep_us"] / 1e3
    return dict(
        value=sweep["sweep_gbs"], unit="GB/s", ms_per_step=ms_step, steps=args.steps,
        dtype="int4 weights, bf16 x, fp32 accumulate",
        config={"workload": sweep["workload"] + " (one step = one layer's 4 GEMVs; "
                            "split_k_us: the split-K GEMM on every shape)",
                "per_kernel": sweep["per_shape"], "step_bytes": sweep["step_bytes"],
                "skinny_gate_up": skinny},
        roofline={"bound": "hbm", "achieved": gu["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": gu["frac"], "traffic": None,
                  "kernel": "w4_strip_kernel<g128, PERM, STORE> gate_up 4096x24576 M=1, "
                            "act-order gather (event-timed single calls)"},
    )


def bench_skinny(args, torch, dev, k=4096, n=24576):
    """Skinny-batch int4 GEMM on one shape (default gate_up: K 4096, N 24576; group 128, no
    act-order) at M = 1, 2, 4, 8, 16 bf16 rows, one launch per call, weight copies rotated
    past the Infinity Cache, mean us per launch: the full-K strip GEMM (no partials) and the
    split-K GEMM (partials reduced by a second kernel)."""
    from moss_tts_lite_amd import _native as N
    from moss_tts_lite_amd import ops

    per_copy = algo_bytes(1, k, n, GROUP, False)
    copies = []
    for c in range(max(2, math.ceil(640e6 / per_copy))):
        qw, qz, sc, _ = make_gptq_weights(torch, dev, k, n, GROUP, seed=4321 + 13 * c, act_order=False)
        copies.append((qw, ops.strip_weights(qw), qz, sc))
    lib = N.load()
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for kind in ("strip_rows", "split_k"):
        res = {}
        for m in (1, 2, 4, 8, 16):
            x = torch.randn(m, k, device=dev, generator=torch.Generator(device=dev).manual_seed(m)).bfloat16()
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            ops.reserve_workspace(dev, ops.gemm_workspace_bytes(m, k, n, GROUP))

            def launch(i):
                qw, qs, qz, sc = copies[i % len(copies)]
                if kind == "split_k":
                    ops.w4_gemm(x, qw, N.META_GPTQ, sc, qz, None, n, GROUP, out=y)
                else:
                    N.check(lib.mtl_w4_gemm_strip_rows(x.data_ptr(), m, k, k, qs.data_ptr(),
                                                       sc.data_ptr(), qz.data_ptr(), n, GROUP, 0,
                                                       y.data_ptr(), n, N.OUT_BF16, stream),
                            "strip rows")

            for i in range(len(copies)):
                launch(i)
            reps = 4 * len(copies)
            a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            torch.cuda._sleep(int(2e8))
            a_ev.record()
            for i in range(reps):
                launch(i)
            b_ev.record()
            torch.cuda.synchronize()
            us = a_ev.elapsed_time(b_ev) * 1e3 / reps
            byts = algo_bytes(m, k, n, GROUP, False)
            res[f"M{m}"] = dict(us=round(us, 3), gbs=round(byts / us / 1e3, 1),
                                frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4),
                                tflops=round(2 * m * k * n / us / 1e6, 2))
        out[kind] = res
    del copies
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """All threads of this process's CPU share: OMP_NUM_THREADS when set, else the
    affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def _median_s(fn, budget_s: float, max_runs: int = 20) -> tuple[float, int]:
    """Median wall time of ``fn`` over up to ``max_runs`` runs (at least 3) after warm-up
    runs (3, or 1 when one run exceeds a fifth of the budget), stopping at ``budget_s``."""
    t = time.perf_counter()
    fn()
    first = time.perf_counter() - t
    for _ in range(0 if first > budget_s / 5 else 2):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (len(times) < max_runs and time.perf_counter() < t_end):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_linear_datapoints(torch, shapes, budget_s: float = 1.2) -> dict:
    """The reference's CPU int4 linear (oracle/cpu_path.py: effective_weight dequant then an
    fp32 x @ W.T, tests/test_quant.py:104-107) and torch's CPU int4 GEMM
    (_weight_int4pack_mm_for_cpu) on each (name, K, N) shape at M = 1, g = 128, seeded
    codes and qsz, at 1 thread and at all of this process's threads: median microseconds
    (20 runs, or fewer within the per-datapoint time budget, at least 3)."""
    from oracle import cpu_path as C

    n_all = _cpu_threads()
    saved = torch.get_num_threads()
    gen = torch.Generator().manual_seed(1234)
    out = {}
    for name, k, n in shapes:
        q = torch.randint(0, 16, (n, k), dtype=torch.int32, generator=gen)
        qsz = torch.stack([torch.rand(k // GROUP, n, generator=gen) * 0.018 + 0.002,
                           torch.rand(k // GROUP, n, generator=gen) * 0.2 - 0.1], 2).bfloat16()
        x = torch.randn(1, k, generator=gen).bfloat16()
        packed = C.pack_for_cpu(q)
        res = {}
        for threads in (1, n_all):
            torch.set_num_threads(threads)
            for label, fn in (("fp32", lambda: C.linear_fp32(x, q, qsz, GROUP)),
                              ("int4_cpu", lambda: C.int4pack_mm_cpu(x, packed, GROUP, qsz))):
                sec, runs = _median_s(fn, budget_s)
                res[f"{label}_{threads}t_us"] = round(sec * 1e6, 1)
                res[f"{label}_{threads}t_runs"] = runs
        res["bytes"] = algo_bytes(1, k, n, GROUP, False)
        out[name] = res
        del q, packed
    torch.set_num_threads(saved)
    return out


def cpu_baseline_gemv(torch, gpu_us: dict):
    """The reference's CPU path on the four decode-step shapes at M = 1 (value: GB/s of
    the fp32 path on gate_up at all threads), with torch's CPU int4 GEMM beside it."""
    n_all = _cpu_threads()
    per = cpu_linear_datapoints(torch, GEMV_SHAPES)
    for name, d in per.items():
        if name in gpu_us:
            d["gpu_speedup_vs_fp32_all"] = round(d[f"fp32_{n_all}t_us"] / gpu_us[name], 1)
    gu = per["gate_up"]
    return {"value": round(gu["bytes"] / gu[f"fp32_{n_all}t_us"] / 1e3, 3), "unit": "GB/s",
            "cores": n_all, "kind": "port", "cpu_model": _cpu_model(),
            "sample": f"gate_up 4096x24576 M=1 g128: effective_weight dequant + fp32 x @ W.T "
                      f"in torch on {n_all} threads (median of up to 20 calls)",
            "per_shape": per}


def bench_decode(args, torch):
    import numpy as np

    from moss_tts_lite_amd.fast import FastDecoder
    from moss_tts_lite_amd.model import BackboneConfig, Int4Backbone, random_weights

    dev = torch.device("cuda:0")
    prompt_len = 256
    total = prompt_len + args.warmup + args.steps
    cfg = BackboneConfig(max_seq=max(1536, ((total + 255) // 256) * 256), group_size=args.group)
    del total
    t0 = time.time()
    model = Int4Backbone(cfg, random_weights(cfg, seed=1234, device=dev, v_keep=args.v_keep), dev)
    if args.plan == "strip":        # one resident int4 copy per linear: the strip copy
        model.keep_strip_copies_only()
    dec = FastDecoder(model, plan=args.plan)
    gen = torch.Generator().manual_seed(1234)
    prompt = torch.randint(0, cfg.vocab, (prompt_len,), generator=gen)
    dec.prefill(prompt)
    dec.capture()
    torch.cuda.synchronize()
    setup_s = time.time() - t0
    gib = 1 << 30
    memory = {"int4_weight_gib": round(model.int4_weight_bytes() / gib, 3),
              "allocated_gib": round(torch.cuda.memory_allocated(dev) / gib, 3),
              "max_allocated_gib": round(torch.cuda.max_memory_allocated(dev) / gib, 3),
              "note": "torch allocator bytes on the device after set-up and at their peak "
                      "(random-init weights built on the device, prefill, graph capture)"}
    # the prompt: every token per launch (fast.py:251-270); the set-up run built the strip
    # copies, so this times the prefill itself (it leaves the same state: cache, pos, ids)
    pf_gpu, pf_wall = [], []
    for _ in range(3):
        a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        a_ev.record()
        dec.prefill(prompt)
        b_ev.record()
        torch.cuda.synchronize()
        pf_wall.append((time.perf_counter() - w0) * 1e3)
        pf_gpu.append(a_ev.elapsed_time(b_ev))
    for _ in range(args.warmup):
        dec.graph.replay()
    # The workload decodes at positions 256 .. 1279 (KV length 257 -> 1280). The timed
    # steps sit in the middle of that range, so their mean cost is the range's: untimed
    # greedy steps advance the cache there first.
    pos_now = int(dec.pos.item())
    start = max(pos_now, (CONFIG4_POSITIONS[0] + CONFIG4_POSITIONS[1] + 1) // 2 - args.steps // 2)
    start = min(start, max(pos_now, CONFIG4_POSITIONS[1] + 1 - args.steps))
    for _ in range(start - pos_now):
        dec.graph.replay()
    torch.cuda.synchronize()
    first_pos = int(dec.pos.item())
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    h0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        dec.graph.replay()
    e1.record()
    host_s = time.perf_counter() - h0
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    final_pos = int(dec.pos.item())

    # The whole range once more, every step timed (a second prompt, same state).
    dec.prefill(prompt)
    n_range = CONFIG4_POSITIONS[1] + 1 - int(dec.pos.item())
    torch.cuda.synchronize()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    for _ in range(n_range):
        dec.graph.replay()
    r1.record()
    torch.cuda.synchronize()
    range_ms = r0.elapsed_time(r1) / n_range

    # Dominant kernel, live: each int4 GEMV launch of the step exactly as the captured plan
    # issues it, over the model's own 36 layers (1.9 GB of distinct gate_up weights, so no
    # Infinity-Cache reuse): 144 launches back to back between one event pair on the
    # launch stream, queued behind a GPU spin so host launch overhead never shows.
    reps = 4 * cfg.n_layers
    gemv_us = {}
    for name in ("gate_up", "down", "qkv", "o"):
        a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2e8))
        a_ev.record()
        for i in range(reps):
            dec.run_gemv(i % cfg.n_layers, name)
        b_ev.record()
        torch.cuda.synchronize()
        gemv_us[name] = a_ev.elapsed_time(b_ev) * 1e3 / reps
    # the decode attention the same way (its q|k|v buffer as the last step left it), at the
    # middle of the range: cache length 768, the range's mean
    attn_pos = (CONFIG4_POSITIONS[0] + CONFIG4_POSITIONS[1]) // 2
    dec.pos.fill_(attn_pos)
    a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))
    a_ev.record()
    for i in range(reps):
        dec.run_attention(i % cfg.n_layers)
    b_ev.record()
    torch.cuda.synchronize()
    attention_us = {"us": round(a_ev.elapsed_time(b_ev) * 1e3 / reps, 3), "cache_length": attn_pos + 1,
                    "timing": "144 launches back to back over the 36 layers' caches, one event pair"}
    gu_us = gemv_us["gate_up"]
    gu_bytes = algo_bytes(1, cfg.hidden, 2 * cfg.intermediate, cfg.group_size, False)
    nv = cfg.n_kv_heads * cfg.head_dim
    layer_bytes = sum(algo_bytes(1, k, n, cfg.group_size, True) for k, n in
                      ((cfg.hidden, cfg.qkv_out - (nv if args.v_keep else 0)),
                       (cfg.hidden, cfg.hidden), (cfg.hidden, 2 * cfg.intermediate),
                       (cfg.intermediate, cfg.hidden)))
    if args.v_keep:                       # the kept v_proj streams bf16 weights
        layer_bytes += 2 * nv * cfg.hidden + 2 * cfg.hidden + 4 * nv
    # config 1: the GPTQ module's own one-row forward on the same four shapes
    module_gemv = module_gemv_sweep(torch, dev, steps=200, warmup=3)
    avg_len = (first_pos + 1 + final_pos) / 2
    kv_bytes = 2 * cfg.n_layers * cfg.n_kv_heads * cfg.head_dim * 2 * avg_len
    step_bytes = cfg.n_layers * layer_bytes + 2 * cfg.vocab * cfg.hidden + kv_bytes
    del np
    return dict(
        value=round(1000.0 / ms_step, 2), unit="steps/s", ms_per_step=ms_step, steps=args.steps,
        dtype="int4 GPTQ weights, bf16 activations, fp32 accumulate",
        config={"workload": f"36-layer Qwen3-8B-shaped int4 GPTQ backbone (act-order g{cfg.group_size}"
                            + (", v_proj kept bf16" if args.v_keep else "") + ") + bf16 "
                            "head 151936x4096, batch 1, prefill 256 random ids then hipGraph greedy "
                            f"decode at positions 256..1279 (KV 257->1280); the timed steps run at "
                            f"KV {first_pos + 1}->{final_pos}, the middle of that range",
                "config4_full_range": {"positions": f"256..{CONFIG4_POSITIONS[1]}",
                                       "steps": n_range, "ms_per_step": round(range_ms, 4),
                                       "steps_per_s": round(1000.0 / range_ms, 2)},
                "hidden": cfg.hidden, "layers": cfg.n_layers, "vocab": cfg.vocab,
                "step_bytes_avg": int(step_bytes),
                "step_hbm_gbs": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
                "host_enqueue_ms_per_step": round(host_s * 1e3 / args.steps, 4),
                "setup_s": round(setup_s, 1), "plan": dec.plan, "memory": memory,
                "prefill_ms": {"tokens": prompt_len, "gpu": round(min(pf_gpu), 3),
                               "wall": round(min(pf_wall), 3)},
                "gemv_us": {k: round(v, 3) for k, v in gemv_us.items()},
                "attention_us": attention_us,
                "module_gemv": module_gemv,
                "gemv_gbs": {k: round(algo_bytes(1, kk, nn, cfg.group_size, False) / gemv_us[k]
                                      / 1e3, 1) for k, kk, nn in
                             (("gate_up", cfg.hidden, 2 * cfg.intermediate),
                              ("down", cfg.intermediate, cfg.hidden),
                              ("qkv", cfg.hidden, cfg.qkv_out), ("o", cfg.hidden, cfg.hidden))}},
        roofline={"bound": "hbm", "achieved": round(gu_bytes / gu_us / 1e3, 1),
                  "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(gu_bytes / gu_us / 1e3 / HBM_PEAK_GBS, 4),
                  "traffic": (profiled_traffic("gate_up", dec.plan)
                              if cfg.group_size == GROUP and not args.v_keep else None),
                  "kernel": GATE_UP_KERNEL.get(dec.plan, "gate_up 4096x24576 M=1"),
                  "timing": "achieved and frac: the step's own gate|up launch, 144 launches "
                            "back to back over the 36 layers' weights between one HIP event "
                            "pair on the launch stream; in_step_trace: the same kernel's "
                            "average duration inside the graph-replayed step, from the "
                            "committed rocprofv3 kernel trace of this workload",
                  "in_step_trace": profiled_in_step("gate_up", dec.plan, gu_bytes)
                                   if cfg.group_size == GROUP and not args.v_keep else None,
                  "bytes_per_launch": gu_bytes},
    )


# The gate|up launch of each decode plan (the dominant kernel of the step).
GATE_UP_KERNEL = {
    "strip": "w4_strip_kernel<g128, RMSNORM, SILU, 8 blocks/wave, 2 strips> gate_up 4096x24576 "
             "M=1 (full-K strips, SiLU*up epilogue)",
    "staged": "w4_gemm_kernel<1,4,GPTQ,XSRC_RMSNORM> gate_up 4096x24576 M=1 (split-K partials)",
}


def profiled_traffic(name: str, plan: str):
    """HBM bytes per launch of one decode-step GEMV of that plan, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (copy-kernel calibrated); None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "gemv_traffic_decode_shapes.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"traffic_bytes {plan} {name}:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def profiled_in_step(name: str, plan: str, nbytes: int):
    """Average duration of one decode-step GEMV of that plan inside the graph-replayed step,
    from the committed rocprofv3 kernel trace (a line ``in_step_us <plan> <name>: <us>``),
    with the rate and roofline fraction it gives; None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "decode_step_36layer_kernel_trace.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"in_step_us {plan} {name}:"):
                    us = float(line.split(":")[1])
                    return {"us": us, "achieved": round(nbytes / us / 1e3, 1),
                            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
    except OSError:
        pass
    return None


def bench_kernels(args, torch):
    """Counter-collection workload: a plain 256 MiB device copy (the calibration kernel
    for the FETCH_SIZE / WRITE_SIZE counters), then each int4 GEMV of the decode step
    exactly as the captured plan launches it, over the model's 36 layers, --steps times."""
    from moss_tts_lite_amd.fast import FastDecoder
    from moss_tts_lite_amd.model import BackboneConfig, Int4Backbone, random_weights

    dev = torch.device("cuda:0")
    cfg = BackboneConfig(max_seq=1536)
    model = Int4Backbone(cfg, random_weights(cfg, seed=1234, device=dev), dev)
    dec = FastDecoder(model, plan=args.plan)
    dec.prefill(torch.randint(0, cfg.vocab, (16,), generator=torch.Generator().manual_seed(1)))
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for name in ("gate_up", "down", "qkv", "o"):
        for i in range(args.steps):
            dec.run_gemv(i % cfg.n_layers, name)
        torch.cuda.synchronize()
    print(json.dumps({"workload": "kernels", "copy_bytes": COPY_BYTES,
                      "gemv_launches_each": args.steps}))


def bench_prefill(args, torch):
    """Prompt-length int4 GEMMs (mtl_w4_gemm_prefill) on the decode shapes at M =
    --prefill-rows, random strip-layout weights, --steps launches each between one event
    pair; the whole prefill is timed by the decode workload (config.prefill_ms)."""
    from moss_tts_lite_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1234)
    m = args.prefill_rows
    shapes = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576),
              "down": (12288, 4096)}
    names = list(shapes) if args.prefill_shape == "all" else [args.prefill_shape]
    out = {}
    for name in names:
        k, n = shapes[name]
        qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 8, n), dtype=torch.int32, device=dev,
                           generator=gen)
        sc = (torch.rand(k // 128, n, device=dev, generator=gen) * 0.01 + 0.002).half()
        qz = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 128, n // 8), dtype=torch.int32,
                           device=dev, generator=gen)
        st = ops.strip_weights(qw)
        ssc, sqz = ops.strip_meta(sc, qz, 128)
        x = torch.randn(m, k, device=dev, generator=gen).bfloat16()
        y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        res = {}
        for split in ((True, False) if args.prefill_split == "auto" else (False,)):
            for _ in range(3):
                ops.prefill_gemm(x, st, ssc, sqz, n, 128, out=y, split=split)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            for _ in range(args.steps):
                ops.prefill_gemm(x, st, ssc, sqz, n, 128, out=y, split=split)
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / args.steps
            res["us" if split else "one_pass_us"] = round(us, 2)
            if split:
                res["tflops"] = round(2.0 * m * n * k / us / 1e6, 1)
        out[name] = res
    print(json.dumps({"workload": "prefill", "rows": m, "launches_each": args.steps,
                      "dtype": "int4 GPTQ weights, bf16 activations, fp32 accumulate",
                      "gemm": out}))


def cpu_baseline_decode(torch, gpu_us: dict):
    """The reference's CPU path for one decode step of the 36-layer model, timed per
    linear: each layer's four int4 linears at M = 1 through effective_weight + fp32 x @ W.T
    (oracle/cpu_path.py, tests/test_quant.py:104-107), plus a 16384-row slice of the bf16
    head (F.linear) scaled to 151936 rows. The step is 36 layers' linears and the head
    (norms, RoPE and attention are under 1 % of it). Also given: the same step with torch's
    CPU int4 GEMM, and every datapoint at 1 thread."""
    n_all = _cpu_threads()
    per = cpu_linear_datapoints(torch, GEMV_SHAPES)
    head = torch.randn(16384, 4096, generator=torch.Generator().manual_seed(5)).bfloat16() * 0.02
    hf = torch.randn(4096, generator=torch.Generator().manual_seed(6)).bfloat16()
    saved = torch.get_num_threads()
    steps = {}
    for threads in (1, n_all):
        torch.set_num_threads(threads)
        t_head = _median_s(lambda: torch.nn.functional.linear(hf, head), 1.0)[0] * 151936 / 16384
        for label in ("fp32", "int4_cpu"):
            t_layers = sum(d[f"{label}_{threads}t_us"] for d in per.values()) * 1e-6
            steps[f"{label}_{threads}t"] = round(1.0 / (36 * t_layers + t_head), 4)
    torch.set_num_threads(saved)
    for name, d in per.items():
        if name in gpu_us:
            d["gpu_speedup_vs_fp32_all"] = round(d[f"fp32_{n_all}t_us"] / gpu_us[name], 1)
            d["gpu_speedup_vs_int4_cpu_all"] = round(d[f"int4_cpu_{n_all}t_us"] / gpu_us[name], 1)
    return {"value": steps[f"fp32_{n_all}t"], "unit": "steps/s", "cores": n_all, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": "one decode step of the 36-layer model from per-linear timings: the four "
                      "decode-step linears at M=1 (effective_weight dequant + fp32 x @ W.T in "
                      f"torch, median of up to 20 calls each) x 36 + the bf16 head, on {n_all} "
                      "threads",
            "steps_per_s": steps, "per_shape": per}


def bench_int4_op(args, torch):
    """The reference's decode operator beside the mtl kernels, same GPU, graph-captured:
    ``torch._weight_int4pack_mm`` on torch's own packed weights (moss_tts_lite/fast.py:118,
    the reference's int4 linear) and the ``mtl_int4pack_mm`` drop-in, M = 1, g = 128, on
    the four decode-step projections.  Each timing replays a graph of ``steps`` launches
    rotating over enough weight copies (>= 400 MB) that no launch reads from the 256 MB
    Infinity Cache; eager calls are timed too (host and wall time per call), as the
    reference's non-captured paths issue them."""
    sys.path.insert(0, ROOT)
    import __graft_entry__
    __graft_entry__.import_package()
    from moss_tts_lite_amd import ops
    dev = torch.device("cuda:0")
    steps = args.steps or 96
    shapes = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
    gen = torch.Generator(device="cpu").manual_seed(11)
    out = {}
    for name, (k, n) in shapes.items():
        copies = int(400e6 // (k * n // 2)) + 1
        ws = []
        for _ in range(copies):
            c = torch.randint(0, 16, (n, k), generator=gen, dtype=torch.int32).to(dev)
            pre = (c[:, 1::2] | (c[:, 0::2] << 4)).to(torch.uint8).contiguous()
            qsz = torch.stack([torch.rand(k // 128, n, generator=gen) * 0.02 + 0.002,
                               torch.rand(k // 128, n, generator=gen) * 0.2 - 0.1],
                              2).to(torch.bfloat16).to(dev).contiguous()
            ws.append((torch.ops.aten._convert_weight_to_int4pack(pre, 8),
                       ops.convert_weight_to_int4pack(pre, 8), qsz))
            del c, pre
        x = torch.randn(1, k, generator=gen).to(torch.bfloat16).to(dev)
        res = {}
        for label, fn in (("torch_weight_int4pack_mm", lambda w: torch._weight_int4pack_mm(x, w[0], 128, w[2])),
                          ("mtl_int4pack_mm", lambda w: ops.weight_int4pack_mm(x, w[1], 128, w[2]))):
            for w in ws:
                fn(w)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(steps):
                    fn(ws[i % copies])
            g.replay()
            torch.cuda.synchronize()
            best = 1e9
            for _ in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                g.replay()
                b.record()
                torch.cuda.synchronize()
                best = min(best, a.elapsed_time(b) * 1e3 / steps)
            res[label] = round(best, 3)
            del g
            # eager calls: host time per call (the loop is enqueue-bound when it exceeds
            # the GPU time) and wall time per call with the final synchronize
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(200):
                fn(ws[i % copies])
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            res[label + "_eager_host_us"] = round((t1 - t0) / 200 * 1e6, 2)
            res[label + "_eager_wall_us"] = round((t2 - t0) / 200 * 1e6, 2)
        res["weight_mb"] = round(k * n / 2 / 1e6, 2)
        out[name] = res
        print(f"{name}: {res}", file=sys.stderr, flush=True)
        del ws
    print(json.dumps({"workload": "int4_op", "m": 1, "group": 128, "launches_each": steps,
                      "us_per_launch": out}))


# bf16 keeps of the reference's two shipped GPTQ presets (moss_tts_lite/export.py:59-72):
# w1 keeps every v_proj, w2 also up_proj of layers 6, 7, 9 and 35; both use group 32
MOSS_PRESETS = {"w1": [(li, "v") for li in range(36)],
                "w2": [(li, "v") for li in range(36)] + [(li, "up") for li in (6, 7, 9, 35)]}


def moss_records(torch, cfg, dev, keep, group, seed=1234):
    """Random-init weights of the MOSS backbone in the reference's record form: per linear
    ``{"packed": torch's int4 tiles [N/8, K/128, 32, 4], "qsz": bf16 [K/g, N, 2]}`` (the
    standalone export's records, moss_tts_lite/export.py:324-334), and the dense bf16
    weight of each kept linear. Codes uniform 0..15, scales U(0.002, 0.02), zero points
    (8 - z) * scale with z uniform 6..9, kept weights N(0, 0.02)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    h, d = cfg.hidden, cfg.head_dim
    shapes = {"q": (cfg.n_heads * d, h), "k": (cfg.n_kv_heads * d, h), "v": (cfg.n_kv_heads * d, h),
              "o": (h, cfg.n_heads * d), "gate": (cfg.intermediate, h), "up": (cfg.intermediate, h),
              "down": (h, cfg.intermediate)}
    keep = set(keep)
    layers, state = [], {}
    for li in range(cfg.n_layers):
        lw, rec = {}, {}
        for name, (n, k) in shapes.items():
            if (li, name) in keep:
                lw[name] = (torch.randn(n, k, device=dev, generator=gen) * 0.02).bfloat16()
                continue
            tiles = torch.randint(-2**31, 2**31 - 1, (n // 8, k // 128, 32, 4), dtype=torch.int32,
                                  device=dev, generator=gen)
            sc = torch.rand(k // group, n, device=dev, generator=gen) * 0.018 + 0.002
            z = torch.randint(6, 10, (k // group, n), device=dev, generator=gen)
            rec[name] = {"packed": tiles, "qsz": torch.stack([sc, (8 - z) * sc], -1).bfloat16()}
        layers.append(lw)
        state[li] = rec
    return layers, state


def moss_generation_rates(torch, dec, prompt_rows, steps: int) -> dict:
    """Whole generation steps per second (step + sampling + state machine) from an audio
    continuation prompt (the last text id AUDIO_START): the device generator
    (moss_tts_lite_amd.generate.generate_fast: sampling on the device, one host read per step
    behind the next step's backbone), and the reference's read pattern (generate_fast,
    moss_tts_lite/fast.py:487-539: every sampled token read to the host with int(), the next
    id row copied back) over the same decoder and the same device sampling ops."""
    from moss_tts_lite_amd import generate as G

    rows = prompt_rows.clone()
    rows[-1, 0] = G.AUDIO_START_TOKEN_ID
    prompt = {"input_ids": rows[None]}
    kw = dict(max_new_tokens=steps, seed=1234, watchdog=False)
    G.generate_fast(dec, prompt, **dict(kw, max_new_tokens=8))          # warm-up
    st = {}
    res = G.generate_fast(dec, prompt, stats=st, **kw)
    out = {"steps": res.n_steps, "device_sampling_steps_per_s": round(res.n_steps / st["wall_s"], 1),
           "host_wait_ms_per_step": round(st["host_wait_s"] * 1e3 / res.n_steps, 3)}
    # the reference's pattern: the same step and sampling ops, then a host read of every token
    dev = dec.dev
    n_vq = dec.m.cfg.n_vq
    dec.prefill(rows)
    torch.cuda.synchronize()
    pos, al = rows.shape[0], 1
    t0 = time.perf_counter()
    for t in range(steps):
        if t:
            dec.step(None, pos, audio2=True)
            pos += 1
        two = dec.two / 1.5
        text = G.sample_rows(two.view(1, -1), top_k=50, top_p=1.0)[0]
        nxt = [G.AUDIO_GEN_SLOT_TOKEN_ID if int(text) == 0 else G.AUDIO_DELAY_SLOT_TOKEN_ID]
        la = dec.la / 1.7
        act = min(al, n_vq)
        toks = G.sample_rows(la[:act].clone(), top_k=25, top_p=0.8)
        nxt += [int(toks[j]) for j in range(act)] + [G.AUDIO_PAD_CODE] * (n_vq - act)
        dec.ids.copy_(torch.tensor(nxt, dtype=torch.int64).to(dev))
        al += 1
    torch.cuda.synchronize()
    out["host_reads_steps_per_s"] = round(steps / (time.perf_counter() - t0), 1)
    return out


def bench_moss(args, torch):
    """The MOSS-TTS decode step at the reference's shape (moss_tts_lite/model.py:9-24: Qwen3-8B
    backbone, text vocabulary 155648, 32 audio codebooks of 1025) on the reference's own
    weight records: a shipped preset's group size and bf16 keeps, (packed, qsz) records
    through W4Dispatch and layers_from_dispatch, qsz read in place by the strip kernels.
    Prefill 256 random id rows, then graph replays of the text-head variant at host-given
    positions (FastMossDecoder.step, the reference's FastMossTTS.step contract), timed in
    the middle of positions 256..1279."""
    from moss_tts_lite_amd.fast import FastMossDecoder
    from moss_tts_lite_amd.gptq import W4Dispatch
    from moss_tts_lite_amd.model import Int4Backbone, layers_from_dispatch, moss_config

    dev = torch.device("cuda:0")
    group = 32
    keep = MOSS_PRESETS[args.preset]
    cfg = moss_config(group_size=group, act_order=False, max_seq=1536)
    t0 = time.time()
    layers, state = moss_records(torch, cfg, dev, keep, group)
    disp = W4Dispatch(layers, w4_group_size=group, bf16_keep=keep, state=state, device=dev)
    del state
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    h = cfg.hidden

    def normal(*shape, std):
        return (torch.randn(*shape, device=dev, generator=gen) * std).bfloat16()

    def norm_w(n):
        return (1.0 + torch.randn(n, device=dev, generator=gen) * 0.05).bfloat16()

    norms = [{"input_layernorm": norm_w(h), "post_attention_layernorm": norm_w(h),
              "q_norm": norm_w(cfg.head_dim), "k_norm": norm_w(cfg.head_dim)}
             for _ in range(cfg.n_layers)]
    w = {"embed_tokens": normal(cfg.text_embed_rows, h, std=1.0), "final_norm": norm_w(h),
         "head": normal(cfg.vocab, h, std=0.02), "layers": layers_from_dispatch(disp, norms),
         "emb_ext": [normal(cfg.audio_vocab, h, std=1.0) for _ in range(cfg.n_vq)],
         "head_audio": normal(cfg.n_vq, cfg.audio_vocab, h, std=0.02)}
    del disp, layers
    model = Int4Backbone(cfg, w, dev)
    del w
    dec = FastMossDecoder(model)
    g = torch.Generator().manual_seed(1234)
    prompt_len = 256
    rows = torch.cat([torch.randint(0, cfg.vocab, (prompt_len, 1), generator=g),
                      torch.randint(0, cfg.audio_vocab - 1, (prompt_len, cfg.n_vq), generator=g)], 1)
    dec.prefill(rows)
    dec.capture()
    torch.cuda.synchronize()
    setup_s = time.time() - t0
    # the 256-row prompt on the prefill GEMMs (the set-up run built the strip copies; a
    # prefill rewrites the same cache rows)
    pf_gpu = []
    for _ in range(3):
        a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a_ev.record()
        dec.prefill(rows)
        b_ev.record()
        torch.cuda.synchronize()
        pf_gpu.append(a_ev.elapsed_time(b_ev))
    row = rows[-1].to(dev)
    mid = (CONFIG4_POSITIONS[0] + CONFIG4_POSITIONS[1] + 1) // 2
    start = max(prompt_len, min(mid - args.steps // 2, CONFIG4_POSITIONS[1] + 1 - args.steps))
    for p in range(prompt_len, start):             # untimed steps fill the cache up to there
        dec.step(row, p)
    for i in range(args.warmup):
        dec.step(row, start + i % max(1, args.steps))
    res = {}
    for audio2 in (False, True):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            dec.step(row, start + i, audio2)
        e1.record()
        torch.cuda.synchronize()
        res[audio2] = e0.elapsed_time(e1) / args.steps
    ms_step = res[False]
    launches = sum(len(p) for p in dec._layers) + len(dec._embed) + len(dec._final_variant(False))
    gen_rates = moss_generation_rates(torch, dec, rows, steps=384)
    return dict(
        value=round(1000.0 / ms_step, 2), unit="steps/s", ms_per_step=ms_step, steps=args.steps,
        dtype="int4 (packed, qsz) weights, bf16 activations, fp32 accumulate",
        config={"workload": f"MOSS-TTS decode step, preset {args.preset} (group {group}, bf16 "
                            f"keeps: {len(keep)} linears): 36-layer Qwen3-8B backbone on the "
                            "reference's (packed, qsz) records, 33-way summed embedding, text "
                            "head 155648x4096 + 32 audio heads of 1025; prefill 256 rows, then "
                            f"graph replays at host-given positions {start}..{start + args.steps - 1}",
                "ms_per_step_audio2": round(res[True], 4),
                "steps_per_s_audio2": round(1000.0 / res[True], 2),
                "launches_per_step": launches, "setup_s": round(setup_s, 1),
                "prefill_ms": {"rows": prompt_len, "gpu": round(min(pf_gpu), 3)},
                "reference_a10g_steps_per_s": {"w1": 81.5, "w2": 78.6}[args.preset],
                "generation": gen_rates},
        roofline=None,
    )


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "gemv", "skinny", "kernels", "prefill", "int4-op", "moss"])
    ap.add_argument("--preset", default="w2", choices=sorted(MOSS_PRESETS),
                    help="the reference's GPTQ preset: group size and bf16 keeps (moss workload)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--group", type=int, default=128, choices=[32, 64, 128, 256],
                    help="int4 group size of every projection (decode workload)")
    ap.add_argument("--v-keep", action="store_true",
                    help="keep v_proj in bf16, as the shipped GPTQ presets do (decode workload)")
    ap.add_argument("--plan", default="strip",
                    choices=["strip", "fused", "staged", "partials", "unfused"],
                    help="decode launch plan (decode workload)")
    ap.add_argument("--prefill-rows", type=int, default=256, help="M (prefill workload)")
    ap.add_argument("--prefill-shape", default="all",
                    choices=["all", "qkv", "o", "gate_up", "down"], help="(prefill workload)")
    ap.add_argument("--prefill-split", default="auto", choices=["auto", "off"],
                    help="K split of small grids, or one pass only (prefill workload)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the package has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__

    pkg = __graft_entry__.import_package()
    if args.workload == "kernels":
        args.steps = 72 if args.steps is None else args.steps
        bench_kernels(args, torch)
        return
    if args.workload == "skinny":
        dev = torch.device("cuda:0")
        print(json.dumps({"workload": "skinny", "group": GROUP,
                          "gate_up 4096x24576": bench_skinny(args, torch, dev),
                          "down 12288x4096": bench_skinny(args, torch, dev, 12288, 4096)}))
        return
    if args.workload == "int4-op":
        return bench_int4_op(args, torch)
    if args.workload == "prefill":
        args.steps = 20 if args.steps is None else args.steps
        bench_prefill(args, torch)
        return
    if args.workload == "moss":
        args.warmup = 16 if args.warmup is None else args.warmup
        args.steps = 256 if args.steps is None else args.steps
        res = bench_moss(args, torch)
        print(json.dumps({"metric": "MOSS-TTS decode steps/s at bs=1", "value": res["value"],
                          "unit": res["unit"], "n_gpus": 1, "steps": res["steps"],
                          "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 6),
                          "higher_is_better": True, "dtype": res["dtype"],
                          "data": "synthetic: random-init records and weights, random id rows",
                          "config": res["config"]}))
        return
    if args.workload == "decode":
        args.warmup = 16 if args.warmup is None else args.warmup
        args.steps = 1024 - args.warmup if args.steps is None else args.steps
        res = bench_decode(args, torch)
        cpu = None if args.no_cpu_baseline else cpu_baseline_decode(torch,
                                                                    res["config"]["gemv_us"])
    else:
        args.warmup = 20 if args.warmup is None else args.warmup
        args.steps = 200 if args.steps is None else args.steps
        res = bench_gemv(args, torch, pkg)
        cpu = None if args.no_cpu_baseline else cpu_baseline_gemv(
            torch, {k: v["us"] for k, v in res["config"]["per_kernel"].items()})
    line = {
        "metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": res["steps"], "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"],
        "data": "synthetic: seeded random-init int4 codes/scales/zeros with act-order "
                "permutations, random norms/embedding/head and prompt ids",
        "config": res["config"], "roofline": res["roofline"], "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
