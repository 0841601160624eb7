"""Benchmark of the decode MoE block on one MI355X: µs per layer and weight-stream HBM GB/s.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--workload cfg2_tp4_fp8] [--rows 1,8,48]

A step is one MoE layer (one persistent launch) over one batch of decode rows.
The layers rotate over ``--layers`` distinct weight sets (each with its own
router, experts and shared expert; 2.8 GB each at the TP4 FP8 shape) so that
no step finds its weights in the 256 MB infinity cache, as in a real model
where every layer has its own weights. Inputs are synthetic: x ~ N(0, 1),
router weight ~ N(0, 1/H) (realistic routing), expert bytes random.

The timed region replays a captured graph of the layer sequence; HIP events
on the launching stream bracket it. Algorithmic bytes per step use the step's
realised union U of routed experts:
B = U * expert bytes + shared bytes + router (E * H * 2 + E * 4) + x and out
(2 * R * H * 2) [+ H * 2 for the norm weight].

Prints one JSON line (rank 0). ``value`` is the weight-stream GB/s at the
headline row count (8); the other row counts are under ``rows``. The CPU
baseline times the oracle (the PyTorch restatement of the reference's golden
MoE) on the host cores on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sgl-amd-mono_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "MoE µs/layer @1/8/48 decode rows + weight-stream HBM GB/s (% of peak), 1 GPU"
HBM_PEAK_GBPS = 8000.0
HEADLINE_ROWS = 8


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layer(preset, g, device):
    """One layer's weights with random contents (GPU-generated), in the kernel's layouts."""
    import torch

    from sgl_amd_mono.moe.runner import MoeWeights

    e, h, i, s = preset.experts, preset.hidden, preset.inter, preset.shared_inter

    def fp8(*shape):
        t = torch.randint(0, 256, shape, generator=g, device=device, dtype=torch.uint8)
        return torch.where((t & 0x7F) == 0x7F, t ^ 1, t)

    def f32s(*shape):
        return torch.rand(*shape, generator=g, device=device) * 1e-4 + 5e-5

    def e8m0(*shape):
        return torch.randint(118, 123, shape, generator=g, device=device, dtype=torch.uint8)

    if preset.routed_fmt == "fp8_b128":
        w13, w13_s = fp8(e, 2 * i, h), f32s(e, 2 * i // 128, h // 128)
        w2, w2_s = fp8(e, h, i), f32s(e, h // 128, i // 128)
    else:
        w13 = torch.randint(0, 256, (e, 2 * i, h // 2), generator=g, device=device, dtype=torch.uint8)
        w13_s = e8m0(e, 2 * i, h // 32)
        w2 = torch.randint(0, 256, (e, h, i // 2), generator=g, device=device, dtype=torch.uint8)
        w2_s = e8m0(e, h, i // 32)
    gate = (torch.randn(e, h, generator=g, device=device) / h**0.5).to(torch.bfloat16)
    norm = None
    if preset.norm_eps is not None:
        norm = (1 + 0.1 * torch.randn(h, generator=g, device=device)).to(torch.bfloat16)
    return MoeWeights(
        gate_w=gate,
        bias=torch.randn(e, generator=g, device=device) * 0.02,
        w13=w13, w13_s=w13_s, w2=w2, w2_s=w2_s,
        sgu=fp8(2 * s, h), sgu_s=f32s(2 * s // 128, h // 128),
        sw2=fp8(h, s), sw2_s=f32s(h // 128, s // 128),
        norm=norm,
    )  # fmt: skip


def time_rows(runner, layers, preset, rows, steps, warmup, device):
    """Replay a graph of one step per layer; -> (µs per step, bytes per step, U per step).
    The rows are seeded by their count alone, so a row count's sample (and its union of
    experts) is the same whichever other row counts the run times."""
    import torch

    L = len(layers)
    g = torch.Generator(device=device).manual_seed(1000 + rows)
    xs = [torch.randn(rows, preset.hidden, generator=g, device=device).to(torch.bfloat16) for _ in range(L)]
    outs = [torch.empty(rows, preset.hidden, dtype=torch.bfloat16, device=device) for _ in range(L)]
    ids = [torch.empty(rows, preset.topk, dtype=torch.int32, device=device) for _ in range(L)]
    for k in range(max(warmup, 1)):
        j = k % L
        runner.moe(layers[j], xs[j], out=outs[j], topk_ids=ids[j])
    torch.cuda.synchronize()
    runner.raise_on_device_error()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for j in range(L):
                runner.moe(layers[j], xs[j], out=outs[j], topk_ids=ids[j])
    torch.cuda.current_stream().wait_stream(cap)
    graph.replay()  # warm the graph
    torch.cuda.synchronize()
    reps = max(1, -(-steps // L))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(reps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    runner.raise_on_device_error()
    ms = t0.elapsed_time(t1)
    n_steps = reps * L
    us = ms * 1e3 / n_steps
    unions = [int(torch.unique(t).numel()) for t in ids]
    bytes_per = sum(preset.algorithmic_bytes(rows, u) for u in unions) / L
    return us, bytes_per, unions, n_steps


def cpu_baseline(workload: str, rows: int, budget_s: float = 25.0):
    """The oracle's MoE partial on the host cores: µs per layer on a bounded sample."""
    import numpy as np
    import torch

    from oracle import gen
    from oracle import moe as om
    from oracle import routing as rt
    from sgl_amd_mono.moe.presets import PRESETS, WORKLOADS, workload_dict

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    p = workload_dict(workload)
    preset = PRESETS[WORKLOADS[workload]["preset"]]
    x = gen.make_x(p, rows, 0)
    dense = gen.make_dense(p, 0)
    xin = rt.rmsnorm_exact(x, dense["norm"], p["norm_eps"]) if p["norm_eps"] is not None else x
    _, ids, _ = rt.route(xin, dense["gate_w"], dense["bias"], p)
    ex = gen.LazyExperts(p, 0)
    for e in np.unique(ids).tolist():  # expert generation is not timed
        ex.get(e)
    # the golden's own form: fp32 matmuls of the dequantized experts, torch silu
    om.moe_partial(x, dense, p, experts=ex, exact=False)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < budget_s:
        t = time.perf_counter()
        om.moe_partial(x, dense, p, experts=ex, exact=False)
        times.append(time.perf_counter() - t)
    us = float(np.median(times)) * 1e6
    u = len(np.unique(ids))
    gbps = preset.algorithmic_bytes(rows, u) / (us * 1e-6) / 1e9
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "us_per_layer": round(us, 1),
        "cores": cores,
        "kind": "port",
        "sample": f"{workload} at {rows} rows (U={u}), median of {len(times)} runs after 1 warm-up, "
        f"expert dequantization included, seeded CPU inputs; {cpu}",
    }


def calibrate_copy(mib: int, reps: int = 4) -> dict:
    """A plain device-to-device copy of known size (torch's copy kernel), for scaling the
    FETCH_SIZE / WRITE_SIZE counters of the MoE launch to bytes."""
    import torch

    n = mib << 20
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes_read": n, "copy_bytes_written": n, "reps": reps}


def measured_traffic(workload: str, rows: int):
    """HBM bytes per launch from the committed counter passes (profiles/), or None."""
    f = ROOT / "profiles" / f"traffic_{workload}_r{rows}.json"
    if not f.exists():
        return None, None
    d = json.loads(f.read_text())
    return d.get("hbm_bytes_per_launch"), f"profiles/{f.name}"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="cfg2_tp4_fp8")
    ap.add_argument("--rows", default="1,8,48")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--staged", action="store_true", help="time the one-launch-per-stage variant")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build runs one TP rank's MoE share on one GPU; figures at several GPUs are "
            "not produced (the all-reduce is outside the benchmarked path). Use --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from sgl_amd_mono.moe.presets import PRESETS, WORKLOADS
    from sgl_amd_mono.moe.runner import MoeRunner

    if args.calibrate_copy:
        print(json.dumps(calibrate_copy(args.calibrate_copy)), flush=True)
        return 0

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    wl = WORKLOADS[args.workload]
    preset = PRESETS[wl["preset"]]
    rows_list = [int(r) for r in args.rows.split(",")]
    g = torch.Generator(device=device).manual_seed(20260101)
    log(f"generating {args.layers} layers of {preset.name} weights on the GPU")
    layers = [make_layer(preset, g, device) for _ in range(args.layers)]
    torch.cuda.synchronize()
    runner = MoeRunner(preset, device, max_rows=max(48, max(rows_list)))
    if args.staged:
        orig = runner.moe
        runner.moe = lambda *a, **k: orig(*a, staged=True, **k)
    res = {}
    for r in rows_list:
        us, b, unions, n = time_rows(runner, layers, preset, r, args.steps, args.warmup, device)
        gbps = b / (us * 1e-6) / 1e9
        res[r] = {
            "us_per_layer": round(us, 2),
            "GBps": round(gbps, 1),
            "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "alg_MB_per_layer": round(b / 1e6, 2),
            "U_mean": round(sum(unions) / len(unions), 1),
            "steps_timed": n,
        }
        log(f"rows={r}: {res[r]}")
    head = HEADLINE_ROWS if HEADLINE_ROWS in res else rows_list[0]
    h = res[head]
    out = {
        "metric": METRIC,
        "value": h["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": h["steps_timed"],
        "warmup": args.warmup,
        "ms_per_step": round(h["us_per_layer"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if preset.routed_fmt == "fp8_b128" else "fp4xfp8",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: one TP rank's MoE block, hidden {preset.hidden}, {preset.experts} experts "
            f"top-{preset.topk} ({preset.n_group} groups, top-{preset.topk_group}), inter {preset.inter}, "
            f"shared {preset.shared_inter}, {preset.routed_fmt} experts, headline {head} rows",
            "rows": head,
            "layers_rotated": args.layers,
            "launch": "staged" if args.staged else "persistent",
        },
        "rows": {str(k): v for k, v in res.items()},
        "roofline": {
            "bound": "hbm",
            "achieved": h["GBps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(h["GBps"] / HBM_PEAK_GBPS, 4),
            "traffic": None,
        },
    }
    traffic, source = measured_traffic(args.workload, head)
    if traffic is not None and not args.staged:
        out["roofline"]["traffic"] = traffic
        out["roofline"]["traffic_source"] = source
        out["roofline"]["alg_bytes_per_launch"] = round(h["alg_MB_per_layer"] * 1e6)
    if not args.no_cpu:
        log("CPU baseline (oracle on the host cores)")
        out["cpu_baseline"] = cpu_baseline(args.workload, head)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
