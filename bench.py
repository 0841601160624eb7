"""Benchmark of the decode MoE block on one MI355X: µs per layer and weight-stream HBM GB/s.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]
                    [--workloads cfg2_tp4_fp8,cfg3_tp4_mxfp4,...] [--rows 1,8,48]
    python bench.py --timeline --workloads cfg3_tp4_mxfp4 --rows 8   # phase timeline
    python bench.py --seam-only [--seam-tokens 1,8,48]               # the FFN seam alone

A step is one MoE layer (one persistent launch) over one batch of decode rows.
Each workload rotates over ``--layers`` distinct weight sets (each with its own
router, experts and shared expert: 2.8 GB each at the TP4 FP8 shape) so that no
step finds its weights in the 256 MB infinity cache, as in a real model where
every layer has its own weights. Inputs are synthetic: x ~ N(0, 1), router
weight ~ N(0, 1/H) (realistic routing), expert bytes random; the Zipf workload
biases router column 0 by log p_e (p_e ~ rank^-1.2 over a seeded permutation of
the experts) and sets x[:, 0] = 1, so expert popularity follows Zipf(1.2).
MXFP4 experts are read in SGLang's loaded gfx950 layout (aiter's shuffles), the one
the reference requires and reads; ``--layout row_major`` times the row-major reading.

Timing: a captured graph of one launch per layer, replayed; HIP events on the
launching stream bracket each replay. Per (workload, rows): at least 200 timed
launches (max(--steps, 200)); ``us_per_layer`` is the median over replays of
the replay's mean launch time, ``us_mean`` the mean over all of them. The
headline (cfg2 at 8 rows, the workload the metric is quoted on) is also timed
over exactly ``--steps`` launches after ``--warmup`` untimed ones: ``steps``
and ``ms_per_step`` are that run's.

Algorithmic bytes per step use the step's realised union U of routed experts:
B = U * expert bytes + shared bytes + router (E * H * 2 + E * 4) + x and out
(2 * R * H * 2) [+ H * 2 for the norm weight]. ``value`` is the headline's
weight-stream GB/s; every workload's rows are under ``workloads``, each with
its roofline fraction (of 8 TB/s) and, where a committed counter pass exists
(profiles/traffic_<workload>_r<rows>.json), its HBM bytes per launch, and, where the
committed GPU parity record has the point (profiles/accuracy_parity.jsonl, written by the
parity tests under MKMOE_ACCURACY_LOG), the default launch's accuracy there against the
oracle and the golden. The CPU baseline times the oracle (the PyTorch restatement of the
reference's golden MoE) on the host cores on a bounded sample of the headline workload, and of
the MXFP4 workloads at 8 rows (``CPU_POINTS``, under their ``workloads`` entries).

The FFN seam before the MoE block (DeepSeek-V4.1's mHC update, H 5120, two launches) is
timed the same way at 1, 8 and 48 tokens (``workloads["v41_ffn_seam"]``), rotating over 144
layers of its weights (283 MB of projection weights, more than the infinity cache holds).
Its algorithmic bytes per call: the attention output and the residual streams in, the new
streams and the normed input out, the mixes, and one layer's projection (1.97 MB fp32).
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
sys.path.insert(0, str(ROOT / "sgl-amd-mono_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "MoE µs/layer @1/8/48 decode rows + weight-stream HBM GB/s (% of peak), 1 GPU"
HBM_PEAK_GBPS = 8000.0
HEADLINE = ("cfg2_tp4_fp8", 8)
# further (workload, rows) points that get a CPU baseline of their own (under ``workloads``)
CPU_POINTS = (("cfg3_tp4_mxfp4", 8), ("cfg5_tp2_mxfp4_norm", 8))
CPU_POINT_BUDGET_S = 15.0
DEFAULT_WORKLOADS = "cfg2_tp4_fp8,cfg3_tp4_mxfp4,cfg4_tp4_mxfp4_zipf,cfg5_tp2_mxfp4_norm,v41_tp4_mxfp4,v41_tp2_mxfp4"
MIN_TIMED = 200
SEAM_TOKENS = "1,8,48"
SEAM_LAYERS = 144
SEAM_H, SEAM_HC, SEAM_MIX = 5120, 4, 24


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layer(preset, g, device, zipf_s=None):
    """One layer's weights with random contents (GPU-generated), in the kernel's layouts: every
    tensor of the preset's weight contract (``MoeWeights.expected``) with its shape and dtype;
    e4m3 and e2m1 bytes uniform (no e4m3 NaN codes), E8M0 codes 118..122, fp32 block scales
    small, the router N(0, 1/H) (logits ~N(0, 1)), the bias N(0, 0.02), the norm weight
    1 + N(0, 0.1)."""
    import torch

    from sgl_amd_mono.moe.runner import MoeWeights

    e, h = preset.experts, preset.hidden
    want = MoeWeights.expected(preset)
    t = {}
    for name, (shape, dtypes) in want.items():
        if name in ("gate_w", "bias", "norm"):
            continue
        if dtypes[0] == torch.float32:  # fp32 block scales
            t[name] = torch.rand(*shape, generator=g, device=device) * 1e-4 + 5e-5
        elif name.endswith("_s"):  # E8M0
            t[name] = torch.randint(118, 123, shape, generator=g, device=device, dtype=torch.uint8)
        else:
            b = torch.randint(0, 256, shape, generator=g, device=device, dtype=torch.uint8)
            t[name] = torch.where((b & 0x7F) == 0x7F, b ^ 1, b)
    gate = torch.randn(e, h, generator=g, device=device) / h**0.5
    if zipf_s:
        # expert popularity p_e ~ rank(e)^-s over a seeded permutation: with x[:, 0] = 1 the
        # logits are log p_e + N(0, 1) noise
        perm = torch.randperm(e, generator=g, device=device)
        rank = torch.empty(e, device=device)
        rank[perm] = torch.arange(1, e + 1, dtype=torch.float32, device=device)
        logp = -zipf_s * torch.log(rank)
        gate[:, 0] = logp - torch.logsumexp(logp, 0)
    norm = None
    if preset.norm_eps is not None:
        norm = (1 + 0.1 * torch.randn(h, generator=g, device=device)).to(torch.bfloat16)
    return MoeWeights(
        gate_w=gate.to(torch.bfloat16), bias=torch.randn(e, generator=g, device=device) * 0.02, norm=norm, **t
    )


class RowsBench:
    """One row count of one workload: inputs per layer, a captured graph of one launch per
    layer, and timed replays. The rows are seeded by the workload and the count alone, so a
    row count's sample (and its union of experts) is the same whichever others a run times."""

    def __init__(self, runner, layers, preset, rows, device, seed, zipf_s=None):
        import torch

        self.runner, self.layers, self.preset, self.rows = runner, layers, preset, rows
        L = len(layers)
        g = torch.Generator(device=device).manual_seed(seed)
        self.xs = [torch.randn(rows, preset.hidden, generator=g, device=device).to(torch.bfloat16) for _ in range(L)]
        if zipf_s:
            for x in self.xs:
                x[:, 0] = 1.0
        self.outs = [torch.empty(rows, preset.hidden, dtype=torch.bfloat16, device=device) for _ in range(L)]
        self.ids = [torch.empty(rows, preset.topk, dtype=torch.int32, device=device) for _ in range(L)]
        self.graphs = {}

    def launch(self, j):
        self.runner.moe(self.layers[j], self.xs[j], out=self.outs[j], topk_ids=self.ids[j])

    def graph(self, n):
        """A captured graph of the launches of layers 0 .. n - 1."""
        import torch

        if n not in self.graphs:
            gr = torch.cuda.CUDAGraph()
            cap = torch.cuda.Stream()
            cap.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(cap):
                with torch.cuda.graph(gr, stream=cap):
                    for j in range(n):
                        self.launch(j)
            torch.cuda.current_stream().wait_stream(cap)
            gr.replay()  # warm the graph
            torch.cuda.synchronize()
            self.graphs[n] = gr
        return self.graphs[n]

    def warm(self, warmup):
        import torch

        for k in range(warmup):
            self.launch(k % len(self.layers))
        torch.cuda.synchronize()
        self.runner.raise_on_device_error()

    def timed(self, launches):
        """Exactly ``launches`` launches: whole replays of the L-layer graph, then one replay of
        a graph of the rest; -> per-replay (launch count, ms) measured with HIP events."""
        import torch

        L = len(self.layers)
        plan = [L] * (launches // L) + ([launches % L] if launches % L else [])
        graphs = [self.graph(n) for n in plan]
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(plan) + 1)]
        torch.cuda.synchronize()
        ev[0].record()
        for k, gr in enumerate(graphs):
            gr.replay()
            ev[k + 1].record()
        torch.cuda.synchronize()
        self.runner.raise_on_device_error()
        return [(n, ev[k].elapsed_time(ev[k + 1])) for k, n in enumerate(plan)]

    def unions(self):
        import torch

        us, maxrows = [], []
        for t in self.ids:
            v, c = torch.unique(t, return_counts=True)
            us.append(int(v.numel()))
            maxrows.append(int(c.max()))
        return us, maxrows


class FfnRowsBench(RowsBench):
    """DeepSeek-V4.1's FFN at one row count (``FfnRunner.ffn``: the seam, the MoE block on its
    normed rows, the seam's gate), over the MoE layers' weights with a seam weight set each."""

    def __init__(self, ffn, layers, seam_ws, preset, rows, device, seed):
        import torch

        from sgl_amd_mono.moe.ffn import FfnWeights

        super().__init__(ffn.moe_runner, layers, preset, rows, device, seed)
        self.ffn = ffn
        h, hc = preset.hidden, SEAM_HC
        g = torch.Generator(device=device).manual_seed(seed + 77)
        self.fw = [FfnWeights(**vars(sw), **{k: v for k, v in vars(m).items() if k != "norm"})
                   for sw, m in zip(seam_ws, layers)]  # fmt: skip
        self.ins, self.fouts = [], []
        for _ in layers:
            res = torch.randn(rows, hc, h, generator=g, device=device)
            res = (res * torch.rsqrt(res.pow(2).mean(-1, keepdim=True))).to(torch.bfloat16)
            comb = torch.rand(rows, hc, hc, generator=g, device=device) + 0.1
            comb = comb / comb.sum(-2, keepdim=True)
            post = torch.sigmoid(torch.randn(rows, hc, 1, generator=g, device=device)) * 2
            pre = torch.sigmoid(torch.randn(rows, hc, generator=g, device=device)) + 1e-6
            a = (torch.randn(rows, h, generator=g, device=device) * 0.5).to(torch.bfloat16)
            self.ins.append((a, res, post, comb, pre))
            self.fouts.append(ffn._outs(rows, res))
        ffn.normed(rows)  # allocated before any capture

    def launch(self, j):
        self.ffn.ffn(self.fw[j], *self.ins[j], outs=self.fouts[j], topk_ids=self.ids[j])


def seam_weight_sets(device, n: int, seed: int = 4101) -> list:
    """``n`` random seam weight sets (the reference test's distributions, check_ffn.py:149-152)."""
    import torch

    from sgl_amd_mono.moe.seam import SeamWeights

    g = torch.Generator(device=device).manual_seed(seed)
    return [
        SeamWeights(
            hc_ffn_fn=torch.randn(SEAM_MIX, SEAM_HC * SEAM_H, generator=g, device=device) * 0.01,
            hc_ffn_scale=torch.rand(3, generator=g, device=device) * 0.5 + 0.5,
            hc_ffn_base=torch.randn(SEAM_MIX, generator=g, device=device) * 0.1,
            ffn_norm=(1 + 0.1 * torch.randn(SEAM_H, generator=g, device=device)).to(torch.bfloat16),
        )
        for _ in range(n)
    ]


def summarize(preset, rb: RowsBench, reps) -> dict:
    n = sum(k for k, _ in reps)
    per = [ms * 1e3 / k for k, ms in reps if k == len(rb.layers)] or [ms * 1e3 / k for k, ms in reps]
    us_med = statistics.median(per)
    us_mean = sum(ms for _, ms in reps) * 1e3 / n
    unions, maxrows = rb.unions()
    b = sum(preset.algorithmic_bytes(rb.rows, u) for u in unions) / len(unions)
    gbps = b / (us_med * 1e-6) / 1e9
    return {
        "us_per_layer": round(us_med, 2),
        "us_mean": round(us_mean, 2),
        "GBps": round(gbps, 1),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "alg_MB_per_layer": round(b / 1e6, 2),
        "U_mean": round(sum(unions) / len(unions), 1),
        "max_rows_per_expert": max(maxrows),
        "launches_timed": n,
    }


def seam_alg_bytes(tokens: int) -> int:
    """Bytes one seam call must move: a, res, the mixes in; res_out, normed, the mixes out; the
    projection, scales, bias and norm weight."""
    h, hc, t = SEAM_H, SEAM_HC, tokens
    io = 2 * t * h + 2 * hc * t * h + t * SEAM_MIX * 4 + 2 * hc * t * h + 2 * t * h + t * SEAM_MIX * 4
    return io + SEAM_MIX * hc * h * 4 + (3 + SEAM_MIX) * 4 + 2 * h


def bench_seam(device, tokens_list, timed_n: int, layers: int = SEAM_LAYERS) -> dict:
    """The FFN seam's µs per call at each token count: a captured graph of one call per layer
    (two launches each), replayed; HIP events bracket each replay."""
    import torch

    from sgl_amd_mono.moe.seam import SeamRunner

    h, hc = SEAM_H, SEAM_HC
    ws = seam_weight_sets(device, layers)
    g = torch.Generator(device=device).manual_seed(4102)
    run = SeamRunner(device)
    out = {}
    for t in tokens_list:
        ins, outs = [], []
        for _ in range(layers):
            res = torch.randn(t, hc, h, generator=g, device=device)
            res = (res * torch.rsqrt(res.pow(2).mean(-1, keepdim=True))).to(torch.bfloat16)
            comb = torch.rand(t, hc, hc, generator=g, device=device) + 0.1
            comb = comb / comb.sum(-2, keepdim=True)
            post = torch.sigmoid(torch.randn(t, hc, 1, generator=g, device=device)) * 2
            pre = torch.sigmoid(torch.randn(t, hc, generator=g, device=device)) + 1e-6
            a = (torch.randn(t, h, generator=g, device=device) * 0.5).to(torch.bfloat16)
            ins.append((a, res, post, comb, pre))
            outs.append((
                torch.empty(t, h, dtype=torch.bfloat16, device=device), torch.empty_like(res),
                torch.empty_like(post), torch.empty_like(comb), torch.empty_like(pre),
            ))  # fmt: skip
        for j in range(layers):
            run.ffn_seam(ws[j], *ins[j], outs=outs[j])
        torch.cuda.synchronize()

        def timed(gate_later: bool) -> list[float]:
            gr = torch.cuda.CUDAGraph()
            cap = torch.cuda.Stream()
            cap.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(cap):
                with torch.cuda.graph(gr, stream=cap):
                    for j in range(layers):
                        run.ffn_seam(ws[j], *ins[j], outs=outs[j], gate_later=gate_later)
                        if gate_later:
                            run.cancel_gate()  # the path to the MoE block's input alone
            torch.cuda.current_stream().wait_stream(cap)
            gr.replay()
            torch.cuda.synchronize()
            reps = max(2, -(-timed_n // layers))
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
            ev[0].record()
            for k in range(reps):
                gr.replay()
                ev[k + 1].record()
            torch.cuda.synchronize()
            return [ev[k].elapsed_time(ev[k + 1]) * 1e3 / layers for k in range(reps)]

        per = timed(False)
        us = statistics.median(per)
        # the path to the MoE block's input: the slice launch and the norm, the gate left out
        us_normed = statistics.median(timed(True))
        reps = len(per)
        b = seam_alg_bytes(t)
        gbps = b / (us * 1e-6) / 1e9
        out[str(t)] = {
            "us_per_layer": round(us, 2),
            "us_mean": round(sum(per) / len(per), 2),
            "us_to_normed": round(us_normed, 2),
            "GBps": round(gbps, 1),
            "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "alg_MB_per_layer": round(b / 1e6, 3),
            "launches_timed": 2 * reps * layers,
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
        }  # fmt: skip
        log(f"v41_ffn_seam tokens={t}: {out[str(t)]}")
        del ins, outs
    return {"preset": f"DeepSeek-V4.1 FFN seam (hidden {h}, {hc} streams, {SEAM_MIX} mixes)", "rows": out}


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
    ex.prefetch(np.unique(ids).tolist(), min(16, cores))  # expert generation is not timed
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


def measured_accuracy(workload: str, rows: int):
    """The default launch's accuracy at this point from the committed GPU parity record
    (profiles/accuracy_parity.jsonl), or None."""
    f = ROOT / "profiles" / "accuracy_parity.jsonl"
    if not f.exists():
        return None
    for rec in map(json.loads, f.read_text().splitlines()):
        if rec["workload"] == workload and rec["rows"] == rows and rec["mode"] == "default":
            keep = ("max_abs", "rel_l2", "cos", "n_over_2e-2", "numel")
            return {
                "vs_golden": {k: rec["vs_golden"][k] for k in keep},
                "vs_oracle": {k: rec["vs_oracle"][k] for k in keep},
                "routing_exact": rec["routing_exact"],
                "source": f"profiles/{f.name}",
            }
    return None


def measured_traffic(workload: str, rows: int):
    """HBM bytes per launch from the committed counter passes (profiles/), or None."""
    f = ROOT / "profiles" / f"traffic_{workload}_r{rows}.json"
    if not f.exists():
        return None, None
    d = json.loads(f.read_text())
    return d.get("hbm_bytes_per_launch"), f"profiles/{f.name}"


def timeline(runner, rb: RowsBench, reps: int = 8) -> dict:
    """Phase timeline of the diagnostic build: per phase, the median / min / max over
    workgroups of its end (µs from the launch's first stamp). Launches rotate over the layers
    (so each finds its weights in HBM, not the infinity cache); of ``reps`` launches the one
    of median total time is kept."""
    import torch

    from sgl_amd_mono.moe import _lib

    end = _lib.TL_NAMES.index("end")
    runs = []
    for k in range(reps):
        rb.launch(k % len(rb.layers))
        torch.cuda.synchronize()
        st = runner.region("timeline").view(torch.int64).cpu().reshape(-1, _lib.TL_SLOTS)
        st = st[st[:, 0] != 0].double()
        t0 = float(st[:, 0].min())
        runs.append((float(st[:, end].max()) - t0, st, t0))
    runner.raise_on_device_error()
    runs.sort(key=lambda r: r[0])
    total, st, t0 = runs[len(runs) // 2]
    tick_us = 0.01  # s_memrealtime: 100 MHz
    out = {"total_us": round(total * tick_us, 2), "workgroups": int(st.shape[0]), "phases": {}}
    counts = ("gate_up units", "down units")
    ends = ("gate_up first unit", "down first unit")
    cols = []  # per phase: every workgroup's value, None where it does not stamp that phase
    for k, name in enumerate(_lib.TL_NAMES):
        col = st[:, k]
        if name.startswith(("gate_up ", "down ")) and name not in counts + ends:
            v = col * tick_us  # time a workgroup's wave 0 spent in that part of its loop
        elif name in counts:
            v = col
        else:
            # a phase end: a workgroup whose path skips the phase (the early shared expert
            # workgroups do not route the step, for one) leaves its stamp at zero
            v = torch.where(col != 0, (col - t0) * tick_us, torch.full_like(col, float("nan")))
        cols.append(v)
        have = v[~torch.isnan(v)]
        out["phases"][name] = None if have.numel() == 0 else {
            "median": round(float(have.median()), 2),
            "min": round(float(have.min()), 2),
            "max": round(float(have.max()), 2),
            "workgroups": int(have.numel()),
        }
    # every workgroup's stamps (µs from the first stamp; the loop parts' sums in µs, the counts
    # as they are; None for a phase it skips), in workgroup order
    out["workgroup_stamps"] = [
        [None if torch.isnan(c[i]) else round(float(c[i]), 2) for c in cols] for i in range(st.shape[0])
    ]
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workloads", default=DEFAULT_WORKLOADS)
    ap.add_argument("--workload", default=None, help="one workload (same as --workloads W)")
    ap.add_argument("--rows", default=None, help="row counts (default: each workload's own)")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--staged", action="store_true", help="time the one-launch-per-stage variant")
    ap.add_argument("--mxfp4-scaled-rows", type=int, default=None,
                    help="MXFP4 launches with at least this many rows on the scaled fp4 x fp8 MFMA")
    ap.add_argument("--mxfp4-scaled-down-rows", type=int, default=None,
                    help="MXFP4 launches with at least this many rows run the down GEMM alone on the scaled MFMA")
    ap.add_argument("--layout", default="aiter", choices=("row_major", "aiter"),
                    help="the MXFP4 workloads' expert layout: SGLang's loaded gfx950 layout (aiter's shuffles, "
                    "the default: the layout the reference reads; the random weight bytes are read as such), "
                    "or row-major")
    ap.add_argument("--timeline", action="store_true",
                    help="phase timeline of the diagnostic build (build.py --timeline); no JSON line")
    ap.add_argument("--seam-tokens", default=SEAM_TOKENS, help="the FFN seam's token counts ('' : none)")
    ap.add_argument("--seam-only", action="store_true", help="time the FFN seam alone and print its results")
    ap.add_argument("--no-ffn", action="store_true",
                    help="skip V4.1's whole-FFN timing (profiles of the MoE launch alone)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain copy of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: the benchmark runs one TP rank's MoE share on one GPU; figures at several GPUs are "
            "not produced (the all-reduce is outside the benchmarked path). Use --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    if args.calibrate_copy:
        print(json.dumps(calibrate_copy(args.calibrate_copy)), flush=True)
        return 0
    if args.timeline:
        from sgl_amd_mono.moe import _lib

        _lib.use_timeline_build()

    from sgl_amd_mono.moe.presets import PRESETS, WORKLOADS
    from sgl_amd_mono.moe.runner import MoeRunner

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    seam_tokens = [int(v) for v in args.seam_tokens.split(",") if v]
    if args.seam_only:
        print(json.dumps({"v41_ffn_seam": bench_seam(device, seam_tokens, max(args.steps, MIN_TIMED))}), flush=True)
        return 0
    names = [args.workload] if args.workload else args.workloads.split(",")
    timed_n = max(args.steps, MIN_TIMED)
    results, head = {}, None
    for wi, name in enumerate(names):
        wl = WORKLOADS[name]
        preset = PRESETS[wl["preset"]]
        zipf = wl.get("zipf_s")
        rows_list = [int(r) for r in args.rows.split(",")] if args.rows else list(wl["rows"])
        g = torch.Generator(device=device).manual_seed(20260101 + wi)
        log(f"{name}: generating {args.layers} layers of {preset.name} weights on the GPU")
        layers = [make_layer(preset, g, device, zipf) for _ in range(args.layers)]
        torch.cuda.synchronize()
        kw = {} if args.mxfp4_scaled_rows is None else {"mxfp4_scaled_rows": args.mxfp4_scaled_rows}
        if args.mxfp4_scaled_down_rows is not None:
            kw["mxfp4_scaled_down_rows"] = args.mxfp4_scaled_down_rows
        if preset.routed_fmt == "mxfp4" and not preset.aiter_only:
            kw["layout"] = args.layout
        runner = MoeRunner(preset, device, max_rows=max(48, max(rows_list)), **kw)
        # V4.1: its whole FFN too (the seam, the MoE block, the seam's gate) on the same weights
        ffn = None
        if preset.hidden == SEAM_H and preset.aiter_only and not (args.staged or args.timeline or args.no_ffn):
            from sgl_amd_mono.moe.ffn import FfnRunner

            ffn = FfnRunner(preset, device, max_rows=max(48, max(rows_list)), **kw)
            seam_ws = seam_weight_sets(device, len(layers), seed=4103)
        if args.staged:
            orig = runner.moe
            runner.moe = lambda *a, **k: orig(*a, staged=True, **k)
        wres = {}
        for r in rows_list:
            rb = RowsBench(runner, layers, preset, r, device, seed=1000 * (wi + 1) + r, zipf_s=zipf)
            if args.timeline:
                rb.warm(max(args.warmup, len(layers)))
                tl = timeline(runner, rb)
                print(json.dumps({"timeline": f"{name} rows={r}", **tl}), flush=True)
                continue
            rb.warm(max(args.warmup, 1))
            if (name, r) == HEADLINE:
                reps = rb.timed(args.steps)  # exactly --steps launches
                ms = sum(m for _, m in reps)
                head = {"steps": args.steps, "ms_per_step": ms / args.steps}
            res = summarize(preset, rb, rb.timed(timed_n))
            traffic, source = measured_traffic(name, r)
            res["roofline"] = {
                "bound": "hbm",
                "achieved": res["GBps"],
                "peak": HBM_PEAK_GBPS,
                "unit": "GB/s",
                "frac": round(res["GBps"] / HBM_PEAK_GBPS, 4),
                "traffic": traffic,
            }
            if traffic is not None and not args.staged:
                res["roofline"]["traffic_source"] = source
            acc = measured_accuracy(name, r)
            if acc is not None:
                res["accuracy"] = acc
            if ffn is not None:
                fb = FfnRowsBench(ffn, layers, seam_ws, preset, r, device, seed=1000 * (wi + 1) + r)
                fb.warm(max(args.warmup, 1))
                f = summarize(preset, fb, fb.timed(timed_n))
                b = f["alg_MB_per_layer"] * 1e6 + seam_alg_bytes(r)
                gbps = b / (f["us_per_layer"] * 1e-6) / 1e9
                res["ffn"] = {
                    "what": "the FFN: seam (2 launches), MoE block, seam gate, per layer",
                    "us_per_layer": f["us_per_layer"],
                    "us_mean": f["us_mean"],
                    "alg_MB_per_layer": round(b / 1e6, 2),
                    "GBps": round(gbps, 1),
                    "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
                    "launches_timed": 4 * f["launches_timed"],
                }
                del fb
            wres[str(r)] = res
            log(f"{name} rows={r}: {res}")
            del rb
        results[name] = {"preset": preset.name, "rows": wres}
        del layers, runner, ffn
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    if args.timeline:
        return 0
    if seam_tokens:
        results["v41_ffn_seam"] = bench_seam(device, seam_tokens, timed_n)

    hname, hrows = HEADLINE
    if hname in results and str(hrows) in results[hname]["rows"]:
        h = results[hname]["rows"][str(hrows)]
    else:  # a run of other workloads: the first timed row count stands in
        hname = next(iter(results))
        hrows = int(next(iter(results[hname]["rows"])))
        h = results[hname]["rows"][str(hrows)]
    hpreset = PRESETS[WORKLOADS[hname]["preset"]]
    if head is not None:
        ms_per_step = head["ms_per_step"]
        steps = head["steps"]
        value = h["alg_MB_per_layer"] * 1e6 / (ms_per_step * 1e-3) / 1e9
    else:
        ms_per_step, steps, value = h["us_per_layer"] / 1e3, h["launches_timed"], h["GBps"]
    traffic, source = measured_traffic(hname, hrows)
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if hpreset.routed_fmt == "fp8_b128" else "fp4xfp8",
        "data": "synthetic",
        "config": {
            "workload": f"{hname}: one TP rank's MoE block, hidden {hpreset.hidden}, {hpreset.experts} experts "
            f"top-{hpreset.topk} ({hpreset.n_group} groups, top-{hpreset.topk_group}), inter {hpreset.inter}, "
            f"shared {hpreset.shared_inter}, {hpreset.routed_fmt} experts, {hrows} decode rows",
            "rows": hrows,
            "layers_rotated": args.layers,
            "launch": "staged" if args.staged else "persistent",
            "layout": "aiter" if hpreset.aiter_only else (args.layout if hpreset.routed_fmt == "mxfp4" else "row_major"),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
        },
        "workloads": results,
    }
    if traffic is not None and not args.staged:
        out["roofline"]["traffic_source"] = source
        out["roofline"]["alg_bytes_per_launch"] = round(h["alg_MB_per_layer"] * 1e6)
    if not args.no_cpu:
        log("CPU baseline (oracle on the host cores)")
        out["cpu_baseline"] = cpu_baseline(hname, hrows)
        for wname, r in CPU_POINTS:
            if wname in results and str(r) in results[wname]["rows"]:
                log(f"CPU baseline of {wname} at {r} rows")
                results[wname]["rows"][str(r)]["cpu_baseline"] = cpu_baseline(wname, r, CPU_POINT_BUDGET_S)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
