"""Parity of the HIP MoE block (through the C ABI) with the CPU oracle, on an MI355X.

Bars: router part sums, activation codes, expert ids and routing weights bit for
bit at every row count; the bf16 output of every row, against both the oracle's
exact restatement of the kernel's order and the golden's fp32-matmul form (the
reference's PyTorch path), within relative L2 1e-2 and max-abs 2e-2 up to the
bf16 combine's own rounding (gpu_case.within_bar), and cosine 0.9999 against
the golden. The default launch runs the expert GEMMs on MFMA; launches forced onto the
fixed-order VALU GEMVs (which the oracle restates) are also bit for bit against the oracle
and the golden vectors, at small and large row counts. The persistent and the staged
launches bit for bit alike; repeated and graph-replayed launches bit for bit alike.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 1e-2  # the output bar (gpu_case.within_bar applies it)
CASES = [
    ("cfg1_plumbing_fp8", 4),
    ("cfg2_tp4_fp8", 1),
    ("cfg2_tp4_fp8", 8),
    ("cfg2_tp4_fp8", 48),
    ("cfg3_tp4_mxfp4", 1),
    ("cfg3_tp4_mxfp4", 8),
    ("cfg3_tp4_mxfp4", 48),
    ("cfg4_tp4_mxfp4_zipf", 48),
    ("cfg5_tp2_mxfp4_norm", 1),
    ("cfg5_tp2_mxfp4_norm", 8),
    ("cfg5_tp2_mxfp4_norm", 48),
    # the RMSNorm inside stage A (up to 16 rows) and the norm stage's hand-off (17)
    ("cfg5_tp2_mxfp4_norm", 16),
    ("cfg5_tp2_mxfp4_norm", 17),
    # 12 rows: stage Q with the shared expert's down inside its hand-off, pick batch whole
    ("cfg2_tp4_fp8", 12),
    ("cfg3_tp4_mxfp4", 12),
    # the last row count every workgroup routes itself (8: the early shared gate_up on
    # workgroups 0 .. n-1) and the first with the routing hand-off (9: on the workgroups past
    # the rows); 16 and 17: the shared down inside the Q hand-off and after the routed one
    ("cfg3_tp4_mxfp4", 9),
    ("cfg3_tp4_mxfp4", 16),
    ("cfg3_tp4_mxfp4", 17),
    ("tp4_fp8_zipf", 16),
    ("tp4_fp8_zipf", 48),
    ("tp2_mxfp4_norm_zipf", 48),
    # V4.1's router scores (sqrt(softplus), one group, check_ffn.py:201-206) on the plumbing
    # shape: local routing (up to 8 rows) and the routing hand-off (16, 24)
    ("plumbing_fp8_softplus", 1),
    ("plumbing_fp8_softplus", 4),
    ("plumbing_fp8_softplus", 16),
    ("plumbing_fp8_softplus", 24),
]
_cache = {}


def _case(workload, rows):
    from gpu_case import build

    key = (workload, rows)
    if key not in _cache:
        _cache.clear()  # one layer's weights on the GPU at a time
        torch.cuda.empty_cache()
        _cache[key] = build(workload, rows)
    return _cache[key]


def _runner(case, mfma_rows=None, **kw):
    """A runner of the case's preset; mfma_rows: (gate_up rows, down rows) from which its
    launches run the expert GEMMs on MFMA (default: the library's, i.e. always)."""
    from sgl_amd_mono.moe.runner import MoeRunner

    if mfma_rows is not None:
        kw["mfma_rows"] = mfma_rows
    return MoeRunner(case.preset, "cuda", **kw)


def test_device_decode_matches_tables():
    from oracle import formats as fm
    from sgl_amd_mono.moe import _lib

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).cuda()
    f8 = torch.empty(256, device="cuda")
    f4 = torch.empty(512, device="cuda")
    _lib.check(
        _lib.testing_lib().mkmoe_device_decode(codes.data_ptr(), f8.data_ptr(), f4.data_ptr(), 256, torch.cuda.current_stream().cuda_stream),
        "decode",
    )
    torch.cuda.synchronize()
    tab = fm.e4m3_table()
    got = f8.cpu().double().numpy()
    ok = ~np.isnan(tab)
    assert np.array_equal(got[ok], tab[ok]) and np.all(np.isnan(got[~ok]))
    want4 = fm.fp4_unpack(torch.arange(256, dtype=torch.int32).to(torch.uint8)).numpy()
    assert np.array_equal(f4.cpu().numpy(), want4)


def _check(c, rows, run, exact, mode="default"):
    """Run the launch; routing bit for bit, the output within the bounds (and, exact: bit for bit)."""
    from gpu_case import errors, record_accuracy, within_bar

    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
    out = run.moe(c.w, c.x, topk_ids=ids, topk_w=wts)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    # router part sums, bit for bit
    parts = run.region("router_parts")[: rows * c.p["experts"] * c.p["router_parts"] * 4]
    parts = parts.view(torch.float32).cpu().numpy().reshape(rows, c.p["router_parts"], c.p["experts"])
    parts = np.ascontiguousarray(parts.transpose(0, 2, 1))
    assert np.array_equal(parts.view(np.uint32), c.parts.view(np.uint32)), "router part sums"
    # the polled copy is back to unset (every byte 0xFF) for the next launch
    assert bool((run.region("router_parts_polled") == 0xFF).all()), "polled part sums left unset"
    # routing, bit for bit
    assert np.array_equal(ids.cpu().numpy(), c.ids), "expert ids"
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), c.wts.view(np.uint32)), "routing weights"
    got = out[torch.from_numpy(c.check).cuda()].cpu()
    e = errors(got, c.ref, c.chain[torch.from_numpy(c.check)])
    print(f"  all {rows} rows vs the oracle's exact order: {e}", flush=True)
    assert not e["nan"] and not torch.isnan(out).any()
    assert within_bar(e, got.numel()), e
    n_diff = int((got.view(torch.int16) != c.ref.view(torch.int16)).sum())
    print(f"  elements differing from the oracle's bits: {n_diff} of {got.numel()}", flush=True)
    if exact:
        assert n_diff == 0, f"{n_diff} output elements differ from the oracle's bits"
    # every row against the golden's own fp32 matmuls (the reference's PyTorch path,
    # check_ffn.py:209-232, which compares every token: check_ffn.py:327-343), to the same bar
    # and the reference's own cosine bound (ffn.moe.cosine, spec.py:305-309)
    g = errors(out.cpu(), c.golden, c.chain)
    print(f"  all {rows} rows vs fp32-matmul golden: {g}", flush=True)
    record_accuracy(c.workload, rows, mode, e, g, True, n_diff)
    assert within_bar(g, out.numel()) and g["cos"] >= 0.9999, g
    assert out.numel() == c.golden.numel() == rows * c.p["hidden"]


@pytest.mark.parametrize("workload,rows", CASES)
def test_parity(workload, rows):
    """The default launch (MFMA expert GEMMs from MFMA_*_ROWS rows; VALU GEMVs, bit for bit, below)."""
    from sgl_amd_mono.moe.runner import MFMA_DOWN_ROWS, MFMA_GATE_ROWS

    c = _case(workload, rows)
    mode = f"gate_up {'MFMA' if rows >= MFMA_GATE_ROWS else 'VALU'}, down {'MFMA' if rows >= MFMA_DOWN_ROWS else 'VALU'}"
    print(f"\n{workload} R={rows} ({mode})", flush=True)
    _check(c, rows, _runner(c), exact=rows < min(MFMA_GATE_ROWS, MFMA_DOWN_ROWS), mode="default")


@pytest.mark.parametrize(
    "workload,rows",
    [
        ("cfg1_plumbing_fp8", 4),
        ("cfg2_tp4_fp8", 1),
        ("cfg2_tp4_fp8", 8),
        ("cfg2_tp4_fp8", 48),
        ("cfg3_tp4_mxfp4", 8),
        ("cfg5_tp2_mxfp4_norm", 1),
        ("cfg5_tp2_mxfp4_norm", 48),
        ("cfg4_tp4_mxfp4_zipf", 48),
        ("plumbing_fp8_softplus", 4),
        ("plumbing_fp8_softplus", 24),
    ],
)
def test_parity_valu_forced(workload, rows):
    """Large launches held on the VALU GEMVs: bit for bit against the oracle."""
    c = _case(workload, rows)
    print(f"\n{workload} R={rows} (VALU forced)", flush=True)
    _check(c, rows, _runner(c, (rows + 1, rows + 1)), exact=True, mode="valu")


@pytest.mark.parametrize(
    "workload,rows",
    [
        ("cfg1_plumbing_fp8", 4),
        ("cfg2_tp4_fp8", 1),
        ("cfg2_tp4_fp8", 48),
        ("cfg3_tp4_mxfp4", 1),
        ("cfg4_tp4_mxfp4_zipf", 48),
        ("cfg5_tp2_mxfp4_norm", 1),
        ("cfg5_tp2_mxfp4_norm", 48),
    ],
)
def test_parity_mfma_forced(workload, rows):
    """Every expert GEMM on MFMA (gate_up included): within the bounds, routing bit for bit."""
    c = _case(workload, rows)
    print(f"\n{workload} R={rows} (MFMA forced)", flush=True)
    _check(c, rows, _runner(c, (1, 1)), exact=False, mode="mfma")


@pytest.mark.parametrize(
    "workload,rows",
    [
        ("cfg3_tp4_mxfp4", 8),
        ("cfg3_tp4_mxfp4", 48),
        ("cfg4_tp4_mxfp4_zipf", 48),
        ("cfg5_tp2_mxfp4_norm", 8),
        ("cfg5_tp2_mxfp4_norm", 48),
        ("tp2_mxfp4_norm_zipf", 48),
    ],
)
@pytest.mark.parametrize("mode", ["both", "down"])
def test_parity_mxfp4_scaled(workload, rows, mode):
    """Both MXFP4 expert GEMMs (or the down GEMM alone) on the scaled fp4 x fp8 MFMA (no
    converts), opt-in options.

    Its internal sum keeps fewer bits than fp32 (test_gpu_scaled_mfma.py bounds it), so it is
    held to the reference's own bounds (cosine 0.9999 and relative error 0.015 of the golden,
    ffn.moe at spec.py:305-309, and a relative L2 of 1e-2 of the output), with routing bit for
    bit; the elements beyond max-abs 2e-2 are reported (measured, both: 1 to 218 of 7168 to
    344064; down alone: 0 to 34), which is why the default launch converts the codes to bf16."""
    from gpu_case import errors, record_accuracy

    c = _case(workload, rows)
    print(f"\n{workload} R={rows} (scaled fp4 x fp8 MFMA: {mode})", flush=True)
    run = _runner(c, **({"mxfp4_scaled_rows": 1} if mode == "both" else {"mxfp4_scaled_down_rows": 1}))
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
    out = run.moe(c.w, c.x, topk_ids=ids, topk_w=wts)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert np.array_equal(ids.cpu().numpy(), c.ids), "expert ids"
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), c.wts.view(np.uint32)), "routing weights"
    res = {}
    for name, ref in (("oracle", c.ref), ("golden", c.golden)):
        e = res[name] = errors(out.cpu(), ref, c.chain)
        print(f"  all {rows} rows vs {name}: {e}", flush=True)
        assert not e["nan"] and e["rel_l2"] <= REL_L2 and e["cos"] >= 0.9999, e
    record_accuracy(c.workload, rows, f"scaled_{mode}", res["oracle"], res["golden"], True)


@pytest.mark.parametrize(
    "workload,rows",
    [
        ("cfg3_tp4_mxfp4", 1),
        ("cfg3_tp4_mxfp4", 8),
        ("cfg3_tp4_mxfp4", 48),
        ("cfg4_tp4_mxfp4_zipf", 48),
        ("cfg5_tp2_mxfp4_norm", 8),
        ("tp2_mxfp4_norm_zipf", 48),
    ],
)
def test_parity_aiter_layout(workload, rows):
    """SGLang's loaded gfx950 MXFP4 layout (aiter's shuffles, check_ffn.py:169-173), read in
    place: the case's experts shuffled (oracle.shuffle, restated from the reference kernel's
    addressing), scales as SGLang's flat [E rows][cols] views, give the row-major launch's
    output bit for bit (persistent, staged, and on the scaled MFMA), and so the oracle's
    parity, checked again here; the VALU GEMVs (row-major rows only) are refused."""
    import dataclasses

    from oracle import shuffle as sh

    c = _case(workload, rows)
    print(f"\n{workload} R={rows} (aiter layout)", flush=True)
    w13, w13_s, w2, w2_s = sh.to_aiter(c.w.w13, c.w.w13_s, c.w.w2, c.w.w2_s)
    e = c.p["experts"]
    ws = dataclasses.replace(c.w, w13=w13, w13_s=w13_s.view(-1, w13_s.shape[-1]), w2=w2, w2_s=w2_s.view(-1, w2_s.shape[-1]))
    assert not torch.equal(w13, c.w.w13) and w13_s.shape[0] == e
    _check(dataclasses.replace(c, w=ws), rows, _runner(c, layout="aiter"), exact=False)
    for kw, opts in (({}, {}), ({"staged": True}, {}), ({}, {"mxfp4_scaled_rows": 1})):
        a = _runner(c, **opts).moe(c.w, c.x, **kw)
        b = _runner(c, layout="aiter", **opts).moe(ws, c.x, **kw)
        torch.cuda.synchronize()
        n = int((a.view(torch.int16) != b.view(torch.int16)).sum())
        print(f"  {kw or opts or 'default'}: {n} elements differ from the row-major launch", flush=True)
        assert n == 0
    with pytest.raises(RuntimeError):
        _runner(c, (rows + 1, rows + 1), layout="aiter").moe(ws, c.x)


@pytest.mark.parametrize("bias_kind", ["zero", "coarse"])
@pytest.mark.parametrize("workload,rows", [("cfg1_plumbing_fp8", 4), ("cfg2_tp4_fp8", 1), ("cfg2_tp4_fp8", 16), ("cfg2_tp4_fp8", 24)])
def test_routing_ties(workload, rows, bias_kind):
    """Zero rows score 0.5 for every expert, so choices tie wherever the bias does: groups and
    experts then go by lower index, as in the oracle's stable sorts (1 row: every workgroup
    routes the step; 16 and 24: a workgroup a row)."""
    import dataclasses

    from oracle import routing as rt

    c = _case(workload, rows)
    e = c.p["experts"]
    if bias_kind == "zero":
        bias = np.zeros(e, np.float32)
    else:
        bias = ((np.arange(e) * 7) % 5).astype(np.float32) * np.float32(0.125)
    w = dataclasses.replace(c.w, bias=torch.from_numpy(bias).cuda())
    x = torch.zeros(rows, c.p["hidden"], dtype=torch.bfloat16, device="cuda")
    scores = rt.sigmoid_exact(np.zeros((rows, e), np.float32))
    want_ids, want_w = rt.grouped_topk(scores, bias, c.p["topk"], c.p["n_group"], c.p["topk_group"],
                                       c.p["routed_scale"], renorm=bool(c.p.get("renorm", True)))
    run = _runner(c)
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
    run.moe(w, x, topk_ids=ids, topk_w=wts)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert np.array_equal(ids.cpu().numpy(), want_ids), "expert ids"
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), want_w.view(np.uint32)), "routing weights"


@pytest.mark.parametrize("workload,rows", [("cfg2_tp4_fp8", 8), ("cfg2_tp4_fp8", 24)])
def test_routing_nan_row(workload, rows):
    """A row of NaN inputs: its logits are NaN, every choice -inf and every weight 0, so it
    picks the first topk experts of the first groups (the oracle's rule, stages/moe.py:345-347);
    the other rows' routing and outputs are those of the case without it."""
    from gpu_case import errors, within_bar

    from oracle import routing as rt

    c = _case(workload, rows)
    bad = 3
    x = c.x.clone()
    x[bad] = float("nan")
    xin = c.xin.clone()
    xin[bad] = float("nan")
    _, want_ids, want_w = rt.route(xin, gen_dense(c)["gate_w"], gen_dense(c)["bias"], c.p)
    assert want_ids[bad].tolist() == list(range(c.p["topk"])) and np.all(want_w[bad] == 0)
    run = _runner(c)
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
    out = run.moe(c.w, x, topk_ids=ids, topk_w=wts)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert np.array_equal(ids.cpu().numpy(), want_ids), "expert ids"
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), want_w.view(np.uint32)), "routing weights"
    assert bool((run.region("router_parts_polled") == 0xFF).all()), "polled part sums left unset"
    keep = [i for i, r in enumerate(c.check.tolist()) if r != bad]
    rows_kept = torch.from_numpy(c.check[keep]).cuda()
    e = errors(out[rows_kept].cpu(), c.ref[keep], c.chain[keep])
    assert within_bar(e, len(keep) * c.p["hidden"]), e


def gen_dense(c):
    from oracle import gen

    return gen.make_dense(c.p, 0)


@pytest.mark.parametrize(
    "workload,rows",
    [
        ("cfg2_tp4_fp8", 8),
        ("cfg3_tp4_mxfp4", 8),
        ("cfg5_tp2_mxfp4_norm", 1),
        ("cfg5_tp2_mxfp4_norm", 8),
        ("cfg5_tp2_mxfp4_norm", 16),
        ("cfg5_tp2_mxfp4_norm", 17),
        ("cfg5_tp2_mxfp4_norm", 24),
    ],
)
def test_activation_codes_bitexact(workload, rows):
    """The kernel's quantized x (and normed x) equal the oracle's bit for bit: up to 16 rows
    every workgroup norms the rows itself as it reads them (the quantize stores the normed
    rows), above the norm stage writes them before a hand-off."""
    from oracle import formats as fm

    c = _case(workload, rows)
    run = _runner(c)
    run.moe(c.w, c.x)
    torch.cuda.synchronize()
    h = c.p["hidden"]
    if c.p["norm_eps"] is not None:
        xn = run.region("x_normed")[: rows * h * 2].view(torch.bfloat16).cpu().reshape(rows, h)
        assert torch.equal(xn.view(torch.int16), c.xin.view(torch.int16)), "normed x"
    q, s = fm.group_fp8_quant(c.xin, 128)
    name_q, name_s = ("x_codes_shared", "x_scales_shared") if c.p["routed_fmt"] == "mxfp4" else ("x_codes", "x_scales")
    assert torch.equal(run.region(name_q)[: rows * h].cpu().reshape(rows, h), q), "group-128 codes"
    got_s = run.region(name_s)[: rows * (h // 128) * 4].view(torch.float32).cpu().reshape(rows, -1)
    assert torch.equal(got_s, s), "group-128 scales"
    if c.p["routed_fmt"] == "mxfp4":
        q, code = fm.mxfp8_quant(c.xin)
        assert torch.equal(run.region("x_codes")[: rows * h].cpu().reshape(rows, h), q), "MXFP8 codes"
        assert torch.equal(run.region("x_scales")[: rows * (h // 32)].cpu().reshape(rows, -1), code), "MXFP8 scales"


@pytest.mark.parametrize("workload,rows", [("cfg1_plumbing_fp8", 4), ("cfg2_tp4_fp8", 8), ("cfg3_tp4_mxfp4", 48), ("cfg5_tp2_mxfp4_norm", 8)])
def test_staged_equals_fused_and_repeats(workload, rows):
    c = _case(workload, rows)
    run = _runner(c)
    a = run.moe(c.w, c.x).clone()
    b = run.moe(c.w, c.x, staged=True).clone()
    d = run.moe(c.w, c.x).clone()
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "staged != fused"
    assert torch.equal(a.view(torch.int16), d.view(torch.int16)), "repeat differs"


def test_row_counts_in_turn_on_one_workspace():
    """Launches of changing row counts (local routing and the routing hand-off in turn) on one
    runner: each launch must find the hand-off flags and the polled part sums as the previous
    one left them, and be checked against its own oracle case."""
    run = None
    for rows in (4, 20, 1, 16, 3):
        c = _case("cfg1_plumbing_fp8", rows)
        if run is None:
            run = _runner(c)
        print(f"\ncfg1_plumbing_fp8 R={rows} on the shared workspace", flush=True)
        _check(c, rows, run, exact=False)


def test_graph_replay_bitwise():
    """Every row count of one preset in one graph, replayed with eager work between replays."""
    c = _case("cfg2_tp4_fp8", 8)
    run = _runner(c)
    xs = [c.x[:r].contiguous() for r in (1, 3, 8)]
    outs = [torch.empty(r, c.p["hidden"], dtype=torch.bfloat16, device="cuda") for r in (1, 3, 8)]
    for x, o in zip(xs, outs):
        run.moe(c.w, x, out=o)
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for x, o in zip(xs, outs):
                run.moe(c.w, x, out=o)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(6):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), f"replay {i}"
        run.moe(c.w, xs[1], out=outs[1])  # eager work between replays
        torch.cuda.synchronize()
    run.raise_on_device_error()


def test_device_e4m3_convert_equals_encoder_on_every_float():
    """The hardware e4m3 convert of the activation quantizers (after the +-448 clamp) against the
    integer-step encoder (host-pinned by the oracle tests) on all 2^32 fp32 patterns but inf and
    NaN, on the device: no code differs."""
    from sgl_amd_mono.moe import _lib

    L = _lib.testing_lib()
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    first_bad = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    for k in range(16):
        _lib.check(L.mkmoe_device_e4m3_sweep(k << 28, 1 << 28, bad.data_ptr(), first_bad.data_ptr(), None), "sweep")
    torch.cuda.synchronize()
    assert int(bad.item()) == 0, f"{int(bad.item())} codes differ, first at {int(first_bad.item()) & 0xffffffff:#010x}"


def test_graph_replay_bitwise_routing_handoff():
    """Rows 24 and 48 (the routing hand-off, stage Q) in one graph, replayed with eager work between."""
    c = _case("cfg2_tp4_fp8", 48)
    run = _runner(c)
    rows = (24, 48)
    xs = [c.x[:r].contiguous() for r in rows]
    outs = [torch.empty(r, c.p["hidden"], dtype=torch.bfloat16, device="cuda") for r in rows]
    for x, o in zip(xs, outs):
        run.moe(c.w, x, out=o)
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for x, o in zip(xs, outs):
                run.moe(c.w, x, out=o)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), f"replay {i}"
        run.moe(c.w, xs[0], out=outs[0])  # eager work between replays
        torch.cuda.synchronize()
    run.raise_on_device_error()


def test_host_validation_errors():
    c = _case("cfg1_plumbing_fp8", 4)
    run = _runner(c)
    with pytest.raises(RuntimeError, match="rows"):
        run.moe(c.w, torch.zeros(49, c.p["hidden"], dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(RuntimeError, match="out"):
        run.moe(c.w, c.x, out=torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda"))
    bad = type(c.w)(**{**c.w.__dict__, "gate_w": c.w.gate_w.float()})
    with pytest.raises(RuntimeError, match="gate_w"):
        run.moe(bad, c.x)


def test_golden_fixtures():
    """The kernel (its fixed-order VALU GEMVs) against the committed golden vectors
    (tests/golden/), bit for bit."""
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import make_golden as mg

    for workload, rows in mg.CASES:
        f = np.load(mg.case_file(workload, rows))
        c = _case(workload, rows)
        assert np.array_equal(c.x.view(torch.int16).cpu().numpy(), f["x_bits"]), "seeded x"
        run = _runner(c, (rows + 1, rows + 1))
        ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
        wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
        out = run.moe(c.w, c.x, topk_ids=ids, topk_w=wts)
        torch.cuda.synchronize()
        run.raise_on_device_error()
        print(f"\n{workload} R={rows} golden", flush=True)
        assert np.array_equal(ids.cpu().numpy(), f["ids"]), "expert ids"
        assert np.array_equal(wts.cpu().numpy().view(np.uint32), f["weights_bits"]), "routing weights"
        assert np.array_equal(out.view(torch.int16).cpu().numpy(), f["out_bits"]), "output bits"
