"""The reference's own MoE shape on an MI355X: DeepSeek-V4.1 at TP4 and TP2, through the C ABI.

Hidden 5120, 384 experts, top-6 by sqrt(softplus) over one group (routed scale 1.5), MXFP4
routed experts in SGLang's loaded gfx950 layout (TP4: the rank's 576 columns padded to 640 with
zero weights, w2's scale columns padded to 24; TP2: 1152 columns, w2's 36 scale columns padded
to 40), and the shared expert's rank share (576 or 1152 columns) in FP8 with E8M0 32 x 32
scales, its activations and intermediate quantized by the MXFP8 "vllm" rule
(the tensors ``check_ffn.py:128-182`` makes, ``FFNWeights`` at ``gfx950/runner.py:130-168``).
The weights are generated as ``make_weights`` draws them, row-major on the CPU, and shuffled
by the oracle's restatement of aiter's layout.

Bars: router part sums, the activation codes of both rules, expert ids and routing weights bit
for bit; the bf16 output of every row against the golden's fp32-matmul form
(``golden_partial``, check_ffn.py:209-232): every element within two bf16 ulps of the largest
magnitude its combine chain held, relative L2 <= 1e-2 and the reference's cosine bound 0.9999
(``ffn.moe.cosine``, spec.py:305-309). (The reference test's weights give outputs up to |out|
~ 30, where one bf16 ulp is 0.125, so the absolute 2e-2 of the DeepSeek-V3 workloads' bar is
not a meaningful cut here: its own bar for this shape is relative.) Persistent and staged
launches bit for bit alike; graph replays bitwise.
"""

import dataclasses

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

WORKLOAD = "v41_tp4_mxfp4"
TP2 = "v41_tp2_mxfp4"
_cache = {}


def _case(rows, workload=WORKLOAD):
    from gpu_case import build

    from oracle import shuffle as sh

    if (workload, rows) not in _cache:
        _cache.clear()
        torch.cuda.empty_cache()
        c = build(workload, rows)
        w13, w13_s, w2, w2_s = sh.to_aiter(c.w.w13, c.w.w13_s, c.w.w2, c.w.w2_s)
        # SGLang's views: fp4x2 weights, the scales as flat [E rows][cols] byte matrices
        w = dataclasses.replace(
            c.w, w13=w13, w13_s=w13_s.reshape(-1, w13_s.shape[-1]), w2=w2, w2_s=w2_s.reshape(-1, w2_s.shape[-1])
        )
        _cache[(workload, rows)] = dataclasses.replace(c, w=w)
    return _cache[(workload, rows)]


def _runner(c):
    from sgl_amd_mono.moe.runner import MoeRunner

    return MoeRunner(c.preset, "cuda")


@pytest.mark.parametrize(
    "workload,rows", [(WORKLOAD, r) for r in (1, 2, 8, 9, 16, 17, 24, 48)] + [(TP2, r) for r in (1, 4, 5, 8, 9, 16, 17, 48)]
)
def test_parity_v41(workload, rows):
    from gpu_case import errors, record_accuracy

    from oracle import formats as fm

    c = _case(rows, workload)
    i, s = c.p["inter"], c.p["shared_inter"]
    assert c.w.w2_s.shape == (384 * 5120, -(-i // 32 // 8) * 8) and c.w.sgu_s.shape == (2 * s // 32, 160)
    run = _runner(c)
    print(f"\n{workload} R={rows} (aiter layout, MX shared expert)", flush=True)
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    wts = torch.zeros(rows, c.p["topk"], dtype=torch.float32, device="cuda")
    out = run.moe(c.w, c.x, topk_ids=ids, topk_w=wts)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    e, p_ = c.p["experts"], c.p["router_parts"]
    parts = run.region("router_parts")[: rows * e * p_ * 4].view(torch.float32).cpu().numpy().reshape(rows, p_, e)
    assert np.array_equal(np.ascontiguousarray(parts.transpose(0, 2, 1)).view(np.uint32), c.parts.view(np.uint32)), "router part sums"
    assert bool((run.region("router_parts_polled") == 0xFF).all()), "polled part sums left unset"
    assert np.array_equal(ids.cpu().numpy(), c.ids), "expert ids"
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), c.wts.view(np.uint32)), "routing weights"
    # the activation codes: MXFP8 "aiter" for the routed experts, "vllm" for the shared one
    h = c.p["hidden"]
    for rule, qn, sn in (("aiter", "x_codes", "x_scales"), ("vllm", "x_codes_shared", "x_scales_shared")):
        q, code = fm.mxfp8_quant(c.xin, rule)
        assert torch.equal(run.region(qn)[: rows * h].cpu().reshape(rows, h), q), f"{rule} codes"
        assert torch.equal(run.region(sn)[: rows * (h // 32)].cpu().reshape(rows, -1), code), f"{rule} scales"
    g = errors(out.cpu(), c.golden, c.chain)
    print(f"  all {rows} rows vs fp32-matmul golden: {g}", flush=True)
    record_accuracy(workload, rows, "default", g, g, True)
    assert not g["nan"] and g["n_over_bar"] == 0 and g["rel_l2"] <= 1e-2 and g["cos"] >= 0.9999, g


@pytest.mark.parametrize("rows", [1, 8, 48])
def test_parity_v41_scaled_down(rows):
    """The down GEMM on the scaled fp4 x fp8 MFMA (the reference's instruction,
    common/mx.py:60-66), held to the reference's own bound against the golden (relative L2 and
    cosine, spec.py:305-309). It misses the element bar on this shape (8 rows: 2 elements past
    two bf16 ulps, 181 of 40960 past 2e-2, where the default path is bit-identical to the
    golden), so the library keeps it off here by default; the case records how far it lands."""
    from gpu_case import errors, record_accuracy

    from sgl_amd_mono.moe.runner import MoeRunner

    c = _case(rows)
    run = MoeRunner(c.preset, "cuda", mxfp4_scaled_down_rows=1)
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    out = run.moe(c.w, c.x, topk_ids=ids)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert np.array_equal(ids.cpu().numpy(), c.ids), "expert ids"
    g = errors(out.cpu(), c.golden, c.chain)
    print(f"\n{WORKLOAD} R={rows} scaled down vs fp32-matmul golden: {g}", flush=True)
    record_accuracy(WORKLOAD, rows, "scaled_down", g, g, True)
    assert not g["nan"] and g["rel_l2"] <= 1e-2 and g["cos"] >= 0.9999, g


@pytest.mark.parametrize("rows", [1, 8])
def test_v41_padding_never_read(rows):
    """The loader's padding (gate and up rows 576 .. 639, w2's K columns 576 .. 639 and their
    E8M0 scales) is never read: filled with random codes and NaN scales (0xFF), the output is
    bit for bit the zero-padded launch's. 1 row quantizes the intermediates in each workgroup,
    8 rows once (stage Q)."""
    from gpu_case import build

    from oracle import shuffle as sh

    c = _case(rows)
    run = _runner(c)
    ref = run.moe(c.w, c.x).clone()
    raw = build(WORKLOAD, rows).w  # row-major, zero-padded
    i, ir = c.p["inter"], c.p["inter_real"]
    g = torch.Generator(device="cuda").manual_seed(7)
    w13, w13_s, w2, w2_s = raw.w13.clone(), raw.w13_s.clone(), raw.w2.clone(), raw.w2_s.clone()
    del raw
    for half in (0, i):
        rows_ = slice(half + ir, half + i)
        w13[:, rows_] = torch.randint(0, 256, w13[:, rows_].shape, generator=g, device="cuda", dtype=torch.uint8)
        w13_s[:, rows_] = 0xFF
    w2[:, :, ir // 2 :] = torch.randint(0, 256, w2[:, :, ir // 2 :].shape, generator=g, device="cuda", dtype=torch.uint8)
    w2_s[:, :, ir // 32 :] = 0xFF
    a13, a13_s, a2, a2_s = sh.to_aiter(w13, w13_s, w2, w2_s)
    del w13, w13_s, w2, w2_s
    w = dataclasses.replace(
        c.w, w13=a13, w13_s=a13_s.reshape(-1, a13_s.shape[-1]), w2=a2, w2_s=a2_s.reshape(-1, a2_s.shape[-1])
    )
    out = run.moe(w, c.x)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), "the padding changed the output"


@pytest.mark.parametrize("workload,rows", [(WORKLOAD, 8), (WORKLOAD, 48), (TP2, 8)])
def test_v41_staged_equals_fused_and_repeats(workload, rows):
    c = _case(rows, workload)
    run = _runner(c)
    a = run.moe(c.w, c.x).clone()
    b = run.moe(c.w, c.x, staged=True).clone()
    d = run.moe(c.w, c.x).clone()
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "staged != fused"
    assert torch.equal(a.view(torch.int16), d.view(torch.int16)), "repeat differs"


@pytest.mark.parametrize("workload", [WORKLOAD, TP2])
def test_v41_graph_replay_bitwise(workload):
    """Row counts on both sides of the routing hand-off and of stage Q in one graph, replayed
    with eager work between the replays."""
    c = _case(48, workload)
    run = _runner(c)
    counts = (1, 8, 24, 48)
    xs = [c.x[:r].contiguous() for r in counts]
    outs = [torch.empty(r, c.p["hidden"], dtype=torch.bfloat16, device="cuda") for r in counts]
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
        run.moe(c.w, xs[1], out=outs[1])
        torch.cuda.synchronize()
    run.raise_on_device_error()


@pytest.mark.parametrize("rows", [1, 8, 48])
def test_v41_ffn_chain(rows):
    """The FFN entry point (``FfnRunner.ffn``: the seam, the MoE block on the seam's normed
    rows, then the seam's gate) against its parts: every seam output bit for bit the seam's
    own launch's, the partial bit for bit the MoE launch's on those normed rows, and the
    routing of the normed rows the oracle's; then a captured graph of the call, replayed."""
    from oracle import gen
    from oracle import routing as rt
    from sgl_amd_mono.moe.ffn import FfnRunner, FfnWeights
    from sgl_amd_mono.moe.runner import MoeRunner
    from sgl_amd_mono.moe.seam import SeamRunner

    c = _case(rows)
    si = {k: v.to("cuda") for k, v in gen.seam_inputs(rows, c.p["hidden"], 300 + rows).items()}
    sw = {k: v.to("cuda") for k, v in gen.seam_weights(c.p["hidden"], 300).items()}
    m = c.w
    fw = FfnWeights(
        hc_ffn_fn=sw["fn"], hc_ffn_scale=sw["scale"], hc_ffn_base=sw["base"], ffn_norm=sw["norm"], gate_w=m.gate_w,
        bias=m.bias, w13=m.w13, w13_s=m.w13_s, w2=m.w2, w2_s=m.w2_s, sgu=m.sgu, sgu_s=m.sgu_s, sw2=m.sw2, sw2_s=m.sw2_s,
    )  # fmt: skip
    args = (si["a"], si["res"], si["post"], si["comb"], si["pre"])
    ffn = FfnRunner(c.preset, "cuda")
    ids = torch.zeros(rows, c.p["topk"], dtype=torch.int32, device="cuda")
    outs = ffn.ffn(fw, *args, topk_ids=ids)
    seam = SeamRunner("cuda").ffn_seam(fw.seam(), *args)
    moe = MoeRunner(c.preset, "cuda").moe(m, seam[0])
    torch.cuda.synchronize()
    ffn.moe_runner.raise_on_device_error()
    assert torch.equal(ffn.normed(rows).view(torch.int16), seam[0].view(torch.int16)), "normed rows"
    assert torch.equal(outs[0].view(torch.int16), moe.view(torch.int16)), "the MoE partial"
    for k, name in enumerate(("res_out", "post_out", "comb_out", "pre_out"), start=1):
        assert torch.equal(outs[k].reshape(-1).view(torch.int16 if k == 1 else torch.int32),
                           seam[k].reshape(-1).view(torch.int16 if k == 1 else torch.int32)), name  # fmt: skip
    xin = seam[0].cpu()
    parts = rt.router_part_sums(xin, m.gate_w.cpu(), c.p["router_parts"])
    scores = rt.score_exact(rt.logits_from_parts(parts), c.p["scoring"])
    want, _ = rt.grouped_topk(scores, m.bias.cpu().numpy(), c.p["topk"], c.p["n_group"], c.p["topk_group"],
                              c.p["routed_scale"])  # fmt: skip
    assert np.array_equal(ids.cpu().numpy(), want), "expert ids of the normed rows"
    # one captured graph of the call, replayed with eager work between the replays
    ref = [t.clone() for t in outs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ffn.ffn(fw, *args, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        for t in outs:
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for t, r in zip(outs, ref):
            assert torch.equal(t, r), f"replay {i}"
        ffn.ffn(fw, *args)
        torch.cuda.synchronize()
    ffn.moe_runner.raise_on_device_error()


def test_v41_refuses_row_major_and_valu():
    """The V4.1 specialisation reads SGLang's layout alone and runs every GEMM on MFMA."""
    from sgl_amd_mono.moe.runner import MoeRunner

    c = _case(1)
    with pytest.raises((RuntimeError, ValueError)):
        MoeRunner(c.preset, "cuda", layout="row_major")
    with pytest.raises(RuntimeError):
        MoeRunner(c.preset, "cuda", mfma_rows=(2, 2)).moe(c.w, c.x)
