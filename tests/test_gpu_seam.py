"""The FFN seam's kernels against the oracle (``oracle/seam.py``), through the C ABI of
include/mkmoe_seam.h (``SeamRunner``): every output bit for bit at every token count the
reference's decode graphs use and at the maximum; graph replays; the reference test's own
bounds (``check_ffn.py:325-336``) against an fp64 residual as a cross-check."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H = 5120


def _inputs(tokens, seed):
    from oracle import gen

    return gen.seam_inputs(tokens, H, seed), gen.seam_weights(H, seed + 1)


def _oracle(i, w):
    from oracle import seam as sm

    return sm.ffn_seam(
        i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), i["comb"].numpy(), i["pre"].numpy(),
        w["fn"].numpy(), w["scale"].numpy(), w["base"].numpy(), w["norm"].float().numpy(),
    )  # fmt: skip


def _device(i, w):
    from sgl_amd_mono.moe.seam import SeamWeights

    dev = torch.device("cuda", 0)
    sw = SeamWeights(
        hc_ffn_fn=w["fn"].to(dev), hc_ffn_scale=w["scale"].to(dev), hc_ffn_base=w["base"].to(dev),
        ffn_norm=w["norm"].to(dev),
    )  # fmt: skip
    ins = (
        i["a"].to(dev), i["res"].to(dev), i["post"].reshape(-1, 4, 1).to(dev), i["comb"].to(dev), i["pre"].to(dev),
    )  # fmt: skip
    return sw, ins


def _bits_equal(dev_t, ref, what):
    got = dev_t.float().cpu().numpy().reshape(ref.shape).astype(np.float32)
    bad = got.view(np.uint32) != np.asarray(ref, np.float32).view(np.uint32)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} differ, first at {np.argwhere(bad)[0].tolist()}"


@pytest.mark.parametrize("tokens", [1, 2, 5, 8, 16, 24, 48, 64])
def test_seam_bitexact_against_oracle(tokens):
    from sgl_amd_mono.moe.seam import SeamRunner

    print(f"\nseam tokens={tokens}", flush=True)
    i, w = _inputs(tokens, 2000 + tokens)
    ref = _oracle(i, w)
    sw, ins = _device(i, w)
    run = SeamRunner()
    normed, res_out, post_out, comb_out, pre_out = run.ffn_seam(sw, *ins)
    torch.cuda.synchronize()
    _bits_equal(res_out, ref["res"], "res_out")
    _bits_equal(normed, ref["normed"], "normed")
    _bits_equal(pre_out, ref["pre"], "pre_out")
    _bits_equal(post_out, ref["post"], "post_out")
    _bits_equal(comb_out, ref["comb"], "comb_out")


def test_seam_reference_bounds_against_fp64():
    """The reference test's checks that need no SGLang: the residual within half a bf16 ulp of
    the fp64 hc_post and its correctly rounded value for all but 0.01 % of the elements; the
    comb's columns summing to 1 (the last Sinkhorn step) and its rows nearly; the normed rows'
    cosine to an fp64 RMSNorm > 0.9999."""
    from sgl_amd_mono.moe.seam import SeamRunner
    from test_oracle_seam import _hc_post_fp64, _residual_ok

    tokens = 48
    i, w = _inputs(tokens, 3000)
    sw, ins = _device(i, w)
    normed, res_out, post_out, comb_out, pre_out = SeamRunner().ffn_seam(sw, *ins)
    torch.cuda.synchronize()
    ref, big = _hc_post_fp64(i)
    assert _residual_ok(res_out.float().cpu().numpy(), ref, big)
    cb = comb_out.double().cpu()
    assert torch.allclose(cb.sum(1), torch.ones(tokens, 4, dtype=torch.float64), atol=1e-5)
    # the rows after 20 rounds: within 1 % for the peaked logits of these weights
    assert torch.allclose(cb.sum(2), torch.ones(tokens, 4, dtype=torch.float64), atol=1e-2)
    assert bool(((post_out > 0) & (post_out < 2)).all()) and bool(((pre_out > 0) & (pre_out < 1.001)).all())
    R = res_out.double().cpu()
    lin = (i["pre"].double()[:, :, None] * R).sum(1)
    n64 = lin / torch.sqrt((lin * lin).mean(1, keepdim=True) + 1e-20) * w["norm"].double()[None, :]
    cos = torch.nn.functional.cosine_similarity(normed.double().cpu().reshape(-1), n64.reshape(-1), dim=0)
    assert cos.item() > 0.9999


@pytest.mark.parametrize("tokens", [1, 8, 48])
def test_seam_gate_later_equals_one_call(tokens):
    """The norm first and the gate after other work on the stream give the one call's bits."""
    from sgl_amd_mono.moe.seam import SeamRunner

    print(f"\nseam gate_later tokens={tokens}", flush=True)
    i, w = _inputs(tokens, 5000 + tokens)
    sw, ins = _device(i, w)
    run = SeamRunner()
    one = [t.clone() for t in run.ffn_seam(sw, *ins)]
    torch.cuda.synchronize()
    outs = tuple(torch.full_like(t, -7) for t in one)
    run.ffn_seam(sw, *ins, outs=outs, gate_later=True)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), one[0].view(torch.int16))  # normed
    assert torch.equal(outs[1].view(torch.int16), one[1].view(torch.int16))  # res_out
    assert bool((outs[2] == -7).all() and (outs[3] == -7).all() and (outs[4] == -7).all())
    filler = torch.randn(1 << 20, device="cuda").sum()  # other work in between
    run.gate()
    torch.cuda.synchronize()
    assert torch.isfinite(filler)
    for a, b in zip(outs[2:], one[2:]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_seam_graph_replays_bitwise():
    from sgl_amd_mono.moe.seam import SeamRunner

    tokens = 8
    i, w = _inputs(tokens, 4000)
    sw, ins = _device(i, w)
    run = SeamRunner()
    eager = [t.clone() for t in run.ffn_seam(sw, *ins)]
    torch.cuda.synchronize()
    outs = tuple(torch.empty_like(t) for t in eager)
    run.workspace(tokens)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run.ffn_seam(sw, *ins, outs=outs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        run.ffn_seam(sw, *ins, outs=outs)
    for rep in range(4):
        for t in outs:
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)), rep
        # eager work between replays
        run.ffn_seam(sw, *ins)
        torch.cuda.synchronize()
