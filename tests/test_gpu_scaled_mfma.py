"""Known-answer tests of v_mfma_scale_f32_16x16x128_f8f6f4 (through mkmoe_device_mfma_scaled).

The MXFP4 option of the expert GEMMs (mkmoe_options.mxfp4_scaled_rows) runs this
instruction with the layout pinned here; the reference runs it through FlyDSL
(``common/mx.py:60-66``, ``stages/moe.py:724-745``). Each tile is one 16 x 16 x 128 product
C[m][n] = sum_k A[m][k] 2^(sa[m][k / 32] - 127) B[n][k] 2^(sb[n][k / 32] - 127), against the
exact dot (float64, exact at these ranges):

- layout: A lane (m, j) holds row m's K [32 j, 32 j + 32) (e2m1: 16 bytes, even K in the low
  nibble; e4m3: the same 32 K as bytes, split like B), B lane (n, j) column n's K
  [16 j, 16 j + 16) in bytes 0-15 and [64 + 16 j, 64 + 16 j + 16) in bytes 16-31, and each
  lane the E8M0 code of its row's / column's 32-K block j. With exactly summable operands the
  result is the exact dot, bit for bit; the same bytes read in any other of the layouts
  considered are far off (the test checks that it tells them apart).
- accuracy, in units of 2^-24 * sum |products| (a correctly rounded fp32 dot is within 0.5):
  realistic MX operands (MXFP4 of N(0, 0.02) weights, MXFP8 of N(0, 1) activations, as the
  kernel's inputs are made) and e4m3 x e4m3, each below a bound measured on gfx950.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TILES = 256
# measured on gfx950 (max over the tiles below), with margin
BOUND_FP4_MX = 400.0  # measured 147 (mean 3.6)
BOUND_FP8 = 8000.0  # measured 2860 (mean 304) here, up to 4410 on other draws


def _e4m3_values():
    from oracle import formats as fm

    return fm.e4m3_table()


def _fp4_values():
    from oracle import formats as fm

    return np.array(fm.FP4_VALUES, np.float64)


def _pack_fp4(c4):
    """[T, 16, 128] e2m1 codes -> [T, 64, 8] words (lane m + 16 j: K 32 j .. 32 j + 31)."""
    t = c4.shape[0]
    out = np.zeros((t, 64, 32), np.uint8)
    for j in range(4):
        blk = c4[:, :, 32 * j : 32 * j + 32]
        out[:, 16 * j : 16 * j + 16, :16] = (blk[:, :, 0::2] | (blk[:, :, 1::2] << 4)).astype(np.uint8)
    return out.view(np.uint32).reshape(t, 64, 8)


def _pack_fp8(c8, split=True):
    """[T, 16, 128] e4m3 codes -> [T, 64, 8] words (split: lane r + 16 j bytes 0-15 = K 16 j ..,
    bytes 16-31 = K 64 + 16 j ..; else K 32 j .. 32 j + 31)."""
    t = c8.shape[0]
    out = np.zeros((t, 64, 32), np.uint8)
    for j in range(4):
        if split:
            out[:, 16 * j : 16 * j + 16, :16] = c8[:, :, 16 * j : 16 * j + 16]
            out[:, 16 * j : 16 * j + 16, 16:] = c8[:, :, 64 + 16 * j : 64 + 16 * j + 16]
        else:
            out[:, 16 * j : 16 * j + 16, :] = c8[:, :, 32 * j : 32 * j + 32]
    return out.view(np.uint32).reshape(t, 64, 8)


def _pack_scales(s):
    """[T, 16, 4] E8M0 codes -> [T, 64] words (lane r + 16 j: block j of row r)."""
    return np.ascontiguousarray(s.transpose(0, 2, 1).reshape(s.shape[0], 64)).astype(np.uint32)


def _run(a_words, b_words, sa, sb, fmt_a):
    from sgl_amd_mono.moe import _lib

    t = a_words.shape[0]
    dev = [torch.from_numpy(np.ascontiguousarray(v).view(np.int32)).cuda() for v in (a_words, b_words, sa, sb)]
    d = torch.zeros(t, 64, 4, dtype=torch.float32, device="cuda")
    rc = _lib.testing_lib().mkmoe_device_mfma_scaled(
        *(x.data_ptr() for x in dev), d.data_ptr(), fmt_a, t, torch.cuda.current_stream().cuda_stream
    )
    _lib.check(rc, "mkmoe_device_mfma_scaled")
    torch.cuda.synchronize()
    d = d.cpu().numpy()
    c = np.zeros((t, 16, 16), np.float32)
    for m in range(16):
        c[:, m, :] = d[:, 16 * (m // 4) : 16 * (m // 4) + 16, m % 4]
    return c


def _exact(av, sa, bv, sb):
    """float64 dot and sum |products| of A [T, 16, 128] and B [T, 16, 128] values with block codes."""
    fa = av * np.exp2(np.repeat(sa.astype(np.float64) - 127, 32, axis=2))
    fb = bv * np.exp2(np.repeat(sb.astype(np.float64) - 127, 32, axis=2))
    dot = np.einsum("tmk,tnk->tmn", fa, fb)
    sabs = np.einsum("tmk,tnk->tmn", np.abs(fa), np.abs(fb))
    return dot, sabs


def _rel(got, dot, sabs):
    return np.abs(got.astype(np.float64) - dot) / np.maximum(sabs * 2.0**-24, 1e-300)


def _narrow_fp8(rng, shape):
    """e4m3 codes with |v| in [2^-3, 8): exponent field 4 .. 10, random sign and mantissa."""
    e = rng.integers(4, 11, shape)
    m = rng.integers(0, 8, shape)
    return ((rng.integers(0, 2, shape) << 7) | (e << 3) | m).astype(np.uint8)


def test_fp4_fp8_layout_exact():
    """Exactly summable e2m1 x e4m3 with unit scales: the exact dot, bit for bit; the same bytes
    under the other layouts considered land far away."""
    rng = np.random.default_rng(1)
    c4 = rng.integers(0, 16, (TILES, 16, 128)).astype(np.uint8)
    c8 = _narrow_fp8(rng, (TILES, 16, 128))
    ones = np.full((TILES, 16, 4), 127, np.uint8)
    got = _run(_pack_fp4(c4), _pack_fp8(c8), _pack_scales(ones), _pack_scales(ones), 4)
    av, bv = _fp4_values()[c4], _e4m3_values()[c8]
    dot, _ = _exact(av, ones, bv, ones)
    assert np.array_equal(got, dot.astype(np.float32)), "scaled MFMA layout"
    # the B bytes read as contiguous 32-K blocks (the bf16 path's layout) would give another dot
    c8_contig = _pack_fp8(c8, split=False)
    got2 = _run(_pack_fp4(c4), c8_contig, _pack_scales(ones), _pack_scales(ones), 4)
    assert np.abs(got2 - dot).max() > 1.0, "the test must tell the layouts apart"


def test_fp4_fp8_block_scales():
    """The E8M0 code of each 32-K block scales that block's products (narrow values: within
    2 units of 2^-24 sum |p| of the exact dot; a correct fp32 rounding is within 0.5)."""
    rng = np.random.default_rng(2)
    c4 = rng.integers(0, 16, (TILES, 16, 128)).astype(np.uint8)
    c8 = _narrow_fp8(rng, (TILES, 16, 128))
    sa = rng.integers(124, 131, (TILES, 16, 4)).astype(np.uint8)
    sb = rng.integers(124, 131, (TILES, 16, 4)).astype(np.uint8)
    got = _run(_pack_fp4(c4), _pack_fp8(c8), _pack_scales(sa), _pack_scales(sb), 4)
    dot, sabs = _exact(_fp4_values()[c4], sa, _e4m3_values()[c8], sb)
    r = _rel(got, dot, sabs)
    print(f"\nfp4 x fp8, narrow values, block scales: err / (2^-24 sum|p|) max {r.max():.3g} mean {r.mean():.3g}")
    assert r.max() <= 2.0


def test_fp4_fp8_mx_operands_bound():
    """The kernel's own operands: MXFP4 of N(0, 0.02) rows times MXFP8 ("aiter" rule) of
    N(0, 1) columns, with their block codes. The instruction's sum keeps fewer bits than fp32:
    bounded here, and far from the bf16 path's 0.42."""
    from oracle import formats as fm

    g = torch.Generator().manual_seed(3)
    w = torch.randn(TILES * 16, 128, generator=g) * 0.02
    x = torch.randn(TILES * 16, 128, generator=g)
    packed, wcode = fm.quant_mxfp4(w)
    xq, xcode = fm.mxfp8_quant(x)
    p = packed.numpy().reshape(TILES, 16, 64)
    c4 = np.stack([p & 15, p >> 4], axis=-1).reshape(TILES, 16, 128).astype(np.uint8)
    c8 = xq.view(torch.uint8).numpy().reshape(TILES, 16, 128)
    sa = wcode.view(torch.uint8).numpy().reshape(TILES, 16, 4)
    sb = xcode.numpy().astype(np.uint8).reshape(TILES, 16, 4)
    got = _run(_pack_fp4(c4), _pack_fp8(c8), _pack_scales(sa), _pack_scales(sb), 4)
    dot, sabs = _exact(_fp4_values()[c4], sa, _e4m3_values()[c8], sb)
    r = _rel(got, dot, sabs)
    exact = float((got == dot.astype(np.float32)).mean())
    print(f"\nfp4 x fp8, MX operands: err / (2^-24 sum|p|) max {r.max():.3g} mean {r.mean():.3g}; "
          f"{100 * exact:.1f}% of the outputs are the rounded exact dot")
    assert r.max() <= BOUND_FP4_MX


def test_fp8_fp8_bound():
    """e4m3 x e4m3 (unit scales, as a 128 x 128-scaled FP8 GEMM would use it): bounded, and
    not exact even on narrow values, which is why the FP8 expert GEMMs convert to bf16."""
    rng = np.random.default_rng(4)
    e4 = _e4m3_values()
    ok = np.where(~np.isnan(e4))[0].astype(np.uint8)
    ca = rng.choice(ok, (TILES, 16, 128))
    cb = rng.choice(ok, (TILES, 16, 128))
    ones = np.full((TILES, 16, 4), 127, np.uint8)
    got = _run(_pack_fp8(ca), _pack_fp8(cb), _pack_scales(ones), _pack_scales(ones), 0)
    dot, sabs = _exact(e4[ca], ones, e4[cb], ones)
    r = _rel(got, dot, sabs)
    print(f"\nfp8 x fp8, all finite codes: err / (2^-24 sum|p|) max {r.max():.3g} mean {r.mean():.3g}")
    assert r.max() <= BOUND_FP8
    cn = _narrow_fp8(rng, (2, TILES, 16, 128))
    got = _run(_pack_fp8(cn[0]), _pack_fp8(cn[1]), _pack_scales(ones), _pack_scales(ones), 0)
    dot, sabs = _exact(e4[cn[0]], ones, e4[cn[1]], ones)
    print(f"fp8 x fp8, narrow codes: {100 * float((got == dot.astype(np.float32)).mean()):.1f}% exact")
    assert not np.array_equal(got, dot.astype(np.float32))
