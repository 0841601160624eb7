"""The oracle's restatement of SGLang's loaded MXFP4 layout (aiter's shuffles) on gfx950.

No aiter in this image: the layouts are pinned against the reference kernel's own index
math (the per-lane address of fp4_tile_load, ``common/mx.py:47-57``; scale_index,
``common/mx.py:40-44``; the gate/up tile pair of ug_wave_pair, ``stages/moe.py:819-824``),
by hand-worked values, and by round trips.
"""

import itertools

import torch

from oracle import shuffle as sh


def _bytes(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)


def test_shuffle_matches_kernel_addressing():
    """Every byte lands where the reference kernel's lane loads read it."""
    n, kb = 48, 192  # three row groups, three 128-K steps
    w = _bytes(n, kb)
    s = sh.shuffle_16x16(w).reshape(-1)
    r = torch.arange(n).view(-1, 1).expand(n, kb)
    k = torch.arange(kb).view(1, -1).expand(n, kb)
    off = sh.shuffled_offset(r, k, kb)
    assert torch.equal(s[off.reshape(-1)], w.reshape(-1))
    # and so the scaled MFMA's lane (m, j) of step st reads 16 contiguous bytes: row m's K
    # [128 st + 32 j, + 32) (even K in the low nibble)
    for rg, st, m, j in itertools.product(range(3), range(3), (0, 7, 15), range(4)):
        lane = m + 16 * j
        got = s[rg * 16 * kb + st * 1024 + lane * 16 :][:16]
        assert torch.equal(got, w[rg * 16 + m, st * 64 + 16 * j : st * 64 + 16 * j + 16])


def test_shuffle_round_trips():
    w = _bytes(2, 64, 96, seed=1)
    assert torch.equal(sh.unshuffle_16x16(sh.shuffle_16x16(w)), w)
    assert not torch.equal(sh.shuffle_16x16(w), w)
    g = _bytes(3, 96, 40, seed=2)
    assert torch.equal(sh.deinterleave_gate_up(sh.interleave_gate_up(g)), g)
    s = _bytes(2, 64, 24, seed=3)
    assert torch.equal(sh.unshuffle_scales(sh.shuffle_scales(s)), s)
    w13, w13_s, w2, w2_s = _bytes(2, 64, 128, seed=4), _bytes(2, 64, 8, seed=5), _bytes(2, 256, 64, seed=6), _bytes(2, 256, 8, seed=7)
    back = sh.from_aiter(*sh.to_aiter(w13, w13_s, w2, w2_s))
    for a, b in zip(back, (w13, w13_s, w2, w2_s)):
        assert torch.equal(a, b)


def test_interleave_gate_up_tiles():
    """Column block b's gate tile is row group 2 b, its up tile row group 2 b + 1."""
    n = 64
    w = torch.arange(2 * n, dtype=torch.int32).view(2 * n, 1)  # row r holds r
    it = sh.interleave_gate_up(w).view(-1)
    for b in range(n // 16):
        for m in range(16):
            assert it[32 * b + m] == 16 * b + m  # gate row 16 b + m
            assert it[32 * b + 16 + m] == n + 16 * b + m  # up row 16 b + m


def test_scale_index_values():
    """Hand-worked positions: the fastest index is the row's 16-row half, then the column's
    4-column half, then the row within 16, then the column within 4, then 8-column chunks,
    then 32-row blocks."""
    assert sh.scale_index(0, 0, 8) == 0
    assert sh.scale_index(16, 0, 8) == 1
    assert sh.scale_index(0, 4, 8) == 2
    assert sh.scale_index(1, 0, 8) == 4
    assert sh.scale_index(0, 1, 8) == 64
    assert sh.scale_index(0, 8, 16) == 256
    assert sh.scale_index(32, 0, 8) == 256
    assert sh.scale_index(32, 0, 16) == 512
    assert sh.scale_index(31, 7, 8) == 255
    # a bijection of [0, R C)
    r, c = 64, 24
    idx = sh.scale_index(torch.arange(r).view(-1, 1), torch.arange(c).view(1, -1), c).reshape(-1)
    assert torch.equal(torch.sort(idx).values, torch.arange(r * c))


def test_scale_dword_per_lane_and_step_pair():
    """What the kernel's scale loads rely on: for a 32-row block (gate rows 16 b .. and up rows
    16 b .. after the interleave), lane (m, j)'s scale bytes of K steps 2 c and 2 c + 1, gate and
    up, are the four bytes of one dword: byte 2 (step % 2) + (up)."""
    rows, cols = 64, 16  # two 32-row blocks, four K steps of 128
    s = _bytes(rows, cols, seed=8)
    flat = sh.shuffle_scales(s).reshape(-1)
    for blk, c8, m, j in itertools.product(range(2), range(2), (0, 5, 15), range(4)):
        dw = blk * 32 * cols + c8 * 256 + (j * 16 + m) * 4
        for st in (2 * c8, 2 * c8 + 1):
            for q in range(2):
                assert flat[dw + 2 * (st % 2) + q] == s[32 * blk + 16 * q + m, 4 * st + j]


def test_padded_down_scales_v41():
    """V4.1's w2 scales: 640 / 32 = 20 E8M0 columns padded by zero codes to 24 (stages/dims.py:
    54-56), shuffled over the padded width; the kernel reads a row's K steps from the dword at
    32-row block h / 32 (24 * 32 bytes each), chunk c (256 bytes), position 16 j + h % 16, and
    from_aiter(w2_cols=20) gives the 20 columns back. A 16-column matrix (I = 512) is left as it is."""
    s = _bytes(2, 96, 20, seed=9)
    p = sh.pad_scale_cols(s)
    assert p.shape == (2, 96, 24) and torch.equal(p[..., :20], s) and not p[..., 20:].any()
    s16 = _bytes(96, 16, seed=10)
    assert sh.pad_scale_cols(s16) is s16
    flat = sh.shuffle_scales(p).reshape(2, -1)
    for e, h, st, j in itertools.product(range(2), (0, 17, 40, 95), range(5), range(4)):
        c = st // 2
        dw = (h // 32) * 24 * 32 + c * 256 + (16 * j + h % 16) * 4
        assert flat[e, dw + 2 * (st % 2) + (h // 16) % 2] == s[e, h, 4 * st + j]
    w13, w13_s, w2 = _bytes(2, 64, 128, seed=11), _bytes(2, 64, 8, seed=12), _bytes(2, 96, 320, seed=13)
    back = sh.from_aiter(*sh.to_aiter(w13, w13_s, w2, s), w2_cols=20)
    assert torch.equal(back[3], s) and torch.equal(back[2], w2)
