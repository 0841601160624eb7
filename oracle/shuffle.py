"""SGLang's loaded MXFP4 expert layout on gfx950 (aiter's shuffles), restated.

TEST INFRASTRUCTURE ONLY (the oracle): imported by ``tests/``, never by the product path.
The kernel reads this layout in place (``MKMOE_FMT_MXFP4_AITER``); the tests make it from the
row-major tensors with these functions and check that the kernel's output does not change.

SGLang's Fp8MoEMethod processes MXFP4 experts on gfx950 with aiter's
``shuffle_weight(w, is_guinterleave=True, gate_up=...)`` and ``shuffle_scale(s, E, True,
gate_up)`` (``test/kernels/deepseek_v41/check_ffn.py:169-173``). aiter is not in this image
and the reference pins no version (``pyproject.toml:12-13``), so the layouts are restated from
the reference kernel's own index math, which is what reads them:

- gate/up interleave (w13 and its scales): row groups of 16 alternate gate and up, so column
  block b's gate tile is row group 2 b and its up tile row group 2 b + 1
  (``deepseek_v41/gfx950/stages/moe.py:819-824`` ug_wave_pair, ``:568-591`` gemv_fp4_pair
  reading tiles rg0 and rg0 + 1 and scale rows t * 16 + lane % 16 of one 32-row block);
- (16, 16) shuffle (w13 after the interleave, and w2): a 16-row group's bytes are stored
  per 128-K step (64 bytes a row) as 1 KB in which lane l = m + 16 j of the scaled MFMA
  finds row m's K [32 j, 32 j + 32) at byte 16 l (``common/mx.py:47-57`` fp4_tile_load:
  dword base + rg * 2k + st * 256 + lane * 4, ``moe.py:696-714``);
- scale order: the E8M0 byte of (row, column) at ``scale_index`` (``common/mx.py:40-44``).

The functions take and return torch tensors of bytes (CPU or device) of the row-major shapes
of ``include/mkmoe.h``: w13 [E][2I][H/2], w13_s [E][2I][H/32], w2 [E][H][I/2], w2_s
[E][H][I/32]; the shuffled tensors keep those shapes.

Parity pins (tests/test_oracle_shuffle.py): the (16, 16) shuffle against the reference
kernel's per-lane address formula (``shuffled_offset``), element by element; scale_index's
hand-worked values and its bijectivity; the interleave against the gate/up tile rule above;
and every shuffle's inverse (round trips).
"""

from __future__ import annotations

import torch


def interleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """[..., 2N, X] gate rows then up rows -> row groups g0-15, u0-15, g16-31, u16-31, ..."""
    *lead, n2, x = w.shape
    n = n2 // 2
    assert n2 % 32 == 0
    return w.reshape(*lead, 2, n // 16, 16, x).transpose(-4, -3).reshape(*lead, n2, x).contiguous()


def deinterleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """The inverse of ``interleave_gate_up``."""
    *lead, n2, x = w.shape
    n = n2 // 2
    return w.reshape(*lead, n // 16, 2, 16, x).transpose(-4, -3).reshape(*lead, n2, x).contiguous()


def shuffle_16x16(w: torch.Tensor) -> torch.Tensor:
    """[..., N, Kb] bytes -> the (16, 16) shuffle: per 16-row group and 32-byte K chunk, the
    chunk's two 16-byte halves in turn, each holding the group's 16 rows."""
    *lead, n, kb = w.shape
    assert n % 16 == 0 and kb % 32 == 0
    return w.reshape(*lead, n // 16, 16, kb // 32, 2, 16).movedim(-4, -2).reshape(*lead, n, kb).contiguous()


def unshuffle_16x16(w: torch.Tensor) -> torch.Tensor:
    """The inverse of ``shuffle_16x16``."""
    *lead, n, kb = w.shape
    return w.reshape(*lead, n // 16, kb // 32, 2, 16, 16).movedim(-2, -4).reshape(*lead, n, kb).contiguous()


def shuffled_offset(row, kb, row_bytes: int):
    """Byte offset of byte ``kb`` of row ``row`` in a (16, 16)-shuffled [N][row_bytes] matrix,
    as the reference kernel addresses it: row group row // 16 (16 rows of row_bytes), K step
    kb // 64 (1 KB), lane (row % 16) + 16 * ((kb % 64) // 16) (16 bytes), byte kb % 16."""
    lane = row % 16 + 16 * ((kb % 64) // 16)
    return (row // 16) * 16 * row_bytes + (kb // 64) * 1024 + lane * 16 + kb % 16


def scale_index(row, col, cols: int):
    """The byte index of E8M0 scale (row, col) of a [rows][cols] scale matrix in aiter's
    shuffle_scale order (``common/mx.py:40-44``): 32-row blocks, in each 8-column chunks of
    [column % 4][row % 16][(column / 4) % 2][(row / 16) % 2]."""
    r32, a, b = row // 32, (row // 16) % 2, row % 16
    c8, d, e = col // 8, (col // 4) % 2, col % 4
    return ((((r32 * (cols // 8) + c8) * 4 + e) * 16 + b) * 2 + d) * 2 + a


def _scale_perm(rows: int, cols: int, device) -> torch.Tensor:
    r = torch.arange(rows, device=device).view(-1, 1)
    c = torch.arange(cols, device=device).view(1, -1)
    return scale_index(r, c, cols).reshape(-1)


def shuffle_scales(s: torch.Tensor) -> torch.Tensor:
    """[..., R, C] E8M0 bytes (R a multiple of 32, C of 8; the leading dims flattened into rows,
    as SGLang views them) -> the same shape in shuffle_scale order."""
    shape = s.shape
    flat = s.reshape(-1, shape[-1])
    rows, cols = flat.shape
    assert rows % 32 == 0 and cols % 8 == 0
    out = torch.empty(rows * cols, dtype=s.dtype, device=s.device)
    out[_scale_perm(rows, cols, s.device)] = flat.reshape(-1)
    return out.view(shape)


def unshuffle_scales(s: torch.Tensor) -> torch.Tensor:
    """The inverse of ``shuffle_scales``."""
    shape = s.shape
    rows, cols = s.reshape(-1, shape[-1]).shape
    return s.reshape(-1)[_scale_perm(rows, cols, s.device)].view(shape).contiguous()


def pad_scale_cols(s: torch.Tensor, mult: int = 8) -> torch.Tensor:
    """[..., C] E8M0 bytes with C padded to a multiple of ``mult`` by zero codes, as SGLang's
    loader pads w2's scales (``down_scale_cols``: I / 32 padded to a multiple of 8,
    ``stages/dims.py:54-56``)."""
    c = s.shape[-1]
    pad = -c % mult
    if pad == 0:
        return s
    return torch.cat([s, torch.zeros(*s.shape[:-1], pad, dtype=s.dtype, device=s.device)], -1)


def to_aiter(w13: torch.Tensor, w13_s: torch.Tensor, w2: torch.Tensor, w2_s: torch.Tensor):
    """Row-major MXFP4 experts -> SGLang's loaded gfx950 layout (check_ffn.py:170-173); w2's
    scale columns padded to a multiple of 8 first (``pad_scale_cols``)."""
    return (
        shuffle_16x16(interleave_gate_up(w13)),
        shuffle_scales(interleave_gate_up(w13_s)),
        shuffle_16x16(w2),
        shuffle_scales(pad_scale_cols(w2_s)),
    )


def from_aiter(w13: torch.Tensor, w13_s: torch.Tensor, w2: torch.Tensor, w2_s: torch.Tensor, w2_cols: int | None = None):
    """The inverse of ``to_aiter`` (w2_cols: w2's scale columns before the padding)."""
    s2 = unshuffle_scales(w2_s)
    return (
        deinterleave_gate_up(unshuffle_16x16(w13)),
        deinterleave_gate_up(unshuffle_scales(w13_s)),
        unshuffle_16x16(w2),
        s2 if w2_cols is None else s2[..., :w2_cols].contiguous(),
    )
