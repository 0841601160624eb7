"""The expert GEMVs and SwiGLU in the exact order the kernel computes them.

TEST INFRASTRUCTURE ONLY (the oracle): imported by ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg.

The reference's golden model multiplies with fp32 matmuls of unspecified
order (``test/kernels/deepseek_v41/check_ffn.py:218,221,226,231``); its kernel
uses MFMA tiles. Neither order can be restated bit for bit, and the gfx950
scaled MFMA's internal accumulation is not an exact dot product rounded once
(measured), so the kernel computes every expert GEMV on the vector ALUs in the
fixed order below, and this module restates it. A GEMV of a weight row w
(length K) with an activation row x:

1. chunks of CE = 16 elements (FP8 weights) or 32 (MXFP4 weights); the chunk's
   unscaled sum d = 0 + w_0 x_0 + w_1 x_1 + ... in element order, in fp32. The
   products of e4m3 x e4m3 and e2m1 x e4m3 codes are exact in fp32, so an FMA
   chain gives the same sum.
2. the chunk's scale: FP8 128 x 128: v = d * fp32(s_w * s_x) with s_w the
   weight block's fp32 scale and s_x the activation group's (128 wide); MXFP4:
   v = d * 2^(e_w + e_x - 254) (exact) with the E8M0 codes of the chunk.
3. the row's chunks are dealt to LPR lanes, chunk c to lane c mod LPR; each
   lane sums its chunks in order from 0; the LPR lane sums are added as a
   halving tree (lanes l and l + d, d = LPR/2 .. 1). For the gate_up GEMVs
   LPR is 64 when the row has a multiple of 64 chunks, else 32, 16 or 8 (the
   largest that divides); the down GEMVs (routed and shared) use LPR = 8.

SwiGLU uses silu(z) = fp32(z * sigmoid(z)) with the exact fp64 sigmoid of
``oracle.routing`` (the same steps as the routing's scores), not torch's silu.

Parity pins (tests/test_oracle_exact.py): the exact GEMV against an fp64
matmul of the dequantized operands (within fp32 accumulation error) and
against an index-by-index scalar restatement on small shapes.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as fm
from . import routing as rt


# lanes a row of the down GEMVs (routed and shared): chunk c to lane c mod 8
DOWN_LANES = 8


def lanes_per_row(chunks: int) -> int:
    """Lanes a row of the gate_up GEMVs: the largest of 64, 32, 16, 8 that divides the chunks."""
    for lpr in (64, 32, 16, 8):
        if chunks % lpr == 0:
            return lpr
    raise ValueError(chunks)


def _tree(a: np.ndarray) -> np.ndarray:
    d = a.shape[-1] // 2
    while d >= 1:
        a = a[..., :d] + a[..., d : 2 * d]
        d //= 2
    return a[..., 0]


def _chunk_sums(wv: np.ndarray, xv: np.ndarray, ce: int) -> np.ndarray:
    """d[t, n, c]: sequential fp32 sums of the exact products of chunk c."""
    n, k = wv.shape
    t = xv.shape[0]
    c = k // ce
    w3 = wv.reshape(n, c, ce)
    x3 = xv.reshape(t, c, ce)
    d = np.zeros((t, n, c), np.float32)
    for i in range(ce):
        d = d + x3[:, None, :, i] * w3[None, :, :, i]
    return d


def _lanes(v: np.ndarray, lpr: int | None = None) -> np.ndarray:
    """Deal chunks to lanes (lpr lanes a row, by default ``lanes_per_row``), sum each lane
    in order, then the halving tree -> [T, N]."""
    t, n, c = v.shape
    lpr = lanes_per_row(c) if lpr is None else lpr
    if c % lpr:
        raise ValueError((c, lpr))
    v4 = v.reshape(t, n, c // lpr, lpr)
    a = np.zeros((t, n, lpr), np.float32)
    for i in range(c // lpr):
        a = a + v4[:, :, i, :]
    return _tree(a)


def gemv_fp8_b128(wq: torch.Tensor, ws: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor, lpr: int | None = None) -> np.ndarray:
    """[N, K] e4m3 codes with fp32 [N/128, K/128] scales . [T, K] e4m3 codes with fp32 [T, K/128] -> [T, N]."""
    wv = fm.e4m3_to_f32(wq).numpy().astype(np.float32)
    xv = fm.e4m3_to_f32(xq).numpy().astype(np.float32)
    n, k = wv.shape
    d = _chunk_sums(wv, xv, 16)
    ws_ = ws.float().numpy().astype(np.float32)
    xs_ = xs.float().numpy().astype(np.float32)
    blk = np.arange(k // 16) // 8  # the chunk's 128-wide K block
    rowblk = np.arange(n) // 128
    f = ws_[rowblk][:, blk][None, :, :] * xs_[:, blk][:, None, :]  # fp32(s_w * s_x)
    return _lanes((d * f).astype(np.float32), lpr)


def gemv_mxfp4(wq: torch.Tensor, ws: torch.Tensor, xq: torch.Tensor, xs: torch.Tensor, lpr: int | None = None) -> np.ndarray:
    """[N, K/2] e2m1 with E8M0 [N, K/32] . [T, K] e4m3 codes with E8M0 [T, K/32] -> [T, N]."""
    wv = fm.fp4_unpack(wq).numpy().astype(np.float32)
    xv = fm.e4m3_to_f32(xq).numpy().astype(np.float32)
    d = _chunk_sums(wv, xv, 32)
    e = ws.view(torch.uint8).numpy().astype(np.int32)[None, :, :] + xs.view(torch.uint8).numpy().astype(np.int32)[:, None, :] - 254
    return _lanes(np.ldexp(d, e).astype(np.float32), lpr)


def silu_exact(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, np.float32)
    return (z * rt.sigmoid_exact(z)).astype(np.float32)


def bf_np(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def swiglu_routed(g: np.ndarray, u: np.ndarray, lim: float) -> np.ndarray:
    """bf16(silu(min(g, L)) * clamp(u, -L, L)) (check_ffn.py:220)."""
    lim = np.float32(lim)
    s = silu_exact(np.minimum(g, lim))
    return bf_np((s * np.clip(u, -lim, lim)).astype(np.float32))


def swiglu_shared(g: np.ndarray, u: np.ndarray, lim: float) -> np.ndarray:
    """bf16(silu(bf16(min(g, L))) * bf16(clamp(u, -L, L))) (check_ffn.py:227-230)."""
    lim = np.float32(lim)
    s = silu_exact(bf_np(np.minimum(g, lim)))
    return bf_np((s * bf_np(np.clip(u, -lim, lim))).astype(np.float32))
