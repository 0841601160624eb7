"""Number formats of the decode MoE block, restated on the CPU.

TEST INFRASTRUCTURE ONLY. This module is part of the oracle: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it,
and only to check results against. The product path never calls it.

Formats:

- e4m3 (OCP "fn": no infinities, 0x7f / 0xff are NaN, max 448), round to
  nearest even after a clamp to +-448, as the reference's golden model
  quantizes (``test/kernels/deepseek_v41/check_ffn.py:104``).
- e2m1 (FP4): the value table of ``check_ffn.py:23-40``; a byte holds two
  values, the even K index in the low nibble (``check_ffn.py:108-115``).
- E8M0: the scale 2 ** (code - 127) (``check_ffn.py:113,120``).
- MXFP8, the "aiter" rule (``check_ffn.py:87-105``): per 32 values, the code is
  the biased exponent of the smallest power of two >= max(amax, 1e-10) / 448,
  clamped to [1, 254].
- Per-token-group FP8 with fp32 scales (the DeepSeek-V3 1 x 128 activation
  convention): scale = max(amax, 1e-10) / 448 in fp32, q = e4m3(x / scale).
- Weights: FP8 with one fp32 scale per 128 x 128 block (scale = amax / 448) and
  MXFP4 per the OCP Microscaling v1.0 spec (shared exponent
  floor(log2 amax) - 2, e2m1 round to nearest even, saturate at 6).

Parity pins (tests/test_oracle_formats.py): the e4m3 conversion against a
brute-force nearest-value search over all 256 codes and torch's
``float8_e4m3fn``; the FP4 table against torch's ``float4_e2m1fn_x2``; E8M0
against torch's ``float8_e8m0fnu``; the MX codes against the closed form
(smallest power of two that keeps |x| / 2**s <= 448) and idempotence.
"""

from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0
AMAX_FLOOR = 1e-10  # both activation rules floor the group amax at 1e-10
# e2m1 values by code (check_ffn.py:23-40)
FP4_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)  # fmt: skip


def bf(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 to bf16 (nearest even) and back (check_ffn.py:124-125)."""
    return x.to(torch.bfloat16).float()


# ---------------------------------------------------------------- e4m3
def e4m3_codes_from_f32(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> e4m3 codes (uint8): clamp to +-448, then round to nearest even."""
    q = x.float().clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(torch.uint8)


def e4m3_to_f32(codes: torch.Tensor) -> torch.Tensor:
    """e4m3 codes (uint8 or float8_e4m3fn) -> fp32."""
    if codes.dtype == torch.uint8:
        codes = codes.view(torch.float8_e4m3fn)
    return codes.float()


def e4m3_table() -> np.ndarray:
    """The 256 e4m3 values by code, decoded from the bit fields (NaN for 0x7f / 0xff)."""
    out = np.empty(256, np.float64)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m / 8.0 * 2.0**-6
        else:
            v = (1 + m / 8.0) * 2.0 ** (e - 7)
        out[c] = -v if s else v
    return out


# ---------------------------------------------------------------- e2m1 / E8M0
def fp4_unpack(packed: torch.Tensor) -> torch.Tensor:
    """[..., K / 2] packed e2m1 bytes -> [..., K] fp32 values (even K in the low nibble)."""
    lut = torch.tensor(FP4_VALUES, dtype=torch.float32)
    p = packed.view(torch.uint8).long()
    return torch.stack([lut[p & 15], lut[p >> 4]], -1).flatten(-2)


def e8m0_to_f32(codes: torch.Tensor) -> torch.Tensor:
    """E8M0 codes -> 2 ** (code - 127) as fp32."""
    return torch.exp2(codes.view(torch.uint8).float() - 127)


def deq_mxfp4(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[N, K / 2] e2m1 with [N, K / 32] E8M0 -> [N, K] fp32 (check_ffn.py:108-115)."""
    v = fp4_unpack(packed)
    return v * e8m0_to_f32(scales).repeat_interleave(32, -1)


def deq_fp8_b128(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """[N, K] e4m3 with [ceil(N / 128), ceil(K / 128)] fp32 scales -> [N, K] fp32.

    The 128 x 128 generalisation of the reference's 32 x 32 ``deq_fp8_block``
    (check_ffn.py:118-121): each weight times its block's scale, in fp32.
    """
    n, k = q.shape
    sf = s.float().repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)[:, :k]
    return e4m3_to_f32(q) * sf


def deq_fp8_mx32(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """[N, K] e4m3 with [N / 32, K / 32] E8M0 block scales -> [N, K] fp32: the reference's
    ``deq_fp8_block`` (check_ffn.py:118-121), each weight times 2 ** (code - 127) of its block."""
    n, k = q.shape
    sf = e8m0_to_f32(s).repeat_interleave(32, 0)[:n].repeat_interleave(32, 1)[:, :k]
    return e4m3_to_f32(q) * sf


# ---------------------------------------------------------------- activation rules
def code_ceil(v: torch.Tensor) -> torch.Tensor:
    """Biased exponent of the smallest power of two >= v (v > 0) (check_ffn.py:87-90)."""
    bits = v.float().contiguous().view(torch.int32)
    return ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0).int()


MX_RULES = ("aiter", "vllm")


def mxfp8_quant(x: torch.Tensor, rule: str = "aiter"):
    """Per-32 MXFP8 (check_ffn.py:93-105): -> (e4m3 codes, E8M0 codes).

    "aiter" (the routed experts' activations): the group amax is floored at 1e-10
    and multiplied by fp32(1 / 448), the code clamped to [1, 254]. "vllm" (the
    V4.1 shared expert's): the amax is floored at the smallest normal fp32 and
    divided by 448, the code clamped to [0, 254]. Either way the values are
    scaled by 2 ** (127 - code) (exact), clamped to +-448 and rounded to nearest
    even.
    """
    if rule not in MX_RULES:
        raise ValueError(rule)
    g = x.float().reshape(*x.shape[:-1], -1, 32)
    amax = g.abs().amax(-1, keepdim=True)
    if rule == "aiter":
        code = code_ceil(amax.clamp_min(AMAX_FLOOR) * torch.tensor(1.0 / FP8_MAX)).clamp(1, 254)
    else:
        code = code_ceil(amax.clamp_min(torch.finfo(torch.float32).tiny) / FP8_MAX).clamp(0, 254)
    inv = torch.exp2(127.0 - code.float())
    q = e4m3_codes_from_f32(g * inv)
    return q.reshape(x.shape), code.squeeze(-1).to(torch.uint8)


def mxfp8_dequant(q: torch.Tensor, code: torch.Tensor) -> torch.Tensor:
    g = e4m3_to_f32(q).reshape(*q.shape[:-1], -1, 32)
    return (g * torch.exp2(code.float() - 127.0)[..., None]).reshape(q.shape)


def mxfp8_qdq(x: torch.Tensor, rule: str = "aiter") -> torch.Tensor:
    return mxfp8_dequant(*mxfp8_quant(x, rule))


def group_fp8_quant(x: torch.Tensor, group: int = 128):
    """Per-token-group FP8, fp32 scales: -> (e4m3 codes [.., K], fp32 scales [.., K / group]).

    scale = max(amax, 1e-10) / 448 (fp32 division); q = e4m3(clamp(x / scale)).
    """
    g = x.float().reshape(*x.shape[:-1], -1, group)
    amax = g.abs().amax(-1, keepdim=True)
    s = amax.clamp_min(AMAX_FLOOR) / FP8_MAX
    q = e4m3_codes_from_f32(g / s)
    return q.reshape(x.shape), s.squeeze(-1)


def group_fp8_dequant(q: torch.Tensor, s: torch.Tensor, group: int = 128) -> torch.Tensor:
    g = e4m3_to_f32(q).reshape(*q.shape[:-1], -1, group)
    return (g * s[..., None]).reshape(q.shape)


def group_fp8_qdq(x: torch.Tensor, group: int = 128) -> torch.Tensor:
    return group_fp8_dequant(*group_fp8_quant(x, group), group)


# ---------------------------------------------------------------- weight quantizers
def quant_fp8_b128(w: torch.Tensor):
    """fp32 [N, K] -> (e4m3 codes [N, K], fp32 scales [ceil(N/128), ceil(K/128)]).

    DeepSeek-V3's block quantization: per 128 x 128 block, scale = amax / 448
    (1.0 for an all-zero block) and q = e4m3(w / scale).
    """
    n, k = w.shape
    nb, kb = -(-n // 128), -(-k // 128)
    pad = torch.zeros(nb * 128, kb * 128)
    pad[:n, :k] = w.float()
    blk = pad.reshape(nb, 128, kb, 128)
    amax = blk.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = e4m3_codes_from_f32(blk / s[:, None, :, None]).reshape(nb * 128, kb * 128)
    return q[:n, :k].contiguous(), s.contiguous()


def e2m1_round(v: torch.Tensor) -> torch.Tensor:
    """Round fp32 to the nearest e2m1 value (ties to the even code), saturating at +-6 -> codes.

    The e2m1 magnitudes are 0.5 apart on [0, 2] (codes 0 .. 4), 1 apart on [2, 4] (codes
    4 .. 6) and 2 apart on [4, 6] (codes 6, 7); a code's low bit is its mantissa bit, so
    "ties to even" is round-half-even of the code. Each branch's scaling (2a, a - 2,
    (a - 4) / 2) is exact in fp32 where it is taken, and torch.round rounds half to even.
    """
    a = v.abs().float()
    c = torch.where(
        a <= 2.0,
        torch.round(a * 2.0),
        torch.where(a <= 4.0, 4.0 + torch.round(a - 2.0), 6.0 + torch.round((a - 4.0) * 0.5)),
    )
    c = c.clamp(max=7.0).to(torch.uint8)
    sign = (v < 0) | ((v == 0) & torch.signbit(v))
    return c | (sign.to(torch.uint8) << 3)


def quant_mxfp4(w: torch.Tensor):
    """fp32 [N, K] -> (packed e2m1 [N, K / 2] uint8, E8M0 [N, K / 32] uint8), OCP MX v1.0.

    Per 32 values: shared exponent X = floor(log2(amax)) - 2 (emax of e2m1), the
    scale code X + 127 (clamped to [0, 254]; an all-zero block gets code 0), the
    values v / 2**X rounded to e2m1 with saturation at +-6.
    """
    n, k = w.shape
    g = w.float().reshape(n, k // 32, 32)
    amax = g.abs().amax(-1)
    _, ex = torch.frexp(amax)  # amax = m * 2**ex, m in [0.5, 1): floor(log2 amax) = ex - 1
    x = torch.where(amax > 0, ex - 1 - 2, torch.full_like(ex, -127))
    code = (x + 127).clamp(0, 254)
    scale = torch.exp2(code.float() - 127)
    c = e2m1_round(g / scale[..., None]).reshape(n, k)
    packed = c[:, 0::2] | (c[:, 1::2] << 4)
    return packed.contiguous(), code.to(torch.uint8).contiguous()
