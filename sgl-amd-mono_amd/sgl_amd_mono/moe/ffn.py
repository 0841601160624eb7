"""DeepSeek-V4.1's FFN on one GPU: the FFN seam, then the MoE block on its normed rows.

Mirrors the reference's FFN entry point for this path:
- ``FfnWeights`` holds ``FFNWeights``' fields (``sgl_amd_mono/deepseek_v41/gfx950/runner.py:
  130-168``): the seam's ``hc_ffn_fn``, ``hc_ffn_scale``, ``hc_ffn_base`` and ``ffn_norm``, and
  the MoE's ``gate_w``, ``bias``, ``w13``/``w13_s``, ``w2``/``w2_s`` (MXFP4 in SGLang's loaded
  gfx950 layout) and ``sgu``/``sgu_s``, ``sw2``/``sw2_s`` (FP8 with E8M0 32 x 32 scales), all read
  in place. ``check`` is ``FFNWeights.check``'s.
- ``FfnRunner.ffn`` takes ``DSV41MonoRunner.ffn``'s arguments and returns its outputs
  (``runner.py:436-510``): ``(out, res_out, post_out, comb_out, pre_out)``, with the same row
  checks and optional caller-provided outputs. ``part`` is the attention output after the TP
  all-reduce, and ``out`` this rank's MoE partial before the FFN's all-reduce: both reduces
  need peers.

The reference runs this as one launch (``gfx950/layer.py:498-598``). Here it is the seam's
launches (``include/mkmoe_seam.h``) and the MoE's persistent launch (``include/mkmoe.h``) on
the current stream, in the reference's order: the residual update and the RMSNorm that makes
the MoE's input first, the MoE on it, and the seam's gate last (the reference runs its gate
inside the MoE stage, ``layer.py:579-586``). No host synchronisation; outputs and workspaces
are allocated on a row count's first call, never inside a graph capture.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .presets import PRESETS, MoePreset
from .runner import MoeRunner, MoeWeights, no_capture
from .seam import HC, HIDDEN, NORM_EPS, SeamRunner, SeamWeights

V41_PRESET = "v41_tp4"


@dataclass
class FfnWeights:
    """One layer's FFN tensors on this rank (``FFNWeights``' names)."""

    hc_ffn_fn: torch.Tensor
    hc_ffn_scale: torch.Tensor
    hc_ffn_base: torch.Tensor
    ffn_norm: torch.Tensor
    gate_w: torch.Tensor
    bias: torch.Tensor
    w13: torch.Tensor
    w13_s: torch.Tensor
    w2: torch.Tensor
    w2_s: torch.Tensor
    sgu: torch.Tensor
    sgu_s: torch.Tensor
    sw2: torch.Tensor
    sw2_s: torch.Tensor

    def seam(self) -> SeamWeights:
        return SeamWeights(self.hc_ffn_fn, self.hc_ffn_scale, self.hc_ffn_base, self.ffn_norm)

    def moe(self) -> MoeWeights:
        return MoeWeights(
            gate_w=self.gate_w, bias=self.bias, w13=self.w13, w13_s=self.w13_s, w2=self.w2, w2_s=self.w2_s,
            sgu=self.sgu, sgu_s=self.sgu_s, sw2=self.sw2, sw2_s=self.sw2_s,
        )  # fmt: skip

    def check(self, preset: MoePreset, device=None) -> None:
        """Raise (a ``RuntimeError`` naming the tensor) unless every tensor has the preset's
        shape and dtype and is contiguous on one GPU."""
        if preset.hidden != HIDDEN:
            raise RuntimeError(f"FFN: the seam is built for hidden {HIDDEN}, the MoE preset has {preset.hidden}")
        self.seam().check(device)
        self.moe().check(preset, device)


class FfnRunner:
    """The V4.1 FFN (seam + MoE block) of one preset on one GPU.

    ``moe_options`` go to the MoE runner as they are (``deadline_s``, ``mfma_rows``,
    ``mxfp4_scaled_rows``, ``mxfp4_scaled_down_rows``, ``max_rows``)."""

    def __init__(self, preset: MoePreset | str = V41_PRESET, device=None, norm_eps: float = NORM_EPS, **moe_options):
        self.preset = PRESETS[preset] if isinstance(preset, str) else preset
        if self.preset.hidden != HIDDEN:
            raise RuntimeError(f"FFN: the seam is built for hidden {HIDDEN}, {self.preset.name} has {self.preset.hidden}")
        self.moe_runner = MoeRunner(self.preset, device, **moe_options)
        self.device = self.moe_runner.device
        self.seam_runner = SeamRunner(self.device, norm_eps=norm_eps)
        self._normed: dict[int, torch.Tensor] = {}

    def supports(self, rows: int) -> bool:
        return 1 <= rows <= self.moe_runner.max_rows and self.seam_runner.supports(rows)

    def _outs(self, m: int, residual: torch.Tensor) -> tuple:
        no_capture("the FFN's outputs")
        f32 = torch.float32
        return (
            torch.empty(m, HIDDEN, dtype=torch.bfloat16, device=self.device),
            torch.empty_like(residual),
            torch.empty(m, HC, 1, dtype=f32, device=self.device),
            torch.empty(m, HC, HC, dtype=f32, device=self.device),
            torch.empty(m, HC, dtype=f32, device=self.device),
        )

    def normed(self, m: int) -> torch.Tensor:
        """The MoE's input rows of an ``m``-row call (the seam's RMSNorm output): one buffer per
        row count, which the last call's rows stay in."""
        t = self._normed.get(m)
        if t is None:
            no_capture("the FFN's normed rows")
            t = self._normed[m] = torch.empty(m, HIDDEN, dtype=torch.bfloat16, device=self.device)
        return t

    def ffn(
        self,
        w: FfnWeights,
        part: torch.Tensor,  # [M, H] bf16: the attention output, all-reduced
        residual: torch.Tensor,  # [M, 4, H] bf16, after the attention seam
        post_mix: torch.Tensor,  # [M, 4, 1] f32, the attention seam's
        res_mix: torch.Tensor,  # [M, 4, 4] f32
        pre_mix: torch.Tensor,  # [M, 4] f32
        outs: tuple | None = None,
        topk_ids: torch.Tensor | None = None,
        topk_w: torch.Tensor | None = None,
    ) -> tuple:
        """-> (out [M, H] bf16: the MoE partial, res_out [M, 4, H], post_out [M, 4, 1],
        comb_out [M, 4, 4], pre_out [M, 4]). ``topk_ids`` / ``topk_w`` (optional, [M, topk]
        int32 / fp32) receive the routing."""
        m = part.shape[0]
        if not self.supports(m):
            raise RuntimeError(f"DSv4.1 FFN: {m} rows, want 1 .. {self.moe_runner.max_rows}")
        if outs is None:
            outs = self._outs(m, residual)
        out, res_out, post_out, comb_out, pre_out = outs
        normed = self.normed(m)
        self.seam_runner.ffn_seam(
            w.seam(), part, residual, post_mix, res_mix, pre_mix, outs=(normed, res_out, post_out, comb_out, pre_out),
            gate_later=True,
        )  # fmt: skip
        try:
            self.moe_runner.moe(w.moe(), normed, out=out, topk_ids=topk_ids, topk_w=topk_w)
        except BaseException:
            self.seam_runner.cancel_gate()
            raise
        self.seam_runner.gate()
        return outs
