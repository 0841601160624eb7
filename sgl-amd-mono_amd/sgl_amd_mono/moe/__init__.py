"""The decode-step MoE block on gfx950: presets, the C-ABI binding, the host runner and the spec.

``runner.MoeRunner.moe`` runs one MoE block of one TP rank (the partial before
the all-reduce) in one persistent HIP launch of ``libmkmoe.so``.
"""

from .presets import PRESETS, WORKLOADS, MoePreset  # noqa: F401
