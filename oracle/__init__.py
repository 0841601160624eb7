"""CPU oracle of the decode MoE block (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only to check results against. The product path
(``sgl-amd-mono_amd/``) never imports it and fails loudly when its HIP
library is missing.

- ``formats``: e4m3, e2m1, E8M0, MXFP8 / per-token-group FP8 activation rules,
  FP8 128 x 128 and MXFP4 weight quantizers.
- ``routing``: fixed-order router logits, exact fp64 sigmoid, grouped top-k,
  fixed-order RMSNorm (the kernel's arithmetic, step for step).
- ``moe``: the golden MoE partial of ``test/kernels/deepseek_v41/check_ffn.py:209-232``,
  generalised over the weight formats.
- ``gen``: seeded CPU inputs and per-expert weights.

Parity status: every function is pinned by the tests named in its module
docstring; none is "parity unpinned" except where a module says so.
"""
