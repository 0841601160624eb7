"""MI355X (gfx950) monokernel plugin for SGLang: the decode-step MoE block.

The package keeps the reference's plugin surface for this path
(``sgl_amd_mono/__init__.py:16-34``, ``pyproject.toml:16-17`` of the
reference): SGLang loads it as a general plugin through the
``sglang.srt.plugins`` entry point, whose ``register_specs`` registers each
spec under the monokernel backend ``amd``. The spec module imports only when a
server runs this backend.

Where SGLang's monokernel interface (``sglang.srt.monokernels.spec``) is not
installed, ``register_specs`` registers with ``sgl_amd_mono.monospec``, a
local registry with the same names, so that the spec and its tests run on
their own.
"""

__version__ = "0.1.0"

# The --monokernel-backend name this package registers
BACKEND = "amd"
# Each spec by the model's HF architecture
SPECS = {
    "DeepseekV3ForCausalLM": "sgl_amd_mono.moe.spec:SPEC",
    # the reference's own model: its FFN (the seam and the MoE block) at TP 4
    "DeepseekV4ForCausalLM": "sgl_amd_mono.moe.spec_v41:SPEC",
}


def registry():
    """SGLang's monokernel spec module, or the local one when SGLang is absent."""
    try:
        from sglang.srt.monokernels import spec as reg  # type: ignore[import-not-found]
    except ImportError:
        from . import monospec as reg
    return reg


def register_specs() -> None:
    """The plugin entry point, which SGLang runs in every process."""
    reg = registry()
    for architecture, path in SPECS.items():
        reg.register(backend=BACKEND, architecture=architecture, path=path)
