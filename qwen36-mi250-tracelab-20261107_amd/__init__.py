"""MI355X-native (gfx950) routed-expert MoE block of the Qwen3.6-35B-A3B serving engine.

The package keeps the reference engine's Python call surfaces for this block and runs
everything through hand-written HIP kernels in libmoe_mi355x.so (C ABI in
include/moe_mi355x.h):

- ``experts.experts_forward`` / ``experts.register``: the Transformers experts
  implementation (engine/experts.py:93-108).
- ``block.moe(x, mlp, top_k)``: the whole block, router to combine
  (engine/fast/model.py:1139, engine/fast/prefill_kernels.py:676).
- ``ops``: the individual operations (route, sort, grouped GEMMs, combine).
- ``fp8``: per-row fp8-e4m3 expert weights; ``checkpoint``: their on-disk format (quantise a
  bf16 safetensors snapshot once, load the fp8 layers).
- ``graphs.MoeGraphs``: the block captured once per decode bucket and replayed.
"""

from . import _lib, block, checkpoint, experts, fp8, graphs, ops, synth  # noqa: F401
from ._lib import MoeLibraryError  # noqa: F401
from .block import moe, pack_router  # noqa: F401
from .experts import NAME, experts_forward, register  # noqa: F401

__all__ = ["MoeLibraryError", "NAME", "block", "checkpoint", "experts", "graphs", "experts_forward", "fp8", "moe", "ops",
           "pack_router", "register"]
