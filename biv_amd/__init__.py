"""biv_amd: the MI355X (gfx950) backend for biv's qwen35moe MoE FFN block.

- `biv_amd.hip`   host side over the C ABI of include/biv_hip.h (HipEngine, HipMoe)
- `biv_amd.synth` synthetic layers and inputs in ggml block formats
- `biv_amd.build` builds libbiv_hip.so in-tree with hipcc
"""
from . import synth  # noqa: F401

__all__ = ["synth", "hip", "build"]
