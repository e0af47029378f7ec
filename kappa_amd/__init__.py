"""MI355X (gfx950) Qwen3 MoE feed-forward block.

The product is libkmoe.so (HIP kernels behind the C ABI in include/kmoe.h);
``kappa_amd.qwen3`` mirrors the reference's Python interface on top of it.
"""

__version__ = "0.1.0"
