"""MI355X-native (gfx950) MoE expert path for GLM-5.3-style layers.

Host code mirrors the reference package ``exlr8``'s MoE-block operators (router, trellis
expert linear/MLP, joined-MXFP4 experts, combine) on PyTorch-ROCm tensors; all compute runs
in the hand-written HIP kernels of ``libmoe_mi355x.so`` through a thin C ABI
(``include/moe_mi355x.h``).  There is no CPU fallback: a missing library raises.
"""
from ._lib import LibraryMissing, lib, check  # noqa: F401

__version__ = "0.1.0"
