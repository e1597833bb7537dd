"""mamba_metal_amd: the Mamba selective-scan inference path on AMD MI355X (gfx950).

Drop-in for createcentury/mamba-metal's public API (mamba_metal/__init__.py:3-20)
on PyTorch-ROCm tensors: the scan, the causal conv1d and the decode state updates
run as hand-written HIP kernels in libmamba_mi355x.so (C ABI in
include/mamba_mi355x.h); projections use torch GEMMs.  There is no CPU fallback.
"""

from mamba_metal_amd._loader import load_kernel
from mamba_metal_amd.generate import (GraphDecoder, GraphPrefill, generate, generate_fast,
                                      generate_fast_ids)
from mamba_metal_amd.load_hf import load_mamba_hf
from mamba_metal_amd.mamba_block import MambaBlock
from mamba_metal_amd.mamba_model import MambaConfig, MambaModel, MambaResidualBlock, init_weights_
from mamba_metal_amd.selective_scan import selective_scan

__all__ = [
    "MambaBlock",
    "MambaConfig",
    "MambaModel",
    "MambaResidualBlock",
    "generate",
    "generate_fast",
    "load_kernel",
    "load_mamba_hf",
    "selective_scan",
    # extensions beyond the reference's API
    "GraphDecoder",
    "GraphPrefill",
    "generate_fast_ids",
    "init_weights_",
]
