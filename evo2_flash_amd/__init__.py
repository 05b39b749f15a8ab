"""evo2_flash_amd: the StripedHyena2 (Evo 2) Hyena mixer hot path on AMD MI355X.

Hand-written HIP kernels for gfx950 behind a C ABI (include/evo2_hyena.h),
with host wrappers that keep evo2_flash's operator surface: the same tensor
layouts, paged-state slot tables and fp8 checkpoint format.
"""

__version__ = "0.1.0"
