"""pih_amd: MI355X (gfx950) Kernel Packs for PIH's linear-layer hot path.

The product is the pair of C-ABI Kernel Packs built under ``pih_amd/lib``
(``libpih_kernels_deepseek_v4_gfx950.so`` and
``libpih_kernels_amd_linear_gfx950.so``).  This package holds their ctypes
mirror (``abi``), device plumbing (``device``), Python callers of the pack
tables (``linear``) and the seeded input generator (``synth``).
"""
__all__ = ["abi", "device", "linear", "synth"]
