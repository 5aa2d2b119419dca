"""kea-kernels for AMD MI355X (gfx950): 1-bit and ternary weight x int8 activation GEMMs on CDNA4 int8 MFMA.

Drop-in for the reference package `kea_kernels` on its low-bit GEMM path: the same operator classes
(binary.layer.Int8MmaLayer, binary.layer_parts, binary.provider), export formats (formats) and entry points, with the
kernels in a prebuilt HIP library (lib/libkea_hip.so, C ABI in include/kea_lowbit.h).
"""
__version__ = "0.1.0"
