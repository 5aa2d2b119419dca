"""kea-kernels for AMD MI355X (gfx950): 1-bit and ternary weight x int8 activation GEMMs on CDNA4 int8 MFMA.

Drop-in for the reference package `kea_kernels` on its low-bit GEMM path: the same operator classes
(binary.layer.Int8MmaLayer, binary.layer_parts, binary.provider), export formats (formats), the package-level
load / transcribe / close (model) and the `python -m kea_kernels` command line, with the kernels in a prebuilt HIP
library (lib/libkea_hip.so, C ABI in include/kea_lowbit.h).

    import kea_kernels
    model = kea_kernels.load("kea-b-0.1")           # a downloaded model directory; mode = the model's default
    print(kea_kernels.transcribe(model, "clip.wav"))
    kea_kernels.close(model)
"""
__version__ = "0.1.0"
__all__ = ["Model", "Transcript", "load", "transcribe", "close", "decoder_graphs_mode", "__version__"]


def __getattr__(name):
    # the model API imports torch and numpy; the GEMM modules do not need it loaded
    if name in ("Model", "Transcript", "load", "transcribe", "close", "decoder_graphs_mode"):
        from kea_kernels import model
        return getattr(model, name)
    raise AttributeError(f"module 'kea_kernels' has no attribute {name!r}")
