"""MI355X (gfx950) int4/int8 quantized matrix-product path.

Drop-in for the quantized matmul hot path of the Gemma-4-12B Vulkan engine
(monstercameron/Gemma4-12B-SnapdragonX2Elite): decode GEMV with fp16 or
e4m3 block scales, W4A16 / W8A8 / W4A8 prefill GEMMs, the int8 activation
quantizer, the GPU quantizer and repacks, and hipGraph record/replay.

``ops`` is the functional API (torch tensors), ``vk_engine`` mirrors the
reference engine's host helpers (``quant``, ``i4``, ``Buf``, ``gemv_ds``,
``gemv``, ``gemm_ds``, ``gmm``) and ``_lib`` is the ctypes binding of
``libq4mi.so``, which must be built (``build.py``); nothing falls back to
the CPU.
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "vk_engine", "build"]


def __getattr__(name):
    # torch is imported lazily so that the ABI can be inspected without it
    if name in ("ops", "vk_engine", "build"):
        import importlib

        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
