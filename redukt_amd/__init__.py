"""redukt_amd — MI355X (gfx950) backbone backend for the redukt neural compressor.

The product is the shared library ``libredukt_gpu.so`` built from ``csrc/``: redukt's
plugin C ABI (include/redukt_backend.h) over hand-written HIP kernels.  This package
holds the host-side mirror of redukt's plugin loader and backend (``ffi``), the .rbin
weight format (``rbin``) and the seeded synthetic workloads (``synth``).
"""
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PACKAGE_DIR, "libredukt_gpu.so")

__all__ = ["PACKAGE_DIR", "LIB_PATH"]
