"""arf_amd -- MI355X (gfx950) GGUF quantized matmul for Arf's decode/prefill/MoE path.

The compute lives in libarfq.so (HIP kernels behind the C ABI in include/arfq.h);
this package is its Python host side (arf_amd.arfq) plus the build script
(arf_amd.build) and seeded synthetic inputs (arf_amd.synth).
"""
from .arfq import (BLOCK, ArfqError, Context, DeviceArray, DType, Gguf, GgufTensor, QType, Weight,
                   add_matmul, add_matmul_m, exported_symbols, load_library)

__all__ = ["BLOCK", "ArfqError", "Context", "DeviceArray", "DType", "Gguf", "GgufTensor", "QType",
           "Weight", "add_matmul", "add_matmul_m", "exported_symbols", "load_library"]
