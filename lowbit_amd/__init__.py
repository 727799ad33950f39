"""lowbit_amd: fused dequantize + GEMM for low-bit LLM weights on AMD MI355X (gfx950).

Drop-in for the reference package's public surface (src/lowbit/__init__.py:2-11):
the same names, packed layouts and call signatures, with the GEMMs running as
hand-written HIP kernels behind a C ABI (include/lowbit_hip.h). Additions:
`to_device` keeps packed weights resident in HBM between calls (host containers
passed to gemm_* are made resident on their first GEMM; `release` drops that copy),
and `quantize_int4_device` / `quantize_mxfp4_device` pack fp32 weights on the device
into the same bytes as the host packers.
"""
from .formats import (GROUP, MXBLOCK, Int4Weights, Int8Acts, MXFP4Weights, quantize_act_int8,
                      quantize_int4, quantize_mxfp4)
from .kernels import (Params, cpu_info, gemm_mxfp4, gemm_w4a8, gemm_w4a16, quantize_int4_device,
                      quantize_mxfp4_device, release, to_device)

__version__ = "0.1.0"
__all__ = [
    "GROUP", "MXBLOCK", "Int4Weights", "Int8Acts", "MXFP4Weights", "Params", "cpu_info",
    "gemm_mxfp4", "gemm_w4a8", "gemm_w4a16", "quantize_act_int8", "quantize_int4",
    "quantize_mxfp4", "quantize_int4_device", "quantize_mxfp4_device", "release", "to_device",
]
