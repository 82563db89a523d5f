"""MI355X (gfx950) quantized-weight GEMM operators with the rdna2_ops API.

Drop-in for the GEMM entry points of the reference package ``rdna2_ops``
(rdna2-ops/rdna2_ops/__init__.py): the module paths ``rdna2_ops.int8_gemm``,
``rdna2_ops.int4_weight_gemm_v07``, ``rdna2_ops.fp8_weight_gemm_v06`` and
``rdna2_ops.comfy_int8`` keep their signatures; the kernels behind them are
hand-written gfx950 HIP in ``lib/librdna2_qgemm.so`` (C ABI: include/qgemm.h).
"""
__version__ = "0.7.0+mi355x"

__all__ = ["int8_gemm", "quantize", "int4_weight_gemm_v07", "fp8_weight_gemm_v06", "comfy_int8"]
