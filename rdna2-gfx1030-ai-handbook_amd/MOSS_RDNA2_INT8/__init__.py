"""ComfyUI custom node: MI355X INT8 GEMM for MOSS with optional transpose-copy removal.

Same switches as the reference node (rdna2-ops/production/MOSS_RDNA2_INT8/
__init__.py:1-10, 22-60):
  MOSS_RDNA2_INT8_PATCH=1       install this library's INT8 -> INT32 GEMM as
                                Kitchen's _int8_matmul_accumulate;
  MOSS_RDNA2_INT8_LAYOUT=view   also replace Kitchen's eager int8_linear export
                                with the weight.T-view version (default);
  MOSS_RDNA2_INT8_LAYOUT=legacy keep Kitchen's original eager linear (rollback);
  MOSS_RDNA2_INT8_STATS=1       optional GEMM counters, no per-call logging.
No installed package or model file is edited. The GPU must be gfx950; a
missing HIP library or another architecture is an error, never a fallback.
The reference node's attention dispatch and measurement hooks are not part of
this package (they are not on the quantized-GEMM path).
"""

import logging
import os
from pathlib import Path
import sys

NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}


def _install():
    layout = os.environ.get("MOSS_RDNA2_INT8_LAYOUT", "view")
    if layout not in {"legacy", "view"}:
        raise ValueError("MOSS_RDNA2_INT8_LAYOUT must be 'legacy' or 'view'")
    import torch

    if torch.version.hip is None or not torch.cuda.is_available():
        raise RuntimeError("MOSS MI355X INT8 patch requires a ROCm GPU")
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if arch != "gfx950":
        raise RuntimeError("This INT8 patch targets MI355X (gfx950), not " + arch)

    import comfy_kitchen.backends.eager.quantization as ck_quant

    pkg_root = str(Path(__file__).resolve().parents[1])  # holds rdna2_ops
    if pkg_root not in sys.path:
        sys.path.insert(0, pkg_root)
    from rdna2_ops import _lib
    from rdna2_ops.int8_gemm import int8_matmul

    _lib.library()  # fail loudly when the gfx950 library is missing
    previous = ck_quant._int8_matmul_accumulate
    try:
        ck_quant._int8_matmul_accumulate = int8_matmul
        if layout == "view":
            from . import backend

            backend.install_backend(int8_matmul)
    except Exception:
        ck_quant._int8_matmul_accumulate = previous
        raise
    logging.getLogger("moss-mi355x").warning(
        "MOSS_RDNA2_INT8_PATCH active on %s: gfx950 int8 MFMA GEMM, layout=%s%s", arch, layout,
        " (FP32 input/output only, eager export, weight.T view)" if layout == "view" else " (original eager linear)")


if os.environ.get("MOSS_RDNA2_INT8_PATCH") == "1":
    _install()
