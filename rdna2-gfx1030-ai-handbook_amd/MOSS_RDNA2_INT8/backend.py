"""The node's eager INT8 linear backend: the rdna2_ops.comfy_int8 module
(the reference keeps the same code twice, production/MOSS_RDNA2_INT8/backend.py
= rdna2_ops/comfy_int8.py; here the node re-exports the one implementation)."""
from pathlib import Path
import sys

_root = str(Path(__file__).resolve().parents[1])
if _root not in sys.path:
    sys.path.insert(0, _root)

from rdna2_ops.comfy_int8 import (  # noqa: E402,F401
    disable_backend, get_stats, install_backend, int8_linear, kitchen_int8_without_transpose_copy,
    reset_stats)
