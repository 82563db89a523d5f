"""ctypes binding of ``librdna2_qgemm.so`` (the C ABI declared in include/qgemm.h).

Same loading convention as the reference's native library
(rdna2-ops/rdna2_ops/normalization.py:16-27): the path comes from the
``RDNA2_OPS_LIBRARY`` environment variable or ``lib/`` next to this file, and a
missing library is an error — there is no Python or CPU fallback anywhere on
the product path.
"""
from __future__ import annotations

import ctypes
import functools
import json
import os
from pathlib import Path

import torch

LIB_NAME = "librdna2_qgemm.so"
ARCH = "gfx950"

# dtype codes of include/qgemm.h (enum qg_dtype)
F32, F16, BF16, I32, I8, U8, E4M3, E5M2 = range(8)
DTYPE_CODE = {
    torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int32: I32,
    torch.int8: I8, torch.uint8: U8, torch.float8_e4m3fn: E4M3, torch.float8_e5m2: E5M2,
}

# enum qg_epilogue
EPI_ORDER_FUSED_FMA = 1
EPI_ORDER_EAGER = 2
EPI_GELU_TANH = 4
# enum qg_rounding
ROUND_HALF_EVEN = 0
ROUND_HALF_AWAY = 1
# enum qg_w4_flags
W4_SIGNED_NIBBLES = 1
W4_ORDER_HIGH = 2
W4_LAYOUT_KN = 4
W4_ZEROS_PACKED = 8
# enum qg_moe_epilogue, QG_MOE_TILE_ROWS
MOE_EPI_I32 = 0
MOE_EPI_SILU_MUL = 1
MOE_EPI_ROUTE = 2
MOE_TILE_ROWS = 192
MOE_COUNTS_PER_EXPERT = 259

_p, _i, _i64, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float

# name -> (restype, argtypes); every symbol include/qgemm.h declares
SIGNATURES = {
    "qg_error_string": (ctypes.c_char_p, [_i]),
    "qg_version": (ctypes.c_char_p, []),
    "qg_read_floor": (_i, [_p, _sz, _p, _p]),
    "qg_mfma_clock": (_i, [_i, _i, _p, _p]),
    "qg_int8_gemm_stages": (_i, [_p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _sz, _p]),
    "qg_quant_rows_i8": (_i, [_p, _i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i, _p]),
    "qg_int8_gemm_workspace_bytes": (_sz, [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64]),
    "qg_int8_gemm": (_i, [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i,
                          _p, _i, _i, _p, _sz, _p]),
    "qg_w8a8_linear_workspace_bytes": (_sz, [_p, _i64, _i64, _i64, _i64]),
    "qg_w8a8_linear": (_i, [_p, _i, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i, _p, _i, _i,
                            _i, _p, _sz, _p]),
    "qg_rot_quant_rows_i8": (_i, [_p, _i, _i64, _i64, _i64, _i, _p, _i64, _p, _i, _p]),
    "qg_w8a8_linear_ex": (_i, [_p, _i, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i, _i, _p, _i, _i64, _p,
                               _i64, _p, _i, _i, _i, _p, _sz, _p]),
    "qg_w8a8_linear_noalloc": (_i, [_p, _i, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i, _p, _i, _i,
                                    _i, _p]),
    "qg_w4_pack": (_i, [_p, _i, _i64, _i64, _i64, _i64, _i, _i, _i, _p, _p, _i, _p, _p, _p]),
    "qg_w4_unpack": (_i, [_p, _i64, _i64, _i, _i, _p, _i, _p, _p, _i, _p]),
    "qg_w4a16_gemm_workspace_bytes": (_sz, [_i64, _i64, _i64, _i, _i]),
    "qg_w4a16_gemm": (_i, [_p, _i, _i64, _i64, _i64, _p, _i64, _i, _i, _p, _i, _p, _p, _i, _p, _i,
                           _p, _sz, _p]),
    "qg_w4a8_gemm": (_i, [_p, _i64, _i64, _i64, _p, _i64, _i, _i, _p, _i, _p, _p, _i64, _p, _p, _i, _p, _i,
                          _p]),
    "qg_fp8_decode": (_i, [_p, _i, _i64, _i64, _i64, _i64, _p, _i, _p]),
    "qg_fp8w_gemm_workspace_bytes": (_sz, [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64]),
    "qg_fp8w_gemm": (_i, [_p, _i, _i64, _i64, _i64, _i64, _p, _i, _i64, _i64, _i64, _p, _p, _i, _p, _i,
                          _p, _sz, _p]),
    "qg_moe_sizes": (_i, [_i64, _i, _i, _i, _p, _p]),
    "qg_moe_dispatch": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p]),
    "qg_moe_dispatch_qx": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64,
                                _i64, _p, _i64, _p, _p]),
    "qg_moe_grouped_gemm": (_i, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _i, _p, _i64, _p, _p,
                                 _p, _p, _i, _p, _i64, _i64, _p]),
    "qg_moe_combine": (_i, [_p, _i64, _i, _i64, _p, _i64, _p]),
}


def library_path() -> Path:
    env = os.environ.get("RDNA2_OPS_LIBRARY")
    return Path(env) if env else Path(__file__).with_name("lib") / LIB_NAME


@functools.lru_cache(maxsize=1)
def library():
    path = library_path()
    if not path.is_file():
        raise RuntimeError(
            f"{path} is missing: build the gfx950 HIP library first "
            "(python -m rdna2_ops.build, or __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = library().qg_error_string(status).decode()
        if status == 1:  # hipErrorInvalidValue: rejected before any HIP call
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: HIP error {status} ({msg})")


@functools.lru_cache(maxsize=None)
def device_arch(index: int) -> str:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def require_gfx950(t: torch.Tensor) -> None:
    if t.device.type != "cuda" or not torch.version.hip:
        raise ValueError("Inputs must be on a ROCm HIP device")
    arch = device_arch(t.device.index if t.device.index is not None else torch.cuda.current_device())
    if arch != ARCH:
        raise ValueError(f"This kernel library targets {ARCH}, not {arch}")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes + 256, dtype=torch.uint8, device=device)


def ws_ptr(ws: torch.Tensor | None):
    if ws is None:
        return None, 0
    addr = ws.data_ptr()
    aligned = (addr + 255) // 256 * 256
    return ctypes.c_void_p(aligned), ws.numel() - (aligned - addr)


@functools.lru_cache(maxsize=1)
def kernel_resources() -> dict:
    path = library_path().with_name("kernel_resources.json")
    return json.loads(path.read_text()) if path.is_file() else {}


def kernel_metadata(variant: str, tile, symbol_hint: str) -> dict:
    """Metadata of the kernel that served a call: variant, tile and the
    compiler-reported register/LDS usage (parsed at build time)."""
    res = {}
    for name, info in kernel_resources().items():
        if symbol_hint in name:
            res = info
            break
    return {"variant": variant, "tile": list(tile) if tile is not None else None,
            "vgpr": res.get("VGPRs"), "agpr": res.get("AGPRs"), "sgpr": res.get("TotalSGPRs"),
            "lds_bytes": res.get("LDS Size [bytes/block]"), "scratch_bytes": res.get("ScratchSize [bytes/lane]"),
            "spills": (res.get("VGPRs Spill") or 0) + (res.get("SGPRs Spill") or 0) if res else None,
            # SGPR spills go to VGPR lanes (v_writelane), VGPR spills to scratch memory
            "vgpr_spills": res.get("VGPRs Spill"), "sgpr_spills": res.get("SGPRs Spill"),
            "occupancy_waves_per_simd": res.get("Occupancy [waves/SIMD]"), "symbol": symbol_hint}
