"""C ABI checks that need no GPU: the library loads, exports every function
include/qgemm.h declares with the argument count the ctypes binding uses, and
rejects invalid arguments with hipErrorInvalidValue before any HIP call
(the convention of rdna2-ops/rdna2_ops/csrc/group_norm_silu.hip:298-317)."""
import ctypes
import re
from pathlib import Path

import pytest

from rdna2_ops import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "qgemm.h"
INVALID = 1  # hipErrorInvalidValue


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(qg_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return decls


@pytest.fixture(scope="module")
def lib():
    return _lib.library()


def test_header_declares_bound_functions():
    decls = declared_functions()
    assert set(decls) == set(_lib.SIGNATURES), set(decls) ^ set(_lib.SIGNATURES)
    for name, nargs in decls.items():
        assert nargs == len(_lib.SIGNATURES[name][1]), name


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name
    assert lib.qg_version().decode().startswith("librdna2_qgemm gfx950")


def test_error_string(lib):
    assert lib.qg_error_string(0)
    assert lib.qg_error_string(INVALID)


def test_int8_gemm_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    base = dict(a=p, a_sm=64, a_sk=1, b=p, b_sk=1, b_sn=64, m=4, n=4, k=64, a_scale=p, b_scale=p,
                b_scale_numel=4, bias=None, bias_dtype=0, out=p, out_dtype=0, epilogue=0,
                workspace=None, workspace_bytes=0, stream=None)

    def call(**kw):
        args = dict(base, **kw)
        return lib.qg_int8_gemm(*args.values())

    assert call(m=-1) == INVALID
    assert call(k=131072) == INVALID                       # int8_gemm.py:142-143
    assert call(a_sm=-64) == INVALID                       # negative strides (:140-141)
    assert call(b_scale_numel=3) == INVALID                # wrong scale length (:168)
    assert call(out_dtype=_lib.I32) == INVALID             # dequant needs a float output
    assert call(a_scale=None, b_scale=None, out_dtype=_lib.F32) == INVALID  # int GEMM -> int32
    assert call(bias=p, bias_dtype=_lib.I8) == INVALID     # bias dtype (:173-175)
    assert call(epilogue=_lib.EPI_ORDER_EAGER | _lib.EPI_GELU_TANH) == INVALID
    assert call(epilogue=64) == INVALID
    assert call(a_sk=2) == INVALID                         # needs packing -> workspace missing
    assert call(m=0) == 0 and call(n=0, b_scale_numel=1) == 0  # empty output: nothing to launch


def test_quant_rows_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)
    assert lib.qg_quant_rows_i8(p, _lib.I8, 8, 1, 2, 8, p, 8, p, 0, None) == INVALID
    assert lib.qg_quant_rows_i8(p, _lib.F16, 8, 1, 2, 8, p, 8, p, 7, None) == INVALID
    assert lib.qg_quant_rows_i8(p, _lib.F16, 8, 1, 2, 8, p, 4, p, 0, None) == INVALID  # q_sm < k
    assert lib.qg_quant_rows_i8(p, _lib.F16, 8, 1, 0, 8, p, 8, p, 0, None) == 0


def test_w8a8_linear_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)
    args = [p, _lib.F16, 64, 4, 64, p, 64, 4, p, 4, None, 0, p, _lib.F16, 0, 0, None, 0, None]
    assert lib.qg_w8a8_linear(*args) == INVALID            # workspace missing
    bad = list(args)
    bad[1] = _lib.I8
    assert lib.qg_w8a8_linear(*bad) == INVALID
    assert lib.qg_w8a8_linear_workspace_bytes(p, 64, 4, 4, 64) >= 4 * 64 + 16


def test_read_floor_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)
    assert lib.qg_read_floor(p, 0, p, None) == 0                   # nothing to read
    assert lib.qg_read_floor(p, 24, p, None) == INVALID             # bytes % 16
    assert lib.qg_read_floor(ctypes.c_void_p(24), 32, p, None) == INVALID  # 16-byte aligned source
    assert lib.qg_read_floor(None, 32, p, None) == INVALID
    assert lib.qg_read_floor(p, 32, None, None) == INVALID


def test_mfma_clock_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)
    assert lib.qg_mfma_clock(3, 10, p, None) == INVALID            # mode
    assert lib.qg_mfma_clock(-1, 10, p, None) == INVALID
    assert lib.qg_mfma_clock(1, 0, p, None) == INVALID             # iterations
    assert lib.qg_mfma_clock(1, (1 << 22) + 1, p, None) == INVALID
    assert lib.qg_mfma_clock(1, 10, None, None) == INVALID         # output


def test_int8_gemm_stages_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(256)
    words = 256 * 8 * 272
    ok = [p, p, 4096, 3072, 3072, p, p, None, p, p, words, None]
    bad_k = list(ok)
    bad_k[4] = 3000                                                # k % 128
    assert lib.qg_int8_gemm_stages(*bad_k) == INVALID
    few = list(ok)
    few[10] = words - 1                                            # stamp buffer too small
    assert lib.qg_int8_gemm_stages(*few) == INVALID
    unaligned = list(ok)
    unaligned[0] = ctypes.c_void_p(264)                            # 16-byte aligned operands
    assert lib.qg_int8_gemm_stages(*unaligned) == INVALID
    for i in (0, 1, 5, 6, 8, 9):                                   # required pointers
        missing = list(ok)
        missing[i] = None
        assert lib.qg_int8_gemm_stages(*missing) == INVALID


def test_rot_quant_rows_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)

    def call(m=0, k=512, x_dtype=_lib.F32, x_sm=512, g=256, q_sm=512, rounding=0):
        return lib.qg_rot_quant_rows_i8(p, x_dtype, x_sm, m, k, g, p, q_sm, p, rounding, None)

    assert call() == 0                                     # valid, nothing to do for m = 0
    for g in (0, 1, 3, 96, 2048):                          # power of two in [2, 1024]
        assert call(g=g) == INVALID, g
    assert call(k=384) == INVALID                          # group must divide K (comfy_int8.py:113-116)
    assert call(k=32768, x_sm=32768, q_sm=32768) == INVALID  # K above QG_ROT_MAX_K
    assert call(x_dtype=_lib.I8) == INVALID
    assert call(x_sm=256) == INVALID
    assert call(q_sm=256) == INVALID
    assert call(rounding=5) == INVALID


def test_w8a8_linear_ex_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)

    def call(m=0, k=512, g=0, residual=None, residual_dtype=_lib.F32, residual_sm=64, rs=None, rs_numel=0,
             epilogue=0):
        return lib.qg_w8a8_linear_ex(p, _lib.F32, k, m, k, p, k, 64, p, 64, None, 0, g, residual, residual_dtype,
                                     residual_sm, rs, rs_numel, p, _lib.F32, 0, epilogue, None, 0, None)

    assert call() == 0
    assert call(g=256, residual=p, rs=p, rs_numel=64) == 0
    assert call(g=256, residual=p, rs=p, rs_numel=1) == 0
    assert call(g=384) == INVALID
    assert call(g=1024, k=1536) == INVALID                 # 1024 does not divide 1536
    assert call(residual=p, residual_dtype=_lib.I32) == INVALID
    assert call(residual=p, residual_sm=63) == INVALID      # row stride below N
    assert call(residual=p, rs=p, rs_numel=7) == INVALID    # residual_scale: 1 or N values
    assert call(residual=p, epilogue=_lib.EPI_ORDER_EAGER) == INVALID
    assert call(m=4) == INVALID                            # workspace missing


def test_w4a8_gemm_rejects_invalid_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    base = dict(a=p, a_sm=256, m=4, k=256, w=p, n=8, group=32, flags=_lib.W4_SIGNED_NIBBLES, scales=p,
                scales_dtype=_lib.F32, zeros=p, prepared=None, prepared_sn=0, a_scale=p, bias=None, bias_dtype=0,
                out=p, integer=0, stream=None)

    def call(**kw):
        return lib.qg_w4a8_gemm(*dict(base, **kw).values())

    assert call(group=48) == INVALID                       # group size 32 / 64 / 128
    assert call(k=96, a_sm=96, group=64) == INVALID        # k % group
    assert call(k=1118496, a_sm=1118496) == INVALID        # k * 128 * 15 >= 2^31 (int4_weight_gemm_v07.py:493)
    assert call(a_sm=264) == INVALID                       # rows on 16-byte boundaries
    assert call(a=ctypes.c_void_p(24)) == INVALID          # 16-byte aligned base
    assert call(a_scale=None) == INVALID                   # float output needs the row scale
    assert call(scales_dtype=_lib.F16) == INVALID
    assert call(flags=64) == INVALID
    assert call(integer=2) == INVALID
    assert call(prepared=p, prepared_sn=100) == INVALID    # prepared rows on 16-byte boundaries
    assert call(m=0) == 0                                  # empty output: nothing to launch


def test_fp8w_gemm_packs_rows_past_32bit_offsets(lib):
    """Rows whose byte offsets do not fit the kernels' 32-bit offsets are packed
    into workspace, never read in place (the offset would wrap to another row);
    without that workspace the call is refused before any HIP call."""
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    m, n, k = 4, 300, 128
    need_ok = lib.qg_fp8w_gemm_workspace_bytes(p, k, 1, p, k, 1, m, n, k)
    assert need_ok == 0                                    # canonical rows: read in place
    w_sn = 1 << 23                                         # (n - 1) * w_sn + k > 2^31
    need = lib.qg_fp8w_gemm_workspace_bytes(p, k, 1, p, w_sn, 1, m, n, k)
    assert need >= n * k                                   # W packed
    a_sm = 1 << 22                                         # m = 300: 2 * ((m - 1) * a_sm + k) > 2^31
    need_a = lib.qg_fp8w_gemm_workspace_bytes(p, a_sm, 1, p, k, 1, 300, n, k)
    assert need_a >= 2 * 300 * k                           # A packed
    base = [p, _lib.BF16, k, 1, m, k, p, _lib.E4M3, w_sn, 1, n, None, None, 0, p, _lib.BF16, None, 0, None]
    assert lib.qg_fp8w_gemm(*base) == INVALID              # packing needs workspace



def test_w4a16_workspace_sizes(lib):
    """qg_w4a16_gemm_workspace_bytes: the dequantised weight (2 * n * k bytes)
    for prefill grids (more than 64 rows, K a multiple of 64) with at least the
    group's number of tiles of 256 x 192 (192 at group 128, 64 at group 64, any
    at group 32); nothing for decode shapes and smaller grids, whose kernels
    read the packed words directly."""
    zp = _lib.W4_ZEROS_PACKED
    assert lib.qg_w4a16_gemm_workspace_bytes(2048, 14336, 4096, 128, zp) == 2 * 14336 * 4096
    assert lib.qg_w4a16_gemm_workspace_bytes(2048, 14336, 4096, 64, 0) == 2 * 14336 * 4096
    for m in (1, 2, 16, 64):
        assert lib.qg_w4a16_gemm_workspace_bytes(m, 14336, 4096, 128, zp) == 0
    assert lib.qg_w4a16_gemm_workspace_bytes(2048, 192, 4096, 128, zp) == 0   # 8 tiles: fused tiled kernel
    assert lib.qg_w4a16_gemm_workspace_bytes(2048, 14336, 4064, 32, zp) == 0  # K not a multiple of 64
    assert lib.qg_w4a16_gemm_workspace_bytes(130, 200, 512, 32, 0) == 2 * 200 * 512     # group 32: any grid
    assert lib.qg_w4a16_gemm_workspace_bytes(130, 200, 512, 64, 0) == 0                 # 2 tiles < 64
    assert lib.qg_w4a16_gemm_workspace_bytes(1024, 4096, 512, 64, 0) == 2 * 4096 * 512  # 88 tiles >= 64
    assert lib.qg_w4a16_gemm_workspace_bytes(1024, 4096, 512, 128, zp) == 0             # 88 tiles < 192
    assert lib.qg_w4a16_gemm_workspace_bytes(64, 200, 512, 32, 0) == 0                  # decode rows


def test_moe_dispatch_qx_rejects_invalid_arguments(lib):
    """The fused routing + x quantization takes bf16 rows of at most 2048
    values, a multiple of 8, 16-byte aligned x and 8-byte aligned xq rows;
    anything else is refused before any HIP call (the caller then runs the
    dispatch and the quantizer separately)."""
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    rows, tiles = ctypes.c_int64(), ctypes.c_int64()
    assert lib.qg_moe_sizes(16, 8, 2, 64, ctypes.byref(rows), ctypes.byref(tiles)) == 0
    base = dict(logits=p, l_sm=8, tokens=16, e=8, top_k=2, pad=64, experts=p, weights=p, counts=p, row_token=p,
                row_weight=p, row_slot=p, rows_max=rows.value, tiles=p, tiles_max=tiles.value, x=p, x_sm=256,
                hidden=256, xq=p, xq_sm=256, xs=p, stream=None)

    def call(**kw):
        args = dict(base, **kw)
        return lib.qg_moe_dispatch_qx(*args.values())

    assert call(hidden=2056, x_sm=2056, xq_sm=2056) == INVALID  # wider than one wave's row
    assert call(hidden=252, x_sm=252, xq_sm=252) == INVALID     # not a multiple of 8
    assert call(x_sm=255) == INVALID                            # x_sm < hidden
    assert call(x_sm=260) == INVALID                            # rows not 16-byte aligned
    assert call(x=ctypes.c_void_p(4104)) == INVALID             # x not 16-byte aligned
    assert call(xq=ctypes.c_void_p(4100)) == INVALID            # xq not 8-byte aligned
    assert call(xs=None) == INVALID
    assert call(rows_max=0) == INVALID                          # the dispatch's own checks come first


def test_moe_grouped_gemm_rejects_plans_beyond_its_item_table(lib):
    """The grouped GEMM keeps each workgroup's share of the work items
    (tiles x 256-column tiles) in LDS: at most 131072 items per launch; one
    more is refused before any HIP call; no tiles at all launch nothing."""
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first

    def call(tiles_max, n, **kw):
        args = dict(a=p, a_sm=256, a_rows=64, row_token=None, rows_max=64, k=256, w=p, w_sn=256,
                    w_estride=256 * n, n=n, n_experts=1, tiles=p, tiles_max=tiles_max, a_scale=p, b_scale=p,
                    row_weight=None, row_slot=None, epilogue=_lib.MOE_EPI_SILU_MUL, out=p, out_sm=n // 2,
                    out_rows=64, stream=None)
        args.update(kw)
        return lib.qg_moe_grouped_gemm(*args.values())

    assert call(131073, 256) == INVALID         # one column tile: 131073 items
    assert call(65537, 512) == INVALID          # two column tiles: 131074 items
    assert call(43691, 768) == INVALID          # three: 131073 items
    assert call(0, 256) == 0                    # no tiles: nothing to launch
