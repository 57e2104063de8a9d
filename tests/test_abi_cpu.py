"""The C-ABI library without a GPU: it loads, exports every symbol the header
declares, and validates geometry on the host before any HIP call.

No kernel is launched here; every call below fails validation (or only sizes
the workspace) before the library touches the device.
"""

import ctypes
import re
from pathlib import Path

import pytest

from oops_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "oops_amd.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(oops_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.oops_abi_version() == _lib.ABI_VERSION


def test_header_constants_match_python():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define\s+(OOPS_\w+)\s+(\d+)", text))
    assert int(consts["OOPS_F32"]) == _lib.F32
    assert int(consts["OOPS_BF16"]) == _lib.BF16
    assert int(consts["OOPS_F16"]) == _lib.F16
    assert int(consts["OOPS_BIAS_NONE"]) == _lib.BIAS_NONE
    assert int(consts["OOPS_BIAS_FULL"]) == _lib.BIAS_FULL
    assert int(consts["OOPS_BIAS_SHARED"]) == _lib.BIAS_SHARED
    assert int(re.search(r"OOPS_TABLE_WIDTH\s*=\s*(\d+)", text).group(1)) == _lib.TABLE_WIDTH
    # table column order: the enum lists the columns in _lib's order
    enum = re.search(r"enum oops_table_column\s*\{(.*?)\}", text, re.S).group(1)
    names = re.findall(r"OOPS_T_(\w+)", re.sub(r"/\*.*?\*/", "", enum, flags=re.S))
    assert names.index("BIAS_MODE") == _lib.T_BIAS_MODE
    assert names.index("L_OFF") == _lib.T_L_OFF
    assert names.index("DB_OFF") == _lib.T_DB_OFF


def _geometry(table, *, heads=4, head_size=32, dtype=_lib.BF16, has_bias=True):
    arr = (ctypes.c_int64 * len(table))(*table)
    geo = _lib.Geometry()
    geo.dtype = dtype
    geo.bias_dtype = dtype
    geo.num_heads = heads
    geo.head_size = head_size
    geo.num_samples = len(table) // _lib.TABLE_WIDTH
    geo.has_bias = int(has_bias)
    geo.has_mask = 0
    geo.vec_ok = 1
    geo.scale = head_size**-0.5
    geo.table_host = ctypes.addressof(arr)
    geo.table_device = 0x1000  # never dereferenced on the host
    return geo, arr


def c3_table(n=768, h=4, c=32):
    """Ending-node row of BASELINE config 3: q[g, i, h, d] at i*(n*h*c) + g*(h*c) + h*c + d."""

    from oops_amd.attention import _core

    qs = (0, h * c, c, n * h * c)
    return _core.table_row(
        groups=n, len_q=n, len_k=n, q=qs, k=qs, v=qs, bias=(0, 0, n * n, n), dbias=(0, 0, n * n, n),
        bias_mode=_lib.BIAS_SHARED, lse_off=0,
    )  # fmt: skip


def test_workspace_sizing(lib):
    geo, keep = _geometry(c3_table())
    ws = lib.oops_attn_backward_workspace_bytes(ctypes.byref(geo))
    # delta: one float per (group, head, query); then partial dBias slabs of H*N*N floats
    delta = 768 * 4 * 768 * 4
    slab = 4 * 768 * 768 * 4  # float32 partial dBias per part
    frag = 4 * 768 * 768 * 2  # fragment-major bias copy (bf16)
    parts, rest = divmod(ws - delta - frag, slab)
    assert rest == 0 and 2 <= parts <= 64, (ws, parts, rest)


def test_forward_workspace_sizing(lib):
    """A row-shared 16-bit bias gets a fragment-major copy: H x ceil(Lq/32)32 x ceil(Lk/32)32 elements."""

    geo, keep = _geometry(c3_table())
    ws = lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo))
    assert ws == 4 * 768 * 768 * 2
    # the backward holds the same copy after delta and the partial slabs
    bwd = lib.oops_attn_backward_workspace_bytes(ctypes.byref(geo))
    assert (bwd - 768 * 4 * 768 * 4 - ws) % (4 * 768 * 768 * 4) == 0
    # no copy for float32, without a bias, or on the generic kernels
    for field, value in (("dtype", _lib.F32), ("has_bias", 0), ("force_generic", 1)):
        geo2, keep2 = _geometry(c3_table())
        setattr(geo2, field, value)
        if field == "dtype":
            geo2.bias_dtype = _lib.F32
        assert lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo2)) == 0, field
    # a forward call without it is refused before anything is enqueued
    assert lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None, 0, None) == 3
    assert "workspace" in lib.oops_last_error().decode()


@pytest.mark.parametrize(
    "field,value,message",
    [
        ("num_heads", 0, "num_heads"),
        ("head_size", 0, "head_size"),
        ("head_size", 257, "head_size"),
        ("dtype", 7, "dtype"),
        ("num_samples", 0, "num_samples"),
    ],
)
def test_geometry_validation(lib, field, value, message):
    geo, keep = _geometry(c3_table())
    setattr(geo, field, value)
    rc = lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None, 0, None)
    assert rc == 1
    assert message in lib.oops_last_error().decode()
    assert lib.oops_attn_backward_workspace_bytes(ctypes.byref(geo)) == 0


def test_table_validation(lib):
    from oops_amd.attention import _core

    row = c3_table()
    bad = list(row)
    bad[_lib.T_LEN_K] = 0
    geo, keep = _geometry(bad)
    assert lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None, 0, None) == 1
    assert "empty axis" in lib.oops_last_error().decode()
    bad = list(row)
    bad[_lib.T_B_SG] = 5  # a shared bias with a group stride
    geo, keep = _geometry(bad)
    assert lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None, 0, None) == 1
    assert "group stride 0" in lib.oops_last_error().decode()
    geo, keep = _geometry(row)
    geo.table_host = None
    assert lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None, 0, None) == 1
    assert lib.oops_attn_forward(None, 1, 1, 1, None, 1, 1, None, 1, None, 0, None) == 1
    assert "NULL" in lib.oops_last_error().decode()
    del _core


def test_pointer_and_workspace_validation(lib):
    geo, keep = _geometry(c3_table())
    # NULL operands
    assert lib.oops_attn_forward(ctypes.byref(geo), None, 1, 1, None, 1, 1, None, 1, None, 0, None) == 1
    # has_bias without a bias pointer
    assert lib.oops_attn_forward(ctypes.byref(geo), 1, 1, 1, None, None, 1, None, 1, None, 0, None) == 1
    assert "bias" in lib.oops_last_error().decode()
    # too small a workspace
    rc = lib.oops_attn_backward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, 1, 1, 1, 1, 1, 256, 16, None)
    assert rc == 3
    assert "workspace" in lib.oops_last_error().decode()
    # misaligned workspace
    need = lib.oops_attn_backward_workspace_bytes(ctypes.byref(geo))
    rc = lib.oops_attn_backward(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, 1, 1, 1, 1, 1, 8, need, None)
    assert rc == 3 and "aligned" in lib.oops_last_error().decode()


def test_row_norm_and_trimul_validation(lib):
    """The LayerNorm and triangle-multiplication entry points reject bad geometry on the host."""

    rg = _lib.RowNormGeometry()
    rg.dtype, rg.width, rg.rows, rg.x_row, rg.y_row, rg.eps = _lib.BF16, 0, 4, 8, 8, 1e-5
    fake = ctypes.c_void_p(16)
    assert lib.oops_layer_norm_rows_forward(ctypes.byref(rg), fake, None, None, fake, fake, fake, None) != 0
    assert b"width" in lib.oops_last_error()
    rg.width, rg.y_row = 8, 4  # y row stride below the width
    assert lib.oops_layer_norm_rows_forward(ctypes.byref(rg), fake, None, None, fake, fake, fake, None) != 0
    rg.width, rg.y_row, rg.x_row = 9000, 9000, 9000
    assert lib.oops_layer_norm_rows_parts(ctypes.byref(rg)) == 0
    assert lib.oops_layer_norm_rows_backward_workspace_bytes(ctypes.byref(rg)) == 0
    rg.width, rg.y_row, rg.x_row, rg.rows = 128, 128, 128, 1 << 18
    parts = lib.oops_layer_norm_rows_parts(ctypes.byref(rg))
    need = lib.oops_layer_norm_rows_backward_workspace_bytes(ctypes.byref(rg))
    assert need >= 2 * parts * 128 * 4 and need % 256 == 0
    # the summed backward needs the workspace when an affine gradient is asked for
    rc = lib.oops_layer_norm_rows_backward_affine(ctypes.byref(rg), fake, None, fake, fake, fake, fake, fake, None,
                                                  None, 0, None)  # fmt: skip
    assert rc == 3 and b"workspace" in lib.oops_last_error()

    tg = _lib.TrimulGeometry()
    tg.dtype, tg.channels, tg.hidden, tg.has_mask = 7, 16, 16, 0  # no such dtype
    tg.groups, tg.positions, tg.c_row, tg.h_row, tg.eps = 1, 16, 16, 16, 1e-5
    assert lib.oops_trimul_factors_forward(ctypes.byref(tg), fake, fake, None, None, fake, None) != 0
    assert b"bfloat16" in lib.oops_last_error()
    tg.dtype, tg.c_row = _lib.BF16, 12  # padded row stride must be a multiple of 8
    assert lib.oops_trimul_output_forward(ctypes.byref(tg), fake, fake, fake, fake, None, None, fake, None) != 0
    tg.c_row, tg.has_mask = 16, 1  # a mask flag without a mask pointer
    assert lib.oops_trimul_factors_forward(ctypes.byref(tg), fake, fake, None, None, fake, None) != 0
    assert b"mask" in lib.oops_last_error()
    tg.has_mask = 0
    assert lib.oops_trimul_mask_parts(ctypes.byref(tg)) == 2
    assert lib.oops_trimul_bias_parts(ctypes.byref(tg)) >= 1
    assert lib.oops_trimul_output_norm_parts(ctypes.byref(tg)) >= 1


def test_forward_noalloc_scratch_limit(lib):
    """A geometry whose bias copy exceeds the no-allocation forward's static scratch is not refused: that
    forward then reads the bias rows directly and needs no scratch (here, with no GPU, the launch itself
    fails, after the host checks)."""

    text = HEADER.read_text()
    assert int(re.search(r"#define\s+OOPS_NOALLOC_SCRATCH_BYTES\s+(\d+)", text).group(1)) == _lib.NOALLOC_SCRATCH_BYTES
    geo, keep = _geometry(c3_table(n=2080))
    assert lib.oops_attn_forward_workspace_bytes(ctypes.byref(geo)) > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.oops_attn_forward_noalloc(ctypes.byref(geo), 1, 1, 1, None, 1, 1, None, 1, None)
    assert rc not in (0, 3), rc  # 3: OOPS_EWORKSPACE
    assert "scratch" not in lib.oops_last_error().decode()
    # pointer checks come before any device call
    geo, keep = _geometry(c3_table())
    assert lib.oops_attn_forward_noalloc(ctypes.byref(geo), None, 1, 1, None, 1, 1, None, 1, None) == 1


def test_sum_partials_validates_on_the_host(lib):
    """oops_sum_partials checks its descriptors before any launch; zero segments launch nothing."""

    text = HEADER.read_text()
    assert int(re.search(r"#define\s+OOPS_SUM_MAX_SEGMENTS\s+(\d+)", text).group(1)) == _lib.SUM_MAX_SEGMENTS
    assert ctypes.sizeof(_lib.SumSegment) == 48
    assert lib.oops_sum_partials(None, 0, None, 0, None) == 0
    segs = (_lib.SumSegment * (_lib.SUM_MAX_SEGMENTS + 1))()
    assert lib.oops_sum_partials(segs, _lib.SUM_MAX_SEGMENTS + 1, None, 0, None) != 0
    assert b"num_segments" in lib.oops_last_error()
    assert lib.oops_sum_partials(None, 1, None, 0, None) != 0
    seg = segs[0]
    seg.parts, seg.out, seg.count, seg.n, seg.part_stride, seg.out_dtype = 16, 16, 2, 8, 4, _lib.F32
    assert lib.oops_sum_partials(segs, 1, None, 0, None) != 0  # part_stride below n
    assert b"part_stride" in lib.oops_last_error()
    seg.part_stride, seg.out_dtype = 8, 9
    assert lib.oops_sum_partials(segs, 1, None, 0, None) != 0
    assert b"out_dtype" in lib.oops_last_error()
    seg.out_dtype, seg.out = _lib.BF16, None
    assert lib.oops_sum_partials(segs, 1, None, 0, None) != 0
    assert b"non-NULL" in lib.oops_last_error()
    seg.out, seg.count = 16, 257  # more than 256 rows: a workspace of 2 chunk rows
    assert lib.oops_sum_partials_workspace_bytes(segs, 1) == 256
    assert lib.oops_sum_partials(segs, 1, None, 0, None) != 0
    assert b"workspace" in lib.oops_last_error()


def test_trimul_output_grad_validation(lib):
    """The output-gradient products serve 16-bit pairs with C = H = 128 only and check strides on the host."""

    tg = _lib.TrimulGeometry()
    tg.dtype, tg.channels, tg.hidden, tg.has_mask = _lib.BF16, 128, 128, 0
    tg.groups, tg.positions, tg.c_row, tg.h_row, tg.eps = 2, 300, 128, 128, 1e-5
    assert lib.oops_trimul_output_grad_parts(ctypes.byref(tg)) >= 1
    fake = ctypes.c_void_p(256)
    args = [fake, 128, fake, 128, fake, 128, fake, 128, fake, fake, None]
    bad = list(args)
    bad[1] = 100  # row stride below 128
    assert lib.oops_trimul_output_grad_products(ctypes.byref(tg), *bad) != 0
    assert b"stride" in lib.oops_last_error()
    bad = list(args)
    bad[4] = ctypes.c_void_p(258)  # misaligned operand
    assert lib.oops_trimul_output_grad_products(ctypes.byref(tg), *bad) != 0
    assert b"aligned" in lib.oops_last_error()
    bad = list(args)
    bad[8] = None
    assert lib.oops_trimul_output_grad_products(ctypes.byref(tg), *bad) != 0
    for dtype, c, h in ((_lib.F32, 128, 128), (_lib.BF16, 64, 128), (_lib.F16, 128, 96)):
        tg.dtype, tg.channels, tg.hidden = dtype, c, h
        assert lib.oops_trimul_output_grad_parts(ctypes.byref(tg)) == 0
        assert lib.oops_trimul_output_grad_products(ctypes.byref(tg), *args) != 0
