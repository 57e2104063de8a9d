"""ctypes binding of the C-ABI library ``oops_amd/lib/liboops_amd.so``.

The library is the product's compute path; nothing here falls back to another
implementation.  If it is missing or fails to load, every operator raises.
The structure and constants mirror ``include/oops_amd.h``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("OOPS_AMD_LIB") or Path(__file__).resolve().parent / "lib" / "liboops_amd.so")

F32, BF16, F16 = 0, 1, 2
BIAS_NONE, BIAS_FULL, BIAS_SHARED = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 32 << 20
PHASE_DELTA, PHASE_DQ, PHASE_DKV, PHASE_DBIAS = 1, 2, 4, 8
TABLE_WIDTH = 40
ABI_VERSION = 6

# geometry table columns (enum oops_table_column)
(
    T_GROUPS, T_LEN_Q, T_LEN_K,
    T_Q_OFF, T_Q_SG, T_Q_SH, T_Q_SI,
    T_K_OFF, T_K_SG, T_K_SH, T_K_SI,
    T_V_OFF, T_V_SG, T_V_SH, T_V_SI,
    T_O_OFF, T_O_SG, T_O_SH, T_O_SI,
    T_DO_OFF, T_DO_SG, T_DO_SH, T_DO_SI,
    T_B_OFF, T_B_SG, T_B_SH, T_B_SI,
    T_M_OFF, T_M_SG, T_M_SI,
    T_L_OFF,
    T_DB_OFF, T_DB_SG, T_DB_SH, T_DB_SI,
    T_BIAS_MODE,
) = range(36)  # fmt: skip

EXPORTED_SYMBOLS = (
    "oops_attn_forward",
    "oops_attn_forward_noalloc",
    "oops_attn_forward_workspace_bytes",
    "oops_attn_backward_workspace_bytes",
    "oops_attn_backward",
    "oops_gate_projection_forward",
    "oops_gate_multiply_forward",
    "oops_gate_multiply_backward",
    "oops_layer_norm_rows_forward",
    "oops_layer_norm_rows_parts",
    "oops_layer_norm_rows_backward",
    "oops_layer_norm_rows_backward_workspace_bytes",
    "oops_layer_norm_rows_backward_affine",
    "oops_trimul_factors_forward",
    "oops_trimul_mask_parts",
    "oops_trimul_bias_parts",
    "oops_trimul_factors_backward",
    "oops_trimul_output_norm_forward",
    "oops_trimul_output_norm_parts",
    "oops_trimul_output_norm_backward",
    "oops_trimul_output_forward",
    "oops_trimul_output_backward",
    "oops_trimul_output_grad_parts",
    "oops_trimul_output_grad_products",
    "oops_sum_partials_workspace_bytes",
    "oops_sum_partials",
    "oops_last_error",
    "oops_abi_version",
)


class Geometry(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("num_samples", ctypes.c_int32),
        ("has_bias", ctypes.c_int32),
        ("has_mask", ctypes.c_int32),
        ("vec_ok", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("phases", ctypes.c_int32),
        ("force_generic", ctypes.c_int32),
        ("table_host", ctypes.c_void_p),
        ("table_device", ctypes.c_void_p),
    ]


class GateGeometry(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("tokens", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("a_sb", ctypes.c_int64),
        ("a_sg", ctypes.c_int64),
        ("a_st", ctypes.c_int64),
        ("a_sh", ctypes.c_int64),
        ("a_sd", ctypes.c_int64),
        ("s_row", ctypes.c_int64),
        ("w_row", ctypes.c_int64),
    ]


class RowNormGeometry(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("x_row", ctypes.c_int64),
        ("y_row", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


class TrimulGeometry(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("has_mask", ctypes.c_int32),
        ("groups", ctypes.c_int64),
        ("positions", ctypes.c_int64),
        ("c_row", ctypes.c_int64),
        ("h_row", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


SUM_MAX_SEGMENTS = 16


class SumSegment(ctypes.Structure):
    _fields_ = [
        ("parts", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("count", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("part_stride", ctypes.c_int64),
        ("out_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises ``RuntimeError`` if it is absent."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"oops_amd native library not built: {LIB_PATH} is missing "
                "(run `python -m oops_amd.csrc.build` or __graft_entry__.build())"
            )
        # torch first: its HIP runtime then serves the library as well
        import torch  # noqa: F401

        lib = ctypes.CDLL(os.fspath(LIB_PATH))
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        geo = ctypes.POINTER(Geometry)
        lib.oops_attn_forward.argtypes = [geo, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.oops_attn_forward.restype = i32
        lib.oops_attn_forward_noalloc.argtypes = [geo, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_attn_forward_noalloc.restype = i32
        lib.oops_attn_forward_workspace_bytes.argtypes = [geo]
        lib.oops_attn_forward_workspace_bytes.restype = sz
        lib.oops_attn_backward_workspace_bytes.argtypes = [geo]
        lib.oops_attn_backward_workspace_bytes.restype = sz
        lib.oops_attn_backward.argtypes = [geo, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.oops_attn_backward.restype = i32
        gg = ctypes.POINTER(GateGeometry)
        lib.oops_gate_projection_forward.argtypes = [gg, vp, vp, vp, vp, vp, vp]
        lib.oops_gate_projection_forward.restype = i32
        lib.oops_gate_multiply_forward.argtypes = [gg, vp, vp, vp, vp]
        lib.oops_gate_multiply_forward.restype = i32
        lib.oops_gate_multiply_backward.argtypes = [gg, vp, vp, vp, vp, vp, vp]
        lib.oops_gate_multiply_backward.restype = i32
        rg = ctypes.POINTER(RowNormGeometry)
        lib.oops_layer_norm_rows_forward.argtypes = [rg, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_layer_norm_rows_forward.restype = i32
        lib.oops_layer_norm_rows_parts.argtypes = [rg]
        lib.oops_layer_norm_rows_parts.restype = sz
        lib.oops_layer_norm_rows_backward.argtypes = [rg, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_layer_norm_rows_backward.restype = i32
        lib.oops_layer_norm_rows_backward_workspace_bytes.argtypes = [rg]
        lib.oops_layer_norm_rows_backward_workspace_bytes.restype = sz
        lib.oops_layer_norm_rows_backward_affine.argtypes = [rg, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.oops_layer_norm_rows_backward_affine.restype = i32
        tg = ctypes.POINTER(TrimulGeometry)
        lib.oops_trimul_factors_forward.argtypes = [tg, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_factors_forward.restype = i32
        lib.oops_trimul_mask_parts.argtypes = [tg]
        lib.oops_trimul_mask_parts.restype = sz
        lib.oops_trimul_bias_parts.argtypes = [tg]
        lib.oops_trimul_bias_parts.restype = sz
        lib.oops_trimul_factors_backward.argtypes = [tg, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_factors_backward.restype = i32
        lib.oops_trimul_output_norm_forward.argtypes = [tg, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_output_norm_forward.restype = i32
        lib.oops_trimul_output_norm_parts.argtypes = [tg]
        lib.oops_trimul_output_norm_parts.restype = sz
        lib.oops_trimul_output_norm_backward.argtypes = [tg, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_output_norm_backward.restype = i32
        lib.oops_trimul_output_forward.argtypes = [tg, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_output_forward.restype = i32
        lib.oops_trimul_output_backward.argtypes = [tg, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.oops_trimul_output_backward.restype = i32
        i64 = ctypes.c_int64
        lib.oops_trimul_output_grad_parts.argtypes = [tg]
        lib.oops_trimul_output_grad_parts.restype = sz
        lib.oops_trimul_output_grad_products.argtypes = [tg, vp, i64, vp, i64, vp, i64, vp, i64, vp, vp, vp]
        lib.oops_trimul_output_grad_products.restype = i32
        lib.oops_sum_partials_workspace_bytes.argtypes = [ctypes.POINTER(SumSegment), ctypes.c_int32]
        lib.oops_sum_partials_workspace_bytes.restype = sz
        lib.oops_sum_partials.argtypes = [ctypes.POINTER(SumSegment), ctypes.c_int32, vp, sz, vp]
        lib.oops_sum_partials.restype = i32
        lib.oops_last_error.argtypes = []
        lib.oops_last_error.restype = ctypes.c_char_p
        lib.oops_abi_version.argtypes = []
        lib.oops_abi_version.restype = i32
        if lib.oops_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"oops_amd native library ABI {lib.oops_abi_version()} does not match the Python side ({ABI_VERSION})"
            )
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        message = load().oops_last_error().decode(errors="replace")
        raise RuntimeError(f"oops_amd {what} failed (code {rc}): {message}")
