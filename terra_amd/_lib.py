"""ctypes binding of ``libterra_swin.so`` (the C ABI declared in include/terra_swin.h).

The library is built in-tree by :func:`terra_amd.build.build_library`.  torch is
imported before the library is opened so that the HIP runtime torch ships
(SONAME ``libamdhip64.so.7``) is the one the library binds to: device pointers
and streams handed over from torch are then valid on the library side.

There is no fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

ABI_VERSION = 1

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_U8 = 3

MASK_NONE = 0
MASK_SHIFT = 1
MASK_EXPLICIT = 2

STATUS_NAMES = {
    0: "TERRA_OK",
    -1: "TERRA_ERR_NULL",
    -2: "TERRA_ERR_DTYPE",
    -3: "TERRA_ERR_SHAPE",
    -4: "TERRA_ERR_ALIGN",
    -5: "TERRA_ERR_UNSUPPORTED",
    -6: "TERRA_ERR_LAUNCH",
}

LIB_NAME = "libterra_swin.so"
# TERRA_SWIN_LIB names another build of the same library (the host
# AddressSanitizer build of the C-ABI checks); by default the in-tree one.
LIB_PATH = os.environ.get("TERRA_SWIN_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# Symbols the header declares; tests check the library exports each of them.
EXPORTED_SYMBOLS = (
    "terra_abi_version",
    "terra_last_error",
    "terra_swin_partition",
    "terra_swin_partition_ln",
    "terra_swin_partition_ln_mixed",
    "terra_swin_partition_ln_bwd",
    "terra_swin_partition_ln_bwd_mixed",
    "terra_swin_reverse",
    "terra_swin_reverse_mixed",
    "terra_swin_partition_mixed",
    "terra_swin_attn_fwd",
    "terra_swin_attn_bwd",
    "terra_swin_attn_bwd_sums",
    "terra_swin_block_fwd",
    "terra_swin_pack_linear",
    "terra_swin_mlp_fwd",
    "terra_swin_gelu_bwd",
    "terra_swin_linear",
    "terra_swin_linear_residual",
)


class SwinGeom(ctypes.Structure):
    """Mirror of ``terra_swin_geom``."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("shift_h", ctypes.c_int32),
        ("shift_w", ctypes.c_int32),
        ("pad_top", ctypes.c_int32),
        ("pad_bottom", ctypes.c_int32),
        ("pad_left", ctypes.c_int32),
        ("pad_right", ctypes.c_int32),
        ("win_row_begin", ctypes.c_int32),
        ("win_rows", ctypes.c_int32),
        ("valid_begin", ctypes.c_int32),
        ("valid_end", ctypes.c_int32),
    ]


class SwinAttnDesc(ctypes.Structure):
    """Mirror of ``terra_swin_attn_desc``."""

    _fields_ = [
        ("num_windows", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("window_h", ctypes.c_int32),
        ("window_w", ctypes.c_int32),
        ("n_real", ctypes.c_int32),
        ("q_stride", ctypes.c_int32),
        ("k_stride", ctypes.c_int32),
        ("v_stride", ctypes.c_int32),
        ("o_stride", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("mask_value", ctypes.c_float),
        ("pad_key_value", ctypes.c_float),
        ("mask_mode", ctypes.c_int32),
        ("mask_windows", ctypes.c_int32),
        ("frame_h", ctypes.c_int32),
        ("frame_w", ctypes.c_int32),
        ("shift_h", ctypes.c_int32),
        ("shift_w", ctypes.c_int32),
        ("win_row_begin", ctypes.c_int32),
        ("win_rows", ctypes.c_int32),
        ("win_cols", ctypes.c_int32),
    ]


class SwinAttnBwdDesc(ctypes.Structure):
    """Mirror of ``terra_swin_attn_bwd_desc``."""

    _fields_ = [
        ("fwd", SwinAttnDesc),
        ("dout_stride", ctypes.c_int32),
        ("dq_stride", ctypes.c_int32),
        ("dk_stride", ctypes.c_int32),
        ("dv_stride", ctypes.c_int32),
    ]


class SwinBlockDesc(ctypes.Structure):
    """Mirror of ``terra_swin_block_desc``."""

    _fields_ = [
        ("geom", SwinGeom),
        ("heads", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("ln_eps", ctypes.c_float),
        ("mask_value", ctypes.c_float),
        ("layernorm", ctypes.c_int32),
        ("shift_mask", ctypes.c_int32),
        ("land_windows", ctypes.c_int32),
        ("packed_weights", ctypes.c_int32),
    ]


class SwinMlpDesc(ctypes.Structure):
    """Mirror of ``terra_swin_mlp_desc``."""

    _fields_ = [
        ("tokens", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("layernorm", ctypes.c_int32),
        ("ln_eps", ctypes.c_float),
    ]


class TerraError(RuntimeError):
    """A C-ABI call returned a launch-time failure."""


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Open the library once and declare the entry-point signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"terra_amd: {LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python -m terra_amd.build` first (there is no non-HIP fallback)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        vp = ctypes.c_void_p
        lib.terra_abi_version.restype = ctypes.c_int
        lib.terra_abi_version.argtypes = []
        lib.terra_last_error.restype = ctypes.c_char_p
        lib.terra_last_error.argtypes = []
        lib.terra_swin_partition.restype = ctypes.c_int
        lib.terra_swin_partition.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(SwinGeom), ctypes.c_float, vp]
        lib.terra_swin_partition_ln.restype = ctypes.c_int
        lib.terra_swin_partition_ln.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(SwinGeom), vp, vp,
                                                ctypes.c_float, ctypes.c_float, vp]
        lib.terra_swin_partition_ln_bwd.restype = ctypes.c_int
        lib.terra_swin_partition_ln_bwd.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.POINTER(SwinGeom), vp,
                                                    ctypes.c_float, vp, vp, vp]
        lib.terra_swin_partition_ln_mixed.restype = ctypes.c_int
        lib.terra_swin_partition_ln_mixed.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.POINTER(SwinGeom),
                                                      vp, vp, ctypes.c_float, ctypes.c_float, vp]
        lib.terra_swin_partition_ln_bwd_mixed.restype = ctypes.c_int
        lib.terra_swin_partition_ln_bwd_mixed.argtypes = [vp, ctypes.c_int, vp, vp, vp, ctypes.c_int,
                                                          ctypes.POINTER(SwinGeom), vp, ctypes.c_float, vp, vp, vp]
        lib.terra_swin_reverse.restype = ctypes.c_int
        lib.terra_swin_reverse.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.POINTER(SwinGeom), vp]
        lib.terra_swin_gelu_bwd.restype = ctypes.c_int
        lib.terra_swin_gelu_bwd.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int, vp, vp]
        lib.terra_swin_reverse_mixed.restype = ctypes.c_int
        lib.terra_swin_reverse_mixed.argtypes = [vp, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.POINTER(SwinGeom),
                                                 vp]
        lib.terra_swin_partition_mixed.restype = ctypes.c_int
        lib.terra_swin_partition_mixed.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, ctypes.POINTER(SwinGeom),
                                                   ctypes.c_float, vp, vp]
        lib.terra_swin_attn_fwd.restype = ctypes.c_int
        lib.terra_swin_attn_fwd.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.POINTER(SwinAttnDesc), vp, vp, vp, vp]
        lib.terra_swin_attn_bwd.restype = ctypes.c_int
        lib.terra_swin_attn_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.POINTER(SwinAttnBwdDesc),
                                            vp, vp, vp, vp, vp]
        lib.terra_swin_attn_bwd_sums.restype = ctypes.c_int
        lib.terra_swin_attn_bwd_sums.argtypes = [vp, vp, vp, vp, vp, vp, vp, ctypes.c_int,
                                                 ctypes.POINTER(SwinAttnBwdDesc), vp, vp, vp, vp, vp, vp, vp, vp]
        lib.terra_swin_block_fwd.restype = ctypes.c_int
        lib.terra_swin_block_fwd.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(SwinBlockDesc), vp, vp, vp, vp, vp,
                                             vp, vp, vp, vp]
        lib.terra_swin_pack_linear.restype = ctypes.c_int
        lib.terra_swin_pack_linear.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        lib.terra_swin_mlp_fwd.restype = ctypes.c_int
        lib.terra_swin_mlp_fwd.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(SwinMlpDesc), vp, vp, vp, vp, vp, vp,
                                           vp]
        i64 = ctypes.c_int64
        lib.terra_swin_linear.restype = ctypes.c_int
        lib.terra_swin_linear.argtypes = [vp, vp, ctypes.c_int, i64, ctypes.c_int, ctypes.c_int, i64, i64, vp, vp,
                                          ctypes.c_int, vp]
        lib.terra_swin_linear_residual.restype = ctypes.c_int
        lib.terra_swin_linear_residual.argtypes = [vp, vp, vp, ctypes.c_int, i64, ctypes.c_int, ctypes.c_int, vp, vp,
                                                   ctypes.POINTER(SwinGeom), vp]
        version = lib.terra_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"terra_amd: {LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def last_error() -> str:
    return load().terra_last_error().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    """Raise the Python exception the reference would raise for a failed call.

    Argument errors (shape, dtype, alignment, NULL, unsupported) become
    ``ValueError``; a rejected launch becomes :class:`TerraError`.
    """
    if status == 0:
        return
    name = STATUS_NAMES.get(status, str(status))
    msg = f"{what}: {name}: {last_error()}"
    if status == -6:
        raise TerraError(msg)
    raise ValueError(msg)
