"""terra_amd — MI355X (gfx950) shifted-window attention hot path of TERRA.

Drop-in modules and helpers (same names and signatures as the reference):

    terra_amd.attention.WindowAttention          models/attention.py:175
    terra_amd.transformer.SequentialSwinTransformer  models/transformer.py:71
    terra_amd.utils.window_partition / window_reverse / get_swin_attention_mask
                                                 models/utils.py:35-94
    terra_amd.window_assignment.get_window_indices
                                                 core/parallel/window_assignment.py:117

Kernels live in ``libterra_swin.so`` (C ABI: include/terra_swin.h), built by
``python -m terra_amd.build``.
"""
from . import config  # noqa: F401
from .kernels import ShiftMask, WindowGeometry, WindowMask, swin_partition, swin_reverse, window_attention  # noqa: F401

__all__ = [
    "ShiftMask",
    "WindowGeometry",
    "WindowMask",
    "swin_partition",
    "swin_reverse",
    "window_attention",
]
