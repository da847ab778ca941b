"""Drop-in replacements for the window helpers of models/utils.py.

``window_partition`` / ``window_reverse`` run the HIP gather / scatter kernels
(device tensors only).  ``get_swin_attention_mask`` builds the dense
``[nW, N, N]`` shift mask on the host, as the reference does once in
``SequentialSwinTransformer.__init__``; the attention kernel itself never reads
it and evaluates the same mask in closed form (``kernels.ShiftMask``).
"""
from __future__ import annotations

from typing import Sequence, Tuple

import torch

from . import kernels
from .kernels import MASK_VALUE, WindowGeometry


def get_pad3d(input_resolution: Sequence[int], window_size: Sequence[int]) -> Tuple[int, ...]:
    """Centred padding that makes each of (Pl, Lat, Lon) a multiple of its window
    (models/utils.py:4-26): the odd pixel goes to the back/bottom/right.

    Returns (left, right, top, bottom, front, back).
    """
    pads = []
    for extent, win in zip(input_resolution, window_size):
        need = (-extent) % win
        pads.append((need // 2, need - need // 2))
    (front, back), (top, bottom), (left, right) = pads
    return left, right, top, bottom, front, back


def get_pad2d(input_resolution: Sequence[int], window_size: Sequence[int]) -> Tuple[int, int, int, int]:
    """(left, right, top, bottom) padding of an (H, W) grid (models/utils.py:28-32)."""
    return get_pad3d([2] + list(input_resolution), [2] + list(window_size))[:4]


def window_partition(x: torch.Tensor, window_size: int) -> torch.Tensor:
    """[B, H, W, C] -> [B * H/ws * W/ws, ws, ws, C] (models/utils.py:35-39), on the GPU."""
    B, H, W, C = x.shape
    if H % window_size or W % window_size:
        raise ValueError(f"grid {H}x{W} is not divisible by window {window_size}")
    geom = WindowGeometry(B, H, W, C, window_size)
    return kernels.swin_partition(x.contiguous(), geom).view(-1, window_size, window_size, C)


def window_reverse(windows: torch.Tensor, window_size: int, H: int, W: int) -> torch.Tensor:
    """[B_, ws, ws, C] -> [B, H, W, C] (models/utils.py:41-45), on the GPU.

    B is recovered from the window count the way the reference does it
    (float division, then int()).
    """
    B = int(windows.shape[0] / (H * W / window_size / window_size))
    C = windows.shape[-1]
    geom = WindowGeometry(B, H, W, C, window_size)
    return kernels.swin_reverse(windows.contiguous(), geom)


def region_ids(extent: int, window_size: int, shift_size: int) -> torch.Tensor:
    """Per-coordinate region id of one axis of the shifted frame: 0 on
    [0, extent-ws), 1 on [extent-ws, extent-shift), 2 on [extent-shift, extent)."""
    coord = torch.arange(extent)
    return (coord >= extent - window_size).to(torch.int64) + (coord >= extent - shift_size).to(torch.int64)


def get_swin_attention_mask(model_type, input_resolution, window_size, shift_size, manager=None) -> torch.Tensor:
    """Dense SW-MSA mask ``[nW, N, N]`` (models/utils.py:56-94): 0 where query and
    key lie in the same shift region of the frame, -100.0 elsewhere.

    Built on the host (the reference builds it at module construction).  Only
    the single-GPU ('sequential') layout exists here; the 'parallel' split of
    the mask across model-parallel ranks belongs to the multi-GPU path.
    """
    if model_type != "sequential":
        raise NotImplementedError("only model_type='sequential' is provided (single-GPU hot path)")
    H, W = input_resolution
    ws = window_size
    rid = 3 * region_ids(H, ws, shift_size)[:, None] + region_ids(W, ws, shift_size)[None, :]  # [H, W]
    # window-major token order: (wh, ww, ti, tj)
    rid = rid.view(H // ws, ws, W // ws, ws).permute(0, 2, 1, 3).reshape(-1, ws * ws)
    diff = rid[:, None, :] != rid[:, :, None]
    return torch.where(diff, torch.tensor(MASK_VALUE), torch.tensor(0.0))


def pack_key_bits(flags: torch.Tensor) -> torch.Tensor:
    """[nW, N] boolean/uint8 per-key flags -> [nW] int64 bit masks (bit j = key j)."""
    if flags.shape[-1] > 64:
        raise ValueError("at most 64 keys per window fit one bit mask")
    f = flags.to(torch.int64)
    bits = torch.zeros(f.shape[0], dtype=torch.int64, device=f.device)
    for j in range(f.shape[-1]):
        bits |= f[:, j] << j
    return bits


def land_window_bits(land: torch.Tensor, geom: WindowGeometry) -> torch.Tensor:
    """Per-window key land bits of the window frame ``geom`` (one image).

    ``land`` is a [H, W] boolean grid on the device; the flags are cut into
    windows with the same HIP gather as the activations, so key j of window w
    is exactly the token the attention kernel sees there.  Padding is ocean.
    """
    if land.dim() != 2 or tuple(land.shape) != (geom.height, geom.width):
        raise ValueError(f"land mask must be [{geom.height}, {geom.width}], got {tuple(land.shape)}")
    g1 = WindowGeometry(1, geom.height, geom.width, 1, geom.window, geom.shift_h, geom.shift_w, geom.pad,
                        geom.win_row_begin, geom.win_rows, geom.valid)
    flags = kernels.swin_partition(land.to(torch.uint8).contiguous().view(1, geom.height, geom.width, 1), g1)
    return pack_key_bits(flags.view(g1.num_windows, -1))
