"""Tensor-level entry points of the HIP hot path.

Each function validates its torch arguments, fills the C descriptor and calls
the C ABI on the current HIP stream of the tensor's device.  There is no CPU
or eager-PyTorch fallback: a tensor that is not on a ROCm device, or a build
without ``libterra_swin.so``, raises.
"""
from __future__ import annotations

import ctypes
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple, Union

import torch

from . import _lib

_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.uint8: _lib.DTYPE_U8,
}

# Additive constants of the reference: the shift mask uses -100.0
# (models/utils.py:84) and padded keys are filled with -10000.0
# (models/attention.py:907).
MASK_VALUE = -100.0
PAD_KEY_VALUE = -10000.0


@dataclass(frozen=True)
class WindowGeometry:
    """Token grid -> window grid geometry (mirror of ``terra_swin_geom``).

    The window frame is the grid zero-padded by ``pad`` = (top, bottom, left,
    right) and rolled by ``(-shift_h, -shift_w)``; windows of the frame rows
    ``[win_row_begin, win_row_begin + win_rows)`` are emitted, and windows of an
    image outside ``valid`` (flat index range) are pad windows.
    """

    batch: int
    height: int
    width: int
    channels: int
    window: int
    shift_h: int = 0
    shift_w: int = 0
    pad: Tuple[int, int, int, int] = (0, 0, 0, 0)
    win_row_begin: int = 0
    win_rows: Optional[int] = None
    valid: Optional[Tuple[int, int]] = None

    @property
    def frame_h(self) -> int:
        return self.height + self.pad[0] + self.pad[1]

    @property
    def frame_w(self) -> int:
        return self.width + self.pad[2] + self.pad[3]

    @property
    def rows(self) -> int:
        return self.win_rows if self.win_rows is not None else self.frame_h // self.window - self.win_row_begin

    @property
    def cols(self) -> int:
        return self.frame_w // self.window

    @property
    def windows_per_image(self) -> int:
        return self.rows * self.cols

    @property
    def num_windows(self) -> int:
        return self.batch * self.windows_per_image

    def to_c(self) -> _lib.SwinGeom:
        g = _lib.SwinGeom()
        g.batch, g.height, g.width, g.channels, g.window = (
            self.batch, self.height, self.width, self.channels, self.window)
        g.shift_h, g.shift_w = self.shift_h, self.shift_w
        g.pad_top, g.pad_bottom, g.pad_left, g.pad_right = self.pad
        g.win_row_begin = self.win_row_begin
        g.win_rows = self.win_rows if self.win_rows is not None else 0
        if self.valid is not None:
            g.valid_begin, g.valid_end = self.valid
        else:
            g.valid_begin, g.valid_end = 0, 0
        return g


@dataclass(frozen=True)
class ShiftMask:
    """Analytic Swin shift mask of a window frame (no [nW, N, N] tensor).

    Equal, element for element, to ``get_swin_attention_mask`` of the frame
    (models/utils.py:56-94) for the emitted window rows.
    """

    frame_h: int
    frame_w: int
    shift_h: int
    shift_w: int
    win_row_begin: int
    win_rows: int
    win_cols: int

    @staticmethod
    def from_geometry(geom: WindowGeometry) -> "ShiftMask":
        return ShiftMask(geom.frame_h, geom.frame_w, geom.shift_h, geom.shift_w,
                         geom.win_row_begin, geom.rows, geom.cols)


@dataclass(frozen=True)
class WindowMask:
    """Mask terms of one attention call: a shift mask (analytic or explicit
    ``[nW, N, N]`` fp32 tensor) plus optional per-window land bits (uint64 bit
    j set: key j is land and receives ``mask_value``)."""

    shift: Union[None, ShiftMask, torch.Tensor] = None
    land_bits: Optional[torch.Tensor] = None


def autocast_bf16(x: torch.Tensor) -> bool:
    """Whether a bf16 autocast region is active for x's device type: there
    F.linear casts fp32 weights to bf16 (core/runtime/run_model.py:424-448
    runs the reference's forward under torch.amp.autocast("cuda", bf16))."""
    dt = x.device.type
    return torch.is_autocast_enabled(dt) and torch.get_autocast_dtype(dt) == torch.bfloat16


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                "terra_amd kernels run on ROCm devices only (got a tensor on "
                f"'{t.device}'); there is no CPU fallback")
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _dtype_code(t: torch.Tensor, allowed: Sequence[torch.dtype]) -> int:
    if t.dtype not in allowed:
        raise TypeError(f"dtype {t.dtype} not supported here (supported: {', '.join(map(str, allowed))})")
    return _DTYPES[t.dtype]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def swin_partition(x: torch.Tensor, geom: WindowGeometry, pad_value: float = 0.0,
                   out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                   column_sums: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused pad + roll(-shift) + window_partition of ``x`` [B, H, W, C].

    Returns windows ``[B * nW, ws*ws, C]`` (the layout of
    ``window_partition(...).view(-1, ws*ws, C)``, models/transformer.py:225)
    in ``out_dtype`` (default: x's dtype; bf16 for fp32 x rounds each value
    once, as a cast of the fp32 result would).  ``column_sums``: an fp32 [C]
    tensor the per-channel sums of the bf16 windows written are ADDED into
    (bf16 output from fp32 x only).
    """
    dev = _require_device(x)
    code = _dtype_code(x, tuple(_DTYPES))
    if x.dim() != 4 or tuple(x.shape) != (geom.batch, geom.height, geom.width, geom.channels):
        raise ValueError(f"x shape {tuple(x.shape)} does not match geometry "
                         f"{(geom.batch, geom.height, geom.width, geom.channels)}")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous [B, H, W, C]")
    odt = x.dtype if out_dtype is None else out_dtype
    mixed = odt != x.dtype
    if mixed and not (x.dtype == torch.float32 and odt == torch.bfloat16):
        raise ValueError(f"out_dtype {odt} is not available for {x.dtype} x (fp32 x may give bf16 windows)")
    if column_sums is not None:
        if not mixed:
            raise ValueError("column_sums are summed by the fp32 -> bf16 partition only")
        if column_sums.dtype != torch.float32 or tuple(column_sums.shape) != (geom.channels,) \
                or not column_sums.is_contiguous() or column_sums.device != dev:
            raise ValueError(f"column_sums must be a contiguous fp32 [{geom.channels}] tensor on {dev}")
    shape = (geom.num_windows, geom.window * geom.window, geom.channels)
    if out is None:
        out = torch.empty(shape, dtype=odt, device=dev)
    elif tuple(out.shape) != shape or out.dtype != odt or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {odt} tensor of shape {shape} on {dev}")
    if geom.batch == 0:  # an empty batch: nothing to launch (torch returns the empty result)
        return out
    c_geom = geom.to_c()
    with torch.cuda.device(dev):
        if mixed:
            st = _lib.load().terra_swin_partition_mixed(_ptr(x), code, _ptr(out), _lib.DTYPE_BF16,
                                                        ctypes.byref(c_geom), float(pad_value), _ptr(column_sums),
                                                        _stream(dev))
        else:
            st = _lib.load().terra_swin_partition(_ptr(x), _ptr(out), code, ctypes.byref(c_geom),
                                                  float(pad_value), _stream(dev))
    _lib.check(st, "terra_swin_partition_mixed" if mixed else "terra_swin_partition")
    return out


def swin_partition_ln(x: torch.Tensor, geom: WindowGeometry, weight: Optional[torch.Tensor],
                      bias: Optional[torch.Tensor], eps: float, pad_value: float = 0.0,
                      out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Fused LayerNorm over C (nn.LayerNorm semantics, fp32 statistics) +
    pad + roll(-shift) + window_partition of ``x`` [B, H, W, C].

    Replaces ``norm1`` followed by the roll and partition of
    models/transformer.py:150-182.  Returns windows ``[B * nW, ws*ws, C]``
    in ``out_dtype`` (default: x's dtype; bf16 for fp32 x gives the fp32
    output rounded once, as autocast's cast at the next Linear would).
    """
    dev = _require_device(x)
    code = _dtype_code(x, (torch.float32, torch.float16, torch.bfloat16))
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype != x.dtype and not (x.dtype == torch.float32 and out_dtype == torch.bfloat16):
        raise ValueError(f"out_dtype {out_dtype} for x of {x.dtype}: the mixed form takes fp32 x and bf16 windows")
    if x.dim() != 4 or tuple(x.shape) != (geom.batch, geom.height, geom.width, geom.channels):
        raise ValueError(f"x shape {tuple(x.shape)} does not match geometry "
                         f"{(geom.batch, geom.height, geom.width, geom.channels)}")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous [B, H, W, C]")
    params = []
    for name, t in (("weight", weight), ("bias", bias)):
        if t is None:
            params.append(None)
            continue
        _require_device(x, t)
        if t.dim() != 1 or t.shape[0] != geom.channels:
            raise ValueError(f"LayerNorm {name} must be [{geom.channels}]")
        params.append(t.detach().to(torch.float32).contiguous())
    shape = (geom.num_windows, geom.window * geom.window, geom.channels)
    if out is None:
        out = torch.empty(shape, dtype=out_dtype, device=dev)
    elif tuple(out.shape) != shape or out.dtype != out_dtype or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {out_dtype} tensor of shape {shape} on {dev}")
    if geom.batch == 0:
        return out
    c_geom = geom.to_c()
    with torch.cuda.device(dev):
        if out_dtype == x.dtype:
            st = _lib.load().terra_swin_partition_ln(_ptr(x), _ptr(out), code, ctypes.byref(c_geom), _ptr(params[0]),
                                                     _ptr(params[1]), float(eps), float(pad_value), _stream(dev))
        else:
            st = _lib.load().terra_swin_partition_ln_mixed(_ptr(x), code, _ptr(out), _lib.DTYPE_BF16,
                                                           ctypes.byref(c_geom), _ptr(params[0]), _ptr(params[1]),
                                                           float(eps), float(pad_value), _stream(dev))
    _lib.check(st, "terra_swin_partition_ln")
    return out


def swin_partition_ln_backward(dwindows: torch.Tensor, x: torch.Tensor, geom: WindowGeometry,
                               weight: Optional[torch.Tensor], eps: float,
                               dresidual: Optional[torch.Tensor] = None, dweight: Optional[torch.Tensor] = None,
                               dbias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gradient of :func:`swin_partition_ln` with respect to ``x`` [B, H, W, C]
    given the windows' gradient ``dwindows`` [B * nW, ws*ws, C] (plus
    ``dresidual``, the gradient reaching x by another path, if given).
    ``dweight`` / ``dbias``: fp32 [C] tensors the LayerNorm weight and bias
    gradients are ADDED into, or None.  ``out`` may be ``dresidual``.
    ``dwindows`` is in x's dtype, or bf16 for fp32 x (the gradient of the
    bf16 windows ``swin_partition_ln(..., out_dtype=torch.bfloat16)`` gives,
    read exactly)."""
    dev = _require_device(dwindows, x)
    code = _dtype_code(x, (torch.float32, torch.float16, torch.bfloat16))
    shape = (geom.batch, geom.height, geom.width, geom.channels)
    if tuple(x.shape) != shape or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous {shape} tensor")
    n = geom.window * geom.window
    mixed = dwindows.dtype == torch.bfloat16 and x.dtype == torch.float32
    if (dwindows.dtype != x.dtype and not mixed) or dwindows.numel() != geom.num_windows * n * geom.channels \
            or not dwindows.is_contiguous():
        raise ValueError(f"dwindows must be a contiguous {x.dtype} (or, for fp32 x, bf16) tensor of "
                         f"{geom.num_windows} x {n} x {geom.channels} elements")
    for name, t in (("dresidual", dresidual), ("out", out)):
        if t is not None and (t.dtype != x.dtype or t.numel() != x.numel() or not t.is_contiguous()
                              or t.device != dev):
            raise ValueError(f"{name} must be a contiguous {x.dtype} tensor like x on {dev}")
    w32 = None
    if weight is not None:
        _require_device(x, weight)
        if weight.dim() != 1 or weight.shape[0] != geom.channels:
            raise ValueError(f"LayerNorm weight must be [{geom.channels}]")
        w32 = weight.detach().to(torch.float32).contiguous()
    for name, t in (("dweight", dweight), ("dbias", dbias)):
        if t is not None and (t.dtype != torch.float32 or tuple(t.shape) != (geom.channels,) or not t.is_contiguous()
                              or t.device != dev):
            raise ValueError(f"{name} must be a contiguous fp32 [{geom.channels}] tensor on {dev}")
    if out is None:
        out = torch.empty(shape, dtype=x.dtype, device=dev)
    if geom.batch == 0:
        return out.view(shape)
    c_geom = geom.to_c()
    with torch.cuda.device(dev):
        if mixed:
            st = _lib.load().terra_swin_partition_ln_bwd_mixed(_ptr(dwindows), _lib.DTYPE_BF16, _ptr(x),
                                                               _ptr(dresidual), _ptr(out), code, ctypes.byref(c_geom),
                                                               _ptr(w32), float(eps), _ptr(dweight), _ptr(dbias),
                                                               _stream(dev))
        else:
            st = _lib.load().terra_swin_partition_ln_bwd(_ptr(dwindows), _ptr(x), _ptr(dresidual), _ptr(out), code,
                                                         ctypes.byref(c_geom), _ptr(w32), float(eps), _ptr(dweight),
                                                         _ptr(dbias), _stream(dev))
    _lib.check(st, "terra_swin_partition_ln_bwd")
    return out.view(shape)


def rows_geometry(tokens: int, channels: int) -> WindowGeometry:
    """The identity frame over ``tokens`` rows of C channels (x viewed as
    [1, tokens, 1, C], window 1, no shift): partition and its LayerNorm /
    backward variants then act on plain token rows."""
    return WindowGeometry(1, tokens, 1, channels, 1)


def swin_reverse(windows: torch.Tensor, geom: WindowGeometry, residual: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Fused window_reverse + roll(+shift) + crop (+ residual) to [B, H, W, C]
    in ``out_dtype`` (default: the windows' dtype; fp32 for bf16 windows
    widens them exactly and adds an fp32 residual in fp32, as torch's type
    promotion does for ``shortcut + x``)."""
    dev = _require_device(windows) if residual is None else _require_device(windows, residual)
    code = _dtype_code(windows, tuple(_DTYPES))
    odt = windows.dtype if out_dtype is None else out_dtype
    mixed = odt != windows.dtype
    if mixed and not (windows.dtype == torch.bfloat16 and odt == torch.float32):
        raise ValueError(f"out_dtype {odt} is not available for {windows.dtype} windows (bf16 windows may give fp32)")
    n = geom.window * geom.window
    if windows.numel() != geom.num_windows * n * geom.channels:
        raise ValueError(f"windows has {windows.numel()} elements, geometry needs "
                         f"{geom.num_windows} x {n} x {geom.channels}")
    if not windows.is_contiguous():
        raise ValueError("windows must be contiguous")
    shape = (geom.batch, geom.height, geom.width, geom.channels)
    if residual is not None:
        if residual.dtype != odt or residual.numel() != geom.batch * geom.height * geom.width * geom.channels:
            raise ValueError("residual must match the output grid in dtype and size")
        if not residual.is_contiguous():
            raise ValueError("residual must be contiguous")
    if out is None:
        out = torch.empty(shape, dtype=odt, device=dev)
    elif out.numel() != geom.batch * geom.height * geom.width * geom.channels or out.dtype != odt \
            or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {odt} tensor with {shape} elements on {dev}")
    if geom.batch == 0:
        return out.view(shape)
    c_geom = geom.to_c()
    with torch.cuda.device(dev):
        if mixed:
            st = _lib.load().terra_swin_reverse_mixed(_ptr(windows), code, _ptr(out), _ptr(residual),
                                                      _lib.DTYPE_F32, ctypes.byref(c_geom), _stream(dev))
        else:
            st = _lib.load().terra_swin_reverse(_ptr(windows), _ptr(out), _ptr(residual), code,
                                                ctypes.byref(c_geom), _stream(dev))
    _lib.check(st, "terra_swin_reverse_mixed" if mixed else "terra_swin_reverse")
    return out.view(shape)


def _row_stride(t: torch.Tensor, name: str, num_windows: int, tokens: int, channels: int) -> int:
    if t.dim() != 3 or tuple(t.shape) != (num_windows, tokens, channels):
        raise ValueError(f"{name} must be [{num_windows}, {tokens}, {channels}], got {tuple(t.shape)}")
    s0, s1, s2 = t.stride()
    if s2 != 1 or s0 != tokens * s1:
        raise ValueError(f"{name} must have unit channel stride and packed windows (strides {t.stride()})")
    return s1


def window_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                     window_size: Tuple[int, int], scale: float,
                     bias_table: Optional[torch.Tensor] = None,
                     mask: Union[None, torch.Tensor, ShiftMask, WindowMask] = None,
                     n_real: Optional[int] = None,
                     mask_value: float = MASK_VALUE, pad_key_value: float = PAD_KEY_VALUE,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused window-attention core: softmax(q k^T * scale + bias + mask) v.

    q, k, v: [B_, N, C] (row stride may exceed C, e.g. slices of a fused qkv
    projection); heads are contiguous D = C / num_heads column blocks.
    Returns o [B_, N, C] contiguous, i.e. ``(attn @ v).transpose(1, 2)
    .reshape(B_, N, C)`` of models/attention.py:278.
    """
    dev = _require_device(q, k, v)
    code = _dtype_code(q, (torch.bfloat16, torch.float32))
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k and v must share a dtype")
    num_windows, tokens, channels = q.shape
    qs = _row_stride(q, "q", num_windows, tokens, channels)
    ks = _row_stride(k, "k", num_windows, tokens, channels)
    vs = _row_stride(v, "v", num_windows, tokens, channels)
    if out is None:
        out = torch.empty((num_windows, tokens, channels), dtype=q.dtype, device=dev)
    elif out.dtype != q.dtype or out.device != dev:
        raise ValueError(f"out must be a {q.dtype} tensor on {dev} (got {out.dtype} on {out.device})")
    os_ = _row_stride(out, "out", num_windows, tokens, channels)
    if num_windows == 0:
        return out

    d = _attn_desc(q, num_heads, window_size, scale, n_real, mask_value, pad_key_value, (qs, ks, vs, os_))
    table = _bias_table(bias_table, d)
    emask, land = _attn_masks(d, num_windows, mask)

    with torch.cuda.device(dev):
        st = _lib.load().terra_swin_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(out), code, ctypes.byref(d),
                                             _ptr(table), _ptr(emask), _ptr(land), _stream(dev))
    _lib.check(st, "terra_swin_attn_fwd")
    return out


def _attn_desc(q: torch.Tensor, num_heads: int, window_size: Tuple[int, int], scale: float,
               n_real: Optional[int], mask_value: float, pad_key_value: float,
               strides: Tuple[int, int, int, int]) -> _lib.SwinAttnDesc:
    num_windows, tokens, channels = q.shape
    d = _lib.SwinAttnDesc()
    d.num_windows, d.tokens, d.channels, d.heads = num_windows, tokens, channels, num_heads
    d.window_h, d.window_w = int(window_size[0]), int(window_size[1])
    d.n_real = tokens if n_real is None else int(n_real)
    d.q_stride, d.k_stride, d.v_stride, d.o_stride = strides
    d.scale, d.mask_value, d.pad_key_value = float(scale), float(mask_value), float(pad_key_value)
    return d


def _attn_masks(d: _lib.SwinAttnDesc, num_windows: int,
                mask: Union[None, torch.Tensor, ShiftMask, WindowMask]):
    """Fills the mask fields of ``d``; returns (explicit fp32 mask, land bits)."""
    shift = mask.shift if isinstance(mask, WindowMask) else mask
    land = mask.land_bits if isinstance(mask, WindowMask) else None
    emask = None
    d.mask_mode = _lib.MASK_NONE
    d.mask_windows = 0
    if isinstance(shift, ShiftMask):
        d.mask_mode = _lib.MASK_SHIFT
        d.frame_h, d.frame_w = shift.frame_h, shift.frame_w
        d.shift_h, d.shift_w = shift.shift_h, shift.shift_w
        d.win_row_begin, d.win_rows, d.win_cols = shift.win_row_begin, shift.win_rows, shift.win_cols
    elif isinstance(shift, torch.Tensor):
        _require_device(shift)
        n_geo = d.window_h * d.window_w
        if shift.dim() != 3 or tuple(shift.shape[1:]) != (n_geo, n_geo):
            raise ValueError(f"mask must be [nW, {n_geo}, {n_geo}], got {tuple(shift.shape)}")
        if num_windows % shift.shape[0] != 0:
            raise ValueError(f"attention batch {num_windows} must be divisible by mask windows {shift.shape[0]}")
        emask = shift.detach().to(torch.float32).contiguous()
        d.mask_mode = _lib.MASK_EXPLICIT
        d.mask_windows = shift.shape[0]
    elif shift is not None:
        raise TypeError(f"unsupported mask type {type(shift).__name__}")
    if land is not None:
        _require_device(land)
        if land.dtype != torch.int64 or land.dim() != 1:
            raise ValueError("land_bits must be a 1-D int64 tensor (one 64-bit key mask per window)")
        if emask is not None and land.shape[0] != emask.shape[0]:
            raise ValueError("land_bits and the explicit mask must cover the same number of windows")
        if num_windows % land.shape[0] != 0:
            raise ValueError(f"attention batch {num_windows} must be divisible by land windows {land.shape[0]}")
        land = land.contiguous()
        d.mask_windows = land.shape[0]
    return emask, land


def _bias_table(bias_table: Optional[torch.Tensor], d: _lib.SwinAttnDesc) -> Optional[torch.Tensor]:
    if bias_table is None:
        return None
    _require_device(bias_table)
    n_rel = (2 * d.window_h - 1) * (2 * d.window_w - 1)
    if tuple(bias_table.shape) != (n_rel, d.heads):
        raise ValueError(f"bias table must be [{n_rel}, {d.heads}], got {tuple(bias_table.shape)}")
    return bias_table.detach().to(torch.float32).contiguous()


def attention_backward_supported(q: torch.Tensor, num_heads: int, window_size: Tuple[int, int],
                                 n_real: Optional[int] = None) -> bool:
    """Whether :func:`window_attention_backward` serves this shape: the
    forward's (bf16 or fp32, windows up to 8x8 in at most 64 token rows,
    head dim 32, 64 or 128; or bf16 windows of a multiple of 128 tokens up to
    4096 without padded keys, head dim 64 or 128, the flash path, which also
    takes no bias and no mask)."""
    tokens, channels = q.shape[-2], q.shape[-1]
    wh, ww = (int(w) for w in window_size)
    if channels % num_heads != 0:
        return False
    if tokens > 64:
        return (q.dtype == torch.bfloat16 and tokens % 128 == 0 and tokens <= 4096 and wh * ww == tokens
                and (n_real is None or int(n_real) == tokens) and channels // num_heads in (64, 128))
    return (q.dtype in (torch.bfloat16, torch.float32) and 1 <= wh <= 8 and 1 <= ww <= 8
            and wh * ww <= tokens <= 64 and (n_real is None or 1 <= int(n_real) <= tokens)
            and channels // num_heads in (32, 64, 128))


def window_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor,
                              num_heads: int, window_size: Tuple[int, int], scale: float,
                              bias_table: Optional[torch.Tensor] = None,
                              mask: Union[None, torch.Tensor, ShiftMask, WindowMask] = None,
                              n_real: Optional[int] = None, mask_value: float = MASK_VALUE,
                              pad_key_value: float = PAD_KEY_VALUE,
                              dq: Optional[torch.Tensor] = None, dk: Optional[torch.Tensor] = None,
                              dv: Optional[torch.Tensor] = None, dbias: Optional[torch.Tensor] = None,
                              column_sums: Optional[torch.Tensor] = None):
    """Gradients of :func:`window_attention` (terra_swin_attn_bwd).

    Returns (dq, dk, dv); each may be given as an output view (e.g. a column
    block of one [B_, N, 3C] buffer).  ``dbias``: an fp32 tensor shaped like
    the bias table that the kernel ADDS the bias gradient into, or None.
    ``column_sums``: an fp32 [3C] tensor the column sums of dq | dk | dv (the
    q / k / v Linear's bias gradient) are ADDED into, or None
    (terra_swin_attn_bwd_sums; bf16 windows of at most 64 tokens only, see
    :func:`attention_backward_sums_supported`).
    """
    dev = _require_device(q, k, v, dout)
    for t in (k, v, dout):
        if t.dtype != q.dtype:
            raise TypeError("q, k, v and dout must share a dtype")
    code = _dtype_code(q, (torch.bfloat16, torch.float32))
    num_windows, tokens, channels = q.shape
    strides = tuple(_row_stride(t, n, num_windows, tokens, channels)
                    for t, n in ((q, "q"), (k, "k"), (v, "v"), (dout, "dout")))
    outs = []
    for t, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        if t is None:
            t = torch.empty((num_windows, tokens, channels), dtype=q.dtype, device=dev)
        elif t.dtype != q.dtype or t.device != dev:
            raise ValueError(f"{n} must be a {q.dtype} tensor on {dev}")
        outs.append(t)
    out_strides = tuple(_row_stride(t, n, num_windows, tokens, channels) for t, n in zip(outs, ("dq", "dk", "dv")))
    if num_windows == 0:  # no windows: empty gradients, nothing added to dbias
        return tuple(outs)
    bd = _lib.SwinAttnBwdDesc()
    bd.fwd = _attn_desc(q, num_heads, window_size, scale, n_real, mask_value, pad_key_value,
                        (strides[0], strides[1], strides[2], strides[3]))
    bd.dout_stride = strides[3]
    bd.dq_stride, bd.dk_stride, bd.dv_stride = out_strides
    table = _bias_table(bias_table, bd.fwd)
    if dbias is not None:
        if table is None:
            raise ValueError("dbias needs the bias table")
        if dbias.dtype != torch.float32 or tuple(dbias.shape) != tuple(table.shape) or not dbias.is_contiguous() \
                or dbias.device != dev:
            raise ValueError(f"dbias must be a contiguous fp32 tensor of shape {tuple(table.shape)} on {dev}")
    if column_sums is not None and (column_sums.dtype != torch.float32 or tuple(column_sums.shape) != (3 * channels,)
                                    or not column_sums.is_contiguous() or column_sums.device != dev):
        raise ValueError(f"column_sums must be a contiguous fp32 [{3 * channels}] tensor on {dev}")
    emask, land = _attn_masks(bd.fwd, num_windows, mask)
    with torch.cuda.device(dev):
        if column_sums is not None:
            base = _ptr(column_sums)
            step = channels * 4
            st = _lib.load().terra_swin_attn_bwd_sums(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(outs[0]),
                                                      _ptr(outs[1]), _ptr(outs[2]), code, ctypes.byref(bd),
                                                      _ptr(table), _ptr(dbias), _ptr(emask), _ptr(land), base,
                                                      base + step, base + 2 * step, _stream(dev))
        else:
            st = _lib.load().terra_swin_attn_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(outs[0]),
                                                 _ptr(outs[1]), _ptr(outs[2]), code, ctypes.byref(bd),
                                                 _ptr(table), _ptr(dbias), _ptr(emask), _ptr(land), _stream(dev))
    _lib.check(st, "terra_swin_attn_bwd_sums" if column_sums is not None else "terra_swin_attn_bwd")
    return tuple(outs)


def attention_backward_sums_supported(q: torch.Tensor, num_heads: int, window_size: Tuple[int, int],
                                      n_real: Optional[int] = None) -> bool:
    """Whether :func:`window_attention_backward` also sums dq | dk | dv
    (``column_sums``): bf16 windows of at most 64 tokens (the MFMA tile
    kernel)."""
    return (q.dtype == torch.bfloat16 and q.shape[-2] <= 64
            and attention_backward_supported(q, num_heads, window_size, n_real))


# (window, heads, channels) the fused half-block serves: 8x8 windows with 6
# or 12 heads of dim 32 or the reference model's 12 heads of dim 64, and 7x7
# windows with 4 heads of dim 32.
BLOCK_SHAPES = ((8, 6, 192), (8, 12, 384), (8, 12, 768), (7, 4, 128))


def swin_block_supported(x: torch.Tensor, geom: WindowGeometry, num_heads: int) -> bool:
    """Whether :func:`swin_block` serves this call (bf16 device tensor,
    (window, heads, channels) in BLOCK_SHAPES)."""
    return (x.device.type == "cuda" and x.dtype == torch.bfloat16
            and (geom.window, num_heads, geom.channels) in BLOCK_SHAPES)


def pack_linear(weight: torch.Tensor) -> torch.Tensor:
    """MFMA fragment order of a bf16 nn.Linear weight [out, in] (out % 16 == 0,
    in % 32 == 0) for :func:`swin_block` with ``packed_weights=True``; returns
    a flat tensor of the same number of elements."""
    dev = _require_device(weight)
    code = _dtype_code(weight, (torch.bfloat16,))
    if weight.dim() != 2 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous 2-D tensor")
    n, k = weight.shape
    out = torch.empty(n * k, dtype=weight.dtype, device=dev)
    with torch.cuda.device(dev):
        st = _lib.load().terra_swin_pack_linear(_ptr(weight), _ptr(out), code, int(n), int(k), _stream(dev))
    _lib.check(st, "terra_swin_pack_linear")
    return out


def swin_block(x: torch.Tensor, geom: WindowGeometry, num_heads: int, scale: float,
               qkv_weight: torch.Tensor, qkv_bias: Optional[torch.Tensor],
               proj_weight: torch.Tensor, proj_bias: Optional[torch.Tensor],
               ln_weight: Optional[torch.Tensor] = None, ln_bias: Optional[torch.Tensor] = None,
               ln_eps: float = 1e-5, layernorm: bool = True,
               bias_table: Optional[torch.Tensor] = None, shift_mask: bool = False,
               land_bits: Optional[torch.Tensor] = None, mask_value: float = MASK_VALUE,
               packed_weights: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused Swin attention half-block on ``x`` [B, H, W, C] (bf16):

        y = x + reverse(proj(attention(qkv(partition(LayerNorm(x))))))

    i.e. SequentialSwinTransformer.forward (models/transformer.py:142-300) with
    the attention of models/attention.py:236-283, in one kernel.  Float
    parameters (LayerNorm affine, biases, bias table) are passed as fp32;
    weights in the activation dtype.  ``shift_mask`` enables the analytic
    shift mask of the padded frame; ``land_bits`` ([emitted windows per
    image] int64) adds ``mask_value`` on land keys.  ``packed_weights``: the
    two weights come from :func:`pack_linear` (flat).  ``out`` may be ``x``.
    """
    if geom.batch == 0 and x.numel() == 0:  # an empty batch: nothing to launch
        _require_device(x)
        if out is None:
            return torch.empty_like(x)
        if out.shape != x.shape or out.dtype != x.dtype or out.device != x.device:
            raise ValueError("out must be a contiguous tensor like x")
        return out
    given = (qkv_weight, qkv_bias, proj_weight, proj_bias, ln_weight, ln_bias, bias_table, land_bits)
    key = ("block", tuple(map(id, given)), geom, num_heads, float(scale), float(ln_eps), bool(layernorm),
           bool(shift_mask), float(mask_value), bool(packed_weights), x.shape, x.dtype, x.device)
    return _prepared(key, given, lambda: _BlockLaunch(
        x, geom, num_heads, scale, qkv_weight, qkv_bias, proj_weight, proj_bias, ln_weight, ln_bias, ln_eps,
        layernorm, bias_table, shift_mask, land_bits, mask_value, packed_weights))(x, out)


# Prepared launches, keyed by the ids of the parameter tensors, the call's
# scalars and the activation shape.  An entry holds weak references to those
# tensors with their data pointers and sizes, and serves a call only while
# each reference still names the tensor passed and its data pointer and size
# are unchanged (so a reused id, a rebound ``.data`` or an in-place resize
# builds a new entry).  Entries are
# made only when the kernel reads the caller's tensors themselves (no
# conversion copies), so in-place updates of them are seen by later calls,
# and an entry keeps no tensor memory alive.
_LAUNCHES: "OrderedDict" = OrderedDict()
_LAUNCHES_MAX = 256


def _prepared(key, given, build) -> "_Launch":
    launch = _LAUNCHES.get(key)
    if launch is None or not launch.serves(given):
        launch = build()
        if launch.keep is None:  # the kernel reads the caller's tensors as they are
            launch.watch(given)
            _LAUNCHES[key] = launch
            if len(_LAUNCHES) > _LAUNCHES_MAX:
                _LAUNCHES.popitem(last=False)
    return launch


class _Launch:
    """A validated library call for one activation shape, dtype and device:
    descriptor and parameter pointers built once; each call checks only x
    and out.  Subclasses set desc, ptrs, fn, name, shape, dtype, device,
    code and keep (the converted copies the pointers name, or None)."""

    refs = ()
    keep = None

    def watch(self, given) -> None:
        self.refs = tuple((None, 0, 0) if t is None else (weakref.ref(t), t.data_ptr(), t.numel()) for t in given)

    def serves(self, given) -> bool:
        for (ref, ptr, n), t in zip(self.refs, given):
            if t is None:
                if ref is not None:
                    return False
            elif ref is None or ref() is not t or t.data_ptr() != ptr or t.numel() != n:
                return False
        return True

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
        if x.shape != self.shape or x.dtype != self.dtype or x.device != self.device or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous {self.dtype} tensor of shape {tuple(self.shape)} on "
                             f"{self.device}")
        if out is None:
            out = torch.empty_like(x)
        elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous() or out.device != self.device:
            raise ValueError("out must be a contiguous tensor like x")
        dev = self.device
        args = (x.data_ptr(), out.data_ptr(), self.code, ctypes.byref(self.desc)) + self.ptrs
        if dev.index is not None and dev.index != torch.cuda.current_device():
            with torch.cuda.device(dev):
                st = self.fn(*args, _stream(dev))
        else:
            st = self.fn(*args, _stream(dev))
        _lib.check(st, self.name)
        return out


class _BlockLaunch(_Launch):
    """terra_swin_block_fwd with its checks (see :func:`swin_block`)."""

    def __init__(self, x, geom, num_heads, scale, qkv_weight, qkv_bias, proj_weight, proj_bias, ln_weight, ln_bias,
                 ln_eps, layernorm, bias_table, shift_mask, land_bits, mask_value, packed_weights):
        dev = _require_device(x, qkv_weight, proj_weight)
        code = _dtype_code(x, (torch.bfloat16,))
        C = geom.channels
        if tuple(x.shape) != (geom.batch, geom.height, geom.width, C) or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous [{geom.batch}, {geom.height}, {geom.width}, {C}] tensor")
        for name, t, shape in (("qkv_weight", qkv_weight, (3 * C, C)), ("proj_weight", proj_weight, (C, C))):
            ok_shape = t.numel() == shape[0] * shape[1] if packed_weights else tuple(t.shape) == shape
            if not ok_shape or t.dtype != x.dtype or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous {x.dtype} tensor of shape {shape}"
                                 + (" (packed)" if packed_weights else ""))
        copies = []

        def f32(t, n, name):
            if t is None:
                return None
            _require_device(x, t)
            if t.numel() != n:
                raise ValueError(f"{name} must have {n} elements")
            r = t.detach().reshape(-1).to(torch.float32).contiguous()
            if r.data_ptr() != t.data_ptr():
                copies.append(r)
            return r

        params = (f32(ln_weight, C, "ln_weight") if layernorm else None,
                  f32(ln_bias, C, "ln_bias") if layernorm else None,
                  f32(qkv_bias, 3 * C, "qkv_bias"), f32(proj_bias, C, "proj_bias"))
        table = None
        if bias_table is not None:
            _require_device(x, bias_table)
            n_rel = (2 * geom.window - 1) ** 2
            if tuple(bias_table.shape) != (n_rel, num_heads):
                raise ValueError(f"bias table must be [{n_rel}, {num_heads}], got {tuple(bias_table.shape)}")
            table = bias_table.detach().to(torch.float32).contiguous()
            if table.data_ptr() != bias_table.data_ptr():
                copies.append(table)
        d = _lib.SwinBlockDesc()
        d.geom = geom.to_c()
        d.heads, d.scale, d.ln_eps, d.mask_value = num_heads, float(scale), float(ln_eps), float(mask_value)
        d.layernorm, d.shift_mask = int(bool(layernorm)), int(bool(shift_mask))
        d.land_windows = 0
        d.packed_weights = int(bool(packed_weights))
        if land_bits is not None:
            _require_device(x, land_bits)
            if land_bits.dtype != torch.int64 or land_bits.dim() != 1:
                raise ValueError("land_bits must be a 1-D int64 tensor (one 64-bit key mask per window)")
            n_land = land_bits.shape[0]
            if n_land == 0 or geom.num_windows % n_land != 0 or n_land % geom.windows_per_image != 0:
                raise ValueError(f"land_bits must hold the emitted windows of one image ({geom.windows_per_image}) "
                                 f"or of several whole images dividing the batch (got {n_land} for "
                                 f"{geom.num_windows} windows)")
            if not land_bits.is_contiguous():
                land_bits = land_bits.contiguous()
                copies.append(land_bits)
            d.land_windows = n_land
        self.desc = d
        self.shape, self.dtype, self.device, self.code = x.shape, x.dtype, dev, code
        self.keep = tuple(copies) or None  # converted copies live as long as this (uncached) launch
        self.ptrs = (_ptr(params[0]), _ptr(params[1]), _ptr(qkv_weight), _ptr(params[2]), _ptr(proj_weight),
                     _ptr(params[3]), _ptr(table), _ptr(land_bits))
        self.fn, self.name = _lib.load().terra_swin_block_fwd, "terra_swin_block_fwd"


MLP_CHANNELS = (128, 192, 384, 768)


LINEAR_OUT_MULTIPLE = 256  # output features per tile of the linear kernels
LINEAR_MAX_OUT = 4096      # output features the linear kernels stage their bias for


def linear_supported(x: torch.Tensor, in_features: int, out_features: int) -> bool:
    """Whether :func:`linear` / :func:`linear_residual` serve this layer: bf16
    device rows, in_features a multiple of 64, out_features a multiple of 256
    up to 4096."""
    return (x.device.type == "cuda" and x.dtype == torch.bfloat16 and in_features > 0 and in_features % 64 == 0
            and 0 < out_features <= LINEAR_MAX_OUT and out_features % LINEAR_OUT_MULTIPLE == 0)


def _linear_checks(x: torch.Tensor, weight_packed: torch.Tensor, out_features: int, bias: Optional[torch.Tensor]):
    dev = _require_device(x, weight_packed)
    code = _dtype_code(x, (torch.bfloat16,))
    if x.dim() < 1 or not x.is_contiguous():
        raise ValueError("x must be a contiguous [..., in_features] tensor")
    k = x.shape[-1]
    if not linear_supported(x, k, out_features):
        raise ValueError(f"the linear kernels serve bf16 rows with in_features % 64 == 0 and out_features % 256 == 0, <= 4096 "
                         f"(got {x.dtype}, {k} -> {out_features})")
    if weight_packed.dtype != x.dtype or weight_packed.numel() != out_features * k or not weight_packed.is_contiguous():
        raise ValueError(f"weight_packed must be a contiguous packed {x.dtype} tensor of {out_features * k} elements "
                         "(pack_linear of the [out, in] weight)")
    if bias is not None:
        _require_device(x, bias)
        if bias.dtype != torch.float32 or bias.numel() != out_features or not bias.is_contiguous():
            raise ValueError(f"bias must be a contiguous fp32 tensor of {out_features} elements")
    return dev, code, k, x.numel() // k if k else 0


def linear(x: torch.Tensor, weight_packed: torch.Tensor, out_features: int, bias: Optional[torch.Tensor] = None,
           gelu: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``bf16(x W^T + b)`` over the token rows of ``x`` [..., in] (bf16), or
    with ``gelu`` ``GELU(bf16(x W^T + b))`` (nn.GELU, erf form, rounded to
    bf16): fc1 + act of SequentialMlp (models/mlp.py:162-165) in one kernel.
    ``weight_packed`` is :func:`pack_linear` of the [out, in] weight, ``bias``
    fp32 or None."""
    dev, code, k, rows = _linear_checks(x, weight_packed, out_features, bias)
    shape = (*x.shape[:-1], out_features)
    if out is None:
        out = torch.empty(shape, dtype=x.dtype, device=dev)
    elif tuple(out.shape) != shape or out.dtype != x.dtype or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {x.dtype} tensor of shape {shape} on {dev}")
    if rows == 0:
        return out
    with torch.cuda.device(dev):
        st = _lib.load().terra_swin_linear(_ptr(x), _ptr(out), code, int(rows), int(k), int(out_features), int(k),
                                           int(out_features), _ptr(weight_packed), _ptr(bias), 1 if gelu else 0,
                                           _stream(dev))
    _lib.check(st, "terra_swin_linear")
    return out


def linear_residual(x: torch.Tensor, weight_packed: torch.Tensor, out_features: int, residual: torch.Tensor,
                    bias: Optional[torch.Tensor] = None, geom: Optional[WindowGeometry] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``residual + bf16(x W^T + b)`` rounded to bf16.

    Without ``geom``: per token row (fc2 + shortcut, models/mlp.py:168-171);
    ``residual`` / ``out`` have ``x``'s rows.  With ``geom`` (8x8 windows,
    every frame window emitted): ``x`` holds the window tokens [B*nW, 64, in]
    and each row goes back to the grid token it was partitioned from, i.e.
    proj + window_reverse + roll + shortcut (models/attention.py:281,
    models/utils.py:41-45, models/transformer.py:246, 296-298); ``residual`` /
    ``out`` are [B, H, W, C].  ``out`` may be ``residual``."""
    dev, code, k, rows = _linear_checks(x, weight_packed, out_features, bias)
    _require_device(x, residual)
    if geom is None:
        shape = (*x.shape[:-1], out_features)
    else:
        if geom.channels != out_features:
            raise ValueError(f"geom.channels ({geom.channels}) must equal out_features ({out_features})")
        shape = (geom.batch, geom.height, geom.width, geom.channels)
    n_out = 1
    for d in shape:
        n_out *= d
    if residual.dtype != x.dtype or residual.numel() != n_out or not residual.is_contiguous():
        raise ValueError(f"residual must be a contiguous {x.dtype} tensor of {n_out} elements")
    if out is None:
        out = torch.empty(shape, dtype=x.dtype, device=dev)
    elif out.numel() != n_out or out.dtype != x.dtype or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {x.dtype} tensor of {n_out} elements on {dev}")
    if rows == 0:
        return out.view(shape)
    c_geom = None if geom is None else geom.to_c()
    with torch.cuda.device(dev):
        st = _lib.load().terra_swin_linear_residual(_ptr(x), _ptr(residual), _ptr(out), code, int(rows), int(k),
                                                    int(out_features), _ptr(weight_packed), _ptr(bias),
                                                    None if c_geom is None else ctypes.byref(c_geom), _stream(dev))
    _lib.check(st, "terra_swin_linear_residual")
    return out.view(shape)


def gelu_backward_supported(h: torch.Tensor) -> bool:
    """Whether :func:`gelu_backward` serves a pre-activation like ``h``
    (a bf16 or fp32 device tensor whose rows are whole 16-byte chunks of at
    most 8192 bytes)."""
    if h.device.type != "cuda" or h.dtype not in (torch.bfloat16, torch.float32) or h.dim() == 0:
        return False
    row_bytes = h.shape[-1] * h.element_size()
    return row_bytes % 16 == 0 and 0 < row_bytes <= 8192


def gelu_backward(dout: torch.Tensor, h: torch.Tensor, column_sums: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The gradient of nn.GELU() (erf form, models/mlp.py:165) at ``h`` for
    the output gradient ``dout`` (same shape and dtype, bf16 or fp32):
    ``dout * (Phi(h) + h phi(h))`` in fp32, rounded once; what
    ``torch.ops.aten.gelu_backward(dout, h)`` computes.  ``column_sums``: an
    fp32 [features] tensor the per-feature sums of the result are ADDED into
    (the bias gradient of the Linear that produced ``h``)."""
    dev = _require_device(dout, h)
    code = _dtype_code(h, (torch.float32, torch.bfloat16))
    if dout.shape != h.shape or dout.dtype != h.dtype:
        raise ValueError(f"dout {tuple(dout.shape)} {dout.dtype} must match h {tuple(h.shape)} {h.dtype}")
    if not (dout.is_contiguous() and h.is_contiguous()):
        raise ValueError("dout and h must be contiguous")
    features = h.shape[-1] if h.dim() > 0 else 1
    rows = h.numel() // features if features else 0
    if column_sums is not None and (column_sums.dtype != torch.float32 or tuple(column_sums.shape) != (features,)
                                    or not column_sums.is_contiguous() or column_sums.device != dev):
        raise ValueError(f"column_sums must be a contiguous fp32 [{features}] tensor on {dev}")
    if out is None:
        out = torch.empty_like(h)
    elif out.shape != h.shape or out.dtype != h.dtype or not out.is_contiguous() or out.device != dev:
        raise ValueError(f"out must be a contiguous {h.dtype} tensor like h on {dev}")
    if rows == 0:
        return out
    with torch.cuda.device(dev):
        st = _lib.load().terra_swin_gelu_bwd(_ptr(dout), _ptr(h), _ptr(out), code, int(rows), int(features),
                                             _ptr(column_sums), _stream(dev))
    _lib.check(st, "terra_swin_gelu_bwd")
    return out


def swin_mlp_supported(x: torch.Tensor, channels: int, hidden: int) -> bool:
    """Whether :func:`swin_mlp` serves this call (bf16 device tensor,
    C in {128, 192, 384, 768}: the widths of the benchmark configurations,
    hidden = 4 C)."""
    return (x.device.type == "cuda" and x.dtype == torch.bfloat16 and channels in MLP_CHANNELS
            and hidden == 4 * channels)


def swin_mlp(x: torch.Tensor, fc1_weight: torch.Tensor, fc1_bias: Optional[torch.Tensor],
             fc2_weight: torch.Tensor, fc2_bias: Optional[torch.Tensor],
             ln_weight: Optional[torch.Tensor] = None, ln_bias: Optional[torch.Tensor] = None,
             ln_eps: float = 1e-5, layernorm: bool = True, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused MLP half-block over the token rows of ``x`` [..., C] (bf16):

        y = x + fc2(GELU(fc1(LayerNorm(x))))

    i.e. SequentialMlp.forward (models/mlp.py:152-172) in one kernel.
    ``fc1_weight`` / ``fc2_weight`` come from :func:`pack_linear` (flat, bf16)
    of the nn.Linear weights [4C, C] / [C, 4C]; biases and the LayerNorm
    affine are passed as fp32 (or None).  ``out`` may be ``x``.
    """
    given = (fc1_weight, fc1_bias, fc2_weight, fc2_bias, ln_weight, ln_bias)
    key = ("mlp", tuple(map(id, given)), float(ln_eps), bool(layernorm), x.shape, x.dtype, x.device)
    launch = _prepared(key, given, lambda: _MlpLaunch(x, fc1_weight, fc1_bias, fc2_weight, fc2_bias, ln_weight,
                                                      ln_bias, ln_eps, layernorm))
    if launch.desc is None:  # no tokens
        return x.clone() if out is None else out
    return launch(x, out)


class _MlpLaunch(_Launch):
    """terra_swin_mlp_fwd with its checks (see :func:`swin_mlp`)."""

    def __init__(self, x, fc1_weight, fc1_bias, fc2_weight, fc2_bias, ln_weight, ln_bias, ln_eps, layernorm):
        dev = _require_device(x, fc1_weight, fc2_weight)
        code = _dtype_code(x, (torch.bfloat16,))
        if not x.is_contiguous() or x.dim() < 1:
            raise ValueError("x must be a contiguous [..., C] tensor")
        C = x.shape[-1]
        H = fc1_weight.numel() // C if C else 0
        if not swin_mlp_supported(x, C, H):
            raise ValueError(f"the fused MLP serves bf16 rows of C in {MLP_CHANNELS} with hidden 4C "
                             f"(got {x.dtype}, C {C}, hidden {H})")
        self.shape, self.dtype, self.device, self.code = x.shape, x.dtype, dev, code
        tokens = x.numel() // C
        self.desc = None
        if tokens == 0:
            return
        for name, t, n in (("fc1_weight", fc1_weight, H * C), ("fc2_weight", fc2_weight, C * H)):
            if t.numel() != n or t.dtype != x.dtype or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous packed {x.dtype} tensor of {n} elements")
        copies = []

        def f32(t, n, name):
            if t is None:
                return None
            _require_device(x, t)
            if t.numel() != n:
                raise ValueError(f"{name} must have {n} elements")
            r = t.detach().reshape(-1).to(torch.float32).contiguous()
            if r.data_ptr() != t.data_ptr():
                copies.append(r)
            return r

        params = (f32(ln_weight, C, "ln_weight") if layernorm else None,
                  f32(ln_bias, C, "ln_bias") if layernorm else None,
                  f32(fc1_bias, H, "fc1_bias"), f32(fc2_bias, C, "fc2_bias"))
        d = _lib.SwinMlpDesc()
        d.tokens, d.channels, d.hidden = int(tokens), int(C), int(H)
        d.layernorm, d.ln_eps = int(bool(layernorm)), float(ln_eps)
        self.desc = d
        self.keep = tuple(copies) or None
        self.ptrs = (_ptr(params[0]), _ptr(params[1]), _ptr(fc1_weight), _ptr(params[2]), _ptr(fc2_weight),
                     _ptr(params[3]))
        self.fn, self.name = _lib.load().terra_swin_mlp_fwd, "terra_swin_mlp_fwd"
