"""Autograd for the hot path: the training step's backward through the HIP
kernels (the reference trains through ATen autograd of the same ops,
core/runtime/run_model.py:362-617 over models/attention.py:231-283 and
models/transformer.py:142-300).

- Partition and reverse are adjoint token permutations: every emitted,
  non-pad window token is gathered from exactly one grid token, and reverse
  scatters it back to that token.  So the gradient of partition is reverse
  (grid tokens no window reads get zero) and the gradient of reverse is
  partition (pad window tokens get zero), both on the same geometry.
- The attention core's backward is ``terra_swin_attn_bwd`` (P recomputed
  from q and k; dq, dk, dv, and the bias-table gradient summed over
  windows): an MFMA tile kernel for every bf16 window (8x8, 7x7, padded
  keys), a plain fp32 kernel for fp32 activations.  For a shape neither serves the forward still runs
  and backward() raises NotImplementedError (there is no non-HIP backward).

Each function runs the plain kernel when no input needs a gradient.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from . import kernels
from .kernels import ShiftMask, WindowGeometry, WindowMask

MaskArg = Union[None, torch.Tensor, ShiftMask, WindowMask]


def _needs_grad(*tensors: Optional[torch.Tensor]) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


class _Partition(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: torch.Tensor, geom: WindowGeometry) -> torch.Tensor:
        ctx.geom = geom
        return kernels.swin_partition(x, geom)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        return kernels.swin_reverse(grad.contiguous(), ctx.geom), None


class _Reverse(torch.autograd.Function):
    @staticmethod
    def forward(ctx, windows: torch.Tensor, geom: WindowGeometry,
                residual: Optional[torch.Tensor]) -> torch.Tensor:
        ctx.geom = geom
        ctx.has_residual = residual is not None
        return kernels.swin_reverse(windows, geom, residual=residual)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        grad = grad.contiguous()
        shape = (ctx.geom.batch, ctx.geom.height, ctx.geom.width, ctx.geom.channels)
        d_windows = kernels.swin_partition(grad.view(shape), ctx.geom)
        return d_windows, None, (grad if ctx.has_residual else None)


def partition(x: torch.Tensor, geom: WindowGeometry) -> torch.Tensor:
    """:func:`kernels.swin_partition` with a gradient (reverse)."""
    if _needs_grad(x):
        return _Partition.apply(x, geom)
    return kernels.swin_partition(x, geom)


def reverse(windows: torch.Tensor, geom: WindowGeometry, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """:func:`kernels.swin_reverse` with gradients (partition for the windows,
    identity for the residual)."""
    if _needs_grad(windows, residual):
        return _Reverse.apply(windows, geom, residual)
    return kernels.swin_reverse(windows, geom, residual=residual)


def _check_backward(q: torch.Tensor, num_heads: int, window_size: Tuple[int, int], n_real: Optional[int]) -> None:
    if not kernels.attention_backward_supported(q, num_heads, window_size, n_real):
        raise NotImplementedError(
            "terra_amd: the attention backward kernels are built for bf16 / fp32 activations, windows up to 8x8 "
            f"in at most 64 token rows and head dim 32, 64 or 128 (got {q.dtype}, window {tuple(window_size)}, "
            f"{q.shape[-2]} tokens, n_real {n_real}, head dim {q.shape[-1] // num_heads})")


class _Attention(torch.autograd.Function):
    """q, k, v as separate inputs (any row strides)."""

    @staticmethod
    def forward(ctx, q, k, v, table, num_heads, window_size, scale, mask, n_real, mask_value):
        ctx.cfg = (num_heads, window_size, scale, mask, n_real, mask_value)
        ctx.save_for_backward(q, k, v, table)
        return kernels.window_attention(q, k, v, num_heads, window_size, scale, bias_table=table, mask=mask,
                                        n_real=n_real, mask_value=mask_value)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        q, k, v, table = ctx.saved_tensors
        num_heads, window_size, scale, mask, n_real, mask_value = ctx.cfg
        _check_backward(q, num_heads, window_size, n_real)
        dbias = None
        if table is not None and ctx.needs_input_grad[3]:
            dbias = torch.zeros(table.shape, dtype=torch.float32, device=table.device)
        dq, dk, dv = kernels.window_attention_backward(q, k, v, grad.contiguous(), num_heads, window_size, scale,
                                                       bias_table=table, mask=mask, n_real=n_real,
                                                       mask_value=mask_value, dbias=dbias)
        dtable = None if dbias is None else dbias.to(table.dtype)
        return dq, dk, dv, dtable, None, None, None, None, None, None


class _AttentionQKV(torch.autograd.Function):
    """One [B_, N, 3C] projection output as input: the gradients of q, k and v
    are written into one [B_, N, 3C] buffer (the input of the projection's
    backward GEMM), with no slice copies."""

    @staticmethod
    def forward(ctx, qkv, table, num_heads, window_size, scale, mask, n_real, mask_value):
        C = qkv.shape[-1] // 3
        ctx.cfg = (num_heads, window_size, scale, mask, n_real, mask_value)
        ctx.save_for_backward(qkv, table)
        return kernels.window_attention(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], num_heads, window_size,
                                        scale, bias_table=table, mask=mask, n_real=n_real, mask_value=mask_value)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        qkv, table = ctx.saved_tensors
        num_heads, window_size, scale, mask, n_real, mask_value = ctx.cfg
        C = qkv.shape[-1] // 3
        _check_backward(qkv[..., :C], num_heads, window_size, n_real)
        dqkv = torch.empty(qkv.shape, dtype=qkv.dtype, device=qkv.device)
        dbias = None
        if table is not None and ctx.needs_input_grad[1]:
            dbias = torch.zeros(table.shape, dtype=torch.float32, device=table.device)
        kernels.window_attention_backward(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], grad.contiguous(),
                                          num_heads, window_size, scale, bias_table=table, mask=mask, n_real=n_real,
                                          mask_value=mask_value, dq=dqkv[..., :C], dk=dqkv[..., C:2 * C],
                                          dv=dqkv[..., 2 * C:], dbias=dbias)
        dtable = None if dbias is None else dbias.to(table.dtype)
        return dqkv, dtable, None, None, None, None, None, None


def window_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                     window_size: Tuple[int, int], scale: float, bias_table: Optional[torch.Tensor] = None,
                     mask: MaskArg = None, n_real: Optional[int] = None,
                     mask_value: float = kernels.MASK_VALUE) -> torch.Tensor:
    """:func:`kernels.window_attention` with gradients for q, k, v and the bias
    table."""
    if _needs_grad(q, k, v, bias_table):
        return _Attention.apply(q, k, v, bias_table, num_heads, tuple(window_size), scale, mask, n_real, mask_value)
    return kernels.window_attention(q, k, v, num_heads, window_size, scale, bias_table=bias_table, mask=mask,
                                    n_real=n_real, mask_value=mask_value)


def window_attention_qkv(qkv: torch.Tensor, num_heads: int, window_size: Tuple[int, int], scale: float,
                         bias_table: Optional[torch.Tensor] = None, mask: MaskArg = None,
                         n_real: Optional[int] = None, mask_value: float = kernels.MASK_VALUE) -> torch.Tensor:
    """Attention over the column blocks q | k | v of one [B_, N, 3C] tensor,
    with gradients (see :class:`_AttentionQKV`)."""
    C = qkv.shape[-1] // 3
    if _needs_grad(qkv, bias_table):
        if not qkv.is_contiguous():
            qkv = qkv.contiguous()
        return _AttentionQKV.apply(qkv, bias_table, num_heads, tuple(window_size), scale, mask, n_real, mask_value)
    return kernels.window_attention(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], num_heads, window_size,
                                    scale, bias_table=bias_table, mask=mask, n_real=n_real, mask_value=mask_value)
