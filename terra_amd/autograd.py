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


class ResidualLink:
    """Hands a half-block's output gradient (the residual's gradient) from the
    scatter's backward to the gather's backward, which adds it into dx in the
    same kernel instead of autograd summing the two paths in a separate pass.
    The scatter then takes its residual detached; the gather's backward runs
    after the scatter's, since the gather's output feeds the scatter."""

    def __init__(self):
        self.grad: Optional[torch.Tensor] = None


class ColumnSumLink:
    """Hands the column sums of a Linear's output gradient (its bias gradient)
    from the backward that produces that gradient, which sums it in the same
    kernel, to the Linear's backward, which then skips its own reduction."""

    def __init__(self):
        self.sums: Optional[torch.Tensor] = None


class _Reverse(torch.autograd.Function):
    """Window reverse + roll + residual.  With bf16 windows and an fp32
    output (autocast's bf16 proj output added to an fp32 shortcut) the kernel
    widens the windows itself, and the backward writes the windows' gradient
    in bf16 (what the cast's backward gives), with the column sums a
    :class:`ColumnSumLink` hands to the producing Linear's bias gradient."""

    @staticmethod
    def forward(ctx, windows: torch.Tensor, geom: WindowGeometry, residual: Optional[torch.Tensor],
                link: Optional[ResidualLink], out_dtype: Optional[torch.dtype],
                bias_sums: Optional[ColumnSumLink]) -> torch.Tensor:
        ctx.geom = geom
        ctx.has_residual = residual is not None
        ctx.link, ctx.bias_sums = link, bias_sums
        ctx.win_dtype = windows.dtype
        return kernels.swin_reverse(windows, geom, residual=residual, out_dtype=out_dtype)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        grad = grad.contiguous()
        shape = (ctx.geom.batch, ctx.geom.height, ctx.geom.width, ctx.geom.channels)
        if ctx.win_dtype != grad.dtype:  # bf16 windows, fp32 output
            sums = None
            if ctx.bias_sums is not None:
                sums = torch.zeros(ctx.geom.channels, dtype=torch.float32, device=grad.device)
                ctx.bias_sums.sums = sums
            d_windows = kernels.swin_partition(grad.view(shape), ctx.geom, out_dtype=ctx.win_dtype, column_sums=sums)
        else:
            d_windows = kernels.swin_partition(grad.view(shape), ctx.geom)
        if ctx.link is not None:
            ctx.link.grad = grad.view(shape)
            return d_windows, None, None, None, None, None
        return d_windows, None, (grad if ctx.has_residual else None), None, None, None


class _PartitionLN(torch.autograd.Function):
    """LayerNorm over C + pad + roll + partition (terra_swin_partition_ln),
    backward by terra_swin_partition_ln_bwd: dx, and the weight / bias
    gradients summed over the tokens.  With out_dtype bf16 for fp32 x the
    windows are the fp32 output rounded once to bf16 and their gradient
    arrives in bf16 (the _mixed entry points)."""

    @staticmethod
    def forward(ctx, x, weight, bias, geom, eps, out_dtype, link):
        ctx.geom, ctx.eps, ctx.link = geom, eps, link
        ctx.save_for_backward(x, weight, bias)
        return kernels.swin_partition_ln(x, geom, weight, bias, eps, out_dtype=out_dtype)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        x, weight, bias = ctx.saved_tensors
        dw = db = None
        if weight is not None and ctx.needs_input_grad[1]:
            dw = torch.zeros(weight.shape, dtype=torch.float32, device=x.device)
        if bias is not None and ctx.needs_input_grad[2]:
            db = torch.zeros(bias.shape, dtype=torch.float32, device=x.device)
        dres = None
        if ctx.link is not None and ctx.link.grad is not None:  # the residual's gradient, added in the kernel
            dres, ctx.link.grad = ctx.link.grad.to(x.dtype).contiguous(), None
        dx = kernels.swin_partition_ln_backward(grad.contiguous(), x, ctx.geom, weight, ctx.eps, dresidual=dres,
                                                dweight=dw, dbias=db)
        return (dx, None if dw is None else dw.to(weight.dtype), None if db is None else db.to(bias.dtype), None, None,
                None, None)


def linear_input_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype F.linear computes in for an input like x: bf16 inside a bf16
    autocast region (which casts its fp32 input to bf16), else x's own."""
    return torch.bfloat16 if kernels.autocast_bf16(x) and x.dtype == torch.float32 else x.dtype


def partition_ln(x: torch.Tensor, geom: WindowGeometry, weight: Optional[torch.Tensor],
                 bias: Optional[torch.Tensor], eps: float, out_dtype: Optional[torch.dtype] = None,
                 link: Optional[ResidualLink] = None) -> torch.Tensor:
    """:func:`kernels.swin_partition_ln` with gradients for x and the
    LayerNorm affine parameters.  ``out_dtype`` bf16 for fp32 x writes the
    bf16 copy a following Linear under bf16 autocast would cast to (and takes
    its bf16 gradient), instead of fp32 windows and a cast each way.
    ``link``: the :class:`ResidualLink` of a :func:`reverse` whose residual
    is x; its gradient is then added into dx by this backward's kernel."""
    if _needs_grad(x, weight, bias):
        return _PartitionLN.apply(x, weight, bias, geom, eps, out_dtype, link)
    return kernels.swin_partition_ln(x, geom, weight, bias, eps, out_dtype=out_dtype)


def weight_grad(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """dy^T x for dy [T, out] and x [T, in] (a Linear's weight gradient, the
    contraction over all T tokens), in fp32.  For large T the tokens are
    split into k slices contracted as one batched GEMM with an fp32 output and
    then summed: hipBLASLt takes no split-K tiles for a contraction this long
    and runs the plain product 3.5-7.7x slower (c3: 524288 tokens, 1.0-1.6 ms
    against 0.10-0.25 ms per weight gradient).  Slices of at least 2048
    tokens, at most 128 of them: at c3, 128 slices of 4096 measured 97-250 us
    per weight gradient against 115-350 us with 64 and 241-266 us with 256."""
    T, o = dy.shape
    i = x.shape[1]
    k = next((k for k in (128, 64, 32, 16, 8) if T % k == 0 and T // k >= 2048), 1)
    if k == 1 or dy.dtype not in (torch.bfloat16, torch.float16):
        return (dy.t() @ x).float()
    # The transposed view is the left operand; the right one is contiguous.
    return torch.bmm(dy.view(k, T // k, o).transpose(1, 2), x.reshape(k, T // k, i).contiguous(),
                     out_dtype=torch.float32).sum(0)


class _Linear(torch.autograd.Function):
    """F.linear for training, in the dtype bf16 autocast gives it (x, weight
    and bias cast to bf16 inside an autocast region, as F.linear's autocast
    rule does), with the weight gradient from :func:`weight_grad`.  The bias
    gradient comes from a :class:`ColumnSumLink` when the output gradient's
    producer summed it (in the order of its own kernel), else from a sum."""

    @staticmethod
    def forward(ctx, x, weight, bias, bias_sums):
        dt = torch.bfloat16 if (torch.is_autocast_enabled(x.device.type)
                                and torch.get_autocast_dtype(x.device.type) == torch.bfloat16) else x.dtype
        xc, wc = x.to(dt), weight.to(dt)
        bc = None if bias is None else bias.to(dt)
        ctx.save_for_backward(xc, wc)
        ctx.dtypes = (x.dtype, weight.dtype, None if bias is None else bias.dtype)
        ctx.bias_sums = bias_sums
        return torch.nn.functional.linear(xc, wc, bc)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        xc, wc = ctx.saved_tensors
        xd, wd, bd = ctx.dtypes
        dy2 = dy.reshape(-1, dy.shape[-1]).to(wc.dtype)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = (dy2 @ wc).view(xc.shape).to(xd)
        if ctx.needs_input_grad[1]:
            dw = weight_grad(dy2, xc.reshape(-1, xc.shape[-1])).to(wd)
        sums = None
        if ctx.bias_sums is not None:
            sums, ctx.bias_sums.sums = ctx.bias_sums.sums, None
        if bd is not None and ctx.needs_input_grad[2]:
            db = (sums if sums is not None and dy.dtype == wc.dtype else dy2.sum(0, dtype=torch.float32)).to(bd)
        return dx, dw, db, None


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
           bias_sums: Optional[ColumnSumLink] = None) -> torch.Tensor:
    """F.linear, through :class:`_Linear` when a gradient is needed.
    ``bias_sums``: a :class:`ColumnSumLink` the backward of the output's
    consumer fills with the output gradient's column sums."""
    if _needs_grad(x, weight, bias):
        return _Linear.apply(x, weight, bias, bias_sums)
    return torch.nn.functional.linear(x, weight, bias)


class _Mlp(torch.autograd.Function):
    """SequentialMlp.forward (models/mlp.py:152-172) for training:
    y = x + fc2(GELU(fc1(LayerNorm(x)))).  The LayerNorm forward and its
    backward (with the residual gradient added in the same kernel) run on
    terra_swin_partition_ln / _bwd over the token rows; the four GEMMs of
    the backward on hipBLASLt through torch, in the dtypes autocast gave the
    forward's GEMMs.  The GELU derivative (the exact, erf one) runs on
    terra_swin_gelu_bwd with fc1's bias gradient summed in the same pass;
    under autocast the output gradient's cast to bf16 sums fc2's bias
    gradient in its pass (terra_swin_partition_mixed over the token rows)."""

    @staticmethod
    def forward(ctx, x, ln_w, ln_b, w1, b1, w2, b2, eps):
        C = x.shape[-1]
        rows = x.reshape(-1, C).contiguous()
        geom = kernels.rows_geometry(rows.shape[0], C)
        # Under bf16 autocast fc1 takes a bf16 copy of the fp32 LayerNorm
        # output: the kernel writes that copy directly.
        xn = kernels.swin_partition_ln(rows.view(1, -1, 1, C), geom, ln_w, ln_b, eps,
                                       out_dtype=linear_input_dtype(rows)).view(-1, C)
        h1 = torch.nn.functional.linear(xn, w1, b1)
        a = torch.nn.functional.gelu(h1)
        h2 = torch.nn.functional.linear(a, w2, b2)
        if h2.dtype == torch.bfloat16 and rows.dtype == torch.float32 and C % 4 == 0 and h2.shape[-1] == C:
            # x + fc2(...) under autocast: the bf16 h2 widened and added to the
            # fp32 rows in one pass (the mixed scatter over an identity frame;
            # bit for bit torch's promoted add).
            y = kernels.swin_reverse(h2.contiguous(), geom, residual=rows.view(1, -1, 1, C),
                                     out_dtype=torch.float32).view(rows.shape)
        else:
            y = rows + h2
        ctx.eps, ctx.geom, ctx.shape = eps, geom, x.shape
        ctx.autocast = torch.is_autocast_enabled(x.device.type)
        ctx.save_for_backward(rows, ln_w, ln_b, xn, h1, a, w1, w2)
        return y.view(x.shape[:-1] + (y.shape[-1],))

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        rows, ln_w, ln_b, xn, h1, a, w1, w2 = ctx.saved_tensors
        C = rows.shape[-1]
        dy = dy.reshape(-1, dy.shape[-1])
        gemm_dtype = h1.dtype  # the forward GEMMs' dtype (bf16 under autocast)
        T, c_out = dy.shape
        db2 = None
        if dy.dtype == torch.float32 and gemm_dtype == torch.bfloat16 and c_out % 4 == 0 and c_out <= 1024:
            # The cast to the GEMMs' bf16 and fc2's bias gradient (the column
            # sums of the bf16 values) in one pass over the token rows.
            if ctx.needs_input_grad[6]:
                db2 = torch.zeros(c_out, dtype=torch.float32, device=dy.device)
            dh2 = kernels.swin_partition(dy.contiguous().view(1, T, 1, c_out), kernels.rows_geometry(T, c_out),
                                         out_dtype=torch.bfloat16, column_sums=db2).view(T, c_out)
        else:
            dh2 = dy.to(gemm_dtype)
            db2 = dh2.sum(0, dtype=torch.float32) if ctx.needs_input_grad[6] else None
        w2c, w1c = w2.to(gemm_dtype), w1.to(gemm_dtype)
        da = dh2 @ w2c
        dw2 = weight_grad(dh2, a.to(gemm_dtype)) if ctx.needs_input_grad[5] else None
        db1 = None
        if kernels.gelu_backward_supported(h1):
            # The GELU derivative and fc1's bias gradient in one pass.
            if ctx.needs_input_grad[4]:
                db1 = torch.zeros(h1.shape[-1], dtype=torch.float32, device=h1.device)
            dh1 = kernels.gelu_backward(da.contiguous(), h1.contiguous(), column_sums=db1)
        else:
            dh1 = torch.ops.aten.gelu_backward(da, h1)
            db1 = dh1.sum(0, dtype=torch.float32) if ctx.needs_input_grad[4] else None
        dxn = dh1 @ w1c
        dw1 = weight_grad(dh1, xn.to(gemm_dtype)) if ctx.needs_input_grad[3] else None
        dlw = torch.zeros(C, dtype=torch.float32, device=rows.device) if (
            ln_w is not None and ctx.needs_input_grad[1]) else None
        dlb = torch.zeros(C, dtype=torch.float32, device=rows.device) if (
            ln_b is not None and ctx.needs_input_grad[2]) else None
        # dxn in xn's dtype (bf16 under autocast, read exactly by the kernel).
        dx = kernels.swin_partition_ln_backward(
            dxn.to(xn.dtype).contiguous().view(-1, 1, C), rows.view(1, -1, 1, C), ctx.geom, ln_w, ctx.eps,
            dresidual=dy.to(rows.dtype).contiguous(), dweight=dlw, dbias=dlb)
        cast = lambda g, p: None if g is None else g.to(p.dtype)  # noqa: E731
        return (dx.view(ctx.shape), cast(dlw, ln_w), cast(dlb, ln_b), cast(dw1, w1), cast(db1, w1),
                cast(dw2, w2), cast(db2, w2), None)


def mlp(x: torch.Tensor, ln_w: Optional[torch.Tensor], ln_b: Optional[torch.Tensor], w1: torch.Tensor,
        b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor, eps: float) -> torch.Tensor:
    """The MLP half with gradients (see :class:`_Mlp`)."""
    return _Mlp.apply(x, ln_w, ln_b, w1, b1, w2, b2, eps)


def partition(x: torch.Tensor, geom: WindowGeometry) -> torch.Tensor:
    """:func:`kernels.swin_partition` with a gradient (reverse)."""
    if _needs_grad(x):
        return _Partition.apply(x, geom)
    return kernels.swin_partition(x, geom)


def reverse(windows: torch.Tensor, geom: WindowGeometry, residual: Optional[torch.Tensor] = None,
            link: Optional[ResidualLink] = None, out_dtype: Optional[torch.dtype] = None,
            bias_sums: Optional[ColumnSumLink] = None) -> torch.Tensor:
    """:func:`kernels.swin_reverse` with gradients (partition for the windows,
    identity for the residual), in ``out_dtype`` (default: the windows'
    dtype; bf16 windows into fp32 are widened by the kernel, other pairs by a
    cast first).  With ``link`` (the residual is the input of the
    :func:`partition_ln` holding the same link) the residual's gradient goes
    through the link instead of autograd.  ``bias_sums``: the
    :class:`ColumnSumLink` of the :func:`linear` whose output the windows are;
    the bf16 backward fills it."""
    odt = windows.dtype if out_dtype is None else out_dtype
    if odt != windows.dtype and not (windows.dtype == torch.bfloat16 and odt == torch.float32):
        windows = windows.to(odt)
    if link is not None and residual is not None:
        return _Reverse.apply(windows, geom, residual.detach(), link, odt, bias_sums)
    if _needs_grad(windows, residual):
        return _Reverse.apply(windows, geom, residual, None, odt, bias_sums)
    return kernels.swin_reverse(windows, geom, residual=residual, out_dtype=odt)


def _check_backward(q: torch.Tensor, num_heads: int, window_size: Tuple[int, int], n_real: Optional[int]) -> None:
    if not kernels.attention_backward_supported(q, num_heads, window_size, n_real):
        raise NotImplementedError(
            "terra_amd: the attention backward kernels are built for bf16 / fp32 activations, windows up to 8x8 "
            "in at most 64 token rows and head dim 32, 64 or 128, and for bf16 windows of a multiple of 128 tokens "
            f"up to 4096 with head dim 64 or 128 (got {q.dtype}, window {tuple(window_size)}, "
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
    backward GEMM), with no slice copies.  With a :class:`ColumnSumLink` the
    bf16 kernel also sums that buffer's columns (the projection's bias
    gradient) while it writes it."""

    @staticmethod
    def forward(ctx, qkv, table, num_heads, window_size, scale, mask, n_real, mask_value, bias_sums):
        C = qkv.shape[-1] // 3
        ctx.cfg = (num_heads, window_size, scale, mask, n_real, mask_value)
        ctx.bias_sums = bias_sums
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
        sums = None
        if ctx.bias_sums is not None and kernels.attention_backward_sums_supported(qkv[..., :C], num_heads,
                                                                                   window_size, n_real):
            sums = torch.zeros(3 * C, dtype=torch.float32, device=qkv.device)
            ctx.bias_sums.sums = sums
        kernels.window_attention_backward(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], grad.contiguous(),
                                          num_heads, window_size, scale, bias_table=table, mask=mask, n_real=n_real,
                                          mask_value=mask_value, dq=dqkv[..., :C], dk=dqkv[..., C:2 * C],
                                          dv=dqkv[..., 2 * C:], dbias=dbias, column_sums=sums)
        dtable = None if dbias is None else dbias.to(table.dtype)
        return dqkv, dtable, None, None, None, None, None, None, None


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
                         n_real: Optional[int] = None, mask_value: float = kernels.MASK_VALUE,
                         bias_sums: Optional[ColumnSumLink] = None) -> torch.Tensor:
    """Attention over the column blocks q | k | v of one [B_, N, 3C] tensor,
    with gradients (see :class:`_AttentionQKV`).  ``bias_sums``: the
    :class:`ColumnSumLink` of the :func:`linear` that produced ``qkv``."""
    C = qkv.shape[-1] // 3
    if _needs_grad(qkv, bias_table):
        if not qkv.is_contiguous():
            qkv = qkv.contiguous()
        return _AttentionQKV.apply(qkv, bias_table, num_heads, tuple(window_size), scale, mask, n_real, mask_value,
                                   bias_sums)
    return kernels.window_attention(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], num_heads, window_size,
                                    scale, bias_table=bias_table, mask=mask, n_real=n_real, mask_value=mask_value)
