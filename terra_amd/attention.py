"""Drop-in ``WindowAttention`` (models/attention.py:175-283) on the HIP core.

Constructor arguments, parameter / buffer names and initialisation order are
the reference's, so its state dicts load unchanged:
``relative_position_bias_table``, ``relative_position_index``, ``q_linear``,
``k_linear``, ``v_linear``, ``proj``.  The forward runs the three q/k/v
projections as one GEMM over the concatenated weights (x is read once), the
fused HIP attention core on the projection output in place (no permute
copies), then ``proj``.  With gradients enabled the core's backward is the
HIP backward kernel (terra_amd.autograd).
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence, Union

import torch
import torch.nn.functional as F

from . import autograd, kernels
from .kernels import ShiftMask, WindowMask


def run_with_seed(init_seed: Optional[int], fn: Callable):
    """Run ``fn`` under ``torch.manual_seed(init_seed)`` and restore the global
    RNG state afterwards (models/model_utils/init_weight.py:31-41)."""
    if init_seed is None:
        return fn()
    devices = list(range(torch.cuda.device_count())) if torch.cuda.is_available() else []
    with torch.random.fork_rng(devices=devices):
        torch.manual_seed(int(init_seed))
        return fn()


def make_linear_with_seed(in_dim: int, out_dim: int, bias: bool = True,
                          init_seed: Optional[int] = None) -> torch.nn.Linear:
    """``nn.Linear`` created under a fixed seed (models/model_utils/init_weight.py:18-28)."""
    return run_with_seed(init_seed, lambda: torch.nn.Linear(in_dim, out_dim, bias=bias))


def relative_position_index(window_size: Sequence[int]) -> torch.Tensor:
    """Swin relative-position index [Wh*Ww, Wh*Ww] (models/attention.py:205-214):
    idx[i, j] = (hi - hj + Wh - 1) * (2*Ww - 1) + (wi - wj + Ww - 1)."""
    wh, ww = int(window_size[0]), int(window_size[1])
    hi = torch.arange(wh).repeat_interleave(ww)
    wi = torch.arange(ww).repeat(wh)
    return (hi[:, None] - hi[None, :] + wh - 1) * (2 * ww - 1) + (wi[:, None] - wi[None, :] + ww - 1)


class WindowAttention(torch.nn.Module):
    """Window multi-head self-attention with relative-position bias.

    ``forward(x[B_, N, C], mask)``; ``mask`` may be None, a dense additive
    ``[nW, N, N]`` tensor (as in the reference), a :class:`kernels.ShiftMask`
    (the same mask in closed form), or a :class:`kernels.WindowMask` adding
    per-window land bits.  ``use_flash_attention`` is accepted for signature
    compatibility; the fused HIP core serves every case.
    """

    def __init__(self, embedding_dim, window_size, num_heads, qkv_bias=True, qk_scale=None,
                 use_attn_mask=True, use_relative_position_bias=True, use_flash_attention=False,
                 init_seed_base=None):
        super().__init__()
        self.use_attn_mask = use_attn_mask
        self.use_relative_position_bias = use_relative_position_bias
        self.use_flash_attention = use_flash_attention
        self.dim = embedding_dim
        self.window_size = tuple(window_size)
        self.num_heads = num_heads
        if self.dim % num_heads != 0:
            raise AssertionError(f"dim {self.dim} must be divisible by num_heads {num_heads}")
        head_dim = self.dim // num_heads
        self.scale = qk_scale or head_dim ** -0.5

        if self.use_relative_position_bias:
            wh, ww = self.window_size
            self.relative_position_bias_table = torch.nn.Parameter(
                torch.zeros((2 * wh - 1) * (2 * ww - 1), num_heads))
            self.register_buffer("relative_position_index", relative_position_index(self.window_size))
            run_with_seed(init_seed_base,
                          lambda: torch.nn.init.trunc_normal_(self.relative_position_bias_table, std=.02))

        seed = (lambda k: None if init_seed_base is None else init_seed_base + k)
        self.q_linear = make_linear_with_seed(self.dim, self.dim, bias=qkv_bias, init_seed=seed(1))
        self.k_linear = make_linear_with_seed(self.dim, self.dim, bias=qkv_bias, init_seed=seed(2))
        self.v_linear = make_linear_with_seed(self.dim, self.dim, bias=qkv_bias, init_seed=seed(3))
        self.proj = make_linear_with_seed(self.dim, self.dim, bias=True, init_seed=seed(4))
        self.softmax = torch.nn.Softmax(dim=-1)

    def _cached(self, name: str, tensors, build):
        """``build()`` cached under ``name`` until any of ``tensors`` changes
        (data pointer, in-place version or dtype).  Only for calls without
        gradients: the result is detached."""
        key = tuple(None if t is None else (t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)
        cache = self.__dict__.setdefault("_derived", {})
        hit = cache.get(name)
        if hit is not None and hit[0] == key:
            return hit[1]
        with torch.no_grad():
            val = build()
        cache[name] = (key, val)
        return val

    def qkv(self, x: torch.Tensor, bias_sums: Optional[autograd.ColumnSumLink] = None) -> torch.Tensor:
        """The three projections as one GEMM: [B_, N, C] -> [B_, N, 3C].
        ``bias_sums``: a link the attention core's backward fills with the
        bias gradient (see :meth:`attend`)."""
        lins = (self.q_linear, self.k_linear, self.v_linear)
        has_bias = self.q_linear.bias is not None
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()):
            w = torch.cat([l.weight for l in lins], 0)
            b = torch.cat([l.bias for l in lins], 0) if has_bias else None
            return autograd.linear(x, w, b, bias_sums=bias_sums)
        else:  # the concatenated weights, kept until a parameter changes
            w, b = self._cached("qkv", [l.weight for l in lins] + [l.bias for l in lins], lambda: (
                torch.cat([l.weight for l in lins], 0), torch.cat([l.bias for l in lins], 0) if has_bias else None))
        return F.linear(x, w, b)

    def _table(self) -> Optional[torch.Tensor]:
        """The bias table as the core takes it: the parameter itself when a
        gradient may flow into it, else an fp32 copy kept until it changes."""
        if not self.use_relative_position_bias:
            return None
        t = self.relative_position_bias_table
        if t.dtype == torch.float32 or (torch.is_grad_enabled() and t.requires_grad):
            return t
        return self._cached("table", [t], lambda: t.detach().to(torch.float32).contiguous())

    def core(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             mask: Union[None, torch.Tensor, ShiftMask, WindowMask] = None,
             n_real: Optional[int] = None) -> torch.Tensor:
        """Fused core on projected q/k/v [B_, N, C] (row strides may exceed C)."""
        return autograd.window_attention(q, k, v, self.num_heads, self.window_size, self.scale,
                                         bias_table=self._table(), mask=mask, n_real=n_real)

    def attend(self, x: torch.Tensor, mask=None) -> torch.Tensor:
        """Everything of forward but the output projection: q/k/v and the
        fused core, O [B_, N, C] (models/attention.py:244-278).  In training
        the core's backward kernel also sums the q | k | v gradient's columns,
        which the projection's backward takes as its bias gradient."""
        link = autograd.ColumnSumLink() if torch.is_grad_enabled() else None
        return autograd.window_attention_qkv(self.qkv(x, bias_sums=link), self.num_heads, self.window_size,
                                             self.scale, bias_table=self._table(), mask=mask, bias_sums=link)

    def forward(self, x: torch.Tensor, mask=None) -> torch.Tensor:
        return autograd.linear(self.attend(x, mask=mask), self.proj.weight, self.proj.bias)

    def proj_packed(self):
        """proj's weight in the fragment-packed layout of the linear kernels
        (bf16; autocast's cast of an fp32 weight) and its bias as fp32,
        cached until either changes; for calls without gradients."""
        w, b = self.proj.weight, self.proj.bias
        return self._cached("proj_packed", [w, b], lambda: (
            kernels.pack_linear(w.detach().to(torch.bfloat16).contiguous()),
            None if b is None else b.detach().to(torch.float32).contiguous()))
