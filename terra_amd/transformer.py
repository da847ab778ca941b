"""Drop-in ``SequentialSwinTransformer`` (models/transformer.py:71-356).

The attention half of a Swin block on one GPU.  For bf16 activations and
(window, heads, C) in kernels.BLOCK_SHAPES (8x8 windows with 6, 12 or 12 heads
at C = 192, 384, 768; 7x7 windows with 4 heads at C = 128) the whole half-block is one HIP
kernel (``kernels.swin_block``: gather + LayerNorm + q/k/v + attention + proj
+ residual + scatter).  Otherwise:

    x -> [norm1 + roll(-s) + window partition]      one HIP gather
      -> q/k/v projection (one GEMM)                 hipBLASLt via torch
      -> fused window-attention core                 one HIP kernel
      -> proj                                        hipBLASLt via torch
      -> [window reverse + roll(+s) + residual add]  one HIP scatter

Module construction, parameter and buffer names (``norm1``, ``attn.*``,
``attn_mask``) follow the reference so its checkpoints load.  The shift mask
is evaluated in closed form inside the attention kernel; the dense
``attn_mask`` buffer is kept only for state-dict compatibility and equals that
closed form element for element.

Additions that the reference does not have (both optional, build-defined):
``land_mask`` — a [H, W] boolean grid whose land keys receive the mask value
-100 in every window (folded into the attention mask); ``geometry`` overrides
(padding, window-row range, valid-window range) for slabs such as one rank's
share of a window-parallel grid.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import autograd, config, kernels
from .attention import WindowAttention
from .kernels import ShiftMask, WindowGeometry, WindowMask
from .utils import get_swin_attention_mask, land_window_bits


class SequentialSwinTransformer(torch.nn.Module):
    def __init__(self, layer_idx=-1, height=720 // 6, width=1440 // 6, embedding_dim=4320,
                 norm_layer=torch.nn.LayerNorm, window_size=6, num_heads=4320 // 72,
                 use_attn_mask=True, use_relative_position_bias=True, use_flash_attention=False,
                 init_seed_base=None, land_mask: Optional[torch.Tensor] = None,
                 pad: Tuple[int, int, int, int] = (0, 0, 0, 0), win_row_begin: int = 0,
                 win_rows: Optional[int] = None, valid_windows: Optional[Tuple[int, int]] = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.init_seed_base = None if init_seed_base is None else int(init_seed_base) + int(layer_idx) * 100
        # W-MSA on even layers, SW-MSA (shift ws//2) on odd ones (models/transformer.py:88-91).
        shift_size = 0 if (self.layer_idx % 2 == 0) else window_size // 2
        if config.use_shift_size_0:
            shift_size = 0
        self.shift_size = shift_size
        self.window_size = window_size
        self.use_attn_mask = use_attn_mask
        if config.use_layernorm:
            self.norm1 = norm_layer(embedding_dim)
        self.input_resolution = (height, width)
        self.embedding_dim = embedding_dim
        self.attn = WindowAttention(embedding_dim, window_size=(window_size, window_size), num_heads=num_heads,
                                    qkv_bias=True, qk_scale=None, use_attn_mask=use_attn_mask,
                                    use_relative_position_bias=use_relative_position_bias,
                                    use_flash_attention=use_flash_attention, init_seed_base=self.init_seed_base)
        self.pad = tuple(int(p) for p in pad)
        self.win_row_begin = int(win_row_begin)
        self.win_rows = win_rows
        self.valid_windows = valid_windows
        frame = (height + self.pad[0] + self.pad[1], width + self.pad[2] + self.pad[3])
        attn_mask = None
        if self.shift_size > 0 and self.use_attn_mask:
            attn_mask = get_swin_attention_mask("sequential", frame, self.window_size, self.shift_size)
        self.register_buffer("attn_mask", attn_mask)
        if land_mask is not None:
            land_mask = torch.as_tensor(land_mask).to(torch.bool)
            if tuple(land_mask.shape) != (height, width):
                raise ValueError(f"land_mask must be [{height}, {width}], got {tuple(land_mask.shape)}")
            self.register_buffer("land_mask", land_mask, persistent=False)
        else:
            self.land_mask = None
        self._land_bits_cache = {}
        self._mask_cache = None
        # Run the whole half-block as one kernel where the shapes allow it
        # (see _fusable_block); False forces the five-stage path.
        self.use_fused_block = True

    def geometry(self, batch: int) -> WindowGeometry:
        H, W = self.input_resolution
        return WindowGeometry(batch, H, W, self.embedding_dim, self.window_size, self.shift_size,
                              self.shift_size, self.pad, self.win_row_begin, self.win_rows, self.valid_windows)

    def window_mask(self, geom: WindowGeometry):
        """Mask argument of the attention core for this block, or None."""
        lm = self.land_mask
        key = (geom, self.shift_size > 0 and self.use_attn_mask,
               None if lm is None else (lm.device, lm.data_ptr(), lm._version))
        cached = self._mask_cache
        if cached is not None and cached[0] == key:
            return cached[1]
        shift = ShiftMask.from_geometry(geom) if key[1] else None
        land = None
        if lm is not None:
            # The bits depend on the frame (shift, padding, emitted rows, valid
            # windows) as well as on the land grid: both key the cache.
            land_geom = WindowGeometry(1, geom.height, geom.width, 1, geom.window, geom.shift_h, geom.shift_w,
                                       geom.pad, geom.win_row_begin, geom.win_rows, geom.valid)
            land_key = (land_geom, key[2])
            land = self._land_bits_cache.get(land_key)
            if land is None:
                land = land_window_bits(lm, land_geom)
                self._land_bits_cache = {land_key: land}
        mask = None if shift is None and land is None else WindowMask(shift=shift, land_bits=land)
        self._mask_cache = (key, mask)
        return mask

    def _fusable_norm(self, dtype: torch.dtype) -> bool:
        """norm1 is a plain LayerNorm over C that the gather kernel computes
        for activations of `dtype` (C <= 1024 in rows of whole 16-byte chunks,
        <= 4096 B)."""
        n = self.norm1
        row_bytes = self.embedding_dim * dtype.itemsize
        return (type(n) is torch.nn.LayerNorm and tuple(n.normalized_shape) == (self.embedding_dim,)
                and dtype in (torch.float32, torch.float16, torch.bfloat16)
                and row_bytes % 16 == 0 and row_bytes <= 4096 and self.embedding_dim <= 1024)

    def _proj_scatter(self, x_windows: torch.Tensor, shortcut: torch.Tensor, geom: WindowGeometry) -> bool:
        """Whether the output projection, the window reverse and the residual
        add can run as one linear-kernel launch: bf16 windows and shortcut,
        8x8 windows, C a multiple of 256 (the kernel's feature tile; C = 1024
        for TERRA's pretrain blocks), every window of the frame emitted, a
        biased nn.Linear proj of the activation dtype (or fp32 under bf16
        autocast)."""
        C = geom.channels
        if x_windows.dtype != torch.bfloat16 or shortcut.dtype != torch.bfloat16 or geom.window != 8:
            return False
        if not kernels.linear_supported(x_windows, C, C):
            return False
        if geom.win_row_begin != 0 or geom.valid is not None or geom.rows != geom.frame_h // geom.window:
            return False
        proj = self.attn.proj
        if type(proj) is not torch.nn.Linear or proj.bias is None:
            return False
        return proj.weight.dtype == torch.bfloat16 or (
            kernels.autocast_bf16(x_windows) and proj.weight.dtype == torch.float32)

    def _fusable_block(self, x: torch.Tensor, geom: WindowGeometry) -> bool:
        """The whole half-block runs as one kernel: bf16, (window, heads, C) in
        kernels.BLOCK_SHAPES, a plain LayerNorm (or none), biased q/k/v, and
        no gradient needed (the fused kernel is forward-only)."""
        attn = self.attn
        if not self.use_fused_block or not kernels.swin_block_supported(x, geom, attn.num_heads):
            return False
        if config.use_layernorm and not self._fusable_norm(x.dtype):
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        lins = (attn.q_linear, attn.k_linear, attn.v_linear, attn.proj)
        # Weights of the activation dtype, or fp32 weights inside a bf16
        # autocast region (where F.linear would cast them to bf16).
        w_ok = all(l.weight.dtype == x.dtype for l in lins) or (
            kernels.autocast_bf16(x) and all(l.weight.dtype == torch.float32 for l in lins))
        return w_ok and attn.q_linear.bias is not None

    def _fused_args(self) -> dict:
        """Fragment-packed bf16 q|k|v and proj weights (cast from fp32 weights
        under autocast, as F.linear would) and fp32 copies of the small
        parameters, cached until any of them changes (data pointer, in-place
        version or dtype)."""
        attn = self.attn
        tensors = [attn.q_linear.weight, attn.k_linear.weight, attn.v_linear.weight, attn.q_linear.bias,
                   attn.k_linear.bias, attn.v_linear.bias, attn.proj.weight, attn.proj.bias]
        if config.use_layernorm:
            tensors += [self.norm1.weight, self.norm1.bias]
        if attn.use_relative_position_bias:
            tensors.append(attn.relative_position_bias_table)
        key = tuple((t.data_ptr(), t._version, t.device, t.dtype) if t is not None else None for t in tensors)
        cached = getattr(self, "_fused_cache", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        with torch.no_grad():
            f32 = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()  # noqa: E731
            bf16 = lambda t: t.detach().to(torch.bfloat16).contiguous()  # noqa: E731
            w_qkv = torch.cat([bf16(attn.q_linear.weight), bf16(attn.k_linear.weight), bf16(attn.v_linear.weight)], 0)
            args = dict(
                qkv_weight=kernels.pack_linear(w_qkv.contiguous()),
                qkv_bias=f32(torch.cat([attn.q_linear.bias, attn.k_linear.bias, attn.v_linear.bias], 0)),
                proj_weight=kernels.pack_linear(bf16(attn.proj.weight)),
                packed_weights=True,
                proj_bias=f32(attn.proj.bias),
                ln_weight=f32(self.norm1.weight) if config.use_layernorm else None,
                ln_bias=f32(self.norm1.bias) if config.use_layernorm else None,
                ln_eps=float(self.norm1.eps) if config.use_layernorm else 0.0,
                layernorm=bool(config.use_layernorm),
                bias_table=f32(attn.relative_position_bias_table) if attn.use_relative_position_bias else None,
            )
        self._fused_cache = (key, args)
        return args

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        H, W = self.input_resolution
        B, L, C = x.shape
        if L != H * W:
            raise AssertionError("input feature has wrong size")
        shortcut = x
        geom = self.geometry(B)
        grid = x.contiguous().view(B, H, W, C)
        if self._fusable_block(grid, geom):
            mask = self.window_mask(geom)
            y = kernels.swin_block(grid, geom, self.attn.num_heads, self.attn.scale,
                                   shift_mask=mask is not None and mask.shift is not None,
                                   land_bits=None if mask is None else mask.land_bits, **self._fused_args())
            return y.view(B, H * W, C)
        # Training: the partition / reverse permutations and the LayerNorm
        # with their HIP backward kernels.
        training = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        link = None
        if config.use_layernorm and not training and self._fusable_norm(grid.dtype):
            n = self.norm1
            ln_w, ln_b = n.weight, n.bias
            if (ln_w is not None and ln_w.dtype != torch.float32) or (ln_b is not None and ln_b.dtype != torch.float32):
                ln_w, ln_b = self.attn._cached("norm1", [n.weight, n.bias], lambda: tuple(
                    None if t is None else t.detach().to(torch.float32).contiguous() for t in (n.weight, n.bias)))
            x_windows = kernels.swin_partition_ln(grid, geom, ln_w, ln_b, n.eps)
        elif config.use_layernorm and self._fusable_norm(grid.dtype):
            # Training: the fused LayerNorm + partition, whose backward kernel
            # also gives the LayerNorm weight and bias gradients.
            n = self.norm1
            # Under bf16 autocast the q/k/v Linear would cast fp32 windows to
            # bf16: the kernel writes that bf16 copy itself.  When x needs a
            # gradient, the residual's gradient is added in the LayerNorm
            # backward's kernel (link).
            link = autograd.ResidualLink() if training and x.requires_grad else None
            x_windows = autograd.partition_ln(grid, geom, n.weight, n.bias, n.eps,
                                              out_dtype=autograd.linear_input_dtype(grid), link=link)
        else:
            if config.use_layernorm:  # a norm layer the gather does not fuse runs on its own
                grid = self.norm1(grid.view(B, L, C)).contiguous().view(B, H, W, C)
            x_windows = autograd.partition(grid, geom)
        bias_sums = None
        if not training and self._proj_scatter(x_windows, shortcut, geom):
            # proj + window reverse + inverse roll + residual in one kernel.
            o = self.attn.attend(x_windows, mask=self.window_mask(geom))
            if o.dtype == torch.bfloat16:
                w, b = self.attn.proj_packed()
                y = kernels.linear_residual(o.contiguous(), w, C, shortcut.contiguous().view(B, H, W, C), b, geom=geom)
                return y.view(B, H * W, C)
            attn_windows = autograd.linear(o, self.attn.proj.weight, self.attn.proj.bias)
        else:
            proj = self.attn.proj
            if training and type(proj) is torch.nn.Linear and proj.bias is not None:
                # proj's bias gradient is summed by the scatter's backward
                # kernel while it writes proj's output gradient.
                bias_sums = autograd.ColumnSumLink()
                o = self.attn.attend(x_windows, mask=self.window_mask(geom))
                attn_windows = autograd.linear(o, proj.weight, proj.bias, bias_sums=bias_sums)
            else:
                attn_windows = self.attn(x_windows, mask=self.window_mask(geom))
        out_dtype = torch.promote_types(attn_windows.dtype, shortcut.dtype)
        residual = shortcut.to(out_dtype).contiguous().view(B, H, W, C)
        # The link carries the residual's gradient only when the residual is
        # the LayerNorm's input itself (same dtype, no copy in between).
        link = link if (config.use_layernorm and residual.data_ptr() == grid.data_ptr()
                        and residual.dtype == grid.dtype) else None
        # bf16 windows into an fp32 result (autocast's proj output plus the
        # fp32 shortcut) are widened by the scatter kernel itself.
        y = autograd.reverse(attn_windows.contiguous(), geom, residual=residual, link=link, out_dtype=out_dtype,
                             bias_sums=bias_sums)
        return y.view(B, H * W, C)
