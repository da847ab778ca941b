"""Seeded synthetic workloads of the benchmark configurations.

Every tensor is drawn on the CPU from ``torch.Generator('cpu')`` so that the
GPU path and any CPU check see bit-identical inputs, then cast and moved.

Configurations (shape and semantics of each; sizes as benchmarked):
  c1  fp32, B=1, 56x56, C=96, 3 heads, window 7, shift 0, no mask
  c2  bf16, B=4, 112x112, C=128, 4 heads, window 7; W-MSA then SW-MSA (shift 3)
  c3  bf16, B=1, 512x1024, C=192, 6 heads, window 8, shift 4, ~30 % land mask
  c4  bf16, B=1, 128x256 token grid, C=768, 12 heads, window 8, shift 4 (odd blocks)
  c5  bf16, B=2, one rank's slab of a 255x64-window grid (2040x512 tokens) split
      7 ways by the ragged row-major assignment: rank 1 owns flat windows
      [2331, 4662), i.e. window rows 36..72 (37 rows, 296 token rows) with 27
      pad windows at the start of its first row and 10 at the end of its last;
      C=384, 12 heads, window 8, shift 4, ~30 % land.  The SW-MSA shift reads 4
      halo rows below the slab, supplied as zero padding (pad_bottom = 8 keeps
      the frame a whole number of windows; its 38th window row is not emitted);
      the width is the full global width, so W stays cyclic.
  w32 bf16, the g1 grid with 32x32 windows (1024 tokens, 153 windows), shift 16
      (odd blocks), no relative-position bias and no mask: the block of
      configs/model/correctness/credit_hierarchical_swin_correctness_seq.yaml
      (:21-30: window_size 32, use_attn_mask False, use_relative_position_bias
      False), whose attention core is MFMA-bound (4 N^2 C flops per window).
  g1  bf16, B=1, 288x544 token grid, C=1024, 8 heads of dim 128, window 8,
      shift 4 (odd blocks), shift mask and relative-position bias on, no land:
      the block every credit_hierarchical_swin pretrain config TERRA ships
      builds (configs/model/pretrain/credit_hierarchical_swin_seq_p4_ws8_0p1b_
      ddp_h200.yaml:27-39: padded_shape 2304x4352, patch 4, embedding_dim 1024,
      num_heads 8, window_size 8; BasicLayer runs at padded_shape / patch / 2,
      models/reference_model/sequential_hierarchical_swin.py:70-91).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch

from .window_assignment import slab_geometry

SEED_BASE = 2026061006  # init_seed_base of the reference blocks (models/transformer.py:87)


@dataclass(frozen=True)
class SwinConfig:
    name: str
    batch: int
    height: int
    width: int
    channels: int
    heads: int
    window: int
    shift: int
    dtype: torch.dtype
    land: bool = False
    pad: Tuple[int, int, int, int] = (0, 0, 0, 0)
    win_row_begin: int = 0
    win_rows: Optional[int] = None
    valid: Optional[Tuple[int, int]] = None
    mlp_ratio: Optional[int] = None
    attn_mask: bool = True       # the block's use_attn_mask
    rel_bias: bool = True        # the block's use_relative_position_bias
    note: str = field(default="", compare=False)

    @property
    def frame(self) -> Tuple[int, int]:
        return self.height + self.pad[0] + self.pad[1], self.width + self.pad[2] + self.pad[3]

    @property
    def windows_per_image(self) -> int:
        fh, fw = self.frame
        rows = fh // self.window - self.win_row_begin if self.win_rows is None else self.win_rows
        return rows * (fw // self.window)

    @property
    def num_windows(self) -> int:
        return self.batch * self.windows_per_image

    @property
    def tokens(self) -> int:
        return self.window * self.window

    @property
    def real_tokens(self) -> int:
        """Tokens of real (non-pad) windows."""
        per_img = self.windows_per_image if self.valid is None else self.valid[1] - self.valid[0]
        return self.batch * per_img * self.tokens

    def scaled(self, height: int, width: int, batch: Optional[int] = None) -> "SwinConfig":
        """Same semantics on a smaller grid (parity tests at oracle-friendly sizes)."""
        return SwinConfig(self.name + f"@{height}x{width}", batch or self.batch, height, width, self.channels,
                          self.heads, self.window, self.shift, self.dtype, self.land, mlp_ratio=self.mlp_ratio,
                          attn_mask=self.attn_mask, rel_bias=self.rel_bias)


def _c5() -> SwinConfig:
    first_row, rows, vb, ve = slab_geometry(255, 64, 7, 1)
    return SwinConfig("c5", 2, rows * 8, 512, 384, 12, 8, 4, torch.bfloat16, land=True,
                      pad=(0, 8, 0, 0), win_row_begin=0, win_rows=rows, valid=(vb, ve),
                      note=f"slab rows {first_row}..{first_row + rows - 1} of a 255x64 window grid, rank 1 of 7")


CONFIGS = {
    "c1": SwinConfig("c1", 1, 56, 56, 96, 3, 7, 0, torch.float32),
    "c2": SwinConfig("c2", 4, 112, 112, 128, 4, 7, 3, torch.bfloat16, mlp_ratio=4),
    "c3": SwinConfig("c3", 1, 512, 1024, 192, 6, 8, 4, torch.bfloat16, land=True),
    "c4": SwinConfig("c4", 1, 128, 256, 768, 12, 8, 4, torch.bfloat16, mlp_ratio=4),
    "c5": _c5(),
    "g1": SwinConfig("g1", 1, 288, 544, 1024, 8, 8, 4, torch.bfloat16, mlp_ratio=4,
                     note="TERRA's shipped pretrain block (credit_hierarchical_swin, C=1024, 8 heads, ws 8)"),
    "w32": SwinConfig("w32", 1, 288, 544, 1024, 8, 32, 16, torch.bfloat16, mlp_ratio=4, attn_mask=False,
                      rel_bias=False,
                      note="TERRA's ws-32 correctness block (C=1024, 8 heads, ws 32, no bias, no mask)"),
}


def generator(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    return g


def activations(shape, seed: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """x ~ N(0, 1) drawn in fp32 on the CPU, then cast."""
    return torch.randn(*shape, generator=generator(seed), dtype=torch.float32).to(dtype)


def _gauss_blur_1d(z: torch.Tensor, sigma: float, dim: int) -> torch.Tensor:
    radius = max(1, int(3 * sigma))
    t = torch.arange(-radius, radius + 1, dtype=torch.float32)
    k = torch.exp(-0.5 * (t / sigma) ** 2)
    k = (k / k.sum()).view(1, 1, -1)
    x = z.movedim(dim, -1)
    shp = x.shape
    x = x.reshape(-1, 1, shp[-1])
    x = torch.nn.functional.pad(x, (radius, radius), mode="circular")
    x = torch.nn.functional.conv1d(x, k).reshape(shp)
    return x.movedim(-1, dim)


def land_mask(height: int, width: int, seed: int, fraction: float = 0.30) -> torch.Tensor:
    """~`fraction` land in contiguous blobs: N(0,1) noise, separable Gaussian blur
    with sigma = height/32 tokens, thresholded at its (1 - fraction) quantile."""
    z = torch.randn(height, width, generator=generator(seed), dtype=torch.float32)
    sigma = max(1.0, height / 32.0)
    z = _gauss_blur_1d(_gauss_blur_1d(z, sigma, 0), sigma, 1)
    thr = torch.quantile(z.flatten()[:: max(1, z.numel() // 4_000_000)].double(), 1.0 - fraction).float()
    return z > thr


def init_block_params(block: torch.nn.Module, layer_idx: int) -> None:
    """Weights and the bias table trunc-normal(std=0.02) from fixed seeds, Linear
    biases zero; LayerNorm weight 1 / bias 0 (torch defaults)."""
    base = SEED_BASE + 100 * layer_idx
    with torch.no_grad():
        attn = block.attn
        if getattr(attn, "relative_position_bias_table", None) is not None:
            t = torch.empty_like(attn.relative_position_bias_table, device="cpu")
            torch.nn.init.trunc_normal_(t, std=0.02, generator=generator(base))
            attn.relative_position_bias_table.copy_(t)
        for k, lin in enumerate((attn.q_linear, attn.k_linear, attn.v_linear, attn.proj), start=1):
            w = torch.empty_like(lin.weight, device="cpu")
            torch.nn.init.trunc_normal_(w, std=0.02, generator=generator(base + k))
            lin.weight.copy_(w)
            if lin.bias is not None:
                lin.bias.zero_()


def mlp_for(cfg: SwinConfig, layer_idx: int):
    """The SequentialMlp that follows block `layer_idx` of `cfg` (hidden
    mlp_ratio * C, 4 when the config names none, as BasicLayer builds it in
    models/reference_model/parallel_layers.py:46-70), weights trunc-normal(std=
    0.02) from fixed seeds, biases zero, LayerNorm defaults, on the CPU."""
    from .mlp import SequentialMlp

    C = cfg.channels
    mlp = SequentialMlp(C, (cfg.mlp_ratio or 4) * C)
    base = SEED_BASE + 100 * layer_idx + 50
    with torch.no_grad():
        for k, lin in enumerate((mlp.fc1, mlp.fc2), start=1):
            w = torch.empty_like(lin.weight, device="cpu")
            torch.nn.init.trunc_normal_(w, std=0.02, generator=generator(base + k))
            lin.weight.copy_(w)
            lin.bias.zero_()
    return mlp


def block_for(cfg: SwinConfig, layer_idx: int, land: Optional[torch.Tensor] = None):
    """A SequentialSwinTransformer of `cfg` for layer `layer_idx` (shift on odd
    layers, as in the reference), with seeded weights, on the CPU."""
    from .transformer import SequentialSwinTransformer

    blk = SequentialSwinTransformer(layer_idx=layer_idx, height=cfg.height, width=cfg.width,
                                    embedding_dim=cfg.channels, window_size=cfg.window, num_heads=cfg.heads,
                                    use_attn_mask=cfg.attn_mask, use_relative_position_bias=cfg.rel_bias,
                                    land_mask=land, pad=cfg.pad, win_row_begin=cfg.win_row_begin,
                                    win_rows=cfg.win_rows, valid_windows=cfg.valid)
    init_block_params(blk, layer_idx)
    return blk
