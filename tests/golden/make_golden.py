"""Writes the small golden fixtures of tests/golden (run from the repository root).

known_answers.json  closed-form / reference-test values (hand-checkable):
  - the reference's own unit-test vector for the ragged row-major window split
    (TERRA tests/unit/test_window_assignment.py:10-23);
  - relative-position index corner values and shift-mask -100 counts.
swin_tiny.npz       seeded inputs and oracle outputs (float64 math, stored as float32) of a tiny
                    SW-MSA case (8x8 tokens, C=64, 2 heads, window 4, shift 2,
                    land mask), used to detect drift of the oracle and as a
                    committed target for the GPU kernels.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import swin_oracle as so  # noqa: E402


def known_answers():
    i7 = so.relative_position_index((7, 7))
    i8 = so.relative_position_index((8, 8))
    m7 = so.shift_mask(56, 56, 7, 3)
    m8 = so.shift_mask(32, 32, 8, 4)
    return {
        "ragged_row_major_2x5_m4": [[0, 1], [2, 3, 4], [5, 6], [7, 8, 9]],
        "rel_index_7x7": {"i00": int(i7[0, 0]), "max": int(i7.max()), "i_48_0": int(i7[48, 0]), "i_0_48": int(i7[0, 48])},
        "rel_index_8x8": {"i00": int(i8[0, 0]), "max": int(i8.max()), "i_63_0": int(i8[63, 0]), "i_0_63": int(i8[0, 63])},
        "shift_mask_ws7_s3_counts": {"last_row": int((m7[56] == -100).sum()), "corner": int((m7[63] == -100).sum())},
        "shift_mask_ws8_s4_counts": {"last_row": int((m8[12] == -100).sum()), "corner": int((m8[15] == -100).sum())},
    }


def tiny_case():
    g = torch.Generator().manual_seed(20261201)
    B, H, W, C, nH, ws, s = 1, 8, 8, 64, 2, 4, 2
    x = torch.randn(B, H, W, C, generator=g).double()
    qkv = torch.randn(B * (H // ws) * (W // ws), ws * ws, 3 * C, generator=g).double()
    table = (torch.randn((2 * ws - 1) ** 2, nH, generator=g) * 0.02).double()
    land = torch.rand(H, W, generator=g) < 0.3
    win = so.roll_partition(x, ws, s)
    mask = so.fold_land(so.shift_mask(H, W, ws, s).double(), so.land_key_flags(land, ws, s, s)).double()
    q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    o = so.window_attention_core(q, k, v, nH, (C // nH) ** -0.5, table, (ws, ws), mask, compute_dtype=torch.float64)
    return dict(x=x.float().numpy(), qkv=qkv.float().numpy(), table=table.float().numpy(), land=land.numpy(),
                windows=win.float().numpy(), mask=mask.float().numpy(), o=o.float().numpy(),
                meta=np.array([B, H, W, C, nH, ws, s], dtype=np.int64))


if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known_answers(), f, indent=1, sort_keys=True)
    np.savez_compressed(os.path.join(HERE, "swin_tiny.npz"), **tiny_case())
    print("wrote", os.listdir(HERE))
