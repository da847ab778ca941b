"""GPU parity of the partition (gather) and reverse (scatter) kernels:
bit-exact against the CPU oracle on identical inputs."""
import pytest
import torch

from oracle import swin_oracle as so
from terra_amd import kernels, utils, workloads
from terra_amd.kernels import WindowGeometry

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]

CASES = [  # (B, H, W, C, ws, shift, pad, win_row_begin, win_rows, valid)
    (2, 14, 21, 96, 7, 3, (0, 0, 0, 0), 0, None, None),
    (1, 16, 24, 128, 8, 4, (0, 0, 0, 0), 0, None, None),
    (2, 14, 14, 32, 7, 0, (0, 0, 0, 0), 0, None, None),
    (1, 13, 21, 40, 7, 3, (0, 1, 0, 0), 0, None, None),
    (2, 10, 17, 24, 4, 2, (1, 1, 2, 1), 1, 2, None),
    (2, 20, 16, 192, 8, 4, (0, 4, 0, 0), 0, 2, (3, 4)),
    (1, 16, 16, 6, 8, 4, (0, 8, 0, 0), 0, 2, (1, 3)),   # 12-byte rows: 4-byte chunks
    (1, 8, 8, 3, 4, 2, (0, 0, 0, 0), 0, None, None),    # odd channel count
]


def _geom(B, H, W, C, ws, s, pad, r0, rows, valid):
    return WindowGeometry(B, H, W, C, ws, s, s, pad, r0, rows, valid)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES)
def test_partition_bit_exact(dev, dtype, case):
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    x = workloads.activations((B, H, W, C), 100, dtype)
    got = kernels.swin_partition(x.to(dev), _geom(*case)).cpu()
    want = so.partition_frame(x, ws, s, s, pad, r0, rows, valid)
    assert got.dtype == want.dtype and torch.equal(got, want)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("with_residual", [False, True])
def test_reverse_bit_exact(dev, dtype, case, with_residual):
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    g = _geom(*case)
    win = workloads.activations((g.num_windows, ws * ws, C), 101, dtype)
    res = workloads.activations((B, H, W, C), 102, dtype) if with_residual else None
    got = kernels.swin_reverse(win.to(dev), g, residual=None if res is None else res.to(dev)).cpu()
    want = so.reverse_frame(win, B, H, W, ws, s, s, pad, r0, rows, valid, residual=res)
    assert torch.equal(got, want)


def test_u8_partition_and_land_bits(dev):
    land = workloads.land_mask(48, 64, seed=7)
    g = WindowGeometry(1, 48, 64, 1, 8, 4, 4)
    bits = utils.land_window_bits(land.to(dev), g).cpu()
    flags = so.land_key_flags(land, 8, 4, 4)
    want = utils.pack_key_bits(flags)
    assert torch.equal(bits, want)
    frac = land.float().mean().item()
    assert 0.25 < frac < 0.35


def test_reverse_in_place_on_residual(dev):
    B, H, W, C, ws, s = 1, 16, 16, 64, 8, 4
    g = WindowGeometry(B, H, W, C, ws, s, s)
    x = workloads.activations((B, H, W, C), 103, torch.bfloat16)
    win = workloads.activations((g.num_windows, 64, C), 104, torch.bfloat16)
    want = so.reverse_frame(win, B, H, W, ws, s, s, residual=x)
    y = x.to(dev)
    kernels.swin_reverse(win.to(dev), g, residual=y, out=y)
    assert torch.equal(y.cpu(), want)


def test_reference_helpers_window_partition_reverse(dev):
    x = workloads.activations((2, 14, 21, 96), 105, torch.bfloat16)
    w = utils.window_partition(x.to(dev), 7)
    assert tuple(w.shape) == (12, 7, 7, 96)
    assert torch.equal(w.cpu().view(12, 49, 96), so.roll_partition(x, 7))
    y = utils.window_reverse(w, 7, 14, 21)
    assert torch.equal(y.cpu(), x)


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_full_size_partition_and_round_trip(dev, name):
    cfg = workloads.CONFIGS[name]
    g = WindowGeometry(cfg.batch, cfg.height, cfg.width, cfg.channels, cfg.window, cfg.shift, cfg.shift,
                       cfg.pad, cfg.win_row_begin, cfg.win_rows, cfg.valid)
    x = workloads.activations((cfg.batch, cfg.height, cfg.width, cfg.channels), 106, cfg.dtype)
    xd = x.to(dev)
    win = kernels.swin_partition(xd, g)
    want = so.partition_frame(x, cfg.window, cfg.shift, cfg.shift, cfg.pad, cfg.win_row_begin, cfg.win_rows,
                              cfg.valid)
    assert torch.equal(win.cpu(), want)
    back = kernels.swin_reverse(win, g)
    if cfg.valid is None and cfg.pad == (0, 0, 0, 0):
        assert torch.equal(back, xd)  # reverse o partition == id on the full grid
    else:
        want_back = so.reverse_frame(want, cfg.batch, cfg.height, cfg.width, cfg.window, cfg.shift, cfg.shift,
                                     cfg.pad, cfg.win_row_begin, cfg.win_rows, cfg.valid)
        assert torch.equal(back.cpu(), want_back)


LN_CASES = [  # (B, H, W, C, ws, shift, pad, win_row_begin, win_rows, valid)
    (2, 14, 21, 96, 7, 3, (0, 0, 0, 0), 0, None, None),
    (1, 16, 24, 192, 8, 4, (0, 0, 0, 0), 0, None, None),
    (2, 20, 16, 384, 8, 4, (0, 4, 0, 0), 0, 2, (3, 4)),
    (1, 16, 16, 768, 8, 4, (0, 8, 0, 0), 0, 2, (1, 3)),
    (1, 6, 6, 64, 4, 2, (1, 1, 1, 1), 0, None, None),
    (1, 8, 16, 512, 8, 4, (0, 0, 0, 0), 0, None, None),   # 16 lanes per token, 4 chunks each
    (2, 8, 8, 640, 8, 0, (0, 0, 0, 0), 0, None, None),    # 16 lanes per token, last chunk group partial
    (1, 16, 8, 1024, 8, 4, (0, 0, 0, 0), 0, None, None),  # TERRA's pretrain width: 8 (bf16) / 16 (fp32) chunks per lane
    (1, 8, 16, 1000, 8, 4, (0, 0, 0, 0), 0, None, None),  # 1000 channels: partial last group in bf16 and fp32
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", LN_CASES)
@pytest.mark.parametrize("affine", [True, False])
def test_partition_ln_matches_layer_norm_then_partition(dev, dtype, case, affine):
    """Fused LayerNorm + partition == F.layer_norm (fp32) then the partition map.
    Tolerance: one rounding of the output dtype (fp32: 2e-6 relative + 1e-6);
    padding and pad windows are bit-exact."""
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    x = workloads.activations((B, H, W, C), 110, torch.float32) * 3 + 0.5
    x = x.to(dtype)
    w = (workloads.activations((C,), 111) * 0.1 + 1.0) if affine else None
    b = (workloads.activations((C,), 112) * 0.1) if affine else None
    g = _geom(*case)
    got = kernels.swin_partition_ln(x.to(dev), g, None if w is None else w.to(dev), None if b is None else b.to(dev),
                                    1e-5).cpu()
    ln = torch.nn.functional.layer_norm(x.float(), (C,), w, b, 1e-5)
    want = so.partition_frame(ln, ws, s, s, pad, r0, rows, valid)
    pad_mask = so.partition_frame(torch.ones(B, H, W, 1), ws, s, s, pad, r0, rows, valid) == 0
    pad_mask = pad_mask.expand_as(want)
    assert torch.all(got[pad_mask] == 0)
    err = (got.float() - want).abs()
    if dtype == torch.float32:
        tol = 2e-6 * want.abs() + 1e-6
    else:
        ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
        tol = ulp * want.abs() + 1e-4
    assert torch.all(err <= tol), float((err - tol).max())


def test_block_uses_fused_layer_norm(dev):
    """The drop-in block routes LayerNorm through the fused gather."""
    from terra_amd.transformer import SequentialSwinTransformer

    blk = SequentialSwinTransformer(layer_idx=1, height=16, width=16, embedding_dim=64, window_size=8,
                                    num_heads=2).to(dev).to(torch.bfloat16)
    assert blk._fusable_norm(torch.bfloat16)
