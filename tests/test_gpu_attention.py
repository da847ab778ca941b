"""GPU parity of the fused window-attention core against the CPU oracle.

Tolerances (written per the path's contract):
  fp32 activations: max |out - ref| <= 1e-5 and <= 1e-5 * max |ref| (+1e-6),
                    ref = oracle in float64 on the same fp32 inputs;
  bf16 activations: max |out - ref| <= 2e-2 * max |ref|, ref = oracle in fp32
                    on the same bf16-rounded inputs (the kernel rounds the
                    probabilities to bf16 before P@V, as autocast does).
The same mask given in closed form or as a dense tensor: bit for bit in fp32
(one kernel); in bf16 the closed-form path runs the ring kernel (bias and
masks added in raw-score units) and the dense one the window-tile kernel
(8x8 windows, 16-byte aligned mask) or the per-wave kernel, both adding the
terms after scaling, so they agree to rounding (see _assert_same_masking).
"""
import pytest
import torch

from oracle import swin_oracle as so
from terra_amd import kernels, utils, workloads
from terra_amd.kernels import ShiftMask, WindowGeometry, WindowMask

pytestmark = pytest.mark.gpu


def _inputs(B_, N, C, heads, ws, dtype, seed, qkv_scale=1.0):
    q = workloads.activations((B_, N, C), seed, torch.float32) * qkv_scale
    k = workloads.activations((B_, N, C), seed + 1, torch.float32) * qkv_scale
    v = workloads.activations((B_, N, C), seed + 2, torch.float32)
    # std 0.5 (not the reference init's 0.02): the bias then moves the outputs
    # by far more than the tolerance, so a dropped or mis-indexed bias fails.
    table = workloads.activations(((2 * ws - 1) ** 2, heads), seed + 3) * 0.5
    return q.to(dtype), k.to(dtype), v.to(dtype), table


def _check(out, ref, dtype):
    out = out.double().cpu()
    ref = ref.double()
    err = (out - ref).abs().max().item()
    scale = ref.abs().max().item()
    if dtype == torch.float32:
        assert err <= 1e-5 and err <= 1e-5 * scale + 1e-6, (err, scale)
    else:
        assert err <= 2e-2 * scale, (err, scale)
    return err / max(scale, 1e-30)


def _assert_same_masking(a, b, dtype):
    """Two kernels given the same mask in different forms.  fp32: one code
    path, bit-identical.  bf16: the closed-form-mask kernel adds bias and
    masks in raw-score units (bias / scale), the dense-mask kernel after
    scaling, so the fp32 logits differ by rounding: a probability may round
    to the other bf16 neighbour before P@V, moving an output by an ulp or two.
    A wrong mask (-100 on a logit) moves outputs by O(max|out|)."""
    if dtype == torch.float32:
        assert torch.equal(a, b)
    else:
        a, b = a.float(), b.float()
        tol = 2.0 ** -7 * b.abs() + 1e-2 * b.abs().max()
        assert ((a - b).abs() <= tol).all(), (a - b).abs().max().item()


def _run(dev, q, k, v, heads, ws, table, mask=None, n_real=None, **kw):
    return kernels.window_attention(q.to(dev), k.to(dev), v.to(dev), heads, (ws, ws), (q.shape[-1] // heads) ** -0.5,
                                    bias_table=None if table is None else table.to(dev), mask=mask, n_real=n_real,
                                    **kw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ws,C,heads", [(7, 96, 3), (8, 192, 6), (8, 768, 12), (7, 128, 4), (6, 64, 2),
                                         (8, 1024, 8), (7, 256, 2)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_core_no_mask(dev, dtype, ws, C, heads, with_bias):
    B_, N = 24, ws * ws
    q, k, v, table = _inputs(B_, N, C, heads, ws, dtype, 200)
    tab = table if with_bias else None
    out = _run(dev, q, k, v, heads, ws, tab)
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, tab, (ws, ws), compute_dtype=cd)
    _check(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,W,ws,s,C,heads", [(56, 56, 7, 3, 96, 3), (32, 48, 8, 4, 192, 6), (16, 24, 8, 4, 128, 2),
                                               (28, 42, 7, 3, 128, 4), (16, 24, 8, 4, 256, 2)])
def test_core_shift_mask_analytic_and_dense(dev, dtype, H, W, ws, s, C, heads):
    """The analytic mask (8x8 bf16 with an even head count: the ring kernel;
    otherwise the per-wave kernel) against the dense mask and the oracle."""
    nW = (H // ws) * (W // ws)
    B = 2
    q, k, v, table = _inputs(B * nW, ws * ws, C, heads, ws, dtype, 210, qkv_scale=2.0)
    dense = so.shift_mask(H, W, ws, s)
    analytic = ShiftMask(H, W, s, s, 0, H // ws, W // ws)
    out_a = _run(dev, q, k, v, heads, ws, table, mask=analytic)
    out_d = _run(dev, q, k, v, heads, ws, table, mask=dense.to(dev))
    _assert_same_masking(out_a, out_d, dtype)
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, table, (ws, ws), dense, compute_dtype=cd)
    _check(out_a, ref, dtype)


@pytest.mark.parametrize("C,heads,land", [(192, 6, False), (192, 6, True), (128, 2, False), (96, 3, False),
                                          (256, 2, False), (256, 2, True)])
@pytest.mark.parametrize("aligned", [True, False])
def test_core_random_dense_mask(dev, C, heads, land, aligned):
    """A random dense mask, asymmetric in (query, key) unlike the shift mask,
    so a transposed or shifted mask read fails: continuous offsets in [-8, 0)
    plus -100 on a third of the pairs, optionally with land keys on top.
    bf16 8x8 windows: an aligned mask runs the window-tile kernel with the
    mask staged in LDS (head dim 32 and 64), a mask at a one-float offset, an
    odd head count of dim 32, or head dim 128, the per-wave kernel."""
    H, W, ws = 32, 48, 8
    nW = (H // ws) * (W // ws)
    q, k, v, table = _inputs(2 * nW, 64, C, heads, ws, torch.bfloat16, 230, qkv_scale=2.0)
    gen = workloads.generator(231)
    dense = -8.0 * torch.rand(nW, 64, 64, generator=gen)
    dense = torch.where(torch.rand(nW, 64, 64, generator=gen) < 1 / 3, torch.full_like(dense, -100.0), dense)
    off = 0 if aligned else 1
    flat = torch.zeros(nW * 64 * 64 + 4, device=dev)
    emask = flat[off:off + nW * 64 * 64].view(nW, 64, 64)
    emask.copy_(dense.to(dev))
    assert (emask.data_ptr() % 16 == 0) == aligned
    mask, total = emask, dense
    if land:
        g = WindowGeometry(1, H, W, 1, ws, 4, 4)
        lm = workloads.land_mask(H, W, seed=9)
        mask = WindowMask(shift=emask, land_bits=utils.land_window_bits(lm.to(dev), g))
        total = so.fold_land(dense, so.land_key_flags(lm, ws, 4, 4))
    out = _run(dev, q, k, v, heads, ws, table, mask=mask)
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, table, (ws, ws), total,
                                   compute_dtype=torch.float32)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,W,ws,s,C,heads", [(32, 64, 8, 4, 192, 6), (28, 42, 7, 3, 128, 4), (32, 64, 8, 4, 256, 2)])
def test_core_land_bits(dev, dtype, H, W, ws, s, C, heads):
    land = workloads.land_mask(H, W, seed=9)
    g = WindowGeometry(1, H, W, 1, ws, s, s)
    bits = utils.land_window_bits(land.to(dev), g)
    nW = g.num_windows
    q, k, v, table = _inputs(nW, ws * ws, C, heads, ws, dtype, 220, qkv_scale=2.0)
    mask = WindowMask(shift=ShiftMask.from_geometry(g), land_bits=bits)
    out = _run(dev, q, k, v, heads, ws, table, mask=mask)
    total = so.fold_land(so.shift_mask(H, W, ws, s), so.land_key_flags(land, ws, s, s))
    out_dense = _run(dev, q, k, v, heads, ws, table, mask=total.to(dev))
    _assert_same_masking(out, out_dense, dtype)
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, table, (ws, ws), total, compute_dtype=cd)
    _check(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_core_padded_tokens_and_keys(dev, dtype):
    # a10: 49 real tokens of a 7x7 window carried in 64-token rows; bias and
    # mask cover the real 49 x 49 block; keys >= 49 get -10000.
    B_, N, C, heads, ws = 16, 64, 128, 4, 7
    q, k, v, table = _inputs(B_, N, C, heads, ws, dtype, 230)
    mask = so.shift_mask(14, 14, 7, 3)
    out = _run(dev, q, k, v, heads, ws, table, mask=mask.to(dev), n_real=49)
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, table, (ws, ws), mask, n_real=49,
                                   compute_dtype=cd)
    _check(out, ref, dtype)


@pytest.mark.parametrize("heads", [4, 2, 1])
def test_core_padded_keys_tile(dev, heads):
    """Padded keys without a dense mask: 49 real tokens of 7x7 windows in
    64-token rows, head dim 32, 64 and 128, bf16."""
    B_, N, C, ws = 16, 64, 128, 7
    q, k, v, table = _inputs(B_, N, C, heads, ws, torch.bfloat16, 235)
    out = _run(dev, q, k, v, heads, ws, table, n_real=49)
    ref = so.window_attention_core(q, k, v, heads, (C // heads) ** -0.5, table, (ws, ws), None, n_real=49,
                                   compute_dtype=torch.float32)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("C,heads", [(192, 6), (128, 4), (128, 2), (192, 3), (256, 2)])
@pytest.mark.parametrize("shifted", [False, True])
def test_core_tiny_scale(dev, C, heads, shifted):
    """A scale below 2^-20 on bf16 8x8 windows: the ring kernel adds bias and
    masks in raw-score units (bias / scale), so these shapes run the window-tile
    kernel instead (head dim 32 with 6 and 4 heads, head dim 64 with 2 and 3),
    and head dim 128 the per-wave kernel.
    q and k are scaled by 2^10 so the logits stay O(1) and the bias and mask
    still move the outputs."""
    H, W, ws, s = 16, 32, 8, 4
    nW = (H // ws) * (W // ws)
    scale = 2.0 ** -21
    q, k, v, table = _inputs(2 * nW, ws * ws, C, heads, ws, torch.bfloat16, 240, qkv_scale=1024.0)
    dense = so.shift_mask(H, W, ws, s) if shifted else None
    mask = ShiftMask(H, W, s, s, 0, H // ws, W // ws) if shifted else None
    out = kernels.window_attention(q.to(dev), k.to(dev), v.to(dev), heads, (ws, ws), scale,
                                   bias_table=table.to(dev), mask=mask)
    ref = so.window_attention_core(q, k, v, heads, scale, table, (ws, ws), dense, compute_dtype=torch.float32)
    _check(out, ref, torch.bfloat16)
    # The same call with the scale folded into q (exact: powers of two) and a
    # normal scale runs the ring kernel; the two kernels agree to rounding.
    out_ring = kernels.window_attention((q * 2.0 ** -11).to(dev), k.to(dev), v.to(dev), heads, (ws, ws), 2.0 ** -10,
                                        bias_table=table.to(dev), mask=mask)
    _assert_same_masking(out, out_ring, torch.bfloat16)


@pytest.mark.parametrize("dtype,ws,C,heads,scale", [
    (torch.bfloat16, 8, 192, 6, None),       # ring kernel, head dim 32
    (torch.bfloat16, 8, 128, 2, None),       # ring kernel, head dim 64
    (torch.bfloat16, 8, 256, 2, None),       # ring kernel, head dim 128
    (torch.bfloat16, 8, 256, 2, 2.0 ** -21),  # per-wave kernel, head dim 128
    (torch.float32, 8, 256, 2, None),        # per-wave kernel, fp32, head dim 128
    (torch.bfloat16, 8, 192, 6, 2.0 ** -21),  # window-tile kernel
    (torch.bfloat16, 7, 96, 3, None),        # per-wave kernel
    (torch.float32, 8, 64, 2, None),         # per-wave kernel, fp32
])
def test_core_nan_query_spoils_only_its_row(dev, dtype, ws, C, heads, scale):
    """A NaN in one query makes that query's row of that head NaN, as torch's
    softmax does (its row max is NaN); every other output is unchanged."""
    B_, N, D = 6, ws * ws, C // heads
    scale = D ** -0.5 if scale is None else scale
    q, k, v, table = _inputs(B_, N, C, heads, ws, dtype, 250)
    clean = kernels.window_attention(q.to(dev), k.to(dev), v.to(dev), heads, (ws, ws), scale,
                                     bias_table=table.to(dev)).float().cpu()
    w, i, h = 3, 5, heads - 1
    q_nan = q.clone()
    q_nan[w, i, h * D] = float("nan")
    out = kernels.window_attention(q_nan.to(dev), k.to(dev), v.to(dev), heads, (ws, ws), scale,
                                   bias_table=table.to(dev)).float().cpu()
    spoiled = torch.zeros_like(out, dtype=torch.bool)
    spoiled[w, i, h * D:(h + 1) * D] = True
    assert torch.isnan(out[spoiled]).all()
    assert not torch.isnan(out[~spoiled]).any()
    assert torch.equal(out[~spoiled], clean[~spoiled])


def test_core_strided_qkv_equals_contiguous(dev):
    B_, N, C, heads, ws = 32, 64, 192, 6, 8
    qkv = workloads.activations((B_, N, 3 * C), 240, torch.bfloat16).to(dev)
    table = (workloads.activations((225, heads), 241) * 0.5).to(dev)
    q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    a = kernels.window_attention(q, k, v, heads, (ws, ws), 32 ** -0.5, bias_table=table)
    b = kernels.window_attention(q.contiguous(), k.contiguous(), v.contiguous(), heads, (ws, ws), 32 ** -0.5,
                                 bias_table=table)
    assert torch.equal(a, b)


def test_core_deterministic(dev):
    B_, N, C, heads, ws = 64, 64, 192, 6, 8
    q, k, v, table = _inputs(B_, N, C, heads, ws, torch.bfloat16, 250)
    a = _run(dev, q, k, v, heads, ws, table)
    b = _run(dev, q, k, v, heads, ws, table)
    assert torch.equal(a, b)


def test_core_reference_autocast_distance(dev):
    """The kernel sits at least as close to the fp32 restatement as the
    reference's own bf16 autocast op sequence does (reported, bounded)."""
    B_, N, C, heads, ws = 64, 64, 192, 6, 8
    q, k, v, table = _inputs(B_, N, C, heads, ws, torch.bfloat16, 260, qkv_scale=2.0)
    out = _run(dev, q, k, v, heads, ws, table).double().cpu()
    ref = so.window_attention_core(q, k, v, heads, 32 ** -0.5, table, (ws, ws)).double()
    ac = so.window_attention_autocast_bf16(q, k, v, heads, 32 ** -0.5, table, (ws, ws)).double()
    e_kernel = (out - ref).abs().max().item()
    e_ref = (ac - ref).abs().max().item()
    assert e_kernel <= e_ref * 1.5 + 1e-6, (e_kernel, e_ref)


@pytest.mark.parametrize("name", ["c3", "c5", "g1"])
def test_core_full_size_sampled_windows(dev, name):
    """Full-size launch (every window computed); a seeded sample of windows is
    checked against the oracle, and the whole output must be finite."""
    cfg = workloads.CONFIGS[name]
    B_, N, C, heads, ws = cfg.num_windows, cfg.tokens, cfg.channels, cfg.heads, cfg.window
    q = workloads.activations((B_, N, C), 270, torch.bfloat16)
    k = workloads.activations((B_, N, C), 271, torch.bfloat16)
    v = workloads.activations((B_, N, C), 272, torch.bfloat16)
    table = workloads.activations(((2 * ws - 1) ** 2, heads), 273) * 0.5
    g = WindowGeometry(cfg.batch, cfg.height, cfg.width, 1, ws, cfg.shift, cfg.shift, cfg.pad,
                       cfg.win_row_begin, cfg.win_rows, cfg.valid)
    land = workloads.land_mask(cfg.height, cfg.width, seed=274)
    bits = utils.land_window_bits(land.to(dev), WindowGeometry(1, cfg.height, cfg.width, 1, ws, cfg.shift,
                                                                cfg.shift, cfg.pad, cfg.win_row_begin,
                                                                cfg.win_rows, cfg.valid))
    mask = WindowMask(shift=ShiftMask.from_geometry(g), land_bits=bits)
    out = _run(dev, q, k, v, heads, ws, table, mask=mask)
    assert torch.isfinite(out.float()).all()
    # dense mask of the emitted windows, for the sampled ones
    fh, fw = g.frame_h, g.frame_w
    full = so.shift_mask(fh, fw, ws, cfg.shift).view(fh // ws, fw // ws, N, N)
    rows = g.rows
    shift_m = full[g.win_row_begin:g.win_row_begin + rows].reshape(rows * (fw // ws), N, N)
    flags = so.land_key_flags(land, ws, cfg.shift, cfg.shift, cfg.pad, cfg.win_row_begin, cfg.win_rows, cfg.valid)
    total = so.fold_land(shift_m, flags)
    per_img = g.windows_per_image
    gen = workloads.generator(275)
    sample = torch.randperm(B_, generator=gen)[:384]
    # always include the boundary windows of the last row / column
    sample = torch.unique(torch.cat([sample, torch.arange(per_img - fw // ws, per_img),
                                     torch.arange(fw // ws - 1, per_img, fw // ws)]))
    # window w uses total[w % per_img]; one mask per sampled window
    ref = so.window_attention_core(q[sample], k[sample], v[sample], heads, (C // heads) ** -0.5, table, (ws, ws),
                                   total[sample % per_img])
    _check(out.cpu()[sample], ref, torch.bfloat16)


def test_kernels_against_committed_golden_fixture(dev):
    """The committed tiny SW-MSA fixture (tests/golden/swin_tiny.npz): partition
    bit-exact, fp32 attention within 1e-5 of the stored float64 target."""
    import os

    import numpy as np

    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "swin_tiny.npz"))
    B, H, W, C, nH, ws, s = (int(v) for v in z["meta"])
    x = torch.from_numpy(z["x"]).to(dev)
    g = WindowGeometry(B, H, W, C, ws, s, s)
    win = kernels.swin_partition(x, g)
    assert np.array_equal(win.cpu().numpy(), z["windows"])
    bits = utils.land_window_bits(torch.from_numpy(z["land"]).to(dev), WindowGeometry(1, H, W, 1, ws, s, s))
    qkv = torch.from_numpy(z["qkv"]).to(dev)
    out = kernels.window_attention(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], nH, (ws, ws),
                                   (C // nH) ** -0.5, bias_table=torch.from_numpy(z["table"]).to(dev),
                                   mask=WindowMask(shift=ShiftMask.from_geometry(g), land_bits=bits))
    err = np.abs(out.cpu().double().numpy() - z["o"].astype(np.float64)).max()
    assert err <= 1e-5, err


# ---- windows of more than 64 tokens (TERRA's ws-32 configuration) ----------

@pytest.mark.parametrize("ws,C,heads,B_", [(32, 1024, 8, 2), (32, 512, 8, 3), (16, 256, 2, 4), (32, 256, 2, 1)])
def test_flash_large_windows_match_oracle(dev, ws, C, heads, B_):
    """ws x ws windows (1024 tokens at ws 32), head dim 128 or 64, no bias and
    no mask (credit_hierarchical_swin_correctness_seq.yaml:21-30 turns both
    off): the flash kernel's online softmax against the oracle's full-row
    softmax, bf16 tolerance.  Scores are spread (q, k scaled by 2) so that the
    running max moves across key tiles and the rescaling is exercised."""
    N = ws * ws
    q, k, v, _ = _inputs(B_, N, C, heads, ws, torch.bfloat16, 700 + ws, qkv_scale=2.0)
    scale = (C // heads) ** -0.5
    out = kernels.window_attention(q.to(dev), k.to(dev), v.to(dev), heads, (ws, ws), scale)
    ref = so.window_attention_core(q.float(), k.float(), v.float(), heads, scale, window_size=(ws, ws))
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("wh,ww,C,heads,B_", [(24, 16, 256, 2, 2), (16, 8, 512, 4, 3)])
def test_flash_non_square_windows_match_oracle(dev, wh, ww, C, heads, B_):
    """Non-square windows, a token count that is an odd multiple of 128
    (24 x 16), and 16 x 8, the smallest window the flash kernel serves (one
    query block, two key tiles)."""
    N = wh * ww
    q, k, v, _ = _inputs(B_, N, C, heads, max(wh, ww), torch.bfloat16, 730 + N, qkv_scale=2.0)
    scale = (C // heads) ** -0.5
    out = kernels.window_attention(q.to(dev), k.to(dev), v.to(dev), heads, (wh, ww), scale)
    ref = so.window_attention_core(q.float(), k.float(), v.float(), heads, scale, window_size=(wh, ww))
    _check(out, ref, torch.bfloat16)


def test_flash_strided_qkv_and_row_independence(dev):
    """q | k | v as column blocks of one [B_, N, 3C] tensor (the module's
    layout), and a window's result independent of the others."""
    ws, C, heads, B_ = 32, 256, 2, 3
    N = ws * ws
    qkv = workloads.activations((B_, N, 3 * C), 711, torch.bfloat16)
    scale = (C // heads) ** -0.5
    qd = qkv.to(dev)
    out = kernels.window_attention(qd[..., :C], qd[..., C:2 * C], qd[..., 2 * C:], heads, (ws, ws), scale)
    ref = so.window_attention_core(qkv[..., :C].float(), qkv[..., C:2 * C].float(), qkv[..., 2 * C:].float(), heads,
                                   scale, window_size=(ws, ws))
    _check(out, ref, torch.bfloat16)
    one = kernels.window_attention(qd[1:2, :, :C], qd[1:2, :, C:2 * C], qd[1:2, :, 2 * C:], heads, (ws, ws), scale)
    assert torch.equal(one.cpu(), out[1:2].cpu())


def test_flash_rejects_what_it_does_not_serve(dev):
    ws, C, heads = 32, 256, 2
    N = ws * ws
    q, k, v, table = _inputs(1, N, C, heads, ws, torch.bfloat16, 720)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    with pytest.raises(ValueError, match="no relative-position bias and no mask"):
        kernels.window_attention(qd, kd, vd, heads, (ws, ws), 0.1, bias_table=table.to(dev))
    with pytest.raises(ValueError, match="bf16 only"):
        kernels.window_attention(qd.float(), kd.float(), vd.float(), heads, (ws, ws), 0.1)
    q12, k12, v12, _ = _inputs(1, 144, C, heads, 12, torch.bfloat16, 721)
    with pytest.raises(ValueError, match="multiple of 128"):
        kernels.window_attention(q12.to(dev), k12.to(dev), v12.to(dev), heads, (12, 12), 0.1)


@pytest.mark.parametrize("layer", [0, 1])
def test_block_ws32_without_bias_or_mask(dev, layer):
    """A block of TERRA's ws-32 configuration (C and heads scaled down to 256
    and 2, head dim 128 as in the config), W-MSA and SW-MSA (shift 16, no
    mask), through the module: LayerNorm gather, q/k/v, the flash core, proj,
    reverse + residual (as one linear-kernel launch: C % 256 == 0, every
    frame window emitted), against the oracle block."""
    from helpers import assert_block_matches, gain_block, params_of
    from terra_amd.transformer import SequentialSwinTransformer
    C, heads, ws, H, W = 256, 2, 32, 64, 96
    blk = SequentialSwinTransformer(layer_idx=layer, height=H, width=W, embedding_dim=C, window_size=ws,
                                    num_heads=heads, use_attn_mask=False, use_relative_position_bias=False)
    workloads.init_block_params(blk, layer)
    gain_block(blk)
    blk = blk.to(dev).to(torch.bfloat16)
    x = workloads.activations((1, H * W, C), 730 + layer, torch.bfloat16)
    with torch.no_grad():
        y = blk(x.to(dev))
    ref = so.swin_block_attention(x, H, W, ws, blk.shift_size, heads, params_of(blk), use_attn_mask=False)
    assert_block_matches(y, ref, x, 2e-2, 3e-2)
