"""Pins the CPU oracle (oracle/swin_oracle.py) before anything is checked against it.

Each oracle function is compared with something it cannot share a mistake
with: brute-force coordinate loops (oracle/brute.py), closed forms and known
answers, library special cases, and the reference's own unit-test vector.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import swin_oracle as so


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)


GRIDS = [  # (B, H, W, C, ws, shift)
    (2, 14, 21, 3, 7, 3),
    (1, 16, 24, 5, 8, 4),
    (2, 14, 14, 2, 7, 0),
    (1, 12, 18, 4, 6, 3),
]


@pytest.mark.parametrize("B,H,W,C,ws,s", GRIDS)
def test_roll_partition_matches_brute(B, H, W, C, ws, s):
    x = _rand((B, H, W, C), 1)
    got = so.roll_partition(x, ws, s).numpy()
    want = brute.partition(x.numpy(), ws, shift_h=s, shift_w=s)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("B,H,W,C,ws,s", GRIDS)
def test_reverse_unroll_matches_brute_and_inverts(B, H, W, C, ws, s):
    x = _rand((B, H, W, C), 2)
    win = so.roll_partition(x, ws, s)
    y = so.reverse_unroll(win, ws, H, W, s)
    assert torch.equal(y, x)  # reverse o partition == id, roll(+s) o roll(-s) == id
    want = brute.reverse(win.numpy(), B, H, W, ws, shift_h=s, shift_w=s)
    assert np.array_equal(y.numpy(), want)


def test_roll_matches_distributed_shift_formula():
    # core/parallel/layout_transform.py:341-348 states the same map as
    # shifted_i = (gi - s) mod H for the position a global row gi lands on.
    H, W, s = 16, 24, 4
    x = torch.arange(H * W, dtype=torch.float64).view(1, H, W, 1)
    shifted = torch.roll(x, (-s, -s), (1, 2))
    for gi in range(H):
        for gj in range(W):
            assert shifted[0, (gi - s) % H, (gj - s) % W, 0] == x[0, gi, gj, 0]


FRAMES = [  # (B, H, W, ws, shift_h, shift_w, pad, win_row_begin, win_rows, valid)
    (1, 13, 21, 7, 3, 3, (0, 1, 0, 0), 0, None, None),
    (2, 10, 17, 4, 2, 1, (1, 1, 2, 1), 1, 2, None),
    (2, 20, 16, 8, 4, 4, (0, 4, 0, 0), 0, 2, (3, 4)),
    (1, 16, 16, 8, 4, 4, (0, 8, 0, 0), 0, 2, (1, 3)),
]


@pytest.mark.parametrize("B,H,W,ws,sh,sw,pad,r0,rows,valid", FRAMES)
def test_partition_frame_matches_brute(B, H, W, ws, sh, sw, pad, r0, rows, valid):
    x = _rand((B, H, W, 3), 3)
    got = so.partition_frame(x, ws, sh, sw, pad, r0, rows, valid).numpy()
    want = brute.partition(x.numpy(), ws, shift_h=sh, shift_w=sw, pad=pad, win_row_begin=r0,
                           win_rows=rows, valid=valid)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("B,H,W,ws,sh,sw,pad,r0,rows,valid", FRAMES)
def test_reverse_frame_matches_brute(B, H, W, ws, sh, sw, pad, r0, rows, valid):
    x = _rand((B, H, W, 3), 4)
    res = _rand((B, H, W, 3), 5)
    win = so.partition_frame(x, ws, sh, sw, pad, r0, rows, valid)
    win = win + _rand(win.shape, 6)  # arbitrary window contents
    got = so.reverse_frame(win, B, H, W, ws, sh, sw, pad, r0, rows, valid, residual=res).numpy()
    want = brute.reverse(win.numpy(), B, H, W, ws, residual=res.numpy(), shift_h=sh, shift_w=sw, pad=pad,
                         win_row_begin=r0, win_rows=rows, valid=valid)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wh,ww", [(7, 7), (8, 8), (6, 6), (3, 5)])
def test_relative_position_index(wh, ww):
    idx = so.relative_position_index((wh, ww))
    assert np.array_equal(idx.numpy(), brute.relative_index(wh, ww))
    centre = (wh - 1) * (2 * ww - 1) + (ww - 1)
    assert torch.all(idx + idx.T == 2 * centre)
    assert torch.all(idx.diagonal() == centre)
    # decoding idx gives back the coordinate difference of the two tokens
    n = wh * ww
    hi = torch.arange(n) // ww
    wi = torch.arange(n) % ww
    dh, dw = torch.div(idx, 2 * ww - 1, rounding_mode="floor") - (wh - 1), idx % (2 * ww - 1) - (ww - 1)
    assert torch.equal(dh, hi[:, None] - hi[None, :])
    assert torch.equal(dw, wi[:, None] - wi[None, :])


def test_relative_position_index_known_values():
    i7 = so.relative_position_index((7, 7))
    assert i7[0, 0] == 84 and i7.max() == 168 and i7[48, 0] == 168 and i7.min() == 0 and i7[0, 48] == 0
    i8 = so.relative_position_index((8, 8))
    assert i8[0, 0] == 112 and i8.max() == 224 and i8[63, 0] == 224 and i8[0, 63] == 0


def test_bias_gather_matches_loops():
    table = _rand((169, 3), 7)
    bias = so.relative_position_bias(table, (7, 7))
    idx = brute.relative_index(7, 7)
    for h in range(3):
        for i in range(0, 49, 5):
            for j in range(0, 49, 3):
                assert bias[h, i, j] == table[idx[i, j], h]


@pytest.mark.parametrize("H,W,ws,s", [(14, 21, 7, 3), (16, 24, 8, 4), (56, 56, 7, 3), (24, 16, 8, 2)])
def test_shift_mask_matches_brute(H, W, ws, s):
    m = so.shift_mask(H, W, ws, s)
    assert np.array_equal(m.numpy(), brute.shift_mask(H, W, ws, s))
    assert torch.equal(m, m.transpose(1, 2))
    assert torch.all(m.diagonal(dim1=1, dim2=2) == 0)
    nww = W // ws
    interior = [w for w in range(m.shape[0]) if w // nww < H // ws - 1 and w % nww < nww - 1]
    assert torch.all(m[interior] == 0)


def test_shift_mask_known_counts():
    m7 = so.shift_mask(56, 56, 7, 3)  # 8 x 8 windows
    assert int((m7[7 * 8 + 0] == -100).sum()) == 1176      # last row, not last column
    assert int((m7[7 * 8 + 7] == -100).sum()) == 1776      # bottom-right
    assert int((m7[0 * 8 + 7] == -100).sum()) == 1176      # last column, not last row
    m8 = so.shift_mask(32, 32, 8, 4)
    assert int((m8[3 * 4 + 0] == -100).sum()) == 2048
    assert int((m8[3 * 4 + 3] == -100).sum()) == 3072
    assert set(torch.unique(m8).tolist()) == {-100.0, 0.0}


def test_land_flags_and_fold():
    g = torch.Generator().manual_seed(11)
    land = torch.rand(16, 24, generator=g) < 0.3
    flags = so.land_key_flags(land, 8, 4, 4)
    src = brute.frame_source(1, 16, 24, 8, shift_h=4, shift_w=4)
    want = np.array([bool(land[s[1], s[2]]) if s is not None else False for s in src]).reshape(-1, 64)
    assert np.array_equal(flags.numpy(), want)
    m = so.shift_mask(16, 24, 8, 4)
    tot = so.fold_land(m, flags)
    for w in range(tot.shape[0]):
        for j in range(64):
            assert torch.equal(tot[w, :, j], m[w, :, j] + (-100.0 if want[w, j] else 0.0))


@pytest.mark.parametrize("with_bias,with_mask,n_real", [(False, False, None), (True, False, None),
                                                       (True, True, None), (True, True, 40)])
def test_attention_core_matches_float64_brute(with_bias, with_mask, n_real):
    B_, N, C, nH = 4, 49, 16, 2
    q, k, v = _rand((B_, N, C), 20), _rand((B_, N, C), 21), _rand((B_, N, C), 22)
    table = _rand((169, nH), 23) if with_bias else None
    mask = so.shift_mask(14, 14, 7, 3).double() if with_mask else None
    scale = (C // nH) ** -0.5
    got = so.window_attention_core(q, k, v, nH, scale, table, (7, 7), mask, n_real, compute_dtype=torch.float64)
    bias = so.relative_position_bias(table, (7, 7)).numpy() if with_bias else None
    want = brute.attention(q.numpy(), k.numpy(), v.numpy(), nH, scale, bias,
                           None if mask is None else mask.numpy(), n_real)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)


def test_attention_core_equals_sdpa_without_bias_and_mask():
    B_, N, C, nH = 6, 64, 64, 2
    q, k, v = _rand((B_, N, C), 30), _rand((B_, N, C), 31), _rand((B_, N, C), 32)
    got = so.window_attention_core(q, k, v, nH, (C // nH) ** -0.5, compute_dtype=torch.float64)
    split = lambda t: t.view(B_, N, nH, C // nH).transpose(1, 2)
    want = F.scaled_dot_product_attention(split(q), split(k), split(v)).transpose(1, 2).reshape(B_, N, C)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_attention_core_gradient_is_the_derivative():
    # Backward parity (row f3) takes torch autograd of this restatement as the
    # reference gradient: finite differences pin it for q, k, v and the bias
    # table, with the shift mask on.
    B_, N, C, nH = 4, 16, 8, 2
    q, k, v = (_rand((B_, N, C), s).requires_grad_(True) for s in (50, 51, 52))
    table = _rand((49, nH), 53).requires_grad_(True)
    mask = so.shift_mask(8, 8, 4, 2).double()
    fn = lambda q_, k_, v_, t_: so.window_attention_core(q_, k_, v_, nH, 0.35, t_, (4, 4), mask,  # noqa: E731
                                                         compute_dtype=torch.float64)
    assert torch.autograd.gradcheck(fn, (q, k, v, table), eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("H,pad,r0,rows,valid", [(16, (0, 0, 0, 0), 0, None, None),
                                                  (20, (0, 4, 0, 0), 1, 2, (1, 7))])
def test_partition_and_reverse_are_adjoint(H, pad, r0, rows, valid):
    # <partition(x), w> == <x, reverse(w)>: the gradient of partition is
    # reverse and vice versa (what the autograd wrappers of the kernels use).
    B, W, C = 2, 32, 3
    x = _rand((B, H, W, C), 60)
    win = so.partition_frame(x, 8, 4, 4, pad, r0, rows, valid)
    w = _rand(tuple(win.shape), 61)
    lhs = (win * w).sum().item()
    rhs = (x * so.reverse_frame(w, B, H, W, 8, 4, 4, pad, r0, rows, valid)).sum().item()
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(lhs))


def test_padded_keys_reduce_to_real_window():
    # keys >= n_real get -10000, so their weight underflows to exactly 0: the
    # result on the real rows equals attention over the first n_real tokens.
    B_, N, C, nH, nr = 3, 64, 32, 1, 49
    q, k, v = _rand((B_, N, C), 40), _rand((B_, N, C), 41), _rand((B_, N, C), 42)
    got = so.window_attention_core(q, k, v, nH, 0.2, n_real=nr, compute_dtype=torch.float64)
    ref = so.window_attention_core(q[:, :nr], k[:, :nr], v[:, :nr], nH, 0.2, compute_dtype=torch.float64)
    torch.testing.assert_close(got[:, :nr], ref, rtol=1e-12, atol=1e-12)


def test_ragged_row_major_reference_vector():
    # tests/unit/test_window_assignment.py:10-23 of the reference
    per_rank = so.ragged_row_major(2, 5, 4)
    ids = [[r * 5 + c for r, c in chunk] for chunk in per_rank]
    assert ids == [[0, 1], [2, 3, 4], [5, 6], [7, 8, 9]]


# ---- committed golden fixtures (tests/golden, written by make_golden.py) ----

import json as _json
import os as _os

_GOLDEN = _os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "golden")


def test_known_answers_fixture():
    ka = _json.load(open(_os.path.join(_GOLDEN, "known_answers.json")))
    ids = [[r * 5 + c for r, c in chunk] for chunk in so.ragged_row_major(2, 5, 4)]
    assert ids == ka["ragged_row_major_2x5_m4"]
    i7, i8 = so.relative_position_index((7, 7)), so.relative_position_index((8, 8))
    assert ka["rel_index_7x7"] == {"i00": 84, "max": 168, "i_48_0": 168, "i_0_48": 0}
    assert ka["rel_index_8x8"] == {"i00": 112, "max": 224, "i_63_0": 224, "i_0_63": 0}
    assert int(i7[48, 0]) == 168 and int(i8[0, 0]) == 112
    assert ka["shift_mask_ws7_s3_counts"] == {"last_row": 1176, "corner": 1776}
    assert ka["shift_mask_ws8_s4_counts"] == {"last_row": 2048, "corner": 3072}


def test_tiny_fixture_oracle_has_not_drifted():
    z = np.load(_os.path.join(_GOLDEN, "swin_tiny.npz"))
    B, H, W, C, nH, ws, s = (int(v) for v in z["meta"])
    x = torch.from_numpy(z["x"]).double()
    win = so.roll_partition(x, ws, s)
    assert np.array_equal(win.float().numpy(), z["windows"])
    land = torch.from_numpy(z["land"])
    mask = so.fold_land(so.shift_mask(H, W, ws, s).double(), so.land_key_flags(land, ws, s, s))
    assert np.array_equal(mask.float().numpy(), z["mask"])
    qkv = torch.from_numpy(z["qkv"]).double()
    o = so.window_attention_core(qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:], nH, (C // nH) ** -0.5,
                                 torch.from_numpy(z["table"]).double(), (ws, ws), mask,
                                 compute_dtype=torch.float64)
    np.testing.assert_allclose(o.numpy(), z["o"], rtol=1e-6, atol=1e-7)
    # and the float64 brute force agrees with the stored target
    bias = so.relative_position_bias(torch.from_numpy(z["table"]).double(), (ws, ws)).numpy()
    want = brute.attention(qkv[..., :C].numpy(), qkv[..., C:2 * C].numpy(), qkv[..., 2 * C:].numpy(), nH,
                           (C // nH) ** -0.5, bias, mask.numpy())
    np.testing.assert_allclose(want, z["o"], rtol=1e-6, atol=1e-7)


# ----------------------------------------------------------------------------
# MLP half (models/mlp.py:152-172)
# ----------------------------------------------------------------------------

def test_gelu_known_values_and_torch():
    # Phi(1) = 0.8413447460685429, Phi(-1) = 0.15865525393145707 (normal table)
    assert abs(brute.gelu(1.0) - 0.8413447460685429) < 1e-15
    assert abs(brute.gelu(-1.0) + 0.15865525393145707) < 1e-15
    assert brute.gelu(0.0) == 0.0 and brute.gelu(40.0) == 40.0 and brute.gelu(-40.0) == 0.0
    xs = torch.linspace(-9, 9, 1001, dtype=torch.float64)
    ref = torch.tensor([brute.gelu(float(v)) for v in xs], dtype=torch.float64)
    assert torch.allclose(F.gelu(xs), ref, rtol=1e-14, atol=1e-15)


def test_bf16_round_matches_torch_cast():
    bits = np.arange(0, 1 << 32, 65537, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    ours = brute.bf16_round(f)
    theirs = torch.from_numpy(f.copy()).bfloat16().float().numpy()
    fin = np.isfinite(f)
    assert np.array_equal(ours[fin].view(np.uint32), theirs[fin].view(np.uint32))
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 and rounds to 1
    assert brute.bf16_round(np.float32(1 + 2 ** -8)) == 1.0
    assert brute.bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)


def _mlp_params(C, hid, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return {
        "norm2.weight": 1 + 0.1 * torch.randn(C, generator=g, dtype=dtype),
        "norm2.bias": 0.1 * torch.randn(C, generator=g, dtype=dtype),
        "fc1.weight": torch.randn(hid, C, generator=g, dtype=dtype) / C ** 0.5,
        "fc1.bias": 0.1 * torch.randn(hid, generator=g, dtype=dtype),
        "fc2.weight": torch.randn(C, hid, generator=g, dtype=dtype) / hid ** 0.5,
        "fc2.bias": 0.1 * torch.randn(C, generator=g, dtype=dtype),
    }


@pytest.mark.parametrize("use_ln", [True, False])
def test_mlp_matches_token_loops(use_ln):
    C, hid = 6, 10  # hid != C: a transposed weight cannot go unnoticed
    p = _mlp_params(C, hid, 3)
    x = _rand((2, 3, C), 4)
    ref = brute.mlp(x.numpy(), {k: v.numpy() for k, v in p.items()}, use_layernorm=use_ln)
    got = so.mlp(x, p, use_layernorm=use_ln).double()
    assert np.allclose(got.numpy(), ref, rtol=1e-5, atol=1e-6)  # so.mlp computes in float32


@pytest.mark.parametrize("use_ln", [True, False])
def test_mlp_bf16_matches_token_loops(use_ln):
    C, hid = 8, 12
    p = {k: v.bfloat16().double() if "weight" in k and "norm" not in k else v for k, v in _mlp_params(C, hid, 5).items()}
    x = _rand((5, C), 6).bfloat16().double()
    ref = brute.mlp(x.numpy(), {k: v.numpy() for k, v in p.items()}, use_layernorm=use_ln, round_bf16=True)
    got = so.mlp_bf16(x, p, use_layernorm=use_ln).numpy()
    # identical rounding points: equal except where float64 summation-order
    # noise crosses a bf16 rounding boundary (then one bf16 ulp)
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)
    assert np.mean(got == ref) > 0.95
    # and within bf16 tolerance of the unrounded float64 module
    exact = brute.mlp(x.numpy(), {k: v.numpy() for k, v in p.items()}, use_layernorm=use_ln)
    assert np.max(np.abs(got - exact)) <= 3e-2 * np.max(np.abs(exact))


# ---- the bf16 autocast restatement and the block composition ----

def _bf16_agree(a: np.ndarray, b: np.ndarray) -> bool:
    """Within one bf16 rounding of each other (2^-7 of the value) plus 2^-9 of
    the largest output: a logit or probability that lands on the other side of
    a bf16 rounding boundary (fp32 vs float64 accumulation) moves an output by
    about that much."""
    return bool((np.abs(a - b) <= 2.0 ** -7 * np.abs(b) + 2.0 ** -9 * np.abs(b).max()).all())


@pytest.mark.parametrize("with_bias,with_mask", [(False, False), (True, True)])
def test_autocast_core_matches_bf16_loops(with_bias, with_mask):
    """window_attention_autocast_bf16 against loops that round to bf16 at the
    same points (q * scale, q.k, probabilities, output).  Logits of standard
    deviation ~3 make the rounding of q.k visible: the fp32 core, which rounds
    only its inputs, must fail the same check."""
    B_, N, C, nH, ws = 4, 16, 16, 2, 4
    q, k, v = (_rand((B_, N, C), s, torch.float32) * f for s, f in ((70, 2.5), (71, 2.5), (72, 1.0)))
    table = _rand(((2 * ws - 1) ** 2, nH), 73, torch.float32) if with_bias else None
    mask = so.shift_mask(8, 8, ws, 2) if with_mask else None
    scale = (C // nH) ** -0.5
    got = so.window_attention_autocast_bf16(q, k, v, nH, scale, table, (ws, ws), mask).double().numpy()
    bias = so.relative_position_bias(table, (ws, ws)).numpy() if with_bias else None
    want = brute.attention_autocast_bf16(q.numpy(), k.numpy(), v.numpy(), nH, scale, bias,
                                         None if mask is None else mask.numpy())
    assert _bf16_agree(got, want)
    assert np.mean(got == want) >= 0.95  # most outputs bit-equal
    fp32 = so.window_attention_core(q.bfloat16(), k.bfloat16(), v.bfloat16(), nH, scale, table, (ws, ws), mask)
    assert not _bf16_agree(fp32.double().numpy(), want)


BLOCK_CASES = [  # (B, H, W, C, heads, ws, shift, land, pad, r0, rows, valid, ln, bias)
    (2, 8, 12, 8, 2, 4, 2, False, (0, 0, 0, 0), 0, None, None, True, True),
    (1, 12, 8, 8, 2, 4, 0, True, (0, 0, 0, 0), 0, None, None, True, True),
    (1, 10, 12, 6, 3, 4, 2, True, (1, 1, 0, 4), 0, None, None, True, False),
    (2, 14, 8, 8, 2, 4, 2, True, (0, 2, 0, 0), 1, 2, (1, 3), True, True),
    (1, 8, 8, 8, 1, 4, 2, False, (0, 0, 0, 0), 0, None, None, False, True),
]


@pytest.mark.parametrize("case", BLOCK_CASES)
def test_block_oracle_matches_token_loops(case):
    """swin_block_attention (LayerNorm, pad / roll / partition, q/k/v, core with
    bias, shift and land masks, proj, reverse, residual) against the float64
    token loops of brute.swin_block, which share none of its reshapes, mask
    construction or index code; slab, pad-window and padded-frame cases
    included."""
    B, H, W, C, nH, ws, s, land_on, pad, r0, rows, valid, ln, bias = case
    x = _rand((B, H, W, C), 80)
    p = {"norm1.weight": 1.0 + 0.2 * _rand((C,), 81), "norm1.bias": 0.2 * _rand((C,), 82),
         "attn.proj.weight": _rand((C, C), 83) * 0.4, "attn.proj.bias": _rand((C,), 84) * 0.1}
    for i, n in enumerate("qkv"):
        p[f"attn.{n}_linear.weight"] = _rand((C, C), 85 + i) * 0.6
        p[f"attn.{n}_linear.bias"] = _rand((C,), 88 + i) * 0.1
    if bias:
        p["attn.relative_position_bias_table"] = _rand(((2 * ws - 1) ** 2, nH), 91)
    land = (_rand((H, W), 92) > 0.4) if land_on else None
    got = so.swin_block_attention(x.view(B, H * W, C), H, W, ws, s, nH, p, land=land, pad=pad, win_row_begin=r0,
                                  win_rows=rows, valid=valid, use_layernorm=ln, compute_dtype=torch.float64)
    want = brute.swin_block(x.numpy(), {k_: v_.numpy() for k_, v_ in p.items()}, ws, s, nH,
                            land=None if land is None else land.numpy(), use_layernorm=ln, pad=pad,
                            win_row_begin=r0, win_rows=rows, valid=valid)
    np.testing.assert_allclose(got.view(B, H, W, C).numpy(), want, rtol=1e-10, atol=1e-10)
    assert not np.allclose(want, x.numpy())  # the attention half changed the tokens it owns


def test_linear_autocast_bf16_known_answers():
    """linear_autocast_bf16: small integers give the exact integer product;
    1 + 2^-8 (exact in the fp32 accumulator) rounds to even, 1.0, in bf16, and
    a bias of 1 + 2^-8 is rounded to bf16 (1.0) before it is added."""
    gen = torch.Generator().manual_seed(93)
    x = torch.randint(-3, 4, (5, 7), generator=gen).float()
    w = torch.randint(-3, 4, (4, 7), generator=gen).float()
    b = torch.randint(-5, 6, (4,), generator=gen).float()
    got = so.linear_autocast_bf16(x, w, b)
    assert got.dtype == torch.bfloat16
    want = x.long() @ w.long().t() + b.long()
    assert torch.equal(got.float(), want.float())
    one = so.linear_autocast_bf16(torch.tensor([[1.0, 2.0 ** -8]]), torch.tensor([[1.0, 1.0]]), None)
    assert one.item() == 1.0
    three_ulp = so.linear_autocast_bf16(torch.tensor([[1.0, 3 * 2.0 ** -8]]), torch.tensor([[1.0, 1.0]]), None)
    assert three_ulp.item() == 1.0 + 2.0 ** -6  # 1 + 3/256 rounds to the even neighbour 1 + 4/256
    biased = so.linear_autocast_bf16(torch.tensor([[0.0]]), torch.tensor([[1.0]]), torch.tensor([1.0 + 2.0 ** -8]))
    assert biased.item() == 1.0


def test_block_autocast_composition_exact_regime():
    """swin_block_attention_autocast_bf16 equals the fp32 block oracle where
    every value it rounds is exact in bf16: rows of +-1 with zero mean (a
    LayerNorm output of exactly +-1 with eps 0), q and k weights zero (uniform
    probabilities 2^-6), v and proj the identity, zero biases and table; o is
    then a window mean k / 64 and y = x + o, both exact.  A dropped residual,
    a transposed or missing proj, or a wrong window map changes y.  In a
    generic case (random weights, bias table, shift mask, land) the two agree
    to bf16 tolerance but not bit for bit (the roundings are really there)."""
    B, H, W, C, nH, ws, s = 1, 8, 8, 8, 2, 4, 2
    gen = torch.Generator().manual_seed(94)
    half = torch.randint(0, 2, (B, H, W, C // 2), generator=gen).float() * 2 - 1
    x = torch.cat([half, -half], -1)[..., torch.randperm(C, generator=gen)]  # +-1, zero mean per token
    eye = torch.eye(C)
    zeros = torch.zeros(C, C)
    p = {"norm1.weight": torch.ones(C), "norm1.bias": torch.zeros(C), "attn.proj.weight": eye,
         "attn.proj.bias": torch.zeros(C), "attn.q_linear.weight": zeros, "attn.q_linear.bias": torch.zeros(C),
         "attn.k_linear.weight": zeros, "attn.k_linear.bias": torch.zeros(C), "attn.v_linear.weight": eye,
         "attn.v_linear.bias": torch.zeros(C), "attn.relative_position_bias_table": torch.zeros((2 * ws - 1) ** 2, nH)}
    xs = x.view(B, H * W, C)
    got = so.swin_block_attention_autocast_bf16(xs, H, W, ws, 0, nH, p, eps=0.0).float()
    win_mean = so.partition_frame(x, ws).mean(1, keepdim=True).expand(-1, ws * ws, -1)
    want = x + so.reverse_frame(win_mean, B, H, W, ws)
    assert torch.equal(got.view(B, H, W, C), want)
    # the fp32 oracle: identical in this regime up to its LayerNorm eps
    ref = so.swin_block_attention(xs, H, W, ws, 0, nH, p)
    assert (ref.view(B, H, W, C) - want).abs().max().item() <= 1e-4
    # generic case
    x = _rand((B, H * W, C), 95) * 2
    for i, n in enumerate("qkv"):
        p[f"attn.{n}_linear.weight"] = _rand((C, C), 96 + i)
        p[f"attn.{n}_linear.bias"] = _rand((C,), 99 + i) * 0.2
    p["attn.proj.weight"] = _rand((C, C), 102)
    p["attn.relative_position_bias_table"] = _rand(((2 * ws - 1) ** 2, nH), 103)
    land = _rand((H, W), 104) > 0.5
    ac = so.swin_block_attention_autocast_bf16(x, H, W, ws, s, nH, p, land=land).double()
    pb = {k_: (v_.bfloat16().float() if "linear" in k_ or "proj" in k_ else v_) for k_, v_ in p.items()}
    ref = so.swin_block_attention(x.bfloat16().float(), H, W, ws, s, nH, pb, land=land).double()
    d_ref = ref - x.bfloat16().double()
    assert (torch.linalg.vector_norm(ac - ref) / torch.linalg.vector_norm(d_ref)).item() <= 3e-2
    assert not torch.equal(ac, ref.bfloat16().double())
