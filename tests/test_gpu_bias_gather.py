"""Bit-exact readback of the relative-position bias gather
(models/attention.py:260-266: table[relative_position_index].view(N, N, nH))
inside each attention kernel.

With q = k = 0 the logits are the bias alone.  A table that is -1000
everywhere except one entry e of head h, set to 0, makes every probability of
query i exactly 1 (the one key j with idx(i, j) == e) or 0 (exp underflows),
or, when no key of query i has index e, uniform.  Values that hold each key's
index (exact small integers) then read back j, the key the kernel paired with
query i for entry e, bit for bit.  Sweeping e over all (2w-1)^2 entries (one
per head per launch) checks the gather of every (i, j) pair against the
brute-force index (oracle/brute.relative_index).  Rows with no such key must
read back the mean of the values (exact in bf16 for these windows).
"""
import numpy as np
import pytest
import torch

from oracle import brute
from oracle import swin_oracle as so
from terra_amd import kernels
from terra_amd.kernels import WindowGeometry

pytestmark = pytest.mark.gpu


def _expected(idx: np.ndarray, e: int, vals: np.ndarray):
    """Per query: the value of the key j with idx[i, j] == e, else the mean."""
    n = idx.shape[0]
    out = np.empty(n, dtype=np.float64)
    hit = np.zeros(n, dtype=bool)
    for i in range(n):
        js = np.nonzero(idx[i] == e)[0]
        assert len(js) <= 1
        if len(js):
            out[i], hit[i] = vals[js[0]], True
        else:
            out[i] = vals.mean()
    return out, hit


@pytest.mark.parametrize("dtype,ws,C,heads,tiny_scale,kernel", [
    (torch.bfloat16, 8, 192, 6, False, "ring (head dim 32, even heads)"),
    (torch.bfloat16, 8, 96, 3, False, "per-wave (odd head count)"),
    (torch.bfloat16, 8, 768, 12, False, "ring (head dim 64)"),
    (torch.bfloat16, 8, 192, 6, True, "window-tile (head dim 32, scale below 2^-20)"),
    (torch.bfloat16, 8, 768, 12, True, "window-tile (head dim 64, scale below 2^-20)"),
    (torch.bfloat16, 8, 1024, 8, False, "ring (head dim 128)"),
    (torch.bfloat16, 8, 1024, 8, True, "per-wave (head dim 128, scale below 2^-20)"),
    (torch.float32, 8, 256, 2, False, "per-wave fp32, head dim 128"),
    (torch.bfloat16, 7, 128, 4, False, "per-wave (7x7 windows)"),
    (torch.float32, 8, 64, 2, False, "per-wave fp32"),
    (torch.float32, 7, 96, 3, False, "per-wave fp32, 7x7"),
])
def test_attention_bias_gather_bit_exact(dev, dtype, ws, C, heads, tiny_scale, kernel):
    N, d, T = ws * ws, C // heads, (2 * ws - 1) ** 2
    # q = k = 0: the logits are the bias whatever the scale; a scale below
    # 2^-20 selects the window-tile kernel for bf16 8x8 windows.
    scale = 2.0 ** -21 if tiny_scale else d ** -0.5
    B_ = 3
    idx = brute.relative_index(ws, ws)
    key_vals = np.arange(N, dtype=np.float64)
    q = torch.zeros(B_, N, C, dtype=dtype, device=dev)
    # v[j, channel c] = j + 64 * (c % 2): exact integers; the channel offset
    # catches a value read from the wrong column.
    offs = 64.0 * (torch.arange(C) % 2).double()
    v = (torch.from_numpy(key_vals)[:, None] + offs[None, :]).expand(B_, N, C).to(dtype).contiguous().to(dev)
    for e0 in range(0, T, heads):
        table = torch.full((T, heads), -1000.0)
        for h in range(heads):
            if e0 + h < T:
                table[e0 + h, h] = 0.0
        out = kernels.window_attention(q, q, v, heads, (ws, ws), scale, bias_table=table.to(dev)).double().cpu()
        for h in range(heads):
            e = e0 + h
            if e >= T:
                continue
            want, hit = _expected(idx, e, key_vals)
            got = out[:, :, h * d:(h + 1) * d] - offs[h * d:(h + 1) * d]
            # one-hot rows: bit-exact in every window and channel
            assert torch.equal(got[:, hit], torch.from_numpy(want[hit])[None, :, None].expand(B_, -1, d)), \
                (kernel, e, h)
            # rows with no key of index e: the mean of the key values (exact in
            # bf16; fp32 divides by a rounded reciprocal of N)
            tol = 0.0 if dtype == torch.bfloat16 else 1e-5
            miss = torch.from_numpy(want[~hit])[None, :, None]
            assert ((got[:, ~hit] - miss).abs() <= tol).all(), (kernel, e, h)


@pytest.mark.parametrize("C,heads,ws", [(192, 6, 8), (384, 12, 8), (768, 12, 8), (128, 4, 7)])
def test_fused_block_bias_gather_bit_exact(dev, C, heads, ws):
    """The fused half-block kernel's gather, through its q/k/v and proj: no
    LayerNorm, q and k weights zero (q = k = 0), v and proj weights the
    identity, so y = x + (attention output) exactly.  Token values are the
    token's index within its window (W-MSA, shift 0), so y - x reads back the
    key each query was paired with."""
    N, T = ws * ws, (2 * ws - 1) ** 2
    H, W = 2 * ws, 3 * ws
    d = C // heads
    geom = WindowGeometry(1, H, W, C, ws)
    hh, ww = torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij")
    tok = ((hh % ws) * ws + (ww % ws)).double()  # index within the window
    x = tok[None, :, :, None].expand(1, H, W, C).to(torch.bfloat16).contiguous().to(dev)
    eye = torch.eye(C, dtype=torch.bfloat16)
    w_qkv = torch.cat([torch.zeros(2 * C, C, dtype=torch.bfloat16), eye], 0).contiguous().to(dev)
    w_proj = eye.contiguous().to(dev)
    idx = brute.relative_index(ws, ws)
    key_vals = np.arange(N, dtype=np.float64)
    xw = so.partition_frame(tok.view(1, H, W, 1), ws)[..., 0]  # [nW, N]: window token -> its value
    assert torch.equal(xw, torch.from_numpy(key_vals)[None].expand_as(xw))
    for e0 in range(0, T, heads):
        table = torch.full((T, heads), -1000.0)
        for h in range(heads):
            if e0 + h < T:
                table[e0 + h, h] = 0.0
        y = kernels.swin_block(x, geom, heads, d ** -0.5, w_qkv, None, w_proj, None, layernorm=False,
                               bias_table=table.to(dev))
        yw = so.partition_frame((y.double() - x.double()).cpu(), ws)  # [nW, N, C]
        for h in range(heads):
            e = e0 + h
            if e >= T:
                continue
            want, _ = _expected(idx, e, key_vals)
            assert torch.equal(yw[:, :, d * h:d * (h + 1)],
                               torch.from_numpy(want)[None, :, None].expand(yw.shape[0], N, d)), (e, h)
