"""CPU oracle of TERRA's shifted-window attention path.

TEST INFRASTRUCTURE ONLY.  This module restates, with torch CPU operations,
the reference's op sequence for the hot path so that the HIP kernels can be
checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``terra_amd``) never does.

Every function cites the reference lines (paths relative to the TERRA tree)
whose semantics it restates.  How each function is pinned (independent
brute-force loops, closed forms, library special cases, known answers):

  roll_partition / reverse_unroll      brute.partition_index / brute.reverse_index,
                                       reverse o partition == id, roll round trip
  partition_frame / reverse_frame      brute loops over the padded, rolled frame
  relative_position_index              brute.relative_index, known values, symmetry
  shift_mask                           brute.shift_mask, known -100 counts, symmetry
  window_attention_core                float64 brute force (brute.attention), SDPA
                                       special case (s=0, no bias, no mask)
  land_key_flags / fold_land           brute loops
  ragged_row_major                     the reference's own unit-test vector
                                       (tests/unit/test_window_assignment.py:10-23)
  window_attention_autocast_bf16       brute.attention_autocast_bf16 (loops rounding
                                       to bf16 at the same points); the fp32 core
                                       must fail the same check
  linear_autocast_bf16                 an exact case (products and sums of small
                                       integers) and the bf16 rounding of the
                                       fp32 result (tests/test_oracle.py)
  swin_block_attention_autocast_bf16   composed of the pinned pieces here; with
                                       bf16-exact inputs whose every intermediate
                                       is exact it equals swin_block_attention
                                       (tests/test_oracle.py)
  swin_block_attention                 brute.swin_block (float64 token loops: own
                                       LayerNorm, frame walk, region ids, relative
                                       index, softmax, reverse), with pad, slab,
                                       pad-window, land and no-LayerNorm cases
  mlp / mlp_bf16                       brute.mlp (token loops, math.erf GELU,
                                       bit-level bf16 rounding); GELU known
                                       values; LayerNorm against its definition
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

MASK_VALUE = -100.0      # models/utils.py:84
PAD_KEY_VALUE = -10000.0  # models/attention.py:907


# ----------------------------------------------------------------------------
# a1-a3: roll, partition, reverse
# ----------------------------------------------------------------------------

def roll_partition(x: torch.Tensor, window_size: int, shift: int = 0) -> torch.Tensor:
    """roll(-s) then window_partition then view(-1, N, C).

    models/transformer.py:179-182 (roll), models/utils.py:35-39 (partition),
    models/transformer.py:225 (view).  x: [B, H, W, C] -> [B*nW, ws*ws, C].
    """
    if shift > 0:
        x = torch.roll(x, shifts=(-shift, -shift), dims=(1, 2))
    B, H, W, C = x.shape
    x = x.view(B, H // window_size, window_size, W // window_size, window_size, C)
    windows = x.permute(0, 1, 3, 2, 4, 5).contiguous().view(-1, window_size, window_size, C)
    return windows.view(-1, window_size * window_size, C)


def reverse_unroll(windows: torch.Tensor, window_size: int, H: int, W: int, shift: int = 0) -> torch.Tensor:
    """window_reverse then roll(+s).

    models/utils.py:41-45 (B recovered with float division), models/transformer.py:245-246.
    windows: [B*nW, ws*ws, C] (or [B*nW, ws, ws, C]) -> [B, H, W, C].
    """
    C = windows.shape[-1]
    B = int(windows.shape[0] / (H * W / window_size / window_size))
    x = windows.reshape(B, H // window_size, W // window_size, window_size, window_size, C)
    x = x.permute(0, 1, 3, 2, 4, 5).contiguous().view(B, H, W, C)
    if shift > 0:
        x = torch.roll(x, shifts=(shift, shift), dims=(1, 2))
    return x


def partition_frame(x: torch.Tensor, window_size: int, shift_h: int = 0, shift_w: int = 0,
                    pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0,
                    win_rows: Optional[int] = None, valid: Optional[Tuple[int, int]] = None,
                    pad_value: float = 0.0) -> torch.Tensor:
    """Pad (model-level ZeroPad2d, models/reference_model/sequential_hierarchical_swin.py:277-278),
    roll by (-shift_h, -shift_w) over the padded frame, partition, keep window rows
    [win_row_begin, +win_rows), and blank the windows outside `valid` (pad windows,
    models/attention.py:890-894).  Returns [B * rows * nWw, ws*ws, C]."""
    B, H, W, C = x.shape
    top, bottom, left, right = pad
    xp = torch.full((B, H + top + bottom, W + left + right, C), pad_value, dtype=x.dtype)
    xp[:, top:top + H, left:left + W] = x
    xp = torch.roll(xp, shifts=(-shift_h, -shift_w), dims=(1, 2))
    Hp, Wp = xp.shape[1], xp.shape[2]
    ws = window_size
    nwh, nww = Hp // ws, Wp // ws
    win = xp.view(B, nwh, ws, nww, ws, C).permute(0, 1, 3, 2, 4, 5).reshape(B, nwh, nww, ws * ws, C)
    rows = nwh - win_row_begin if win_rows is None else win_rows
    win = win[:, win_row_begin:win_row_begin + rows].reshape(B, rows * nww, ws * ws, C).clone()
    if valid is not None:
        keep = torch.zeros(rows * nww, dtype=torch.bool)
        keep[valid[0]:valid[1]] = True
        win[:, ~keep] = pad_value
    return win.reshape(B * rows * nww, ws * ws, C)


def reverse_frame(windows: torch.Tensor, B: int, H: int, W: int, window_size: int, shift_h: int = 0,
                  shift_w: int = 0, pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0,
                  win_rows: Optional[int] = None, valid: Optional[Tuple[int, int]] = None,
                  residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Inverse of partition_frame: windows back into the frame (windows not emitted
    and pad windows contribute 0), roll(+shift), crop the padding, then
    ``residual + x`` (models/transformer.py:296-298).  Returns [B, H, W, C]."""
    C = windows.shape[-1]
    top, bottom, left, right = pad
    Hp, Wp = H + top + bottom, W + left + right
    ws = window_size
    nwh, nww = Hp // ws, Wp // ws
    rows = nwh - win_row_begin if win_rows is None else win_rows
    win = windows.reshape(B, rows * nww, ws * ws, C).clone()
    if valid is not None:
        keep = torch.zeros(rows * nww, dtype=torch.bool)
        keep[valid[0]:valid[1]] = True
        win[:, ~keep] = 0
    full = torch.zeros(B, nwh, nww, ws * ws, C, dtype=windows.dtype)
    full[:, win_row_begin:win_row_begin + rows] = win.view(B, rows, nww, ws * ws, C)
    frame = full.view(B, nwh, nww, ws, ws, C).permute(0, 1, 3, 2, 4, 5).reshape(B, Hp, Wp, C)
    frame = torch.roll(frame, shifts=(shift_h, shift_w), dims=(1, 2))
    y = frame[:, top:top + H, left:left + W].contiguous()
    if residual is not None:
        y = residual.view(B, H, W, C) + y
    return y


# ----------------------------------------------------------------------------
# a4-a6, a12: relative-position index, bias gather, shift mask, land fold
# ----------------------------------------------------------------------------

def relative_position_index(window_size: Sequence[int]) -> torch.Tensor:
    """models/attention.py:205-214 (meshgrid 'ij', pairwise differences, offsets)."""
    wh, ww = window_size
    coords = torch.stack(torch.meshgrid([torch.arange(wh), torch.arange(ww)], indexing="ij"))
    flat = torch.flatten(coords, 1)
    rel = (flat[:, :, None] - flat[:, None, :]).permute(1, 2, 0).contiguous()
    rel[:, :, 0] += wh - 1
    rel[:, :, 1] += ww - 1
    rel[:, :, 0] *= 2 * ww - 1
    return rel.sum(-1)


def relative_position_bias(table: torch.Tensor, window_size: Sequence[int]) -> torch.Tensor:
    """Bias gather [nH, N, N] (models/attention.py:260-263)."""
    n = window_size[0] * window_size[1]
    idx = relative_position_index(window_size)
    return table[idx.view(-1)].view(n, n, -1).permute(2, 0, 1).contiguous()


def shift_mask(H: int, W: int, window_size: int, shift: int) -> torch.Tensor:
    """get_swin_attention_mask('sequential', ...) (models/utils.py:56-94): region
    image from the 3x3 slices, partitioned, pairwise compare, -100 / 0."""
    img = torch.zeros((1, H, W, 1))
    slices = (slice(0, -window_size), slice(-window_size, -shift), slice(-shift, None))
    cnt = 0
    for hs in slices:
        for wsl in slices:
            img[:, hs, wsl, :] = cnt
            cnt += 1
    mw = roll_partition(img, window_size).view(-1, window_size * window_size)
    m = mw.unsqueeze(1) - mw.unsqueeze(2)
    return m.masked_fill(m != 0, MASK_VALUE).masked_fill(m == 0, 0.0)


def land_key_flags(land: torch.Tensor, window_size: int, shift_h: int = 0, shift_w: int = 0,
                   pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0,
                   win_rows: Optional[int] = None, valid: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """[H, W] bool land grid -> [nW, N] bool flags of each window's keys, cut with
    the same pad/roll/partition as the activations (build-defined land fold)."""
    H, W = land.shape
    f = partition_frame(land.to(torch.float32).view(1, H, W, 1), window_size, shift_h, shift_w, pad,
                        win_row_begin, win_rows, valid)
    return f.view(f.shape[0], -1) > 0.5


def fold_land(mask: Optional[torch.Tensor], land_flags: torch.Tensor) -> torch.Tensor:
    """M_total[w, i, j] = M_shift[w, i, j] + (land[w, j] ? -100 : 0)."""
    land_term = torch.where(land_flags, torch.tensor(MASK_VALUE), torch.tensor(0.0))[:, None, :]
    n = land_flags.shape[1]
    land_term = land_term.expand(land_flags.shape[0], n, n)
    return land_term.clone() if mask is None else mask + land_term


# ----------------------------------------------------------------------------
# a7, a10: attention core (with padded windows / keys)
# ----------------------------------------------------------------------------

def window_attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int, scale: float,
                          bias_table: Optional[torch.Tensor] = None, window_size: Optional[Sequence[int]] = None,
                          mask: Optional[torch.Tensor] = None, n_real: Optional[int] = None,
                          compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """softmax(q*scale @ k^T + bias + mask) @ v per window and head.

    models/attention.py:256-278 (core), :874-907 (bias/mask zero-padded to the
    full token count, keys >= n_real masked_fill -10000).  q, k, v: [B_, N, C];
    computed in `compute_dtype`; returns [B_, N, C] in `compute_dtype`.
    """
    B_, N, C = q.shape
    d = C // num_heads
    q = q.to(compute_dtype).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    k = k.to(compute_dtype).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    v = v.to(compute_dtype).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    q = q * scale
    attn = q @ k.transpose(-2, -1)
    n_geo = N if window_size is None else window_size[0] * window_size[1]
    if bias_table is not None:
        rpb = relative_position_bias(bias_table.to(compute_dtype), window_size)
        if n_geo != N:
            full = rpb.new_zeros(num_heads, N, N)
            full[:, :n_geo, :n_geo] = rpb
            rpb = full
        attn = attn + rpb.unsqueeze(0)
    if mask is not None:
        nW = mask.shape[0]
        m = mask.to(compute_dtype)
        if n_geo != N:
            full = m.new_zeros(nW, N, N)
            full[:, :n_geo, :n_geo] = m
            m = full
        attn = attn.view(B_ // nW, nW, num_heads, N, N) + m.unsqueeze(1).unsqueeze(0)
        attn = attn.view(-1, num_heads, N, N)
    if n_real is not None and n_real < N:
        valid = torch.arange(N) < n_real
        attn = attn.masked_fill(~valid.view(1, 1, 1, N), PAD_KEY_VALUE)
    attn = torch.softmax(attn, dim=-1)
    return (attn @ v).transpose(1, 2).reshape(B_, N, C)


def window_attention_autocast_bf16(q, k, v, num_heads, scale, bias_table=None, window_size=None, mask=None):
    """The reference's core under CUDA autocast(bf16) (core/runtime/run_model.py:424-448):
    q*scale and q@k^T rounded to bf16, bias/mask promote to fp32, fp32 softmax,
    probabilities re-cast to bf16 for attn@v, bf16 output.  Used to report how
    far the reference itself sits from the fp32 restatement, and as the
    yardstick of the drop-ins run under autocast."""
    B_, N, C = q.shape
    d = C // num_heads
    q = q.to(torch.bfloat16).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    k = k.to(torch.bfloat16).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    v = v.to(torch.bfloat16).reshape(B_, N, num_heads, d).permute(0, 2, 1, 3)
    q = (q.float() * scale).to(torch.bfloat16)
    attn = (q.float() @ k.float().transpose(-2, -1)).to(torch.bfloat16)
    attn = attn.float()
    if bias_table is not None:
        attn = attn + relative_position_bias(bias_table.float(), window_size).unsqueeze(0)
    if mask is not None:
        nW = mask.shape[0]
        attn = (attn.view(B_ // nW, nW, num_heads, N, N) + mask.float().unsqueeze(1).unsqueeze(0)).view(-1, num_heads, N, N)
    attn = torch.softmax(attn, dim=-1).to(torch.bfloat16)
    out = (attn.float() @ v.float()).to(torch.bfloat16)
    return out.transpose(1, 2).reshape(B_, N, C)


# ----------------------------------------------------------------------------
# a8, a9: the block's attention half, and the MLP half (context for configs 2/4)
# ----------------------------------------------------------------------------

def swin_block_attention(x: torch.Tensor, H: int, W: int, window_size: int, shift: int, num_heads: int,
                         params: dict, land: Optional[torch.Tensor] = None, use_attn_mask: bool = True,
                         pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0,
                         win_rows: Optional[int] = None, valid: Optional[Tuple[int, int]] = None,
                         use_layernorm: bool = True, compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """SequentialSwinTransformer.forward (models/transformer.py:138-298) in fp32.

    params: 'norm1.weight', 'norm1.bias', 'attn.{q,k,v}_linear.{weight,bias}',
    'attn.proj.{weight,bias}', 'attn.relative_position_bias_table' (state-dict
    names of the reference).  The frame/slab arguments extend the reference's
    square-grid case (pad, window-row range, pad windows) as in partition_frame.
    """
    B, L, C = x.shape
    # Parameters that require a gradient stay in the graph (backward parity).
    p = {k_: (v_ if v_.requires_grad else v_.detach()).to(compute_dtype).cpu() for k_, v_ in params.items()}
    x = x.to(compute_dtype)
    shortcut = x
    if use_layernorm:
        x = F.layer_norm(x, (C,), p["norm1.weight"], p["norm1.bias"])
    x = x.view(B, H, W, C)
    win = partition_frame(x, window_size, shift, shift, pad, win_row_begin, win_rows, valid)
    q = F.linear(win, p["attn.q_linear.weight"], p["attn.q_linear.bias"])
    k = F.linear(win, p["attn.k_linear.weight"], p["attn.k_linear.bias"])
    v = F.linear(win, p["attn.v_linear.weight"], p["attn.v_linear.bias"])
    Hp, Wp = H + pad[0] + pad[1], W + pad[2] + pad[3]
    nwh, nww = Hp // window_size, Wp // window_size
    rows = nwh - win_row_begin if win_rows is None else win_rows
    mask = None
    if shift > 0 and use_attn_mask:
        full = shift_mask(Hp, Wp, window_size, shift).view(nwh, nww, window_size ** 2, window_size ** 2)
        mask = full[win_row_begin:win_row_begin + rows].reshape(rows * nww, window_size ** 2, window_size ** 2)
    if land is not None:
        flags = land_key_flags(land, window_size, shift, shift, pad, win_row_begin, win_rows, valid)
        mask = fold_land(mask, flags)
    d = C // num_heads
    table = p.get("attn.relative_position_bias_table")
    o = window_attention_core(q, k, v, num_heads, d ** -0.5, table, (window_size, window_size), mask,
                              compute_dtype=compute_dtype)
    o = F.linear(o, p["attn.proj.weight"], p["attn.proj.bias"])
    y = reverse_frame(o, B, H, W, window_size, shift, shift, pad, win_row_begin, win_rows, valid,
                      residual=shortcut)
    return y.view(B, H * W, C)


def linear_autocast_bf16(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
    """F.linear under CUDA autocast(bf16): input, weight and bias cast to bf16,
    products accumulated in fp32 (the GEMM's accumulator, with the bias added in
    its fp32 epilogue), the result rounded once to bf16.  Returns bf16."""
    y = x.to(torch.bfloat16).float() @ weight.to(torch.bfloat16).float().t()
    if bias is not None:
        y = y + bias.to(torch.bfloat16).float()
    return y.to(torch.bfloat16)


def swin_block_attention_autocast_bf16(x: torch.Tensor, H: int, W: int, window_size: int, shift: int,
                                       num_heads: int, params: dict, land: Optional[torch.Tensor] = None,
                                       eps: float = 1e-5) -> torch.Tensor:
    """SequentialSwinTransformer.forward (models/transformer.py:138-298) as the
    reference runs it under CUDA autocast(bf16) (core/runtime/run_model.py:
    424-448) on bf16 activations: LayerNorm in fp32 (autocast's fp32 list),
    the q/k/v and proj Linears as linear_autocast_bf16, the core as
    window_attention_autocast_bf16, and the residual sum of two bf16 tensors
    rounded to bf16.  Composed of the pinned restatements above; returns bf16
    [B, H*W, C]."""
    B, L, C = x.shape
    p = {k_: v_.detach().float().cpu() for k_, v_ in params.items()}
    xb = x.to(torch.bfloat16)
    xn = F.layer_norm(xb.float(), (C,), p["norm1.weight"], p["norm1.bias"], eps).view(B, H, W, C)
    win = partition_frame(xn, window_size, shift, shift)
    q = linear_autocast_bf16(win, p["attn.q_linear.weight"], p["attn.q_linear.bias"])
    k = linear_autocast_bf16(win, p["attn.k_linear.weight"], p["attn.k_linear.bias"])
    v = linear_autocast_bf16(win, p["attn.v_linear.weight"], p["attn.v_linear.bias"])
    mask = shift_mask(H, W, window_size, shift) if shift > 0 else None
    if land is not None:
        mask = fold_land(mask, land_key_flags(land, window_size, shift, shift))
    o = window_attention_autocast_bf16(q, k, v, num_heads, (C // num_heads) ** -0.5,
                                       p.get("attn.relative_position_bias_table"), (window_size, window_size), mask)
    o = linear_autocast_bf16(o, p["attn.proj.weight"], p["attn.proj.bias"])
    y = reverse_frame(o.float(), B, H, W, window_size, shift, shift)
    return (xb.float().view(B, H, W, C) + y).to(torch.bfloat16).view(B, H * W, C)


def mlp(x: torch.Tensor, params: dict, use_layernorm: bool = True) -> torch.Tensor:
    """SequentialMlp.forward (models/mlp.py:152-172): LN -> fc1 -> GELU -> fc2 -> +x."""
    p = {k_: v_.detach().float().cpu() for k_, v_ in params.items()}
    x = x.float()
    h = F.layer_norm(x, (x.shape[-1],), p["norm2.weight"], p["norm2.bias"]) if use_layernorm else x
    h = F.gelu(F.linear(h, p["fc1.weight"], p["fc1.bias"]))
    return F.linear(h, p["fc2.weight"], p["fc2.bias"]) + x


def _bf16(t: torch.Tensor) -> torch.Tensor:
    """Round to bfloat16 through float32 (the GPU's fp32 epilogues), as float64."""
    return t.float().bfloat16().double()


def mlp_bf16(x: torch.Tensor, params: dict, use_layernorm: bool = True, eps: float = 1e-5) -> torch.Tensor:
    """SequentialMlp.forward (models/mlp.py:152-172) of a bf16 module: float64
    arithmetic on the bf16 input and bf16-rounded weights, rounded to bf16 where
    the bf16 module rounds (LayerNorm output, fc1 output with its fp32 bias,
    GELU output, fc2 output, the residual sum).  Returns float64 [.., C]."""
    p = {k_: v_.detach().cpu() for k_, v_ in params.items()}
    C = x.shape[-1]
    xb = _bf16(x.detach().cpu())
    h = xb
    if use_layernorm:
        h = _bf16(F.layer_norm(xb, (C,), p["norm2.weight"].double(), p["norm2.bias"].double(), eps))
    h = _bf16(F.linear(h, _bf16(p["fc1.weight"]), p["fc1.bias"].float().double()))
    h = _bf16(0.5 * h * (1.0 + torch.special.erf(h / 2.0 ** 0.5)))
    y = _bf16(F.linear(h, _bf16(p["fc2.weight"]), p["fc2.bias"].float().double()))
    return _bf16(xb + y)


# ----------------------------------------------------------------------------
# a11: ragged row-major window ownership
# ----------------------------------------------------------------------------

def ragged_row_major(num_windows_h: int, num_windows_w: int, m: int):
    """_assign_terra_m1_ragged_row_major (core/parallel/window_assignment.py:64-76):
    rank r owns flat ids [(r*T)//m, ((r+1)*T)//m), coordinates (id // nWw, id % nWw)."""
    total = num_windows_h * num_windows_w
    if total < m:
        raise ValueError(f"terra_m1_ragged_row_major requires total_windows={total} >= m={m}")
    out = []
    for r in range(m):
        ids = range((r * total) // m, ((r + 1) * total) // m)
        out.append([(i // num_windows_w, i % num_windows_w) for i in ids])
    return out
