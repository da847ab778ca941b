"""Brute-force restatements used to pin the oracle — TEST INFRASTRUCTURE ONLY.

Plain Python loops over coordinates, written from the definitions rather than
from tensor reshapes, so that a transposed permute, an off-by-one roll or a
wrong region slice in ``swin_oracle`` shows up as a mismatch.  Sizes must stay
tiny (a few thousand tokens).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np


def frame_source(B: int, H: int, W: int, ws: int, shift_h: int = 0, shift_w: int = 0,
                 pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0, win_rows: Optional[int] = None,
                 valid: Optional[Tuple[int, int]] = None) -> List[Optional[Tuple[int, int, int]]]:
    """For every output (window, token) in order, the (b, h, w) source token of the
    unpadded grid, or None where the output is padding / a pad window.

    Definition: shifted[b, i, j] = padded[b, (i + sh) mod Hp, (j + sw) mod Wp]
    (torch.roll by -s); window (wr, wc) holds shifted rows wr*ws..wr*ws+ws-1,
    columns wc*ws..; token t = ti*ws + tj; windows image-major, row-major.
    """
    top, bottom, left, right = pad
    Hp, Wp = H + top + bottom, W + left + right
    nwh, nww = Hp // ws, Wp // ws
    rows = nwh - win_row_begin if win_rows is None else win_rows
    out = []
    for b in range(B):
        for r in range(rows):
            for wc in range(nww):
                flat = r * nww + wc
                is_valid = valid is None or (valid[0] <= flat < valid[1])
                wr = r + win_row_begin
                for ti in range(ws):
                    for tj in range(ws):
                        i, j = wr * ws + ti, wc * ws + tj
                        ph, pw = (i + shift_h) % Hp, (j + shift_w) % Wp
                        sh, sw = ph - top, pw - left
                        if is_valid and 0 <= sh < H and 0 <= sw < W:
                            out.append((b, sh, sw))
                        else:
                            out.append(None)
    return out


def partition(x: np.ndarray, ws: int, **geom) -> np.ndarray:
    """x [B, H, W, C] -> [B_, N, C] through frame_source (pad value 0)."""
    B, H, W, C = x.shape
    src = frame_source(B, H, W, ws, **geom)
    out = np.zeros((len(src), C), dtype=x.dtype)
    for n, s in enumerate(src):
        if s is not None:
            out[n] = x[s]
    return out.reshape(-1, ws * ws, C)


def reverse(windows: np.ndarray, B: int, H: int, W: int, ws: int, residual: Optional[np.ndarray] = None,
            **geom) -> np.ndarray:
    """Inverse map: every grid token takes the one window token whose source it is;
    tokens no emitted window reads stay 0; then + residual."""
    C = windows.shape[-1]
    flat = windows.reshape(-1, C)
    y = np.zeros((B, H, W, C), dtype=windows.dtype)
    for n, s in enumerate(frame_source(B, H, W, ws, **geom)):
        if s is not None:
            y[s] = flat[n]
    if residual is not None:
        y = residual.reshape(B, H, W, C) + y
    return y


def relative_index(wh: int, ww: int) -> np.ndarray:
    """idx[i, j] for i = (hi, wi), j = (hj, wj): the (dh, dw) offset pair mapped
    row-major onto a (2wh-1) x (2ww-1) table with (0, 0) at the centre."""
    n = wh * ww
    idx = np.zeros((n, n), dtype=np.int64)
    for i in range(n):
        hi, wi = divmod(i, ww)
        for j in range(n):
            hj, wj = divmod(j, ww)
            idx[i, j] = (hi - hj + wh - 1) * (2 * ww - 1) + (wi - wj + ww - 1)
    return idx


def _region(coord: int, extent: int, ws: int, shift: int) -> int:
    if coord < extent - ws:
        return 0
    if coord < extent - shift:
        return 1
    return 2


def shift_mask(H: int, W: int, ws: int, shift: int) -> np.ndarray:
    """[nW, N, N]: -100 where the two tokens of a window come from different
    regions of the rolled frame, else 0."""
    nwh, nww = H // ws, W // ws
    n = ws * ws
    m = np.zeros((nwh * nww, n, n), dtype=np.float32)
    for wr in range(nwh):
        for wc in range(nww):
            rid = []
            for t in range(n):
                ti, tj = divmod(t, ws)
                rid.append((_region(wr * ws + ti, H, ws, shift), _region(wc * ws + tj, W, ws, shift)))
            for i in range(n):
                for j in range(n):
                    if rid[i] != rid[j]:
                        m[wr * nww + wc, i, j] = -100.0
    return m


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_heads: int, scale: float,
              bias: Optional[np.ndarray] = None, mask: Optional[np.ndarray] = None,
              n_real: Optional[int] = None) -> np.ndarray:
    """float64 loops: for each window, head and query row, logits over keys,
    max-subtracted exponentials, normalised weights, weighted sum of values.
    bias: [nH, N, N] or None; mask: [nW, N, N] (window w uses mask[w % nW])."""
    B_, N, C = q.shape
    d = C // num_heads
    out = np.zeros((B_, N, C), dtype=np.float64)
    for w in range(B_):
        for h in range(num_heads):
            cs = slice(h * d, (h + 1) * d)
            for i in range(N):
                logits = []
                for j in range(N):
                    s = float(np.dot(q[w, i, cs].astype(np.float64) * scale, k[w, j, cs].astype(np.float64)))
                    if bias is not None:
                        s += float(bias[h, i, j])
                    if mask is not None:
                        s += float(mask[w % mask.shape[0], i, j])
                    if n_real is not None and j >= n_real:
                        s = -10000.0
                    logits.append(s)
                mx = max(logits)
                e = [math.exp(s - mx) for s in logits]
                tot = sum(e)
                acc = np.zeros(d, dtype=np.float64)
                for j in range(N):
                    acc += (e[j] / tot) * v[w, j, cs].astype(np.float64)
                out[w, i, cs] = acc
    return out


def bf16_round(v: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), as float32, by bit arithmetic
    on the float32 encoding (NaN kept quiet)."""
    f = np.asarray(v, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, (u.astype(np.uint32) & 0xFFFF0000) | 0x00400000, r).astype(np.uint32)
    return r.view(np.float32)


def gelu(v: float) -> float:
    """nn.GELU() (exact form): x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2))."""
    return 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))


def mlp(x: np.ndarray, p: dict, use_layernorm: bool = True, eps: float = 1e-5,
        round_bf16: bool = False) -> np.ndarray:
    """SequentialMlp.forward (models/mlp.py:152-172) token by token with loops:
    LayerNorm over C, fc1 (weight [hid, C]), GELU, fc2 (weight [C, hid]),
    + x.  With ``round_bf16`` the float64 results are rounded to float32 and
    then to bf16 where a bf16 module rounds: LayerNorm output, fc1 output,
    GELU output, fc2 output and the residual sum."""
    rnd = (lambda a: bf16_round(np.float32(a)).astype(np.float64)) if round_bf16 else (lambda a: a)  # noqa: E731
    w1, b1 = np.asarray(p["fc1.weight"], np.float64), np.asarray(p["fc1.bias"], np.float64)
    w2, b2 = np.asarray(p["fc2.weight"], np.float64), np.asarray(p["fc2.bias"], np.float64)
    hid, C = w1.shape
    xs = np.asarray(x, np.float64).reshape(-1, C)
    out = np.empty_like(xs)
    for t in range(xs.shape[0]):
        row = xs[t]
        if use_layernorm:
            mean = sum(row) / C
            var = sum((c - mean) ** 2 for c in row) / C
            g, b = np.asarray(p["norm2.weight"], np.float64), np.asarray(p["norm2.bias"], np.float64)
            xn = [rnd((row[c] - mean) / math.sqrt(var + eps) * g[c] + b[c]) for c in range(C)]
        else:
            xn = list(row)
        h = [rnd(gelu(rnd(sum(w1[j, c] * xn[c] for c in range(C)) + b1[j]))) for j in range(hid)]
        for c in range(C):
            y = rnd(sum(w2[c, j] * h[j] for j in range(hid)) + b2[c])
            out[t, c] = rnd(row[c] + y)
    return out.reshape(np.asarray(x).shape)


def _bf16_scalar(a: float) -> float:
    """float64 -> float32 -> nearest bf16, as float64 (a GPU fp32 result cast to bf16)."""
    return float(bf16_round(np.float32(a)))


def attention_autocast_bf16(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_heads: int, scale: float,
                            bias: Optional[np.ndarray] = None, mask: Optional[np.ndarray] = None) -> np.ndarray:
    """The attention core as a bf16 autocast region runs it, by loops: bf16
    inputs; q * scale rounded to bf16; each logit q.k accumulated exactly and
    rounded to bf16 (autocast's matmul output); bias and mask added in fp32;
    softmax in float64 then rounded to bf16 (the probabilities are cast before
    attn @ v); each output accumulated exactly and rounded to bf16.
    bias: [nH, N, N] or None; mask: [nW, N, N] (window w uses mask[w % nW])."""
    B_, N, C = q.shape
    d = C // num_heads
    qb = bf16_round(np.asarray(q, np.float32)).astype(np.float64)
    kb = bf16_round(np.asarray(k, np.float32)).astype(np.float64)
    vb = bf16_round(np.asarray(v, np.float32)).astype(np.float64)
    out = np.zeros((B_, N, C), dtype=np.float64)
    for w in range(B_):
        for h in range(num_heads):
            cs = slice(h * d, (h + 1) * d)
            qs = [[_bf16_scalar(float(np.float32(a) * np.float32(scale))) for a in qb[w, i, cs]] for i in range(N)]
            for i in range(N):
                logits = []
                for j in range(N):
                    s = _bf16_scalar(sum(a * b for a, b in zip(qs[i], kb[w, j, cs])))
                    if bias is not None:
                        s = float(np.float32(s) + np.float32(bias[h, i, j]))
                    if mask is not None:
                        s = float(np.float32(s) + np.float32(mask[w % mask.shape[0], i, j]))
                    logits.append(s)
                mx = max(logits)
                e = [math.exp(s - mx) for s in logits]
                tot = sum(e)
                p = [_bf16_scalar(x / tot) for x in e]
                for c in range(d):
                    out[w, i, h * d + c] = _bf16_scalar(sum(p[j] * vb[w, j, h * d + c] for j in range(N)))
    return out


def layer_norm_row(row: Sequence[float], gamma: Optional[Sequence[float]], beta: Optional[Sequence[float]],
                   eps: float = 1e-5) -> List[float]:
    """nn.LayerNorm over one token from its definition: biased variance."""
    C = len(row)
    mean = sum(row) / C
    var = sum((c - mean) ** 2 for c in row) / C
    inv = 1.0 / math.sqrt(var + eps)
    return [(row[c] - mean) * inv * (1.0 if gamma is None else gamma[c]) + (0.0 if beta is None else beta[c])
            for c in range(C)]


def swin_block(x: np.ndarray, params: dict, ws: int, shift: int, num_heads: int,
               land: Optional[np.ndarray] = None, use_attn_mask: bool = True, use_layernorm: bool = True,
               pad: Sequence[int] = (0, 0, 0, 0), win_row_begin: int = 0, win_rows: Optional[int] = None,
               valid: Optional[Tuple[int, int]] = None, eps: float = 1e-5) -> np.ndarray:
    """The attention half of a Swin block, token by token in float64:
    LayerNorm each token, cut the (padded, shifted) frame into windows through
    frame_source (padding tokens and pad windows are zero vectors after the
    LayerNorm), q/k/v = W xn + b per token, per window and head
    softmax(q.k * d^-1/2 + table[relative index] + mask) v with the mask
    -100 for keys of another shift region (regions of the padded frame) or on
    land, proj, and every grid token takes back the output of the window token
    it was read into, plus the input token (the residual).  Tokens that no
    emitted window reads get the residual only.
    x: [B, H, W, C]; params: state-dict names as numpy arrays (norm1.weight /
    .bias, attn.{q,k,v}_linear.weight / .bias, attn.proj.weight / .bias,
    attn.relative_position_bias_table); land: [H, W] bool or None.
    Returns [B, H, W, C]."""
    B, H, W, C = x.shape
    top, bottom, left, right = pad
    Hp, Wp = H + top + bottom, W + left + right
    nww = Wp // ws
    N = ws * ws
    d = C // num_heads
    scale = d ** -0.5
    P = {k_: np.asarray(v_, np.float64) for k_, v_ in params.items()}
    table = P.get("attn.relative_position_bias_table")
    rel = relative_index(ws, ws)
    src = frame_source(B, H, W, ws, shift, shift, pad, win_row_begin, win_rows, valid)
    rows = (Hp // ws - win_row_begin) if win_rows is None else win_rows
    xs = np.asarray(x, np.float64)
    y = xs.copy()
    for wi in range(len(src) // N):
        toks = src[wi * N:(wi + 1) * N]
        xn = []
        for s in toks:
            if s is None:
                xn.append([0.0] * C)
            elif use_layernorm:
                xn.append(layer_norm_row(list(xs[s]), P["norm1.weight"], P["norm1.bias"], eps))
            else:
                xn.append(list(xs[s]))
        lin = {}
        for name in ("q", "k", "v"):
            wgt, bia = P[f"attn.{name}_linear.weight"], P[f"attn.{name}_linear.bias"]
            lin[name] = [[sum(wgt[o, c] * t[c] for c in range(C)) + bia[o] for o in range(C)] for t in xn]
        # frame window of this emitted window and the region id of each token
        r_local = (wi % (rows * nww)) // nww
        wr, wc = r_local + win_row_begin, wi % nww
        rid = [(_region(wr * ws + t // ws, Hp, ws, shift), _region(wc * ws + t % ws, Wp, ws, shift))
               for t in range(N)]
        is_land = [s is not None and land is not None and bool(land[s[1], s[2]]) for s in toks]
        o = [[0.0] * C for _ in range(N)]
        for h in range(num_heads):
            for i in range(N):
                logits = []
                for j in range(N):
                    s_ = scale * sum(lin["q"][i][h * d + c] * lin["k"][j][h * d + c] for c in range(d))
                    if table is not None:
                        s_ += table[rel[i, j], h]
                    if shift > 0 and use_attn_mask and rid[i] != rid[j]:
                        s_ += -100.0
                    if is_land[j]:
                        s_ += -100.0
                    logits.append(s_)
                mx = max(logits)
                e = [math.exp(a - mx) for a in logits]
                tot = sum(e)
                for c in range(d):
                    o[i][h * d + c] = sum(e[j] / tot * lin["v"][j][h * d + c] for j in range(N))
        wp, bp = P["attn.proj.weight"], P["attn.proj.bias"]
        for t, s in enumerate(toks):
            if s is not None:
                y[s] = xs[s] + np.array([sum(wp[f, c] * o[t][c] for c in range(C)) + bp[f] for f in range(C)])
    return y
