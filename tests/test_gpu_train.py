"""The training path's kernels: the backward of the fused LayerNorm +
partition (terra_swin_partition_ln_bwd), alone and inside the block, and the
MLP half's backward (autograd.mlp), against torch autograd of the oracle's
restatement; the mixed-dtype gather / scatter of bf16 autocast and the GELU
backward (terra_swin_gelu_bwd), each with its bias-gradient column sums,
against the separate ops they replace and float64 arithmetic.

Tolerances: fp32 activations, every gradient within 1e-5 of the float64
reference (max-abs relative, per tensor); bf16, within one bf16 rounding of
the output (2^-7 relative) plus 1e-2 of the tensor's max-abs for dx, and
2e-2 max-abs relative for the parameter gradients (fp32 sums over tokens of
bf16 products); module-level bf16 / autocast cases 3e-2 normwise, the
block tests' bound."""
import copy

import pytest
import torch

from helpers import gain_block, params_of
from oracle import swin_oracle as so
from terra_amd import kernels, workloads
from terra_amd.kernels import WindowGeometry

pytestmark = pytest.mark.gpu

CASES = [  # (B, H, W, C, ws, shift, pad, win_row_begin, win_rows, valid)
    (2, 16, 24, 192, 8, 4, (0, 0, 0, 0), 0, None, None),
    (2, 14, 21, 96, 7, 3, (0, 0, 0, 0), 0, None, None),
    (2, 20, 16, 384, 8, 4, (0, 4, 0, 0), 0, 2, (3, 4)),      # slab: rows not emitted, pad windows
    (1, 16, 16, 768, 8, 4, (0, 8, 0, 0), 0, 2, (1, 3)),      # 16 lanes per token
    (1, 16, 8, 1024, 8, 4, (0, 0, 0, 0), 0, None, None),     # C = 1024
    (1, 6, 6, 64, 4, 2, (1, 1, 1, 1), 0, None, None),        # frame padding on every side
]


def _geom(B, H, W, C, ws, s, pad, r0, rows, valid):
    return WindowGeometry(B, H, W, C, ws, s, s, pad, r0, rows, valid)


def _rel(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("residual", [False, True])
def test_partition_ln_backward_matches_autograd(dev, dtype, case, residual):
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    g = _geom(*case)
    x = (workloads.activations((B, H, W, C), 500) * 2 + 0.3).to(dtype)
    w = workloads.activations((C,), 501) * 0.2 + 1.0
    b = workloads.activations((C,), 502) * 0.2
    gw = workloads.activations((g.num_windows, ws * ws, C), 503).to(dtype)
    dres = workloads.activations((B, H, W, C), 504).to(dtype) if residual else None
    cd = torch.float64
    xr = x.to(cd).requires_grad_(True)
    wr = w.to(cd).requires_grad_(True)
    br = b.to(cd).requires_grad_(True)
    win = so.partition_frame(torch.nn.functional.layer_norm(xr, (C,), wr, br, 1e-5), ws, s, s, pad, r0, rows, valid)
    win.backward(gw.to(cd))
    want_dx = xr.grad + (dres.to(cd) if residual else 0)
    dw = torch.zeros(C, device=dev)
    db = torch.zeros(C, device=dev)
    got = kernels.swin_partition_ln_backward(gw.to(dev), x.to(dev), g, w.to(dev), 1e-5,
                                             dresidual=None if dres is None else dres.to(dev), dweight=dw, dbias=db)
    assert got.dtype == dtype and tuple(got.shape) == (B, H, W, C)
    if dtype == torch.float32:
        assert _rel(got, want_dx) <= 1e-5
        assert _rel(dw, wr.grad) <= 1e-5 and _rel(db, br.grad) <= 1e-5
    else:
        err = (got.double().cpu() - want_dx).abs()
        assert bool((err <= 2.0 ** -7 * want_dx.abs() + 1e-2 * want_dx.abs().max()).all()), err.max().item()
        assert _rel(dw, wr.grad) <= 2e-2 and _rel(db, br.grad) <= 2e-2
    # tokens no window reads: dx is the residual gradient alone (or 0)
    reads = so.partition_frame(torch.ones(B, H, W, 1), ws, s, s, pad, r0, rows, valid)
    mask = so.reverse_frame(reads, B, H, W, ws, s, s, pad, r0, rows, valid)[..., 0] == 0
    if mask.any():
        want_free = dres.float()[mask] if residual else torch.zeros_like(got.float().cpu()[mask])
        assert torch.equal(got.float().cpu()[mask], want_free)


def test_partition_ln_backward_in_place_on_residual(dev):
    """dx may be the residual-gradient tensor itself."""
    B, H, W, C, ws, s = 1, 16, 16, 192, 8, 4
    g = WindowGeometry(B, H, W, C, ws, s, s)
    x = workloads.activations((B, H, W, C), 510, torch.bfloat16).to(dev)
    gw = workloads.activations((g.num_windows, 64, C), 511, torch.bfloat16).to(dev)
    dres = workloads.activations((B, H, W, C), 512, torch.bfloat16).to(dev)
    want = kernels.swin_partition_ln_backward(gw, x, g, None, 1e-5, dresidual=dres.clone())
    got = kernels.swin_partition_ln_backward(gw, x, g, None, 1e-5, dresidual=dres, out=dres)
    assert got.data_ptr() == dres.data_ptr()
    assert torch.equal(got, want)


def _mlp_case(C, seed):
    cfg = workloads.CONFIGS["c3"]
    m = workloads.mlp_for(cfg, 1) if C == 192 else workloads.mlp_for(
        workloads.CONFIGS["c4" if C == 768 else "g1"], 1)
    with torch.no_grad():
        m.fc1.weight.mul_(4.0)
        m.fc2.weight.mul_(8.0)
        m.fc1.bias.copy_(workloads.activations(m.fc1.bias.shape, seed) * 0.1)
        m.fc2.bias.copy_(workloads.activations(m.fc2.bias.shape, seed + 1) * 0.1)
        m.norm2.weight.copy_(1.0 + 0.1 * workloads.activations((C,), seed + 2))
        m.norm2.bias.copy_(0.1 * workloads.activations((C,), seed + 3))
    return m


def _oracle_mlp_grads(m, x, gy, cd, bf16_weights=False):
    p = {k: v.detach().to(cd).clone() for k, v in m.state_dict().items()}
    if bf16_weights:
        p = {k: (v.to(torch.bfloat16).to(cd) if k.startswith("fc") else v) for k, v in p.items()}
    p = {k: v.requires_grad_(True) for k, v in p.items()}
    xr = x.to(cd).requires_grad_(True)
    h = torch.nn.functional.layer_norm(xr, (x.shape[-1],), p["norm2.weight"], p["norm2.bias"])
    h = torch.nn.functional.gelu(torch.nn.functional.linear(h, p["fc1.weight"], p["fc1.bias"]))
    y = torch.nn.functional.linear(h, p["fc2.weight"], p["fc2.bias"]) + xr
    y.backward(gy.to(cd))
    return y.detach(), xr.grad, {k: v.grad for k, v in p.items()}


def _normwise(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).norm() / ref.norm()).item()


@pytest.mark.parametrize("C", [192, 1024])
def test_mlp_backward_fp32(dev, C):
    """fp32 activations and parameters: the HIP LayerNorm forward / backward
    and fp32 GEMMs against float64 autograd, 1e-5 normwise per gradient."""
    m = _mlp_case(C, 520)
    x = workloads.activations((2, 150, C), 521)
    gy = workloads.activations((2, 150, C), 522)
    md = copy.deepcopy(m).to(dev)
    xd = x.to(dev).requires_grad_(True)
    y = md(xd)
    y.backward(gy.to(dev))
    yr, xg, pg = _oracle_mlp_grads(m, x, gy, torch.float64)
    assert _normwise(y.detach(), yr) <= 1e-5
    assert _normwise(xd.grad, xg) <= 1e-5
    for n, p in md.named_parameters():
        assert _normwise(p.grad, pg[n]) <= 1e-5, n


@pytest.mark.parametrize("C", [192, 768])
def test_mlp_backward_autocast(dev, C):
    """The reference's training mode: fp32 input and parameters under bf16
    autocast (bf16 GEMMs); every gradient within 3e-2 normwise of fp32
    autograd on bf16-rounded weights, and the module routes through the HIP
    LayerNorm kernels."""
    m = _mlp_case(C, 530)
    x = workloads.activations((2, 200, C), 531)
    gy = workloads.activations((2, 200, C), 532)
    md = copy.deepcopy(m).to(dev)
    calls = {"fwd": 0, "bwd": 0}
    f0, b0 = kernels.swin_partition_ln, kernels.swin_partition_ln_backward

    def cf(*a, **k):
        calls["fwd"] += 1
        return f0(*a, **k)

    def cb(*a, **k):
        calls["bwd"] += 1
        return b0(*a, **k)

    kernels.swin_partition_ln, kernels.swin_partition_ln_backward = cf, cb
    try:
        xd = x.to(dev).requires_grad_(True)
        with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
            y = md(xd)
        y.backward(gy.to(dev))
    finally:
        kernels.swin_partition_ln, kernels.swin_partition_ln_backward = f0, b0
    assert calls == {"fwd": 1, "bwd": 1}
    assert y.dtype == torch.float32
    yr, xg, pg = _oracle_mlp_grads(m, x, gy, torch.float32, bf16_weights=True)
    assert _normwise(y.detach(), yr) <= 2e-2
    assert _normwise(xd.grad, xg) <= 3e-2
    for n, p in md.named_parameters():
        assert p.grad is not None and p.grad.dtype == torch.float32, n
        assert _normwise(p.grad, pg[n]) <= 3e-2, n


def test_block_training_routes_layernorm_through_hip(dev):
    """A bf16 block's training forward / backward runs its LayerNorm on the
    fused gather and its backward kernel (no torch LayerNorm)."""
    cfg = workloads.CONFIGS["c3"].scaled(16, 32)
    blk = gain_block(workloads.block_for(cfg, 1)).to(dev).to(torch.bfloat16)
    calls = {"bwd": 0}
    b0 = kernels.swin_partition_ln_backward

    def cb(*a, **k):
        calls["bwd"] += 1
        return b0(*a, **k)

    ln_calls = {"n": 0}
    orig_ln = torch.nn.functional.layer_norm

    def count_ln(*a, **k):
        ln_calls["n"] += 1
        return orig_ln(*a, **k)

    kernels.swin_partition_ln_backward = cb
    torch.nn.functional.layer_norm = count_ln
    try:
        x = workloads.activations((1, 16 * 32, cfg.channels), 540, torch.bfloat16).to(dev).requires_grad_(True)
        blk(x).sum().backward()
    finally:
        kernels.swin_partition_ln_backward = b0
        torch.nn.functional.layer_norm = orig_ln
    assert calls["bwd"] == 1 and ln_calls["n"] == 0
    assert blk.norm1.weight.grad is not None and torch.isfinite(blk.norm1.weight.grad.float()).all()


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("residual", [False, True])
def test_partition_ln_mixed_equals_fp32_and_cast(dev, case, residual):
    """The mixed-dtype forms (fp32 x, bf16 windows / bf16 windows gradient)
    that bf16-autocast training uses: the forward equals the fp32 LayerNorm +
    partition followed by a cast to bf16, and the backward equals the fp32
    backward on the bf16 gradient cast to fp32, bit for bit (dγ / dβ up to
    the atomics' summation order)."""
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    g = _geom(*case)
    x = (workloads.activations((B, H, W, C), 510) * 2 + 0.3).to(dev)
    w = (workloads.activations((C,), 511) * 0.2 + 1.0).to(dev)
    b = (workloads.activations((C,), 512) * 0.2).to(dev)
    want = kernels.swin_partition_ln(x, g, w, b, 1e-5, pad_value=0.5).to(torch.bfloat16)
    got = kernels.swin_partition_ln(x, g, w, b, 1e-5, pad_value=0.5, out_dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    gw = workloads.activations((g.num_windows, ws * ws, C), 513).to(torch.bfloat16).to(dev)
    dres = workloads.activations((B, H, W, C), 514).to(dev) if residual else None
    dw0, db0 = torch.zeros(C, device=dev), torch.zeros(C, device=dev)
    dw1, db1 = torch.zeros(C, device=dev), torch.zeros(C, device=dev)
    want_dx = kernels.swin_partition_ln_backward(gw.float(), x, g, w, 1e-5, dresidual=dres, dweight=dw0, dbias=db0)
    got_dx = kernels.swin_partition_ln_backward(gw, x, g, w, 1e-5, dresidual=dres, dweight=dw1, dbias=db1)
    assert got_dx.dtype == torch.float32
    assert torch.equal(got_dx, want_dx)
    assert _rel(dw1, dw0) < 1e-5 and _rel(db1, db0) < 1e-5


def test_partition_ln_mixed_rejects_other_pairs(dev):
    g = WindowGeometry(1, 8, 8, 64, 8)
    x = torch.zeros((1, 8, 8, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        kernels.swin_partition_ln(x, g, None, None, 1e-5, out_dtype=torch.float32)
    with pytest.raises(ValueError):
        kernels.swin_partition_ln_backward(torch.zeros((1, 64, 64), dtype=torch.float16, device=dev), x.float(), g,
                                           None, 1e-5)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("residual", [False, True])
def test_reverse_mixed_equals_widen_and_reverse(dev, case, residual):
    """bf16 windows into an fp32 grid (plus an fp32 residual): bit for bit
    the fp32 reverse of the windows cast to fp32 (the widening is exact and
    the add is the fp32 add either way)."""
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    g = _geom(*case)
    win = workloads.activations((g.num_windows, ws * ws, C), 520).to(torch.bfloat16).to(dev)
    res = (workloads.activations((B, H, W, C), 521) * 3).to(dev) if residual else None
    want = kernels.swin_reverse(win.float(), g, residual=res)
    got = kernels.swin_reverse(win, g, residual=res, out_dtype=torch.float32)
    assert got.dtype == torch.float32
    assert torch.equal(got, want)
    if residual:  # in place on the residual
        res2 = res.clone()
        kernels.swin_reverse(win, g, residual=res2, out=res2, out_dtype=torch.float32)
        assert torch.equal(res2, want)


def _sum_bound(vals: torch.Tensor, dims) -> torch.Tensor:
    """Worst-case error of fp32 summation in any order: n u sum |x| (n terms,
    u = 2^-24), per column."""
    n = 1
    for d in dims:
        n *= vals.shape[d]
    return n * 2.0 ** -24 * vals.double().abs().sum(dims).cpu() + 1e-30


@pytest.mark.parametrize("case", CASES)
def test_partition_mixed_equals_partition_and_cast(dev, case):
    """fp32 grid into bf16 windows: bit for bit the fp32 partition followed
    by a cast (pad slots included), and the column sums of the values written
    within the fp32 summation bound of their float64 sums; the sums
    accumulate over calls."""
    B, H, W, C, ws, s, pad, r0, rows, valid = case
    g = _geom(*case)
    x = (workloads.activations((B, H, W, C), 522) * 3).to(dev)
    want = kernels.swin_partition(x, g, pad_value=0.5).to(torch.bfloat16)
    sums = torch.zeros(C, device=dev)
    got = kernels.swin_partition(x, g, pad_value=0.5, out_dtype=torch.bfloat16, column_sums=sums)
    assert got.dtype == torch.bfloat16
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    ref = want.double().sum((0, 1)).cpu()
    bound = _sum_bound(want, (0, 1))
    assert ((sums.double().cpu() - ref).abs() <= bound).all()
    got2 = kernels.swin_partition(x, g, pad_value=0.5, out_dtype=torch.bfloat16, column_sums=sums)
    assert torch.equal(got2.view(torch.int16), want.view(torch.int16))
    assert ((sums.double().cpu() - 2 * ref).abs() <= 2 * bound).all()
    # without sums; and the identity frame over token rows (the MLP half's cast)
    assert torch.equal(kernels.swin_partition(x, g, pad_value=0.5, out_dtype=torch.bfloat16).view(torch.int16),
                       want.view(torch.int16))
    T = B * H * W
    rows_sums = torch.zeros(C, device=dev)
    flat = kernels.swin_partition(x.view(1, T, 1, C), kernels.rows_geometry(T, C), out_dtype=torch.bfloat16,
                                  column_sums=rows_sums).view(T, C)
    assert torch.equal(flat.view(torch.int16), x.view(T, C).to(torch.bfloat16).view(torch.int16))
    assert ((rows_sums.double().cpu() - flat.double().sum(0).cpu()).abs() <= _sum_bound(flat, (0,))).all()


def _gelu_grad64(g: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """d/dh of 0.5 h (1 + erf(h / sqrt 2)) times g, in float64."""
    g, h = g.double().cpu(), h.double().cpu()
    cdf = 0.5 * (1 + torch.erf(h / 2 ** 0.5))
    pdf = torch.exp(-0.5 * h * h) / (2 * torch.pi) ** 0.5
    return g * (cdf + h * pdf)


@pytest.mark.parametrize("dtype,features", [(torch.bfloat16, 256), (torch.bfloat16, 512), (torch.bfloat16, 768),
                                            (torch.bfloat16, 1536),
                                            (torch.bfloat16, 3072), (torch.bfloat16, 4096), (torch.float32, 768),
                                            (torch.float32, 2048)])
@pytest.mark.parametrize("rows", [1, 37, 2053])
def test_gelu_backward(dev, dtype, features, rows):
    """terra_swin_gelu_bwd against the float64 derivative (one rounding to
    the dtype plus fp32 arithmetic: 2^-8 relative for bf16, 1e-6 for fp32,
    with an absolute floor of 1e-6 of the tensor's scale for values that
    cancel to near zero) and against torch's gelu_backward (at most one bf16
    unit in the last place, and equal for at least 99.9 % of the values);
    fc1's bias gradient (the column sums of the values written) within the
    fp32 summation bound."""
    h = (workloads.activations((rows, features), 530) * 2.5).to(dtype).to(dev)
    gy = workloads.activations((rows, features), 531).to(dtype).to(dev)
    sums = torch.zeros(features, device=dev)
    got = kernels.gelu_backward(gy, h, column_sums=sums)
    assert got.dtype == dtype and got.shape == h.shape
    ref = _gelu_grad64(gy, h)
    rel = 2.0 ** -8 if dtype == torch.bfloat16 else 1e-6
    err = (got.double().cpu() - ref).abs()
    assert (err <= rel * ref.abs() + 1e-6 * ref.abs().max()).all(), err.max().item()
    want = torch.ops.aten.gelu_backward(gy, h)
    if dtype == torch.bfloat16:
        gi, wi = got.view(torch.int16).int().cpu(), want.view(torch.int16).int().cpu()
        assert (gi - wi).abs().max().item() <= 1
        assert (gi == wi).float().mean().item() >= 0.999
    else:
        assert ((got - want).abs() <= 1e-6 * want.abs() + 1e-30).float().mean().item() >= 0.999
    assert ((sums.double().cpu() - got.double().sum(0).cpu()).abs() <= _sum_bound(got, (0,))).all()
    # without sums: the same values
    assert torch.equal(kernels.gelu_backward(gy, h), got)


def test_gelu_backward_special_values(dev):
    """Zeros, tiny and huge inputs, infinities and NaN give torch's values."""
    vals = [0.0, -0.0, 1e-30, -1e-30, 2.0 ** -26, -(2.0 ** -20), 0.5, -0.5, 3.0, -3.0, 6.0, -6.0, 32.0, -32.0,
            1e4, -1e4, float("inf"), float("-inf"), float("nan")]
    h = torch.tensor(vals * 8, dtype=torch.float32)[:152].view(1, 152)
    h = torch.cat([h, torch.zeros(1, 8)], 1).to(torch.bfloat16).to(dev)  # 160 features: 20 chunks
    gy = torch.full(h.shape, -1.5, dtype=torch.bfloat16, device=dev)
    got = kernels.gelu_backward(gy, h)
    want = torch.ops.aten.gelu_backward(gy, h)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    fin = ~torch.isnan(want)
    assert torch.equal(got[fin], want[fin])


def test_gelu_backward_rejects_bad_arguments(dev):
    h = torch.zeros((4, 12), dtype=torch.bfloat16, device=dev)  # 24-byte rows
    with pytest.raises(ValueError, match="16-byte"):
        kernels.gelu_backward(h, h)
    h = torch.zeros((4, 16), dtype=torch.float16, device=dev)
    with pytest.raises(TypeError):
        kernels.gelu_backward(h, h)
    h = torch.zeros((4, 16), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        kernels.gelu_backward(h, h, column_sums=torch.zeros(8, device=dev))
    with pytest.raises(ValueError, match="overlap"):  # dh overlapping dout
        kernels.gelu_backward(h, h.clone(), out=h)


def test_mlp_backward_autocast_routes_through_fused_kernels(dev):
    """Under autocast the MLP half's backward casts the output gradient with
    terra_swin_partition_mixed (fc2's bias gradient summed there) and runs
    the GELU derivative on terra_swin_gelu_bwd (fc1's bias gradient summed
    there): one call each."""
    m = _mlp_case(192, 560)
    md = copy.deepcopy(m).to(dev)
    calls = {"part": 0, "gelu": 0}
    p0, g0 = kernels.swin_partition, kernels.gelu_backward

    def cp(*a, **k):
        if k.get("column_sums") is not None:
            calls["part"] += 1
        return p0(*a, **k)

    def cg(*a, **k):
        calls["gelu"] += 1
        return g0(*a, **k)

    kernels.swin_partition, kernels.gelu_backward = cp, cg
    try:
        x = workloads.activations((2, 96, 192), 561).to(dev).requires_grad_(True)
        with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
            y = md(x)
        y.backward(workloads.activations(tuple(y.shape), 562).to(dev))
    finally:
        kernels.swin_partition, kernels.gelu_backward = p0, g0
    assert calls["part"] == 1 and calls["gelu"] == 1
    assert md.fc1.bias.grad is not None and md.fc2.bias.grad is not None


def test_block_autocast_training_sums_biases_in_kernels(dev):
    """A block's training step under autocast: the scatter's backward writes
    proj's bf16 output gradient with its column sums (terra_swin_partition_mixed)
    and the attention core's backward sums the q | k | v gradient
    (terra_swin_attn_bwd_sums); the forward's scatter widens the bf16 proj
    output itself (terra_swin_reverse_mixed).  The bias gradients equal the
    column sums torch takes of the same gradients, within the fp32 summation
    bound."""
    cfg = workloads.CONFIGS["c3"].scaled(16, 32)
    blk = gain_block(workloads.block_for(cfg, 1)).to(dev)
    calls = {"part": 0, "attn": 0, "rev": 0}
    p0, a0, r0 = kernels.swin_partition, kernels.window_attention_backward, kernels.swin_reverse
    seen = {}

    def cp(*a, **k):
        if k.get("column_sums") is not None:
            calls["part"] += 1
            out = p0(*a, **k)
            seen["dproj"] = out.detach().clone()
            return out
        return p0(*a, **k)

    def ca(*a, **k):
        if k.get("column_sums") is not None:
            calls["attn"] += 1
            outs = a0(*a, **k)
            seen["dqkv"] = torch.cat([t.detach() for t in outs], -1).clone()
            return outs
        return a0(*a, **k)

    def cr(*a, **k):
        if k.get("out_dtype") == torch.float32 and a[0].dtype == torch.bfloat16:
            calls["rev"] += 1
        return r0(*a, **k)

    kernels.swin_partition, kernels.window_attention_backward, kernels.swin_reverse = cp, ca, cr
    try:
        x = workloads.activations((1, 16 * 32, cfg.channels), 570).to(dev).requires_grad_(True)
        with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
            y = blk(x)
        y.backward(workloads.activations(tuple(y.shape), 571).to(dev))
    finally:
        kernels.swin_partition, kernels.window_attention_backward, kernels.swin_reverse = p0, a0, r0
    assert calls == {"part": 1, "attn": 1, "rev": 1}
    C = cfg.channels
    dproj = seen["dproj"].reshape(-1, C)
    want = dproj.double().sum(0).cpu()
    got = blk.attn.proj.bias.grad.double().cpu()
    assert ((got - want).abs() <= dproj.shape[0] * 2.0 ** -24 * dproj.double().abs().sum(0).cpu() + 1e-30).all()
    dqkv = seen["dqkv"].reshape(-1, 3 * C)
    want = dqkv.double().sum(0).cpu()
    bound = dqkv.shape[0] * 2.0 ** -24 * dqkv.double().abs().sum(0).cpu() + 1e-30
    got = torch.cat([blk.attn.q_linear.bias.grad, blk.attn.k_linear.bias.grad, blk.attn.v_linear.bias.grad])
    assert ((got.double().cpu() - want).abs() <= bound).all()
