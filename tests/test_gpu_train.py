"""The training path's LayerNorm kernels: the backward of the fused
LayerNorm + partition (terra_swin_partition_ln_bwd), alone and inside the
block, and the MLP half's backward (autograd.mlp), against torch autograd of
the oracle's restatement.

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
