"""GPU parity of the token-row linear kernels (terra_swin_linear,
terra_swin_linear_residual): the GEMM against a float64 CPU product of the
same bf16 operands, and the epilogues (GELU, residual add, the scatter back to
the grid) bit-exact where the GEMM is exact (an identity weight)."""
import pytest
import torch

from oracle import swin_oracle as so
from terra_amd import kernels, workloads
from terra_amd.kernels import WindowGeometry

pytestmark = pytest.mark.gpu


def _weights(n, k, seed, scale=0.03):
    w = (workloads.activations((n, k), seed) * scale).to(torch.bfloat16)
    b = workloads.activations((n,), seed + 1) * 0.1
    return w, b


def _ref_linear(x, w, b):
    """float64 x W^T + b of the bf16 operands (the fp32-bias module's sum)."""
    return x.double() @ w.double().t() + b.double()


def _assert_bf16_close(got, want64, what):
    """got (bf16) against the exact sum rounded to bf16: fp32 accumulation in
    another order may land one bf16 step away, nothing more."""
    got = got.double().cpu()
    want = want64.float().bfloat16().double()
    step = want.abs().clamp_min(2.0 ** -30) * 2.0 ** -7  # one bf16 ulp or less
    bad = (got - want).abs() > step + 1e-6
    assert bad.float().mean().item() < 1e-3, f"{what}: {int(bad.sum())} of {bad.numel()} values off by more than 1 ulp"
    rel = ((got - want64).norm() / want64.norm()).item()
    assert rel < 4e-3, f"{what}: normwise error {rel:.2e}"


@pytest.mark.parametrize("rows,k,n", [(512, 64, 256), (700, 1024, 1024), (300, 1024, 4096), (256, 4096, 1024),
                                      (1, 64, 256)])
def test_linear_store_against_float64(dev, rows, k, n):
    x = workloads.activations((rows, k), 11).to(torch.bfloat16)
    w, b = _weights(n, k, 12)
    got = kernels.linear(x.to(dev), kernels.pack_linear(w.to(dev)), n, b.to(dev))
    torch.cuda.synchronize()
    _assert_bf16_close(got, _ref_linear(x, w, b), f"linear {rows}x{k}->{n}")


def test_linear_without_bias_and_strided_rows_of_a_batch(dev):
    x = workloads.activations((3, 100, 256), 13).to(torch.bfloat16)
    w, _ = _weights(512, 256, 14)
    got = kernels.linear(x.to(dev), kernels.pack_linear(w.to(dev)), 512)
    assert got.shape == (3, 100, 512)
    _assert_bf16_close(got.reshape(-1, 512), x.reshape(-1, 256).double() @ w.double().t(), "no bias")


def _special_inputs(rows, n):
    """bf16 pre-activations covering the GELU table and its closed forms."""
    x = workloads.activations((rows, n), 15) * 3.0
    # (no inf / nan: the identity GEMM multiplies them by the zeros of W)
    specials = torch.tensor([0.0, -0.0, 2.0 ** -30, -(2.0 ** -30), 2.0 ** -22, -(2.0 ** -22), 31.875, -31.875, 32.0,
                             -32.0, 100.0, -100.0, 3e4, -3e4, 1e-3, -1e-3, 5.5, -5.5])
    x.view(-1)[: specials.numel()] = specials
    x.view(-1)[-specials.numel():] = specials
    return x.to(torch.bfloat16)


def test_linear_gelu_bit_exact_with_identity_weight(dev):
    """W = I and a bf16 bias keep the sum exact (x + b in fp32, one rounding),
    so the output must equal nn.GELU of that bf16 tensor bit for bit,
    including the closed forms outside the table (|x| < 2^-22, |x| >= 32)."""
    rows, n = 300, 256
    x = _special_inputs(rows, n)
    b = (workloads.activations((n,), 16) * 0.5).to(torch.bfloat16).float()
    b[:32] = 0.0  # the special values of the first and last rows stay as they are
    b[-32:] = 0.0
    eye = torch.eye(n, dtype=torch.bfloat16)
    got = kernels.linear(x.to(dev), kernels.pack_linear(eye.to(dev)), n, b.to(dev), gelu=True)
    pre = (x.float() + b).bfloat16()
    want = torch.nn.functional.gelu(pre.to(dev))  # the module's op on the same bf16 tensor
    torch.cuda.synchronize()
    assert torch.equal(got.isnan(), want.isnan())
    ok = ~want.isnan()
    assert torch.equal(got[ok], want[ok])


@pytest.mark.parametrize("rows,k,n", [(513, 1024, 4096), (256, 256, 512)])
def test_linear_gelu_against_float64(dev, rows, k, n):
    x = workloads.activations((rows, k), 17).to(torch.bfloat16)
    w, b = _weights(n, k, 18, scale=0.06)
    got = kernels.linear(x.to(dev), kernels.pack_linear(w.to(dev)), n, b.to(dev), gelu=True).double().cpu()
    pre = _ref_linear(x, w, b).float().bfloat16().double()
    want = 0.5 * pre * (1.0 + torch.special.erf(pre / 2.0 ** 0.5))
    # the pre-activation may sit one bf16 step away (summation order); GELU's slope is below 1.13
    err = (got - want).abs()
    assert (err <= pre.abs() * 2.0 ** -7 * 1.2 + want.abs() * 2.0 ** -8 + 1e-6).float().mean().item() > 0.999
    assert ((got - want).norm() / want.norm()).item() < 4e-3


def test_linear_residual_bit_exact_with_identity_weight(dev):
    rows, n = 777, 512
    x = workloads.activations((rows, n), 19).to(torch.bfloat16)
    r = workloads.activations((rows, n), 20).to(torch.bfloat16)
    b = (workloads.activations((n,), 21) * 0.25).to(torch.bfloat16).float()
    eye = torch.eye(n, dtype=torch.bfloat16)
    got = kernels.linear_residual(x.to(dev), kernels.pack_linear(eye.to(dev)), n, r.to(dev), b.to(dev)).cpu()
    want = r + (x.float() + b).bfloat16()  # bf16 + bf16: fp32 sum, one rounding
    assert torch.equal(got, want)


def test_linear_residual_in_place_against_float64(dev):
    rows, k, n = 600, 4096, 1024
    x = workloads.activations((rows, k), 22).to(torch.bfloat16)
    r = workloads.activations((rows, n), 23).to(torch.bfloat16)
    w, b = _weights(n, k, 24, scale=0.01)
    rd = r.to(dev)
    got = kernels.linear_residual(x.to(dev), kernels.pack_linear(w.to(dev)), n, rd, b.to(dev), out=rd)
    assert got.data_ptr() == rd.data_ptr()
    y = _ref_linear(x, w, b).float().bfloat16().double()
    want = r.double() + y
    got = got.double().cpu()
    assert ((got - want).norm() / want.norm()).item() < 4e-3
    assert ((got - want).abs() <= want.abs() * 2.0 ** -7 + y.abs() * 2.0 ** -7 + 1e-6).float().mean().item() > 0.999


SCATTER_CASES = [  # (B, H, W, shift, pad): every window of the padded frame emitted
    (2, 16, 24, 4, (0, 0, 0, 0)),
    (1, 20, 36, 4, (0, 4, 0, 4)),
    (2, 13, 21, 0, (1, 2, 0, 3)),
    (1, 24, 40, 3, (0, 0, 0, 0)),
]


@pytest.mark.parametrize("case", SCATTER_CASES)
def test_linear_scatter_bit_exact_with_identity_weight(dev, case):
    """W = I: y must be the oracle's window reverse (+ roll, crop) plus the
    residual, bit for bit: the row map of the epilogue is the partition's."""
    B, H, W, s, pad = case
    C = 256
    geom = WindowGeometry(B, H, W, C, 8, s, s, pad)
    win = workloads.activations((geom.num_windows, 64, C), 25).to(torch.bfloat16)
    r = workloads.activations((B, H, W, C), 26).to(torch.bfloat16)
    eye = torch.eye(C, dtype=torch.bfloat16)
    got = kernels.linear_residual(win.to(dev), kernels.pack_linear(eye.to(dev)), C, r.to(dev), None, geom=geom).cpu()
    want = so.reverse_frame(win, B, H, W, 8, s, s, pad, residual=r)
    assert torch.equal(got, want)


@pytest.mark.parametrize("shape", [(1, 32, 48), (1, 288, 544)], ids=["small", "g1-grid"])
def test_linear_scatter_matches_proj_then_reverse(dev, shape):
    """proj + reverse + residual in one kernel against the five-stage order
    (torch's bf16 Linear, then the reverse kernel), C = 1024."""
    B, H, W = shape
    C = 1024
    geom = WindowGeometry(B, H, W, C, 8, 4, 4)
    o = workloads.activations((geom.num_windows, 64, C), 27).to(torch.bfloat16).to(dev)
    x = workloads.activations((B, H, W, C), 28).to(torch.bfloat16).to(dev)
    w, b = _weights(C, C, 29, scale=0.02)
    wd, bd = w.to(dev), b.to(dev)
    got = kernels.linear_residual(o, kernels.pack_linear(wd), C, x, bd, geom=geom)
    proj = torch.nn.functional.linear(o, wd, bd.to(torch.bfloat16))
    want = kernels.swin_reverse(proj.contiguous(), geom, residual=x)
    torch.cuda.synchronize()
    d = (got.float() - want.float())
    assert torch.isfinite(got.float()).all()
    assert (d.norm() / want.float().norm()).item() < 4e-3
    y = (want.float() - x.float())
    assert ((got.float() - x.float() - y).norm() / y.norm()).item() < 2e-2


def test_linear_empty_rows(dev):
    x = torch.empty(0, 256, dtype=torch.bfloat16, device=dev)
    w = kernels.pack_linear(torch.zeros(256, 256, dtype=torch.bfloat16, device=dev))
    assert kernels.linear(x, w, 256).shape == (0, 256)
    assert kernels.linear_residual(x, w, 256, torch.empty(0, 256, dtype=torch.bfloat16, device=dev)).shape == (0, 256)
