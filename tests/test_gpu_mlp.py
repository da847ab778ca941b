"""The fused MLP half-block kernel (LayerNorm + fc1 + GELU + fc2 + residual in
one launch, ``terra_swin_mlp_fwd``) against the oracle's bf16 restatement
(``oracle.swin_oracle.mlp_bf16``, float64 arithmetic rounded where a bf16
module rounds) and against the reference's own torch module sequence in bf16
on the GPU.

Tolerances: kernel and oracle round the same intermediates to bf16 and differ
only in summation order (fp32 MFMA accumulation against float64), so an
output differs by at most one bf16 ulp of y plus the effect of an occasional
one-ulp flip of a hidden value: elementwise |y - ref| <= 2^-7 |ref| +
1e-2 max|delta|, with delta = ref - x the MLP's contribution, and at least
90 % of the outputs are bit-equal.  The GELU table is checked bit-exactly
against torch's GPU GELU over every finite bf16 input.  Rows are independent,
so a full-size run is checked on sampled rows and bit-exactly against a
second launch over just those rows.
"""
import pytest
import torch

from oracle import brute
from oracle import swin_oracle as so
from terra_amd import config, kernels, workloads
from terra_amd.mlp import SequentialMlp

pytestmark = pytest.mark.gpu


def _params(C, seed, ln=True):
    g = workloads.generator(seed)
    H = 4 * C
    p = {
        "fc1.weight": (torch.randn(H, C, generator=g) / C ** 0.5).bfloat16(),
        "fc1.bias": 0.1 * torch.randn(H, generator=g),
        "fc2.weight": (torch.randn(C, H, generator=g) / H ** 0.5).bfloat16(),
        "fc2.bias": 0.1 * torch.randn(C, generator=g),
    }
    if ln:
        p["norm2.weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        p["norm2.bias"] = 0.1 * torch.randn(C, generator=g)
    return p


def _run(x, p, dev, ln=True, out=None):
    packed = {k: kernels.pack_linear(p[k].to(dev).contiguous()) for k in ("fc1.weight", "fc2.weight")}
    f = {k: v.to(dev) for k, v in p.items() if "weight" not in k or "norm" in k}
    return kernels.swin_mlp(x, packed["fc1.weight"], f["fc1.bias"], packed["fc2.weight"], f["fc2.bias"],
                            ln_weight=f.get("norm2.weight"), ln_bias=f.get("norm2.bias"), layernorm=ln, out=out)


def _check(y, x, ref):
    y, x, ref = y.double().cpu(), x.double().cpu(), ref.double().cpu()
    delta = (ref - x).abs().max()
    err = (y - ref).abs()
    assert bool((err <= 2.0 ** -7 * ref.abs() + 1e-2 * delta).all()), (err.max().item(), delta.item())
    assert (y == ref).double().mean().item() >= 0.9


@pytest.mark.parametrize("C", [128, 192, 384, 768])
@pytest.mark.parametrize("ln", [True, False])
@pytest.mark.parametrize("tokens", [1, 63, 1000])
def test_mlp_kernel_matches_oracle(dev, C, ln, tokens):
    p = _params(C, 7 + C + tokens, ln)
    x = workloads.activations((tokens, C), 11 + tokens, torch.bfloat16)
    y = _run(x.to(dev), p, dev, ln)
    ref = so.mlp_bf16(x, p, use_layernorm=ln)
    _check(y, x, ref)


@pytest.mark.parametrize("C,tokens", [(192, 256 * 64 * 3 + 37), (384, 256 * 64 * 2 + 5), (128, 256 * 64 * 3 + 37),
                                      (768, 256 * 64 * 2 + 5)])
def test_mlp_kernel_many_tiles_per_workgroup(dev, C, tokens):
    """Several 64-token tiles per persistent workgroup (double-buffered rows
    for C = 128 and 192; for C = 768 the rows share the LayerNorm tile) and a
    ragged last tile: sampled rows against the oracle, and every sampled row
    bit-equal to a launch over the sampled rows alone."""
    p = _params(C, 21 + C)
    x = workloads.activations((tokens, C), 23, torch.bfloat16)
    xd = x.to(dev)
    y = _run(xd, p, dev)
    g = workloads.generator(5)
    idx = torch.cat([torch.arange(0, 70), torch.arange(tokens - 70, tokens),
                     torch.randint(0, tokens, (1500,), generator=g)])
    _check(y.cpu()[idx], x[idx], so.mlp_bf16(x[idx], p))
    y_rows = _run(xd[idx.to(dev)].contiguous(), p, dev)
    assert torch.equal(y_rows.cpu(), y.cpu()[idx])


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_mlp_kernel_config_size_row_independence(dev, name):
    """The token grids of c2 (C = 128), c3 (C = 192) and c4 (C = 768) at full
    size, as the bench runs them."""
    cfg = workloads.CONFIGS[name]
    C = cfg.channels
    tokens = cfg.batch * cfg.height * cfg.width
    p = _params(C, 31)
    x = workloads.activations((tokens, C), 33, torch.bfloat16).to(dev)
    y = _run(x, p, dev)
    idx = torch.randint(0, tokens, (2000,), generator=workloads.generator(6)).to(dev)
    _check(y[idx], x[idx], so.mlp_bf16(x[idx].cpu(), p))
    assert torch.equal(_run(x[idx].contiguous(), p, dev), y[idx])


@pytest.mark.parametrize("C", [192, 768])
def test_mlp_kernel_in_place(dev, C):
    tokens = 777
    p = _params(C, 41)
    x = workloads.activations((tokens, C), 43, torch.bfloat16).to(dev)
    y = _run(x, p, dev)
    x2 = x.clone()
    out = _run(x2, p, dev, out=x2)
    assert out.data_ptr() == x2.data_ptr()
    assert torch.equal(x2, y)


@pytest.mark.parametrize("C", [128, 192, 384, 768])
def test_gelu_table_every_finite_bf16_input(dev, C):
    """fc1 = [I; 0] and fc2 = [I, 0] without LayerNorm make the MLP
    y = bf16(x + GELU(x)) exactly (one unit product per accumulation), so
    every finite bf16 value of x checks one GELU table entry or closed-form
    range against torch's own bf16 GELU on the GPU."""
    H = 4 * C
    bits = torch.arange(0, 1 << 16, dtype=torch.int32)
    finite = (bits & 0x7F80) != 0x7F80
    vals = bits[finite].to(torch.int16).view(torch.bfloat16)
    n = vals.numel()
    rows = (n + C - 1) // C
    x = torch.zeros(rows * C, dtype=torch.bfloat16)
    x[:n] = vals
    x = x.view(rows, C)
    eye = torch.eye(C)
    p = {"fc1.weight": torch.cat([eye, torch.zeros(H - C, C)]).bfloat16(), "fc1.bias": torch.zeros(H),
         "fc2.weight": torch.cat([eye, torch.zeros(C, H - C)], 1).bfloat16(), "fc2.bias": torch.zeros(C)}
    xd = x.to(dev)
    y = _run(xd, p, dev, ln=False)
    ref = (xd.float() + torch.nn.functional.gelu(xd).float()).bfloat16()
    assert torch.equal(y, ref)  # == on values: -0 and +0 compare equal
    # and within one bf16 ulp of GELU computed exactly (float64 erf)
    # for inputs whose GELU is a normal number (|x| >= 2^-124; the subnormal
    # range is covered by the comparison above); x + GELU(x) = 2x overflows to
    # inf for x > 2^127, in torch as here
    xs = x.view(-1)[:n:17].double()
    ys = y.view(-1)[:n:17].double().cpu()
    fin = torch.isfinite(ys)
    assert bool((xs[~fin] > 2.0 ** 127).all())
    sel = fin & (xs.abs() >= 2.0 ** -124)
    g = torch.tensor([brute.gelu(float(v)) for v in xs[sel]], dtype=torch.float64)
    err = (ys[sel] - xs[sel] - g).abs()
    assert bool((err <= 2.0 ** -7 * (xs[sel].abs() + g.abs())).all())


def test_gelu_table_special_values(dev):
    """GELU(+inf) = +inf and GELU(-inf) = NaN: with fc1 = [I; 0], an fc1 bias
    of +-3e38 on one hidden unit and x = +-3e38 in that channel, the fp32
    accumulation overflows to +-inf there and nowhere else in the row.  A NaN
    input makes its whole row NaN (0 * NaN in fc1).  Rows are independent."""
    C = 192
    b1 = torch.zeros(4 * C)
    b1[5], b1[7] = 3e38, -3e38
    p = {"fc1.weight": torch.cat([torch.eye(C), torch.zeros(3 * C, C)]).bfloat16(), "fc1.bias": b1,
         "fc2.weight": torch.cat([torch.eye(C), torch.zeros(C, 3 * C)], 1).bfloat16(), "fc2.bias": torch.zeros(C)}
    x = workloads.activations((4, C), 51, torch.bfloat16)
    x[1, 5] = 3e38
    x[2, 7] = -3e38
    x[3, 9] = float("nan")
    y = _run(x.to(dev), p, dev, ln=False).cpu()
    assert y[1, 5] == float("inf")           # x + GELU(inf)
    assert torch.isnan(y[2, 7])              # x + GELU(-inf) = x + NaN
    assert torch.isnan(y[3]).all()
    h = (x[0].float() + b1[:C]).bfloat16()   # fc1 output of row 0 (finite)
    ref0 = (x[0].float() + torch.nn.functional.gelu(h.to(dev)).float().cpu()).bfloat16()
    assert torch.equal(y[0], ref0)


@pytest.mark.parametrize("C", [128, 192, 384, 768])
def test_module_fused_matches_torch_bf16_module(dev, C):
    """SequentialMlp's kernel path against the same module run as the
    reference's torch sequence in bf16 on the GPU (use_fused_mlp = False),
    and the state dict keeps the reference's names."""
    torch.manual_seed(0)
    m = SequentialMlp(C, 4 * C, init_seed_base=workloads.SEED_BASE).to(dev).to(torch.bfloat16)
    assert sorted(m.state_dict()) == ["fc1.bias", "fc1.weight", "fc2.bias", "fc2.weight", "norm2.bias",
                                      "norm2.weight"]
    with torch.no_grad():
        m.norm2.weight.uniform_(0.5, 1.5)
        m.fc2.weight.mul_(8.0)  # the MLP's delta comparable to x
    x = workloads.activations((2, 300, C), 61, torch.bfloat16).to(dev)
    with torch.no_grad():
        y = m(x)
        m.use_fused_mlp = False
        ref = m(x)
        m.use_fused_mlp = True
    assert y.shape == x.shape
    d = (ref.float() - x.float()).abs().max()
    assert ((y.float() - ref.float()).abs() <= 2.0 ** -6 * ref.float().abs() + 2e-2 * d).all()
    # and against the oracle (module parameters in their bf16 / fp32 form)
    p = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    p = {k: (v if "fc" in k and "weight" in k else v.float()) for k, v in p.items()}
    _check(y.view(-1, C), x.view(-1, C).cpu(), so.mlp_bf16(x.view(-1, C).cpu(), p))


def test_module_caches_packed_weights_until_a_parameter_changes(dev):
    m = SequentialMlp(192, 768).to(dev).to(torch.bfloat16)
    x = workloads.activations((1, 64, 192), 71, torch.bfloat16).to(dev)
    with torch.no_grad():
        y0 = m(x)
        a = m._fused_cache[1]["fc1_weight"]
        m(x)
        assert m._fused_cache[1]["fc1_weight"] is a
        m.fc2.bias.add_(1.0)
        y1 = m(x)
    assert m._fused_cache[1]["fc1_weight"] is not a
    assert not torch.equal(y0, y1)


def test_module_unsupported_shapes_run_the_torch_sequence(dev):
    """fp32 activations (c1) are outside the kernel: the module runs norm2 /
    fc1 / GELU / fc2 / + x as torch ops (the reference's sequence), and
    gradients flow through it."""
    m = SequentialMlp(96, 384).to(dev)
    x = workloads.activations((2, 49, 96), 81).to(dev).requires_grad_(True)
    y = m(x)
    ref = so.mlp(x.detach().cpu(), {k: v.cpu() for k, v in m.state_dict().items()})
    assert torch.allclose(y.detach().cpu(), ref, rtol=1e-4, atol=1e-4)
    y.sum().backward()
    assert x.grad is not None and m.fc1.weight.grad is not None


def test_module_mlp_switch_off_is_identity(dev, monkeypatch):
    monkeypatch.setattr(config, "use_MLP", False)
    m = SequentialMlp(192, 768).to(dev).to(torch.bfloat16)
    assert not any(p.requires_grad for p in m.parameters())
    x = workloads.activations((1, 64, 192), 91, torch.bfloat16).to(dev)
    assert m(x) is x


@pytest.mark.parametrize("tokens", [1, 300, 2 * 288 * 544 // 64])
def test_module_c1024_linear_kernels_match_oracle(dev, tokens):
    """C = 1024 (TERRA's pretrain width): the module runs the HIP LayerNorm,
    fc1 + GELU on the linear kernel and fc2 + x on hipBLASLt; against the
    oracle and against the module's own torch sequence in bf16."""
    C = 1024
    m = SequentialMlp(C, 4 * C, init_seed_base=workloads.SEED_BASE).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        m.norm2.weight.uniform_(0.5, 1.5)
        m.norm2.bias.uniform_(-0.1, 0.1)
        m.fc1.bias.uniform_(-0.2, 0.2)
        m.fc2.weight.mul_(8.0)
    x = workloads.activations((1, tokens, C), 91, torch.bfloat16).to(dev)
    with torch.no_grad():
        assert m._gemm_path(x)
        y = m(x)
        m.use_fused_mlp = False
        ref_mod = m(x)
        m.use_fused_mlp = True
    d = (ref_mod.float() - x.float()).abs().max()
    assert ((y.float() - ref_mod.float()).abs() <= 2.0 ** -6 * ref_mod.float().abs() + 2e-2 * d).all()
    p = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    p = {k: (v if "fc" in k and "weight" in k else v.float()) for k, v in p.items()}
    rows = torch.arange(tokens) if tokens <= 300 else torch.randperm(tokens, generator=workloads.generator(9))[:300]
    xr = x.view(-1, C).cpu()[rows]
    _check(y.view(-1, C).cpu()[rows], xr, so.mlp_bf16(xr, p))
