"""The drop-ins inside torch.amp.autocast("cuda", dtype=torch.bfloat16) with
fp32 parameters, the way the reference's training and evaluation steps run
its model (core/runtime/run_model.py:424-448).

Under bf16 autocast F.linear computes in bf16 from bf16-cast weights,
layer_norm and softmax in fp32, and `shortcut + x` promotes to the wider of
the two operands.  So:
  - bf16 activations: the fused half-block and MLP kernels serve the call
    (the module packs bf16 copies of its fp32 weights, as F.linear casts
    them) and the result is bf16;
  - fp32 activations: the five-stage path (fp32 LayerNorm + partition, bf16
    q/k/v and core, fp32 residual) and the reference's MLP sequence; the
    result is fp32.
Each is checked against the fp32 oracle on the same bf16-rounded weights with
the bf16 tolerances (2e-2 max-abs on y, 3e-2 normwise on y - x), and the
backward (fp32 input, fp32 parameters) against oracle autograd within 3e-2
normwise.  Weights are gained (helpers.gain_block) so the attention term is
O(1).
"""
import pytest
import torch

from helpers import assert_block_matches, gain_block, params_of
from oracle import swin_oracle as so
from terra_amd import kernels, workloads

pytestmark = pytest.mark.gpu

AUTOCAST = dict(device_type="cuda", dtype=torch.bfloat16)


def _bf16_weights(params: dict) -> dict:
    """The oracle's parameters as F.linear sees them under bf16 autocast:
    Linear weights and biases rounded to bf16, everything else fp32."""
    return {k: (v.bfloat16().float() if k.endswith(("weight", "bias")) and ("linear" in k or "proj" in k or "fc" in k)
                else v)
            for k, v in params.items()}


class _Count:
    def __init__(self, name):
        self.name, self.n = name, 0

    def __enter__(self):
        self.orig = getattr(kernels, self.name)

        def wrapped(*a, **kw):
            self.n += 1
            return self.orig(*a, **kw)

        setattr(kernels, self.name, wrapped)
        return self

    def __exit__(self, *exc):
        setattr(kernels, self.name, self.orig)


@pytest.mark.parametrize("name,layer,land", [("c3", 1, True), ("c5", 1, True), ("c3", 0, False)])
def test_block_autocast_bf16_activations_run_the_fused_kernel(dev, name, layer, land):
    cfg = workloads.CONFIGS[name].scaled(32, 64)
    lm = workloads.land_mask(cfg.height, cfg.width, seed=700) if land else None
    blk = gain_block(workloads.block_for(cfg, layer, land=lm)).to(dev)  # fp32 parameters
    x = workloads.activations((cfg.batch, cfg.height * cfg.width, cfg.channels), 701, torch.bfloat16)
    with torch.no_grad(), torch.amp.autocast(**AUTOCAST), _Count("swin_block") as calls:
        y = blk(x.to(dev))
    assert calls.n == 1, "the fused kernel did not serve the autocast call"
    assert y.dtype == torch.bfloat16
    ref = so.swin_block_attention(x, cfg.height, cfg.width, cfg.window, blk.shift_size, cfg.heads,
                                  _bf16_weights(params_of(blk)), land=lm)
    assert_block_matches(y, ref, x, 2e-2, 3e-2)


@pytest.mark.parametrize("layer", [0, 1])
def test_block_autocast_against_reference_autocast_sequence(dev, layer):
    """The fused kernel under autocast against the reference's own autocast op
    sequence (oracle.swin_block_attention_autocast_bf16: bf16 q/k/v with bf16
    biases, bf16 logits, bf16 P, bf16 proj), within the bf16 tolerances, and at
    least as close to the fp32 restatement as that sequence is (the kernel
    keeps the logits in fp32 and rounds neither q * scale nor q k^T)."""
    cfg = workloads.CONFIGS["c3"].scaled(32, 64)
    lm = workloads.land_mask(cfg.height, cfg.width, seed=708)
    blk = gain_block(workloads.block_for(cfg, layer, land=lm)).to(dev)
    x = workloads.activations((cfg.batch, cfg.height * cfg.width, cfg.channels), 709, torch.bfloat16)
    with torch.no_grad(), torch.amp.autocast(**AUTOCAST), _Count("swin_block") as calls:
        y = blk(x.to(dev))
    assert calls.n == 1
    p = params_of(blk)
    ac = so.swin_block_attention_autocast_bf16(x, cfg.height, cfg.width, cfg.window, blk.shift_size, cfg.heads, p,
                                               land=lm)
    assert_block_matches(y, ac.float(), x, 2e-2, 3e-2)
    ref = so.swin_block_attention(x, cfg.height, cfg.width, cfg.window, blk.shift_size, cfg.heads,
                                  _bf16_weights(p), land=lm).double()
    d_ref = ref - x.double()
    e_kernel = (torch.linalg.vector_norm(y.double().cpu() - x.double() - d_ref) / torch.linalg.vector_norm(d_ref)).item()
    e_ac = (torch.linalg.vector_norm(ac.double() - x.double() - d_ref) / torch.linalg.vector_norm(d_ref)).item()
    assert e_kernel <= 1.5 * e_ac + 1e-3, (e_kernel, e_ac)


@pytest.mark.parametrize("name", ["c3", "c4", "c2"])
def test_block_autocast_fp32_activations(dev, name):
    cfg = workloads.CONFIGS[name].scaled(32, 64) if name != "c2" else workloads.CONFIGS[name].scaled(28, 42)
    blk = gain_block(workloads.block_for(cfg, 1)).to(dev)
    x = workloads.activations((cfg.batch, cfg.height * cfg.width, cfg.channels), 702)
    with torch.no_grad(), torch.amp.autocast(**AUTOCAST), _Count("swin_block") as calls:
        y = blk(x.to(dev))
    assert calls.n == 0 and y.dtype == torch.float32
    ref = so.swin_block_attention(x, cfg.height, cfg.width, cfg.window, blk.shift_size, cfg.heads,
                                  _bf16_weights(params_of(blk)))
    assert_block_matches(y, ref, x, 2e-2, 3e-2)


def _normwise(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).norm() / ref.norm()).item()


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_block_autocast_backward(dev, name):
    """A training step's backward under autocast: fp32 input and parameters,
    bf16 GEMMs and attention kernels inside; the input gradient and every
    parameter gradient against oracle autograd (fp32, bf16-rounded weights)."""
    cfg = workloads.CONFIGS[name].scaled(32, 48)
    lm = workloads.land_mask(32, 48, seed=703)
    blk = gain_block(workloads.block_for(cfg, 1, land=lm))
    params = {n: p.detach().clone() for n, p in blk.named_parameters()}
    params = {n: v.requires_grad_(True) for n, v in _bf16_weights(params).items()}
    blk = blk.to(dev)
    x = workloads.activations((2, 32 * 48, cfg.channels), 704)
    gy = workloads.activations(tuple(x.shape), 705)
    xd = x.to(dev).requires_grad_(True)
    with torch.amp.autocast(**AUTOCAST):
        y = blk(xd)
    y.backward(gy.to(dev))
    xr = x.clone().requires_grad_(True)
    yr = so.swin_block_attention(xr, 32, 48, cfg.window, blk.shift_size, cfg.heads, params, land=lm)
    yr.backward(gy)
    assert _normwise(y.detach(), yr.detach()) <= 2e-2
    assert _normwise(xd.grad, xr.grad) <= 3e-2
    for n, p in blk.named_parameters():
        assert p.grad is not None and p.grad.dtype == torch.float32, n
        if n == "attn.k_linear.bias":  # 0 in exact arithmetic (softmax ignores q . b_k)
            assert p.grad.double().norm().item() <= 3e-2 * params["attn.q_linear.bias"].grad.norm().item()
            continue
        assert _normwise(p.grad, params[n].grad) <= 3e-2, n


@pytest.mark.parametrize("C", [128, 192, 768])
def test_mlp_autocast(dev, C):
    """bf16 activations: the fused MLP kernel from fp32 parameters; fp32
    activations: the reference's torch sequence under autocast."""
    cfg = workloads.CONFIGS["c3"]
    mlp = workloads.mlp_for(cfg, 1) if C == 192 else workloads.mlp_for(
        workloads.CONFIGS["c2" if C == 128 else "c4"], 1)
    with torch.no_grad():
        mlp.fc1.weight.mul_(4.0)
        mlp.fc2.weight.mul_(8.0)
    mlp = mlp.to(dev)
    p = {k: v.detach().float().cpu() for k, v in mlp.state_dict().items()}
    for dtype in (torch.bfloat16, torch.float32):
        x = workloads.activations((3, 100, C), 706, dtype)
        with torch.no_grad(), torch.amp.autocast(**AUTOCAST), _Count("swin_mlp") as calls:
            y = mlp(x.to(dev))
        assert calls.n == (1 if dtype == torch.bfloat16 else 0)
        assert y.dtype == dtype
        ref = so.mlp(x.float(), _bf16_weights(p))
        d = (ref - x.float()).abs().max().item()
        assert d > 0.5
        err = (y.float().cpu() - ref).abs().max().item()
        assert err <= 2e-2 * ref.abs().max().item() + 2e-2 * d, (dtype, err, d)
