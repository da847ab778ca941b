"""Empty inputs (a batch of 0 images or 0 windows) give empty outputs, as the
reference's torch ops do, on every path: the fused half-block, the five-stage
path, its backward, the attention core and the MLP."""
import pytest
import torch

from terra_amd import kernels, workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c3", "c4", "c2"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fused", [True, False])
def test_block_empty_batch(dev, name, dtype, fused):
    cfg = workloads.CONFIGS[name].scaled(16, 32) if name != "c2" else workloads.CONFIGS[name].scaled(14, 28)
    blk = workloads.block_for(cfg, 1).to(dev).to(dtype)
    blk.use_fused_block = fused
    x = torch.zeros(0, cfg.height * cfg.width, cfg.channels, device=dev, dtype=dtype)
    with torch.no_grad():
        y = blk(x)
    assert y.shape == x.shape and y.dtype == dtype


def test_block_empty_batch_backward(dev):
    cfg = workloads.CONFIGS["c3"].scaled(16, 32)
    blk = workloads.block_for(cfg, 1).to(dev)
    x = torch.zeros(0, cfg.height * cfg.width, cfg.channels, device=dev, requires_grad=True)
    y = blk(x)
    y.sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape
    assert all(p.grad is None or bool((p.grad == 0).all()) for p in blk.parameters())


def test_attention_core_no_windows(dev):
    q = torch.zeros(0, 64, 192, device=dev, dtype=torch.bfloat16)
    table = torch.zeros(225, 6, device=dev)
    o = kernels.window_attention(q, q, q, 6, (8, 8), 0.17, bias_table=table)
    assert o.shape == q.shape
    dbias = torch.zeros(225, 6, device=dev)
    dq, dk, dv = kernels.window_attention_backward(q, q, q, q, 6, (8, 8), 0.17, bias_table=table, dbias=dbias)
    assert dq.shape == dk.shape == dv.shape == q.shape
    assert bool((dbias == 0).all())


def test_mlp_no_tokens(dev):
    mlp = workloads.mlp_for(workloads.CONFIGS["c3"], 1).to(dev).to(torch.bfloat16)
    x = torch.zeros(0, 5, 192, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        assert mlp(x).shape == x.shape
