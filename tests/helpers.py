"""Shared helpers of the GPU parity tests (weights that make the attention
term visible, and the checks applied to it)."""
from __future__ import annotations

import math

import torch

from terra_amd import workloads


def params_of(block) -> dict:
    """State dict as fp32 CPU tensors (the oracle's parameter form)."""
    return {k: v.detach().float().cpu() for k, v in block.state_dict().items() if k != "attn_mask"}


def gain_block(blk, seed: int = 409, gain_qkv: float = None, gain_proj: float = None, bias_gain: float = 50.0):
    """Scale the trunc-normal(0.02) weights of an attention block so that the
    attention term y - x is O(1) and every part of it shows in the output:
    q/k/v by 60/sqrt(C) (logits of standard deviation ~1.5), proj by 4x that,
    the relative-position bias table by ``bias_gain`` (std ~1), Linear biases
    0.1 N(0,1), LayerNorm affine 1 + 0.1 N(0,1) / 0.1 N(0,1).  In place on the
    CPU module (before it is moved and cast); returns it."""
    C = blk.norm1.weight.shape[0]
    gq = gain_qkv if gain_qkv is not None else 60.0 / math.sqrt(C)
    gp = gain_proj if gain_proj is not None else 4.0 * gq
    attn = blk.attn
    with torch.no_grad():
        for i, lin in enumerate((attn.q_linear, attn.k_linear, attn.v_linear, attn.proj)):
            lin.weight.mul_(gp if lin is attn.proj else gq)
            lin.bias.copy_(workloads.activations(lin.bias.shape, seed + i, torch.float32) * 0.1)
        if getattr(attn, "relative_position_bias_table", None) is not None:
            attn.relative_position_bias_table.mul_(bias_gain)
        blk.norm1.weight.copy_(1.0 + 0.1 * workloads.activations((C,), seed + 5, torch.float32))
        blk.norm1.bias.copy_(0.1 * workloads.activations((C,), seed + 6, torch.float32))
    return blk


def rel_maxabs(out, ref) -> float:
    out, ref = out.double().cpu(), ref.double().cpu()
    return ((out - ref).abs().max() / ref.abs().max()).item()


def rel_norm(out, ref) -> float:
    out, ref = out.double().cpu(), ref.double().cpu()
    return (torch.linalg.vector_norm(out - ref) / torch.linalg.vector_norm(ref)).item()


def assert_block_matches(y, ref, x, tol_y: float, tol_delta: float, min_delta: float = 0.5):
    """y against the oracle: max-abs relative on y, and normwise relative on
    the attention term y - x (the residual x would otherwise hide it)."""
    x = x.double().cpu().view(ref.shape)
    y = y.double().cpu().view(ref.shape)
    d_ref = ref.double() - x
    assert d_ref.abs().max().item() >= min_delta, "attention term too small to test"
    e_y = rel_maxabs(y, ref)
    e_d = rel_norm(y - x, d_ref)
    assert e_y <= tol_y and e_d <= tol_delta, (e_y, e_d)
    return e_y, e_d
