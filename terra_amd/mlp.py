"""Drop-in ``SequentialMlp`` (models/mlp.py:138-172), the MLP half of a Swin
block: ``x + fc2(GELU(fc1(norm2(x))))`` per token.

For bf16 activations with C in {128, 192, 384, 768} and hidden = 4C, the forward is one
HIP kernel (``kernels.swin_mlp``): LayerNorm, fc1 on MFMA, exact GELU, fc2 on
MFMA and the residual add, with the hidden layer kept on chip.  The module
packs ``fc1.weight`` / ``fc2.weight`` with ``kernels.pack_linear`` and caches
the packed weights and fp32 copies of the small parameters until a
parameter's data pointer or in-place version changes.

Inference at other widths with C % 64 == 0 and 4C <= 4096 (C = 1024, the
width of TERRA's pretrain blocks): the LayerNorm on the HIP LayerNorm kernel
over the token rows, fc1 + exact GELU on the linear kernel's GELU epilogue,
fc2 + residual on hipBLASLt.

A call that needs a gradient runs autograd.mlp: the LayerNorm forward and
backward (residual gradient included) on the HIP LayerNorm kernels over the
token rows, the GEMMs on hipBLASLt.  Other shapes and dtypes run the
reference's own sequence of torch modules on the device (norm2, fc1, act,
fc2, residual).  Parameter names (``norm2``, ``fc1``, ``fc2``) and the seeded
initialisation follow the reference so its checkpoints load.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import autograd, config, kernels
from .attention import make_linear_with_seed


def _disable_parameters_if_mlp_off(module: torch.nn.Module) -> None:
    """models/mlp.py:18-21."""
    if not config.use_MLP:
        for param in module.parameters():
            param.requires_grad_(False)


class SequentialMlp(torch.nn.Module):
    def __init__(self, in_features, hidden_features=None, out_features=None, act_layer=torch.nn.GELU, drop=0.,
                 init_seed_base=None):
        super().__init__()
        out_features = out_features or in_features
        hidden_features = hidden_features or in_features
        if config.use_layernorm:
            self.norm2 = torch.nn.LayerNorm(in_features)
        seed = (lambda k: None if init_seed_base is None else init_seed_base + k)  # noqa: E731
        self.fc1 = make_linear_with_seed(in_features, hidden_features, init_seed=seed(1))
        self.act = act_layer()
        self.fc2 = make_linear_with_seed(hidden_features, out_features, init_seed=seed(2))
        _disable_parameters_if_mlp_off(self)
        self.use_fused_mlp = True

    def _fusable(self, x: torch.Tensor) -> bool:
        """One kernel serves the call: bf16 rows of C in {128, 192, 384, 768}, hidden
        4C, out C, the exact GELU, a plain LayerNorm over C (or none), biased
        linears of the activation dtype (or fp32 under bf16 autocast), and no
        gradient needed."""
        if not self.use_fused_mlp or x.dim() < 1:
            return False
        C = x.shape[-1]
        fc1, fc2 = self.fc1, self.fc2
        if not kernels.swin_mlp_supported(x, C, fc1.out_features) or fc1.in_features != C or fc2.out_features != C:
            return False
        if type(self.act) is not torch.nn.GELU or self.act.approximate != "none":
            return False
        if config.use_layernorm:
            n = self.norm2
            if type(n) is not torch.nn.LayerNorm or tuple(n.normalized_shape) != (C,) or n.weight is None:
                return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        # Weights of the activation dtype, or fp32 weights inside a bf16
        # autocast region (where F.linear would cast them to bf16).
        w_ok = all(l.weight.dtype == x.dtype for l in (fc1, fc2)) or (
            kernels.autocast_bf16(x) and all(l.weight.dtype == torch.float32 for l in (fc1, fc2)))
        return w_ok and all(l.bias is not None for l in (fc1, fc2))

    def _trainable(self, x: torch.Tensor) -> bool:
        """A call that needs gradients through a plain LayerNorm over C <= 1024
        (rows of whole 16-byte chunks), the exact GELU and biased linears:
        the LayerNorm and its backward run on the HIP kernels
        (autograd.mlp), the GEMMs on hipBLASLt."""
        if not (torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))):
            return False
        C = x.shape[-1]
        if not config.use_layernorm or type(self.norm2) is not torch.nn.LayerNorm:
            return False
        if tuple(self.norm2.normalized_shape) != (C,) or C > 1024 or (C * x.element_size()) % 16 != 0:
            return False
        if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            return False
        if type(self.act) is not torch.nn.GELU or self.act.approximate != "none":
            return False
        return all(l.bias is not None for l in (self.fc1, self.fc2)) and self.fc2.out_features == C

    def _gemm_path(self, x: torch.Tensor) -> bool:
        """Inference for widths the one-kernel MLP does not take (C = 1024,
        TERRA's pretrain width): bf16 rows, C a multiple of 64 with 4C <= 4096,
        hidden 4C, a plain LayerNorm, the exact GELU, biased bf16 linears (or
        fp32 ones under bf16 autocast), no gradient.  The LayerNorm runs on
        the HIP LayerNorm kernel over the token rows and fc1 + GELU on the
        linear kernel with the GELU epilogue; fc2 + residual on hipBLASLt,
        which is faster than the linear kernel for the 4C -> C product."""
        if not self.use_fused_mlp or x.dim() < 1 or x.dtype != torch.bfloat16 or x.device.type != "cuda":
            return False
        C = x.shape[-1]
        fc1, fc2 = self.fc1, self.fc2
        if fc1.in_features != C or fc1.out_features != 4 * C or fc2.out_features != C:
            return False
        if not kernels.linear_supported(x, C, 4 * C) or C > 1024:
            return False
        if not config.use_layernorm or type(self.norm2) is not torch.nn.LayerNorm or self.norm2.weight is None \
                or tuple(self.norm2.normalized_shape) != (C,):
            return False
        if type(self.act) is not torch.nn.GELU or self.act.approximate != "none":
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        w_ok = all(l.weight.dtype == x.dtype for l in (fc1, fc2)) or (
            kernels.autocast_bf16(x) and all(l.weight.dtype == torch.float32 for l in (fc1, fc2)))
        return w_ok and all(l.bias is not None for l in (fc1, fc2))

    def _gemm_forward(self, x: torch.Tensor) -> torch.Tensor:
        a = self._fused_args()
        C = x.shape[-1]
        rows = x.contiguous().view(-1, C)
        n = rows.shape[0]
        xn = kernels.swin_partition_ln(rows.view(1, n, 1, C), kernels.rows_geometry(n, C), a["ln_weight"],
                                       a["ln_bias"], a["ln_eps"]).view(n, C)
        h = kernels.linear(xn, a["fc1_weight"], 4 * C, a["fc1_bias"], gelu=True)
        w2, b2 = self._fc2_bf16()
        return (F.linear(h, w2, b2) + rows).view(x.shape)

    def _fc2_bf16(self):
        """fc2's weight and bias as bf16 (autocast's cast of fp32 ones), cached."""
        w, b = self.fc2.weight, self.fc2.bias
        if w.dtype == torch.bfloat16 and b.dtype == torch.bfloat16:
            return w, b
        key = (w.data_ptr(), w._version, b.data_ptr(), b._version)
        hit = getattr(self, "_fc2_cache", None)
        if hit is None or hit[0] != key:
            with torch.no_grad():
                hit = (key, (w.detach().to(torch.bfloat16), b.detach().to(torch.bfloat16)))
            self._fc2_cache = hit
        return hit[1]

    def _fused_args(self) -> dict:
        tensors = [self.fc1.weight, self.fc1.bias, self.fc2.weight, self.fc2.bias]
        if config.use_layernorm:
            tensors += [self.norm2.weight, self.norm2.bias]
        key = tuple((t.data_ptr(), t._version, t.device, t.dtype) if t is not None else None for t in tensors)
        cached = getattr(self, "_fused_cache", None)
        if cached is not None and cached[0] == key:
            return cached[1]
        with torch.no_grad():
            f32 = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()  # noqa: E731
            args = dict(
                fc1_weight=kernels.pack_linear(self.fc1.weight.detach().to(torch.bfloat16).contiguous()),
                fc1_bias=f32(self.fc1.bias),
                fc2_weight=kernels.pack_linear(self.fc2.weight.detach().to(torch.bfloat16).contiguous()),
                fc2_bias=f32(self.fc2.bias),
                ln_weight=f32(self.norm2.weight) if config.use_layernorm else None,
                ln_bias=f32(self.norm2.bias) if config.use_layernorm else None,
                ln_eps=float(self.norm2.eps) if config.use_layernorm else 0.0,
                layernorm=bool(config.use_layernorm),
            )
        self._fused_cache = (key, args)
        return args

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not config.use_MLP:
            return x
        if x.device.type != "cuda":
            raise RuntimeError("terra_amd: SequentialMlp runs on device tensors only (got a CPU tensor)")
        if self._fusable(x):
            return kernels.swin_mlp(x.contiguous(), out=out, **self._fused_args())
        if self._gemm_path(x):
            return self._gemm_forward(x)
        if self._trainable(x):
            n = self.norm2
            return autograd.mlp(x, n.weight, n.bias, self.fc1.weight, self.fc1.bias, self.fc2.weight,
                                self.fc2.bias, n.eps)
        shortcut = x
        if config.use_layernorm:
            x = self.norm2(x)
        x = self.fc2(self.act(self.fc1(x)))
        return x + shortcut
