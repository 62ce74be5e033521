"""*_and_mul activations over [..., 2d] -> [..., d] (reference
src/plastic_infer/kernel/triton/activation.py:116-150):

    y = round(act(x[..., :d]) * x[..., d:])        halves widened to fp32, result in x's dtype

silu g/(1+e^-g), gelu 0.5g(1+erf(g/sqrt 2)), gelu_tanh 0.5g(1+tanh(sqrt(2/pi)(g+0.044715g^3))).
One HIP kernel (pia_act_and_mul), bf16, fp16 and fp32.
"""

from __future__ import annotations

import torch

from .. import _native as N
from .moe_ops import ACTIVATION_CODES


def _act_and_mul(kind: str, x: torch.Tensor, out: torch.Tensor | None) -> torch.Tensor:
    dev = N.require_device(x, names=("x",))
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    d = x.shape[-1] // 2
    if out is None:
        out = torch.empty(x.shape[:-1] + (d,), device=dev, dtype=x.dtype)
    elif out.shape != x.shape[:-1] + (d,) or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be contiguous [..., d] of x's dtype")
    rows = x.numel() // max(1, x.shape[-1])
    N.call("pia_act_and_mul", out.data_ptr(), x.data_ptr(), rows, d, ACTIVATION_CODES[kind],
           N.dtype_code(x.dtype), N.stream_of(dev))
    return out


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _act_and_mul("silu", x, out)


def gelu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _act_and_mul("gelu", x, out)


def gelu_tanh_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _act_and_mul("gelu_tanh", x, out)


__all__ = ["silu_and_mul", "gelu_and_mul", "gelu_tanh_and_mul"]
