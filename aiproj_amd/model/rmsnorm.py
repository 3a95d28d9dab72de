"""RMSNorm, reference `src/torch_llm/model/rmsnorm.py:14-113`.

`RMSNorm(d_model, eps=1e-5, weight=None)` keeps the reference module's constructor,
parameter and contract: `forward(x)` takes a contiguous packed `[T, d_model]`
tensor and returns `(x * inv_rms) * weight` computed in float32 and stored in x's
dtype, with `inv_rms = 1 / sqrt(mean(x^2) + eps)` per row.

The forward runs the gfx950 HIP kernel `rmsnorm_kernel` through the C ABI
`kvfp8_rmsnorm_forward`; `add_rmsnorm` is the residual add fused with the norm
that follows it (`kvfp8_add_rmsnorm_forward`). The backward (training, outside
this path) is written with PyTorch operations from the saved `inv_rms`.
"""

from __future__ import annotations

import torch as t
from torch import nn

from aiproj_amd import _native

_DTYPES = (t.float32, t.float16, t.bfloat16)


def _check(x: t.Tensor, weight: t.Tensor):
    if x.ndim != 2:
        raise ValueError("RMSNorm takes packed [T, d_model] input")
    if x.dtype not in _DTYPES or weight.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtypes {x.dtype}, {weight.dtype}")
    if weight.shape != (x.shape[1],):
        raise ValueError("weight must have shape (d_model,)")
    if x.stride(1) != 1:
        raise ValueError("rows of x must be contiguous")
    return _native.require_gpu(x, weight, what="rmsnorm")


def rmsnorm_forward(x: t.Tensor, weight: t.Tensor, eps: float):
    """(out [T, d_model] in x's dtype, inv_rms [T] float32)."""
    device = _check(x, weight)
    weight = weight.contiguous()
    out = t.empty_like(x, memory_format=t.contiguous_format)
    inv_rms = t.empty(x.shape[0], dtype=t.float32, device=x.device)
    rc = _native.lib().kvfp8_rmsnorm_forward(
        x.data_ptr(), _native.dtype_code(x.dtype), x.stride(0), x.shape[0], x.shape[1],
        weight.data_ptr(), _native.dtype_code(weight.dtype), float(eps),
        out.data_ptr(), out.stride(0), inv_rms.data_ptr(), _native.stream_handle(device))
    _native.check(rc, "kvfp8_rmsnorm_forward")
    return out, inv_rms


def add_rmsnorm(x: t.Tensor, update: t.Tensor, weight: t.Tensor, eps: float):
    """Residual add fused with the next norm: (state = x + update, rmsnorm(state))."""
    device = _check(x, weight)
    if update.shape != x.shape or update.dtype != x.dtype or update.stride(1) != 1:
        raise ValueError("update must match x in shape and dtype with contiguous rows")
    weight = weight.contiguous()
    state = t.empty_like(x, memory_format=t.contiguous_format)
    out = t.empty_like(x, memory_format=t.contiguous_format)
    rc = _native.lib().kvfp8_add_rmsnorm_forward(
        x.data_ptr(), update.data_ptr(), _native.dtype_code(x.dtype), x.stride(0), update.stride(0),
        x.shape[0], x.shape[1], weight.data_ptr(), _native.dtype_code(weight.dtype), float(eps),
        state.data_ptr(), state.stride(0), out.data_ptr(), out.stride(0), None, _native.stream_handle(device))
    _native.check(rc, "kvfp8_add_rmsnorm_forward")
    return state, out


class RMSNormFunction(t.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        output, inv_rms = rmsnorm_forward(x, weight, eps)
        ctx.save_for_backward(x, weight, inv_rms)
        return output

    @staticmethod
    @t.autograd.function.once_differentiable
    def backward(ctx, grad_output):
        x, weight, inv_rms = ctx.saved_tensors
        x32, g32, w32 = x.float(), grad_output.float(), weight.float()
        inv = inv_rms.unsqueeze(1)
        xhat = x32 * inv
        gw = g32 * w32
        dx = inv * (gw - xhat * (gw * xhat).mean(dim=1, keepdim=True))
        dw = (g32 * xhat).sum(dim=0)
        return dx.to(x.dtype), dw.to(weight.dtype), None


class RMSNorm(nn.Module):
    def __init__(self, d_model: int, eps: float = 1e-5, weight: t.Tensor | None = None):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.weight = nn.Parameter(t.ones(d_model) if weight is None else weight)

    def forward(self, x: t.Tensor) -> t.Tensor:
        assert x.is_contiguous()
        assert x.ndim == 2
        assert self.weight.shape == (self.d_model,)
        return RMSNormFunction.apply(x, self.weight, self.eps)
