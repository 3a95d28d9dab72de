"""Varlen causal attention over packed prompts, reference `src/torch_llm/kernals/flash_attention.py`.

Same interface as the reference:

* `flash_attention_forward(q, k, v, cum_seq, batch_max_seq_len, scale) -> (output, lse)`
  (reference `:51-100`): q [T, Hq, D], k and v [T, Hkv, D], contiguous, one dtype;
  `cum_seq` [B + 1] int32/int64 on the device; `batch_max_seq_len` a host int. Row i of
  sequence b (tokens `cum_seq[b]:cum_seq[b + 1]`) attends keys 0..i of that sequence; q
  head h reads KV head h // (Hq / Hkv). `output` is a new tensor like q (rows outside
  every sequence are left unwritten, as `t.empty_like` leaves them in the reference);
  `lse` [T, Hq] float32 is `max + log(sum exp(s - max))` of the scaled scores. The work is
  one launch of the HIP kernel `prefill_attention_kernel` through the C ABI
  `kvfp8_prefill_attention`; nothing is synchronized with the host.
* `FlashAttentionFunction.apply(q, k, v, cum_seq, batch_max_seq_len)` (reference
  `:10-48`) with `scale = 1/sqrt(D)`.

The backward (`flash_attention_backward`, reference `:213-...`) is training-side and not
part of the prefill path: it is written with PyTorch float32 operations on the device
from the saved `lse`, sequence by sequence (it reads the sequence bounds on the host).

Head sizes 1 to 512 (`ValueError` otherwise), like the reference, which pads any size
to a power of two (`:72`): multiples of 8 up to 128 run on the matrix-core kernels, every
other size on a vector-ALU kernel.
"""

from __future__ import annotations

import math

import torch as t

from aiproj_amd import _native

_DTYPES = (t.float32, t.float16, t.bfloat16)


def flash_attention_forward(q: t.Tensor, k: t.Tensor, v: t.Tensor, cum_seq: t.Tensor,
                            batch_max_seq_len: int, scale: float) -> tuple[t.Tensor, t.Tensor]:
    assert k.shape == v.shape
    assert q.shape[0] == k.shape[0]
    assert q.shape[2] == k.shape[2]
    total, hq, d = q.shape
    hkv = k.shape[1]
    batch = cum_seq.shape[0] - 1
    assert hq % hkv == 0
    assert q.is_contiguous() and k.is_contiguous() and v.is_contiguous()
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"flash_attention_forward: q, k, v must share one of {_DTYPES}")
    if cum_seq.dtype not in (t.int32, t.int64) or cum_seq.ndim != 1:
        raise ValueError("flash_attention_forward: cum_seq must be a vector of int32/int64 offsets")
    device = _native.require_gpu(q, k, v, cum_seq, what="flash_attention_forward")
    output = t.empty_like(q)
    lse = t.empty((total, hq), device=q.device, dtype=t.float32)
    if total == 0 or batch <= 0 or int(batch_max_seq_len) <= 0:
        return output, lse
    rc = _native.lib().kvfp8_prefill_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _native.dtype_code(q.dtype), total, hq, hkv, d,
        cum_seq.data_ptr(), _native.dtype_code(cum_seq.dtype), batch, int(batch_max_seq_len), float(scale),
        output.data_ptr(), lse.data_ptr(), _native.stream_handle(device))
    _native.check(rc, "kvfp8_prefill_attention")
    return output, lse


def flash_attention_backward(q, k, v, output, lse, cum_seq, grad_output, batch_max_seq_len, scale):
    """dq, dk, dv of the causal varlen attention (float32 math, per sequence)."""
    total, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    dq = t.zeros(q.shape, device=q.device, dtype=t.float32)
    dk = t.zeros(k.shape, device=q.device, dtype=t.float32)
    dv = t.zeros(v.shape, device=q.device, dtype=t.float32)
    bounds = cum_seq.tolist()
    for b in range(len(bounds) - 1):
        s0, s1 = int(bounds[b]), int(bounds[b + 1])
        n = min(s1 - s0, int(batch_max_seq_len))
        if n <= 0:
            continue
        rows = slice(s0, s0 + n)
        qs = q[rows].float().permute(1, 0, 2).contiguous()                                 # [Hq, n, D]
        ks = k[rows].float().permute(1, 0, 2).repeat_interleave(g, dim=0).contiguous()      # [Hq, n, D]
        vs = v[rows].float().permute(1, 0, 2).repeat_interleave(g, dim=0).contiguous()
        os_ = output[rows].float().permute(1, 0, 2).contiguous()
        dos = grad_output[rows].float().permute(1, 0, 2).contiguous()
        ls = lse[rows].float().permute(1, 0).unsqueeze(-1)                                  # [Hq, n, 1]
        scores = t.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
        causal = t.ones(n, n, dtype=t.bool, device=q.device).tril()
        p = t.where(causal, t.exp(scores - ls), t.zeros((), device=q.device))
        dvs = t.matmul(p.transpose(1, 2).contiguous(), dos)
        dp = t.matmul(dos, vs.transpose(1, 2).contiguous())
        delta = (dos * os_).sum(-1, keepdim=True)
        ds = p * (dp - delta) * scale
        dqs = t.matmul(ds, ks)
        dks = t.matmul(ds.transpose(1, 2).contiguous(), qs)
        dq[rows] = dqs.permute(1, 0, 2)
        dk[rows] = dks.view(hkv, g, n, d).sum(1).permute(1, 0, 2)
        dv[rows] = dvs.view(hkv, g, n, d).sum(1).permute(1, 0, 2)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


class FlashAttentionFunction(t.autograd.Function):
    """Packed varlen causal attention (reference `:10-48`); scale = 1/sqrt(D)."""

    @staticmethod
    def forward(ctx, q, k, v, cum_seq, batch_max_seq_len):
        d = q.shape[-1]
        scale = 1.0 / math.sqrt(d)
        output, lse = flash_attention_forward(q, k, v, cum_seq, batch_max_seq_len, scale)
        ctx.save_for_backward(q, k, v, output, lse, cum_seq)
        ctx.batch_max_seq_len = batch_max_seq_len
        ctx.scale = scale
        return output

    @staticmethod
    @t.autograd.function.once_differentiable
    def backward(ctx, grad_output):
        q, k, v, output, lse, cum_seq = ctx.saved_tensors
        dq, dk, dv = flash_attention_backward(q, k, v, output, lse, cum_seq, grad_output.contiguous(),
                                              ctx.batch_max_seq_len, ctx.scale)
        return dq, dk, dv, None, None
