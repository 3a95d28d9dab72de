"""Helpers shared by the test modules (not collected as tests)."""

from __future__ import annotations

import math

import numpy as np
import torch as t

FP8 = t.float8_e4m3fn
FP8_MAX = t.finfo(FP8).max


def torch_reference_quantize(x):
    """The reference's test oracle, written with the torch library routines it calls
    (`tests/test_kv_cache_quantization.py:60-66`: amax, float32 division, clamp,
    `.to(float8_e4m3fn)`). Returns (uint8 codes, float32 scales) as numpy arrays."""
    x32 = x.float()
    amax = x32.abs().amax(dim=-1)
    scales = t.where(amax > 0, amax / FP8_MAX, t.ones_like(amax))
    codes = (x32 / scales.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return codes.view(t.uint8).cpu().numpy(), scales.cpu().numpy()


def error_bound(x, scales):
    """|x - x_hat| <= 2^-4 |x| + scale 2^-9 (reference `tests/test_kv_cache_quantization.py:28-32`)."""
    return 2 ** -4 * np.abs(x) + scales[..., None] * 2 ** -9


def scattered_locations(num_tokens, num_blocks, block_size, device, seed=0):
    """Distinct (block, offset) pairs spread over the pool in random order
    (reference `tests/test_kv_cache_quantization.py:77-81`)."""
    generator = t.Generator().manual_seed(seed)
    flat = t.randperm(num_blocks * block_size, generator=generator)[:num_tokens]
    return (flat // block_size).to(device), (flat % block_size).to(device)


def brute_force_decode(q, k, v):
    """Pure-Python float64 attention for tiny inputs: q [Hq][D]; k, v [L][Hkv][D]."""
    hq, d = len(q), len(q[0])
    length = len(k)
    out = [[0.0] * d for _ in range(hq)]
    if length == 0:
        return out
    hkv = len(k[0])
    group = hq // hkv
    for h in range(hq):
        kv = h // group
        scores = [sum(q[h][i] * k[t_][kv][i] for i in range(d)) / math.sqrt(d) for t_ in range(length)]
        top = max(scores)
        weights = [math.exp(s - top) for s in scores]
        total = sum(weights)
        for i in range(d):
            out[h][i] = sum(weights[t_] * v[t_][kv][i] for t_ in range(length)) / total
    return out
