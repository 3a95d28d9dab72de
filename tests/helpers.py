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


def torch_prefill_attention(q: t.Tensor, k: t.Tensor, v: t.Tensor, seq_lens: list[int],
                            chunk_bytes: int = 1 << 30) -> t.Tensor:
    """Causal GQA attention of packed prompts q [T, Hq, D], k/v [T, Hkv, D] -> [T, Hq, D],
    a float32 torch reference for the prefill kernel.

    Float32 math with contiguous operands, sequences of equal length batched
    together in chunks whose score tensor stays under `chunk_bytes`."""
    total, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = t.empty_like(q)
    start = 0
    i = 0
    while i < len(seq_lens):
        length = seq_lens[i]
        per_seq = hq * length * length * 4
        n = 1
        while (i + n < len(seq_lens) and seq_lens[i + n] == length and (n + 1) * per_seq <= chunk_bytes):
            n += 1
        end = start + n * length
        qs = q[start:end].float().view(n, length, hkv, g, d).permute(0, 2, 3, 1, 4).contiguous()
        ks = k[start:end].float().view(n, length, hkv, d).permute(0, 2, 3, 1).unsqueeze(2).contiguous()
        vs = v[start:end].float().view(n, length, hkv, d).permute(0, 2, 1, 3).unsqueeze(2).contiguous()
        scores = t.matmul(qs, ks) * (1.0 / math.sqrt(d))                      # [n, hkv, g, L, L]
        causal = t.ones(length, length, dtype=t.bool, device=q.device).triu(1)
        scores.masked_fill_(causal, float("-inf"))
        probs = scores.softmax(dim=-1)
        o = t.matmul(probs, vs)                                                # [n, hkv, g, L, d]
        out[start:end] = o.permute(0, 3, 1, 2, 4).reshape(n * length, hq, d).to(q.dtype)
        start = end
        i += n
    return out


def torch_paged_decode(q: t.Tensor, cache, slots: t.Tensor, lengths: t.Tensor, block_table: t.Tensor) -> t.Tensor:
    """Dequantize-then-attend in float32 on the device (the reference's CPU test oracle,
    `tests/test_kv_cache_quantization.py:428-446`, batched): every sequence's K/V rows
    gathered through its block-table row, `codes * scale` for an FP8 cache, GQA
    softmax(q k^T / sqrt(D)) v over its first `lengths[b]` positions. -> [B, Hq, D] float32."""
    b, hq, d = q.shape
    hkv = cache.k.shape[2]
    bs = cache.block_size
    lengths = lengths.long()
    width = int(lengths.max())
    pos = t.arange(width, device=q.device)
    rows = block_table[slots.long()][:, pos // bs].long().clamp_min(0)            # [B, W]
    offs = (pos % bs).expand(b, width)

    def gather(values, scales):
        x = values[rows, offs].float()                                            # [B, W, Hkv, D]
        if scales is not None:
            x = x * scales[rows, offs].unsqueeze(-1)
        return x

    live = (pos[None, :] < lengths[:, None])[:, None, None, :]                   # [B, 1, 1, W]
    k = gather(cache.k, cache.k_scales).permute(0, 2, 3, 1).contiguous()          # [B, Hkv, D, W]
    # Positions past a sequence's length read whatever its pages (or page 0) hold,
    # NaN codes included: zero them, as probability 0 times NaN would be NaN.
    v = gather(cache.v, cache.v_scales).permute(0, 2, 1, 3)                       # [B, Hkv, W, D]
    v = v.masked_fill(~live.transpose(-1, -2), 0.0).contiguous()
    qg = q.float().view(b, hkv, hq // hkv, d)
    scores = t.matmul(qg, k) / math.sqrt(d)                                       # [B, Hkv, G, W]
    scores = scores.masked_fill(~live, float("-inf"))
    probs = t.nan_to_num(scores.softmax(dim=-1), nan=0.0)
    return t.matmul(probs, v).reshape(b, hq, d)
