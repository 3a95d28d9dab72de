"""numpy restatement of the reference's FP8 KV-cache oracle (test infrastructure only).

Every function names the reference file:line it follows. Inputs are numpy arrays;
float inputs are float32 (the reference converts every input with `x.float()` first,
`tests/test_kv_cache_quantization.py:62`, and bf16/f16 -> f32 is exact), codes are
uint8 bit patterns of OCP float8_e4m3fn.
"""

from __future__ import annotations

import math

import numpy as np

# Largest finite float8_e4m3fn value: torch.finfo(float8_e4m3fn).max used at
# reference `tests/test_kv_cache_quantization.py:48` and `quantized_append.py:50-51`.
FP8_MAX = np.float32(448.0)


# ---------------------------------------------------------------------------
# float8_e4m3fn encoding (OCP: 1 sign, 4 exponent bits with bias 7, 3 mantissa
# bits, no infinities, S.1111.111 is NaN, max finite 1.75 * 2**8 = 448).
# ---------------------------------------------------------------------------

def _decode_table() -> np.ndarray:
    """The 256 code values, derived from the format definition."""
    table = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 0x7
        if exponent == 0xF and mantissa == 0x7:
            table[code] = math.nan
        elif exponent == 0:
            table[code] = sign * mantissa * 2.0 ** -9          # subnormal step 2**-9
        else:
            table[code] = sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
    return table.astype(np.float32)


E4M3_TABLE = _decode_table()


def e4m3fn_to_f32(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (exact)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32 -> float8_e4m3fn codes, round-to-nearest-even, non-saturating.

    This is the cast `.to(torch.float8_e4m3fn)` the reference oracle applies at
    `tests/test_kv_cache_quantization.py:65`: NaN keeps its sign bit (0x7F/0xFF),
    magnitudes that round above 448 become NaN (e4m3fn has no infinity), signed
    zero is kept, and the subnormal range has step 2**-9.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag_bits = bits & np.uint32(0x7FFFFFFF)
    mag = mag_bits.view(np.float32)

    out = np.zeros(x.shape, dtype=np.uint8)

    # Normal e4m3 range: |x| >= 2**-6. Keep the top 3 of the 23 fp32 mantissa
    # bits and round the 20 dropped bits half-to-even; a carry out of the
    # mantissa moves into the exponent field, which is the correct next code.
    normal = mag_bits >= np.uint32(0x3C800000)                 # 2**-6
    exponent = (mag_bits >> 23).astype(np.int64) - 127 + 7
    kept = ((mag_bits >> 20) & 0x7).astype(np.int64)
    dropped = (mag_bits & 0xFFFFF).astype(np.int64)
    round_up = (dropped > 0x80000) | ((dropped == 0x80000) & ((kept & 1) == 1))
    normal_code = (exponent << 3) + kept + round_up.astype(np.int64)

    # Subnormal range: |x| < 2**-6 is an integer count of 2**-9 steps; scaling by
    # 2**9 is exact in fp32 and rint rounds half to even. A count of 8 is the
    # smallest normal code 0x08, so the two ranges join without a special case.
    sub_src = np.where(normal, np.float32(0.0), mag)
    sub_code = np.rint(sub_src * np.float32(512.0)).astype(np.int64)

    code = np.where(normal, normal_code, sub_code)
    # Anything that rounds past 448 (code 0x7E) or is NaN encodes as S.1111.111.
    overflow = (code > 0x7E) | (mag_bits > np.uint32(0x7F800000)) | (mag_bits == np.uint32(0x7F800000))
    code = np.where(overflow, 0x7F, code)
    out[...] = code.astype(np.uint8) | sign
    return out


# ---------------------------------------------------------------------------
# Quantization contract, reference `tests/test_kv_cache_quantization.py:20-32`
# and `reference_quantize` at `:60-66`.
# ---------------------------------------------------------------------------

def _nan_propagating_absmax(x32: np.ndarray) -> np.ndarray:
    """max |x| over the last axis; NaN if any element is NaN (torch.amax semantics)."""
    amax = np.abs(x32).max(axis=-1)  # numpy max propagates NaN, like torch.amax
    return amax.astype(np.float32)


def quantize(x: np.ndarray):
    """x [..., D] float32 -> (codes [..., D] uint8, scales [...] float32).

    amax  = max |x|                  (float32)
    scale = amax / 448 if amax > 0 else 1.0     (IEEE float32 division)
    code  = e4m3fn(clamp(x / scale, -448, 448)) (IEEE float32 division, then RNE)
    """
    x32 = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = _nan_propagating_absmax(x32)
        positive = amax > np.float32(0.0)                     # False for NaN, like torch
        scales = np.where(positive, amax / FP8_MAX, np.float32(1.0)).astype(np.float32)
        ratio = (x32 / scales[..., None]).astype(np.float32)
        # torch.clamp keeps NaN; np.clip does too.
        clamped = np.clip(ratio, -FP8_MAX, FP8_MAX).astype(np.float32)
    return f32_to_e4m3fn(clamped), scales


def dequantize(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """codes.float() * scales, reference `tests/test_kv_cache_quantization.py:69-70` (float32)."""
    return (e4m3fn_to_f32(codes) * np.asarray(scales, dtype=np.float32)[..., None]).astype(np.float32)


# ---------------------------------------------------------------------------
# Storage: layout `[num_blocks, block_size, H_kv, D]` and scales
# `[num_blocks, block_size, H_kv]` (reference `inference/paged_kv_cache.py:27-38`).
# ---------------------------------------------------------------------------

def scatter_append(k_cache, v_cache, k_scales, v_scales, ks, vs, blocks, offsets):
    """Quantize ks/vs [T, H_kv, D] and store them at (blocks[t], offsets[t]) in place.

    Address math of reference `kernals/kv_cache/quantized_append.py:103-105`:
    code  index ((block * BS + offset) * H_kv + head) * D + d
    scale index  (block * BS + offset) * H_kv + head
    which is `cache[block, offset, head, d]` for the 4-D layout.
    """
    kc, kscale = quantize(ks)
    vc, vscale = quantize(vs)
    blocks = np.asarray(blocks, dtype=np.int64)
    offsets = np.asarray(offsets, dtype=np.int64)
    k_cache[blocks, offsets] = kc
    v_cache[blocks, offsets] = vc
    k_scales[blocks, offsets] = kscale
    v_scales[blocks, offsets] = vscale


def physical_location(block_table, slots, positions, block_size):
    """Page-table gather for writes: (block_table[slot, pos // BS], pos % BS).

    Reference `inference/page_allocator.py:240-245`.
    """
    slots = np.asarray(slots, dtype=np.int64)
    positions = np.asarray(positions, dtype=np.int64)
    return block_table[slots, positions // block_size].astype(np.int64), positions % block_size


def paged_history(k_cache, v_cache, k_scales, v_scales, block_table, slot, length, block_size):
    """Dequantized K, V history [L, H_kv, D] float64 for one sequence.

    Reference `cache_history`, `tests/test_kv_cache_quantization.py:428-437`: the codes
    are gathered through block_table[slot, pos // BS] at offset pos % BS, widened to
    float64 and multiplied by the float64 scales. With `k_scales is None` the cache is
    unquantized and its values are used as stored.
    """
    positions = np.arange(length, dtype=np.int64)
    blocks = block_table[slot, positions // block_size].astype(np.int64)
    offsets = positions % block_size
    if k_scales is None:
        return k_cache[blocks, offsets].astype(np.float64), v_cache[blocks, offsets].astype(np.float64)
    k = e4m3fn_to_f32(k_cache[blocks, offsets]).astype(np.float64)
    v = e4m3fn_to_f32(v_cache[blocks, offsets]).astype(np.float64)
    k = k * k_scales[blocks, offsets].astype(np.float64)[..., None]
    v = v * v_scales[blocks, offsets].astype(np.float64)[..., None]
    return k, v


def decode_one(q, k, v):
    """One decode step in float64: q [H_q, D]; k, v [L, H_kv, D] -> [H_q, D].

    Reference `reference_decode`, `tests/test_kv_cache_quantization.py:440-446`:
    query head h attends KV head h // (H_q / H_kv) (`kernals/decode_attention.py:248-249`),
    scores are scaled by 1/sqrt(D) (`kernals/decode_attention.py:74`). A sequence with
    no context returns zeros (`kernals/decode_attention.py:536-540`).
    """
    q = np.asarray(q, dtype=np.float64)
    num_q_heads, head_dim = q.shape
    length, num_kv_heads, _ = k.shape
    if length == 0:
        return np.zeros((num_q_heads, head_dim), dtype=np.float64)
    group = num_q_heads // num_kv_heads
    # Query heads grouped by their KV head: [H_kv, G, D]; the reference's
    # repeat_interleave(group) over KV heads is the same pairing.
    qg = q.reshape(num_kv_heads, group, head_dim)
    kh = np.ascontiguousarray(np.transpose(k, (1, 2, 0)), dtype=np.float64)   # [H_kv, D, L]
    vh = np.ascontiguousarray(np.transpose(v, (1, 0, 2)), dtype=np.float64)   # [H_kv, L, D]
    scores = np.matmul(qg, kh) / math.sqrt(head_dim)                           # [H_kv, G, L]
    scores = scores - scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights = weights / weights.sum(axis=-1, keepdims=True)
    return np.matmul(weights, vh).reshape(num_q_heads, head_dim)


def paged_decode(q, k_cache, v_cache, k_scales, v_scales, block_table, slots, context_lengths, block_size):
    """Attention of every row of q [B, H_q, D] over its paged history -> float64 [B, H_q, D].

    The per-row stack of reference `tests/test_kv_cache_quantization.py:475-478`.
    """
    q = np.asarray(q, dtype=np.float64)
    rows = []
    for row in range(q.shape[0]):
        k, v = paged_history(k_cache, v_cache, k_scales, v_scales, block_table,
                             int(slots[row]), int(context_lengths[row]), block_size)
        rows.append(decode_one(q[row], k, v))
    return np.stack(rows) if rows else np.zeros(q.shape, dtype=np.float64)


def causal_varlen_attention(q, k, v, cu_seqlens, max_seq_len, scale):
    """Packed causal attention in float64 -> (out [T, H_q, D], lse [T, H_q]).

    Reference `tests/test_flash_attention.py:44-85` (the ragged PyTorch reference: per
    sequence, `softmax(scale q k^T)` under a lower-triangular mask, KV heads repeated
    per query group) and the kernel's outputs at `kernals/flash_attention.py:205-210`:
    `lse = max + log(sum exp(s - max))` of the scaled scores. Only the first
    `max_seq_len` rows of each sequence are produced (the reference grid covers
    `cdiv(batch_max_seq_len, BLOCK_M)` query blocks); every other row is NaN.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    total, num_q_heads, head_dim = q.shape
    group = num_q_heads // k.shape[1]
    out = np.full(q.shape, np.nan)
    lse = np.full((total, num_q_heads), np.nan)
    bounds = [int(x) for x in cu_seqlens]
    for b in range(len(bounds) - 1):
        s0, s1 = bounds[b], bounds[b + 1]
        n = min(s1 - s0, int(max_seq_len))
        if n <= 0:
            continue
        length = s1 - s0
        qs = np.transpose(q[s0:s0 + n], (1, 0, 2))                                     # [H_q, n, D]
        ks = np.repeat(np.transpose(k[s0:s1], (1, 0, 2)), group, axis=0)               # [H_q, L, D]
        vs = np.repeat(np.transpose(v[s0:s1], (1, 0, 2)), group, axis=0)
        scores = scale * np.matmul(qs, np.transpose(ks, (0, 2, 1)))                    # [H_q, n, L]
        mask = np.arange(length)[None, :] <= np.arange(n)[:, None]
        scores = np.where(mask[None], scores, -np.inf)
        mx = scores.max(axis=-1, keepdims=True)
        weights = np.exp(scores - mx)
        total_w = weights.sum(axis=-1, keepdims=True)
        out[s0:s0 + n] = np.transpose(np.matmul(weights / total_w, vs), (1, 0, 2))
        lse[s0:s0 + n] = np.transpose((mx + np.log(total_w))[..., 0], (1, 0))
    return out, lse


# ---------------------------------------------------------------------------
# Algorithmic byte counts (the roofline numerators).
# ---------------------------------------------------------------------------

def decode_algorithmic_bytes(context_lengths, num_q_heads, num_kv_heads, head_dim, block_size,
                             q_bytes=2, out_bytes=2, kv_bytes=1, scale_bytes=4):
    """Bytes one decode call must move: K/V codes and scales of every attended token,
    Q in, O out, and one block-table entry per attended page."""
    lengths = np.asarray(context_lengths, dtype=np.int64)
    tokens = int(lengths.sum())
    pages = int(((lengths + block_size - 1) // block_size).sum())
    batch = lengths.shape[0]
    kv = tokens * num_kv_heads * 2 * (head_dim * kv_bytes + (scale_bytes if kv_bytes == 1 else 0))
    return kv + batch * num_q_heads * head_dim * (q_bytes + out_bytes) + pages * 4


def append_algorithmic_bytes(num_tokens, num_kv_heads, head_dim, in_bytes=2):
    """Bytes one quantize-and-scatter call must move: K and V in, codes and scales out."""
    return num_tokens * num_kv_heads * (2 * head_dim * in_bytes + 2 * head_dim + 8)
