"""Pins the numpy oracle (CPU).

The oracle restates the reference's test oracle; these tests check it against
  * torch's own cast and the torch-op quantizer the reference oracle is written in
    (`tests/test_kv_cache_quantization.py:60-66`) - sweeps over fp32/bf16/fp16;
  * the committed golden fixtures (written from torch, tests/golden/make_golden.py);
  * the reference's known-answer and bound tests (`:95-142`);
  * brute-force float64 attention and invariants that a dropped term, a wrong
    sign/index or a transposed operand would break.
"""

from __future__ import annotations

import hashlib
import math
from pathlib import Path

import numpy as np
import pytest
import torch as t

import oracle
from tests.helpers import FP8, brute_force_decode, error_bound, torch_reference_quantize

GOLDEN = Path(__file__).resolve().parent / "golden"


def torch_cast(x: np.ndarray) -> np.ndarray:
    return t.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(FP8).view(t.uint8).numpy()


# ---------------------------------------------------------------------------
# e4m3fn encoding
# ---------------------------------------------------------------------------

def test_decode_table_matches_torch():
    ref = t.arange(256, dtype=t.uint8).view(FP8).float().numpy()
    assert np.array_equal(np.isnan(ref), np.isnan(oracle.E4M3_TABLE))
    finite = ~np.isnan(ref)
    assert np.array_equal(ref[finite], oracle.E4M3_TABLE[finite])
    # Spot values of the format: max finite, min subnormal, signed zero.
    assert oracle.E4M3_TABLE[0x7E] == 448.0 and oracle.E4M3_TABLE[0x01] == 2.0 ** -9
    assert np.signbit(oracle.E4M3_TABLE[0x80])


def test_cast_matches_torch_on_strided_fp32_sweep():
    # Every 61st fp32 bit pattern: all exponents, NaN/inf, both signs.
    for start in range(0, 2 ** 32, 2 ** 27):
        bits = np.arange(start, start + 2 ** 27, 61, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        assert np.array_equal(oracle.f32_to_e4m3fn(x), torch_cast(x)), hex(start)


def test_cast_matches_torch_on_every_bf16_and_f16_value():
    bf16 = (np.arange(2 ** 16, dtype=np.uint32) << 16).view(np.float32)
    assert np.array_equal(oracle.f32_to_e4m3fn(bf16), torch_cast(bf16))
    f16 = np.arange(2 ** 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(oracle.f32_to_e4m3fn(f16), torch_cast(f16))


def test_cast_matches_torch_at_every_rounding_boundary():
    # Midpoints between consecutive e4m3 values and their fp32 neighbours: exactly
    # where a wrong tie rule or an off-by-one in the kept mantissa shows up.
    values = np.unique(np.abs(oracle.E4M3_TABLE[~np.isnan(oracle.E4M3_TABLE)]))
    mids = ((values[1:] + values[:-1]) / 2).astype(np.float32)
    probes = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                             values, np.float32([464.0, 470.0, 480.0, 2 ** -10, 3 * 2 ** -11])])
    probes = np.concatenate([probes, -probes]).astype(np.float32)
    assert np.array_equal(oracle.f32_to_e4m3fn(probes), torch_cast(probes))


def test_cast_known_answers():
    # Known answers of the cast (torch probe): -0 -> 0x80, 2^-10 -> 0x00 (tie to even),
    # 1.0625 -> 0x38, 1.1875 -> 0x3A, 464 -> 0x7E, 470 -> 0x7F, NaN keeps its sign.
    x = np.float32([-0.0, 2 ** -10, 1.0625, 1.1875, 464.0, 470.0, np.nan, -np.nan])
    assert oracle.f32_to_e4m3fn(x).tolist() == [0x80, 0x00, 0x38, 0x3A, 0x7E, 0x7F, 0x7F, 0xFF]


# ---------------------------------------------------------------------------
# Quantization contract
# ---------------------------------------------------------------------------

def test_golden_manifest_is_intact():
    for line in (GOLDEN / "MANIFEST.sha256").read_text().splitlines():
        digest, name = line.split()
        assert hashlib.sha256((GOLDEN / name).read_bytes()).hexdigest() == digest, name


def test_quantize_matches_golden_fixtures():
    cases = np.load(GOLDEN / "quantize_cases.npz")
    names = sorted({key.split("__")[0] for key in cases.files})
    assert len(names) >= 15
    for name in names:
        codes, scales = oracle.quantize(cases[f"{name}__x"])
        assert np.array_equal(codes, cases[f"{name}__codes"]), name
        assert np.array_equal(scales.view(np.uint32), cases[f"{name}__scales"].view(np.uint32)), name


@pytest.mark.parametrize("dtype", [t.float32, t.float16, t.bfloat16])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize_matches_torch_oracle(dtype, seed):
    g = t.Generator().manual_seed(seed)
    x = (t.randn(256, 4, 128, generator=g) * t.logspace(-4, 4, 256).view(-1, 1, 1)).to(dtype)
    ref_codes, ref_scales = torch_reference_quantize(x)
    codes, scales = oracle.quantize(x.float().numpy())
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(scales, ref_scales)


def test_quantize_nan_row_follows_torch():
    x = np.float32([[1.0, np.nan, -2.0, 0.5]])
    codes, scales = oracle.quantize(x)
    ref_codes, ref_scales = torch_reference_quantize(t.from_numpy(x))
    assert np.array_equal(codes, ref_codes) and np.array_equal(scales, ref_scales)
    assert scales[0] == 1.0                      # NaN > 0 is False


@pytest.mark.parametrize("magnitude", [1e-3, 1.0, 1e3])
def test_round_trip_within_e4m3_bound(magnitude):
    # reference tests/test_kv_cache_quantization.py:95-107
    x = (np.random.default_rng(0).standard_normal((64, 4, 128)) * magnitude).astype(np.float32)
    codes, scales = oracle.quantize(x)
    assert (scales > 0).all()
    assert (np.abs(x - oracle.dequantize(codes, scales)) <= error_bound(x, scales)).all()


def test_largest_element_maps_to_fp8_max():
    # reference :110-114
    codes, scales = oracle.quantize(np.float32([[0.1, -3.0, 2.0, 0.5]]))
    assert oracle.e4m3fn_to_f32(codes)[0, 1] == -448.0
    assert math.isclose(oracle.dequantize(codes, scales)[0, 1], -3.0, rel_tol=1e-6)


def test_zero_vector_has_unit_scale_and_zero_codes():
    # reference :117-120
    codes, scales = oracle.quantize(np.zeros((3, 2, 16), dtype=np.float32))
    assert (scales == 1.0).all() and (codes == 0).all()


def test_outlier_channel_still_within_bound():
    # reference :123-131
    x = np.random.default_rng(1).standard_normal((32, 2, 64)).astype(np.float32)
    x[..., 7] *= 1000
    codes, scales = oracle.quantize(x)
    assert (np.abs(x - oracle.dequantize(codes, scales)) <= error_bound(x, scales)).all()


def test_never_produces_nan_or_inf():
    # reference :134-142
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal((16, 2, 32)) * 1e30, rng.standard_normal((16, 2, 32)) * 1e-30,
                        np.full((16, 2, 32), 65504.0)]).astype(np.float32)
    codes, scales = oracle.quantize(x)
    assert np.isfinite(oracle.e4m3fn_to_f32(codes)).all() and np.isfinite(scales).all()


def test_scatter_append_address_math():
    rng = np.random.default_rng(3)
    nb, bs, h, d = 6, 4, 2, 16
    k_cache = np.full((nb, bs, h, d), 0x55, dtype=np.uint8)
    v_cache = k_cache.copy()
    k_scales = np.full((nb, bs, h), -1.0, dtype=np.float32)
    v_scales = k_scales.copy()
    flat = rng.permutation(nb * bs)[:9]
    blocks, offsets = flat // bs, flat % bs
    ks = rng.standard_normal((9, h, d)).astype(np.float32)
    vs = rng.standard_normal((9, h, d)).astype(np.float32)
    oracle.scatter_append(k_cache, v_cache, k_scales, v_scales, ks, vs, blocks, offsets)
    # Flat index ((block * BS + offset) * H + head) * D + d, reference quantized_append.py:103-105.
    codes, scales = oracle.quantize(ks)
    flat_cache = k_cache.reshape(-1)
    for i in range(9):
        for head in range(h):
            base = ((blocks[i] * bs + offsets[i]) * h + head) * d
            assert np.array_equal(flat_cache[base:base + d], codes[i, head])
            assert k_scales.reshape(-1)[(blocks[i] * bs + offsets[i]) * h + head] == scales[i, head]
    written = np.zeros((nb, bs), dtype=bool)
    written[blocks, offsets] = True
    assert (k_cache[~written] == 0x55).all() and (v_scales[~written] == -1.0).all()


# ---------------------------------------------------------------------------
# Decode oracle
# ---------------------------------------------------------------------------

def _random_paged(rng, lengths, hq, hkv, d, bs=16):
    pages = [-(-n // bs) for n in lengths]
    nb = sum(pages) + 2
    perm = rng.permutation(nb)
    width = max(pages) + 1
    table = np.full((len(lengths), width), -1, dtype=np.int32)
    start = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[start:start + n]
        start += n
    k_cache = rng.integers(0, 256, (nb, bs, hkv, d)).astype(np.uint8)
    k_cache[(k_cache & 0x7F) == 0x7F] = 0x10          # no NaN codes in live data
    v_cache = rng.integers(0, 256, (nb, bs, hkv, d)).astype(np.uint8)
    v_cache[(v_cache & 0x7F) == 0x7F] = 0x20
    k_scales = rng.uniform(0.001, 0.02, (nb, bs, hkv)).astype(np.float32)
    v_scales = rng.uniform(0.001, 0.02, (nb, bs, hkv)).astype(np.float32)
    q = rng.standard_normal((len(lengths), hq, d)).astype(np.float32)
    return q, k_cache, v_cache, k_scales, v_scales, table


def test_decode_matches_brute_force_on_tiny_inputs():
    rng = np.random.default_rng(4)
    lengths = [1, 3, 17]
    q, kc, vc, ks, vs, table = _random_paged(rng, lengths, 4, 2, 8, bs=4)
    out = oracle.paged_decode(q, kc, vc, ks, vs, table, np.arange(3), lengths, 4)
    for b, n in enumerate(lengths):
        k, v = oracle.paged_history(kc, vc, ks, vs, table, b, n, 4)
        expected = brute_force_decode(q[b].tolist(), k.tolist(), v.tolist())
        np.testing.assert_allclose(out[b], np.array(expected), rtol=1e-12, atol=1e-12)


def test_decode_matches_torch_float64_attention():
    rng = np.random.default_rng(5)
    lengths = [5, 64, 65, 141]
    q, kc, vc, ks, vs, table = _random_paged(rng, lengths, 8, 2, 32)
    out = oracle.paged_decode(q, kc, vc, ks, vs, table, np.arange(4), lengths, 16)
    for b, n in enumerate(lengths):
        k, v = oracle.paged_history(kc, vc, ks, vs, table, b, n, 16)
        kt, vt = t.from_numpy(k), t.from_numpy(v)
        kh = kt.transpose(0, 1).repeat_interleave(4, 0)
        vh = vt.transpose(0, 1).repeat_interleave(4, 0)
        scores = (t.from_numpy(q[b]).double().unsqueeze(1) @ kh.transpose(-1, -2)).squeeze(1) / math.sqrt(32)
        ref = (scores.softmax(-1).unsqueeze(1) @ vh).squeeze(1).numpy()
        np.testing.assert_allclose(out[b], ref, rtol=1e-12, atol=1e-12)


def test_decode_invariants():
    rng = np.random.default_rng(6)
    lengths = [40, 100]
    q, kc, vc, ks, vs, table = _random_paged(rng, lengths, 8, 2, 16)
    base = oracle.paged_decode(q, kc, vc, ks, vs, table, np.arange(2), lengths, 16)

    # Physical page placement is invisible: move every page and rewrite the table.
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    table2 = np.where(table >= 0, inv[np.maximum(table, 0)], -1).astype(np.int32)
    moved = oracle.paged_decode(q, kc[perm], vc[perm], ks[perm], vs[perm], table2, np.arange(2), lengths, 16)
    np.testing.assert_allclose(moved, base, rtol=1e-13, atol=1e-13)

    # Slots select table rows: swapping rows and slots swaps nothing in the output.
    swapped = oracle.paged_decode(q, kc, vc, ks, vs, table[::-1].copy(), np.array([1, 0]), lengths, 16)
    np.testing.assert_allclose(swapped, base, rtol=1e-13, atol=1e-13)

    # GQA: query head h reads KV head h // 4 (a mixed-up mapping changes the output).
    q_same = q.copy()
    q_same[:, 4:] = q_same[:, :4]
    out_same = oracle.paged_decode(q_same, kc, vc, ks, vs, table, np.arange(2), lengths, 16)
    assert not np.allclose(out_same[:, :4], out_same[:, 4:])

    # Attention weights sum to one: a constant V row gives that constant back.
    vc_const = np.full_like(vc, 0x38)                  # 1.0
    vs_const = np.full_like(vs, 0.5)
    const = oracle.paged_decode(q, kc, vc_const, ks, vs_const, table, np.arange(2), lengths, 16)
    np.testing.assert_allclose(const, 0.5, rtol=1e-13)

    # One token: the output is that token's V row.
    one = oracle.paged_decode(q, kc, vc, ks, vs, table, np.arange(2), [1, 1], 16)
    _, v0 = oracle.paged_history(kc, vc, ks, vs, table, 0, 1, 16)
    np.testing.assert_allclose(one[0], np.repeat(v0[0], 4, axis=0), rtol=1e-13)

    # Empty context gives zeros (reference decode_attention.py:536-540).
    empty = oracle.paged_decode(q, kc, vc, ks, vs, table, np.arange(2), [0, 0], 16)
    assert (empty == 0).all()

    # The K scale multiplies the score, not the probability: doubling every K scale
    # sharpens the softmax (changes the output) while V scales scale the output.
    vs2 = oracle.paged_decode(q, kc, vc, ks, vs * 2, table, np.arange(2), lengths, 16)
    np.testing.assert_allclose(vs2, 2 * base, rtol=1e-12)
    ks2 = oracle.paged_decode(q, kc, vc, ks * 2, vs, table, np.arange(2), lengths, 16)
    assert not np.allclose(ks2, base)


def test_decode_matches_golden_cfg1():
    g = np.load(GOLDEN / "cfg1_decode.npz")
    nb = int(g["num_blocks"])
    hkv, d = g["k_codes"].shape[1:]
    k_cache = np.zeros((nb, 16, hkv, d), dtype=np.uint8)
    v_cache = np.zeros_like(k_cache)
    k_scales = np.ones((nb, 16, hkv), dtype=np.float32)
    v_scales = np.ones_like(k_scales)
    ks = (g["ks_bf16_bits"].astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    vs = (g["vs_bf16_bits"].astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    oracle.scatter_append(k_cache, v_cache, k_scales, v_scales, ks, vs, g["blocks"], g["offsets"])
    assert np.array_equal(k_cache[g["blocks"], g["offsets"]], g["k_codes"])
    assert np.array_equal(v_scales[g["blocks"], g["offsets"]], g["v_scales"])
    q = (g["q_bf16_bits"].astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    out = oracle.paged_decode(q, k_cache, v_cache, k_scales, v_scales, g["block_table"],
                              np.arange(len(g["lengths"])), g["lengths"], 16)
    np.testing.assert_allclose(out, g["expected_out"], rtol=1e-12, atol=1e-12)


def test_algorithmic_bytes_north_star():
    # 32 x 4096 tokens x 8 heads x (2*128 + 8) + 2 * 32*32*128*2 + 32*256*4 = 277.4 MB.
    nbytes = oracle.decode_algorithmic_bytes([4096] * 32, 32, 8, 128, 16)
    assert nbytes == 32 * 4096 * 8 * 264 + 2 * 32 * 32 * 128 * 2 + 32 * 256 * 4
    assert abs(nbytes / 1e6 - 277.4) < 0.1


@pytest.mark.parametrize("kv_dtype", [np.uint8, np.float16])
def test_decode_bytes_equal_the_arrays_one_call_touches(kv_dtype):
    """The byte count of a decode call, recounted from numpy `nbytes` of what the
    oracle gathers: every attended K and V row and its scale (fp8 only), q, the
    output, and the block-table entry of every attended page."""
    rng = np.random.default_rng(12)
    lengths = [0, 1, 15, 16, 17, 100]
    hq, hkv, d, bs = 8, 2, 24, 16
    q, kc, vc, ks, vs, table = _random_paged(rng, lengths, hq, hkv, d, bs)
    quantized = kv_dtype == np.uint8
    if not quantized:
        kc, vc, ks, vs = kc.astype(kv_dtype), vc.astype(kv_dtype), None, None
    q16 = q.astype(np.float16)
    touched = q16.nbytes + np.zeros((len(lengths), hq, d), np.float16).nbytes
    for b, n in enumerate(lengths):
        pos = np.arange(n)
        pages = table[b, pos // bs]
        touched += np.unique(pages).size * table.itemsize
        for cache in (kc, vc):
            touched += cache[pages, pos % bs].nbytes
        if quantized:
            touched += ks[pages, pos % bs].nbytes + vs[pages, pos % bs].nbytes
    got = oracle.decode_algorithmic_bytes(lengths, hq, hkv, d, bs, q_bytes=2, out_bytes=2,
                                          kv_bytes=np.dtype(kv_dtype).itemsize)
    assert got == touched


@pytest.mark.parametrize("in_dtype", [np.float32, np.float16])
def test_append_bytes_equal_the_arrays_one_call_touches(in_dtype):
    """The byte count of a quantize-and-scatter call, recounted from numpy `nbytes`:
    the K and V rows read in their input dtype, and the cache codes and scales the
    oracle's scatter writes (read back from the cache slices it changed)."""
    rng = np.random.default_rng(13)
    nb, bs, hkv, d, tokens = 9, 4, 3, 40, 17
    k_cache = np.zeros((nb, bs, hkv, d), np.uint8)
    v_cache = k_cache.copy()
    k_scales = np.zeros((nb, bs, hkv), np.float32)
    v_scales = k_scales.copy()
    flat = rng.permutation(nb * bs)[:tokens]
    blocks, offsets = flat // bs, flat % bs
    ks = rng.standard_normal((tokens, hkv, d)).astype(in_dtype)
    vs = rng.standard_normal((tokens, hkv, d)).astype(in_dtype)
    oracle.scatter_append(k_cache, v_cache, k_scales, v_scales, ks.astype(np.float32), vs.astype(np.float32),
                          blocks, offsets)
    written = sum(x[blocks, offsets].nbytes for x in (k_cache, v_cache, k_scales, v_scales))
    got = oracle.append_algorithmic_bytes(tokens, hkv, d, in_bytes=np.dtype(in_dtype).itemsize)
    assert got == ks.nbytes + vs.nbytes + written
    # And the cfg5 prefill write: 65,536 tokens x 4 heads x (2 x 128 x 2 + 2 x 128 + 8) = 203.4 MB.
    assert oracle.append_algorithmic_bytes(65536, 4, 128) == 65536 * 4 * 776


# ---------------------------------------------------------------------------
# Page-table gather (reference inference/page_allocator.py:225-245)
# ---------------------------------------------------------------------------

def test_physical_location_matches_a_page_walk():
    """Walking a slot's positions one at a time, with an offset counter that wraps
    at the page size and a page counter that advances on the wrap, visits the
    pages of the table row in order: the oracle's (page, offset) must agree at
    every position, for scalar and broadcast (slot, position) arguments."""
    rng = np.random.default_rng(14)
    for bs, width, slots in ((1, 7, 2), (4, 5, 3), (16, 3, 4)):
        table = rng.permutation(slots * width + 3)[:slots * width].reshape(slots, width).astype(np.int32)
        positions = np.arange(width * bs)
        for slot in range(slots):
            blocks, offsets = oracle.physical_location(table, slot, positions, bs)
            page_index, offset = 0, 0
            for pos in positions:
                assert (blocks[pos], offsets[pos]) == (table[slot, page_index], offset)
                offset += 1
                if offset == bs:
                    offset, page_index = 0, page_index + 1
        # A (slot, position) grid: every pair lands on its own cache row.
        grid_slots = np.repeat(np.arange(slots), width * bs)
        grid_pos = np.tile(positions, slots)
        blocks, offsets = oracle.physical_location(table, grid_slots, grid_pos, bs)
        rows = blocks * bs + offsets
        assert np.unique(rows).size == rows.size


# ---------------------------------------------------------------------------
# Causal varlen (prefill) attention
# ---------------------------------------------------------------------------

def _packed(rng, lengths, hq, hkv, d):
    total = sum(lengths)
    q = rng.standard_normal((total, hq, d))
    k = rng.standard_normal((total, hkv, d))
    v = rng.standard_normal((total, hkv, d))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return q, k, v, cu


def test_prefill_oracle_matches_brute_force_loops():
    rng = np.random.default_rng(21)
    lengths = [1, 4, 6]
    hq, hkv, d = 4, 2, 3
    q, k, v, cu = _packed(rng, lengths, hq, hkv, d)
    scale = 0.7
    out, lse = oracle.causal_varlen_attention(q, k, v, cu, max(lengths), scale)
    for b, n in enumerate(lengths):
        s0 = int(cu[b])
        for i in range(n):
            for h in range(hq):
                kv = h // (hq // hkv)
                s = [scale * sum(q[s0 + i, h, e] * k[s0 + t_, kv, e] for e in range(d)) for t_ in range(i + 1)]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                tot = sum(w)
                for e in range(d):
                    expected = sum(w[t_] * v[s0 + t_, kv, e] for t_ in range(i + 1)) / tot
                    assert abs(out[s0 + i, h, e] - expected) < 1e-12
                assert abs(lse[s0 + i, h] - (mx + math.log(tot))) < 1e-12


def test_prefill_oracle_matches_torch_sdpa():
    rng = np.random.default_rng(22)
    lengths = [3, 73, 141]                 # the reference test's ragged batch
    hq, hkv, d = 8, 2, 16
    q, k, v, cu = _packed(rng, lengths, hq, hkv, d)
    scale = 1.0 / math.sqrt(d)
    out, lse = oracle.causal_varlen_attention(q, k, v, cu, max(lengths), scale)
    for b, n in enumerate(lengths):
        s0 = int(cu[b])
        qs = t.from_numpy(q[s0:s0 + n]).transpose(0, 1)
        ks = t.from_numpy(k[s0:s0 + n]).transpose(0, 1).repeat_interleave(hq // hkv, 0)
        vs = t.from_numpy(v[s0:s0 + n]).transpose(0, 1).repeat_interleave(hq // hkv, 0)
        ref = t.nn.functional.scaled_dot_product_attention(qs, ks, vs, is_causal=True, scale=scale)
        np.testing.assert_allclose(out[s0:s0 + n], ref.transpose(0, 1).numpy(), rtol=1e-10, atol=1e-10)
        scores = scale * (qs @ ks.transpose(-1, -2))
        scores = scores.masked_fill(t.ones(n, n, dtype=t.bool).triu(1), float("-inf"))
        np.testing.assert_allclose(lse[s0:s0 + n], t.logsumexp(scores, -1).transpose(0, 1).numpy(),
                                   rtol=1e-10, atol=1e-10)


def test_prefill_oracle_invariants():
    rng = np.random.default_rng(23)
    lengths = [5, 0, 9]
    hq, hkv, d = 6, 3, 4
    q, k, v, cu = _packed(rng, lengths, hq, hkv, d)
    out, lse = oracle.causal_varlen_attention(q, k, v, cu, 9, 0.5)
    # Row 0 of a sequence attends only itself: its output is its own V row.
    for b in (0, 2):
        s0 = int(cu[b])
        for h in range(hq):
            np.testing.assert_allclose(out[s0, h], v[s0, h // 2], rtol=1e-13)
            assert abs(lse[s0, h] - 0.5 * float(q[s0, h] @ k[s0, h // 2])) < 1e-12
    # Causality: changing later tokens leaves earlier rows unchanged.
    k2, v2 = k.copy(), v.copy()
    k2[cu[2] + 6:] += 3.0
    v2[cu[2] + 6:] -= 2.0
    out2, _ = oracle.causal_varlen_attention(q, k2, v2, cu, 9, 0.5)
    np.testing.assert_array_equal(out2[: cu[2] + 6], out[: cu[2] + 6])
    assert not np.allclose(out2[cu[2] + 6:], out[cu[2] + 6:])
    # Truncation at max_seq_len: rows past it are not produced.
    out3, lse3 = oracle.causal_varlen_attention(q, k, v, cu, 4, 0.5)
    assert np.isnan(out3[cu[0] + 4]).all() and np.isnan(lse3[cu[2] + 4:]).all()
    np.testing.assert_array_equal(out3[cu[2]:cu[2] + 4], out[cu[2]:cu[2] + 4])
