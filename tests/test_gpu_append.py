"""HIP quantize-and-scatter append vs the oracle (GPU).

Mirrors section E of reference tests/test_kv_cache_quantization.py:242-391, with a
stricter bar: codes and scales must be bit-identical to the torch/numpy oracle
(the reference allowed 1% code mismatch for its Triton division).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch as t

import oracle
from aiproj_amd.inference.kv_cache import KVCache
from aiproj_amd.inference.page_allocator import PageAllocator
from aiproj_amd.inference.paged_kv_cache import PagedKVCache
from tests.helpers import FP8, error_bound, scattered_locations, torch_reference_quantize

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def stored(cache, blocks, offsets):
    """(k codes, k scales, v codes, v scales) at the given locations, as numpy."""
    return (cache.k[blocks, offsets].view(t.uint8).cpu().numpy(), cache.k_scales[blocks, offsets].cpu().numpy(),
            cache.v[blocks, offsets].view(t.uint8).cpu().numpy(), cache.v_scales[blocks, offsets].cpu().numpy())


def assert_bit_exact(cache, blocks, offsets, ks, vs):
    kc, ksc, vc, vsc = stored(cache, blocks, offsets)
    for x, codes, scales in ((ks, kc, ksc), (vs, vc, vsc)):
        ref_codes, ref_scales = torch_reference_quantize(x.cpu())
        assert np.array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
        mismatch = codes != ref_codes
        assert not mismatch.any(), f"{mismatch.sum()} of {codes.size} codes differ"
        o_codes, o_scales = oracle.quantize(x.float().cpu().numpy())
        assert np.array_equal(codes, o_codes) and np.array_equal(scales, o_scales)


@t.inference_mode()
@pytest.mark.parametrize("input_dtype", [t.float32, t.float16, t.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 64, 80, 128, 256])
def test_fp8_append_is_bit_exact(input_dtype, head_dim):
    t.manual_seed(2)
    num_blocks, block_size, num_kv_heads, num_tokens = 16, 16, 4, 100
    cache = PagedKVCache(num_blocks, block_size, num_kv_heads, head_dim, "cuda", FP8)
    blocks, offsets = scattered_locations(num_tokens, num_blocks, block_size, "cuda")
    ks = (t.randn(num_tokens, num_kv_heads, head_dim, device="cuda") * 3).to(input_dtype)
    vs = t.randn(num_tokens, num_kv_heads, head_dim, device="cuda").to(input_dtype)
    cache.append_kv(blocks, offsets, ks, vs)
    assert_bit_exact(cache, blocks, offsets, ks, vs)


@t.inference_mode()
def test_fp8_append_writes_only_targeted_slots():
    cache = PagedKVCache(8, 4, 2, 32, "cuda", FP8)
    cache.k.copy_(t.full(cache.k.shape, 5.0, device="cuda").to(FP8))
    cache.v.copy_(t.full(cache.v.shape, 5.0, device="cuda").to(FP8))
    cache.k_scales.fill_(-1.0)
    cache.v_scales.fill_(-1.0)
    blocks, offsets = scattered_locations(11, 8, 4, "cuda")
    cache.append_kv(blocks, offsets, t.randn(11, 2, 32, device="cuda"), t.randn(11, 2, 32, device="cuda"))
    written = t.zeros(8, 4, dtype=t.bool, device="cuda")
    written[blocks, offsets] = True
    for storage in (cache.k, cache.v):
        assert (storage[~written].float() == 5.0).all()
    for scales in (cache.k_scales, cache.v_scales):
        assert (scales[~written] == -1.0).all()
        assert (scales[written] > 0).all()


@t.inference_mode()
def test_fp8_append_accepts_non_contiguous_input():
    t.manual_seed(3)
    cache = PagedKVCache(8, 4, 2, 32, "cuda", FP8)
    blocks, offsets = scattered_locations(10, 8, 4, "cuda")
    ks = t.randn(2, 10, 32, device="cuda").transpose(0, 1)
    vs = t.randn(2, 10, 32, device="cuda").transpose(0, 1)
    assert not ks.is_contiguous()
    cache.append_kv(blocks, offsets, ks, vs)
    assert_bit_exact(cache, blocks, offsets, ks, vs)
    # A view whose last dimension is strided is copied, not misread.
    ks2 = t.randn(10, 32, 2, device="cuda").transpose(1, 2)
    cache.append_kv(blocks, offsets, ks2, ks2)
    assert_bit_exact(cache, blocks, offsets, ks2, ks2)


@t.inference_mode()
@pytest.mark.parametrize("input_dtype,peak", [(t.float32, 1e30), (t.float32, 1e-30), (t.float16, 65504.0),
                                              (t.bfloat16, 1e30)])
def test_fp8_append_extreme_magnitudes(input_dtype, peak):
    t.manual_seed(4)
    cache = PagedKVCache(8, 8, 2, 64, "cuda", FP8)
    blocks, offsets = scattered_locations(40, 8, 8, "cuda")
    x = t.randn(40, 2, 64, device="cuda", dtype=t.float64)
    x = (x / x.abs().amax(-1, keepdim=True) * peak).to(input_dtype)
    cache.append_kv(blocks, offsets, x, x)
    assert_bit_exact(cache, blocks, offsets, x, x)
    k = cache.k[blocks, offsets].float() * cache.k_scales[blocks, offsets].unsqueeze(-1)
    assert t.isfinite(k).all()
    assert (cache.k_scales[blocks, offsets] > 0).all()


@t.inference_mode()
def test_fp8_append_zero_vectors():
    cache = PagedKVCache(4, 4, 2, 16, "cuda", FP8)
    blocks, offsets = scattered_locations(5, 4, 4, "cuda")
    zeros = t.zeros(5, 2, 16, device="cuda")
    cache.append_kv(blocks, offsets, zeros, zeros)
    assert (cache.k_scales[blocks, offsets] == 1.0).all()
    assert (cache.k[blocks, offsets].float() == 0).all()


@t.inference_mode()
def test_fp8_append_nan_rows_follow_torch():
    cache = PagedKVCache(4, 4, 1, 16, "cuda", FP8)
    blocks, offsets = scattered_locations(3, 4, 4, "cuda")
    x = t.randn(3, 1, 16, device="cuda")
    x[1, 0, 5] = float("nan")
    x[2, 0, 0] = -float("nan")
    cache.append_kv(blocks, offsets, x, x)
    assert_bit_exact(cache, blocks, offsets, x, x)


@t.inference_mode()
def test_fp8_append_through_cache_manager_round_trips():
    t.manual_seed(5)
    manager = PageAllocator(16, 4, 2, 32, "cuda")
    cache = PagedKVCache(16, 4, 2, 32, "cuda", FP8)
    length = 13
    slot = manager.allocate_request(0, length)
    ks = t.randn(length, 2, 32, device="cuda", dtype=t.bfloat16)
    vs = t.randn_like(ks)
    manager.append_request(0, t.arange(length, device="cuda"), ks, vs, cache)
    positions = t.arange(length, device="cuda")
    blocks = manager.block_table[slot, positions // 4]
    offsets = positions % 4
    assert_bit_exact(cache, blocks, offsets, ks, vs)
    k = (cache.k[blocks, offsets].float() * cache.k_scales[blocks, offsets].unsqueeze(-1)).cpu().numpy()
    _, k_scales = oracle.quantize(ks.float().cpu().numpy())
    assert (np.abs(ks.float().cpu().numpy() - k) <= 2 * error_bound(ks.float().cpu().numpy(), k_scales)).all()


@t.inference_mode()
@pytest.mark.parametrize("index_dtype", [t.int32, t.int64])
def test_fp8_append_index_dtypes_and_out_of_pool_rows(index_dtype):
    cache = PagedKVCache(6, 4, 2, 64, "cuda", FP8)
    cache.k.view(t.uint8).fill_(0x11)
    cache.k_scales.fill_(-2.0)
    blocks = t.tensor([0, 5, -1, 6, 2, 1], dtype=index_dtype, device="cuda")
    offsets = t.tensor([3, 0, 1, 1, 4, 2], dtype=index_dtype, device="cuda")   # rows 2, 3, 4 are outside
    x = t.randn(6, 2, 64, device="cuda")
    cache.append_kv(blocks, offsets, x, x)
    good = t.tensor([0, 1, 5], device="cuda")
    assert_bit_exact(cache, blocks[good].long(), offsets[good].long(), x[good], x[good])
    written = t.zeros(6, 4, dtype=t.bool)
    written[[0, 5, 1], [3, 0, 2]] = True
    assert (cache.k.view(t.uint8)[~written.cuda()] == 0x11).all()
    assert (cache.k_scales[~written.cuda()] == -2.0).all()


@t.inference_mode()
def test_golden_quantize_cases_on_gpu():
    cases = np.load(GOLDEN / "quantize_cases.npz")
    for name in sorted({key.split("__")[0] for key in cases.files}):
        x = cases[f"{name}__x"]
        dtype = {"torch.float32": t.float32, "torch.float16": t.float16,
                 "torch.bfloat16": t.bfloat16}[str(cases[f"{name}__dtype"])]
        rows = x.reshape(-1, x.shape[-1])
        n, d = rows.shape
        cache = PagedKVCache(-(-n // 16), 16, 1, d, "cuda", FP8)
        flat = t.arange(n, device="cuda")
        xt = t.from_numpy(rows).to(dtype).cuda().unsqueeze(1)
        cache.append_kv(flat // 16, flat % 16, xt, xt)
        codes = cache.k.view(t.uint8).reshape(-1, d)[:n].cpu().numpy()
        scales = cache.k_scales.reshape(-1)[:n].cpu().numpy()
        assert np.array_equal(codes, cases[f"{name}__codes"].reshape(-1, d)), name
        assert np.array_equal(scales.view(np.uint32), cases[f"{name}__scales"].reshape(-1).view(np.uint32)), name


@t.inference_mode()
@pytest.mark.parametrize("input_dtype,head_dim,hkv,index_dtype,tokens", [
    (t.bfloat16, 128, 4, t.int32, 65536 + 37),       # the cfg5 prefill layer plus a ragged tail
    (t.float16, 80, 2, t.int64, 131072 + 11),        # lanes past D in every row
    (t.float32, 64, 8, t.int32, 65536 + 5),          # four lanes per row
])
def test_fp8_append_at_prefill_sizes(input_dtype, head_dim, hkv, index_dtype, tokens):
    # Row counts above the multi-row kernel's threshold (4096 blocks of 4 passes):
    # shuffled slots, a few write locations outside the pool, bit-exact against the
    # oracle, untouched slots unchanged.
    g = t.Generator(device="cuda").manual_seed(tokens)
    num_blocks = tokens // 16 + 8
    slots = t.randperm(num_blocks * 16, device="cuda", generator=g)[:tokens]
    blocks, offsets = (slots // 16).to(index_dtype), (slots % 16).to(index_dtype)
    outside = t.tensor([0, 7, tokens // 2, tokens - 1], device="cuda")
    blocks[outside[:2]] = t.tensor([-1, num_blocks], dtype=index_dtype, device="cuda")
    offsets[outside[2:]] = t.tensor([16, -3], dtype=index_dtype, device="cuda")
    cache = PagedKVCache(num_blocks, 16, hkv, head_dim, "cuda", FP8)
    cache.k.view(t.uint8).fill_(0x5A)
    cache.k_scales.fill_(-1.0)
    ks = t.randn(tokens, hkv, head_dim, device="cuda", generator=g).to(input_dtype)
    vs = (t.randn(tokens, hkv, head_dim, device="cuda", generator=g) * 1e-3).to(input_dtype)
    cache.append_kv(blocks, offsets, ks, vs)
    keep = t.ones(tokens, dtype=t.bool, device="cuda")
    keep[outside] = False
    b, o = blocks[keep].long(), offsets[keep].long()
    for x, codes, scales in ((ks, cache.k, cache.k_scales), (vs, cache.v, cache.v_scales)):
        got_codes = codes[b, o].view(t.uint8).cpu().numpy()
        got_scales = scales[b, o].cpu().numpy()
        want_codes, want_scales = oracle.quantize(x[keep].float().cpu().numpy())
        assert np.array_equal(got_scales.view(np.uint32), want_scales.view(np.uint32))
        assert np.array_equal(got_codes, want_codes), f"{(got_codes != want_codes).sum()} codes differ"
    written = t.zeros(num_blocks, 16, dtype=t.bool, device="cuda")
    written[b, o] = True
    assert (cache.k.view(t.uint8)[~written] == 0x5A).all()
    assert (cache.k_scales[~written] == -1.0).all()


@t.inference_mode()
@pytest.mark.parametrize("input_dtype", [t.bfloat16, t.float32])
def test_fp8_append_large_random_sweep_is_bit_exact(input_dtype):
    # 262144 rows over 16 decades of magnitude: every division and rounding path.
    g = t.Generator(device="cuda").manual_seed(11)
    rows, d = 1 << 18, 128
    scale = t.logspace(-30, 30, rows, device="cuda").view(-1, 1, 1)
    x = (t.randn(rows, 1, d, device="cuda", generator=g) * scale).to(input_dtype)
    cache = PagedKVCache(rows // 16, 16, 1, d, "cuda", FP8)
    flat = t.arange(rows, device="cuda")
    cache.append_kv(flat // 16, flat % 16, x, x)
    codes = cache.k.view(t.uint8).reshape(rows, d).cpu().numpy()
    scales = cache.k_scales.reshape(rows).cpu().numpy()
    o_codes, o_scales = oracle.quantize(x.float().cpu().numpy().reshape(rows, d))
    assert np.array_equal(scales.view(np.uint32), o_scales.view(np.uint32))
    assert np.array_equal(codes, o_codes), f"{(codes != o_codes).sum()} codes differ"


@t.inference_mode()
@pytest.mark.parametrize("cache_dtype", [t.float16, t.bfloat16, t.float32])
@pytest.mark.parametrize("input_dtype", [t.float32, t.bfloat16])
def test_unquantized_device_append(cache_dtype, input_dtype):
    cache = PagedKVCache(6, 4, 2, 80, "cuda", cache_dtype)
    cache.k.fill_(-7.0)
    cache.v.fill_(-7.0)
    blocks, offsets = scattered_locations(9, 6, 4, "cuda")
    ks = t.randn(9, 2, 80, device="cuda").to(input_dtype)
    vs = t.randn(9, 2, 80, device="cuda").to(input_dtype)
    cache.append_kv(blocks, offsets, ks, vs)
    assert t.equal(cache.k[blocks, offsets], ks.to(cache_dtype))
    assert t.equal(cache.v[blocks, offsets], vs.to(cache_dtype))
    written = t.zeros(6, 4, dtype=t.bool, device="cuda")
    written[blocks, offsets] = True
    assert (cache.k[~written] == -7.0).all()


@t.inference_mode()
def test_golden_cfg1_cache_bytes():
    g = np.load(GOLDEN / "cfg1_decode.npz")
    nb = int(g["num_blocks"])
    hkv, d = g["k_codes"].shape[1:]
    cache = PagedKVCache(nb, 16, int(hkv), int(d), "cuda", FP8)
    ks = t.from_numpy(g["ks_bf16_bits"]).view(t.bfloat16).cuda()
    vs = t.from_numpy(g["vs_bf16_bits"]).view(t.bfloat16).cuda()
    blocks = t.from_numpy(g["blocks"]).cuda()
    offsets = t.from_numpy(g["offsets"]).cuda()
    cache.append_kv(blocks, offsets, ks, vs)
    kc, ksc, vc, vsc = stored(cache, blocks, offsets)
    assert np.array_equal(kc, g["k_codes"]) and np.array_equal(vc, g["v_codes"])
    assert np.array_equal(ksc.view(np.uint32), g["k_scales"].view(np.uint32))
    assert np.array_equal(vsc.view(np.uint32), g["v_scales"].view(np.uint32))


def test_hardware_encoder_matches_software_encoder_on_every_fast_path_value():
    # The append kernel converts finite rows with the hardware RNE converter; it must
    # agree with the software encoder (pinned to the oracle on the CPU) on every
    # float32 the corrected division can produce, |x| <= 448 (1 + 2^-19), both signs.
    from aiproj_amd import _native
    mismatches = t.zeros(1, dtype=t.int64, device="cuda")
    rc = _native.lib().kvfp8_selftest_fp8_encoder(mismatches.data_ptr(), _native.stream_handle(mismatches.device))
    _native.check(rc, "kvfp8_selftest_fp8_encoder")
    t.cuda.synchronize()
    assert mismatches.item() == 0


@t.inference_mode()
@pytest.mark.parametrize("cache_dtype,input_dtype", [(t.bfloat16, t.float32), (t.float16, t.bfloat16),
                                                     (t.float32, t.float16)])
def test_dense_cache_device_writes_match_host_cache(cache_dtype, input_dtype):
    """The dense cache's HIP store equals the reference's indexed store (host cache),
    bit for bit, over ragged prompts into a subset of slots and then decode steps."""
    g = t.Generator().manual_seed(41)
    hkv, d, slots_total, capacity = 4, 128, 9, 300
    dev = KVCache(slots_total, capacity, hkv, d, cache_dtype, "cuda")
    host = KVCache(slots_total, capacity, hkv, d, cache_dtype, "cpu")
    for c in (dev, host):
        c.k_cache.zero_()
        c.v_cache.zero_()
    slots = [7, 0, 3, 5, 2]
    lengths = [0, 1, 17, 200, 64]
    cu = t.tensor([0, *np.cumsum(lengths).tolist()], dtype=t.int32)
    k = (t.randn(int(cu[-1]), hkv, d, generator=g) * 3).to(input_dtype)
    v = (t.randn(int(cu[-1]), hkv, d, generator=g) * 3).to(input_dtype)
    host.append_prefill(k, v, cu, slots)
    dev.append_prefill(k.cuda(), v.cuda(), cu.cuda(), t.tensor(slots, device="cuda"))
    for step in range(3):
        chosen = [3, 7, 8] if step != 1 else [0, 5]
        nk = t.randn(len(chosen), hkv, d, generator=g).to(input_dtype)
        nv = t.randn(len(chosen), hkv, d, generator=g).to(input_dtype)
        host.append_decode(nk, nv, chosen)
        dev.append_decode(nk.cuda(), nv.cuda(), chosen)
    assert dev.seq_lens.cpu().tolist() == host.seq_lens.tolist()
    assert t.equal(dev.k_cache.cpu(), host.k_cache) and t.equal(dev.v_cache.cpu(), host.v_cache)
    assert host.seq_lens.tolist()[4] == 0 and bool((host.k_cache[4] == 0).all())
