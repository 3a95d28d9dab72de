"""Quantize-and-scatter append, reference `src/torch_llm/kernals/kv_cache/quantized_append.py:35-72`.

`quantize_append_wrapper(paged_kv_cache, ks, vs, physical_blocks, block_offsets)`
keeps the reference signature and contract (per token and KV head, over head_dim):

    amax  = max |x|                          (float32)
    scale = amax / 448 if amax > 0 else 1.0  (IEEE float32 division)
    code  = float8_e4m3fn(clamp(x / scale, -448, 448))   (round to nearest even)

and writes codes and scales in place at (block, offset, head). The work is one
launch of the gfx950 kernel `quantize_append_kernel` through the C ABI
`kvfp8_quantize_append` (include/kvfp8.h). Unlike the reference's Triton kernel,
whose float32 division may differ from torch's on a few codes
(reference `tests/test_kv_cache_quantization.py:246-266`), the codes and scales
are bit-identical to the torch oracle's.

Inputs are read through their strides when the head dimension is contiguous, so
non-contiguous views are not copied (the reference calls `.contiguous()`).
"""

from __future__ import annotations

import torch as t

from aiproj_amd import _native

_INPUT_DTYPES = (t.float32, t.float16, t.bfloat16)


def _prepare_input(x: t.Tensor) -> t.Tensor:
    if x.dtype not in _INPUT_DTYPES:
        x = x.float()          # the reference kernel works in float32 too
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _same_dtype(ks: t.Tensor, vs: t.Tensor):
    """K and V in one dtype for the kernel, with neither rounded again: when they
    differ both become float32, which holds every f16 and bf16 value exactly (the
    reference converts each input to float32 on its own)."""
    if ks.dtype == vs.dtype:
        return ks, vs
    return ks.float(), vs.float()


def quantize_append_wrapper(
    paged_kv_cache,
    ks,
    vs,
    physical_blocks,
    block_offsets,
):
    assert ks.shape == vs.shape
    assert paged_kv_cache.k.shape == paged_kv_cache.v.shape
    assert ks.shape[-2:] == paged_kv_cache.k.shape[-2:]
    assert paged_kv_cache.k.dtype == t.float8_e4m3fn

    num_blocks, block_size, num_kv_heads, head_dim = paged_kv_cache.k.shape
    num_tokens = ks.shape[0]
    device = _native.require_gpu(ks, vs, physical_blocks, block_offsets, paged_kv_cache.k,
                                 what="quantize_append_wrapper")
    if num_tokens == 0:
        return
    ks, vs = _same_dtype(_prepare_input(ks), _prepare_input(vs))

    rc = _native.fn("kvfp8_quantize_append")(
        ks.data_ptr(), vs.data_ptr(), _native.dtype_code(ks.dtype),
        ks.stride(0), ks.stride(1), vs.stride(0), vs.stride(1),
        physical_blocks.data_ptr(), _native.dtype_code(physical_blocks.dtype),
        block_offsets.data_ptr(), _native.dtype_code(block_offsets.dtype),
        num_tokens, num_kv_heads, head_dim, num_blocks, block_size,
        paged_kv_cache.k.data_ptr(), paged_kv_cache.v.data_ptr(),
        paged_kv_cache.k_scales.data_ptr(), paged_kv_cache.v_scales.data_ptr(),
        _native.stream_handle(device),
    )
    _native.check(rc, "kvfp8_quantize_append")


def store_append(paged_kv_cache, ks, vs, physical_blocks, block_offsets):
    """Plain (unquantized) device cache: cache[block, offset] = x.to(cache dtype).

    The device counterpart of reference `inference/paged_kv_cache.py:77-79`, one
    launch of `store_append_kernel` through `kvfp8_store_append`.
    """
    store_rows(paged_kv_cache.k, paged_kv_cache.v, ks, vs, physical_blocks, block_offsets, what="store_append")


def store_rows(k_cache, v_cache, ks, vs, rows, cols, what="store_rows"):
    """k_cache[rows[t], cols[t]] = ks[t] (and the same for V) for [R, C, H_kv, D] device caches.

    One launch of `store_append_kernel`: the cache is addressed as R pages of C slots.
    Entries with rows[t] outside [0, R) or cols[t] outside [0, C) are skipped.
    """
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    num_tokens = ks.shape[0]
    device = _native.require_gpu(ks, vs, rows, cols, k_cache, what=what)
    if num_tokens == 0:
        return
    ks, vs = _same_dtype(_prepare_input(ks), _prepare_input(vs))
    rc = _native.fn("kvfp8_store_append")(
        ks.data_ptr(), vs.data_ptr(), _native.dtype_code(ks.dtype),
        ks.stride(0), ks.stride(1), vs.stride(0), vs.stride(1),
        rows.data_ptr(), _native.dtype_code(rows.dtype),
        cols.data_ptr(), _native.dtype_code(cols.dtype),
        num_tokens, num_kv_heads, head_dim, num_blocks, block_size,
        k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype),
        _native.stream_handle(device),
    )
    _native.check(rc, "kvfp8_store_append")
