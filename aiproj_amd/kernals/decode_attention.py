"""Paged decode attention, reference `src/torch_llm/kernals/decode_attention.py:39-191`.

`decode_attention_wrapper(q, paged_kv_cache, cache_batch_context) -> Tensor` keeps the
reference signature and contract:
  * q [B, Hq, D]; the cache exposes k, v (+ k_scales, v_scales, quantized, block_size);
    the context exposes cache_slots [B], context_lengths [B] and the full block_table.
  * returns a new [B, Hq, D] tensor in q's dtype; query head h reads KV head
    h // (Hq / Hkv); scores are scaled by 1/sqrt(D); a sequence with no context
    gives zeros.
The optional second calling form of the reference's planned state API (handoff D18),
`decode_attention_wrapper(q, kv)` with `kv` a `PagedKVRead`, is accepted too.

Unlike the reference wrapper, this one never synchronizes with the host: the split
plan is built on the device inside the kernel (reference `:87-103` reads
`cum_splits[-1].item()`), and no dummy scale tensors are allocated for plain caches.
The work is two launches through the C ABI `kvfp8_paged_decode` (include/kvfp8.h);
`prepare_decode` returns the prepared call so the two launches can also be enqueued
one at a time.

`append_decode_attention(q, ks, vs, paged_kv_cache, cache_batch_context)` is the
decode step's append and attention together (reference `model/attention.py:86-99`
makes the two calls back to back). On an FP8 cache the decode kernel itself
writes each sequence's new token (`kvfp8_append_paged_decode`), after checking on the
device that its location is the sequence's last attended position, so the step has no
separate append launch; other caches and shapes make the two calls.
"""

from __future__ import annotations

import functools
import math
from dataclasses import dataclass

import torch as t

from aiproj_amd import _native

_Q_DTYPES = (t.float32, t.float16, t.bfloat16)


@dataclass(frozen=True)
class PagedKVRead:
    """What a paged-attention kernel reads (reference handoff D18, `todo:81-83`)."""

    k: t.Tensor
    v: t.Tensor
    k_scales: t.Tensor | None
    v_scales: t.Tensor | None
    block_table: t.Tensor
    slots: t.Tensor
    context_lengths: t.Tensor
    block_size: int

    @property
    def quantized(self) -> bool:
        return self.k_scales is not None


def _index_tensor(x: t.Tensor) -> t.Tensor:
    if x.dtype not in (t.int32, t.int64):
        raise ValueError("cache slots and context lengths must be int32 or int64")
    return x if x.is_contiguous() else x.contiguous()


def decode_attention_wrapper(q, paged_kv_cache, cache_batch_context=None):
    call = prepare_decode(q, paged_kv_cache, cache_batch_context, _launch_now=True)
    if call.args is not None:
        call.run()
    return call.output


@dataclass
class DecodeCall:
    """One prepared decode call: its output tensor, its workspace and the C-ABI
    argument tuple. `run()` enqueues both launches (`kvfp8_paged_decode`);
    `split()` and `reduce()` enqueue them one at a time (`kvfp8_paged_decode_split`
    then `kvfp8_paged_decode_reduce`, reference split and reduction kernels,
    `decode_attention.py:146-189`). `args` is None for an empty batch."""

    output: t.Tensor
    workspace: t.Tensor | None
    args: tuple | None
    keep: tuple = ()          # every tensor whose address is in `args`

    def run(self) -> None:
        _native.check(_native.fn("kvfp8_paged_decode")(*self.args), "kvfp8_paged_decode")

    def split(self) -> None:
        _native.check(_native.fn("kvfp8_paged_decode_split")(*self.args), "kvfp8_paged_decode_split")

    def reduce(self) -> None:
        _native.check(_native.fn("kvfp8_paged_decode_reduce")(*self.args), "kvfp8_paged_decode_reduce")


@functools.lru_cache(maxsize=256)
def _workspace_bytes(b, hq, hkv, d, bt_width, block_size, kv_code) -> int:
    """kvfp8_decode_workspace_bytes, which depends on shapes only (cached per shape)."""
    return _native.lib().kvfp8_decode_workspace_bytes(b, hq, hkv, d, bt_width, block_size, kv_code)


# Decode workspaces of the calls that launch at once (decode_attention_wrapper and the
# fused step), one per (device, stream): such calls run in stream order, so each can
# reuse the previous call's block (the workspace needs no initialization; every call
# rewrites what it reads). A call that needs more gets a larger block. Prepared calls
# (prepare_decode), which may be launched later and in halves, and every call under
# graph capture take a block of their own, so no two of them share one.
_WORKSPACES: dict = {}


def _workspace(device: t.device, stream: int, nbytes: int) -> t.Tensor:
    nbytes = max(nbytes, 1)
    if t.cuda.is_current_stream_capturing():
        return t.empty(nbytes, dtype=t.uint8, device=device)
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = t.empty(nbytes, dtype=t.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def prepare_decode(q, paged_kv_cache, cache_batch_context=None, _launch_now=False) -> DecodeCall:
    """Validate the arguments of `decode_attention_wrapper` (same forms, same
    asserts and errors), allocate its output and workspace, and return the
    prepared call without launching anything. (`_launch_now`: the caller launches the
    call right away on the current stream, so it may take the stream's shared
    workspace.)"""
    if cache_batch_context is None:
        kv = paged_kv_cache                       # PagedKVRead form
        k_cache, v_cache = kv.k, kv.v
        k_scales, v_scales = kv.k_scales, kv.v_scales
        quantized = kv.k_scales is not None
        block_size = kv.block_size
        cache_slots, context_lengths, block_table = kv.slots, kv.context_lengths, kv.block_table
    else:
        k_cache, v_cache = paged_kv_cache.k, paged_kv_cache.v
        quantized = paged_kv_cache.quantized
        k_scales = paged_kv_cache.k_scales if quantized else None
        v_scales = paged_kv_cache.v_scales if quantized else None
        block_size = paged_kv_cache.block_size
        cache_slots = cache_batch_context.cache_slots
        context_lengths = cache_batch_context.context_lengths
        block_table = cache_batch_context.block_table

    b, hq, d = q.shape
    assert k_cache.shape == v_cache.shape
    assert k_cache.ndim == 4
    num_blocks, cache_block_size, hkv, cache_d = k_cache.shape
    assert cache_d == d
    assert hq % hkv == 0
    assert cache_block_size == block_size
    assert block_size > 0 and block_size & (block_size - 1) == 0
    assert context_lengths.shape[0] == b
    assert cache_slots.shape[0] == b
    assert block_table.ndim == 2 and block_table.dtype == t.int32
    if quantized:
        assert k_cache.dtype == t.float8_e4m3fn
        assert k_scales.dtype == t.float32 and v_scales.dtype == t.float32

    device = _native.require_gpu(q, k_cache, v_cache, block_table, cache_slots, context_lengths,
                                 what="decode_attention_wrapper")
    output = t.empty((b, hq, d), dtype=q.dtype, device=q.device)
    if b == 0:
        return DecodeCall(output, None, None)

    if q.dtype not in _Q_DTYPES:
        raise ValueError(f"decode_attention_wrapper: unsupported q dtype {q.dtype}")
    if q.stride(-1) != 1:
        q = q.contiguous()
    for name, x in (("k", k_cache), ("v", v_cache), ("k_scales", k_scales), ("v_scales", v_scales)):
        if x is not None and not x.is_contiguous():
            raise ValueError(f"decode_attention_wrapper: cache tensor {name} must be contiguous")
    block_table = block_table if block_table.is_contiguous() else block_table.contiguous()
    cache_slots = _index_tensor(cache_slots)
    context_lengths = _index_tensor(context_lengths)

    kv_code = _native.dtype_code(k_cache.dtype)
    ws_bytes = _workspace_bytes(b, hq, hkv, d, block_table.shape[1], block_size, kv_code)
    stream = _native.stream_handle(device)
    if _launch_now:
        workspace = _workspace(device, stream, ws_bytes)
    else:
        workspace = t.empty(max(ws_bytes, 1), dtype=t.uint8, device=q.device)

    args = (
        q.data_ptr(), _native.dtype_code(q.dtype), q.stride(0), q.stride(1),
        b, hq, hkv, d,
        k_cache.data_ptr(), v_cache.data_ptr(), kv_code,
        _native.ptr(k_scales), _native.ptr(v_scales),
        num_blocks, block_size,
        block_table.data_ptr(), block_table.shape[0], block_table.shape[1],
        cache_slots.data_ptr(), _native.dtype_code(cache_slots.dtype),
        context_lengths.data_ptr(), _native.dtype_code(context_lengths.dtype),
        1.0 / math.sqrt(d),
        output.data_ptr(), workspace.data_ptr(), workspace.numel(),
        stream,
    )
    keep = (q, k_cache, v_cache, k_scales, v_scales, block_table, cache_slots, context_lengths)
    return DecodeCall(output, workspace, args, keep)


@functools.lru_cache(maxsize=256)
def _fused_supported(b, hq, hkv, d, bt_rows, bt_width, block_size, kv_code) -> bool:
    """kvfp8_append_decode_supported, which depends on shapes only (cached per shape)."""
    return _native.lib().kvfp8_append_decode_supported(b, hq, hkv, d, bt_rows, bt_width, block_size, kv_code) == 1


def append_decode_attention(q, ks, vs, paged_kv_cache, cache_batch_context, refused=None):
    """`paged_kv_cache.append_kv(ctx.physical_blocks, ctx.block_offsets, ks, vs)` followed by
    `decode_attention_wrapper(q, paged_kv_cache, ctx)`, the decode step of reference
    `model/attention.py:86-99`, with the same results (cache codes, scales and output
    bit-identical).

    ks, vs: [B, Hkv, D], the new token of every sequence of the batch.

    The step is one fused call (`kvfp8_append_paged_decode`) when the container says
    its write locations are the sequences' last attended positions
    (`appends_last_position`: set by `PageAllocator.create_container` after validating a
    one-token-per-sequence batch at the committed lengths, and by the runtime's decode
    step, which builds such metadata) and the cache is e4m3fn with a shape the MFMA
    kernel handles. The decode kernel writes row b at (physical_blocks[b],
    block_offsets[b]) before it reads that position. It checks every location against
    the block table on the device: a sequence whose location is not its last attended
    position has its row refused (not written; its output attends the cache as it is)
    and 1 is stored into `refused` (an int32 device tensor of one element that the
    caller zeroes, or None). Every other case makes the two calls.
    """
    cache, ctx = paged_kv_cache, cache_batch_context
    b, hq, d = q.shape
    hkv = cache.k.shape[2]
    expected = (b, hkv, d)
    if ks.shape != expected or vs.shape != expected:
        raise ValueError(f"append_decode_attention: new K/V must be {expected}")
    if refused is not None and (refused.dtype != t.int32 or refused.numel() != 1):
        raise ValueError("append_decode_attention: refused must be one int32 element")
    blocks, offsets = ctx.physical_blocks, ctx.block_offsets
    fused = (getattr(ctx, "appends_last_position", False)
             and cache.quantized and ks.dtype in _Q_DTYPES and vs.dtype in _Q_DTYPES
             and q.device.type == "cuda" and blocks.shape == (b,) and offsets.shape == (b,)
             and _fused_supported(b, hq, hkv, d, ctx.block_table.shape[0], ctx.block_table.shape[1],
                                  cache.block_size, _native.dtype_code(cache.k.dtype)))
    if not fused:
        cache.append_kv(blocks, offsets, ks, vs)
        return decode_attention_wrapper(q, cache, ctx)
    _native.require_gpu(ks, vs, cache.k, blocks, offsets, refused, what="append_decode_attention")
    call = prepare_decode(q, cache, ctx, _launch_now=True)
    if call.args is None:
        return call.output
    if vs.dtype != ks.dtype:
        # One dtype for both rows: float32 holds f16 and bf16 values exactly, so
        # neither row is rounded again before it is quantized.
        ks, vs = ks.float(), vs.float()
    if ks.stride(2) != 1 or ks.stride(1) != d:
        ks = ks.contiguous()
    if vs.stride(2) != 1 or vs.stride(1) != d:
        vs = vs.contiguous()
    blocks, offsets = _index_tensor(blocks), _index_tensor(offsets)
    rc = _native.fn("kvfp8_append_paged_decode")(
        *call.args, ks.data_ptr(), vs.data_ptr(), _native.dtype_code(ks.dtype),
        ks.stride(0), ks.stride(1), vs.stride(0), vs.stride(1),
        blocks.data_ptr(), _native.dtype_code(blocks.dtype), offsets.data_ptr(), _native.dtype_code(offsets.dtype),
        _native.ptr(refused))
    _native.check(rc, "kvfp8_append_paged_decode")
    return call.output
