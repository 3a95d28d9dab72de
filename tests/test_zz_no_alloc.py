"""kvfp8_paged_decode_noalloc (the decode entry point that allocates nothing) against
kvfp8_paged_decode, through the C ABI.

The no-allocation call keeps its workspace in the library's static per-device array.
Its output must equal the allocating call's bit for bit. Checked here:
  * two calls in a row, the second on a smaller batch (the array keeps the first
    call's contents, and the second must not read them);
  * MFMA (one wave per KV head, and replicated heads) and generic kernels;
  * a shape whose workspace exceeds the array, refused on the host with KVFP8_ELIMIT
    before anything is launched.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch as t

from aiproj_amd import _native, workloads
from aiproj_amd.inference.paged_kv_cache import PagedKVCache
from aiproj_amd.kernals.decode_attention import prepare_decode

ELIMIT = -6
SCRATCH_BYTES = 32 << 20


def _decode_both(q, cache, ctx):
    """(allocating call's output, no-allocation call's output) for one decode."""
    call = prepare_decode(q, cache, ctx)
    call.run()
    want = call.output.clone()
    out = t.full_like(call.output, float("nan"))
    args = list(call.args)
    args[23] = out.data_ptr()                      # out
    rc = _native.lib().kvfp8_paged_decode_noalloc(*args[:24], args[26])
    _native.check(rc, "kvfp8_paged_decode_noalloc")
    t.cuda.synchronize()
    return want, out


def _cache_for(spec, dtype=t.float8_e4m3fn):
    w = workloads.build(spec, "cuda")
    cache = PagedKVCache(w.num_blocks, spec.block_size, spec.num_kv_heads, spec.head_dim, "cuda", dtype)
    workloads.fill_cache(w, cache, "cuda")
    k, v = workloads.new_kv(w, "cuda")
    cache.append_kv(w.new_blocks, w.new_offsets, k, v)
    return w, cache


@pytest.mark.gpu
@t.inference_mode()
@pytest.mark.parametrize("first,second", [("north", "cfg1"), ("cfg4", "cfg2")])
def test_noalloc_equals_allocating_decode_on_two_calls(first, second):
    """Second call smaller than the first: fewer sequences, fewer partial states."""
    for name in (first, second):
        spec = workloads.spec(name)
        w, cache = _cache_for(spec)
        want, got = _decode_both(w.q, cache, workloads.make_context(w))
        assert t.equal(got, want), name


@pytest.mark.gpu
@t.inference_mode()
def test_noalloc_with_replicated_heads():
    """16q/4kv shapes that run 8-wave workgroups with two replicas per KV head (their
    states merged in LDS), twice in a row, the second smaller."""
    for name, batch, length in (("rep_a", 64, 1040), ("rep_b", 8, 3000)):
        spec = workloads.WorkloadSpec(name, batch, 16, 4, 128, [length - 7 * (i % 3) for i in range(batch)],
                                      seed=52)
        w, cache = _cache_for(spec)
        want, got = _decode_both(w.q, cache, workloads.make_context(w))
        assert t.equal(got, want), name


@pytest.mark.gpu
@t.inference_mode()
def test_noalloc_on_the_generic_kernel():
    """Head size 80 and an f32 cache take the VALU kernel and its own workspace layout."""
    lengths = [1, 300, 17, 1000]
    for dtype, d, hq, hkv in ((t.float8_e4m3fn, 80, 8, 2), (t.float32, 64, 8, 2)):
        spec = workloads.WorkloadSpec("generic", len(lengths), hq, hkv, d, lengths, seed=51)
        w, cache = _cache_for(spec, dtype)
        want, got = _decode_both(w.q, cache, workloads.make_context(w))
        assert t.equal(got, want), (dtype, d)


@pytest.mark.gpu
@t.inference_mode()
def test_noalloc_in_a_captured_graph_replays_like_eager():
    """The call inside a HIP graph (the callers it is for), replayed three times with
    eager calls in between; every replay equals the allocating call."""
    spec = workloads.spec("cfg2")
    w, cache = _cache_for(spec)
    ctx = workloads.make_context(w)
    call = prepare_decode(w.q, cache, ctx)
    call.run()
    want = call.output.clone()
    out = t.empty_like(want)
    args = list(call.args)
    args[23] = out.data_ptr()
    lib = _native.lib()
    _native.check(lib.kvfp8_paged_decode_noalloc(*args[:24], args[26]), "noalloc")   # first call on the device
    t.cuda.synchronize()
    stream = t.cuda.Stream()
    graph = t.cuda.CUDAGraph()
    with t.cuda.stream(stream):
        with t.cuda.graph(graph, stream=stream):
            out.fill_(float("nan"))
            rc = lib.kvfp8_paged_decode_noalloc(*args[:24], stream.cuda_stream)
    _native.check(rc, "noalloc under capture")
    small = workloads.spec("cfg1")
    w1, cache1 = _cache_for(small)
    for _ in range(3):
        graph.replay()
        t.cuda.synchronize()
        assert t.equal(out, want)
        _decode_both(w1.q, cache1, workloads.make_context(w1))      # eager use of the same array
        out.zero_()
        t.cuda.synchronize()


@pytest.mark.gpu
def test_noalloc_refuses_shapes_beyond_its_array():
    """A workspace larger than the array: KVFP8_ELIMIT, before any launch. 512 q heads
    over 64 KV heads of D 128 on the MFMA kernel need 2 x 256 workgroups x 512 heads x
    130 floats = 136 MB of partial states."""
    lib = _native.lib()
    hq, hkv, d, batch = 512, 64, 128, 4
    need = lib.kvfp8_decode_workspace_bytes(batch, hq, hkv, d, 64, 16, _native.E4M3FN)
    assert need > SCRATCH_BYTES
    q = t.zeros(batch, hq, d, dtype=t.bfloat16, device="cuda")
    k = t.zeros(8, 16, hkv, d, dtype=t.uint8, device="cuda")
    scales = t.zeros(8, 16, hkv, dtype=t.float32, device="cuda")
    table = t.zeros(batch, 64, dtype=t.int32, device="cuda")
    idx = t.zeros(batch, dtype=t.int32, device="cuda")
    out = t.empty_like(q)
    rc = lib.kvfp8_paged_decode_noalloc(
        q.data_ptr(), _native.BF16, q.stride(0), q.stride(1), batch, hq, hkv, d,
        k.data_ptr(), k.data_ptr(), _native.E4M3FN, scales.data_ptr(), scales.data_ptr(), 8, 16,
        table.data_ptr(), batch, 64, idx.data_ptr(), _native.I32, idx.data_ptr(), _native.I32,
        1.0 / math.sqrt(d), out.data_ptr(), ctypes.c_void_p(t.cuda.current_stream().cuda_stream))
    assert rc == ELIMIT
