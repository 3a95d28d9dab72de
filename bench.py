#!/usr/bin/env python
"""Benchmark of the FP8 paged KV-cache decode step on one MI355X.

A step is one pass of the hot path over one batch: quantize-and-scatter the new
K/V token of every sequence into the FP8 paged cache, then paged decode attention
of every sequence over its whole context (reference call site
`src/torch_llm/model/attention.py:86-99`). Inputs are synthetic and resident in HBM
before timing starts. Independent cache pools are rotated step to step so their
total exceeds twice the 256 MB Infinity Cache: every step reads its KV from HBM.
The timed steps are replayed from HIP graphs of 32 steps, the decode step of a
32-layer model (Llama-3-8B) with one attention step per layer.

Default workload ("north"): B=32, 32 q / 8 KV heads, D=128, page 16, every
context 4096 tokens, e4m3fn cache, bf16 q (the metric's "B=32 4k ctx"). The
cfg2 draw (contexts ~ U[512, 4096]) is measured too and reported as `secondary`.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "FP8 paged decode-attn HBM GB/s (% of peak) + KV tokens/s, B=32 4k ctx"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0     # dense bf16 MFMA
MALL_BYTES = 256 * 2 ** 20
MAX_POOLS = 64
# Steps per HIP graph: the decode step of a 32-layer model (Llama-3-8B, whose attention shape
# the north star and cfg2 name) is one graph holding one attention step per layer.
LAYERS_PER_GRAPH = 32


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="north",
                   choices=["north", "cfg2", "cfg3", "cfg4", "cfg1", "cfg5", "prefill", "kernels"],
                   help="cfg5 runs only the decoder-LM leg, prefill only the two prefill legs, kernels only "
                        "the bf16-cache, MFMA-vs-VALU and D-80 decode legs; each prints its own JSON line")
    p.add_argument("--no-kernels", action="store_true", help="skip the bf16-cache and MFMA-vs-VALU decode legs")
    p.add_argument("--secondary", default="cfg2", help="second workload to report ('' for none)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-prefill", action="store_true", help="skip the prefill-size append and attention legs")
    p.add_argument("--no-model", action="store_true", help="skip the cfg5 model decode leg")
    p.add_argument("--no-others", action="store_true", help="skip the cfg1/cfg3/cfg4 decode legs")
    p.add_argument("--no-sweep", action="store_true", help="skip the reference-style batch x context sweep")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    return p.parse_args()


class Setup:
    """Rotating cache pools, the batch metadata and per-step new tokens of one workload."""

    def __init__(self, name: str, device):
        import torch as t
        from aiproj_amd import workloads
        from aiproj_amd.inference.paged_kv_cache import PagedKVCache
        import oracle

        self.spec = workloads.spec(name)
        s = self.spec
        self.w = workloads.build(s, device)
        self.context = workloads.make_context(self.w)
        self.decode_bytes = oracle.decode_algorithmic_bytes(s.lengths, s.num_q_heads, s.num_kv_heads,
                                                            s.head_dim, s.block_size)
        self.append_bytes = oracle.append_algorithmic_bytes(s.batch, s.num_kv_heads, s.head_dim, in_bytes=2)
        pool_bytes = self.w.num_blocks * s.block_size * s.num_kv_heads * (2 * s.head_dim + 8)
        # Enough pools to exceed twice the Infinity Cache; a tiny (launch-bound)
        # workload such as cfg1 is capped at MAX_POOLS and stays cache-resident.
        self.num_pools = min(MAX_POOLS, max(2, math.ceil(2 * MALL_BYTES / pool_bytes) + 1))
        self.pool_bytes = pool_bytes
        self.caches = []
        for _ in range(self.num_pools):
            cache = PagedKVCache(self.w.num_blocks, s.block_size, s.num_kv_heads, s.head_dim, device, t.float8_e4m3fn)
            workloads.fill_cache(self.w, cache, device)
            self.caches.append(cache)
        self.new_tokens = [workloads.new_kv(self.w, device, step) for step in range(4)]
        t.cuda.synchronize()

    # The step: the 1-token append and the decode attention of reference
    # model/attention.py:86-99. `fused` takes the single call that writes the new
    # token inside the decode kernel; otherwise the two calls, append_kv then
    # decode_attention_wrapper.
    fused = True

    def step(self, i: int):
        from aiproj_amd.kernals.decode_attention import append_decode_attention, decode_attention_wrapper

        cache = self.caches[i % self.num_pools]
        k, v = self.new_tokens[i % len(self.new_tokens)]
        if self.fused:
            return append_decode_attention(self.w.q, k, v, cache, self.context)
        cache.append_kv(self.w.new_blocks, self.w.new_offsets, k, v)
        return decode_attention_wrapper(self.w.q, cache, self.context)

    def capture(self, steps: int):
        """HIP graphs holding whole steps (the append and the decode), as a multi-layer
        model captures its decode step: LAYERS_PER_GRAPH steps per graph, step i on cache
        pool i % num_pools (each layer on its own cache; the pools together exceed twice
        the last-level cache, so no step finds its cache resident; the cfg5 leg captures
        all 16 layers of its model the same way). Returns (graph of LAYERS_PER_GRAPH
        steps, graph of steps % LAYERS_PER_GRAPH steps or None): replaying the first
        steps // LAYERS_PER_GRAPH times and the second once runs exactly `steps` steps."""
        import torch as t

        def graph_of(n):
            g = t.cuda.CUDAGraph()
            with t.cuda.graph(g):
                for i in range(n):
                    self.step(i)
            return g

        full = graph_of(LAYERS_PER_GRAPH)
        rest = steps % LAYERS_PER_GRAPH
        tail = graph_of(rest) if rest else None
        t.cuda.synchronize()
        return full, tail


class _NoGC:
    """Python's cyclic garbage collector off inside a timed region (a collection
    pause would leave the GPU idle between launches)."""

    def __enter__(self):
        gc.collect()
        gc.disable()

    def __exit__(self, *exc):
        gc.enable()


def time_steps(setup: Setup, steps: int, warmup: int):
    """Timed regions of `steps` calls each, after `warmup` eager steps:
      * graph replay of whole steps, LAYERS_PER_GRAPH steps per graph (no host work
        between steps, one graph launch per model step): ms per step, for the step as
        the two separate calls and as the fused call;
      * the split (decode) kernel alone, `steps` launches back to back on the
        current stream between two HIP events, pools rotating: its mean launch
        duration, the figure the roofline divides by; then the whole call (split and
        combine) the same way, and the split's median with events around each launch;
      * eager steps (the fused call): ms per step; then the same steps with HIP events
        on the dispatch packet of every decode-kernel launch (hipExtLaunchKernel, here
        the fused kernel): per-dispatch kernel ms;
      * eager steps as the reference runtime makes them, the two calls with no graph.
    """
    import ctypes
    import torch as t
    from aiproj_amd import _native
    from aiproj_amd.kernals.decode_attention import prepare_decode

    lib = _native.lib()
    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)

    def graph_ms_per_step():
        for i in range(warmup):
            setup.step(i)
        t.cuda.synchronize()
        full, tail = setup.capture(steps)
        full.replay()
        if tail is not None:
            tail.replay()
        t.cuda.synchronize()
        with _NoGC():
            start.record()
            for _ in range(steps // LAYERS_PER_GRAPH):
                full.replay()
            if tail is not None:
                tail.replay()
            end.record()
            t.cuda.synchronize()
        return start.elapsed_time(end) / steps

    # The step as the reference's two calls, then the fused call (the step measured).
    fused = setup.fused
    setup.fused = False
    separate_ms = graph_ms_per_step()
    setup.fused = fused
    graph_ms = graph_ms_per_step()

    calls = [prepare_decode(setup.w.q, cache, setup.context) for cache in setup.caches]
    for c in calls:
        c.split()
    t.cuda.synchronize()
    with _NoGC():
        start.record()
        for i in range(steps):
            calls[i % len(calls)].split()
        end.record()
        t.cuda.synchronize()
    split_ms = start.elapsed_time(end) / steps
    # The whole decode call as the reference defines it (split kernel, then the
    # combine): `steps` calls back to back, pools rotating.
    with _NoGC():
        start.record()
        for i in range(steps):
            calls[i % len(calls)].run()
        end.record()
        t.cuda.synchronize()
    call_ms = start.elapsed_time(end) / steps
    # The same launches one at a time, each between its own pair of events: the median.
    pairs = [(t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)) for _ in range(steps)]
    with _NoGC():
        for i, (e0, e1) in enumerate(pairs):
            e0.record()
            calls[i % len(calls)].split()
            e1.record()
        t.cuda.synchronize()
    split_median_ms = float(sorted(e0.elapsed_time(e1) for e0, e1 in pairs)[steps // 2])
    del calls, pairs

    # Eager steps (the fused call) with no instrumentation, then the same steps with
    # HIP events on every decode-kernel dispatch (those events slow the eager loop, so
    # they give only the per-dispatch kernel time).
    with _NoGC():
        start.record()
        for i in range(steps):
            setup.step(warmup + i)
        end.record()
        t.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / steps
    _native.check(lib.kvfp8_timing_enable(steps), "kvfp8_timing_enable")
    t.cuda.synchronize()
    with _NoGC():
        for i in range(steps):
            setup.step(warmup + i)
        t.cuda.synchronize()
    total_ms = ctypes.c_double(0.0)
    launches = ctypes.c_int64(0)
    _native.check(lib.kvfp8_timing_read(ctypes.byref(total_ms), ctypes.byref(launches)), "kvfp8_timing_read")
    dispatch_ms = total_ms.value / max(1, launches.value)
    # The drop-in under the reference's own runtime: eager steps as its two calls
    # (append_kv, then decode_attention_wrapper; model/attention.py:88-99), no graph.
    setup.fused = False
    for i in range(warmup):
        setup.step(i)
    t.cuda.synchronize()
    with _NoGC():
        start.record()
        for i in range(steps):
            setup.step(warmup + i)
        end.record()
        t.cuda.synchronize()
    eager_two_calls_ms = start.elapsed_time(end) / steps
    setup.fused = fused
    return {"graph_ms": graph_ms, "separate_ms": separate_ms, "eager_ms": eager_ms, "split_ms": split_ms,
            "call_ms": call_ms, "split_median_ms": split_median_ms, "dispatch_ms": dispatch_ms,
            "dispatch_launches": launches.value, "eager_two_calls_ms": eager_two_calls_ms}


def prefill_write(steps: int):
    """Bulk quantized append at the cfg5 prefill size: every layer writes
    T = 64 sequences x 1024 prompt tokens = 65,536 tokens of 4 KV heads, D = 128,
    bf16 input, to shuffled slots (reference call site `model/attention.py:111-116`).
    Three rotating pools, their writes captured in one HIP graph; mean over
    `steps // 3` replays between two events."""
    import torch as t
    import oracle
    from aiproj_amd.inference.paged_kv_cache import PagedKVCache

    tokens, heads, dim = 64 * 1024, 4, 128
    num_blocks = tokens // 16 + 64
    gen = t.Generator(device="cuda").manual_seed(5)
    slots = t.randperm(num_blocks * 16, device="cuda", generator=gen)[:tokens]
    blocks, offsets = slots // 16, slots % 16
    pools = []
    for _ in range(3):
        cache = PagedKVCache(num_blocks, 16, heads, dim, "cuda", t.float8_e4m3fn)
        k = t.randn(tokens, heads, dim, device="cuda", dtype=t.bfloat16, generator=gen)
        v = t.randn(tokens, heads, dim, device="cuda", dtype=t.bfloat16, generator=gen)
        pools.append((cache, k, v))
    for i in range(6):
        cache, k, v = pools[i % 3]
        cache.append_kv(blocks, offsets, k, v)
    t.cuda.synchronize()
    # One graph holds the three pools' writes, so the timed launches follow each
    # other with no host time between them (a 40 us kernel is near Python's call cost).
    graph = t.cuda.CUDAGraph()
    with t.cuda.graph(graph):
        for cache, k, v in pools:
            cache.append_kv(blocks, offsets, k, v)
    graph.replay()
    t.cuda.synchronize()
    reps = max(1, steps // 3)
    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
    with _NoGC():
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        t.cuda.synchronize()
    us = start.elapsed_time(end) / (3 * reps) * 1e3
    del graph
    nbytes = oracle.append_algorithmic_bytes(tokens, heads, dim, in_bytes=2)
    gbs = nbytes / (us * 1e-6) / 1e9
    del pools
    t.cuda.empty_cache()
    log(f"[prefill write] T={tokens} Hkv={heads} D={dim}: {us:.1f} us ({gbs:.0f} GB/s)")
    return {
        "workload": f"cfg5 prefill layer write: {tokens} tokens x {heads} KV heads x D {dim}, bf16 in, shuffled slots",
        "kernel": "quantize_append_kernel",
        "us_per_call": round(us, 2),
        "algorithmic_bytes_per_call": nbytes,
        "achieved": round(gbs, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(gbs / PEAK_HBM_GBS, 4),
        "tokens_per_s": round(tokens / (us * 1e-6)),
    }


def prefill_attention(steps: int):
    """Varlen causal prefill attention at the cfg5 prefill size: 64 packed prompts of
    1024 tokens, 16 q / 4 KV heads, D = 128, bf16 (reference call site
    `model/attention.py:101-110`, kernel `kernals/flash_attention.py:51-211`). Three
    input sets rotate; `steps` back-to-back launches between two events. Roofline:
    matrix cores, algorithmic flops 4 D Hq sum_b L_b (L_b + 1) / 2 (QK^T and PV over
    the causal triangle)."""
    import torch as t
    from aiproj_amd.kernals.flash_attention import flash_attention_forward

    batch, length, hq, hkv, d = 64, 1024, 16, 4, 128
    total = batch * length
    gen = t.Generator(device="cuda").manual_seed(7)
    cu = t.arange(0, total + 1, length, device="cuda", dtype=t.int32)
    sets = []
    for _ in range(3):
        q = t.randn(total, hq, d, device="cuda", dtype=t.bfloat16, generator=gen)
        k = t.randn(total, hkv, d, device="cuda", dtype=t.bfloat16, generator=gen)
        v = t.randn(total, hkv, d, device="cuda", dtype=t.bfloat16, generator=gen)
        sets.append((q, k, v))
    scale = 1.0 / math.sqrt(d)
    for i in range(3):
        flash_attention_forward(*sets[i], cu, length, scale)
    t.cuda.synchronize()
    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
    with _NoGC():
        start.record()
        for i in range(steps):
            flash_attention_forward(*sets[i % 3], cu, length, scale)
        end.record()
        t.cuda.synchronize()
    us = start.elapsed_time(end) / steps * 1e3
    flops = 4 * d * hq * batch * length * (length + 1) // 2
    tflops = flops / (us * 1e-6) / 1e12
    del sets
    t.cuda.empty_cache()
    log(f"[prefill attention] {batch} x {length} tokens, {hq}q/{hkv}kv, D {d}, bf16: {us:.1f} us "
        f"({tflops:.0f} TFLOP/s)")
    return {
        "workload": f"cfg5 prefill attention: {batch} packed causal prompts x {length} tokens, {hq}q/{hkv}kv heads, "
                    f"D {d}, bf16",
        "kernel": "prefill_fa_kernel",
        "bound": "mfma",
        "us_per_call": round(us, 2),
        "algorithmic_flops_per_call": flops,
        "achieved": round(tflops, 1),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "tokens_per_s": round(total / (us * 1e-6)),
    }


def model_decode(steps: int):
    """Config 5: random-init decoder LM (16 layers, d 2048, 16q/4kv, D 128, SwiGLU
    5632, vocab 32000, bf16 weights ~ N(0, 0.02)); 64 random-id prompts of 1024
    tokens prefilled into the FP8 paged cache, then 128 greedy decode steps, the
    step captured once in a HIP graph. Reports the replayed decode step."""
    import torch as t
    from aiproj_amd.inference.greedy_decoder import GreedyDecoder
    from aiproj_amd.model.transformer import ModelConfig, TransformerLM

    cfg = ModelConfig()
    gen = t.Generator(device="cuda").manual_seed(6)
    model = TransformerLM(cfg).to(device="cuda", dtype=t.bfloat16).init_weights(gen).eval()
    batch, prompt, new = 64, 1024, 128
    prompts = t.randint(0, cfg.vocab_size, (batch, prompt), device="cuda", generator=gen)
    dec = GreedyDecoder(model, batch=batch, max_len=prompt + new)
    with t.inference_mode():
        t.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompts)
        t.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        dec.generate(2, use_graph=True)          # eager warm-up step, capture, one replay
        t.cuda.synchronize()
        start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        timed = min(steps, new - 2)
        with _NoGC():
            start.record()
            dec.generate(timed, use_graph=True)
            end.record()
            t.cuda.synchronize()
    ms = start.elapsed_time(end) / timed
    kv_bytes = cfg.num_layers * batch * (prompt + 64) * cfg.num_kv_heads * (2 * cfg.head_dim + 8)
    weight_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    log(f"[cfg5] decode step {ms * 1e3:.1f} us ({batch / (ms * 1e-3):.0f} tokens/s), prefill {prefill_s * 1e3:.0f} ms")
    out = {
        "workload": ("cfg5: 16-layer decoder LM, d 2048, 16q/4kv, D 128, SwiGLU 5632, vocab 32000, bf16 random "
                     "weights; 64 x 1024-token prompts in the FP8 paged cache; greedy decode, step replayed "
                     "from one HIP graph"),
        "decode_step_ms": round(ms, 4),
        "decode_tokens_per_s": round(batch / (ms * 1e-3), 1),
        "timed_steps": timed,
        "prefill_s": round(prefill_s, 3),
        "bytes_per_step": {"weights": weight_bytes, "kv_cache_mean": kv_bytes},
        "step_gbs": round((weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9, 1),
    }
    del dec, model
    t.cuda.empty_cache()
    return out


def _time_decode(caches, q, context, steps: int):
    """Mean µs of the split kernel alone and of the whole call (split + combine), each
    `steps` launches back to back between two HIP events, the caches rotating."""
    import torch as t
    from aiproj_amd.kernals.decode_attention import prepare_decode

    calls = [prepare_decode(q, cache, context) for cache in caches]
    for c in calls:
        c.run()
    t.cuda.synchronize()
    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
    out = []
    for phase in ("split", "run"):
        with _NoGC():
            start.record()
            for i in range(steps):
                getattr(calls[i % len(calls)], phase)()
            end.record()
            t.cuda.synchronize()
        out.append(start.elapsed_time(end) / steps * 1e3)
    return out


def _misaligned(cache):
    """The same cache with its K and V codes copied 4 bytes past a 16-byte boundary:
    the MFMA kernel needs 16-byte aligned caches, so decode takes the grouped VALU
    kernel (with its 4-byte loads) on identical bytes (scales and table unchanged)."""
    import types

    import torch as t

    def shifted(x):
        nbytes = x.numel() * x.element_size()
        raw = t.empty(nbytes + 16, dtype=t.uint8, device=x.device)
        view = raw[4:4 + nbytes].view(x.dtype).view(x.shape)
        view.view(t.uint8).copy_(x.view(t.uint8))
        return view

    return types.SimpleNamespace(k=shifted(cache.k), v=shifted(cache.v), k_scales=cache.k_scales,
                                 v_scales=cache.v_scales, quantized=cache.quantized, block_size=cache.block_size)


def kernel_legs(steps: int):
    """Decode kernels beside the FP8 MFMA path, each timed as `_time_decode` does with
    enough rotating pools to exceed twice the 256 MB last-level cache:
      * unquantized bf16 caches (the reference's default cache dtype and the control of
        its FP8 tests) at the north-star shape and cfg2, on the same MFMA kernel;
      * f16 (with f16 q, on the MFMA kernel) and f32 (grouped VALU kernel) caches at the
        north-star shape;
      * MFMA against the grouped VALU kernel on the same FP8 bytes (north, cfg4);
      * the grouped kernel at head size 80, a shape the MFMA kernel does not take."""
    import torch as t
    import oracle
    from aiproj_amd import workloads
    from aiproj_amd.inference.paged_kv_cache import PagedKVCache

    legs = {}

    def pools_for(w, dtype, spec):
        esize = t.empty((), dtype=dtype).element_size()
        per_token = spec.num_kv_heads * (2 * spec.head_dim * esize + (8 if dtype == t.float8_e4m3fn else 0))
        pool = w.num_blocks * spec.block_size * per_token
        count = max(2, math.ceil(2 * MALL_BYTES / pool) + 1)
        caches = []
        for _ in range(count):
            cache = PagedKVCache(w.num_blocks, spec.block_size, spec.num_kv_heads, spec.head_dim, "cuda", dtype)
            workloads.fill_cache(w, cache, "cuda")
            k, v = workloads.new_kv(w, "cuda")
            cache.append_kv(w.new_blocks, w.new_offsets, k, v)
            caches.append(cache)
        return caches

    def entry(spec, kv_bytes, split_us, call_us, kernel, q_bytes=2):
        nbytes = oracle.decode_algorithmic_bytes(spec.lengths, spec.num_q_heads, spec.num_kv_heads, spec.head_dim,
                                                 spec.block_size, q_bytes=q_bytes, out_bytes=q_bytes,
                                                 kv_bytes=kv_bytes)
        return {"kernel": kernel, "kv_tokens": spec.total_tokens, "algorithmic_bytes": nbytes,
                "split_us": round(split_us, 2), "split_frac": round(nbytes / (split_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                "call_us": round(call_us, 2), "call_frac": round(nbytes / (call_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}

    with t.inference_mode():
        for name in ("north", "cfg2"):
            spec = workloads.spec(name)
            w = workloads.build(spec, "cuda")
            caches = pools_for(w, t.bfloat16, spec)
            split_us, call_us = _time_decode(caches, w.q, workloads.make_context(w), steps)
            legs[f"bf16_cache_{name}"] = entry(spec, 2, split_us, call_us, "decode_mfma_kernel (bf16 cache)")
            log(f"[bf16 cache {name}] split {split_us:.1f} us, split + combine {call_us:.1f} us")
            del caches
            t.cuda.empty_cache()
        # The other unquantized cache dtypes the reference accepts: f16 read with f16 q
        # (an f16 model) on the MFMA kernel's f16 products, f32 on the grouped VALU kernel.
        spec = workloads.spec("north")
        w = workloads.build(spec, "cuda")
        for dtype, esize, tag, kernel in ((t.float16, 2, "f16", "decode_mfma_kernel (f16 cache, f16 q)"),
                                          (t.float32, 4, "f32", "decode_split_grouped + decode_combine (f32 cache)")):
            caches = pools_for(w, dtype, spec)
            q = w.q.to(dtype)
            split_us, call_us = _time_decode(caches, q, workloads.make_context(w), max(4, steps // 2))
            legs[f"{tag}_cache_north"] = entry(spec, esize, split_us, call_us, kernel, q_bytes=esize)
            log(f"[{tag} cache north] split {split_us:.1f} us, split + combine {call_us:.1f} us")
            del caches
            t.cuda.empty_cache()
        for name in ("north", "cfg4"):
            spec = workloads.spec(name)
            w = workloads.build(spec, "cuda")
            caches = pools_for(w, t.float8_e4m3fn, spec)
            ctx = workloads.make_context(w)
            mfma = _time_decode(caches, w.q, ctx, steps)
            shifted = [_misaligned(c) for c in caches]
            del caches
            t.cuda.empty_cache()
            grouped = _time_decode(shifted, w.q, ctx, max(4, steps // 4))
            legs[f"fp8_{name}_mfma"] = entry(spec, 1, *mfma, "decode_mfma_kernel + combine_mfma_kernel")
            legs[f"fp8_{name}_valu"] = entry(spec, 1, *grouped, "decode_split_grouped + decode_combine")
            log(f"[A/B {name}] MFMA split {mfma[0]:.1f} / call {mfma[1]:.1f} us; "
                f"VALU split {grouped[0]:.1f} / call {grouped[1]:.1f} us")
            del shifted
            t.cuda.empty_cache()
        spec = workloads.WorkloadSpec("d80", 32, 32, 8, 80, [4096] * 32, seed=2)
        w = workloads.build(spec, "cuda")
        caches = pools_for(w, t.float8_e4m3fn, spec)
        split_us, call_us = _time_decode(caches, w.q, workloads.make_context(w), max(4, steps // 4))
        legs["fp8_d80_valu"] = entry(spec, 1, split_us, call_us, "decode_split_grouped + decode_combine (D 80)")
        log(f"[grouped D80] split {split_us:.1f} us, split + combine {call_us:.1f} us")
        del caches
        t.cuda.empty_cache()
    return legs


def reference_sweep(iterations: int = 50, warmup: int = 10):
    """The reference's own decode benchmark (benchmarks/bench_kv_cache_fp8.py:38-158) on
    this library: batch sizes {1, 8, 32} x context lengths {512, 2048, 8192}, 8 q / 4 KV
    heads, D 64, page 16, one bf16 and one FP8 cache holding the same seeded K/V
    history, q bf16. Each point times `iterations` eager `decode_attention_wrapper` calls
    between two events after `warmup` calls, as the reference does (no pool rotation;
    the smaller working sets stay in the 256 MB last-level cache, as in the reference's
    own runs). Per dtype, a least-squares fit of time = overhead + kv_bytes / bandwidth
    over the nine points, and the fp8-over-bf16 speedup per point."""
    import torch as t
    from aiproj_amd.inference.page_allocator import PageAllocator
    from aiproj_amd.inference.paged_kv_cache import PagedKVCache
    from aiproj_amd.kernals.decode_attention import decode_attention_wrapper

    fp8 = t.float8_e4m3fn
    hq, hkv, dim, bs = 8, 4, 64, 16
    gen = t.Generator(device="cuda").manual_seed(11)

    def per_token(cache):
        per_vector = dim * cache.k.element_size() + (cache.k_scales.element_size() if cache.quantized else 0)
        return 2 * hkv * per_vector

    rows = []
    with t.inference_mode():
        for batch in (1, 8, 32):
            for ctx in (512, 2048, 8192):
                num_blocks = batch * (-(-ctx // bs)) + 1
                manager = PageAllocator(num_blocks, bs, batch + 1, ctx + bs, "cuda")
                caches = {d: PagedKVCache(num_blocks, bs, hkv, dim, "cuda", d) for d in (t.bfloat16, fp8)}
                slots = []
                for rid in range(batch):
                    slots.append(manager.allocate_request(rid, ctx))
                    k = t.randn(ctx, hkv, dim, device="cuda", dtype=t.bfloat16, generator=gen)
                    v = t.randn(ctx, hkv, dim, device="cuda", dtype=t.bfloat16, generator=gen)
                    for cache in caches.values():
                        manager.append_request(rid, t.arange(ctx, device="cuda"), k, v, cache)
                    manager.advance(rid, ctx - 1)
                context = manager.create_container(t.tensor(slots, device="cuda"),
                                                   t.arange(batch + 1, dtype=t.int32, device="cuda"),
                                                   t.full((batch,), ctx - 1, device="cuda"))
                q = t.randn(batch, hq, dim, device="cuda", dtype=t.bfloat16, generator=gen)
                for dtype, cache in caches.items():
                    for _ in range(warmup):
                        decode_attention_wrapper(q, cache, context)
                    t.cuda.synchronize()
                    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
                    with _NoGC():
                        start.record()
                        for _ in range(iterations):
                            decode_attention_wrapper(q, cache, context)
                        end.record()
                        t.cuda.synchronize()
                    ms = start.elapsed_time(end) / iterations
                    rows.append(("fp8" if dtype == fp8 else "bf16", batch, ctx, batch * ctx * per_token(cache), ms))
                del caches, context, q, manager
                t.cuda.empty_cache()
    fits = {}
    for name in ("bf16", "fp8"):
        pts = [(kv, ms * 1e-3) for d, _, _, kv, ms in rows if d == name]
        design = t.tensor([[1.0, float(kv)] for kv, _ in pts], dtype=t.float64)
        seconds = t.tensor([[sec] for _, sec in pts], dtype=t.float64)
        overhead, slope = t.linalg.lstsq(design, seconds).solution.flatten().tolist()
        fits[name] = {"overhead_us": round(overhead * 1e6, 2),
                      "bandwidth_gbs": round(1.0 / slope / 1e9, 1) if slope > 0 else None}
    timing = {(d, b, c): ms for d, b, c, _, ms in rows}
    points = [{"dtype": d, "batch": b, "context": c, "kv_mb": round(kv / 2 ** 20, 2), "us_per_call": round(ms * 1e3, 2),
               "gbs": round(kv / (ms * 1e-3) / 1e9, 1)} for d, b, c, kv, ms in rows]
    speedup = [{"batch": b, "context": c, "fp8_speedup": round(timing[("bf16", b, c)] / timing[("fp8", b, c)], 3)}
               for b in (1, 8, 32) for c in (512, 2048, 8192)]
    for name, f in fits.items():
        log(f"[sweep] {name}: time = {f['overhead_us']:.1f} us + kv_bytes / {f['bandwidth_gbs']} GB/s")
    return {"workload": "reference decode sweep: batch {1, 8, 32} x context {512, 2048, 8192}, 8q/4kv, D 64, "
                        "page 16, eager decode_attention_wrapper calls (benchmarks/bench_kv_cache_fp8.py defaults)",
            "fit": fits, "points": points, "speedup": speedup}


def copy_bandwidth_gbs(nbytes: int = 2 * 2 ** 30) -> float:
    """Device-to-device copy of nbytes (read + write), the practical HBM roofline."""
    import torch as t

    src = t.empty(nbytes, dtype=t.uint8, device="cuda")
    dst = t.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    t.cuda.synchronize()
    start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        dst.copy_(src)
    end.record()
    t.cuda.synchronize()
    ms = start.elapsed_time(end) / 10
    del src, dst
    t.cuda.empty_cache()
    return 2 * nbytes / (ms * 1e-3) / 1e9


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_threads() -> int:
    """Host threads for the CPU baseline: every core this process may run on, capped
    by OMP_NUM_THREADS when the environment sets it (the GPU box's CPU share)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(setup: Setup, budget_s: float):
    """The reference's CPU path on the host cores, on host copies of the same inputs:
    the quantize-and-scatter of the new tokens (torch amax, float32 division, clamp,
    cast to float8_e4m3fn, indexed store: reference tests/test_kv_cache_quantization.py:60-66)
    and, per sequence, the gather through the block table, fp32 dequantize and GQA
    attention (`:428-446`), in torch float32 with every host thread. A bounded sample
    of the step's sequences keeps the leg to about `budget_s` seconds."""
    import torch as t

    threads = cpu_threads()
    saved = t.get_num_threads()
    t.set_num_threads(threads)
    s = setup.spec
    fp8 = t.float8_e4m3fn
    fp8_max = t.finfo(fp8).max
    cache = setup.caches[0]
    k_codes, v_codes = cache.k.cpu(), cache.v.cpu()
    k_scales, v_scales = cache.k_scales.cpu(), cache.v_scales.cpu()
    table = setup.w.block_table.cpu().long()
    q = setup.w.q.cpu().float()
    new_k, new_v = (x.cpu() for x in setup.new_tokens[0])
    new_blocks, new_offsets = setup.w.new_blocks.cpu(), setup.w.new_offsets.cpu()
    group = s.num_q_heads // s.num_kv_heads
    scale = 1.0 / math.sqrt(s.head_dim)

    def quantize(x):
        x32 = x.float()
        amax = x32.abs().amax(dim=-1)
        sc = t.where(amax > 0, amax / fp8_max, t.ones_like(amax))
        return (x32 / sc.unsqueeze(-1)).clamp(-fp8_max, fp8_max).to(fp8), sc

    def step(n):
        kc, ks = quantize(new_k[:n])
        vc, vs = quantize(new_v[:n])
        k_codes[new_blocks[:n], new_offsets[:n]] = kc
        v_codes[new_blocks[:n], new_offsets[:n]] = vc
        k_scales[new_blocks[:n], new_offsets[:n]] = ks
        v_scales[new_blocks[:n], new_offsets[:n]] = vs
        out = t.empty(n, s.num_q_heads, s.head_dim)
        for b in range(n):
            pos = t.arange(s.lengths[b])
            pages, offs = table[b, pos // s.block_size], pos % s.block_size
            k = k_codes[pages, offs].float() * k_scales[pages, offs].unsqueeze(-1)      # [L, Hkv, D]
            v = v_codes[pages, offs].float() * v_scales[pages, offs].unsqueeze(-1)
            qg = q[b].view(s.num_kv_heads, group, s.head_dim)
            scores = t.matmul(qg, k.permute(1, 2, 0).contiguous()) * scale            # [Hkv, G, L]
            probs = scores.softmax(dim=-1)
            out[b] = t.matmul(probs, v.permute(1, 0, 2).contiguous()).reshape(s.num_q_heads, s.head_dim)
        return out

    t0 = time.perf_counter()
    step(1)
    per_seq = max(time.perf_counter() - t0, 1e-4)
    n = int(max(1, min(s.batch, budget_s / 4 / per_seq)))
    step(n)                                                    # warm rep
    times = []
    while len(times) < 3 or (sum(times) < budget_s / 2 and len(times) < 50):
        t0 = time.perf_counter()
        step(n)
        times.append(time.perf_counter() - t0)
    t.set_num_threads(saved)
    sec = float(sorted(times)[len(times) // 2])
    import oracle      # the byte counter only
    nbytes = (oracle.decode_algorithmic_bytes(s.lengths[:n], s.num_q_heads, s.num_kv_heads, s.head_dim,
                                              s.block_size)
              + oracle.append_algorithmic_bytes(n, s.num_kv_heads, s.head_dim))
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"torch float32 on the host: quantize-and-scatter of {n} new tokens, then gather, dequantize and "
                   f"GQA attention for {n} of {s.batch} sequences of the {s.name} step "
                   f"({sum(s.lengths[:n])} KV tokens); median of {len(times)} timed reps after one warm rep, "
                   f"{sec:.3f} s each"),
        "kv_tokens_per_s": round(sum(s.lengths[:n]) / sec, 1),
        "torch_num_threads": threads,
        "host_cpu_count": os.cpu_count(),
        "host_cpu": _cpu_model(),
    }


def traffic_for(kernel: str, workload: str):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3 FETCH_SIZE +
    WRITE_SIZE summary of this workload (calibrated against a 2 GiB copy), or None."""
    path = ROOT / "profiles" / f"{kernel}_{workload}_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def measure(name: str, steps: int, warmup: int):
    import torch as t

    setup = Setup(name, "cuda")
    times = time_steps(setup, steps, warmup)
    ms, eager_ms, kernel_ms = times["graph_ms"], times["eager_ms"], times["split_ms"]
    s = setup.spec
    result = {
        "setup": setup,
        "ms_per_step": ms,
        "separate_ms_per_step": times["separate_ms"],
        "eager_ms_per_step": eager_ms,
        "eager_two_calls_ms_per_step": times["eager_two_calls_ms"],
        "split_kernel_ms": kernel_ms,
        "call_ms": times["call_ms"],
        "call_gbs": setup.decode_bytes / (times["call_ms"] * 1e-3) / 1e9,
        "split_median_ms": times["split_median_ms"],
        "dispatch_kernel_ms": times["dispatch_ms"],
        "dispatch_launches": times["dispatch_launches"],
        "step_bytes": setup.decode_bytes + setup.append_bytes,
        "gbs": (setup.decode_bytes + setup.append_bytes) / (ms * 1e-3) / 1e9,
        "kernel_gbs": setup.decode_bytes / (kernel_ms * 1e-3) / 1e9,
        "kv_tokens_per_s": s.total_tokens / (ms * 1e-3),
        "pools": setup.num_pools,
        "pool_mb": setup.pool_bytes / 1e6,
    }
    log(f"[{name}] B={s.batch} Hq={s.num_q_heads} Hkv={s.num_kv_heads} D={s.head_dim} tokens={s.total_tokens} "
        f"pools={setup.num_pools}x{setup.pool_bytes / 1e6:.0f}MB: {ms * 1e3:.1f} us/step (graph; "
        f"{times['separate_ms'] * 1e3:.1f} as two calls), "
        f"{eager_ms * 1e3:.1f} us/step (eager; {times['eager_two_calls_ms'] * 1e3:.1f} as two calls), decode kernel {kernel_ms * 1e3:.1f} us back to back "
        f"({result['kernel_gbs']:.0f} GB/s), split + combine {times['call_ms'] * 1e3:.1f} us "
        f"({result['call_gbs']:.0f} GB/s), {times['dispatch_ms'] * 1e3:.1f} us per-dispatch events, "
        f"step {result['gbs']:.0f} GB/s")
    t.cuda.synchronize()
    return result


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch as t

    if not t.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from aiproj_amd import _native

    _native.lib()
    log(f"device {t.cuda.get_device_name()} torch {t.__version__} lib {_native.lib().kvfp8_version().decode()}")

    if args.workload == "cfg5":
        print(json.dumps({"workload": "cfg5", "model_decode": model_decode(args.steps)}), flush=True)
        return
    if args.workload == "kernels":
        print(json.dumps({"workload": "kernels", "decode_kernels": kernel_legs(args.steps)}), flush=True)
        return
    if args.workload == "prefill":
        print(json.dumps({"workload": "prefill", "prefill_write": prefill_write(args.steps),
                          "prefill_attention": prefill_attention(args.steps)}), flush=True)
        return

    copy_gbs = copy_bandwidth_gbs()
    log(f"device copy bandwidth: {copy_gbs:.0f} GB/s")

    main_result = measure(args.workload, args.steps, args.warmup)
    secondary = None
    if args.secondary and args.secondary != args.workload:
        r = measure(args.secondary, max(10, args.steps // 2), max(3, args.warmup // 2))
        secondary = {
            "workload": args.secondary,
            "lengths": "U[512, 4096] seeded draw" if args.secondary == "cfg2" else "see aiproj_amd/workloads.py",
            "value": round(r["gbs"], 1),
            "unit": "GB/s",
            "pct_of_peak": round(100 * r["gbs"] / PEAK_HBM_GBS, 2),
            "kv_tokens_per_s": round(r["kv_tokens_per_s"]),
            "ms_per_step": round(r["ms_per_step"], 5),
            "separate_ms_per_step": round(r["separate_ms_per_step"], 5),
            "eager_ms_per_step": round(r["eager_ms_per_step"], 5),
            "eager_two_calls_ms_per_step": round(r["eager_two_calls_ms_per_step"], 5),
            "decode_kernel_us": round(r["split_kernel_ms"] * 1e3, 2),
            "decode_kernel_gbs": round(r["kernel_gbs"], 1),
            "decode_kernel_frac": round(r["kernel_gbs"] / PEAK_HBM_GBS, 4),
            "decode_call_us": round(r["call_ms"] * 1e3, 2),
            "decode_call_frac": round(r["call_gbs"] / PEAK_HBM_GBS, 4),
        }
        del r

    s = main_result["setup"].spec
    cpu = None if args.no_cpu else cpu_baseline(main_result["setup"], args.cpu_seconds)
    others = {}
    if not args.no_others:
        for name in ("cfg1", "cfg3", "cfg4"):
            if name == args.workload:
                continue
            r = measure(name, max(10, args.steps // 2), max(3, args.warmup // 2))
            spec = r["setup"].spec
            others[name] = {
                "batch": spec.batch, "heads": f"{spec.num_q_heads}q/{spec.num_kv_heads}kv", "head_dim": spec.head_dim,
                "kv_tokens": spec.total_tokens,
                "step_us": round(r["ms_per_step"] * 1e3, 2),
                "separate_step_us": round(r["separate_ms_per_step"] * 1e3, 2),
                "step_gbs": round(r["gbs"], 1),
                "decode_kernel_us": round(r["split_kernel_ms"] * 1e3, 2),
                "decode_kernel_gbs": round(r["kernel_gbs"], 1),
                "decode_kernel_frac": round(r["kernel_gbs"] / PEAK_HBM_GBS, 4),
                "decode_call_us": round(r["call_ms"] * 1e3, 2),
                "decode_call_frac": round(r["call_gbs"] / PEAK_HBM_GBS, 4),
                "kv_tokens_per_s": round(r["kv_tokens_per_s"]),
            }
            del r
    prefill = None if args.no_prefill else prefill_write(max(10, args.steps // 2))
    if prefill is not None:
        # Mixed read + write traffic: the device copy is its practical ceiling.
        prefill["pct_of_copy"] = round(100 * prefill["achieved"] / copy_gbs, 2)
    prefill_attn = None if args.no_prefill else prefill_attention(max(10, args.steps // 2))
    kernels = None if args.no_kernels else kernel_legs(max(10, args.steps // 2))
    model = None if args.no_model else model_decode(100)
    sweep = None if args.no_sweep else reference_sweep()
    kernel_gbs = main_result["kernel_gbs"]
    line = {
        "metric": METRIC,
        "value": round(main_result["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_result["ms_per_step"], 5),
        "separate_ms_per_step": round(main_result["separate_ms_per_step"], 5),
        "eager_ms_per_step": round(main_result["eager_ms_per_step"], 5),
        "eager_two_calls_ms_per_step": round(main_result["eager_two_calls_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn",
        "data": "synthetic (seeded N(0,1) bf16 K/V quantized to e4m3fn, bf16 q)",
        "config": {
            "workload": (f"{s.name}: B={s.batch}, {s.num_q_heads}q/{s.num_kv_heads}kv heads, D={s.head_dim}, "
                         f"page {s.block_size}, contexts {min(s.lengths)}..{max(s.lengths)} "
                         f"(total {s.total_tokens} KV tokens), FP8 e4m3fn paged cache with per-(page slot, "
                         f"kv head) scales, shuffled page pool; step = 1-token quantized append + decode, "
                         f"the append done by the decode kernel (kvfp8_append_paged_decode)"),
            "timing": (f"steps replayed from HIP graphs of {LAYERS_PER_GRAPH} steps, the decode step of a "
                       f"{LAYERS_PER_GRAPH}-layer model (Llama-3-8B) with one attention step per layer, the layers "
                       f"cycling through {main_result['pools']} cache pools (together over twice the 256 MB "
                       "last-level cache); separate_ms_per_step: the same step as the two calls append_kv + decode; "
                       "eager_ms_per_step: the fused step launched eagerly, no graph; eager_two_calls_ms_per_step: "
                       "the reference runtime's own pattern (model/attention.py:88-99), the two calls launched "
                       "eagerly with no graph"),
            "pools_rotated": main_result["pools"],
            "pool_mb": round(main_result["pool_mb"], 1),
        },
        "pct_of_peak": round(100 * main_result["gbs"] / PEAK_HBM_GBS, 2),
        "kv_tokens_per_s": round(main_result["kv_tokens_per_s"]),
        "copy_gbs": round(copy_gbs, 1),
        "pct_of_copy": round(100 * main_result["gbs"] / copy_gbs, 2),
        "roofline": {
            "kernel": "decode_mfma_kernel",
            "bound": "hbm",
            "achieved": round(kernel_gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic_for("decode_mfma_kernel", s.name),
            "algorithmic_bytes_per_launch": main_result["setup"].decode_bytes,
            "mean_launch_us": round(main_result["split_kernel_ms"] * 1e3, 2),
            "timing": (f"{args.steps} back-to-back launches of the decode kernel alone "
                       "(kvfp8_paged_decode_split, pools rotating) between two HIP events on its stream"),
            "decode_call": {
                "what": ("decode attention as the reference defines it (decode_attention.py:146-189): the split "
                         "kernel and the combine kernel, kvfp8_paged_decode, same launches back to back"),
                "us": round(main_result["call_ms"] * 1e3, 2),
                "achieved": round(main_result["call_gbs"], 1),
                "frac": round(main_result["call_gbs"] / PEAK_HBM_GBS, 4),
            },
            "fused_dispatch_event_us": round(main_result["dispatch_kernel_ms"] * 1e3, 2),
            "median_launch_us": round(main_result["split_median_ms"] * 1e3, 2),
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
        "other_workloads": others,
        "prefill_write": prefill,
        "prefill_attention": prefill_attn,
        "decode_kernels": kernels,
        "model_decode": model,
        "reference_sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
