"""HIP varlen causal prefill attention vs the oracle (GPU).

Mirrors reference tests/test_flash_attention.py (the ragged batch [3, 73, 141], 8q/2kv,
D 16, float32, forward and backward against the PyTorch ragged reference at 1e-2) and
adds: the float64 oracle over dtypes, head sizes, GQA groups and lengths that cross the
kernel's 32-row and 64-key blocks; lse; rows outside every sequence and past
max_seq_len left unwritten; the config-5 prefill shape against float32 torch.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch as t

import oracle
from aiproj_amd import _native
from aiproj_amd.kernals.flash_attention import FlashAttentionFunction, flash_attention_forward

pytestmark = pytest.mark.gpu

LENGTHS = [1, 3, 31, 32, 33, 63, 64, 65, 129, 200]
TOLERANCE = {t.float32: 1e-4, t.float16: 2e-3, t.bfloat16: 1.6e-2}
LSE_TOLERANCE = 1e-3


def packed_inputs(lengths, hq, hkv, d, dtype, seed, index_dtype=t.int32):
    g = t.Generator(device="cuda").manual_seed(seed)
    total = sum(lengths)
    q = t.randn(total, hq, d, device="cuda", generator=g).to(dtype)
    k = t.randn(total, hkv, d, device="cuda", generator=g).to(dtype)
    v = t.randn(total, hkv, d, device="cuda", generator=g).to(dtype)
    cu = t.tensor([0] + list(np.cumsum(lengths)), dtype=index_dtype, device="cuda")
    return q, k, v, cu


def oracle_of(q, k, v, cu, max_len, scale):
    return oracle.causal_varlen_attention(q.double().cpu().numpy(), k.double().cpu().numpy(),
                                          v.double().cpu().numpy(), cu.cpu().numpy(), max_len, scale)


@t.inference_mode()
@pytest.mark.parametrize("dtype", [t.float32, t.float16, t.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 64, 80, 128])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (6, 2), (4, 2), (16, 2)])
def test_prefill_matches_oracle(dtype, head_dim, hq, hkv):
    q, k, v, cu = packed_inputs(LENGTHS, hq, hkv, head_dim, dtype, seed=31)
    scale = 1.0 / math.sqrt(head_dim)
    out, lse = flash_attention_forward(q, k, v, cu, max(LENGTHS), scale)
    assert out.dtype == dtype and out.shape == q.shape and lse.dtype == t.float32
    want, want_lse = oracle_of(q, k, v, cu, max(LENGTHS), scale)
    tol = TOLERANCE[dtype]
    t.testing.assert_close(out.double().cpu(), t.from_numpy(want), rtol=tol, atol=tol)
    t.testing.assert_close(lse.double().cpu(), t.from_numpy(want_lse), rtol=LSE_TOLERANCE, atol=LSE_TOLERANCE)


def test_reference_ragged_batch_forward_and_backward():
    """Reference tests/test_flash_attention.py:9-150, same shapes, dtype and tolerance."""
    lengths = [3, 73, 141]
    hq, hkv, d = 8, 2, 16
    q0, k0, v0, cu = packed_inputs(lengths, hq, hkv, d, t.float32, seed=32)
    scale = 1.0 / math.sqrt(d)
    q_ref, k_ref, v_ref = (x.detach().clone().requires_grad_(True) for x in (q0, k0, v0))
    q_hip, k_hip, v_hip = (x.detach().clone().contiguous().requires_grad_(True) for x in (q0, k0, v0))
    parts = []
    for b in range(len(lengths)):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        n = s1 - s0
        qb = q_ref[s0:s1].transpose(0, 1)
        kb = k_ref[s0:s1].transpose(0, 1).repeat_interleave(hq // hkv, 0)
        vb = v_ref[s0:s1].transpose(0, 1).repeat_interleave(hq // hkv, 0)
        scores = scale * (qb @ kb.transpose(-1, -2).contiguous())
        scores = scores.masked_fill(~t.tril(t.ones(n, n, dtype=t.bool, device="cuda")), float("-inf"))
        parts.append((t.softmax(scores, -1) @ vb).transpose(0, 1))
    reference = t.cat(parts, 0)
    actual = FlashAttentionFunction.apply(q_hip, k_hip, v_hip, cu, max(lengths))
    t.testing.assert_close(actual, reference, rtol=1e-2, atol=1e-2)
    grad = t.randn_like(reference)
    reference.backward(grad)
    actual.backward(grad)
    for got, want in ((q_hip.grad, q_ref.grad), (k_hip.grad, k_ref.grad), (v_hip.grad, v_ref.grad)):
        t.testing.assert_close(got, want, rtol=1e-2, atol=1e-2)


@t.inference_mode()
def test_unwritten_rows_truncation_and_int64_offsets():
    """Rows outside every sequence and rows past max_seq_len keep their old contents."""
    hq, hkv, d = 8, 2, 64
    total = 60
    g = t.Generator(device="cuda").manual_seed(33)
    q = t.randn(total, hq, d, device="cuda", generator=g).to(t.bfloat16)
    k = t.randn(total, hkv, d, device="cuda", generator=g).to(t.bfloat16)
    v = t.randn(total, hkv, d, device="cuda", generator=g).to(t.bfloat16)
    cu = t.tensor([2, 10, 10, 45], dtype=t.int64, device="cuda")     # tokens 0-1 and 45-59 belong to none
    max_len = 20                                                        # the last sequence has 35 tokens
    out = t.full_like(q, 7.0)
    lse = t.full((total, hq), -3.0, device="cuda")
    rc = _native.lib().kvfp8_prefill_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _native.BF16, total, hq, hkv, d, cu.data_ptr(), _native.I64,
        3, max_len, 1.0 / math.sqrt(d), out.data_ptr(), lse.data_ptr(), _native.stream_handle(q.device))
    _native.check(rc, "kvfp8_prefill_attention")
    t.cuda.synchronize()
    want, want_lse = oracle_of(q, k, v, cu, max_len, 1.0 / math.sqrt(d))
    written = ~np.isnan(want[:, 0, 0])
    assert written.sum() == 8 + 20
    got = out.double().cpu().numpy()
    np.testing.assert_allclose(got[written], want[written], rtol=1.6e-2, atol=1.6e-2)
    assert (got[~written] == 7.0).all()
    got_lse = lse.double().cpu().numpy()
    np.testing.assert_allclose(got_lse[written], want_lse[written], rtol=LSE_TOLERANCE, atol=LSE_TOLERANCE)
    assert (got_lse[~written] == -3.0).all()


@t.inference_mode()
@pytest.mark.parametrize("dtype,head_dim", [(t.bfloat16, 128), (t.float16, 64)])
def test_large_ragged_batch_over_persistent_workgroups(dtype, head_dim):
    """Many sequences: the 16-bit kernel's persistent workgroups walk several items each,
    its per-XCD unit ranges end in partial groups (152 units: 19 per XCD, in groups of
    8, 8 and 3), zero-length sequences and query blocks past a short sequence's end are
    skipped, and the longest sequence is cut at max_seq_len (its later rows stay
    unwritten)."""
    hq, hkv = 8, 2
    rng = np.random.default_rng(36)
    lengths = [int(x) for x in rng.integers(0, 300, size=74)] + [0, 900]
    lengths[5] = 0
    max_len = 640
    q, k, v, cu = packed_inputs(lengths, hq, hkv, head_dim, dtype, seed=36)
    total = q.shape[0]
    scale = 1.0 / math.sqrt(head_dim)
    out = t.full_like(q, 5.0)
    lse = t.full((total, hq), -2.0, device="cuda")
    rc = _native.lib().kvfp8_prefill_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _native.BF16 if dtype == t.bfloat16 else _native.F16, total,
        hq, hkv, head_dim, cu.data_ptr(), _native.I32, len(lengths), max_len, scale, out.data_ptr(), lse.data_ptr(),
        _native.stream_handle(q.device))
    _native.check(rc, "kvfp8_prefill_attention")
    t.cuda.synchronize()
    want, want_lse = oracle_of(q, k, v, cu, max_len, scale)
    written = ~np.isnan(want[:, 0, 0])
    assert written.sum() == sum(min(n, max_len) for n in lengths)
    got = out.double().cpu().numpy()
    tol = TOLERANCE[dtype]
    np.testing.assert_allclose(got[written], want[written], rtol=tol, atol=tol)
    assert (got[~written] == 5.0).all()
    got_lse = lse.double().cpu().numpy()
    np.testing.assert_allclose(got_lse[written], want_lse[written], rtol=LSE_TOLERANCE, atol=LSE_TOLERANCE)
    assert (got_lse[~written] == -2.0).all()


@t.inference_mode()
def test_config5_prefill_shape_against_float32_torch():
    """Config-5 prompts (1024 tokens, 16q/4kv, D 128, bf16), four sequences of the 64."""
    from tests.helpers import torch_prefill_attention

    lengths = [1024] * 4
    q, k, v, cu = packed_inputs(lengths, 16, 4, 128, t.bfloat16, seed=34)
    scale = 1.0 / math.sqrt(128)
    out, lse = flash_attention_forward(q, k, v, cu, 1024, scale)
    want = torch_prefill_attention(q, k, v, lengths).float()   # float32 math, contiguous operands
    t.testing.assert_close(out.float(), want, rtol=1.6e-2, atol=1.6e-2)
    qs = q[:1024].float().transpose(0, 1)
    ks = k[:1024].float().transpose(0, 1).repeat_interleave(4, 0)
    scores = scale * t.matmul(qs, ks.transpose(-1, -2).contiguous())
    scores = scores.masked_fill(t.ones(1024, 1024, dtype=t.bool, device="cuda").triu(1), float("-inf"))
    t.testing.assert_close(lse[:1024], t.logsumexp(scores, -1).transpose(0, 1), rtol=1e-3, atol=1e-3)


@t.inference_mode()
@pytest.mark.parametrize("dtype", [t.float32, t.float16, t.bfloat16])
@pytest.mark.parametrize("head_dim", [12, 20, 24, 96, 136, 192, 256, 300])
def test_prefill_head_sizes_the_reference_takes(dtype, head_dim):
    """Head sizes beyond the matrix-core kernels' (not a multiple of 8, or above 128)
    run on the vector-ALU kernel; 24 and 96 stay on the matrix cores. Against the
    float64 oracle over ragged lengths, with lse (reference kernals/flash_attention.py:72
    takes any head size)."""
    q, k, v, cu = packed_inputs(LENGTHS, 8, 2, head_dim, dtype, seed=36)
    scale = 1.0 / math.sqrt(head_dim)
    out, lse = flash_attention_forward(q, k, v, cu, max(LENGTHS), scale)
    want, want_lse = oracle_of(q, k, v, cu, max(LENGTHS), scale)
    tol = TOLERANCE[dtype]
    t.testing.assert_close(out.double().cpu(), t.from_numpy(want), rtol=tol, atol=tol)
    t.testing.assert_close(lse.double().cpu(), t.from_numpy(want_lse), rtol=LSE_TOLERANCE, atol=LSE_TOLERANCE)


@t.inference_mode()
def test_prefill_rejects_unsupported_shapes_and_handles_empty():
    q, k, v, cu = packed_inputs([5, 7], 4, 2, 520, t.bfloat16, seed=35)
    with pytest.raises(ValueError):
        flash_attention_forward(q, k, v, cu, 7, 0.3)                  # head size above 512
    q, k, v, cu = packed_inputs([5, 7], 4, 2, 16, t.bfloat16, seed=35)
    with pytest.raises(ValueError):
        flash_attention_forward(q, k.float(), v, cu, 7, 0.3)          # mixed dtypes
    out, lse = flash_attention_forward(q, k, v, cu, 0, 0.3)           # nothing to do
    assert out.shape == q.shape and lse.shape == (12, 4)
    empty = t.zeros(0, 4, 16, device="cuda", dtype=t.bfloat16)
    out, lse = flash_attention_forward(empty, empty[:, :2], empty[:, :2], t.zeros(1, dtype=t.int32, device="cuda"), 0, 0.3)
    assert out.shape == (0, 4, 16)
