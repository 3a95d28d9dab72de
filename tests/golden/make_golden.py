"""Write the committed golden fixtures for the FP8 paged KV-cache path.

Expected values come from the torch library routines the reference's test oracle
calls (`tests/test_kv_cache_quantization.py:60-66`: amax, float32 division, clamp,
`.to(float8_e4m3fn)`; `:428-446`: float64 gather, dequantize, GQA softmax attention),
run on the CPU; nothing from the reference repository is imported or executed.
The numpy oracle in `oracle/` and the HIP kernels are both checked against these
files. Run from the repository root:

    python tests/golden/make_golden.py

Fixtures:
  quantize_cases.npz  - rows of the reference test shapes and edge cases with their
                        expected e4m3fn codes (uint8) and float32 scales.
  cfg1_decode.npz     - the cfg1 decode step (B=4, 8q/2kv, D=64, page 16,
                        L ~ U[64, 256], shuffled pool): inputs, expected cache bytes
                        and scales, expected float64 attention output.
  MANIFEST.sha256     - SHA-256 of each fixture.
"""

from __future__ import annotations

import hashlib
import math
import sys
from pathlib import Path

import numpy as np
import torch as t

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from aiproj_amd import workloads  # noqa: E402

FP8 = t.float8_e4m3fn
FP8_MAX = t.finfo(FP8).max


def torch_quantize(x: t.Tensor):
    x32 = x.float()
    amax = x32.abs().amax(dim=-1)
    scales = t.where(amax > 0, amax / FP8_MAX, t.ones_like(amax))
    codes = (x32 / scales.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return codes.view(t.uint8), scales


def torch_decode(q, k, v):
    """float64 GQA decode for one row: q [Hq, D]; k, v [L, Hkv, D]."""
    group = q.shape[0] // k.shape[1]
    kh = k.transpose(0, 1).repeat_interleave(group, 0)
    vh = v.transpose(0, 1).repeat_interleave(group, 0)
    scores = (q.double().unsqueeze(1) @ kh.transpose(-1, -2)).squeeze(1) / math.sqrt(q.shape[-1])
    return (scores.softmax(-1).unsqueeze(1) @ vh).squeeze(1)


def quantize_cases() -> dict[str, np.ndarray]:
    cases = {}

    def add(name, x):
        codes, scales = torch_quantize(x)
        cases[f"{name}__x"] = x.float().numpy()
        cases[f"{name}__dtype"] = np.array(str(x.dtype))
        cases[f"{name}__codes"] = codes.numpy()
        cases[f"{name}__scales"] = scales.numpy()

    # The append test shapes of reference tests/test_kv_cache_quantization.py:269-285.
    for dtype in (t.float32, t.float16, t.bfloat16):
        for d in (16, 80, 128):
            g = t.Generator().manual_seed(2)
            add(f"append_{str(dtype)[6:]}_{d}", (t.randn(100, 4, d, generator=g) * 3).to(dtype))
    # Magnitudes of the round-trip test (:95-107), outliers (:123-131), extremes (:134-142, :332-349).
    g = t.Generator().manual_seed(0)
    for mag in (1e-3, 1.0, 1e3):
        add(f"magnitude_{mag:g}", (t.randn(64, 4, 128, generator=g) * mag).to(t.bfloat16))
    x = t.randn(32, 2, 64, generator=g)
    x[..., 7] *= 1000
    add("outlier", x)
    for peak, dtype in ((1e30, t.float32), (1e-30, t.float32), (65504.0, t.float16), (1e30, t.bfloat16)):
        y = t.randn(40, 2, 64, generator=g, dtype=t.float64)
        add(f"peak_{peak:g}_{str(dtype)[6:]}", (y / y.abs().amax(-1, keepdim=True) * peak).to(dtype))
    add("zeros", t.zeros(5, 2, 16))
    add("known_answer", t.tensor([[0.1, -3.0, 2.0, 0.5]]))
    # Rows whose quotients land on e4m3 rounding ties and in the subnormal range.
    ties = t.tensor([[448.0, 1.0625, 1.1875, 2 ** -9 * 1.5, 2 ** -9 * 2.5, -2 ** -10, 3 * 2 ** -11, 0.0]])
    add("ties", ties)
    return cases


def cfg1_decode() -> dict[str, np.ndarray]:
    spec = workloads.spec("cfg1")
    w = workloads.build(spec, "cpu")
    hist_k, hist_v = workloads.history_kv(w, "cpu")
    new_k, new_v = workloads.new_kv(w, "cpu")
    blocks = t.cat([w.history_blocks, w.new_blocks])
    offsets = t.cat([w.history_offsets, w.new_offsets])
    ks = t.cat([hist_k, new_k])
    vs = t.cat([hist_v, new_v])

    k_codes, k_scales = torch_quantize(ks)
    v_codes, v_scales = torch_quantize(vs)

    nb, bs, hkv, d = w.num_blocks, spec.block_size, spec.num_kv_heads, spec.head_dim
    k_cache = t.zeros(nb, bs, hkv, d, dtype=t.uint8)
    v_cache = t.zeros_like(k_cache)
    ksc = t.ones(nb, bs, hkv)
    vsc = t.ones(nb, bs, hkv)
    k_cache[blocks, offsets] = k_codes
    v_cache[blocks, offsets] = v_codes
    ksc[blocks, offsets] = k_scales
    vsc[blocks, offsets] = v_scales

    out = []
    for b, length in enumerate(spec.lengths):
        pos = t.arange(length)
        pb = w.block_table[b, pos // bs].long()
        po = pos % bs
        k = k_cache[pb, po].view(FP8).double() * ksc[pb, po].double().unsqueeze(-1)
        v = v_cache[pb, po].view(FP8).double() * vsc[pb, po].double().unsqueeze(-1)
        out.append(torch_decode(w.q[b], k, v))

    return {
        "lengths": np.array(spec.lengths, dtype=np.int32),
        "num_blocks": np.array(nb),
        "block_table": w.block_table.numpy(),
        "q_bf16_bits": w.q.view(t.int16).numpy(),
        "ks_bf16_bits": ks.view(t.int16).numpy(),
        "vs_bf16_bits": vs.view(t.int16).numpy(),
        "blocks": blocks.numpy(),
        "offsets": offsets.numpy(),
        "k_codes": k_codes.numpy(),
        "v_codes": v_codes.numpy(),
        "k_scales": k_scales.numpy(),
        "v_scales": v_scales.numpy(),
        "expected_out": t.stack(out).numpy(),
    }


def main() -> None:
    files = {"quantize_cases.npz": quantize_cases(), "cfg1_decode.npz": cfg1_decode()}
    lines = []
    for name, arrays in files.items():
        path = HERE / name
        np.savez_compressed(path, **arrays)
        lines.append(f"{hashlib.sha256(path.read_bytes()).hexdigest()}  {name}")
        print(f"wrote {path} ({path.stat().st_size} bytes)")
    (HERE / "MANIFEST.sha256").write_text("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
