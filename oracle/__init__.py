"""CPU oracle for the FP8 paged KV-cache path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`aiproj_amd`) imports
this package; only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s
`cpu_baseline` leg use it, and only as the checker or the timed CPU baseline.

The oracle restates, in numpy, the reference's own test oracle:
  * `quantize`        - reference `tests/test_kv_cache_quantization.py:60-66`
  * `dequantize`      - reference `tests/test_kv_cache_quantization.py:69-70`
  * `paged_history`   - reference `tests/test_kv_cache_quantization.py:428-437`
  * `decode_one`      - reference `tests/test_kv_cache_quantization.py:440-446`
  * `paged_decode`    - the per-row stack at `tests/test_kv_cache_quantization.py:475-478`
  * `scatter_append`  - address math of `kernals/kv_cache/quantized_append.py:103-105`
  * `causal_varlen_attention` - the ragged reference of `tests/test_flash_attention.py:44-85`
    and the lse of `kernals/flash_attention.py:205-210`
and the page-table gather of `inference/page_allocator.py:225-245`.
"""

from .kvfp8 import (  # noqa: F401
    FP8_MAX,
    E4M3_TABLE,
    f32_to_e4m3fn,
    e4m3fn_to_f32,
    quantize,
    dequantize,
    scatter_append,
    physical_location,
    paged_history,
    decode_one,
    paged_decode,
    causal_varlen_attention,
    decode_algorithmic_bytes,
    append_algorithmic_bytes,
)
