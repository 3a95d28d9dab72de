"""Bindings of `libkvfp8.so`, the gfx950 HIP kernels behind the reference API.

The library is built in-tree by `aiproj_amd.build` (or `__graft_entry__.build()`).
Every entry point is bound through ctypes; the per-step ones (decode, fused append +
decode, the appends) also have fast-call bindings in the `_kvfp8_fast` extension,
which `fn()` prefers. There is no fallback to another implementation: if the library
is missing or fails to load, every entry point that needs it raises, so a GPU run can
never silently take another code path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libkvfp8.so"

# enum kvfp8_dtype in include/kvfp8.h
F32, F16, BF16, E4M3FN, I32, I64 = 0, 1, 2, 3, 4, 5

TORCH_TO_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.float8_e4m3fn: E4M3FN,
    torch.int32: I32,
    torch.int64: I64,
}

# Exported symbols and their C signatures (include/kvfp8.h).
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_DECODE_ARGS = [_P, _INT, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _INT, _P, _P, _I64, _I32, _P, _I64, _I64,
                _P, _INT, _P, _INT, ctypes.c_float, _P, _P, _I64, _P]
SIGNATURES = {
    "kvfp8_quantize_append": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _INT, _P, _INT,
                                     _I64, _I32, _I32, _I64, _I32, _P, _P, _P, _P, _P]),
    "kvfp8_store_append": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _INT, _P, _INT,
                                  _I64, _I32, _I32, _I64, _I32, _P, _P, _INT, _P]),
    "kvfp8_decode_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I64, _I32, _INT]),
    "kvfp8_paged_decode": (_INT, _DECODE_ARGS),
    "kvfp8_paged_decode_split": (_INT, _DECODE_ARGS),
    "kvfp8_paged_decode_reduce": (_INT, _DECODE_ARGS),
    "kvfp8_paged_decode_noalloc": (_INT, _DECODE_ARGS[:-3] + [_P]),
    "kvfp8_append_paged_decode": (_INT, _DECODE_ARGS + [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _INT, _P, _INT, _P]),
    "kvfp8_append_decode_supported": (_INT, [_I32, _I32, _I32, _I32, _I64, _I64, _I32, _INT]),
    "kvfp8_rmsnorm_forward": (_INT, [_P, _INT, _I64, _I64, _I32, _P, _INT, ctypes.c_float, _P, _I64, _P, _P]),
    "kvfp8_add_rmsnorm_forward": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I32, _P, _INT, ctypes.c_float,
                                         _P, _I64, _P, _I64, _P, _P]),
    "kvfp8_rope_inplace": (_INT, [_P, _INT, _I64, _I32, _I32, _I64, _I64, _P, _INT, _P, _P, _INT, _I64, _P]),
    "kvfp8_silu_mul": (_INT, [_P, _INT, _I64, _I32, _I64, _P, _I64, _P]),
    "kvfp8_prefill_attention": (_INT, [_P, _P, _P, _INT, _I64, _I32, _I32, _I32, _P, _INT, _I32, _I32,
                                       ctypes.c_float, _P, _P, _P]),
    "kvfp8_timing_enable": (_INT, [_I32]),
    "kvfp8_timing_read": (_INT, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]),
    "kvfp8_strerror": (ctypes.c_char_p, [_INT]),
    "kvfp8_version": (ctypes.c_char_p, []),
    "kvfp8_host_encode_e4m3fn": (None, [_P, _P, _I64]),
    "kvfp8_host_quantize_rows": (None, [_P, _I64, _I32, _P, _P]),
    "kvfp8_host_row_quotients": (None, [_P, _I64, _I32, _P]),
    "kvfp8_selftest_fp8_encoder": (_INT, [_P, _P]),
}

_lock = threading.Lock()
_lib = None


class NativeLibraryError(RuntimeError):
    """libkvfp8.so is missing or unusable."""


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises NativeLibraryError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise NativeLibraryError(
                    f"{LIBRARY_PATH} is not built; run `python -m aiproj_amd.build` "
                    "(the FP8 KV-cache path has no non-HIP implementation)"
                )
            handle = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


_fast_fns: dict = {}


def _fast_module():
    """The fast-call extension (csrc/pyfast.c, linked to the in-tree libkvfp8.so), or
    None when it is not built or LIBRARY_PATH points at another library (it would
    still call the in-tree one)."""
    if LIBRARY_PATH != Path(__file__).resolve().parent / "libkvfp8.so":
        return None
    lib()     # load (and check) the library first; the extension shares it
    try:
        from aiproj_amd import _kvfp8_fast
    except ImportError:
        return None
    return _kvfp8_fast


def fn(name: str):
    """The callable for C-ABI entry point `name`: the fast-call binding where the
    extension provides it, else the ctypes function. Both take the arguments of
    include/kvfp8.h in order (ints, None for a null pointer, floats) and return the
    C return code."""
    f = _fast_fns.get(name)
    if f is None:
        mod = _fast_module()
        f = getattr(mod, name, None) if mod is not None else None
        if f is None:
            f = getattr(lib(), name)
        _fast_fns[name] = f
    return f


def strerror(code: int) -> str:
    return lib().kvfp8_strerror(code).decode()


def check(code: int, what: str) -> None:
    """Map a C-ABI return code to the reference's exception types."""
    if code == 0:
        return
    if code < 0:
        raise ValueError(f"{what}: {strerror(code)} (code {code})")
    raise RuntimeError(f"{what}: HIP error {code}: {strerror(code)}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return TORCH_TO_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(tensor) -> int | None:
    return None if tensor is None else tensor.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The current HIP stream of `device`, as the raw handle the C ABI takes. Read
    straight from torch's stream state when it offers that (no Python stream object
    per call, which costs about 2.5 µs), else through torch.cuda.current_stream."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors, what: str) -> torch.device:
    """All tensors on one GPU device; the FP8 path has no CPU implementation. The common
    case compares device indices (get_device: -1 on the CPU) without building device
    objects; any mismatch takes the descriptive path."""
    first = None
    index = None
    for x in tensors:
        if x is None:
            continue
        i = x.get_device()
        if first is None:
            first, index = x, i
        elif i != index or (i < 0 and x.device != first.device):
            index = None
            break
    if first is not None and index is not None and index >= 0 and first.is_cuda:
        return first.device
    devices = {x.device for x in tensors if x is not None}
    if len(devices) != 1:
        raise ValueError(f"{what}: tensors span devices {sorted(map(str, devices))}")
    device = devices.pop()
    if device.type != "cuda":
        raise RuntimeError(
            f"{what}: tensors are on {device}; the FP8 KV-cache kernels run on the GPU only "
            "(like the reference, there is no CPU FP8 path)"
        )
    return device
