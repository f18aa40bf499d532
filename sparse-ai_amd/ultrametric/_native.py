"""ctypes binding of libsparseattn.so (the C ABI declared in include/sparse_attn.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (both carry the SONAME libamdhip64.so.7); every launch is
issued on torch's current stream of the tensor's device. There is no CPU
fallback: when the library or a GPU is missing, the public functions raise.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "libsparseattn.so")
ABI_VERSION = 1

SA_OK, SA_EINVAL, SA_EUNSUPPORTED, SA_ELAUNCH = 0, -1, -2, -3
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int32: 3,
               torch.int64: 4, torch.uint8: 5, torch.bool: 5}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_I64P = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "sa_abi_version": (_I, []),
    "sa_last_error": (ctypes.c_char_p, []),
    "sa_build_block_lists": (_I, [_P, _I, _I64P, _I, _I, _I, _I, _P, _I, _I64, _I, _I, _I, _I, _P, _I, _P, _P]),
    "sa_build_block_lists_mask": (_I, [_P, _I64P, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P]),
    "sa_block_sparse_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                 _I64P, _I64P, _I64P, _I64P, _I64P, ctypes.c_float, _I, _I, _P]),
    "sa_routed_block_sparse_fwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I64P, _I, _P, _I, _I64, _I, _I, _P, _P,
                                        _I, _I, _I, _I, _I, _I, _I64P, _I64P, _I64P, _I64P, ctypes.c_float, _I,
                                        _I, _P]),
    "sa_decode_workspace_bytes": (ctypes.c_size_t, [_I, _I, _I, _I, _I]),
    "sa_sparse_paged_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                    _I, _I, _I, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                    _P, ctypes.c_size_t, _I, _P]),
    "sa_pack_page_codes": (_I, [_P, _I64P, _I, _I, _I, _I, _P, _P]),
    "sa_sparse_paged_decode_codes": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                          _I, _I, _I, _I, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                          _I64P, _P, ctypes.c_size_t, _I, _P]),
    "sa_sparse_paged_decode_seq_codes": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                              _I, _I, _I, _I, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                              _I64P, _P, ctypes.c_size_t, _I, _P]),
    "sa_route_block_vote": (_I, [_P, _I, _I64P, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "sa_block_sparse_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _I, _I64P, _P, _P, _P, _P,
                                 _P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _I64P, _I64P, _I64P, _I64P,
                                 _I64P, _I64P, _I64P, _I64P, ctypes.c_float, _I, _I, _P]),
    "sa_transpose_block_lists": (_I, [_P, _P, _I, _I, _I, _I, _P, _I, _P, _P]),
    "sa_ternary_pack": (_I, [_P, _I, _I64P, _I, _I, _I, _P, _P, _P]),
    "sa_ternary_prefill_fwd": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I,
                                    _I64P, _I64P, _I64P, _I64P, _I64P, _I64P, _P]),
    "sa_block_sparse_bwd_plan_bytes": (ctypes.c_size_t, [_I, _I, _I, _I, _I, _I]),
    "sa_block_sparse_bwd_plan": (_I, [_P, _P, _I, _P, _P, _I, _P, _I, _I64P, _I, _I, _I, _I, _I, _P,
                                      ctypes.c_size_t, _P, _P]),
    "sa_paged_kv_write": (_I, [_P, _P, _I64P, _I64P, _P, _I64P, _P, _I, _I, _I, _I, _I, _P, _P, _I64P, _I64P,
                               _P, _I64P, _P, _I, _I, _I, _P, _I, _I64P, _I, _P, _P]),
    "sa_paged_advance": (_I, [_P, _P, _I, _I, _P]),
    "sa_sparse_paged_decode_seq_codes_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                                      _I, _I, _I, _I, _I, _I64P, _I64P, _I64P, _I64P, _I64P, _I64P,
                                                      _I64P, _I, _P]),
    "sa_noalloc_scratch_bytes": (ctypes.c_size_t, []),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _try_load() -> Optional[ctypes.CDLL]:
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        _load_error = f"{LIB_PATH} is not built (run __graft_entry__.build())"
        return None
    try:
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.sa_abi_version() != ABI_VERSION:
            raise OSError(f"ABI version {lib.sa_abi_version()} != {ABI_VERSION}")
    except (OSError, AttributeError) as ex:
        _load_error = f"cannot load {LIB_PATH}: {ex}"
        return None
    _lib = lib
    return lib


def available() -> bool:
    """True when libsparseattn.so loads (it may still lack a GPU to run on)."""
    return _try_load() is not None


def lib() -> ctypes.CDLL:
    l = _try_load()
    if l is None:
        raise RuntimeError(f"sparse-ai HIP backend unavailable: {_load_error}")
    return l


def check(rc: int) -> None:
    if rc == SA_OK:
        return
    msg = lib().sa_last_error().decode(errors="replace")
    if rc == SA_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; raises RuntimeError otherwise (no CPU fallback)."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError("the sparse-ai HIP kernels need tensors on a HIP (cuda) device; "
                           f"got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def strides(t: torch.Tensor, n: Optional[int] = None):
    s = list(t.stride())
    if n is not None:
        s = s + [0] * (n - len(s))
    return (ctypes.c_int64 * len(s))(*s)


def ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def dtype_code(dt: torch.dtype, allowed: Sequence[torch.dtype]) -> int:
    if dt not in allowed:
        raise ValueError(f"unsupported dtype {dt}; expected one of {list(allowed)}")
    return DTYPE_CODES[dt]
