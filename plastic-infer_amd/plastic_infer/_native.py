"""Loader and thin ctypes binding of libplastic_infer_amd.so (the gfx950 HIP library).

Every data-movement op of this package runs through this library. There is no host fallback:
if the library is missing, or a tensor handed to an op is not on a HIP device, the op raises.
The C-ABI is declared in include/plastic_infer_amd.h; argument types here mirror it one to one.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libplastic_infer_amd.so"

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
_DTYPE_CODES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes)
_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "pia_last_error": (ctypes.c_char_p, []),
    "pia_abi_version": (_I, []),
    "pia_kv_scatter": (_I, [_P, _P, _P, _P, _P, _L, _L, _L, _I, _I, _I, _L, _I, _P]),
    "pia_kv_gather": (_I, [_P, _P, _P, _P, _P, _L, _P, _I, _L, _I, _I, _I, _L, _I, _P]),
    "pia_kv_pages_chunk_copy": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _L, _I, _I, _P]),
    "pia_kv_pages_chunks_copy": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _L, _I, _I, _P]),
    "pia_paged_decode_workspace_bytes": (_L, [_I, _I, _I, _I, _I, _L]),
    "pia_paged_decode_scratch_layout": (_I, [_I, _I, _I, _P, _P]),
    "pia_paged_decode_attention": (
        _I, [_P, _P, _L, _P, _P, _P, _L, _P, _I, _I, _I, _I, _I, _L, _F, _I, _P, _L, _P]),
    "pia_paged_decode_append_attention": (
        _I, [_P, _P, _L, _P, _P, _P, _L, _P, _P, _P, _L, _I, _I, _I, _I, _I, _L, _F, _I, _P, _L,
             _P]),
    "pia_paged_decode_noalloc_scratch_bytes": (_L, [_I, _I]),
    "pia_paged_decode_attention_noalloc": (
        _I, [_P, _P, _L, _P, _P, _P, _L, _P, _I, _I, _I, _I, _I, _L, _F, _I, _P]),
    "pia_paged_attention": (
        _I, [_P, _P, _P, _P, _P, _L, _P, _P, _P, _I, _L, _I, _I, _I, _I, _L, _F, _I, _P]),
    "pia_host_stream_attention_workspace_bytes": (_L, [_L, _I, _I, _I, _I, _L, _L, _L]),
    "pia_host_stream_attention": (
        _I, [_P, _P, _L, _I, _P, _P, _I, _L, _L, _P, _P, _L, _L, _I, _I, _L, _I, _F, _I, _P, _L,
             _P]),
    "pia_moe_topk": (_I, [_P, _P, _P, _I, _L, _I, _I, _I, _I, _L, _P]),
    "pia_moe_align_workspace_bytes": (_L, [_I]),
    "pia_moe_align_block_size": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _L, _P, _L, _P]),
    "pia_moe_topk_align": (_I, [_P, _P, _P, _I, _L, _I, _I, _I, _I, _L, _P, _P, _P, _P, _I, _L,
                                _P, _L, _P]),
    "pia_moe_permute": (_I, [_P, _P, _P, _P, _P, _L, _L, _I, _L, _L, _P]),
    "pia_moe_unpermute": (_I, [_P, _P, _L, _P, _P, _L, _I, _I, _I, _P]),
    "pia_moe_sum_reduce": (_I, [_P, _P, _L, _I, _I, _I, _P]),
    "pia_moe_expert_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _L, _I, _L, _I, _L, _I, _I, _I, _L,
                                 _I, _I, _I, _P, _L, _P]),
    "pia_moe_expert_gemm_workspace_bytes": (_L, [_L, _I]),
    "pia_act_and_mul": (_I, [_P, _P, _L, _L, _I, _I, _P]),
    "pia_index_copy_rows": (_I, [_P, _P, _L, _P, _P, _L, _L, _P, _L, _I, _P]),
    "pia_index_copy_rows_multi": (_I, [_P, _P, _P, _I, _P, _P, _L, _P, _I, _P]),
    "pia_device_pointer": (_I, [_P, _P]),
    "pia_copy_rows_async": (_I, [_P, _P, _P, _P, _L, _L, _P, _P]),
    "pia_lru_ensure": (_I, [_P, _L, _P, _L, _P, _P, _L, _P, _P, _P, _P, _P, _P, _L, _P]),
    "pia_slot_cache_reset": (_I, [_P, _L, _P, _P, _L, _P, _P, _I, _P, _P]),
    "pia_slot_cache_materialize": (_I, [_P, _L, _P, _P, _L, _P, _P, _P, _P, _I, _I, _P]),
    "pia_slot_cache_invalidate": (_I, [_P, _L, _P, _P, _L, _L, _L, _P]),
    "pia_prefill_hit_compact": (_I, [_P, _P, _P, _P, _L, _L, _I, _P]),
    "pia_hbm_read_probe": (_I, [_P, _L, _P, _L, _P, _P]),
    "pia_hbm_read_rows_probe": (_I, [_P, _L, _I, _I, _P, _P]),
}

EXPECTED_ABI = 10

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """A non-zero status from the HIP library (message from pia_last_error)."""


def load(path: pathlib.Path | None = None) -> ctypes.CDLL:
    """dlopen the library once and declare every exported signature."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = pathlib.Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"plastic_infer HIP library not built: {p} is missing "
                "(run `python plastic-infer_amd/csrc/build.py` or __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        abi = lib.pia_abi_version()
        if abi != EXPECTED_ABI:
            raise RuntimeError(f"{p}: ABI version {abi}, expected {EXPECTED_ABI}")
        _lib = lib
        return lib


def call(name: str, *args) -> int:
    """Call an int-returning entry point and raise NativeError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.pia_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed ({rc}): {msg}")
    return rc


def query(name: str, *args) -> int:
    """Call a size-query entry point (returns int64)."""
    return int(getattr(load(), name)(*args))


# ---------------------------------------------------------------------------------------------
# Tensor plumbing
# ---------------------------------------------------------------------------------------------

def require_device(*tensors: torch.Tensor, names: tuple[str, ...] | None = None) -> torch.device:
    """All tensors must live on the same HIP device; returns it. CPU tensors are rejected:
    this package keeps KV pages and expert slots in HBM and has no host execution path."""
    dev = None
    for i, t in enumerate(tensors):
        label = names[i] if names else f"argument {i}"
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{label}: expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda" or torch.version.hip is None:
            raise ValueError(
                f"{label} is on {t.device}; the plastic_infer data path runs on a HIP (ROCm) "
                "device only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{label} is on {t.device}, expected {dev}")
    assert dev is not None
    return dev


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
