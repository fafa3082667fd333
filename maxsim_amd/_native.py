"""ctypes binding of the C ABI in ``include/maxsim_hip.h``.

The shared library ``maxsim_amd/libmaxsim_hip.so`` is built in-tree by
``python -m maxsim_amd.build``.  There is no fallback: if the library is
missing or cannot be loaded, every device entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmaxsim_hip.so")

MSIM_OK, MSIM_EINVAL, MSIM_ERUNTIME, MSIM_ENOTSUP = 0, 1, 2, 3

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_dbl = ctypes.c_double
c_vp = ctypes.c_void_p
c_str = ctypes.c_char_p

# name -> argtypes (all functions return int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "msim_last_error": [],
    "msim_abi_version": [],
    "msim_set_docs_per_wave": [c_int],
    "msim_get_docs_per_wave": [],
    "msim_set_fused_topk": [c_int],
    "msim_pack_int4": [c_vp, c_i64, c_int, c_int, c_dbl, c_vp, c_vp, c_vp, c_vp],
    "msim_pack_int4_async": [c_vp, c_i64, c_int, c_int, c_dbl, c_vp, c_vp, c_vp, c_vp, c_vp],
    "msim_get_fused_topk": [],
    "msim_set_fused_wait_ticks": [c_i64],
    "msim_get_fused_wait_ticks": [],
    "msim_int4_fused_giveups": [c_vp, c_vp],
    "msim_set_scan_partition": [c_int],
    "msim_get_scan_partition": [],
    "msim_set_prefix_scan": [c_int],
    "msim_get_prefix_scan": [],
    "msim_set_hamming_fp4": [c_int],
    "msim_get_hamming_fp4": [],
    # int4 handle
    "msim_int4_create": [c_vp, c_i64, c_i64, c_vp, c_i64, c_int, c_dbl, c_vp],
    "msim_int4_destroy": [c_vp],
    "msim_int4_set_token_scale": [c_vp, c_vp, c_i64],
    "msim_int4_clear_token_scale": [c_vp],
    "msim_int4_set_residual": [c_vp, c_vp, c_i64, c_i64, c_dbl, c_vp, c_i64],
    "msim_int4_clear_residual": [c_vp],
    "msim_int4_get_props": [c_vp, c_vp],
    "msim_int4_maxsim_batch_int8q": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp],
    "msim_int4_topk_batch_int8q": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    "msim_int4_maxsim_int8q_async": [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp],
    "msim_int4_topk_int8q_async": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "msim_int4_topk_int8q_noalloc": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "msim_int4_quantize_int8q_async": [c_vp, c_vp, c_i64, c_i64, c_vp],
    "msim_int4_score_int8q_async": [c_vp, c_i64, c_i64, c_vp, c_vp],
    "msim_int4_topk_quantized_async": [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "msim_topk_async": [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "msim_int4_maxsim_batch": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp],
    "msim_int4_topk_batch": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    "msim_int4_score": [c_vp, c_vp, c_i64, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64, c_dbl,
                        c_vp, c_i64, c_int, c_vp],
    "msim_int4_topk_score": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64, c_dbl, c_int,
                             c_vp, c_vp],
    "msim_binary_topk_score": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64, c_dbl, c_dbl,
                               c_int, c_int, c_vp, c_vp, c_vp],
    "msim_int4_score_async": [c_vp, c_vp, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64, c_dbl, c_int, c_vp,
                              c_vp],
    "msim_int4_cascade_topk": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64,
                               c_dbl, c_vp, c_vp],
    # binary handle
    "msim_binary_create": [c_vp, c_i64, c_i64, c_vp, c_i64, c_int, c_vp],
    "msim_binary_destroy": [c_vp],
    "msim_binary_set_scale_vector": [c_vp, c_vp, c_i64],
    "msim_binary_clear_scale_vector": [c_vp],
    "msim_binary_set_token_scale": [c_vp, c_vp, c_i64],
    "msim_binary_clear_token_scale": [c_vp],
    "msim_binary_get_props": [c_vp, c_vp],
    "msim_binary_maxsim_batch": [c_vp, c_vp, c_i64, c_i64, c_i64, c_dbl, c_int, c_int, c_vp],
    "msim_binary_topk_batch": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_dbl, c_int, c_int, c_vp, c_vp],
    "msim_binary_maxsim_batch_int8q": [c_vp, c_vp, c_i64, c_i64, c_i64, c_dbl, c_int, c_int, c_vp],
    "msim_binary_topk_batch_int8q": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_dbl, c_int, c_int, c_vp, c_vp],
    "msim_binary_score": [c_vp, c_vp, c_i64, c_i64, c_i64, c_str, c_vp, c_i64, c_i64, c_i64, c_dbl,
                          c_dbl, c_int, c_int, c_vp, c_vp, c_i64, c_vp],
    "msim_binary_hamming_batch": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp],
    "msim_binary_topk_hamming": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    "msim_binary_topk_hamming_async": [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
    "msim_binary_set_residual": [c_vp, c_vp, c_i64, c_i64, c_dbl, c_vp, c_i64],
    "msim_binary_clear_residual": [c_vp],
    "msim_binary_set_rescore_limbs": [c_vp, c_int],
    "msim_binary_get_rescore_limbs": [c_vp, c_vp],
    "msim_binary_binres_score": [c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_vp, c_i64, c_vp],
    "msim_binary_binres_topk": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    "msim_binary_cascade_topk": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp],
    "msim_binary_cascade_topk_async": [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp],
}

_RESTYPES = {"msim_last_error": ctypes.c_char_p, "msim_get_fused_wait_ticks": c_i64}


class Int4Props(ctypes.Structure):
    _fields_ = [
        ("dim", c_i64),
        ("num_docs", c_i64),
        ("num_tokens", c_i64),
        ("scale", c_dbl),
        ("residual_scale", c_dbl),
        ("packed_size", ctypes.c_uint64),
        ("has_token_scale_vector", c_i64),
        ("token_scale_vector_size", ctypes.c_uint64),
        ("has_residual_int4", c_i64),
        ("resident_bytes", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
    ]


class BinaryProps(ctypes.Structure):
    _fields_ = [
        ("dim", c_i64),
        ("num_docs", c_i64),
        ("num_tokens", c_i64),
        ("packed_size", ctypes.c_uint64),
        ("has_scale_vector", c_i64),
        ("scale_vector_size", ctypes.c_uint64),
        ("has_token_scale_vector", c_i64),
        ("token_scale_vector_size", ctypes.c_uint64),
        ("resident_bytes", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
    ]


_lib = None


class NativeLibraryMissing(ImportError):
    pass


def load():
    """Load libmaxsim_hip.so (raises NativeLibraryMissing when absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built; run `python -m maxsim_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def check(status: int) -> None:
    """Raise the Python exception matching a C ABI status code."""
    if status == MSIM_OK:
        return
    message = load().msim_last_error().decode("utf-8", "replace")
    if status == MSIM_EINVAL:
        raise ValueError(message)
    if status == MSIM_ENOTSUP:
        raise NotImplementedError(message)
    raise RuntimeError(message)


def ptr(array) -> int | None:
    """Address of a NumPy array's data or a torch tensor's storage (or None),
    as an int (every pointer argument of the binding is a c_void_p)."""
    if array is None:
        return None
    data_ptr = getattr(array, "data_ptr", None)
    if data_ptr is not None:
        return data_ptr()
    return array.__array_interface__["data"][0]
