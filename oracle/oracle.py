"""NumPy-facing wrapper over the C oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product package ``maxsim_amd`` never imports it.

Each function restates the reference behaviour cited in
``oracle/maxsim_oracle.h``; this file only marshals arrays.
"""
from __future__ import annotations

import ctypes
import glob
import importlib.util
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

MAXSIM, WEIGHTED, TOPK2, TOPK4, SMOOTHSIM = 0, 1, 2, 3, 4
REDUCER_CODES = {
    "maxsim": MAXSIM,
    "weighted_maxsim": WEIGHTED,
    "topk2": TOPK2,
    "topk4": TOPK4,
    "smoothsim": SMOOTHSIM,
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_pairwise_sum_f64.restype = ctypes.c_double
        _lib.orc_pairwise_sum_f32.restype = ctypes.c_float
        _lib.orc_pack_int4_tensor.restype = ctypes.c_double
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


I64 = ctypes.c_int64


def pairwise_sum_f64(a) -> float:
    a = _c(a, np.float64)
    return float(_load().orc_pairwise_sum_f64(_p(a), I64(a.size)))


def pairwise_sum_f32(a) -> np.float32:
    a = _c(a, np.float32)
    return np.float32(_load().orc_pairwise_sum_f32(_p(a), I64(a.size)))


def pack_int4_token(x):
    x = _c(x, np.float32)
    t, d = x.shape
    codes = np.zeros((t, d // 2), np.uint8)
    values = np.zeros((t, d), np.int8)
    scale = np.zeros(t, np.float32)
    _load().orc_pack_int4_token(_p(x), I64(t), ctypes.c_int(d), _p(codes), _p(values), _p(scale))
    return codes, values, scale


def pack_int4_tensor(x):
    x = _c(x, np.float32)
    t, d = x.shape
    codes = np.zeros((t, d // 2), np.uint8)
    values = np.zeros((t, d), np.int8)
    scale = _load().orc_pack_int4_tensor(_p(x), I64(t), ctypes.c_int(d), _p(codes), _p(values))
    return codes, values, float(scale)


def unpack_int4(codes, dim):
    codes = _c(codes, np.uint8)
    values = np.zeros((codes.shape[0], dim), np.int8)
    _load().orc_unpack_int4(_p(codes), I64(codes.shape[0]), ctypes.c_int(dim), _p(values))
    return values


def pack_signs(x):
    x = _c(x, np.float32)
    t, d = x.shape
    out = np.zeros((t, d // 8), np.uint8)
    _load().orc_pack_signs(_p(x), I64(t), ctypes.c_int(d), _p(out))
    return out


def quantize_int8(q):
    q = _c(q, np.float32)
    dim = q.shape[-1]
    rows = int(np.prod(q.shape[:-1]))
    q8 = np.zeros(q.shape, np.int8)
    scale = np.zeros(q.shape[:-1], np.float32)
    _load().orc_quantize_int8(_p(q), I64(rows), ctypes.c_int(dim), _p(q8), _p(scale))
    return q8, scale


def int4_int8q_scores(query, values, offsets, token_scale=None, scale=1.0):
    """query f32 [B,Q,D] -> f32 [B,N] (tests/test_int4_int8q.py:7-26)."""
    query = _c(query, np.float32)
    b, q, d = query.shape
    q8, qs = quantize_int8(query)
    values = _c(values, np.int8)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    ts = None if token_scale is None else _c(token_scale, np.float32)
    out = np.zeros((b, n), np.float32)
    _load().orc_int4_int8q_scores(
        _p(q8), _p(qs), I64(b), I64(q), ctypes.c_int(d), _p(values), _p(ts),
        ctypes.c_double(scale), _p(offsets), I64(n), _p(out))
    return out


def int8_dots(q8, values):
    q8 = _c(q8, np.int8).reshape(-1, values.shape[1])
    values = _c(values, np.int8)
    out = np.zeros((q8.shape[0], values.shape[0]), np.int32)
    _load().orc_int8_dots(_p(q8), I64(q8.shape[0]), ctypes.c_int(values.shape[1]), _p(values),
                          I64(values.shape[0]), _p(out))
    return out


def _weights(weights, b, q):
    if weights is None:
        return None
    w = np.asarray(weights, np.float32)
    if w.ndim == 1:
        w = np.broadcast_to(w[None, :], (b, q))
    return _c(w, np.float32)


def int4_fp32_scores(query, values, offsets, *, scale=1.0, token_scale=None, reducer="maxsim",
                     weights=None, temperature=1.0, candidates=None):
    query = _c(query, np.float32)
    b, q, d = query.shape
    values = _c(values, np.int8)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    cand = None if candidates is None else _c(candidates, np.int64)
    targets = n if cand is None else cand.shape[0]
    ts = None if token_scale is None else _c(token_scale, np.float32)
    w = _weights(weights, b, q)
    out = np.zeros((b, targets), np.float32)
    _load().orc_int4_fp32_scores(
        _p(query), I64(b), I64(q), ctypes.c_int(d), _p(values), ctypes.c_float(scale), _p(ts),
        _p(offsets), I64(n), _p(cand), I64(0 if cand is None else cand.shape[0]),
        ctypes.c_int(REDUCER_CODES[reducer]), _p(w), ctypes.c_float(temperature), _p(out))
    return out


def dense_scores(query, docs, offsets, *, reducer="maxsim", weights=None, temperature=1.0,
                 candidates=None):
    query = _c(query, np.float32)
    b, q, d = query.shape
    docs = _c(docs, np.float32)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    cand = None if candidates is None else _c(candidates, np.int64)
    targets = n if cand is None else cand.shape[0]
    w = _weights(weights, b, q)
    out = np.zeros((b, targets), np.float32)
    _load().orc_dense_scores(
        _p(query), I64(b), I64(q), ctypes.c_int(d), _p(docs), _p(offsets), I64(n), _p(cand),
        I64(0 if cand is None else cand.shape[0]), ctypes.c_int(REDUCER_CODES[reducer]), _p(w),
        ctypes.c_float(temperature), _p(out))
    return out


def binary_lut_maxsim(query, codes, offsets, dim, scale=1.0):
    """One query [Q, D] -> f32 [N] (cpp/maxsim/cpu_extension.cpp:82-126)."""
    query = _c(query, np.float32)
    codes = _c(codes, np.uint8)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    out = np.zeros(n, np.float32)
    _load().orc_binary_lut_maxsim(_p(query), I64(query.shape[0]), ctypes.c_int(dim), _p(codes),
                                  _p(offsets), I64(n), ctypes.c_float(scale), _p(out))
    return out


def binary_hamming_maxsim(qbits, codes, offsets, dim):
    """qbits u8 [B, Q, D/8] -> int32 [B, N]."""
    qbits = _c(qbits, np.uint8)
    b, q, _ = qbits.shape
    codes = _c(codes, np.uint8)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    out = np.zeros((b, n), np.int32)
    _load().orc_binary_hamming_maxsim(_p(qbits), I64(b), I64(q), ctypes.c_int(dim), _p(codes),
                                      _p(offsets), I64(n), _p(out))
    return out


def topk(scores, k, tie_ids=None):
    scores = _c(scores, np.float32)
    squeeze = scores.ndim == 1
    s2 = scores[None, :] if squeeze else scores
    b, n = s2.shape
    ties = None
    if tie_ids is not None:
        ties = _c(np.broadcast_to(np.asarray(tie_ids, np.int64), s2.shape), np.int64)
    out_s = np.zeros((b, k), np.float32)
    out_i = np.zeros((b, k), np.int64)
    _load().orc_topk(_p(s2), I64(b), I64(n), I64(k), _p(ties), _p(out_s), _p(out_i))
    return (out_s[0], out_i[0]) if squeeze else (out_s, out_i)


def pack_binary_residual(x):
    x = _c(x, np.float32)
    t, d = x.shape
    signs = np.zeros((t, d // 8), np.uint8)
    a = np.zeros(t, np.float32)
    rcodes = np.zeros((t, d // 2), np.uint8)
    rvalues = np.zeros((t, d), np.int8)
    rscale = np.zeros(t, np.float32)
    _load().orc_pack_binary_residual(_p(x), I64(t), ctypes.c_int(d), _p(signs), _p(a),
                                     _p(rcodes), _p(rvalues), _p(rscale))
    return signs, a, rcodes, rvalues, rscale


def binres_prefix_scores(query, signs, prefix_scale, offsets):
    query = _c(query, np.float32)
    b, q, d = query.shape
    q8, qs = quantize_int8(query)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    out = np.zeros((b, n), np.float32)
    _load().orc_binres_prefix_scores(_p(q8), _p(qs), I64(b), I64(q), ctypes.c_int(d),
                                     _p(_c(signs, np.uint8)), _p(_c(prefix_scale, np.float32)),
                                     _p(offsets), I64(n), _p(out))
    return out


def binres_fused_scores(query, signs, prefix_scale, residual_values, residual_scale, offsets,
                        candidates=None):
    """candidates: None (all docs) or int64 [B, M] per batch row."""
    query = _c(query, np.float32)
    b, q, d = query.shape
    q8, qs = quantize_int8(query)
    offsets = _c(offsets, np.int64)
    n = offsets.shape[0] - 1
    cand = None if candidates is None else _c(candidates, np.int64)
    m = 0 if cand is None else cand.shape[1]
    out = np.zeros((b, n if cand is None else m), np.float32)
    _load().orc_binres_fused_scores(
        _p(q8), _p(qs), I64(b), I64(q), ctypes.c_int(d), _p(_c(signs, np.uint8)),
        _p(_c(prefix_scale, np.float32)), _p(_c(residual_values, np.int8)),
        _p(_c(residual_scale, np.float32)), _p(offsets), I64(n), _p(cand), I64(m), _p(out))
    return out


def reference_cpu_extension():
    """The reference's own compiled CPU extension (oracle/_ref), or None.

    Built by ``make -C oracle ref`` from /root/reference/cpp/maxsim/cpu_extension.cpp.
    """
    paths = glob.glob(os.path.join(_HERE, "_ref", "_maxsim_cpp*.so"))
    if not paths:
        return None
    spec = importlib.util.spec_from_file_location("_maxsim_cpp", paths[0])
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module
