"""Resident-corpus device handles over the C ABI (libmaxsim_hip.so).

This module is the MI355X replacement for the reference's native handle
module ``maxsim._maxsim_cuda`` (pybind11, cpp/maxsim/cuda_extension.cu:3416-3514).
Class names, method names, argument order, defaults, return shapes and error
types/messages follow that module so that the reference's Python layer
(which probes it with ``hasattr``/``getattr``) and code written against it can
use these handles unchanged.  Arrays are accepted the way pybind11's
``array_t<T, c_style | forcecast>`` accepts them: anything NumPy can convert,
copied to a C-contiguous array of the target dtype.

Every scoring call runs on the GPU through HIP kernels; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import threading as _threading

import numpy as np

from maxsim_amd import _native
from maxsim_amd._native import check, ptr


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _i64(a):
    return np.ascontiguousarray(a, dtype=np.int64)


def _query3(query):
    q = _f32(query)
    if q.ndim != 3:
        raise ValueError("query must have shape [batch, query_tokens, dim]")
    return q


def _weights(query_weights):
    """(array, ndim, dim0, dim1) for the C ABI's reducer weights."""
    if query_weights is None:
        return None, 0, 0, 0
    try:
        w = np.ascontiguousarray(query_weights, dtype=np.float32)
    except (TypeError, ValueError) as exc:
        raise ValueError("query_weights must be convertible to a float32 array") from exc
    if w.ndim == 1:
        return w, 1, w.shape[0], 0
    if w.ndim == 2:
        return w, 2, w.shape[0], w.shape[1]
    raise ValueError("query_weights must have shape [query_tokens] or [batch, query_tokens]")


def _candidates(candidate_indices):
    c = _i64(candidate_indices)
    if c.ndim != 1:
        raise ValueError("candidate_indices must be a 1-D array")
    return c


def set_docs_per_wave(value: int) -> None:
    """Routing knob: documents per wave of the streaming kernels (0 = auto)."""
    check(_native.load().msim_set_docs_per_wave(int(value)))


def get_docs_per_wave() -> int:
    return int(_native.load().msim_get_docs_per_wave())


def set_fused_topk(mode: int) -> None:
    """Top-k selection of the int8-query search: 1 = in the scan's workgroup 0
    when the call fits (default), 0 = separate launch, 2 = fused with the
    k-round selection path forced (testing)."""
    check(_native.load().msim_set_fused_topk(int(mode)))


def get_fused_topk() -> int:
    return int(_native.load().msim_get_fused_topk())


def set_fused_wait_ticks(ticks: int) -> None:
    """How long the int8-query search's fused selection waits for the scan's
    other workgroups, in ticks of the GPU's 100 MHz clock (default 10**7 =
    100 ms).  A selection that runs out of time gives up: synchronous calls
    raise RuntimeError, the *_async forms leave id -1 / NaN in the row.  0
    makes every fused selection give up at once (tests of that path)."""
    check(_native.load().msim_set_fused_wait_ticks(int(ticks)))


def get_fused_wait_ticks() -> int:
    return int(_native.load().msim_get_fused_wait_ticks())


# The reference module's launch-shape knobs (cuda_extension.cu:24-76,
# 3482-3513).  They pick among the reference's SM89 kernels: shared-memory
# reducer warps, residual reducer warps, and the dim-128 unrolled / q-tiled
# binary kernels.  Every gfx950 scoring path here is one MFMA kernel whose
# launch shape comes from the corpus (msim_set_docs_per_wave), so these
# settings change no result and no launch.  They are kept with the
# reference's defaults, scope (the warp knobs per thread, the dim-128 ones
# per process), validation and messages, so that code and tests written
# against the reference's module run unchanged.
_routing = _threading.local()
_dim128_unrolled_min_avg_tokens = 256
_dim128_qtile_min_packed_bytes = (1 << 64) - 1


def _thread_knob(name: str, default: int) -> int:
    return int(getattr(_routing, name, default))


def set_shared_reducer_warps(value: int) -> None:
    """Reference: cu:3486-3492 (no effect on gfx950)."""
    value = int(value)
    if value not in (0, 4, 8):
        raise ValueError("shared reducer warps must be one of 0, 4, or 8")
    _routing.shared_reducer_warps = value


def get_shared_reducer_warps() -> int:
    return _thread_knob("shared_reducer_warps", 4)


def set_residual_reducer_warps(value: int) -> None:
    """Reference: cu:3493-3499 (no effect on gfx950)."""
    value = int(value)
    if value not in (0, 4, 8):
        raise ValueError("residual reducer warps must be one of 0, 4, or 8")
    _routing.residual_reducer_warps = value


def get_residual_reducer_warps() -> int:
    return _thread_knob("residual_reducer_warps", 8)


def set_residual_reducer_force_warps(value: int) -> None:
    """Reference: cu:3500-3507 (no effect on gfx950)."""
    value = int(value)
    if value not in (-1, 0, 4, 8):
        raise ValueError("residual reducer force warps must be one of -1, 0, 4, or 8")
    _routing.residual_reducer_force_warps = value


def get_residual_reducer_force_warps() -> int:
    return _thread_knob("residual_reducer_force_warps", -1)


def get_effective_residual_reducer_warps(query_tokens: int) -> int:
    """The reference's residual launch policy (cu:58-76) applied to the knobs
    above; reported only."""
    query_tokens = int(query_tokens)
    if query_tokens <= 0:
        raise ValueError("query tokens must be positive")
    forced = get_residual_reducer_force_warps()
    if forced >= 0:
        return forced
    warps = get_residual_reducer_warps()
    if warps == 8:
        return 8 if query_tokens >= 8 else 4
    return warps if warps <= query_tokens else 0


def set_dim128_unrolled_min_avg_tokens(value: int) -> None:
    """Reference: cu:3482 (no effect on gfx950)."""
    global _dim128_unrolled_min_avg_tokens
    _dim128_unrolled_min_avg_tokens = int(value)


def get_dim128_unrolled_min_avg_tokens() -> int:
    return _dim128_unrolled_min_avg_tokens


def set_dim128_qtile_min_packed_bytes(value: int) -> None:
    """Reference: cu:3484 (no effect on gfx950).  The reference's argument is a
    size_t: negative values and values of 2**64 or more are rejected."""
    global _dim128_qtile_min_packed_bytes
    if isinstance(value, bool) or not isinstance(value, (int, np.integer)):
        raise TypeError("set_dim128_qtile_min_packed_bytes(): incompatible function arguments")
    value = int(value)
    if value < 0 or value >= (1 << 64):
        raise TypeError("set_dim128_qtile_min_packed_bytes(): incompatible function arguments")
    _dim128_qtile_min_packed_bytes = value


def get_dim128_qtile_min_packed_bytes() -> int:
    return _dim128_qtile_min_packed_bytes


def set_prefix_scan(mode: int) -> None:
    """Prefix pass of binary-prefix + int4-residual cascades: 1 = the int8-query
    scan kernel over the sign stream when it applies (default), 0 = the
    generalized scorer (testing)."""
    check(_native.load().msim_set_prefix_scan(int(mode)))


def get_prefix_scan() -> int:
    return int(_native.load().msim_get_prefix_scan())


def set_hamming_fp4(mode: int) -> None:
    """Sign-query (Hamming) scoring: 1 = the fp4 MFMA kernel (default), 0 = the
    int8 MFMA scorer (testing); results are identical."""
    check(_native.load().msim_set_hamming_fp4(int(mode)))


def get_hamming_fp4() -> int:
    return int(_native.load().msim_get_hamming_fp4())


def set_scan_partition(mode: int) -> None:
    """Work split of the int8-query scan: 0 = longest-first document
    assignment (default), 1 = contiguous document ranges."""
    check(_native.load().msim_set_scan_partition(int(mode)))


def get_scan_partition() -> int:
    return int(_native.load().msim_get_scan_partition())


class CudaInt4PackedDocs:
    """Resident int4 corpus (reference: CudaInt4PackedDocs, cu:2677-3306)."""

    def __init__(self, packed, offsets, dim: int, scale: float):
        lib = _native.load()
        packed = _u8(packed)
        offsets = _i64(offsets)
        if packed.ndim != 2:
            raise ValueError("packed must have shape [num_doc_tokens, dim / 2]")
        if offsets.ndim != 1:
            raise ValueError("offsets must be a 1-D array")
        handle = ctypes.c_void_p()
        check(lib.msim_int4_create(ptr(packed), packed.shape[0], packed.shape[1], ptr(offsets),
                                   offsets.shape[0], int(dim), float(scale), ctypes.byref(handle)))
        self._lib = lib
        self._h = handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.msim_int4_destroy(h)
            self._h = None

    # ---------------------------------------------------------- residency
    def set_token_scale_vector(self, token_scales):
        ts = _f32(token_scales)
        if ts.ndim != 1:
            raise ValueError("token scale vector must have shape [num_doc_tokens]")
        check(self._lib.msim_int4_set_token_scale(self._h, ptr(ts), ts.shape[0]))

    def clear_token_scale_vector(self):
        check(self._lib.msim_int4_clear_token_scale(self._h))

    def set_residual_int4(self, packed, scale, token_scales):
        p = _u8(packed)
        ts = _f32(token_scales)
        if p.ndim != 2:
            raise ValueError("residual packed data must have shape [num_doc_tokens, dim / 2]")
        if ts.ndim != 1:
            raise ValueError("residual token scale vector must have shape [num_doc_tokens]")
        check(self._lib.msim_int4_set_residual(self._h, ptr(p), p.shape[0], p.shape[1], float(scale),
                                               ptr(ts), ts.shape[0]))

    def clear_residual_int4(self):
        check(self._lib.msim_int4_clear_residual(self._h))

    # ------------------------------------------------------------ scoring
    def maxsim_batch(self, query):
        q = _query3(query)
        out = np.empty((q.shape[0], self.num_docs), np.float32)
        check(self._lib.msim_int4_maxsim_batch(self._h, ptr(q), *q.shape, ptr(out)))
        return out

    def topk_batch(self, query, k):
        q = _query3(query)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(self._lib.msim_int4_topk_batch(self._h, ptr(q), *q.shape, k, ptr(scores), ptr(indices)))
        return scores, indices

    def maxsim_batch_int8q(self, query):
        q = _query3(query)
        out = np.empty((q.shape[0], self.num_docs), np.float32)
        check(self._lib.msim_int4_maxsim_batch_int8q(self._h, ptr(q), *q.shape, ptr(out)))
        return out

    def topk_batch_int8q(self, query, k):
        q = _query3(query)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(self._lib.msim_int4_topk_batch_int8q(self._h, ptr(q), *q.shape, k, ptr(scores),
                                                   ptr(indices)))
        return scores, indices

    def _score(self, query, candidate_indices, reducer, query_weights, temperature, residual):
        q = _query3(query)
        w, wnd, w0, w1 = _weights(query_weights)
        cand = None if candidate_indices is None else _candidates(candidate_indices)
        targets = self.num_docs if cand is None else cand.shape[0]
        out = np.empty((q.shape[0], targets), np.float32)
        if not isinstance(reducer, str):
            raise ValueError("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'")
        check(self._lib.msim_int4_score(
            self._h, ptr(q), *q.shape, reducer.encode(), ptr(w), wnd, w0, w1, float(temperature),
            ptr(cand), 0 if cand is None else cand.shape[0], 1 if residual else 0, ptr(out)))
        return out

    def score_batch(self, query, reducer="maxsim", query_weights=None, temperature=1.0):
        return self._score(query, None, reducer, query_weights, temperature, False)

    def score_candidates_batch(self, query, candidate_indices, reducer="maxsim", query_weights=None,
                               temperature=1.0):
        return self._score(query, candidate_indices, reducer, query_weights, temperature, False)

    def score_residual_batch(self, query, reducer="maxsim", query_weights=None, temperature=1.0):
        return self._score(query, None, reducer, query_weights, temperature, True)

    def score_residual_candidates_batch(self, query, candidate_indices, reducer="maxsim",
                                        query_weights=None, temperature=1.0):
        return self._score(query, candidate_indices, reducer, query_weights, temperature, True)

    def topk_score_batch(self, query, k, reducer="maxsim", query_weights=None, temperature=1.0, residual=False):
        """Top-k under any reducer, selected on the device."""
        q = _query3(query)
        w, wnd, w0, w1 = _weights(query_weights)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        if not isinstance(reducer, str):
            raise ValueError("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(self._lib.msim_int4_topk_score(self._h, ptr(q), *q.shape, k, reducer.encode(), ptr(w), wnd, w0, w1,
                                             float(temperature), 1 if residual else 0, ptr(scores), ptr(indices)))
        return scores, indices

    def cascade_topk(self, query, k, candidates, reducer="maxsim", query_weights=None, temperature=1.0):
        """Prefix top-M -> fused residual rescoring -> top-k, all on the device
        (the pipeline of cascade_topk, cascade.py:294-393)."""
        q = _query3(query)
        w, wnd, w0, w1 = _weights(query_weights)
        k, m = int(k), int(candidates)
        scores = np.empty((q.shape[0], max(k, 0)), np.float32)
        indices = np.empty((q.shape[0], max(k, 0)), np.int64)
        if not isinstance(reducer, str):
            raise ValueError("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'")
        check(self._lib.msim_int4_cascade_topk(self._h, ptr(q), *q.shape, k, m, reducer.encode(), ptr(w), wnd, w0,
                                               w1, float(temperature), ptr(scores), ptr(indices)))
        return scores, indices

    # ------------------------------------------------- device-resident (torch)
    def maxsim_int8q_async(self, query, out, stream=None):
        """Enqueue int8-query MaxSim on device tensors: query f32[B,Q,128] and
        out f32[B,N] (torch tensors on this handle's device, contiguous)."""
        b, q = int(query.shape[0]), int(query.shape[1])
        check(self._lib.msim_int4_maxsim_int8q_async(self._h, ptr(query), b, q, ptr(out),
                                                     _stream_ptr(stream)))

    def fused_giveups(self) -> int:
        """Fused int8-query selections of this handle that gave up waiting
        (their rows hold id -1); waits for the device first."""
        out = ctypes.c_uint64()
        check(self._lib.msim_int4_fused_giveups(self._h, ctypes.byref(out)))
        return int(out.value)

    def topk_int8q_async(self, query, k, scores, indices, stream=None):
        """Enqueue int8-query MaxSim + top-k on device tensors (scores f32[B,k],
        indices i64[B,k]).  A row whose fused selection gave up holds id -1 and
        NaN scores (see set_fused_wait_ticks)."""
        b, q = int(query.shape[0]), int(query.shape[1])
        check(self._lib.msim_int4_topk_int8q_async(self._h, ptr(query), b, q, int(k), ptr(scores),
                                                   ptr(indices), _stream_ptr(stream)))

    # --------------------------------------------------------- properties
    def _props(self):
        props = _native.Int4Props()
        check(self._lib.msim_int4_get_props(self._h, ctypes.byref(props)))
        return props

    @property
    def dim(self) -> int:
        return int(self._props().dim)

    @property
    def num_docs(self) -> int:
        return int(self._props().num_docs)

    @property
    def num_tokens(self) -> int:
        return int(self._props().num_tokens)

    @property
    def scale(self) -> float:
        return float(np.float32(self._props().scale))

    @property
    def packed_size(self) -> int:
        return int(self._props().packed_size)

    @property
    def has_token_scale_vector(self) -> bool:
        return bool(self._props().has_token_scale_vector)

    @property
    def token_scale_vector_size(self) -> int:
        return int(self._props().token_scale_vector_size)

    @property
    def has_residual_int4(self) -> bool:
        return bool(self._props().has_residual_int4)

    @property
    def resident_bytes(self) -> int:
        return int(self._props().resident_bytes)

    @property
    def workspace_bytes(self) -> int:
        return int(self._props().workspace_bytes)


class CudaPackedDocs:
    """Resident sign-bit corpus (reference: CudaPackedDocs, cu:1872-2675).

    Every scoring method runs the MFMA kernels of score.hip: fp32 queries are
    split into three int8 limbs, int8 queries (``*_int8q``) use one, and
    sign-bit queries (``hamming_batch`` / ``topk_hamming``) are exact +-1
    dot products, i.e. dim - 2 popcount(q ^ d)."""

    def __init__(self, packed, offsets, dim: int):
        lib = _native.load()
        packed = _u8(packed)
        offsets = _i64(offsets)
        if packed.ndim != 2:
            raise ValueError("packed must have shape [num_doc_tokens, dim / 8]")
        if offsets.ndim != 1:
            raise ValueError("offsets must be a 1-D array")
        handle = ctypes.c_void_p()
        check(lib.msim_binary_create(ptr(packed), packed.shape[0], packed.shape[1], ptr(offsets),
                                     offsets.shape[0], int(dim), ctypes.byref(handle)))
        self._lib = lib
        self._h = handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.msim_binary_destroy(h)
            self._h = None

    # ---------------------------------------------------------- residency
    def set_scale_vector(self, scale):
        v = _f32(scale)
        if v.ndim != 1:
            raise ValueError("scale vector must have shape [num_docs]")
        check(self._lib.msim_binary_set_scale_vector(self._h, ptr(v), v.shape[0]))

    def clear_scale_vector(self):
        check(self._lib.msim_binary_clear_scale_vector(self._h))

    def set_token_scale_vector(self, token_scales):
        v = _f32(token_scales)
        if v.ndim != 1:
            raise ValueError("token scale vector must have shape [num_doc_tokens]")
        check(self._lib.msim_binary_set_token_scale(self._h, ptr(v), v.shape[0]))

    def clear_token_scale_vector(self):
        check(self._lib.msim_binary_clear_token_scale(self._h))

    # ------------------------------------------------------------ scoring
    def maxsim_batch(self, query, scale=1.0, use_scale_vector=False, use_token_scale=False):
        q = _query3(query)
        out = np.empty((q.shape[0], self.num_docs), np.float32)
        check(self._lib.msim_binary_maxsim_batch(self._h, ptr(q), *q.shape, float(scale), int(bool(use_scale_vector)),
                                                 int(bool(use_token_scale)), ptr(out)))
        return out

    def _topk(self, fn, query, k, scale, use_scale_vector, use_token_scale):
        q = _query3(query)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(fn(self._h, ptr(q), *q.shape, k, float(scale), int(bool(use_scale_vector)),
                 int(bool(use_token_scale)), ptr(scores), ptr(indices)))
        return scores, indices

    def topk_batch(self, query, k, scale=1.0, use_scale_vector=False, use_token_scale=False):
        return self._topk(self._lib.msim_binary_topk_batch, query, k, scale, use_scale_vector, use_token_scale)

    def topk_lut_batch(self, query, k, scale=1.0, use_scale_vector=False, use_token_scale=False):
        """Same scores as topk_batch (the reference's LUT kernel is a different
        evaluation of the same sum); dim 128 only, as cu:2165-2211."""
        if self.dim != 128:
            raise ValueError("topk_lut_batch currently requires dim=128")
        return self.topk_batch(query, k, scale, use_scale_vector, use_token_scale)

    def streaming_topk_batch(self, query, k, scale=1.0, use_scale_vector=False):
        """Top-k without a token scale (cu:2270-2329)."""
        return self.topk_batch(query, k, scale, use_scale_vector, False)

    def topk_centroid_batch(self, query, weights, k, scale=1.0, use_scale_vector=False, use_token_scale=False):
        """Top-k of the query with every dim multiplied by weights[dim] (cu:2111-2163)."""
        q = _query3(query)
        w = _f32(weights)
        if w.ndim != 1 or w.shape[0] != self.dim:
            raise ValueError("weights must have shape [dim]")
        return self.topk_batch(q * w[None, None, :], k, scale, use_scale_vector, use_token_scale)

    def maxsim_batch_int8q(self, query, scale=1.0, use_scale_vector=False, use_token_scale=False):
        q = _query3(query)
        out = np.empty((q.shape[0], self.num_docs), np.float32)
        check(self._lib.msim_binary_maxsim_batch_int8q(self._h, ptr(q), *q.shape, float(scale),
                                                       int(bool(use_scale_vector)), int(bool(use_token_scale)),
                                                       ptr(out)))
        return out

    def topk_batch_int8q(self, query, k, scale=1.0, use_scale_vector=False, use_token_scale=False):
        return self._topk(self._lib.msim_binary_topk_batch_int8q, query, k, scale, use_scale_vector,
                          use_token_scale)

    def _score(self, query, candidate_indices, reducer, query_weights, temperature, scale, use_scale_vector,
               use_token_scale, scale_vector_override):
        q = _query3(query)
        w, wnd, w0, w1 = _weights(query_weights)
        cand = None if candidate_indices is None else _candidates(candidate_indices)
        targets = self.num_docs if cand is None else cand.shape[0]
        override = None
        if scale_vector_override is not None:
            override = _f32(scale_vector_override)
            if override.ndim != 1 or override.shape[0] != self.num_docs:
                raise ValueError("scale vector must have shape [num_docs]")
        if not isinstance(reducer, str):
            raise ValueError("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'")
        out = np.empty((q.shape[0], targets), np.float32)
        check(self._lib.msim_binary_score(
            self._h, ptr(q), *q.shape, reducer.encode(), ptr(w), wnd, w0, w1, float(temperature), float(scale),
            int(bool(use_scale_vector)), int(bool(use_token_scale)), ptr(override), ptr(cand),
            0 if cand is None else cand.shape[0], ptr(out)))
        return out

    def score_batch(self, query, reducer="maxsim", query_weights=None, temperature=1.0, scale=1.0,
                    use_scale_vector=False, use_token_scale=False, scale_vector_override=None):
        return self._score(query, None, reducer, query_weights, temperature, scale, use_scale_vector,
                           use_token_scale, scale_vector_override)

    def score_candidates_batch(self, query, candidate_indices, reducer="maxsim", query_weights=None,
                               temperature=1.0, scale=1.0, use_scale_vector=False, use_token_scale=False,
                               scale_vector_override=None):
        return self._score(query, candidate_indices, reducer, query_weights, temperature, scale,
                           use_scale_vector, use_token_scale, scale_vector_override)

    def topk_score_batch(self, query, k, reducer="maxsim", query_weights=None, temperature=1.0, scale=1.0,
                         use_scale_vector=False, use_token_scale=False, scale_vector_override=None):
        """Top-k under any reducer, selected on the device."""
        q = _query3(query)
        w, wnd, w0, w1 = _weights(query_weights)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        override = None
        if scale_vector_override is not None:
            override = _f32(scale_vector_override)
            if override.ndim != 1 or override.shape[0] != self.num_docs:
                raise ValueError("scale vector must have shape [num_docs]")
        if not isinstance(reducer, str):
            raise ValueError("reducer must be one of 'maxsim', 'weighted_maxsim', 'topk2', 'topk4', or 'smoothsim'")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(self._lib.msim_binary_topk_score(self._h, ptr(q), *q.shape, k, reducer.encode(), ptr(w), wnd, w0, w1,
                                               float(temperature), float(scale), int(bool(use_scale_vector)),
                                               int(bool(use_token_scale)), ptr(override), ptr(scores), ptr(indices)))
        return scores, indices

    # ------------------------------------------------- sign-bit queries
    def hamming_batch(self, qbits):
        """int32 [B, N]: sum_q max_t (dim - 2 popcount(qbits[b, q] ^ d_t)) for
        sign-bit queries u8 [B, Q, dim / 8] in pack_signs order."""
        qb = _u8(qbits)
        if qb.ndim != 3 or qb.shape[2] != self.dim // 8:
            raise ValueError("qbits must have shape [batch, query_tokens, dim / 8]")
        out = np.empty((qb.shape[0], self.num_docs), np.int32)
        check(self._lib.msim_binary_hamming_batch(self._h, ptr(qb), qb.shape[0], qb.shape[1], self.dim, ptr(out)))
        return out

    def topk_hamming(self, qbits, k):
        qb = _u8(qbits)
        if qb.ndim != 3 or qb.shape[2] != self.dim // 8:
            raise ValueError("qbits must have shape [batch, query_tokens, dim / 8]")
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        scores = np.empty((qb.shape[0], k), np.float32)
        indices = np.empty((qb.shape[0], k), np.int64)
        check(self._lib.msim_binary_topk_hamming(self._h, ptr(qb), qb.shape[0], qb.shape[1], self.dim, k,
                                                 ptr(scores), ptr(indices)))
        return scores, indices

    def topk_hamming_async(self, qbits, k, scores, indices, stream=None):
        """Enqueue on device tensors: qbits u8[B, Q, 16], scores f32[B, k], indices i64[B, k]."""
        b, q = int(qbits.shape[0]), int(qbits.shape[1])
        check(self._lib.msim_binary_topk_hamming_async(self._h, ptr(qbits), b, q, int(k), ptr(scores),
                                                       ptr(indices), _stream_ptr(stream)))

    # ------------------------- binary prefix + int4 residual (this build)
    def set_residual_int4(self, packed, scale, token_scales):
        p = _u8(packed)
        ts = _f32(token_scales)
        if p.ndim != 2:
            raise ValueError("residual packed data must have shape [num_doc_tokens, dim / 2]")
        if ts.ndim != 1:
            raise ValueError("residual token scale vector must have shape [num_doc_tokens]")
        check(self._lib.msim_binary_set_residual(self._h, ptr(p), p.shape[0], p.shape[1], float(scale), ptr(ts),
                                                 ts.shape[0]))

    def clear_residual_int4(self):
        check(self._lib.msim_binary_clear_residual(self._h))

    def set_rescore_limbs(self, limbs):
        """Query limbs of fused scoring and cascade rescoring: 1 = int8 query,
        3 = fp32 query (three int8 limbs)."""
        check(self._lib.msim_binary_set_rescore_limbs(self._h, int(limbs)))

    def get_rescore_limbs(self) -> int:
        v = ctypes.c_int(0)
        check(self._lib.msim_binary_get_rescore_limbs(self._h, ctypes.byref(v)))
        return int(v.value)

    def binres_score_batch(self, query, fused=True, candidate_indices=None):
        """int8-query coarse (fused=False) or fused scores; candidate_indices
        None or i64 [B, M] per batch row."""
        q = _query3(query)
        cand = None
        if candidate_indices is not None:
            cand = _i64(candidate_indices)
            if cand.ndim != 2 or cand.shape[0] != q.shape[0]:
                raise ValueError("candidate_indices must have shape [batch, candidates]")
        targets = self.num_docs if cand is None else cand.shape[1]
        out = np.empty((q.shape[0], targets), np.float32)
        check(self._lib.msim_binary_binres_score(self._h, ptr(q), *q.shape, int(bool(fused)), ptr(cand),
                                                 0 if cand is None else cand.shape[1], ptr(out)))
        return out

    def binres_topk_batch(self, query, k):
        """Top-k of the fused scores of every document, selected on the device."""
        q = _query3(query)
        k = int(k)
        if k < 1 or k > self.num_docs:
            raise ValueError("k must be between 1 and num_docs")
        scores = np.empty((q.shape[0], k), np.float32)
        indices = np.empty((q.shape[0], k), np.int64)
        check(self._lib.msim_binary_binres_topk(self._h, ptr(q), *q.shape, k, ptr(scores), ptr(indices)))
        return scores, indices

    def cascade_topk(self, query, k, candidates):
        q = _query3(query)
        k, m = int(k), int(candidates)
        scores = np.empty((q.shape[0], max(k, 0)), np.float32)
        indices = np.empty((q.shape[0], max(k, 0)), np.int64)
        check(self._lib.msim_binary_cascade_topk(self._h, ptr(q), *q.shape, k, m, ptr(scores), ptr(indices)))
        return scores, indices

    def cascade_topk_async(self, query, k, candidates, scores, indices, stream=None):
        """Enqueue on device tensors: query f32 [B, Q, 128], scores f32 [B, k], indices i64 [B, k]."""
        b, q = int(query.shape[0]), int(query.shape[1])
        check(self._lib.msim_binary_cascade_topk_async(self._h, ptr(query), b, q, int(k), int(candidates),
                                                       ptr(scores), ptr(indices), _stream_ptr(stream)))

    # --------------------------------------------------------- properties
    def _props(self):
        props = _native.BinaryProps()
        check(self._lib.msim_binary_get_props(self._h, ctypes.byref(props)))
        return props

    @property
    def dim(self) -> int:
        return int(self._props().dim)

    @property
    def num_docs(self) -> int:
        return int(self._props().num_docs)

    @property
    def num_tokens(self) -> int:
        return int(self._props().num_tokens)

    @property
    def packed_size(self) -> int:
        return int(self._props().packed_size)

    @property
    def has_scale_vector(self) -> bool:
        return bool(self._props().has_scale_vector)

    @property
    def scale_vector_size(self) -> int:
        return int(self._props().scale_vector_size)

    @property
    def has_token_scale_vector(self) -> bool:
        return bool(self._props().has_token_scale_vector)

    @property
    def token_scale_vector_size(self) -> int:
        return int(self._props().token_scale_vector_size)

    @property
    def resident_bytes(self) -> int:
        return int(self._props().resident_bytes)

    @property
    def workspace_bytes(self) -> int:
        return int(self._props().workspace_bytes)

    @property
    def maxsim_kernel_variant(self) -> str:
        """The reference's route label for this corpus (cu:2342-2347, 2625-2634:
        "dim128_qtile" when dim is 128 and packed_size reaches
        get_dim128_qtile_min_packed_bytes(), "dim128_unrolled" for dim 128 with
        at most 128 documents or an average of at least
        get_dim128_unrolled_min_avg_tokens() tokens, else "generic").  On
        gfx950 all three routes are the same MFMA sign-document scorer."""
        if self.dim != 128:
            return "generic"
        if self.packed_size >= _dim128_qtile_min_packed_bytes:
            return "dim128_qtile"
        if self.num_docs <= 128:
            return "dim128_unrolled"
        avg_tokens = self.num_tokens // max(self.num_docs, 1)
        return "dim128_unrolled" if avg_tokens >= _dim128_unrolled_min_avg_tokens else "generic"


def _binary_free_inputs(query, packed, offsets, dim, query_ndim):
    """validate_inputs / validate_batch_inputs (cuda_extension.cu:1826-1870):
    the reference's order of checks and messages."""
    q, p, o = _f32(query), _u8(packed), _i64(offsets)
    if q.ndim != query_ndim:
        raise ValueError("query must have shape [query_tokens, dim]" if query_ndim == 2
                         else "query must have shape [batch, query_tokens, dim]")
    if p.ndim != 2:
        raise ValueError("packed must have shape [num_doc_tokens, dim / 8]")
    if o.ndim != 1:
        raise ValueError("offsets must be a 1-D array")
    dim = int(dim)
    if dim <= 0 or dim % 8 != 0:
        raise ValueError("dim must be positive and divisible by 8")
    if q.shape[-1] != dim or p.shape[1] != dim // 8:
        raise ValueError("query/packed shapes do not match dim")
    return q, p, o, dim


def maxsim_cuda(query, packed, offsets, dim: int, scale: float = 1.0):
    """maxsim_cuda(query f32[Q, dim], packed u8[T, dim/8], offsets i64[N+1],
    dim, scale) -> f32[N] (cuda_extension.cu:3308-3358): binary MaxSim of one
    fp32 query against host-resident sign-bit documents, uploaded for the
    call (the reference's _score_binary calls it for CPU-resident documents
    with device="cuda", _api.py:357-371)."""
    q, p, o, dim = _binary_free_inputs(query, packed, offsets, dim, 2)
    return CudaPackedDocs(p, o, dim).maxsim_batch(q[None], scale=float(scale))[0]


def maxsim_cuda_batch(query, packed, offsets, dim: int, scale: float = 1.0):
    """maxsim_cuda_batch(query f32[B, Q, dim], ...) -> f32[B, N]
    (cuda_extension.cu:3360-3411): maxsim_cuda for a batch of queries."""
    q, p, o, dim = _binary_free_inputs(query, packed, offsets, dim, 3)
    return CudaPackedDocs(p, o, dim).maxsim_batch(q, scale=float(scale))


def _stream_ptr(stream):
    if stream is None:
        try:
            import torch

            return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        except Exception:  # pragma: no cover - torch absent
            return None
    handle = getattr(stream, "cuda_stream", stream)
    return ctypes.c_void_p(int(handle))
