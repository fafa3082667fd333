"""Binary sign corpus, shared validation and reducer options (reference: src/maxsim/_api.py).

Scoring always runs on the GPU through the device handles in
``maxsim_amd._maxsim_hip``; ``device="cpu"`` is rejected.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import numpy as np

Reducer = Literal["maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"]
_REDUCERS = frozenset(("maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"))


# ---------------------------------------------------------------- helpers


def _as_numpy(value) -> np.ndarray:
    """NumPy view of arrays, torch tensors (detached to host) or sequences (_api.py:500-509)."""
    if isinstance(value, np.ndarray):
        return value
    detach = getattr(value, "detach", None)
    if detach is not None:
        return detach().cpu().numpy()
    return np.asarray(value)


def _resolve_device(device) -> str:
    if device not in ("auto", "cpu", "cuda"):
        raise ValueError("device must be 'auto', 'cpu', or 'cuda'")
    if device == "cpu":
        raise NotImplementedError(
            "maxsim_amd scores on the GPU only; use device='cuda' (or 'auto')"
        )
    return "cuda"


def _query_batches(query_tokens, dim: int):
    """[Q, D] or [B, Q, D] -> (float32 [B, Q, D], squeeze)."""
    query = _as_numpy(query_tokens)
    if query.ndim == 2:
        batches, squeeze = query[np.newaxis], True
    elif query.ndim == 3:
        batches, squeeze = query, False
    else:
        raise ValueError("query_tokens must have shape [query_tokens, dim] or [batch, query_tokens, dim]")
    if batches.shape[2] != dim:
        raise ValueError(f"query dim={batches.shape[2]} does not match packed dim={dim}")
    return batches.astype(np.float32, copy=False), squeeze


def _normalize_reducer_options(reducer, query_weights, temperature, *, batch: int, query_tokens: int):
    """Validate reducer, weights and temperature (_api.py:512-543, same messages)."""
    if not isinstance(reducer, str) or reducer not in _REDUCERS:
        raise ValueError(f"reducer must be one of: {', '.join(sorted(_REDUCERS))}")
    try:
        temperature_value = float(temperature)
    except (TypeError, ValueError) as exc:
        raise ValueError("temperature must be a finite value greater than 0") from exc
    if not np.isfinite(temperature_value) or temperature_value <= 0.0:
        raise ValueError("temperature must be a finite value greater than 0")
    if reducer != "weighted_maxsim":
        if query_weights is not None:
            raise ValueError("query_weights is only supported with reducer='weighted_maxsim'")
        return reducer, None, temperature_value
    if query_weights is None:
        raise ValueError("query_weights is required with reducer='weighted_maxsim'")
    weights = _as_numpy(query_weights).astype(np.float32, copy=False)
    if weights.ndim == 1:
        if weights.shape[0] != query_tokens:
            raise ValueError("query_weights must have shape [query_tokens] or [batch, query_tokens]")
        weights = np.broadcast_to(weights[np.newaxis, :], (batch, query_tokens))
    elif weights.ndim != 2 or weights.shape != (batch, query_tokens):
        raise ValueError("query_weights must have shape [query_tokens] or [batch, query_tokens]")
    if not np.all(np.isfinite(weights)):
        raise ValueError("query_weights must contain only finite values")
    return reducer, np.ascontiguousarray(weights, dtype=np.float32), temperature_value


def _normalize_candidate_indices(candidate_indices, num_docs: int) -> np.ndarray | None:
    """1-D integer candidates in [0, num_docs) (_api.py:546-555)."""
    if candidate_indices is None:
        return None
    values = _as_numpy(candidate_indices)
    if values.ndim != 1 or not np.issubdtype(values.dtype, np.integer):
        raise ValueError("candidate_indices must be a one-dimensional integer array")
    normalized = np.ascontiguousarray(values, dtype=np.int64)
    if np.any(normalized < 0) or np.any(normalized >= num_docs):
        raise ValueError("candidate_indices must be between 0 and packed.num_docs - 1")
    return normalized


def _normalize_offsets(doc_offsets, num_tokens: int) -> np.ndarray:
    """Offsets [N+1] spanning all tokens; None means one token per doc (_api.py:588-603)."""
    if doc_offsets is None:
        return np.arange(num_tokens + 1, dtype=np.int64)
    offsets = _as_numpy(doc_offsets).astype(np.int64, copy=False)
    if offsets.ndim != 1:
        raise ValueError("doc_offsets must be a 1-D array")
    if offsets.shape[0] < 2:
        raise ValueError("doc_offsets must contain at least [0, num_doc_tokens]")
    if int(offsets[0]) != 0:
        raise ValueError("doc_offsets must start at 0")
    if int(offsets[-1]) != num_tokens:
        raise ValueError("doc_offsets must end at num_doc_tokens")
    if np.any(offsets[1:] < offsets[:-1]):
        raise ValueError("doc_offsets must be monotonically nondecreasing")
    return offsets.copy()


def _topk_indices_1d(scores: np.ndarray, k: int) -> np.ndarray:
    """lexsort((ids, -scores))[:k] (_api.py:732-735)."""
    order = np.lexsort((np.arange(scores.shape[0], dtype=np.int64), -scores))
    return order[:k].astype(np.int64, copy=False)


# ------------------------------------------------------------ binary format


@dataclass(frozen=True)
class PackedDocs:
    """Reference: PackedDocs (_api.py:23-31)."""

    data: object
    doc_offsets: np.ndarray
    dim: int
    num_docs: int
    scale: object = None
    device: Literal["cpu", "cuda"] = "cpu"
    token_scale: object = None


def pack_signs(doc_embeddings, doc_offsets=None, *, dim=None, scale=None, token_scale=None,
               device="cpu") -> PackedDocs:
    """Sign bits, bit j of byte j/8 LSB-first, x >= 0 -> 1 (_api.py:34-77)."""
    if device not in ("cpu", "cuda"):
        raise ValueError("device must be 'cpu' or 'cuda'")
    docs = _as_numpy(doc_embeddings)
    if docs.ndim != 2:
        raise ValueError("doc_embeddings must have shape [num_doc_tokens, dim]")
    actual_dim = int(docs.shape[1])
    if dim is not None and int(dim) != actual_dim:
        raise ValueError(f"dim={dim} does not match doc_embeddings dim={actual_dim}")
    if actual_dim % 8 != 0:
        raise ValueError("dim must be divisible by 8")
    offsets = _normalize_offsets(doc_offsets, docs.shape[0])
    bits = (docs >= 0).reshape(docs.shape[0], actual_dim // 8, 8).astype(np.uint8)
    packed = np.ascontiguousarray((bits << np.arange(8, dtype=np.uint8)).sum(axis=2, dtype=np.uint8))

    if isinstance(scale, str) and scale == "global":
        stored_scale = float(np.mean(np.abs(docs), dtype=np.float64))
    elif isinstance(scale, str) and scale in {"doc", "per_doc"}:
        stored_scale = _doc_mean_abs_scale(docs, offsets)
    elif scale is None:
        stored_scale = None
    else:
        stored_scale = _normalize_explicit_scale(scale, int(offsets.shape[0] - 1))

    result = PackedDocs(
        data=packed,
        doc_offsets=offsets,
        dim=actual_dim,
        num_docs=int(offsets.shape[0] - 1),
        scale=stored_scale,
        device="cpu",
        token_scale=_resolve_pack_token_scale(token_scale, docs),
    )
    return result if device == "cpu" else to_device(result, "cuda")


def _resolve_pack_token_scale(token_scale, docs: np.ndarray):
    """Token scale options of _api.py:80-103."""
    if token_scale is None:
        return None
    if isinstance(token_scale, str):
        mean_abs = lambda: np.mean(np.abs(docs), axis=1, dtype=np.float64).astype(np.float32)  # noqa: E731
        if token_scale == "mean_abs":
            return mean_abs()
        if token_scale == "l2":
            return (np.linalg.norm(docs.astype(np.float64), axis=1) / np.sqrt(docs.shape[1])).astype(np.float32)
        if token_scale == "mean_abs_fp16":
            return mean_abs().astype(np.float16).astype(np.float32)
        if token_scale == "mean_abs_u8":
            return _log_quantized_scales(mean_abs(), 256)
        if token_scale == "mean_abs_u4":
            return _log_quantized_scales(mean_abs(), 16)
        raise ValueError(
            "token_scale must be None, 'mean_abs', 'mean_abs_fp16', 'mean_abs_u8', 'mean_abs_u4', 'l2', or a [num_doc_tokens] vector"
        )
    values = np.ascontiguousarray(_as_numpy(token_scale), dtype=np.float32)
    if values.ndim != 1 or values.shape[0] != docs.shape[0]:
        raise ValueError("token_scale vector must have shape [num_doc_tokens]")
    return values


def _log_quantized_scales(scales: np.ndarray, levels: int) -> np.ndarray:
    """Log-spaced scale quantisation (_api.py:106-116)."""
    logs = np.log(np.maximum(scales.astype(np.float64), 1e-12))
    lo, hi = float(logs.min()), float(logs.max())
    if hi <= lo:
        return scales.astype(np.float32)
    steps = float(levels - 1)
    codes = np.clip(np.rint((logs - lo) * (steps / (hi - lo))), 0, steps)
    return np.exp(lo + codes * ((hi - lo) / steps)).astype(np.float32)


def _doc_mean_abs_scale(docs: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    scales = np.zeros(offsets.shape[0] - 1, dtype=np.float32)
    absdocs = np.abs(docs).astype(np.float32, copy=False)
    for i, (start, end) in enumerate(zip(offsets[:-1], offsets[1:])):
        if int(start) != int(end):
            scales[i] = np.float32(np.mean(absdocs[int(start) : int(end)], dtype=np.float64))
    return scales


def _normalize_explicit_scale(scale, num_docs: int):
    values = _as_numpy(scale)
    if values.ndim == 0:
        return float(values)
    normalized = np.ascontiguousarray(values, dtype=np.float32)
    if normalized.ndim != 1 or normalized.shape[0] != num_docs:
        raise ValueError("scale vector must have shape [num_docs]")
    return normalized


def _scale_is_vector(scale) -> bool:
    return isinstance(scale, np.ndarray)


def _resolve_scale(scale, packed: PackedDocs):
    """Effective per-call scale (_api.py:669-684)."""
    if scale is None:
        return 1.0 if packed.scale is None else packed.scale
    if isinstance(scale, str) and scale == "global":
        if packed.scale is None:
            raise ValueError("scale='global' requires a PackedDocs object with stored scale")
        if _scale_is_vector(packed.scale):
            raise ValueError("scale='global' requires a scalar stored scale")
        return float(packed.scale)
    if isinstance(scale, str) and scale in {"doc", "per_doc"}:
        if not _scale_is_vector(packed.scale):
            raise ValueError("scale='doc' requires a PackedDocs object with stored per-document scale")
        return packed.scale
    if isinstance(scale, str):
        raise ValueError("scale must be None, 'global', 'doc', a scalar, or a [num_docs] vector")
    return _normalize_explicit_scale(scale, packed.num_docs)


def _validate_packed(packed: PackedDocs) -> None:
    """Structural checks of _api.py:606-629."""
    if not isinstance(packed, PackedDocs):
        raise TypeError("packed must be a PackedDocs instance")
    if packed.dim % 8 != 0:
        raise ValueError("packed.dim must be divisible by 8")
    if isinstance(packed.scale, np.ndarray):
        if packed.scale.ndim != 1 or packed.scale.shape[0] != packed.num_docs:
            raise ValueError("packed.scale vector must have shape [num_docs]")
    elif packed.scale is not None:
        float(packed.scale)
    if packed.token_scale is not None:
        if not isinstance(packed.token_scale, np.ndarray):
            raise ValueError("packed.token_scale must be a [num_doc_tokens] vector or None")
        if packed.token_scale.ndim != 1 or packed.token_scale.shape[0] != int(packed.doc_offsets[-1]):
            raise ValueError("packed.token_scale must have shape [num_doc_tokens]")
    if packed.device == "cuda":
        if packed.doc_offsets.ndim != 1 or packed.doc_offsets.shape[0] != packed.num_docs + 1:
            raise ValueError("packed.doc_offsets must have shape [num_docs + 1]")
        return
    if packed.device != "cpu":
        raise ValueError("packed.device must be 'cpu' or 'cuda'")
    if packed.data.ndim != 2 or packed.data.shape[1] != packed.dim // 8:
        raise ValueError("packed.data must have shape [num_doc_tokens, dim / 8]")
    if packed.doc_offsets.ndim != 1 or packed.doc_offsets.shape[0] != packed.num_docs + 1:
        raise ValueError("packed.doc_offsets must have shape [num_docs + 1]")


def to_device(packed: PackedDocs, device: Literal["cpu", "cuda"] = "cuda") -> PackedDocs:
    """Upload a binary corpus to a device handle (_api.py:119-149)."""
    if device not in ("cpu", "cuda"):
        raise ValueError("device must be 'cpu' or 'cuda'")
    _validate_packed(packed)
    if device == packed.device:
        return packed
    if device == "cpu":
        raise NotImplementedError("copying CUDA PackedDocs back to CPU is not implemented")
    from maxsim_amd import _maxsim_hip

    offsets = np.ascontiguousarray(packed.doc_offsets, dtype=np.int64)
    handle = _maxsim_hip.CudaPackedDocs(np.ascontiguousarray(packed.data, dtype=np.uint8), offsets, packed.dim)
    stored_scale = packed.scale.copy() if isinstance(packed.scale, np.ndarray) else packed.scale
    if isinstance(stored_scale, np.ndarray):
        handle.set_scale_vector(np.ascontiguousarray(stored_scale, dtype=np.float32))
    stored_token_scale = packed.token_scale.copy() if isinstance(packed.token_scale, np.ndarray) else packed.token_scale
    if isinstance(stored_token_scale, np.ndarray):
        handle.set_token_scale_vector(np.ascontiguousarray(stored_token_scale, dtype=np.float32))
    return PackedDocs(handle, offsets.copy(), packed.dim, packed.num_docs, stored_scale, "cuda", stored_token_scale)


# -------------------------------------------------------------- scoring


def score(query_tokens, packed, *, reducer: Reducer = "maxsim", query_weights=None,
          temperature: float = 1.0, candidate_indices=None, scale=None, device="auto"):
    """Generalized reducer scoring for binary or int4 corpora (_api.py:152-200)."""
    if isinstance(packed, PackedDocs):
        return _score_binary(query_tokens, packed, scale=scale, device=device, reducer=reducer,
                             query_weights=query_weights, temperature=temperature,
                             candidate_indices=candidate_indices)
    from maxsim_amd.experimental import Int4PackedDocs, _int4_score

    if isinstance(packed, Int4PackedDocs):
        if scale is not None:
            raise ValueError("scale is stored by Int4PackedDocs and cannot be overridden")
        return _int4_score(query_tokens, packed, device=device, reducer=reducer,
                           query_weights=query_weights, temperature=temperature,
                           candidate_indices=candidate_indices, force_generalized=True)
    raise TypeError("packed must be a PackedDocs or Int4PackedDocs instance")


def maxsim(query_tokens, packed: PackedDocs, *, scale=None, device="auto", reducer: Reducer = "maxsim",
           query_weights=None, temperature: float = 1.0, candidate_indices=None):
    """Binary MaxSim / reducers (_api.py:203-224)."""
    return _score_binary(query_tokens, packed, scale=scale, device=device, reducer=reducer,
                         query_weights=query_weights, temperature=temperature,
                         candidate_indices=candidate_indices)


def _on_device(packed: PackedDocs, device) -> PackedDocs:
    _resolve_device(device)
    return packed if packed.device == "cuda" else to_device(packed, "cuda")


def _score_binary(query_tokens, packed: PackedDocs, *, scale, device, reducer, query_weights,
                  temperature, candidate_indices):
    """Binary scoring dispatch (_api.py:227-422), device only.

    Scale semantics: a scalar scale multiplies every doc score; a per-doc
    vector multiplies each doc's score; SmoothSim applies both before its
    log-sum-exp; token scales multiply each token similarity before reduction.
    """
    _validate_packed(packed)
    batches, squeeze = _query_batches(query_tokens, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    candidates = _normalize_candidate_indices(candidate_indices, packed.num_docs)
    targets = packed.num_docs if candidates is None else candidates.shape[0]
    shape = (batches.shape[0], targets)
    resolved_scale = _resolve_scale(scale, packed)
    if targets == 0 or batches.shape[0] == 0:
        result = np.empty(shape, np.float32)
        return result[0] if squeeze else result
    if batches.shape[1] == 0:
        result = np.zeros(shape, np.float32)
        return result[0] if squeeze else result
    resident = _on_device(packed, device)
    use_token_scale = isinstance(packed.token_scale, np.ndarray)
    vector = resolved_scale if _scale_is_vector(resolved_scale) else None
    kernel_scale = 1.0 if vector is not None else float(resolved_scale)
    query = np.ascontiguousarray(batches, dtype=np.float32)
    args = (reducer_value, weights, float(temperature_value), kernel_scale, False, use_token_scale, vector)
    if candidates is None:
        result = resident.data.score_batch(query, *args)
    else:
        result = resident.data.score_candidates_batch(query, candidates, *args)
    return result[0] if squeeze else result


def topk_maxsim(query_tokens, packed: PackedDocs, k: int, *, scale=None, device="auto",
                reducer: Reducer = "maxsim", query_weights=None, temperature: float = 1.0):
    """Top-k by (score desc, doc id asc) (_api.py:425-497).

    Integer-dtype queries whose entries are all +/-1 are sign-binarised and
    scored with XOR/popcount; the result equals the +/-1 float scoring.
    """
    if k < 1:
        raise ValueError("k must be >= 1")
    if k > packed.num_docs:
        raise ValueError("k cannot exceed packed.num_docs")
    _validate_packed(packed)
    query = _as_numpy(query_tokens)
    batches, squeeze = _query_batches(query, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    if batches.shape[0] == 0:
        return np.empty((0, k), np.float32), np.empty((0, k), np.int64)
    resolved_scale = _resolve_scale(scale, packed)
    resident = _on_device(packed, device)
    use_token_scale = isinstance(packed.token_scale, np.ndarray)
    if reducer_value == "maxsim" and not _scale_is_vector(resolved_scale):
        signs_only = (
            packed.dim == 128
            and np.issubdtype(query.dtype, np.integer)
            and not use_token_scale
            and float(resolved_scale) == 1.0
            and batches.shape[1] > 0
            and np.all(np.abs(query) == 1)
        )
        if signs_only:
            scores, indices = resident.data.topk_hamming(pack_query_signs(batches), int(k))
        else:
            scores, indices = resident.data.topk_batch(np.ascontiguousarray(batches, dtype=np.float32), int(k),
                                                       float(resolved_scale), False, use_token_scale)
        return (scores[0], indices[0]) if squeeze else (scores, indices)
    if batches.shape[1] == 0:
        zeros = np.zeros((batches.shape[0], packed.num_docs), np.float32)
        order = np.stack([_topk_indices_1d(row, k) for row in zeros])
        scores = np.take_along_axis(zeros, order, axis=1)
        return (scores[0], order[0]) if squeeze else (scores, order)
    # Any reducer: scores and the selection stay on the device.
    vector = resolved_scale if _scale_is_vector(resolved_scale) else None
    kernel_scale = 1.0 if vector is not None else float(resolved_scale)
    scores, indices = resident.data.topk_score_batch(np.ascontiguousarray(batches, dtype=np.float32), int(k),
                                                     reducer_value, weights, float(temperature_value), kernel_scale,
                                                     False, use_token_scale, vector)
    return (scores[0], indices[0]) if squeeze else (scores, indices)


def pack_query_signs(query) -> np.ndarray:
    """Sign bits of a [B, Q, D] query in pack_signs order (x >= 0 -> 1)."""
    q = np.asarray(query)
    bits = (q >= 0).reshape(*q.shape[:-1], q.shape[-1] // 8, 8).astype(np.uint8)
    return np.ascontiguousarray((bits << np.arange(8, dtype=np.uint8)).sum(axis=-1, dtype=np.uint8))
