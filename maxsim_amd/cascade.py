"""Residual int4 corpora and the coarse -> fine cascade (reference: src/maxsim/cascade.py).

Storage: per token a per-token int4 prefix of x and a per-token int4 residual
of x - prefix_reconstruction (cascade.py:60-93).  Scoring is GPU-only: the
fused similarity p s^p_t (q . v^p_t) + r s^r_t (q . v^r_t) is reduced once
(not as two separately reduced streams), and ``cascade_topk`` keeps the
coarse scores, the top-M candidate lists and the rescoring on the device
(the reference copies the coarse matrix to the host and loops over batch rows).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from maxsim_amd._api import _as_numpy, _normalize_candidate_indices, _normalize_reducer_options, _resolve_device
from maxsim_amd.experimental import (
    Int4PackedDocs,
    _pack_signed_int4_values,
    _validate_int4_data_matches_values,
    _validate_int4_packed,
    int4_maxsim,
    int4_to_device,
    pack_int4_symmetric,
    topk_int4_maxsim,
)

_NATIVE_PREFIX_TOPK_LIMIT = 32


@dataclass(frozen=True)
class ResidualInt4PackedDocs:
    """Reference: ResidualInt4PackedDocs (cascade.py:27-57)."""

    prefix_data: object
    prefix_values: np.ndarray | None
    prefix_scale: float
    prefix_token_scale: np.ndarray
    residual_data: object
    residual_values: np.ndarray | None
    residual_scale: float
    residual_token_scale: np.ndarray
    doc_offsets: np.ndarray
    dim: int
    num_docs: int
    device: str = "cpu"

    @property
    def num_tokens(self) -> int:
        return int(self.doc_offsets[-1])

    @property
    def storage_bytes(self) -> int:
        code_bytes = self.num_tokens * self.dim // 2
        prefix = self.prefix_data.nbytes if isinstance(self.prefix_data, np.ndarray) else code_bytes
        residual = self.residual_data.nbytes if isinstance(self.residual_data, np.ndarray) else code_bytes
        return int(prefix + residual + 8 + self.prefix_token_scale.nbytes + self.residual_token_scale.nbytes)


def _reconstruct_int4(values, scale, token_scale) -> np.ndarray:
    if values is None:
        raise ValueError("CPU reconstruction requires unpacked int4 values")
    return values.astype(np.float32, copy=False) * np.float32(scale) * token_scale[:, np.newaxis]


def pack_residual_int4(doc_embeddings, doc_offsets=None) -> ResidualInt4PackedDocs:
    """Prefix = per-token int4 of x; residual = per-token int4 of x - prefix (cascade.py:60-93)."""
    docs = _as_numpy(doc_embeddings).astype(np.float32, copy=False)
    prefix = pack_int4_symmetric(docs, doc_offsets, scale_granularity="token")
    residual = np.asarray(docs - _reconstruct_int4(prefix.values, prefix.scale, prefix.token_scale), np.float32)
    res = pack_int4_symmetric(residual, prefix.doc_offsets, scale_granularity="token")
    packed = ResidualInt4PackedDocs(
        prefix_data=prefix.data, prefix_values=prefix.values, prefix_scale=prefix.scale,
        prefix_token_scale=prefix.token_scale, residual_data=res.data, residual_values=res.values,
        residual_scale=res.scale, residual_token_scale=res.token_scale, doc_offsets=prefix.doc_offsets,
        dim=prefix.dim, num_docs=prefix.num_docs, device="cpu")
    _validate_residual_packed(packed)
    return packed


def _prefix_view(packed: ResidualInt4PackedDocs) -> Int4PackedDocs:
    return Int4PackedDocs(data=packed.prefix_data, values=packed.prefix_values, doc_offsets=packed.doc_offsets,
                          dim=packed.dim, num_docs=packed.num_docs, scale=packed.prefix_scale,
                          device=packed.device, token_scale=packed.prefix_token_scale)


def residual_int4_to_device(packed: ResidualInt4PackedDocs, device: str = "cuda") -> ResidualInt4PackedDocs:
    """Upload both streams into one device handle (cascade.py:96-130)."""
    if device != "cuda":
        raise ValueError("device must be 'cuda'")
    _validate_residual_packed(packed, verify_packed_values=True)
    if packed.device == "cuda":
        return packed
    cuda_prefix = int4_to_device(_prefix_view(packed))
    cuda_prefix.data.set_residual_int4(np.ascontiguousarray(packed.residual_data, dtype=np.uint8),
                                       float(packed.residual_scale),
                                       np.ascontiguousarray(packed.residual_token_scale, dtype=np.float32))
    return ResidualInt4PackedDocs(
        prefix_data=cuda_prefix.data, prefix_values=None, prefix_scale=cuda_prefix.scale,
        prefix_token_scale=cuda_prefix.token_scale, residual_data=cuda_prefix.data, residual_values=None,
        residual_scale=packed.residual_scale, residual_token_scale=packed.residual_token_scale.copy(),
        doc_offsets=packed.doc_offsets.copy(), dim=packed.dim, num_docs=packed.num_docs, device="cuda")


def _on_device(packed: ResidualInt4PackedDocs, device) -> ResidualInt4PackedDocs:
    _resolve_device(device)
    return packed if packed.device == "cuda" else residual_int4_to_device(packed)


def prefix_score(query_tokens, packed: ResidualInt4PackedDocs, *, device: str = "auto", reducer: str = "maxsim",
                 query_weights=None, temperature: float = 1.0, candidate_indices=None) -> np.ndarray:
    """Coarse scores from the prefix stream alone (cascade.py:133-154)."""
    _validate_residual_packed(packed)
    batches, squeeze = _normalize_query(query_tokens, packed.dim)
    return int4_maxsim(batches[0] if squeeze else batches, _prefix_view(packed), device=device, reducer=reducer,
                       query_weights=query_weights, temperature=temperature, candidate_indices=candidate_indices)


def prefix_topk(query_tokens, packed: ResidualInt4PackedDocs, k: int, *, device: str = "auto",
                reducer: str = "maxsim", query_weights=None, temperature: float = 1.0):
    """Prefix top-k with stable ties (cascade.py:157-193); selection on the device."""
    _validate_residual_packed(packed)
    if not isinstance(k, (int, np.integer)) or isinstance(k, (bool, np.bool_)):
        raise ValueError("k must be an integer")
    if k < 1 or k > packed.num_docs:
        raise ValueError("k must satisfy 1 <= k <= num_docs")
    batches, squeeze = _normalize_query(query_tokens, packed.dim)
    query = batches[0] if squeeze else batches
    if k <= _NATIVE_PREFIX_TOPK_LIMIT:
        return topk_int4_maxsim(query, _prefix_view(packed), k, device=device, reducer=reducer,
                                query_weights=query_weights, temperature=temperature)
    scores = prefix_score(query, packed, device=device, reducer=reducer, query_weights=query_weights,
                          temperature=temperature)
    return _stable_topk(scores, k)


def residual_score(query_tokens, packed: ResidualInt4PackedDocs, *, device: str = "auto", reducer: str = "maxsim",
                   query_weights=None, temperature: float = 1.0, candidate_indices=None) -> np.ndarray:
    """Fused prefix + residual scores (cascade.py:196-291)."""
    _validate_residual_packed(packed)
    batches, squeeze = _normalize_query(query_tokens, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    candidates = _normalize_candidate_indices(candidate_indices, packed.num_docs)
    targets = packed.num_docs if candidates is None else int(candidates.shape[0])
    shape = (batches.shape[0], targets)
    if batches.shape[0] == 0 or targets == 0:
        result = np.empty(shape, np.float32)
        return result[0] if squeeze else result
    if batches.shape[1] == 0:
        result = np.zeros(shape, np.float32)
        return result[0] if squeeze else result
    resident = _on_device(packed, device)
    query = np.ascontiguousarray(batches, dtype=np.float32)
    if candidates is None:
        result = resident.prefix_data.score_residual_batch(query, reducer_value, weights, float(temperature_value))
    else:
        result = resident.prefix_data.score_residual_candidates_batch(query, candidates, reducer_value, weights,
                                                                      float(temperature_value))
    return result[0] if squeeze else result


# Largest k the device selectors take (msim_*_topk_* entry points).
DEVICE_TOPK_MAX_K = 4096


def _residual_topk(query_tokens, packed: ResidualInt4PackedDocs, k: int, *, device: str = "auto",
                   reducer: str = "maxsim", query_weights=None, temperature: float = 1.0):
    """Top-k of the fused scores over every document, selected on the device:
    the same result as ``_stable_topk(residual_score(...), k)`` (score desc,
    document id asc; the sdk's full residual search, sdk.py:497-559) without
    bringing the [B, N] scores to the host."""
    _validate_residual_packed(packed)
    batches, squeeze = _normalize_query(query_tokens, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    if batches.shape[0] == 0 or batches.shape[1] == 0 or k > DEVICE_TOPK_MAX_K:
        # Beyond the device selector's k: the reference's own route for this
        # mode, the stable top-k of the full fused score rows (sdk.py:523-533).
        return _stable_topk(residual_score(query_tokens, packed, device=device, reducer=reducer,
                                           query_weights=query_weights, temperature=temperature), k)
    resident = _on_device(packed, device)
    scores, indices = resident.prefix_data.topk_score_batch(np.ascontiguousarray(batches, dtype=np.float32), int(k),
                                                            reducer_value, weights, float(temperature_value),
                                                            residual=True)
    return (scores[0], indices[0]) if squeeze else (scores, indices)


def cascade_topk(query_tokens, packed: ResidualInt4PackedDocs, k: int, *, candidates: int, device: str = "auto",
                 reducer: str = "maxsim", query_weights=None, temperature: float = 1.0):
    """Prefix top-``candidates`` -> fused rescoring -> top-k (cascade.py:294-393).

    Same result contract as the reference: coarse candidates by (prefix score
    desc, id asc), final order by (fused score desc, document id asc); with
    ``candidates == num_docs`` the full fused top-k.  All stages run on the
    device in one call.
    """
    _validate_residual_packed(packed)
    if device not in {"auto", "cpu", "cuda"}:
        raise ValueError("device must be 'auto', 'cpu', or 'cuda'")
    if not isinstance(k, (int, np.integer)) or isinstance(k, (bool, np.bool_)):
        raise ValueError("k must be an integer")
    if not isinstance(candidates, (int, np.integer)) or isinstance(candidates, (bool, np.bool_)):
        raise ValueError("candidates must be an integer")
    if k < 1 or k > candidates or candidates > packed.num_docs:
        raise ValueError("cascade sizes must satisfy 1 <= k <= candidates <= num_docs")
    batches, squeeze = _normalize_query(query_tokens, packed.dim)
    _reducer, weights, _temperature = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    if batches.shape[0] == 0:
        return np.empty((0, k), np.float32), np.empty((0, k), np.int64)
    resident = _on_device(packed, device)
    scores, indices = resident.prefix_data.cascade_topk(np.ascontiguousarray(batches, np.float32), int(k),
                                                        int(candidates), _reducer, weights, float(_temperature))
    return (scores[0], indices[0]) if squeeze else (scores, indices)


def _stable_topk(scores: np.ndarray, k: int):
    values = np.asarray(scores, dtype=np.float32)
    if values.ndim == 1:
        idx = _stable_topk_indices(values, k)
        return values[idx], idx
    if values.shape[0] == 0:
        return np.empty((0, k), np.float32), np.empty((0, k), np.int64)
    idx = np.stack([_stable_topk_indices(row, k) for row in values])
    return np.take_along_axis(values, idx, axis=1), idx


def _stable_topk_indices(scores: np.ndarray, k: int, *, tie_ids=None) -> np.ndarray:
    """(score desc, tie id asc) (cascade.py:436-453)."""
    positions = np.arange(scores.shape[0], dtype=np.int64)
    ids = positions if tie_ids is None else np.asarray(tie_ids, dtype=np.int64)
    order = np.lexsort((ids, -scores))[:k]
    return np.ascontiguousarray(positions[order], dtype=np.int64)


def _normalize_query(query_tokens, dim: int):
    """[dim], [Q, dim] or [B, Q, dim] (cascade.py:497-517)."""
    query = _as_numpy(query_tokens).astype(np.float32, copy=False)
    if query.ndim == 1:
        batches, squeeze = query[np.newaxis, np.newaxis, :], True
    elif query.ndim == 2:
        batches, squeeze = query[np.newaxis, :, :], True
    elif query.ndim == 3:
        batches, squeeze = query, False
    else:
        raise ValueError("query_tokens must have shape [dim], [query_tokens, dim], or [batch, query_tokens, dim]")
    if batches.shape[2] != dim:
        raise ValueError(f"query dim={batches.shape[2]} does not match packed dim={dim}")
    if not np.all(np.isfinite(batches)):
        raise ValueError("query_tokens must contain only finite values")
    return np.ascontiguousarray(batches, dtype=np.float32), squeeze


def _validate_residual_packed(packed, *, verify_packed_values: bool = False) -> None:
    """Structural checks of cascade.py:520-600 (same messages)."""
    if not isinstance(packed, ResidualInt4PackedDocs):
        raise TypeError("packed must be a ResidualInt4PackedDocs instance")
    prefix = _prefix_view(packed)
    _validate_int4_packed(prefix)
    if verify_packed_values:
        _validate_int4_data_matches_values(prefix)
    if packed.prefix_token_scale is None:
        raise ValueError("prefix_token_scale must have shape [num_doc_tokens]")
    if packed.device == "cpu":
        if not isinstance(packed.residual_data, np.ndarray):
            raise ValueError("CPU residual_data must be a NumPy array")
        if packed.residual_data.dtype != np.uint8:
            raise ValueError("CPU residual_data must have dtype uint8")
        if packed.residual_data.shape != (packed.num_tokens, packed.dim // 2):
            raise ValueError("residual_data must have shape [num_doc_tokens, dim / 2]")
        if not isinstance(packed.residual_values, np.ndarray):
            raise ValueError("CPU residual_values must be a NumPy array")
        if packed.residual_values.shape != (packed.num_tokens, packed.dim):
            raise ValueError("residual_values must have shape [num_doc_tokens, dim]")
        if packed.residual_values.dtype != np.int8:
            raise ValueError("residual_values must have dtype int8")
        if np.any(packed.residual_values < -7) or np.any(packed.residual_values > 7):
            raise ValueError("residual_values must be symmetric int4 values in [-7, 7]")
        if verify_packed_values and not np.array_equal(packed.residual_data,
                                                       _pack_signed_int4_values(packed.residual_values)):
            raise ValueError("residual_data does not encode residual_values")
    elif packed.device == "cuda":
        if packed.residual_values is not None:
            raise ValueError("CUDA residual_values must be None")
        if packed.prefix_data is not packed.residual_data:
            raise ValueError("CUDA prefix_data and residual_data must share one handle")
        handle = packed.prefix_data
        for name, expected in (("dim", packed.dim), ("num_docs", packed.num_docs),
                               ("num_tokens", packed.num_tokens)):
            actual = getattr(handle, name, None)
            if actual is None or int(actual) != int(expected):
                raise ValueError(f"CUDA residual handle {name} does not match metadata")
        if getattr(handle, "has_token_scale_vector", None) is not True:
            raise ValueError("CUDA residual handle is missing prefix token scales")
        if getattr(handle, "has_residual_int4", None) is not True:
            raise ValueError("CUDA residual handle is missing residual int4 data")
    else:
        raise ValueError("device must be 'cpu' or 'cuda'")
    try:
        residual_scale = float(packed.residual_scale)
    except (TypeError, ValueError) as exc:
        raise ValueError("residual_scale must be a finite scalar > 0") from exc
    if not np.isfinite(residual_scale) or residual_scale <= 0.0:
        raise ValueError("residual_scale must be a finite scalar > 0")
    ts = packed.residual_token_scale
    if not isinstance(ts, np.ndarray) or ts.ndim != 1 or ts.shape[0] != packed.num_tokens:
        raise ValueError("residual_token_scale must have shape [num_doc_tokens]")
    if ts.dtype != np.float32:
        raise ValueError("residual_token_scale must have dtype float32")
    if not np.all(np.isfinite(ts)) or np.any(ts <= 0.0):
        raise ValueError("residual_token_scale values must be finite and > 0")
