"""Binary-prefix + int4-residual corpora.

The reference ships no such format (its cascade is int4 prefix + int4
residual, cascade.py:60-93); this module defines it:

* prefix: the sign bits of x (pack_signs order, x >= 0 -> 1) with one scale
  per token a_t = mean|x_t| (float64 mean, stored as float32) -- the scale
  that minimises the L1 error of a_t * sign(x_t);
* residual: r = x - a_t * sign(x) (float32), packed as per-token int4
  (pack_int4_symmetric, scale_granularity="token");
* 16 B signs + 4 B a_t + 64 B codes + 4 B residual scale = 88 B per token at
  dim 128.

Queries are quantised to int8 per row (sigma = max|q| / 127, as the int4
int8-query path); the fused scores (and a cascade's rescoring) can instead
take the fp32 query as three int8 limbs (query_precision="fp32").  Coarse
similarity a_t (q . sign_t); fused similarity a_t (q . sign_t) +
s^r_t (q . v^r_t), i.e. q . x'_t with x'_t = a_t sign_t + s^r_t v^r_t the
reconstructed token; both reduced with MaxSim.  The cascade takes the
coarse top-M per batch row, rescores them fused and returns the top-k (ties
by document id), all on the GPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from maxsim_amd._api import _as_numpy, _normalize_offsets
from maxsim_amd.cascade import DEVICE_TOPK_MAX_K, _stable_topk
from maxsim_amd.experimental import pack_int4_symmetric


@dataclass(frozen=True)
class BinaryResidualPackedDocs:
    sign_data: object               # u8 [T, dim / 8] (cpu) or the device handle
    prefix_scale: np.ndarray        # f32 [T], a_t
    residual_data: object           # u8 [T, dim / 2] (cpu) or the device handle
    residual_values: np.ndarray | None
    residual_token_scale: np.ndarray  # f32 [T]
    doc_offsets: np.ndarray
    dim: int
    num_docs: int
    device: str = "cpu"

    @property
    def num_tokens(self) -> int:
        return int(self.doc_offsets[-1])

    @property
    def storage_bytes(self) -> int:
        t = self.num_tokens
        return int(t * (self.dim // 8) + t * 4 + t * (self.dim // 2) + t * 4)


def pack_binary_residual(doc_embeddings, doc_offsets=None) -> BinaryResidualPackedDocs:
    docs = _as_numpy(doc_embeddings).astype(np.float32, copy=False)
    if docs.ndim != 2:
        raise ValueError("doc_embeddings must have shape [num_doc_tokens, dim]")
    if docs.shape[1] % 8 != 0:
        raise ValueError("dim must be divisible by 8")
    if not np.all(np.isfinite(docs)):
        raise ValueError("doc_embeddings must contain only finite values")
    offsets = _normalize_offsets(doc_offsets, docs.shape[0])
    dim = int(docs.shape[1])
    bits = (docs >= 0).reshape(docs.shape[0], dim // 8, 8).astype(np.uint8)
    signs = np.ascontiguousarray((bits << np.arange(8, dtype=np.uint8)).sum(axis=2, dtype=np.uint8))
    a = (np.add.reduce(np.abs(docs).astype(np.float64), axis=1) / dim).astype(np.float32)
    residual = (docs - np.where(docs >= 0, a[:, None], -a[:, None])).astype(np.float32)
    res = pack_int4_symmetric(residual, offsets, scale_granularity="token")
    return BinaryResidualPackedDocs(sign_data=signs, prefix_scale=np.ascontiguousarray(a),
                                    residual_data=res.data, residual_values=res.values,
                                    residual_token_scale=res.token_scale, doc_offsets=offsets, dim=dim,
                                    num_docs=int(offsets.shape[0] - 1), device="cpu")


def binres_to_device(packed: BinaryResidualPackedDocs, device: str = "cuda") -> BinaryResidualPackedDocs:
    if device != "cuda":
        raise ValueError("device must be 'cuda'")
    if packed.device == "cuda":
        return packed
    from maxsim_amd._maxsim_hip import CudaPackedDocs

    offsets = np.ascontiguousarray(packed.doc_offsets, dtype=np.int64)
    handle = CudaPackedDocs(np.ascontiguousarray(packed.sign_data, dtype=np.uint8), offsets, packed.dim)
    handle.set_token_scale_vector(np.ascontiguousarray(packed.prefix_scale, dtype=np.float32))
    handle.set_residual_int4(np.ascontiguousarray(packed.residual_data, dtype=np.uint8), 1.0,
                             np.ascontiguousarray(packed.residual_token_scale, dtype=np.float32))
    return BinaryResidualPackedDocs(sign_data=handle, prefix_scale=packed.prefix_scale.copy(),
                                    residual_data=handle, residual_values=None,
                                    residual_token_scale=packed.residual_token_scale.copy(), doc_offsets=offsets,
                                    dim=packed.dim, num_docs=packed.num_docs, device="cuda")


def _query(query_tokens, dim):
    q = _as_numpy(query_tokens).astype(np.float32, copy=False)
    squeeze = q.ndim == 2
    if squeeze:
        q = q[np.newaxis]
    if q.ndim != 3 or q.shape[2] != dim:
        raise ValueError("query_tokens must have shape [query_tokens, dim] or [batch, query_tokens, dim]")
    return np.ascontiguousarray(q), squeeze


_LIMBS = {"int8": 1, "fp32": 3}


class _RescorePrecision:
    """Sets the handle's rescoring query precision for one call."""

    def __init__(self, handle, query_precision):
        if query_precision not in _LIMBS:
            raise ValueError("query_precision must be 'int8' or 'fp32'")
        self.handle, self.limbs = handle, _LIMBS[query_precision]

    def __enter__(self):
        self.saved = self.handle.get_rescore_limbs()
        self.handle.set_rescore_limbs(self.limbs)

    def __exit__(self, *exc):
        self.handle.set_rescore_limbs(self.saved)


def binres_score(query_tokens, packed: BinaryResidualPackedDocs, *, fused: bool = True,
                 candidate_indices=None, query_precision: str = "int8") -> np.ndarray:
    """Coarse (fused=False) or fused scores; candidate_indices None or i64 [B, M].

    query_precision: the query of the fused scores, "int8" (one int8 limb) or
    "fp32" (three int8 limbs); the coarse scores always use the int8 query."""
    q, squeeze = _query(query_tokens, packed.dim)
    resident = binres_to_device(packed)
    cand = None if candidate_indices is None else np.asarray(candidate_indices, dtype=np.int64)
    if cand is not None and squeeze and cand.ndim == 1:
        cand = cand[np.newaxis]
    with _RescorePrecision(resident.sign_data, query_precision):
        out = resident.sign_data.binres_score_batch(q, fused=fused, candidate_indices=cand)
    return out[0] if squeeze else out


def _binres_topk(query_tokens, packed: BinaryResidualPackedDocs, k: int, *, query_precision: str = "int8"):
    """Top-k of the fused scores of every document (score desc, id asc),
    selected on the device: the same result as the stable top-k of
    ``binres_score(...)`` without the [B, N] scores leaving the device."""
    q, squeeze = _query(query_tokens, packed.dim)
    if q.shape[0] == 0 or q.shape[1] == 0 or k > DEVICE_TOPK_MAX_K:
        # Beyond the device selector's k: the stable top-k of the full fused
        # score rows, as the reference's residual search selects.
        return _stable_topk(binres_score(query_tokens, packed, query_precision=query_precision), k)
    resident = binres_to_device(packed)
    with _RescorePrecision(resident.sign_data, query_precision):
        scores, indices = resident.sign_data.binres_topk_batch(q, int(k))
    return (scores[0], indices[0]) if squeeze else (scores, indices)


def binres_cascade_topk(query_tokens, packed: BinaryResidualPackedDocs, k: int, *, candidates: int,
                        query_precision: str = "int8"):
    """Coarse top-``candidates`` -> fused rescoring -> top-k, on the GPU.

    query_precision: the rescoring pass's query ("int8" or "fp32"); the coarse
    pass uses the int8 query."""
    if k < 1 or k > candidates or candidates > packed.num_docs:
        raise ValueError("cascade sizes must satisfy 1 <= k <= candidates <= num_docs")
    q, squeeze = _query(query_tokens, packed.dim)
    resident = binres_to_device(packed)
    with _RescorePrecision(resident.sign_data, query_precision):
        scores, indices = resident.sign_data.cascade_topk(q, int(k), int(candidates))
    return (scores[0], indices[0]) if squeeze else (scores, indices)
