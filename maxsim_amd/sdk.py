"""Index / Reranker: the reference's product API (src/maxsim/sdk.py) over the GPU handles.

``Index.from_embeddings(doc_ids, embeddings, offsets, mode=...)`` packs a
corpus on the host; ``Reranker(index, device="cuda", int4_query=...)`` makes
it resident on the GPU once and ``search`` / ``rerank`` return
``SearchResult`` lists exactly as the reference formats them
(sdk.py:1134-1162).  Scoring never runs on the CPU: ``device="cpu"`` raises.

Modes: the reference's binary, binary_token_scale(_u8, _u4), pooled_binary,
int4, int4_per_token and int4_residual, plus ``binary_residual`` (sign-bit
prefix with a per-token scale + per-token int4 residual; see
``maxsim_amd.binres``).  Index files use the reference's .npz format
(``maxsim_amd.index_io``).  ``binary_q40`` is not provided.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Literal

import numpy as np

from maxsim_amd._api import PackedDocs, _as_numpy, maxsim, pack_signs, to_device, topk_maxsim
from maxsim_amd.binres import (
    BinaryResidualPackedDocs,
    _binres_topk,
    binres_cascade_topk,
    binres_score,
    binres_to_device,
    pack_binary_residual,
)
from maxsim_amd.cascade import (
    _residual_topk,
    cascade_topk,
    pack_residual_int4,
    residual_int4_to_device,
    residual_score,
)
from maxsim_amd.experimental import int4_maxsim, int4_to_device, pack_int4_symmetric, topk_int4_maxsim

MODES = (
    "binary",
    "binary_token_scale",
    "binary_token_scale_u8",
    "binary_token_scale_u4",
    "pooled_binary",
    "int4",
    "int4_per_token",
    "int4_residual",
    "binary_residual",
)
_BINARY_MODES = frozenset(MODES[:5])

# Named presets of sdk.py:46-52.
MODE_PRESETS = {
    "balanced": "binary_token_scale",
    "max_quality": "int4_per_token",
    "max_compression": "pooled_binary",
    "compact": "binary_token_scale_u4",
    "max_speed": "binary",
}


def resolve_auto_mode(num_docs: int, embeddings: np.ndarray | None = None) -> str:
    """The per-token int4 preset (sdk.py:56-59)."""
    del num_docs, embeddings
    return "int4_per_token"


@dataclass(frozen=True)
class CorpusMemoryReport:
    """Byte counts of an encoded corpus and of its current residency
    (reference: CorpusMemoryReport, sdk.py:62-70)."""

    encoded_bytes: int
    host_array_bytes: int
    device_index_bytes: int
    device_workspace_bytes: int | None
    serialized_bytes: int | None


@dataclass(frozen=True)
class SearchResult:
    doc_id: str
    score: float
    rank: int


@dataclass(frozen=True)
class Corpus:
    """Reference: Corpus / Index (sdk.py:81-470)."""

    doc_ids: tuple[str, ...]
    mode: str
    packed: PackedDocs | None = None
    int4_packed: object | None = None
    calibration: object | None = None
    metadata: dict[str, Any] | None = None
    _source_path: Path | None = field(default=None, repr=False, compare=False)

    @classmethod
    def from_embeddings(cls, doc_ids, embeddings, offsets, *, mode: str = "auto", pool_factor: int | None = None,
                        metadata: dict[str, Any] | None = None) -> "Corpus":
        requested = mode
        ids = _normalize_doc_ids(doc_ids)
        docs = _as_numpy(embeddings).astype(np.float32, copy=False)
        mode = resolve_auto_mode(len(ids), docs) if mode == "auto" else MODE_PRESETS.get(mode, mode)
        offs = _normalize_sdk_offsets(offsets, docs.shape[0])
        _validate_corpus_inputs(ids, docs, offs, mode)
        meta = {} if metadata is None else dict(metadata)
        if mode == "pooled_binary":
            from maxsim_amd.pooling import pool_doc_tokens

            factor = 3 if requested == "max_compression" and pool_factor is None else pool_factor
            factor = 2 if factor is None else factor
            if isinstance(factor, bool) or not isinstance(factor, (int, np.integer)) or int(factor) < 1:
                raise ValueError("pool_factor must be an integer >= 1")
            original = int(docs.shape[0])
            docs, offs = pool_doc_tokens(docs, offs, int(factor))
            meta.update({"pool_factor": int(factor), "original_tokens": original, "pooled_tokens": int(docs.shape[0])})
            return cls(doc_ids=ids, mode=mode, packed=pack_signs(docs, offs), metadata=meta)
        token_scales = {"binary": None, "binary_token_scale": "mean_abs_fp16", "binary_token_scale_u8": "mean_abs_u8",
                        "binary_token_scale_u4": "mean_abs_u4"}
        if mode in token_scales:
            return cls(doc_ids=ids, mode=mode, packed=pack_signs(docs, offs, token_scale=token_scales[mode]),
                       metadata=meta)
        if mode == "int4":
            return cls(doc_ids=ids, mode=mode, int4_packed=pack_int4_symmetric(docs, offs), metadata=meta)
        if mode == "int4_per_token":
            return cls(doc_ids=ids, mode=mode, metadata=meta,
                       int4_packed=pack_int4_symmetric(docs, offs, scale_granularity="token"))
        if mode == "int4_residual":
            return cls(doc_ids=ids, mode=mode, int4_packed=pack_residual_int4(docs, offs), metadata=meta)
        if mode == "binary_residual":
            return cls(doc_ids=ids, mode=mode, int4_packed=pack_binary_residual(docs, offs), metadata=meta)
        raise ValueError("unsupported corpus mode")  # unreachable: validated above

    @property
    def num_docs(self) -> int:
        return len(self.doc_ids)

    @property
    def dim(self) -> int:
        if self.packed is not None:
            return int(self.packed.dim)
        if self.int4_packed is not None:
            return int(self.int4_packed.dim)
        raise ValueError("corpus has no packed payload")

    @property
    def encoded_bytes(self) -> int:
        """Logical payload bytes (sdk.py:424-446)."""
        if self.packed is not None:
            extra = 0
            if isinstance(self.packed.scale, np.ndarray):
                extra += int(self.packed.scale.astype(np.float32, copy=False).nbytes)
            elif self.packed.scale is not None:
                extra += 4
            if self.packed.token_scale is not None:
                count = int(self.packed.token_scale.shape[0])
                if self.mode == "binary_token_scale_u8":
                    extra += count + 16
                elif self.mode == "binary_token_scale_u4":
                    extra += (count + 1) // 2 + 16
                else:
                    extra += count * 2
            return int(self.packed.doc_offsets[-1] * (self.packed.dim // 8) + extra)
        if self.int4_packed is not None:
            return int(self.int4_packed.storage_bytes)
        return 0

    @property
    def storage_bytes(self) -> int:
        return self.encoded_bytes

    def save(self, path) -> None:
        """Write the reference's .npz index format (sdk.py:203-288)."""
        from maxsim_amd.index_io import save_corpus

        written = save_corpus(self, path)
        object.__setattr__(self, "_source_path", Path(written).resolve())

    @classmethod
    def load(cls, path) -> "Corpus":
        """Read a .npz index of schema version 1 or 2 (sdk.py:290-410)."""
        from maxsim_amd.index_io import load_corpus

        corpus = load_corpus(path)
        object.__setattr__(corpus, "_source_path", Path(path).resolve())
        return corpus

    def memory_report(self, serialized_path=None) -> CorpusMemoryReport:
        """Logical size and current host / device residency (sdk.py:453-469).

        host_array_bytes counts the NumPy buffers the corpus owns (not Python
        object overhead); the device figures come from the resident handle's
        resident_bytes / workspace_bytes (0 for a host corpus);
        serialized_bytes is the size of the index file this corpus was saved
        to or loaded from, or of ``serialized_path``, else None."""
        source = self._source_path if serialized_path is None else Path(serialized_path)
        return CorpusMemoryReport(
            encoded_bytes=self.encoded_bytes,
            host_array_bytes=_corpus_host_array_bytes(self),
            device_index_bytes=_corpus_device_bytes(self, "resident_bytes"),
            device_workspace_bytes=_corpus_device_bytes(self, "workspace_bytes"),
            serialized_bytes=None if source is None else int(source.stat().st_size),
        )


Index = Corpus


class Reranker:
    """Reference: Reranker (sdk.py:472-635); the corpus is made resident on
    the GPU once, at construction."""

    def __init__(self, corpus: Corpus, *, device: Literal["cpu", "cuda"] = "cuda",
                 int4_query: Literal["fp32", "int8"] = "fp32"):
        if device not in {"cpu", "cuda"}:
            raise ValueError("device must be 'cpu' or 'cuda'")
        if int4_query not in {"fp32", "int8"}:
            raise ValueError("int4_query must be 'fp32' or 'int8'")
        if device == "cpu":
            raise NotImplementedError("maxsim_amd scores on the GPU only; use device='cuda'")
        if not isinstance(corpus, Corpus):
            raise TypeError("corpus must be a Corpus instance")
        self.corpus = _move_corpus(corpus)
        self.device = device
        self.int4_query = int4_query
        self._doc_index = {doc_id: idx for idx, doc_id in enumerate(self.corpus.doc_ids)}

    @classmethod
    def from_corpus(cls, corpus: Corpus, *, device: Literal["cpu", "cuda"] = "cuda",
                    int4_query: Literal["fp32", "int8"] = "fp32") -> "Reranker":
        return cls(corpus, device=device, int4_query=int4_query)

    @classmethod
    def load(cls, path, *, device: Literal["cpu", "cuda"] = "cuda",
             int4_query: Literal["fp32", "int8"] = "fp32") -> "Reranker":
        return cls.from_corpus(Corpus.load(path), device=device, int4_query=int4_query)

    def search(self, query_embeddings, *, k: int = 10, rescore_candidates: int | None = None,
               reducer: str = "maxsim", query_weights=None, temperature: float = 1.0):
        """Top-k documents per query (sdk.py:497-559)."""
        _validate_k(k, self.corpus.num_docs)
        kk = min(k, self.corpus.num_docs)
        mode = self.corpus.mode
        if rescore_candidates is not None and mode not in {"int4_residual", "binary_residual"}:
            raise ValueError("rescore_candidates requires corpus mode='int4_residual'")
        opts = dict(reducer=reducer, query_weights=query_weights, temperature=temperature)
        if mode in _BINARY_MODES:
            scores, indices = topk_maxsim(query_embeddings, self.corpus.packed, kk, device="auto", **opts)
        elif mode == "int4_residual":
            if rescore_candidates is None:
                scores, indices = _residual_topk(query_embeddings, self.corpus.int4_packed, kk, device="auto", **opts)
            else:
                scores, indices = cascade_topk(query_embeddings, self.corpus.int4_packed, kk,
                                               candidates=rescore_candidates, device="auto", **opts)
        elif mode == "binary_residual":
            _require_maxsim_reducer(mode, reducer, query_weights, temperature)
            if rescore_candidates is None:
                scores, indices = _binres_topk(query_embeddings, self.corpus.int4_packed, kk)
            else:
                scores, indices = binres_cascade_topk(query_embeddings, self.corpus.int4_packed, kk,
                                                      candidates=rescore_candidates)
        elif mode in {"int4", "int4_per_token"}:
            scores, indices = topk_int4_maxsim(query_embeddings, self.corpus.int4_packed, kk, device="auto",
                                               prefer_int8_query=self.int4_query == "int8", **opts)
        else:
            raise ValueError(f"unsupported corpus mode: {mode}")
        return _format_topk_results(scores, indices, self.corpus.doc_ids)

    def rerank(self, query_embeddings, candidate_ids, *, k: int = 10, reducer: str = "maxsim", query_weights=None,
               temperature: float = 1.0):
        """Score only the given documents (sdk.py:561-583)."""
        candidates = _dedupe_candidate_ids(candidate_ids)
        indices = self._candidate_indices(candidates)
        if not candidates:
            return []
        scores = self._score_candidates(query_embeddings, indices, reducer=reducer, query_weights=query_weights,
                                        temperature=temperature)
        positions = np.arange(len(candidates), dtype=np.int64)
        return _format_candidate_results(scores, positions, candidates, min(k, len(candidates)))

    def _score_candidates(self, query_embeddings, candidate_indices, *, reducer, query_weights, temperature):
        mode = self.corpus.mode
        opts = dict(device="auto", reducer=reducer, query_weights=query_weights, temperature=temperature,
                    candidate_indices=candidate_indices)
        if mode in _BINARY_MODES:
            return maxsim(query_embeddings, self.corpus.packed, **opts)
        if mode in {"int4", "int4_per_token"}:
            return int4_maxsim(query_embeddings, self.corpus.int4_packed, **opts)
        if mode == "int4_residual":
            return residual_score(query_embeddings, self.corpus.int4_packed, **opts)
        if mode == "binary_residual":
            _require_maxsim_reducer(mode, reducer, query_weights, temperature)
            q = _as_numpy(query_embeddings)
            rows = 1 if q.ndim == 2 else q.shape[0]
            cand = np.broadcast_to(np.asarray(candidate_indices, np.int64), (rows, len(candidate_indices)))
            return binres_score(q, self.corpus.int4_packed, candidate_indices=np.ascontiguousarray(cand))
        raise ValueError(f"unsupported corpus mode: {mode}")

    def _candidate_indices(self, candidate_ids: tuple[str, ...]) -> np.ndarray:
        out = []
        for doc_id in candidate_ids:
            try:
                out.append(self._doc_index[doc_id])
            except KeyError as exc:
                raise KeyError(doc_id) from exc
        return np.asarray(out, dtype=np.int64)


# NumPy fields of each payload type that a memory report counts
# (sdk.py:944-984 lists the reference's own payloads the same way).
_HOST_ARRAY_FIELDS = {
    "packed": ("data", "doc_offsets", "scale", "token_scale"),
    "int4": ("data", "values", "doc_offsets", "token_scale"),
    "int4_residual": ("prefix_data", "prefix_values", "prefix_token_scale", "residual_data", "residual_values",
                      "residual_token_scale", "doc_offsets"),
    "binary_residual": ("sign_data", "prefix_scale", "residual_data", "residual_values", "residual_token_scale",
                        "doc_offsets"),
}


def _corpus_payload(corpus: Corpus):
    """(payload, kind, device handle attribute) of a corpus."""
    if corpus.packed is not None:
        return corpus.packed, "packed", "data"
    if corpus.mode == "int4_residual":
        return corpus.int4_packed, "int4_residual", "prefix_data"
    if isinstance(corpus.int4_packed, BinaryResidualPackedDocs):
        return corpus.int4_packed, "binary_residual", "sign_data"
    return corpus.int4_packed, "int4", "data"


def _corpus_host_array_bytes(corpus: Corpus) -> int:
    payload, kind, _ = _corpus_payload(corpus)
    total = 0
    if payload is not None:
        for name in _HOST_ARRAY_FIELDS[kind]:
            value = getattr(payload, name, None)
            if isinstance(value, np.ndarray):
                total += int(value.nbytes)
    if corpus.calibration is not None:
        for name in ("thresholds", "negative_centroids", "positive_centroids"):
            value = getattr(corpus.calibration, name, None)
            if isinstance(value, np.ndarray):
                total += int(value.nbytes)
    return total


def _corpus_device_bytes(corpus: Corpus, accessor: str) -> int:
    payload, _, handle_name = _corpus_payload(corpus)
    if payload is None or getattr(payload, "device", "cpu") != "cuda":
        return 0
    return int(getattr(getattr(payload, handle_name), accessor))


def _move_corpus(corpus: Corpus) -> Corpus:
    """Resident copy of the corpus (sdk.py:1011-1045)."""
    if corpus.packed is not None:
        return Corpus(corpus.doc_ids, corpus.mode, to_device(corpus.packed, "cuda"), corpus.int4_packed,
                      corpus.calibration, corpus.metadata, corpus._source_path)
    if corpus.mode == "int4_residual":
        return Corpus(corpus.doc_ids, corpus.mode, None, residual_int4_to_device(corpus.int4_packed),
                      corpus.calibration, corpus.metadata, corpus._source_path)
    if isinstance(corpus.int4_packed, BinaryResidualPackedDocs):
        return Corpus(corpus.doc_ids, corpus.mode, None, binres_to_device(corpus.int4_packed), corpus.calibration,
                      corpus.metadata, corpus._source_path)
    if corpus.int4_packed is not None:
        return Corpus(corpus.doc_ids, corpus.mode, None, int4_to_device(corpus.int4_packed), corpus.calibration,
                      corpus.metadata, corpus._source_path)
    return corpus


def _normalize_doc_ids(doc_ids) -> tuple[str, ...]:
    values = tuple(str(d) for d in doc_ids)
    if not values:
        raise ValueError("doc_ids must contain at least one id")
    if len(set(values)) != len(values):
        raise ValueError("doc_ids must be unique")
    return values


def _normalize_sdk_offsets(offsets, num_tokens: int) -> np.ndarray:
    raw = _as_numpy(offsets)
    if not np.issubdtype(raw.dtype, np.integer):
        raise ValueError("offsets must contain integers")
    values = raw.astype(np.int64, copy=False)
    if values.ndim != 1 or values.shape[0] < 2:
        raise ValueError("offsets must have shape [num_docs + 1]")
    if int(values[0]) != 0 or int(values[-1]) != num_tokens:
        raise ValueError("offsets must span embeddings")
    if np.any(values[1:] < values[:-1]):
        raise ValueError("offsets must be monotonically nondecreasing")
    return values.copy()


def _validate_corpus_inputs(doc_ids, docs: np.ndarray, offsets: np.ndarray, mode: str) -> None:
    if docs.ndim != 2:
        raise ValueError("embeddings must have shape [total_doc_tokens, dim]")
    if docs.shape[1] % 8 != 0:
        raise ValueError("embedding dim must be divisible by 8")
    if offsets.shape[0] != len(doc_ids) + 1:
        raise ValueError("offsets must have one more entry than doc_ids")
    if mode == "binary_q40":
        raise NotImplementedError("corpus mode 'binary_q40' is not supported by maxsim_amd")
    if mode not in MODES:
        raise ValueError("mode must be 'auto', one of " + ", ".join(f"'{m}'" for m in MODES)
                         + f", or a preset in {sorted(MODE_PRESETS)}")


def _validate_k(k: int, max_count: int) -> None:
    if k < 1:
        raise ValueError("k must be >= 1")
    if max_count < 1:
        raise ValueError("corpus must contain at least one document")


def _require_maxsim_reducer(mode: str, reducer, query_weights, temperature) -> None:
    if reducer != "maxsim":
        raise ValueError(f"corpus mode '{mode}' currently supports only reducer='maxsim'")
    if query_weights is not None:
        raise ValueError("query_weights is only supported with reducer='weighted_maxsim'")
    try:
        value = float(temperature)
    except (TypeError, ValueError) as exc:
        raise ValueError("temperature must be a finite value greater than 0") from exc
    if not np.isfinite(value) or value <= 0.0:
        raise ValueError("temperature must be a finite value greater than 0")


def _dedupe_candidate_ids(candidate_ids) -> tuple[str, ...]:
    seen, out = set(), []
    for c in candidate_ids:
        v = str(c)
        if v not in seen:
            seen.add(v)
            out.append(v)
    return tuple(out)


def _format_topk_results(scores, indices, doc_ids):
    s = np.asarray(scores, dtype=np.float32)
    i = np.asarray(indices, dtype=np.int64)
    if i.size and int(i.min()) < 0:
        raise RuntimeError("top-k selection returned no document for some rank (a device selection gave up)")
    # Python floats and ints once per array (tolist), not per numpy scalar.
    if s.ndim == 1:
        return _format_result_row(s.tolist(), i.tolist(), doc_ids)
    return [_format_result_row(rs, ri, doc_ids) for rs, ri in zip(s.tolist(), i.tolist())]


def _format_candidate_results(scores, candidate_indices, candidate_ids, k: int):
    s = np.asarray(scores, dtype=np.float32)
    if s.ndim == 1:
        return _format_candidate_row(s, candidate_indices, candidate_ids, k)
    return [_format_candidate_row(row, candidate_indices, candidate_ids, k) for row in s]


def _format_candidate_row(scores, candidate_indices, candidate_ids, k: int):
    cs = scores[candidate_indices]
    order = np.lexsort((np.arange(cs.shape[0], dtype=np.int64), -cs))[:k]
    return [SearchResult(doc_id=candidate_ids[int(p)], score=float(cs[int(p)]), rank=r)
            for r, p in enumerate(order, start=1)]


_new_object = object.__new__
_set_attribute = object.__setattr__


def _format_result_row(scores, indices, doc_ids):
    # The frozen dataclass's fields set in one step (its generated __init__
    # sets them one by one through object.__setattr__, about twice the time
    # per result); the objects are the same SearchResult values.
    out = []
    for rank, (score, index) in enumerate(zip(scores, indices), start=1):
        result = _new_object(SearchResult)
        _set_attribute(result, "__dict__", {"doc_id": doc_ids[index], "score": score, "rank": rank})
        out.append(result)
    return out
