"""Int4 corpus format and int4 scoring dispatch (reference: src/maxsim/experimental.py).

Packing is host NumPy (offline index build, as in the reference), with a GPU
packer beside it (``pack_int4_symmetric_device``, same result).  Scoring
always runs on the GPU: CPU-resident packed docs are uploaded to a device
handle first; ``device="cpu"`` is rejected because this engine has no CPU
scoring path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from maxsim_amd._api import (
    _as_numpy,
    _normalize_candidate_indices,
    _normalize_offsets,
    _normalize_reducer_options,
    _query_batches,
    _resolve_device,
)


@dataclass(frozen=True)
class Int4PackedDocs:
    """Reference: Int4PackedDocs (experimental.py:48-66)."""

    data: object
    values: np.ndarray | None
    doc_offsets: np.ndarray
    dim: int
    num_docs: int
    scale: float
    device: str = "cpu"
    token_scale: np.ndarray | None = None

    @property
    def storage_bytes(self) -> int:
        if isinstance(self.data, np.ndarray):
            code_bytes = int(self.data.nbytes)
        else:
            code_bytes = int(getattr(self.data, "packed_size", 0))
        return code_bytes + 4 + (0 if self.token_scale is None else int(self.token_scale.nbytes))


def _pack_signed_int4_values(values: np.ndarray) -> np.ndarray:
    """Two's-complement nibbles, even dim in the low nibble (experimental.py:604-609)."""
    v = values.astype(np.int16)
    return np.ascontiguousarray(((v[:, 0::2] & 0x0F) | ((v[:, 1::2] & 0x0F) << 4)).astype(np.uint8))


def _unpack_signed_int4_data(data: np.ndarray, dim: int) -> np.ndarray:
    """Inverse of _pack_signed_int4_values (sdk.py:1085-1093)."""
    low = (data & 0x0F).astype(np.int8)
    high = (data >> 4).astype(np.int8)
    values = np.empty((data.shape[0], dim), np.int8)
    values[:, 0::2] = np.where(low >= 8, low - 16, low)
    values[:, 1::2] = np.where(high >= 8, high - 16, high)
    return values


def pack_int4_symmetric(doc_embeddings, doc_offsets=None, *, scale: float | None = None,
                        scale_granularity: str = "tensor") -> Int4PackedDocs:
    """Symmetric int4 packing (experimental.py:218-268).

    token granularity: s_t = f32(max|x_t|) / f32(7) (zero rows -> 1.0), values
    clip(rint(x / s_t), -7, 7), tensor scale 1.0.  tensor granularity: one scale
    max|x| / 7 (or the given one) for the whole corpus.
    """
    docs = _as_numpy(doc_embeddings).astype(np.float32, copy=False)
    if docs.ndim != 2:
        raise ValueError("doc_embeddings must have shape [num_doc_tokens, dim]")
    if docs.shape[1] <= 0:
        raise ValueError("dim must be positive")
    if docs.shape[1] % 2 != 0:
        raise ValueError("dim must be divisible by 2 for int4 packing")
    if docs.shape[1] % 8 != 0:
        raise ValueError("dim must be divisible by 8")
    if not np.all(np.isfinite(docs)):
        raise ValueError("doc_embeddings must contain only finite values")
    if scale_granularity not in {"tensor", "token"}:
        raise ValueError("scale_granularity must be 'tensor' or 'token'")

    token_scale = None
    if scale_granularity == "token":
        if scale is not None:
            raise ValueError("scale cannot be provided when scale_granularity='token'")
        token_scale = np.max(np.abs(docs), axis=1).astype(np.float32) / np.float32(7.0)
        token_scale[token_scale == 0.0] = np.float32(1.0)
        scale_value = 1.0
        values = np.clip(np.rint(docs / token_scale[:, None]), -7, 7).astype(np.int8)
    else:
        if scale is None:
            peak = float(np.max(np.abs(docs))) if docs.size else 0.0
            scale_value = 1.0 if peak == 0.0 else peak / 7.0
        else:
            scale_value = float(scale)
            if not np.isfinite(scale_value) or scale_value <= 0.0:
                raise ValueError("scale must be finite and > 0")
        values = np.clip(np.rint(docs / np.float32(scale_value)), -7, 7).astype(np.int8)

    offsets = _normalize_offsets(doc_offsets, docs.shape[0])
    return Int4PackedDocs(
        data=_pack_signed_int4_values(values),
        values=np.ascontiguousarray(values),
        doc_offsets=offsets,
        dim=int(docs.shape[1]),
        num_docs=int(offsets.shape[0] - 1),
        scale=scale_value,
        device="cpu",
        token_scale=token_scale,
    )


def pack_int4_symmetric_device(doc_embeddings, doc_offsets=None, *, scale: float | None = None,
                               scale_granularity: str = "tensor", values: bool = True) -> Int4PackedDocs:
    """pack_int4_symmetric on the GPU (msim_pack_int4 / msim_pack_int4_async):
    the same arguments, checks, messages and result, bit for bit, for a fast
    index build.  A torch CUDA tensor is packed in place on its device (no
    host copy of the embeddings); other inputs are uploaded.  ``values=False``
    skips the int8 values array (``values`` is then None).
    """
    from maxsim_amd import _native

    granularity = {"tensor": 0, "token": 1}.get(scale_granularity, -1)
    scale_arg = 0.0 if scale is None else float(scale)
    if scale is not None and scale_arg == 0.0:
        scale_arg = -1.0  # an explicit 0 is invalid (0 means None in the C ABI)
    lib = _native.load()
    is_cuda = getattr(doc_embeddings, "is_cuda", False)
    if is_cuda:
        import torch

        x = doc_embeddings.detach()
        if x.ndim != 2:
            raise ValueError("doc_embeddings must have shape [num_doc_tokens, dim]")
        x = x.to(torch.float32).contiguous()
        t, d = int(x.shape[0]), int(x.shape[1])
        if d <= 0:
            raise ValueError("dim must be positive")
        if d % 2 != 0:
            raise ValueError("dim must be divisible by 2 for int4 packing")
        if d % 8 != 0:
            raise ValueError("dim must be divisible by 8")
        codes = torch.empty((t, d // 2), dtype=torch.uint8, device=x.device)
        tscale = torch.empty((t,), dtype=torch.float32, device=x.device)
        vals = torch.empty((t, d), dtype=torch.int8, device=x.device) if values else None
        work = torch.zeros(2, dtype=torch.int32, device=x.device)
        if granularity not in (0, 1) or (granularity == 1 and scale is not None) or \
                (granularity == 0 and scale is not None and not (np.isfinite(scale_arg) and scale_arg > 0.0)):
            # Finiteness is checked first, as the host packer does.
            if not bool(torch.isfinite(x).all()):
                raise ValueError("doc_embeddings must contain only finite values")
        stream = torch.cuda.current_stream(x.device).cuda_stream
        with torch.cuda.device(x.device):
            _native.check(lib.msim_pack_int4_async(_native.ptr(x), t, d, granularity, scale_arg, _native.ptr(codes),
                                                   _native.ptr(tscale), _native.ptr(vals), _native.ptr(work),
                                                   ctypes.c_void_p(stream)))
            w = work.cpu().numpy().view(np.uint32)
        if w[1] != 0:
            raise ValueError("doc_embeddings must contain only finite values")
        if granularity == 1:
            scale_value = 1.0
        elif scale is not None:
            scale_value = scale_arg
        else:
            peak = float(w[:1].view(np.float32)[0])
            scale_value = 1.0 if peak == 0.0 else peak / 7.0
        data = codes.cpu().numpy()
        token_scale = tscale.cpu().numpy() if granularity == 1 else None
        values_np = vals.cpu().numpy() if vals is not None else None
    else:
        docs = np.ascontiguousarray(_as_numpy(doc_embeddings), dtype=np.float32)
        if docs.ndim != 2:
            raise ValueError("doc_embeddings must have shape [num_doc_tokens, dim]")
        t, d = int(docs.shape[0]), int(docs.shape[1])
        data = np.empty((t, max(d, 0) // 2), np.uint8)
        token_scale = np.empty((t,), np.float32) if scale_granularity == "token" else None
        values_np = np.empty((t, d), np.int8) if values else None
        out_scale = ctypes.c_double(0.0)
        _native.check(lib.msim_pack_int4(_native.ptr(docs), t, d, granularity, scale_arg, _native.ptr(data),
                                         _native.ptr(token_scale), _native.ptr(values_np), ctypes.byref(out_scale)))
        scale_value = float(out_scale.value)
    offsets = _normalize_offsets(doc_offsets, t)
    return Int4PackedDocs(
        data=data,
        values=values_np,
        doc_offsets=offsets,
        dim=d,
        num_docs=int(offsets.shape[0] - 1),
        scale=scale_value,
        device="cpu",
        token_scale=token_scale,
    )


def _device_module():
    from maxsim_amd import _maxsim_hip

    return _maxsim_hip


def int4_to_device(packed: Int4PackedDocs, device: str = "cuda") -> Int4PackedDocs:
    """Upload codes, offsets and token scales once (experimental.py:271-305)."""
    if device != "cuda":
        raise ValueError("device must be 'cuda'")
    _validate_int4_packed(packed)
    if packed.device == "cuda":
        return packed
    _validate_int4_data_matches_values(packed)
    handle = _device_module().CudaInt4PackedDocs(
        np.ascontiguousarray(packed.data, dtype=np.uint8),
        np.ascontiguousarray(packed.doc_offsets, dtype=np.int64),
        packed.dim,
        float(packed.scale),
    )
    token_scale = None if packed.token_scale is None else packed.token_scale.copy()
    if token_scale is not None:
        handle.set_token_scale_vector(np.ascontiguousarray(token_scale, dtype=np.float32))
    return Int4PackedDocs(
        data=handle,
        values=None,
        doc_offsets=packed.doc_offsets.copy(),
        dim=packed.dim,
        num_docs=packed.num_docs,
        scale=packed.scale,
        device="cuda",
        token_scale=token_scale,
    )


def _on_device(packed: Int4PackedDocs, device) -> Int4PackedDocs:
    _resolve_device(device)
    return packed if packed.device == "cuda" else int4_to_device(packed)


def int4_maxsim(query_tokens, packed: Int4PackedDocs, *, device="auto", reducer="maxsim",
                query_weights=None, temperature: float = 1.0, candidate_indices=None) -> np.ndarray:
    """int4 scoring with a reducer (experimental.py:308-327)."""
    return _int4_score(query_tokens, packed, device=device, reducer=reducer,
                       query_weights=query_weights, temperature=temperature,
                       candidate_indices=candidate_indices, force_generalized=False)


def _int4_score(query_tokens, packed: Int4PackedDocs, *, device, reducer, query_weights,
                temperature, candidate_indices, force_generalized: bool) -> np.ndarray:
    """Dispatch of experimental.py:330-420 onto the device handle."""
    _validate_int4_packed(packed)
    batches, squeeze = _query_batches(query_tokens, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    candidates = _normalize_candidate_indices(candidate_indices, packed.num_docs)
    targets = packed.num_docs if candidates is None else candidates.shape[0]
    shape = (batches.shape[0], targets)
    if targets == 0 or batches.shape[0] == 0:
        result = np.empty(shape, np.float32)
        return result[0] if squeeze else result
    if batches.shape[1] == 0:
        result = np.zeros(shape, np.float32)
        return result[0] if squeeze else result
    resident = _on_device(packed, device)
    query = np.ascontiguousarray(batches, dtype=np.float32)
    if force_generalized or reducer_value != "maxsim" or candidates is not None:
        if candidates is None:
            result = resident.data.score_batch(query, reducer_value, weights, float(temperature_value))
        else:
            result = resident.data.score_candidates_batch(query, candidates, reducer_value, weights,
                                                          float(temperature_value))
    else:
        result = resident.data.maxsim_batch(query)
    return result[0] if squeeze else result


def int4_maxsim_int8q(query_tokens, packed: Int4PackedDocs, *, device="auto") -> np.ndarray:
    """int8-quantised query x int4 MaxSim on MFMA, dim 128 (experimental.py:423-454)."""
    _validate_int4_packed(packed)
    batches, squeeze = _query_batches(query_tokens, packed.dim)
    if batches.shape[0] == 0:
        return np.empty((0, packed.num_docs), dtype=np.float32)
    if batches.shape[1] == 0:
        result = np.zeros((batches.shape[0], packed.num_docs), dtype=np.float32)
        return result[0] if squeeze else result
    resident = _on_device(packed, device)
    result = resident.data.maxsim_batch_int8q(np.ascontiguousarray(batches, dtype=np.float32))
    return result[0] if squeeze else result


def topk_int4_maxsim(query_tokens, packed: Int4PackedDocs, k: int, *, device="auto",
                     prefer_int8_query: bool = False, reducer="maxsim", query_weights=None,
                     temperature: float = 1.0):
    """Top-k by (score desc, doc id asc) (experimental.py:457-535); selection on device."""
    if k < 1:
        raise ValueError("k must be >= 1")
    if k > packed.num_docs:
        raise ValueError("k cannot exceed packed.num_docs")
    _validate_int4_packed(packed)
    batches, squeeze = _query_batches(query_tokens, packed.dim)
    reducer_value, weights, temperature_value = _normalize_reducer_options(
        reducer, query_weights, temperature, batch=batches.shape[0], query_tokens=batches.shape[1])
    if batches.shape[0] == 0:
        return np.empty((0, k), np.float32), np.empty((0, k), np.int64)
    resident = _on_device(packed, device)
    query = np.ascontiguousarray(batches, dtype=np.float32)
    if reducer_value == "maxsim" and prefer_int8_query and packed.dim == 128:
        scores, indices = resident.data.topk_batch_int8q(query, int(k))
    elif reducer_value == "maxsim":
        scores, indices = resident.data.topk_batch(query, int(k))
    elif batches.shape[1] == 0:
        scores, indices = _topk_rows(np.zeros((batches.shape[0], packed.num_docs), np.float32), k)
    else:
        scores, indices = resident.data.topk_score_batch(query, int(k), reducer_value, weights,
                                                         float(temperature_value))
    return (scores[0], indices[0]) if squeeze else (scores, indices)


def _topk_rows(scores: np.ndarray, k: int):
    order = np.stack([np.lexsort((np.arange(row.shape[0], dtype=np.int64), -row))[:k] for row in scores])
    return np.take_along_axis(scores, order, axis=1), order.astype(np.int64)


def _validate_int4_packed(packed: Int4PackedDocs) -> None:
    """Structural checks of experimental.py:650-700 (same messages).

    A device-resident pack (device "cuda") gets the shape and dtype checks on
    every call, but not the scans over every offset and token scale: those
    values were checked when the pack was uploaded (int4_to_device, and the
    handle again), and the kernels read the handle's own copies, so a scan of
    the host copies would cost about 50 us per search at 0.5 M tokens and
    check nothing the search uses."""
    if not isinstance(packed, Int4PackedDocs):
        raise TypeError("packed must be an Int4PackedDocs instance")
    if not isinstance(packed.dim, (int, np.integer)) or packed.dim <= 0 or packed.dim % 8 != 0:
        raise ValueError("packed.dim must be positive and divisible by 8")
    if not isinstance(packed.num_docs, (int, np.integer)) or packed.num_docs < 0:
        raise ValueError("packed.num_docs must be a nonnegative integer")
    if packed.values is not None:
        if not isinstance(packed.values, np.ndarray) or packed.values.ndim != 2 or packed.values.shape[1] != packed.dim:
            raise ValueError("packed.values must have shape [num_doc_tokens, dim]")
        if packed.values.dtype != np.int8:
            raise ValueError("packed.values must have dtype int8")
        if np.any(packed.values < -7) or np.any(packed.values > 7):
            raise ValueError("packed.values must be symmetric int4 values in [-7, 7]")
    if packed.device == "cpu":
        if packed.values is None:
            raise ValueError("CPU Int4PackedDocs must include values")
        data = packed.data
        if (not isinstance(data, np.ndarray) or data.dtype != np.uint8 or data.ndim != 2
                or data.shape != (packed.values.shape[0], packed.dim // 2)):
            raise ValueError("packed.data must have shape [num_doc_tokens, dim / 2]")
    elif packed.device != "cuda":
        raise ValueError("packed.device must be 'cpu' or 'cuda'")
    offsets = packed.doc_offsets
    if not isinstance(offsets, np.ndarray) or offsets.ndim != 1 or offsets.shape[0] != packed.num_docs + 1:
        raise ValueError("packed.doc_offsets must have shape [num_docs + 1]")
    if not np.issubdtype(offsets.dtype, np.integer):
        raise ValueError("packed.doc_offsets must contain integers")
    num_tokens = int(packed.values.shape[0]) if packed.values is not None else int(offsets[-1])
    if int(offsets[0]) != 0 or int(offsets[-1]) != num_tokens:
        raise ValueError("packed.doc_offsets must span all document tokens")
    resident = packed.device == "cuda"
    if not resident and np.any(offsets[1:] < offsets[:-1]):
        raise ValueError("packed.doc_offsets must be monotonically nondecreasing")
    try:
        scale_array = np.asarray(packed.scale)
        if scale_array.ndim != 0:
            raise ValueError
        scale_value = float(scale_array)
    except (TypeError, ValueError) as exc:
        raise ValueError("packed.scale must be a finite scalar > 0") from exc
    if not np.isfinite(scale_value) or scale_value <= 0.0:
        raise ValueError("packed.scale must be a finite scalar > 0")
    ts = packed.token_scale
    if ts is not None:
        if not isinstance(ts, np.ndarray) or ts.ndim != 1 or ts.shape[0] != num_tokens:
            raise ValueError("packed.token_scale must have shape [num_doc_tokens]")
        if ts.dtype != np.float32:
            raise ValueError("packed.token_scale must have dtype float32")
        if not resident and (not np.all(np.isfinite(ts)) or np.any(ts <= 0.0)):
            raise ValueError("packed.token_scale values must be finite and > 0")


def _validate_int4_data_matches_values(packed: Int4PackedDocs) -> None:
    """Reject payloads whose codes do not encode their values (experimental.py:703-709)."""
    if packed.device != "cpu":
        return
    if not np.array_equal(packed.data, _pack_signed_int4_values(packed.values)):
        raise ValueError("packed.data does not encode packed.values")
