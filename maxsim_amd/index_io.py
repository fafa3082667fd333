"""Index files: the reference's ``.npz`` corpus format (sdk.py:203-410).

``save_corpus`` writes schema version 2 with the same keys the reference
writes, so files move between the two packages in both directions;
``load_corpus`` accepts versions 1 and 2.  Loading executes nothing from the
file (``numpy.load(allow_pickle=False)``) and validates every array before
building a Corpus, with the reference's error messages.  This build adds one
mode, ``binary_residual`` (keys ``packed_data``, ``prefix_scale``,
``residual_int4_data``, ``residual_int4_token_scale``).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

SCHEMA_VERSION = 2
_BINARY_MODES = ("binary", "binary_token_scale", "binary_token_scale_u8", "binary_token_scale_u4", "pooled_binary")


def _encode_scale(scale):
    if scale is None:
        return "none", np.empty((0,), dtype=np.float32)
    if isinstance(scale, np.ndarray):
        return "vector", np.ascontiguousarray(scale, dtype=np.float32)
    return "scalar", np.array([float(scale)], dtype=np.float32)


def _decode_scale(kind: str, values: np.ndarray):
    if kind == "none":
        return None
    if kind == "scalar":
        return float(values.reshape(-1)[0])
    if kind == "vector":
        return np.ascontiguousarray(values, dtype=np.float32)
    raise ValueError(f"unknown scale kind: {kind}")


def _encode_log_codes(values: np.ndarray, levels: int):
    """Log-spaced codes and their [lo, hi] range (sdk.py:1066-1074)."""
    logs = np.log(np.maximum(values.astype(np.float64), 1e-12))
    lo, hi = float(logs.min()), float(logs.max())
    if hi <= lo:
        return np.zeros(values.shape[0], dtype=np.uint8), np.array([lo, lo], dtype=np.float64)
    steps = float(levels - 1)
    codes = np.clip(np.rint((logs - lo) * (steps / (hi - lo))), 0, steps).astype(np.uint8)
    return codes, np.array([lo, hi], dtype=np.float64)


def _decode_log_codes(codes: np.ndarray, params: np.ndarray, levels: int) -> np.ndarray:
    lo, hi = float(params[0]), float(params[1])
    if hi <= lo:
        return np.full(codes.shape[0], np.exp(lo), dtype=np.float32)
    return np.exp(lo + codes.astype(np.float64) * ((hi - lo) / float(levels - 1))).astype(np.float32)


def unpack_signed_int4(data: np.ndarray, dim: int) -> np.ndarray:
    """Nibbles to int8 values, low nibble first, 8..15 -> -8..-1 (sdk.py:1085-1093)."""
    low = (data & 0x0F).astype(np.int16)
    high = ((data >> 4) & 0x0F).astype(np.int16)
    values = np.empty((data.shape[0], dim), dtype=np.int8)
    values[:, 0::2] = np.where(low >= 8, low - 16, low)
    values[:, 1::2] = np.where(high >= 8, high - 16, high)
    return values


def _uint8(data, name):
    values = np.asarray(data[name])
    if values.dtype != np.uint8:
        raise ValueError(f"serialized {name} must have dtype uint8")
    return np.ascontiguousarray(values)


def _float32(data, name):
    values = np.asarray(data[name])
    if values.dtype != np.float32:
        raise ValueError(f"serialized {name} must have dtype float32")
    return np.ascontiguousarray(values)


def validate_offset_values(offsets, num_docs: int, num_tokens: int) -> None:
    """sdk.py:846-856 (same messages)."""
    if not isinstance(offsets, np.ndarray) or not np.issubdtype(offsets.dtype, np.integer):
        raise ValueError("doc_offsets must be an integer NumPy array")
    if offsets.ndim != 1 or offsets.shape[0] != num_docs + 1:
        raise ValueError("doc_offsets must have shape [num_docs + 1]")
    if int(offsets[0]) != 0:
        raise ValueError("doc_offsets must start at 0")
    if np.any(offsets[1:] < offsets[:-1]):
        raise ValueError("doc_offsets must be monotonically nondecreasing")
    if int(offsets[-1]) != num_tokens:
        raise ValueError("doc_offsets must end at num_doc_tokens")


def _check_data(offsets, num_docs, data, dim, bytes_per_token):
    if dim <= 0 or dim % 8 != 0:
        raise ValueError("serialized dim must be positive and divisible by 8")
    if data.ndim != 2 or data.shape[1] != bytes_per_token:
        raise ValueError("serialized packed data shape does not match dim")
    validate_offset_values(offsets, num_docs, int(data.shape[0]))


def save_corpus(corpus, path) -> Path:
    from maxsim_amd.binres import BinaryResidualPackedDocs
    from maxsim_amd.cascade import _validate_residual_packed
    from maxsim_amd.experimental import _validate_int4_data_matches_values, _validate_int4_packed

    out = Path(path)
    out.parent.mkdir(parents=True, exist_ok=True)
    arrays = {
        "schema_version": np.array(SCHEMA_VERSION, dtype=np.int64),
        "format": np.array("maxsim_corpus"),
        "mode": np.array(corpus.mode),
        "doc_ids": np.asarray(corpus.doc_ids),
        "metadata_json": np.array(json.dumps({} if corpus.metadata is None else corpus.metadata, sort_keys=True)),
    }
    n = len(corpus.doc_ids)
    if corpus.packed is not None:
        p = corpus.packed
        if p.device != "cpu":
            raise ValueError("Corpus.save requires CPU packed docs")
        data = np.ascontiguousarray(p.data, dtype=np.uint8)
        offsets = np.asarray(p.doc_offsets)
        validate_offset_values(offsets, n, int(data.shape[0]))
        kind, values = _encode_scale(p.scale)
        arrays.update({"packed_data": data, "doc_offsets": np.ascontiguousarray(offsets, dtype=np.int64),
                       "dim": np.array(p.dim, dtype=np.int64), "scale_kind": np.array(kind),
                       "scale_values": values})
        if p.token_scale is not None:
            if corpus.mode == "binary_token_scale_u8":
                codes, params = _encode_log_codes(p.token_scale, 256)
                arrays["token_scale_u8_codes"] = codes
                arrays["token_scale_u8_params"] = params
            elif corpus.mode == "binary_token_scale_u4":
                codes, params = _encode_log_codes(p.token_scale, 16)
                padded = np.concatenate([codes, np.zeros(len(codes) % 2, dtype=np.uint8)])
                arrays["token_scale_u4_codes"] = (padded[0::2] | (padded[1::2] << 4)).astype(np.uint8)
                arrays["token_scale_u4_params"] = params
                arrays["token_scale_u4_count"] = np.array(len(codes), dtype=np.int64)
            else:
                arrays["token_scale_fp16"] = np.ascontiguousarray(p.token_scale, dtype=np.float16)
    elif isinstance(corpus.int4_packed, BinaryResidualPackedDocs):
        b = corpus.int4_packed
        if b.device != "cpu":
            raise ValueError("Corpus.save requires CPU binary residual packed docs")
        validate_offset_values(np.asarray(b.doc_offsets), n, int(np.asarray(b.sign_data).shape[0]))
        arrays.update({"packed_data": np.ascontiguousarray(b.sign_data, dtype=np.uint8),
                       "doc_offsets": np.ascontiguousarray(b.doc_offsets, dtype=np.int64),
                       "dim": np.array(b.dim, dtype=np.int64),
                       "prefix_scale": np.ascontiguousarray(b.prefix_scale, dtype=np.float32),
                       "residual_int4_data": np.ascontiguousarray(b.residual_data, dtype=np.uint8),
                       "residual_int4_token_scale": np.ascontiguousarray(b.residual_token_scale, dtype=np.float32)})
    elif corpus.int4_packed is not None and corpus.mode == "int4_residual":
        r = corpus.int4_packed
        if r.device != "cpu":
            raise ValueError("Corpus.save requires CPU residual int4 packed docs")
        _validate_residual_packed(r, verify_packed_values=True)
        arrays.update({"int4_data": np.ascontiguousarray(r.prefix_data, dtype=np.uint8),
                       "doc_offsets": np.ascontiguousarray(r.doc_offsets, dtype=np.int64),
                       "dim": np.array(r.dim, dtype=np.int64),
                       "int4_scale": np.array(r.prefix_scale, dtype=np.float32),
                       "int4_token_scale": np.ascontiguousarray(r.prefix_token_scale, dtype=np.float32),
                       "residual_int4_data": np.ascontiguousarray(r.residual_data, dtype=np.uint8),
                       "residual_int4_scale": np.array(r.residual_scale, dtype=np.float32),
                       "residual_int4_token_scale": np.ascontiguousarray(r.residual_token_scale, dtype=np.float32)})
    elif corpus.int4_packed is not None:
        q = corpus.int4_packed
        if q.device != "cpu":
            raise ValueError("Corpus.save requires CPU int4 packed docs")
        _validate_int4_packed(q)
        _validate_int4_data_matches_values(q)
        arrays.update({"int4_data": np.ascontiguousarray(q.data, dtype=np.uint8),
                       "doc_offsets": np.ascontiguousarray(q.doc_offsets, dtype=np.int64),
                       "dim": np.array(q.dim, dtype=np.int64),
                       "int4_scale": np.array(q.scale, dtype=np.float32)})
        if q.token_scale is not None:
            arrays["int4_token_scale"] = np.ascontiguousarray(q.token_scale, dtype=np.float32)
    else:
        raise ValueError("corpus has no packed payload")
    with out.open("wb") as fh:
        np.savez_compressed(fh, **arrays)
    return out.resolve()


def load_corpus(path):
    from maxsim_amd._api import PackedDocs
    from maxsim_amd.binres import BinaryResidualPackedDocs
    from maxsim_amd.cascade import ResidualInt4PackedDocs, _validate_residual_packed
    from maxsim_amd.experimental import Int4PackedDocs, _validate_int4_packed
    from maxsim_amd.sdk import Corpus

    source = Path(path).resolve()
    with np.load(source, allow_pickle=False) as data:
        if int(np.asarray(data["schema_version"]).item()) not in {1, 2}:
            raise ValueError("unsupported corpus schema_version")
        if str(np.asarray(data["format"]).item()) != "maxsim_corpus":
            raise ValueError("unsupported corpus format")
        mode = str(np.asarray(data["mode"]).item())
        doc_ids = tuple(str(v) for v in np.asarray(data["doc_ids"]))
        metadata = json.loads(str(np.asarray(data["metadata_json"]).item()))
        raw = np.asarray(data["doc_offsets"])
        if not np.issubdtype(raw.dtype, np.integer):
            raise ValueError("serialized doc_offsets must contain integers")
        offsets = np.ascontiguousarray(raw, dtype=np.int64)
        dim = int(np.asarray(data["dim"]).item())
        n = len(doc_ids)
        if mode in _BINARY_MODES:
            packed_data = _uint8(data, "packed_data")
            _check_data(offsets, n, packed_data, dim, dim // 8)
            token_scale = None
            if "token_scale_fp16" in data:
                token_scale = np.ascontiguousarray(data["token_scale_fp16"]).astype(np.float32)
            elif "token_scale_u8_codes" in data:
                token_scale = _decode_log_codes(np.asarray(data["token_scale_u8_codes"]),
                                                np.asarray(data["token_scale_u8_params"]), 256)
            elif "token_scale_u4_codes" in data:
                packed_codes = np.asarray(data["token_scale_u4_codes"])
                count = int(np.asarray(data["token_scale_u4_count"]).item())
                codes = np.empty(packed_codes.shape[0] * 2, dtype=np.uint8)
                codes[0::2] = packed_codes & 0x0F
                codes[1::2] = packed_codes >> 4
                token_scale = _decode_log_codes(codes[:count], np.asarray(data["token_scale_u4_params"]), 16)
            if token_scale is not None and token_scale.shape[0] != packed_data.shape[0]:
                raise ValueError("packed.token_scale must have shape [num_doc_tokens]")
            scale = _decode_scale(str(np.asarray(data["scale_kind"]).item()), np.asarray(data["scale_values"]))
            packed = PackedDocs(data=packed_data, doc_offsets=offsets, dim=dim, num_docs=n, scale=scale,
                                device="cpu", token_scale=token_scale)
            return Corpus(doc_ids=doc_ids, mode=mode, packed=packed, metadata=metadata)
        if mode == "binary_residual":
            signs = _uint8(data, "packed_data")
            residual = _uint8(data, "residual_int4_data")
            _check_data(offsets, n, signs, dim, dim // 8)
            _check_data(offsets, n, residual, dim, dim // 2)
            values = unpack_signed_int4(residual, dim)
            if np.any(values < -7):
                raise ValueError("residual_values must be symmetric int4 values in [-7, 7]")
            packed = BinaryResidualPackedDocs(sign_data=signs, prefix_scale=_float32(data, "prefix_scale"),
                                              residual_data=residual, residual_values=values,
                                              residual_token_scale=_float32(data, "residual_int4_token_scale"),
                                              doc_offsets=offsets, dim=dim, num_docs=n, device="cpu")
            return Corpus(doc_ids=doc_ids, mode=mode, int4_packed=packed, metadata=metadata)
        if mode == "int4_residual":
            prefix = _uint8(data, "int4_data")
            residual = _uint8(data, "residual_int4_data")
            _check_data(offsets, n, prefix, dim, dim // 2)
            _check_data(offsets, n, residual, dim, dim // 2)
            packed = ResidualInt4PackedDocs(
                prefix_data=prefix, prefix_values=unpack_signed_int4(prefix, dim),
                prefix_scale=float(np.asarray(data["int4_scale"]).item()),
                prefix_token_scale=_float32(data, "int4_token_scale"), residual_data=residual,
                residual_values=unpack_signed_int4(residual, dim),
                residual_scale=float(np.asarray(data["residual_int4_scale"]).item()),
                residual_token_scale=_float32(data, "residual_int4_token_scale"), doc_offsets=offsets, dim=dim,
                num_docs=n, device="cpu")
            _validate_residual_packed(packed, verify_packed_values=True)
            return Corpus(doc_ids=doc_ids, mode=mode, int4_packed=packed, metadata=metadata)
        if mode in {"int4", "int4_per_token"}:
            q = _uint8(data, "int4_data")
            token_scale = _float32(data, "int4_token_scale") if "int4_token_scale" in data else None
            _check_data(offsets, n, q, dim, dim // 2)
            packed = Int4PackedDocs(data=q, values=unpack_signed_int4(q, dim), doc_offsets=offsets, dim=dim,
                                    num_docs=n, scale=float(np.asarray(data["int4_scale"]).item()), device="cpu",
                                    token_scale=token_scale)
            _validate_int4_packed(packed)
            return Corpus(doc_ids=doc_ids, mode=mode, int4_packed=packed, metadata=metadata)
        raise ValueError("unsupported corpus mode")
