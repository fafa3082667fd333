"""Index construction and validation of the SDK layer (no GPU): the
reference's tests/test_sdk.py expectations that do not score."""
import numpy as np
import pytest

import maxsim_amd as maxsim


def _tiny():
    docs = np.array([[1] * 8, [-1] * 8, [1, -1] * 4], dtype=np.float32)
    return docs, np.array([0, 1, 2, 3], dtype=np.int64)


def test_corpus_metadata_and_storage():
    """tests/test_sdk.py:22-38."""
    docs, offsets = _tiny()
    c = maxsim.Corpus.from_embeddings(["positive", "negative", "mixed"], docs, offsets, mode="binary",
                                      metadata={"model": "tiny"})
    assert c.doc_ids == ("positive", "negative", "mixed")
    assert (c.num_docs, c.dim, c.mode, c.metadata, c.storage_bytes) == (3, 8, "binary", {"model": "tiny"}, 3)


def test_int4_storage_bytes():
    """tests/test_sdk.py:118-127: 3 tokens x 4 bytes + 4-byte scale."""
    docs, offsets = _tiny()
    assert maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode="int4").storage_bytes == 3 * 8 // 2 + 4


def test_corpus_validation():
    """tests/test_sdk.py:94-102, 630-640."""
    docs, offsets = _tiny()
    with pytest.raises(ValueError, match="unique"):
        maxsim.Corpus.from_embeddings(["dup", "dup", "mixed"], docs, offsets, mode="binary")
    with pytest.raises(ValueError, match="one more entry"):
        maxsim.Corpus.from_embeddings(["one", "two"], docs, offsets, mode="binary")
    with pytest.raises(ValueError, match="mode"):
        maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode="bad")
    with pytest.raises(ValueError, match="integers"):
        maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets.astype(np.float32), mode="binary")


def test_auto_and_presets():
    """tests/test_sdk.py:321-370."""
    rng = np.random.default_rng(211)
    docs = rng.standard_normal((18, 16)).astype(np.float32)
    offsets = np.array([0, 6, 12, 18], dtype=np.int64)
    ids = ["a", "b", "c"]
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets).mode == "int4_per_token"
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="max_quality").int4_packed.token_scale is not None
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="int4").int4_packed.token_scale is None
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="max_compression").metadata["pool_factor"] == 3
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="max_compression",
                                         pool_factor=2).metadata["pool_factor"] == 2
    assert maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="pooled_binary").metadata["pool_factor"] == 2
    with pytest.raises(ValueError, match="integer"):
        maxsim.Corpus.from_embeddings(ids, docs, offsets, mode="pooled_binary", pool_factor=2.5)
    assert maxsim.Index is maxsim.Corpus


def test_pooling_reduces_to_ceil_count():
    rng = np.random.default_rng(5)
    docs = rng.standard_normal((17, 16)).astype(np.float32)
    offsets = np.array([0, 7, 7, 17], dtype=np.int64)
    from maxsim_amd.pooling import pool_doc_tokens

    pooled, poff = pool_doc_tokens(docs, offsets, 2)
    assert np.diff(poff).tolist() == [4, 0, 5]
    assert pooled.shape == (9, 16)


def test_encoded_bytes_include_binary_scales():
    """tests/test_sdk.py:453-462."""
    docs, offsets = _tiny()
    packed = maxsim.pack_signs(docs, offsets, scale="doc")
    c = maxsim.Corpus(doc_ids=("a", "b", "c"), mode="binary", packed=packed)
    assert c.encoded_bytes == packed.data.nbytes + packed.scale.nbytes


def test_binary_residual_mode_bytes():
    rng = np.random.default_rng(6)
    docs = rng.standard_normal((10, 128)).astype(np.float32)
    c = maxsim.Corpus.from_embeddings(["a", "b"], docs, np.array([0, 4, 10]), mode="binary_residual")
    assert c.encoded_bytes == 10 * 88


def test_reranker_cpu_device_is_rejected():
    docs, offsets = _tiny()
    c = maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode="binary")
    with pytest.raises(NotImplementedError):
        maxsim.Reranker(c, device="cpu")
    with pytest.raises(ValueError, match="int4_query"):
        maxsim.Reranker(c, int4_query="fp16")


@pytest.mark.parametrize("mode", ["binary", "binary_token_scale", "binary_token_scale_u8", "binary_token_scale_u4",
                                  "pooled_binary", "int4", "int4_per_token", "int4_residual", "binary_residual"])
def test_save_load_roundtrip(tmp_path, mode):
    rng = np.random.default_rng(11)
    docs = rng.standard_normal((30, 16)).astype(np.float32)
    offsets = np.array([0, 5, 5, 12, 30], dtype=np.int64)
    ids = ["a", "b", "c", "d"]
    c = maxsim.Corpus.from_embeddings(ids, docs, offsets, mode=mode, metadata={"k": 1})
    path = tmp_path / f"{mode}.maxsim.npz"
    c.save(path)
    back = maxsim.Corpus.load(path)
    assert back.mode == mode and back.doc_ids == tuple(ids) and back.metadata == c.metadata
    assert back.encoded_bytes == c.encoded_bytes
    a, b = (c.packed, back.packed) if c.packed is not None else (c.int4_packed, back.int4_packed)
    for name in ("data", "sign_data", "prefix_data", "residual_data", "values", "residual_values", "prefix_values",
                 "doc_offsets", "token_scale", "prefix_token_scale", "residual_token_scale", "prefix_scale"):
        x, y = getattr(a, name, None), getattr(b, name, None)
        if isinstance(x, np.ndarray):
            tol = 2e-3 if name == "token_scale" and mode != "int4_per_token" else 0
            np.testing.assert_allclose(y, x, rtol=tol, atol=0)


def test_load_accepts_schema_v1(tmp_path):
    """tests/test_sdk.py:465-486."""
    docs = np.array([[1] * 8, [-1] * 8, [1, -1] * 4], dtype=np.float32)
    offsets = np.array([0, 1, 2, 3], dtype=np.int64)
    packed = maxsim.pack_int4_symmetric(docs, offsets)
    path = tmp_path / "legacy.npz"
    np.savez_compressed(path, schema_version=np.array(1, dtype=np.int64), format=np.array("maxsim_corpus"),
                        mode=np.array("int4"), doc_ids=np.array(["p", "n", "m"]), metadata_json=np.array("{}"),
                        int4_data=packed.data, doc_offsets=offsets, dim=np.array(8, dtype=np.int64),
                        int4_scale=np.array(packed.scale, dtype=np.float32))
    np.testing.assert_array_equal(maxsim.Corpus.load(path).int4_packed.values, packed.values)


def _resave(tmp_path, mode, edit):
    docs = np.array([[1] * 8, [-1] * 8, [1, -1] * 4], dtype=np.float32)
    path = tmp_path / "valid.npz"
    maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, np.array([0, 1, 2, 3]), mode=mode).save(path)
    with np.load(path, allow_pickle=False) as data:
        payload = {k: np.asarray(data[k]) for k in data.files}
    edit(payload)
    bad = tmp_path / "bad.npz"
    np.savez_compressed(bad, **payload)
    return bad


@pytest.mark.parametrize("offsets,message", [([1, 1, 2, 3], "start at 0"), ([0, 2, 1, 3], "monotonically"),
                                             ([0, 1, 2, 4], "end at num_doc_tokens")])
def test_load_rejects_corrupt_offsets(tmp_path, offsets, message):
    """tests/test_sdk.py:518-540."""
    bad = _resave(tmp_path, "binary", lambda p: p.__setitem__("doc_offsets", np.array(offsets, dtype=np.int64)))
    with pytest.raises(ValueError, match=message):
        maxsim.Corpus.load(bad)


def test_load_rejects_bad_dtypes_and_negative_eight(tmp_path):
    """tests/test_sdk.py:543-593."""
    bad = _resave(tmp_path, "binary", lambda p: p.__setitem__("packed_data", p["packed_data"].astype(np.float32)))
    with pytest.raises(ValueError, match="dtype uint8"):
        maxsim.Corpus.load(bad)
    bad = _resave(tmp_path, "int4_per_token",
                  lambda p: p.__setitem__("int4_token_scale", p["int4_token_scale"].astype(np.float64)))
    with pytest.raises(ValueError, match="dtype float32"):
        maxsim.Corpus.load(bad)

    def eight(p):
        p["int4_data"] = p["int4_data"].copy()
        p["int4_data"][0, 0] = (p["int4_data"][0, 0] & 0xF0) | 0x08

    with pytest.raises(ValueError, match="symmetric int4"):
        maxsim.Corpus.load(_resave(tmp_path, "int4", eight))


def test_save_rejects_invalid_payloads(tmp_path):
    """tests/test_sdk.py:596-627."""
    from dataclasses import replace

    docs = np.array([[1] * 8, [-1] * 8, [1, -1] * 4], dtype=np.float32)
    c = maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, np.array([0, 1, 2, 3]), mode="int4_per_token")
    data = c.int4_packed.data.copy()
    data[0, 0] ^= np.uint8(1)
    with pytest.raises(ValueError, match="does not encode"):
        replace(c, int4_packed=replace(c.int4_packed, data=data)).save(tmp_path / "x.npz")
    packed = maxsim.pack_signs(docs)
    invalid = maxsim.PackedDocs(data=packed.data, doc_offsets=np.array([0, 2, 1, 3], dtype=np.int64),
                                dim=packed.dim, num_docs=packed.num_docs)
    with pytest.raises(ValueError, match="monotonically"):
        maxsim.Corpus(doc_ids=("a", "b", "c"), mode="binary", packed=invalid).save(tmp_path / "y.npz")


def _report_docs():
    rng = np.random.default_rng(382)
    docs = rng.standard_normal((11, 16)).astype(np.float32)
    return docs, np.array([0, 4, 7, 11], dtype=np.int64)


def test_memory_report_counts_encoded_host_and_serialized_bytes(tmp_path):
    """tests/test_sdk.py:382-408: host bytes are the payload's NumPy buffers;
    serialized bytes follow save / load / an explicit path."""
    docs, offsets = _report_docs()
    corpus = maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode="int4_per_token")
    report = corpus.memory_report()
    p = corpus.int4_packed
    assert isinstance(report, maxsim.CorpusMemoryReport)
    assert report.encoded_bytes == corpus.storage_bytes
    assert report.host_array_bytes == p.data.nbytes + p.values.nbytes + p.doc_offsets.nbytes + p.token_scale.nbytes
    assert (report.device_index_bytes, report.device_workspace_bytes, report.serialized_bytes) == (0, 0, None)
    path = tmp_path / "memory.maxsim.npz"
    corpus.save(path)
    size = path.stat().st_size
    assert corpus.memory_report().serialized_bytes == size
    assert corpus.memory_report(path).serialized_bytes == size
    assert maxsim.Corpus.load(path).memory_report().serialized_bytes == size


def test_memory_report_path_without_npz_suffix(tmp_path):
    """tests/test_sdk.py:411-426."""
    docs, offsets = _report_docs()
    corpus = maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode="int4_per_token")
    path = tmp_path / "corpus.index"
    corpus.save(path)
    assert path.is_file() and not path.with_suffix(path.suffix + ".npz").exists()
    assert corpus.memory_report().serialized_bytes == path.stat().st_size


def test_memory_report_reads_the_device_handle_accessors():
    """tests/test_sdk.py:429-450: a resident payload reports its handle's
    resident_bytes and workspace_bytes."""

    class FakeHandle:
        dim = 8
        num_docs = 3
        packed_size = 3
        resident_bytes = 91
        workspace_bytes = 37

    packed = maxsim.PackedDocs(data=FakeHandle(), doc_offsets=np.array([0, 1, 2, 3], dtype=np.int64), dim=8,
                               num_docs=3, device="cuda")
    report = maxsim.Corpus(doc_ids=("a", "b", "c"), mode="binary", packed=packed).memory_report()
    assert report.host_array_bytes == packed.doc_offsets.nbytes
    assert (report.device_index_bytes, report.device_workspace_bytes) == (91, 37)


@pytest.mark.parametrize("mode", ["binary", "binary_token_scale", "int4", "int4_residual", "binary_residual"])
def test_memory_report_host_bytes_every_mode(mode):
    docs, offsets = _report_docs()
    corpus = maxsim.Corpus.from_embeddings(["a", "b", "c"], docs, offsets, mode=mode)
    payload = corpus.packed if corpus.packed is not None else corpus.int4_packed
    arrays = [v for v in vars(payload).values() if isinstance(v, np.ndarray)]
    assert corpus.memory_report().host_array_bytes == sum(a.nbytes for a in arrays)
