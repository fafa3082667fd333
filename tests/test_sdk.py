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
