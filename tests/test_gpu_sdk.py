"""Index / Reranker on the GPU: the reference's tests/test_sdk.py search and
rerank expectations with device="cuda", and the config-2 route end to end."""
import numpy as np
import pytest

import maxsim_amd as maxsim

pytestmark = pytest.mark.gpu


def _tiny():
    docs = np.array([[1] * 8, [-1] * 8, [1, -1] * 4], dtype=np.float32)
    return docs, np.array([0, 1, 2, 3], dtype=np.int64)


def _reranker(mode, **kw):
    docs, offsets = _tiny()
    c = maxsim.Corpus.from_embeddings(["positive", "negative", "mixed"], docs, offsets, mode=mode)
    return maxsim.Reranker.from_corpus(c, device="cuda", **kw)


@pytest.mark.parametrize("mode", ["binary", "binary_token_scale", "int4", "int4_per_token", "int4_residual"])
def test_search_single_and_batched(gpu, mode):
    """tests/test_sdk.py:41-70."""
    r = _reranker(mode)
    res = r.search(np.ones((1, 8), np.float32), k=2)
    assert [x.doc_id for x in res] == ["positive", "mixed"]
    assert [x.rank for x in res] == [1, 2] and all(isinstance(x.score, float) for x in res)
    q = np.array([[[1] * 8], [[-1] * 8]], np.float32)
    out = r.search(q, k=1)
    assert [[x.doc_id for x in row] for row in out] == [["positive"], ["negative"]]


def test_rerank_candidates_and_unknown_id(gpu):
    """tests/test_sdk.py:73-91."""
    r = _reranker("binary")
    res = r.rerank(np.ones((1, 8), np.float32), candidate_ids=["negative", "mixed", "mixed"], k=3)
    assert [x.doc_id for x in res] == ["mixed", "negative"] and [x.rank for x in res] == [1, 2]
    with pytest.raises(KeyError, match="missing"):
        r.rerank(np.ones((1, 8), np.float32), candidate_ids=["missing"], k=1)


def test_residual_mode_search_rerank_cascade(gpu):
    """tests/test_sdk.py:214-246."""
    from maxsim_amd.cascade import cascade_topk, residual_score

    rng = np.random.default_rng(197)
    lengths = np.array([2, 4, 1, 3, 5], np.int64)
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    docs = rng.normal(size=(int(offsets[-1]), 8)).astype(np.float32)
    query = rng.normal(size=(3, 8)).astype(np.float32)
    ids = [f"doc-{i}" for i in range(5)]
    corpus = maxsim.Index.from_embeddings(ids, docs, offsets, mode="int4_residual")
    r = maxsim.Reranker.from_corpus(corpus, device="cuda")
    cs, ci = cascade_topk(query, corpus.int4_packed, 2, candidates=4)
    res = r.search(query, k=2, rescore_candidates=4)
    assert [x.doc_id for x in res] == [ids[i] for i in ci]
    np.testing.assert_allclose([x.score for x in res], cs, rtol=0, atol=1e-5)
    reranked = r.rerank(query, ["doc-4", "doc-1", "doc-3"], k=3)
    exp = residual_score(query, corpus.int4_packed, candidate_indices=np.array([4, 1, 3]))
    order = np.lexsort((np.arange(3), -exp))
    assert [x.doc_id for x in reranked] == [["doc-4", "doc-1", "doc-3"][i] for i in order]


@pytest.mark.parametrize("reducer", ["maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"])
def test_residual_full_search_equals_stable_topk_of_the_scores(gpu, reducer):
    """Reranker.search on an int4_residual index without rescore_candidates
    selects on the device; it must return what the reference's search does
    (its stable top-k of the fused scores, sdk.py:497-559), ties included
    (every document appears twice)."""
    from maxsim_amd.cascade import _stable_topk, residual_score

    rng = np.random.default_rng(211)
    lengths = rng.integers(1, 12, size=60)
    lengths = np.concatenate([lengths, lengths])
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    half = rng.normal(size=(int(lengths[:60].sum()), 128)).astype(np.float32)
    docs = np.concatenate([half, half])
    ids = [f"d{i}" for i in range(120)]
    corpus = maxsim.Index.from_embeddings(ids, docs, offsets, mode="int4_residual")
    r = maxsim.Reranker.from_corpus(corpus, device="cuda")
    query = rng.normal(size=(3, 7, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=(3, 7)).astype(np.float32) if reducer == "weighted_maxsim" else None
    opts = dict(reducer=reducer, query_weights=w, temperature=0.7)
    es, ei = _stable_topk(residual_score(query, corpus.int4_packed, **opts), 15)
    res = r.search(query, k=15, **opts)
    for row, s, i in zip(res, es, ei):
        assert [x.doc_id for x in row] == [ids[j] for j in i]
        assert [x.score for x in row] == [float(v) for v in s]


def test_rescore_candidates_requires_residual_mode(gpu):
    with pytest.raises(ValueError, match="int4_residual"):
        _reranker("int4_per_token").search(np.ones((1, 8), np.float32), k=2, rescore_candidates=3)


def test_config2_route_int8_query_matches_oracle(gpu, oracle):
    """Reranker(device='cuda', int4_query='int8').search on a per-token int4
    index: ids and scores of the top-10 equal the C oracle's."""
    from maxsim_amd import synthetic

    corpus = synthetic.make_corpus(600, 64, 192, seed=7)
    query = synthetic.make_queries(corpus, 4)
    ids = [f"doc{i}" for i in range(600)]
    index = maxsim.Index.from_embeddings(ids, corpus.embeddings, corpus.offsets, mode="int4_per_token")
    r = maxsim.Reranker(index, device="cuda", int4_query="int8")
    res = r.search(query, k=10)
    p = index.int4_packed
    exp = oracle.int4_int8q_scores(query, p.values, p.doc_offsets, token_scale=p.token_scale)
    es, ei = oracle.topk(exp, 10)
    assert [[x.doc_id for x in row] for row in res] == [[ids[i] for i in row] for row in ei]
    assert [[x.score for x in row] for row in res] == es.astype(np.float64).tolist()


def test_binary_residual_mode(gpu, oracle):
    from maxsim_amd import synthetic

    corpus = synthetic.make_corpus(300, 64, 192, seed=8)
    query = synthetic.make_queries(corpus, 2)
    ids = [f"d{i}" for i in range(300)]
    index = maxsim.Index.from_embeddings(ids, corpus.embeddings, corpus.offsets, mode="binary_residual")
    r = maxsim.Reranker(index, device="cuda")
    full = r.search(query, k=5)
    casc = r.search(query, k=5, rescore_candidates=300)
    assert [[x.doc_id for x in row] for row in full] == [[x.doc_id for x in row] for row in casc]
    signs, a, _, rv, rs = oracle.pack_binary_residual(corpus.embeddings)
    exp = oracle.binres_fused_scores(query, signs, a, rv, rs, corpus.offsets)
    for b in range(2):
        got = np.array([x.score for x in full[b]])
        idx = [ids.index(x.doc_id) for x in full[b]]
        np.testing.assert_allclose(got, exp[b][idx], rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("precision", ["int8", "fp32"])
def test_binary_residual_full_search_equals_stable_topk_of_the_scores(gpu, precision):
    """The full search of a binary_residual index selects on the device; it
    returns the stable top-k of the fused scores (score desc, id asc), ties
    included (every document appears twice), for both query precisions."""
    from maxsim_amd.binres import _binres_topk, binres_score, pack_binary_residual
    from maxsim_amd.cascade import _stable_topk

    rng = np.random.default_rng(223)
    lengths = rng.integers(1, 20, size=80)
    lengths = np.concatenate([lengths, lengths])
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    half = rng.normal(size=(int(lengths[:80].sum()), 128)).astype(np.float32)
    packed = pack_binary_residual(np.concatenate([half, half]), offsets)
    query = rng.normal(size=(3, 9, 128)).astype(np.float32)
    es, ei = _stable_topk(binres_score(query, packed, query_precision=precision), 12)
    gs, gi = _binres_topk(query, packed, 12, query_precision=precision)
    np.testing.assert_array_equal(gi, ei)
    np.testing.assert_array_equal(gs, es)
    ids = [f"d{i}" for i in range(160)]
    index = maxsim.Index.from_embeddings(ids, np.concatenate([half, half]), offsets, mode="binary_residual")
    res = maxsim.Reranker(index, device="cuda").search(query, k=12)
    if precision == "int8":
        assert [[x.doc_id for x in row] for row in res] == [[ids[j] for j in row] for row in ei]


@pytest.mark.parametrize("mode", ["binary_token_scale", "int4_per_token", "int4_residual", "binary_residual"])
def test_saved_index_searches_the_same(gpu, tmp_path, mode):
    """tests/test_sdk.py:130-306: an index read back from its .npz file gives
    the same results."""
    rng = np.random.default_rng(199)
    docs = rng.normal(size=(40, 128)).astype(np.float32)
    offsets = np.array([0, 3, 5, 9, 12, 20, 40], dtype=np.int64)
    ids = list("abcdef")
    query = rng.normal(size=(2, 4, 128)).astype(np.float32)
    index = maxsim.Index.from_embeddings(ids, docs, offsets, mode=mode)
    index.save(tmp_path / "i.npz")
    loaded = maxsim.Index.load(tmp_path / "i.npz")
    kw = {"rescore_candidates": 4} if mode in {"int4_residual", "binary_residual"} else {}
    a = maxsim.Reranker(index, device="cuda").search(query, k=3, **kw)
    b = maxsim.Reranker.load(tmp_path / "i.npz", device="cuda").search(query, k=3, **kw)
    assert [[x.doc_id for x in r] for r in a] == [[x.doc_id for x in r] for r in b]
    np.testing.assert_allclose([[x.score for x in r] for r in a], [[x.score for x in r] for r in b], rtol=0,
                               atol=1e-5 if mode == "binary_token_scale" else 0)
    assert loaded.encoded_bytes == index.encoded_bytes
