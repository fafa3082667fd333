"""GPU parity of the cascades (int4 residual, binary prefix + int4 residual)
and of the public API routes over the device handles."""
import numpy as np
import pytest

from conftest import ragged_fixture

pytestmark = pytest.mark.gpu

REDUCERS = ("maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim")


def _close(actual, expected, rtol=1e-5):
    scale = max(1.0, float(np.max(np.abs(expected)))) if np.size(expected) else 1.0
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=rtol * scale)


def _stable(scores, k, tie_ids=None):
    ids = np.arange(scores.shape[0]) if tie_ids is None else tie_ids
    return np.lexsort((ids, -scores))[:k]


def _corpus(n=300, seed=40, lo=1, hi=60):
    from maxsim_amd import synthetic

    c = synthetic.make_corpus(n, lo, hi, seed=seed)
    return c.embeddings, c.offsets


# ----------------------------------------------------------- int4 residual


@pytest.mark.parametrize("reducer", REDUCERS)
def test_int4_residual_cascade_equals_host_procedure(gpu, oracle, reducer):
    """The device cascade returns what cascade.py:294-453 computes from the
    same prefix and fused scores: coarse stable top-M, per-row rescoring,
    final order by (fused score desc, document id asc)."""
    from maxsim_amd import synthetic
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, prefix_score, residual_int4_to_device, residual_score

    docs, offsets = _corpus()
    query = synthetic.make_queries(synthetic.make_corpus(300, 1, 60, seed=40), 3)
    weights = np.random.default_rng(41).uniform(0.5, 1.5, size=(3, 32)).astype(np.float32)
    w = weights if reducer == "weighted_maxsim" else None
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    k, m = 10, 64
    top_s, top_i = cascade_topk(query, packed, k, candidates=m, reducer=reducer, query_weights=w, temperature=0.7)
    coarse = prefix_score(query, packed, reducer=reducer, query_weights=w, temperature=0.7)
    for b in range(3):
        cands = _stable(coarse[b], m)
        fine = residual_score(query[b], packed, reducer=reducer, query_weights=None if w is None else w[b],
                              temperature=0.7, candidate_indices=cands)
        order = _stable(fine, k, tie_ids=cands)
        np.testing.assert_array_equal(top_i[b], cands[order])
        np.testing.assert_array_equal(top_s[b], fine[order])
    # and the fused scores are the oracle's
    pcodes, pv, ps = oracle.pack_int4_token(docs)
    prefix = pv.astype(np.float32) * ps[:, None]
    _, rv, rs = oracle.pack_int4_token(docs - prefix)
    recon = prefix + rv.astype(np.float32) * rs[:, None]
    full = oracle.dense_scores(query, recon, offsets, reducer=reducer, weights=w, temperature=0.7)
    _close(top_s, np.take_along_axis(full, top_i, axis=1))


def test_int4_residual_cascade_full_budget_is_full_topk(gpu):
    """candidates == num_docs gives the fused full top-k (tests/test_cascade.py:405-432)."""
    from maxsim_amd import synthetic
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, residual_int4_to_device, residual_score

    docs, offsets = _corpus(120, 42)
    query = synthetic.make_queries(synthetic.make_corpus(120, 1, 60, seed=42), 2)
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    s, i = cascade_topk(query, packed, 7, candidates=packed.num_docs)
    full = residual_score(query, packed)
    for b in range(2):
        order = _stable(full[b], 7)
        np.testing.assert_array_equal(i[b], order)
        np.testing.assert_array_equal(s[b], full[b][order])


def test_cascade_tie_order_by_document_id(gpu):
    """Identical documents tie: the cascade keeps the lower ids (tests/test_cascade.py:389-402)."""
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, residual_int4_to_device

    rng = np.random.default_rng(43)
    base = rng.standard_normal((4, 128)).astype(np.float32)
    docs = np.concatenate([base] * 6)  # six identical 4-token documents
    offsets = np.arange(0, 25, 4, dtype=np.int64)
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    _, idx = cascade_topk(rng.standard_normal((3, 128)).astype(np.float32), packed, 3, candidates=5)
    np.testing.assert_array_equal(idx, [0, 1, 2])


def test_cascade_many_ties_at_the_candidate_threshold(gpu):
    """3,000 documents that are 12 distinct ones repeated (ties in whole
    groups of 250), 512 candidates: the threshold falls inside a group, so the
    selector must keep that group's lowest ids (the radix rounds reach the
    position bits).  Equal to the host procedure on the device's scores."""
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, prefix_score, residual_int4_to_device, \
        residual_score

    rng = np.random.default_rng(44)
    distinct = [rng.standard_normal((int(rng.integers(3, 40)), 128)).astype(np.float32) for _ in range(12)]
    order = np.repeat(np.arange(12), 250)
    rng.shuffle(order)
    docs = np.concatenate([distinct[i] for i in order])
    offsets = np.concatenate([[0], np.cumsum([distinct[i].shape[0] for i in order])]).astype(np.int64)
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    query = rng.standard_normal((2, 8, 128)).astype(np.float32)
    k, m = 10, 512
    ts, ti = cascade_topk(query, packed, k, candidates=m)
    coarse = prefix_score(query, packed)
    for b in range(2):
        cands = np.sort(_stable(coarse[b], m))
        fine = residual_score(query[b], packed, candidate_indices=cands)
        top = _stable(fine, k, tie_ids=cands)
        np.testing.assert_array_equal(ti[b], cands[top])
        np.testing.assert_array_equal(ts[b], fine[top])


# --------------------------------------------------- binary prefix + residual


def _binres(docs, offsets):
    from maxsim_amd.binres import binres_to_device, pack_binary_residual

    return binres_to_device(pack_binary_residual(docs, offsets))


def test_binres_scores_match_oracle(gpu, oracle):
    from maxsim_amd.binres import binres_score

    docs, offsets = ragged_fixture(150, 44, lo=1, hi=50)
    query = np.random.default_rng(45).standard_normal((3, 9, 128)).astype(np.float32)
    packed = _binres(docs, offsets)
    signs, a, _, rv, rs = oracle.pack_binary_residual(docs)
    _close(binres_score(query, packed, fused=False), oracle.binres_prefix_scores(query, signs, a, offsets), 1e-6)
    _close(binres_score(query, packed, fused=True),
           oracle.binres_fused_scores(query, signs, a, rv, rs, offsets), 1e-6)
    cand = np.random.default_rng(46).integers(0, 150, size=(3, 20)).astype(np.int64)
    _close(binres_score(query, packed, fused=True, candidate_indices=cand),
           oracle.binres_fused_scores(query, signs, a, rv, rs, offsets, candidates=cand), 1e-6)


@pytest.fixture
def prefix_scan():
    from maxsim_amd import _maxsim_hip

    yield _maxsim_hip.set_prefix_scan
    _maxsim_hip.set_prefix_scan(1)


@pytest.mark.parametrize("shape", [(3, 9), (4, 32), (2, 64), (1, 5), (8, 16)])
def test_binres_prefix_scan_is_bit_exact(gpu, oracle, prefix_scan, shape):
    """The prefix pass on the int8-query scan (sign documents: A bytes 0 / 2,
    the query sums in the MFMA's C operand) equals the oracle's prefix scores
    bit for bit; the generalized scorer agrees to rtol 1e-6."""
    from maxsim_amd.binres import binres_score

    docs, offsets = ragged_fixture(220, 53, lo=1, hi=90)  # short (< 16), long and one empty document
    batch, qt = shape
    query = np.random.default_rng(54 + qt).standard_normal((batch, qt, 128)).astype(np.float32)
    packed = _binres(docs, offsets)
    signs, a, _, _, _ = oracle.pack_binary_residual(docs)
    exp = oracle.binres_prefix_scores(query, signs, a, offsets)
    prefix_scan(1)
    np.testing.assert_array_equal(binres_score(query, packed, fused=False), exp)
    prefix_scan(0)
    _close(binres_score(query, packed, fused=False), exp, 1e-6)


@pytest.mark.parametrize("mode,qt", [(1, 32), (0, 32), (1, 64)])
def test_binres_cascade_equals_host_procedure(gpu, prefix_scan, mode, qt):
    """qt = 64: passes of 64 query rows (eight row blocks) in the rescoring
    pass's one-document-per-wave form."""
    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_cascade_topk, binres_score

    prefix_scan(mode)

    corpus = synthetic.make_corpus(400, 64, 192, seed=47)
    query = synthetic.make_queries(corpus, 4)
    if qt != query.shape[1]:
        query = np.concatenate([query, query[:, ::-1] * np.float32(0.5)], axis=1)
    packed = _binres(corpus.embeddings, corpus.offsets)
    k, m = 10, 128
    top_s, top_i = binres_cascade_topk(query, packed, k, candidates=m)
    coarse = binres_score(query, packed, fused=False)
    cands = np.stack([_stable(coarse[b], m) for b in range(4)])
    fine = binres_score(query, packed, fused=True, candidate_indices=cands)
    for b in range(4):
        order = _stable(fine[b], k, tie_ids=cands[b])
        np.testing.assert_array_equal(top_i[b], cands[b][order])
        np.testing.assert_array_equal(top_s[b], fine[b][order])
    # the source document of each query is found
    full = binres_score(query, packed, fused=True)
    full_top = np.stack([_stable(full[b], k) for b in range(4)])
    overlap = np.mean([len(set(top_i[b]) & set(full_top[b])) / k for b in range(4)])
    assert overlap >= 0.9


def _binres_recon(oracle, docs):
    """Reconstructed tokens a_t sign_t + s^r_t v^r_t (the oracle's packing):
    the fused similarity is q . x'_t, so the fp32-query fused scores are the
    dense MaxSim over them."""
    signs, a, _, rv, rs = oracle.pack_binary_residual(docs)
    sign = np.where(np.asarray(docs) >= 0, 1.0, -1.0)
    return (a[:, None].astype(np.float64) * sign + rs[:, None].astype(np.float64) * rv).astype(np.float32)


def test_binres_fp32_fused_scores_match_dense_oracle(gpu, oracle):
    """Fused scores with the fp32 query (three int8 limbs) against the dense
    MaxSim over the reconstructed tokens, at the fp32 bar (rtol 1e-5); the
    int8-query scores differ from it by the query rounding."""
    from maxsim_amd.binres import binres_score

    docs, offsets = ragged_fixture(150, 44, lo=1, hi=50)
    query = np.random.default_rng(45).standard_normal((3, 9, 128)).astype(np.float32)
    packed = _binres(docs, offsets)
    recon = _binres_recon(oracle, docs)
    exp = oracle.dense_scores(query, recon, offsets)
    got = binres_score(query, packed, fused=True, query_precision="fp32")
    _close(got, exp, 1e-5)
    assert np.max(np.abs(binres_score(query, packed, fused=True) - exp)) > np.max(np.abs(got - exp))
    cand = np.random.default_rng(46).integers(0, 150, size=(3, 20)).astype(np.int64)
    got_c = binres_score(query, packed, fused=True, candidate_indices=cand, query_precision="fp32")
    np.testing.assert_array_equal(got_c, np.take_along_axis(got, cand, axis=1))
    # the setting is per call: the handle is back on the int8 query
    assert packed.sign_data.get_rescore_limbs() == 1


@pytest.mark.parametrize("qt", [32, 64])
def test_binres_cascade_fp32_rescoring_equals_host_procedure(gpu, qt):
    """int8-query coarse pass -> top-M -> fp32-query rescoring -> top-k equals
    the same steps through the scoring calls; with every document a candidate
    it is the fp32 fused top-k."""
    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_cascade_topk, binres_score

    corpus = synthetic.make_corpus(400, 64, 192, seed=48)
    query = synthetic.make_queries(corpus, 3)
    if qt != query.shape[1]:
        query = np.random.default_rng(qt).standard_normal((3, qt, 128)).astype(np.float32)
    packed = _binres(corpus.embeddings, corpus.offsets)
    k, m = 10, 96
    top_s, top_i = binres_cascade_topk(query, packed, k, candidates=m, query_precision="fp32")
    coarse = binres_score(query, packed, fused=False)
    cands = np.stack([_stable(coarse[b], m) for b in range(3)])
    fine = binres_score(query, packed, fused=True, candidate_indices=cands, query_precision="fp32")
    for b in range(3):
        order = _stable(fine[b], k, tie_ids=cands[b])
        np.testing.assert_array_equal(top_i[b], cands[b][order])
        np.testing.assert_array_equal(top_s[b], fine[b][order])
    full = binres_score(query, packed, fused=True, query_precision="fp32")
    fs, fi = binres_cascade_topk(query, packed, k, candidates=400, query_precision="fp32")
    for b in range(3):
        np.testing.assert_array_equal(fi[b], _stable(full[b], k))
        np.testing.assert_array_equal(fs[b], full[b][fi[b]])


def test_binres_fp32_cascade_config5_scale_against_oracle(gpu, oracle):
    """The config-5 workload (4,096 documents of 64-192 tokens, query
    [4, 32, 128]) with the fp32-query rescoring of M = 512 candidates:
    * the fused fp32 scores of every document against the dense oracle over
      the reconstructed tokens, at the fp32 bar (rtol 1e-5);
    * the top-10 against the oracle pipeline (cascade.py:294-453): coarse
      scores from the oracle's int8-query prefix scores (which the device
      prefix pass equals bit for bit), stable top-512, dense fp32 rescoring
      of those candidates, top-10 by (score desc, document id asc).  The
      device's ten documents must be candidates of the oracle's coarse top-512
      and carry, in order, the oracle's ten best rescored values (the device's
      own fused scores agree with the oracle's to the fp32 bar, so documents
      whose oracle scores tie within it may trade places)."""
    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_cascade_topk, binres_score

    cfg = synthetic.CONFIGS[5]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"], seed=55)
    query = synthetic.make_queries(corpus, cfg["batch"], seed=56)
    docs, offsets = corpus.embeddings, corpus.offsets
    packed = _binres(docs, offsets)
    signs, a, _, _, _ = oracle.pack_binary_residual(docs)
    recon = _binres_recon(oracle, docs)
    k, m = 10, 512
    print("case: config-5 fp32 fused scores, 4096 docs", flush=True)
    full = binres_score(query, packed, fused=True, query_precision="fp32")
    _close(full, oracle.dense_scores(query, recon, offsets), 1e-5)
    print("case: config-5 fp32-rescoring cascade, M=512", flush=True)
    top_s, top_i = binres_cascade_topk(query, packed, k, candidates=m, query_precision="fp32")
    coarse = oracle.binres_prefix_scores(query, signs, a, offsets)
    for b in range(cfg["batch"]):
        cands = np.sort(_stable(coarse[b], m))
        fine = oracle.dense_scores(query[b:b + 1], recon, offsets, candidates=cands)[0]
        exp_pos = _stable(fine, k, tie_ids=cands)
        exp_scores = fine[exp_pos]
        pos = np.searchsorted(cands, top_i[b])
        assert np.all(pos < m) and np.array_equal(cands[pos], top_i[b]), "a result outside the coarse top-512"
        _close(fine[pos], exp_scores, 1e-5)
        _close(top_s[b], fine[pos], 1e-5)
        overlap = len(set(top_i[b].tolist()) & set(cands[exp_pos].tolist()))
        assert overlap >= k - 1, (b, overlap)


def test_binres_rescore_limbs_validation(gpu):
    docs, offsets = ragged_fixture(20, 3, lo=1, hi=20)
    h = _binres(docs, offsets).sign_data
    for bad in (0, 2, 4):
        with pytest.raises(ValueError):
            h.set_rescore_limbs(bad)
    h.set_rescore_limbs(3)
    assert h.get_rescore_limbs() == 3
    h.set_rescore_limbs(1)


# ------------------------------------------------------------- public API


def test_public_int4_routes(gpu, oracle):
    import maxsim_amd as ms

    docs, offsets = ragged_fixture(100, 48, lo=1, hi=30)
    query = np.random.default_rng(49).standard_normal((2, 6, 128)).astype(np.float32)
    packed = ms.pack_int4_symmetric(docs, offsets, scale_granularity="token")
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale)
    _close(ms.int4_maxsim(query, packed), exp)
    _close(ms.score(query, packed, reducer="topk2"),
           oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale, reducer="topk2"))
    s, i = ms.topk_int4_maxsim(query, packed, 5, reducer="smoothsim", temperature=0.5)
    full = ms.int4_maxsim(query, packed, reducer="smoothsim", temperature=0.5)
    for b in range(2):
        np.testing.assert_array_equal(i[b], _stable(full[b], 5))
    s8, i8 = ms.topk_int4_maxsim(query, packed, 5, prefer_int8_query=True)
    q8 = oracle.int4_int8q_scores(query, packed.values, offsets, token_scale=packed.token_scale)
    np.testing.assert_array_equal(i8, oracle.topk(q8, 5)[1])


def test_public_binary_routes(gpu, oracle):
    import maxsim_amd as ms

    docs, offsets = ragged_fixture(100, 50, lo=1, hi=30)
    query = np.random.default_rng(51).standard_normal((2, 6, 128)).astype(np.float32)
    packed = ms.pack_signs(docs, offsets, scale="doc", token_scale="mean_abs")
    got = ms.maxsim(query, packed)
    doc_of_token = np.repeat(np.arange(100), np.diff(offsets))
    signs = np.where(docs >= 0, 1.0, -1.0).astype(np.float32)
    recon = signs * (packed.token_scale * packed.scale[doc_of_token])[:, None]
    _close(got, oracle.dense_scores(query, recon, offsets))
    # +-1 integer queries take the sign-bit route; the result equals the float scoring
    plain = ms.pack_signs(docs, offsets)
    qi = np.where(query >= 0, 1, -1).astype(np.int8)
    s, i = ms.topk_maxsim(qi, plain, 8)
    full = ms.maxsim(qi.astype(np.float32), plain)
    for b in range(2):
        np.testing.assert_array_equal(i[b], _stable(full[b], 8))
        _close(s[b], full[b][i[b]], 1e-6)


def test_cascade_over_4096_docs_uses_general_selector(gpu):
    """More documents than the in-LDS selector holds: radix top-M + row sort."""
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, prefix_score, residual_int4_to_device, residual_score

    docs, offsets = ragged_fixture(5000, 52, lo=1, hi=6)
    query = np.random.default_rng(53).standard_normal((2, 4, 128)).astype(np.float32)
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    top_s, top_i = cascade_topk(query, packed, 5, candidates=300)
    coarse = prefix_score(query, packed)
    for b in range(2):
        cands = _stable(coarse[b], 300)
        fine = residual_score(query[b], packed, candidate_indices=cands)
        order = _stable(fine, 5, tie_ids=cands)
        np.testing.assert_array_equal(top_i[b], cands[order])
        np.testing.assert_array_equal(top_s[b], fine[order])


@pytest.mark.parametrize("reducer", ["weighted_maxsim", "topk2", "smoothsim"])
def test_public_topk_under_reducers_selects_on_device(gpu, reducer):
    """topk_maxsim / topk_int4_maxsim with a non-MaxSim reducer: the device
    selection equals the stable order of the full scores (_api.py:481-497,
    experimental.py:523-535)."""
    import maxsim_amd as ms

    docs, offsets = ragged_fixture(90, 54, lo=1, hi=25)
    rng = np.random.default_rng(55)
    query = rng.standard_normal((3, 5, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=(3, 5)).astype(np.float32) if reducer == "weighted_maxsim" else None
    kw = dict(reducer=reducer, query_weights=w, temperature=0.6)
    for packed, top, full in (
        (ms.pack_signs(docs, offsets, scale="doc", token_scale="mean_abs"), ms.topk_maxsim, ms.maxsim),
        (ms.pack_int4_symmetric(docs, offsets, scale_granularity="token"), ms.topk_int4_maxsim, ms.int4_maxsim),
    ):
        s, i = top(query, packed, 7, **kw)
        f = full(query, packed, **kw)
        for b in range(3):
            order = _stable(f[b], 7)
            np.testing.assert_array_equal(i[b], order)
            np.testing.assert_array_equal(s[b], f[b][order])
