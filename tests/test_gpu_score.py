"""GPU parity of the generalized scoring path (score.hip) against the C oracle.

fp32 queries are scored with three int8 limbs; the bar is the reference's
fp32 tolerance (rtol 1e-5, atol 1e-5 relative to the score scale).  Integer
paths (sign-bit queries) are bit-exact.
"""
import numpy as np
import pytest

from conftest import ragged_fixture

pytestmark = pytest.mark.gpu

REDUCERS = ("maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim")
RTOL = 1e-5


def _close(actual, expected, rtol=RTOL):
    scale = max(1.0, float(np.max(np.abs(expected)))) if expected.size else 1.0
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=rtol * scale)


def _int4_handle(docs, offsets, granularity):
    from maxsim_amd._maxsim_hip import CudaInt4PackedDocs
    from maxsim_amd.experimental import pack_int4_symmetric

    packed = pack_int4_symmetric(docs, offsets, scale_granularity=granularity)
    h = CudaInt4PackedDocs(packed.data, packed.doc_offsets, packed.dim, packed.scale)
    if packed.token_scale is not None:
        h.set_token_scale_vector(packed.token_scale)
    return packed, h


def _reducer_fixture(dim=128):
    """tests/test_cuda_reducers.py:18-29."""
    rng = np.random.default_rng(20260713)
    lengths = np.array([0, 1, 2, 3, 4, 7], np.int64)
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    docs = rng.normal(size=(int(offsets[-1]), dim)).astype(np.float32)
    query = rng.normal(size=(2, 5, dim)).astype(np.float32)
    weights = np.array([[1.0, 0.25, 1.5, 0.0, 0.75], [0.5, 2.0, 0.125, 1.0, 0.25]], np.float32)
    candidates = np.array([5, 1, 5, 0, 2], np.int64)
    return docs, offsets, query, weights, candidates


# ---------------------------------------------------------------- int4 fp32


@pytest.mark.parametrize("granularity", ["token", "tensor"])
@pytest.mark.parametrize("shape", [(2, 5), (1, 1), (4, 32), (3, 40), (1, 130)])
def test_int4_fp32_maxsim_ragged(gpu, oracle, granularity, shape):
    docs, offsets = ragged_fixture(150, 71, lo=1, hi=40)
    query = np.random.default_rng(73).standard_normal((*shape, 128)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, granularity)
    got = h.maxsim_batch(query)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, scale=packed.scale, token_scale=packed.token_scale)
    _close(got, exp)
    empty = np.flatnonzero(np.diff(offsets) == 0)
    assert np.all(got[:, empty] == 0.0)


@pytest.mark.parametrize("reducer", REDUCERS)
@pytest.mark.parametrize("granularity", ["token", "tensor"])
@pytest.mark.parametrize("with_candidates", [False, True])
def test_int4_reducers_match_oracle(gpu, oracle, reducer, granularity, with_candidates):
    docs, offsets, query, weights, cand = _reducer_fixture()
    packed, h = _int4_handle(docs, offsets, granularity)
    w = weights if reducer == "weighted_maxsim" else None
    kwargs = dict(reducer=reducer, query_weights=w, temperature=0.35)
    got = h.score_candidates_batch(query, cand, **kwargs) if with_candidates else h.score_batch(query, **kwargs)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, scale=packed.scale, token_scale=packed.token_scale,
                                  reducer=reducer, weights=w, temperature=0.35,
                                  candidates=cand if with_candidates else None)
    _close(got, exp)


@pytest.mark.parametrize("reducer", REDUCERS)
def test_int4_reducers_ragged_many_rows(gpu, oracle, reducer):
    """Ragged docs up to 70 tokens (several tiles), 3 x 24 query rows (two passes)."""
    docs, offsets = ragged_fixture(120, 5, lo=1, hi=70)
    rng = np.random.default_rng(6)
    query = rng.standard_normal((3, 24, 128)).astype(np.float32)
    weights = rng.uniform(0.5, 1.5, size=(3, 24)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, "token")
    w = weights if reducer == "weighted_maxsim" else None
    got = h.score_batch(query, reducer=reducer, query_weights=w, temperature=0.7)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale, reducer=reducer,
                                  weights=w, temperature=0.7)
    _close(got, exp)


@pytest.mark.parametrize("reducer", REDUCERS)
@pytest.mark.parametrize("corpus", ["tiny_docs", "three_docs"])
def test_int4_work_units(gpu, oracle, reducer, corpus):
    """The row-block pipeline's work units (fp32 queries of more than 32
    rows over the whole corpus): 3000 documents of 0..20 tokens, a fifth
    empty (units of several documents each), or three documents (fewer
    units than the workgroup's eight waves)."""
    print(f"case: work units corpus={corpus} reducer={reducer}", flush=True)
    if corpus == "tiny_docs":
        rng = np.random.default_rng(17)
        lengths = rng.integers(0, 21, size=3000)
        lengths[rng.random(3000) < 0.2] = 0
        offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
        docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    else:
        docs, offsets = ragged_fixture(3, 18, lo=1, hi=90, empty=None)
    rng = np.random.default_rng(19)
    query = rng.standard_normal((2, 40, 128)).astype(np.float32)
    weights = rng.uniform(0.5, 1.5, size=(2, 40)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, "token")
    w = weights if reducer == "weighted_maxsim" else None
    got = h.score_batch(query, reducer=reducer, query_weights=w, temperature=0.7)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale, reducer=reducer,
                                  weights=w, temperature=0.7)
    _close(got, exp)
    assert np.all(got[:, np.diff(offsets) == 0] == 0.0)


@pytest.mark.parametrize("shape", ["1d", "1xQ", "BxQ"])
def test_weight_shapes(gpu, oracle, shape):
    docs, offsets, query, weights, _ = _reducer_fixture()
    packed, h = _int4_handle(docs, offsets, "token")
    w = {"1d": weights[0], "1xQ": weights[:1], "BxQ": weights}[shape]
    got = h.score_batch(query, reducer="weighted_maxsim", query_weights=w)
    full = np.broadcast_to(np.asarray(w).reshape(-1, 5), (2, 5))
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale,
                                  reducer="weighted_maxsim", weights=full)
    _close(got, exp)


def test_weights_change_between_calls_on_one_handle(gpu, oracle):
    """The handle keeps the last weight vector on the device and copies a
    new one only when it differs: alternating weights (including a change of
    sign of zero only) each give the oracle's scores."""
    docs, offsets, query, weights, _ = _reducer_fixture()
    packed, h = _int4_handle(docs, offsets, "token")
    w2 = weights[::-1].copy()
    w3 = weights.copy()
    w3[0, 3] = -0.0
    for w in (weights, w2, weights, w3, w3, weights):
        got = h.score_batch(query, reducer="weighted_maxsim", query_weights=w)
        exp = oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale,
                                      reducer="weighted_maxsim", weights=w)
        _close(got, exp)
        if w is w3:
            np.testing.assert_array_equal(np.signbit(got), np.signbit(exp))


def test_smoothsim_large_values_stay_finite(gpu):
    docs, offsets, query, _, _ = _reducer_fixture()
    _, h = _int4_handle(docs, offsets, "token")
    got = h.score_batch(query * np.float32(1e5), reducer="smoothsim", temperature=0.125)
    assert np.all(np.isfinite(got))


def test_candidates_equal_gather_of_full(gpu):
    docs, offsets, query, weights, cand = _reducer_fixture()
    _, h = _int4_handle(docs, offsets, "token")
    for reducer in REDUCERS:
        w = weights if reducer == "weighted_maxsim" else None
        full = h.score_batch(query, reducer=reducer, query_weights=w, temperature=0.5)
        part = h.score_candidates_batch(query, cand, reducer=reducer, query_weights=w, temperature=0.5)
        np.testing.assert_array_equal(part, full[:, cand])


def test_int4_fp32_topk_is_stable_order(gpu, oracle):
    docs, offsets = ragged_fixture(300, 11, lo=1, hi=30)
    query = np.random.default_rng(12).standard_normal((3, 7, 128)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, "token")
    scores = h.maxsim_batch(query)
    top_s, top_i = h.topk_batch(query, 10)
    for row, si, ii in zip(scores, top_s, top_i):
        order = np.lexsort((np.arange(row.shape[0]), -row))[:10]
        np.testing.assert_array_equal(ii, order)
        np.testing.assert_array_equal(si, row[order])


@pytest.mark.parametrize("dim", [64, 128])
def test_int4_fp32_topk_consecutive_calls(gpu, oracle, dim):
    """Synchronous top-k calls stage their query (widened to 128 dims) and
    their results in the handle's pinned host buffers: calls in a row with
    other queries, shapes and k each match the device's own full scores."""
    docs, offsets = ragged_fixture(200, 15, lo=1, hi=30, dim=dim)
    packed, h = _int4_handle(docs, offsets, "token")
    rng = np.random.default_rng(16)
    queries = [rng.standard_normal(s + (dim,)).astype(np.float32) for s in [(3, 7), (1, 40), (2, 2)]]
    for i, (query, k) in enumerate([(queries[0], 10), (queries[1], 3), (queries[0], 10), (queries[2], 25)]):
        print(f"call {i}: query {query.shape} k={k}", flush=True)
        scores = h.maxsim_batch(query)
        _close(scores, oracle.int4_fp32_scores(query, packed.values, offsets, scale=packed.scale,
                                               token_scale=packed.token_scale))
        top_s, top_i = h.topk_batch(query, k)
        for row, si, ii in zip(scores, top_s, top_i):
            order = np.lexsort((np.arange(row.shape[0]), -row))[:k]
            np.testing.assert_array_equal(ii, order)
            np.testing.assert_array_equal(si, row[order])


@pytest.mark.parametrize("dim", [8, 64])
def test_int4_small_dim(gpu, oracle, dim):
    docs, offsets = ragged_fixture(40, 13, lo=1, hi=20, dim=dim)
    query = np.random.default_rng(14).standard_normal((2, 3, dim)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, "token")
    _close(h.maxsim_batch(query), oracle.int4_fp32_scores(query, packed.values, offsets,
                                                           token_scale=packed.token_scale))


def test_scale_before_max_kat_10(gpu):
    """tests/test_int4_reference.py:105-126 through the device path."""
    docs = np.array([[1.0] * 8, [10.0] + [0.0] * 7], np.float32)
    _, h = _int4_handle(docs, np.array([0, 2]), "token")
    np.testing.assert_allclose(h.maxsim_batch(np.ones((1, 1, 8), np.float32)), [[10.0]], rtol=1e-6)


# ------------------------------------------------------------ int4 residual


def _residual_handle(oracle, docs, offsets):
    from maxsim_amd._maxsim_hip import CudaInt4PackedDocs

    pcodes, pv, ps = oracle.pack_int4_token(docs)
    prefix = pv.astype(np.float32) * ps[:, None]
    rcodes, rv, rs = oracle.pack_int4_token(docs - prefix)
    h = CudaInt4PackedDocs(pcodes, offsets, docs.shape[1], 1.0)
    h.set_token_scale_vector(ps)
    h.set_residual_int4(rcodes, 1.0, rs)
    recon = prefix + rv.astype(np.float32) * rs[:, None]
    return h, prefix, recon


@pytest.mark.parametrize("reducer", REDUCERS)
def test_residual_fused_matches_oracle(gpu, oracle, reducer):
    docs, offsets, query, weights, cand = _reducer_fixture()
    h, _, recon = _residual_handle(oracle, docs, offsets)
    w = weights if reducer == "weighted_maxsim" else None
    got = h.score_residual_batch(query, reducer=reducer, query_weights=w, temperature=0.35)
    _close(got, oracle.dense_scores(query, recon, offsets, reducer=reducer, weights=w, temperature=0.35))
    got_c = h.score_residual_candidates_batch(query, cand, reducer=reducer, query_weights=w, temperature=0.35)
    np.testing.assert_array_equal(got_c, got[:, cand])


def test_residual_kat_fused_not_separate(gpu, oracle):
    """tests/test_cascade.py:242-275 on the device."""
    docs = np.array(
        [[0, 20, 13, 12, 8, 5, -7, 20], [-1, -12, 14, -14, 15, 5, -16, -19], [-2, -19, -15, 1, 19, -1, 13, 17]],
        np.float32,
    )
    offsets = np.array([0, 3], np.int64)
    query = np.array([[[2, 1, 0, 0, -2, 0, -1, -2]]], np.float32)
    h, prefix, recon = _residual_handle(oracle, docs, offsets)
    fused = h.score_residual_batch(query)
    _close(fused, oracle.dense_scores(query, recon, offsets))
    separate = oracle.dense_scores(query, prefix, offsets) + oracle.dense_scores(query, recon - prefix, offsets)
    assert not np.allclose(fused, separate, rtol=0, atol=1e-6)


def test_residual_requires_loaded_stream(gpu):
    docs, offsets, query, _, _ = _reducer_fixture()
    _, h = _int4_handle(docs, offsets, "token")
    with pytest.raises(ValueError, match="residual int4 data was requested"):
        h.score_residual_batch(query)


# ------------------------------------------------------------------- binary


def _binary_handle(oracle, docs, offsets):
    from maxsim_amd._maxsim_hip import CudaPackedDocs

    codes = oracle.pack_signs(docs)
    return codes, CudaPackedDocs(codes, offsets, docs.shape[1])


@pytest.mark.parametrize("shape", [(1, 2), (2, 5), (4, 32), (2, 70)])
def test_binary_fp32_maxsim_matches_reference_lut(gpu, oracle, shape):
    docs, offsets = ragged_fixture(120, 21, lo=1, hi=40)
    query = np.random.default_rng(22).standard_normal((*shape, 128)).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    got = h.maxsim_batch(query, scale=0.5)
    exp = np.stack([oracle.binary_lut_maxsim(qb, codes, offsets, 128, 0.5) for qb in query])
    _close(got, exp)


def test_binary_fp32_topk_consecutive_calls(gpu, oracle):
    """The binary handle's synchronous top-k also stages its query and results
    in pinned host memory: calls in a row with other queries, shapes and k
    each match the reference LUT scores of their own query."""
    docs, offsets = ragged_fixture(150, 26, lo=1, hi=40)
    codes, h = _binary_handle(oracle, docs, offsets)
    rng = np.random.default_rng(27)
    queries = [rng.standard_normal(s + (128,)).astype(np.float32) for s in [(2, 5), (3, 32), (1, 2)]]
    for i, (query, k) in enumerate([(queries[0], 7), (queries[1], 20), (queries[0], 7), (queries[2], 3)]):
        print(f"call {i}: query {query.shape} k={k}", flush=True)
        scores = h.maxsim_batch(query)
        _close(scores, np.stack([oracle.binary_lut_maxsim(qb, codes, offsets, 128, 1.0) for qb in query]))
        top_s, top_i = h.topk_batch(query, k)
        for row, si, ii in zip(scores, top_s, top_i):
            order = np.lexsort((np.arange(row.shape[0]), -row))[:k]
            np.testing.assert_array_equal(ii, order)
            np.testing.assert_array_equal(si, row[order])


@pytest.mark.parametrize("reducer", REDUCERS)
def test_binary_reducers_with_scales(gpu, oracle, reducer):
    docs, offsets, query, weights, cand = _reducer_fixture()
    rng = np.random.default_rng(23)
    ts = rng.uniform(0.25, 1.75, size=docs.shape[0]).astype(np.float32)
    sv = rng.uniform(0.5, 2.0, size=offsets.shape[0] - 1).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    h.set_token_scale_vector(ts)
    h.set_scale_vector(sv)
    w = weights if reducer == "weighted_maxsim" else None
    got = h.score_candidates_batch(query, cand, reducer=reducer, query_weights=w, temperature=0.7,
                                   use_scale_vector=True, use_token_scale=True)
    doc_of_token = np.repeat(np.arange(offsets.shape[0] - 1), np.diff(offsets))
    signs = np.where(docs >= 0, 1.0, -1.0).astype(np.float32)
    recon = signs * (ts * sv[doc_of_token])[:, None]
    exp = oracle.dense_scores(query, recon, offsets, reducer=reducer, weights=w, temperature=0.7, candidates=cand)
    _close(got, exp)


def test_binary_scale_override_and_errors(gpu, oracle):
    docs, offsets, query, _, _ = _reducer_fixture()
    codes, h = _binary_handle(oracle, docs, offsets)
    with pytest.raises(ValueError, match="scale vector was requested"):
        h.maxsim_batch(query, use_scale_vector=True)
    with pytest.raises(ValueError, match="token scale vector was requested"):
        h.maxsim_batch(query, use_token_scale=True)
    sv = np.linspace(0.5, 1.5, offsets.shape[0] - 1).astype(np.float32)
    got = h.score_batch(query, scale_vector_override=sv)
    base = h.maxsim_batch(query)
    _close(got, base * sv[None, :])


def test_binary_int8q_closed_form(gpu, oracle):
    """2 (q8 . bits) - sum(q8) with q8 = rint(q * (1 / sigma)) (cu:1328-1447)."""
    docs, offsets = ragged_fixture(80, 24, lo=1, hi=30)
    query = np.random.default_rng(25).standard_normal((2, 6, 128)).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    got = h.maxsim_batch_int8q(query)
    signs = np.where(docs >= 0, 1, -1).astype(np.int64)
    exp = np.zeros_like(got)
    for b in range(2):
        m = np.max(np.abs(query[b]), axis=1)
        s = np.where(m == 0, np.float32(1), (m / np.float32(127)).astype(np.float32)).astype(np.float32)
        inv = (np.float32(1) / s).astype(np.float32)
        q8 = np.clip(np.rint((query[b] * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int64)
        for d in range(offsets.shape[0] - 1):
            lo, hi = offsets[d], offsets[d + 1]
            if lo == hi:
                continue
            best = (q8 @ signs[lo:hi].T).max(axis=1).astype(np.float32)
            acc = np.float32(0)
            for qi in range(6):
                acc = np.float32(acc + best[qi] * s[qi])
            exp[b, d] = acc
    _close(got, exp, rtol=1e-6)


def test_hamming_bit_exact(gpu, oracle):
    docs, offsets = ragged_fixture(200, 26, lo=1, hi=50)
    q = np.random.default_rng(27).standard_normal((3, 9, 128)).astype(np.float32)
    qbits = oracle.pack_signs(q.reshape(-1, 128)).reshape(3, 9, 16)
    codes, h = _binary_handle(oracle, docs, offsets)
    got = h.hamming_batch(qbits)
    exp = oracle.binary_hamming_maxsim(qbits, codes, offsets, 128)
    np.testing.assert_array_equal(got, exp)
    top_s, top_i = h.topk_hamming(qbits, 10)
    ref_s, ref_i = oracle.topk(exp.astype(np.float32), 10)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s, ref_s)


def test_hamming_many_query_rows(gpu, oracle):
    """More query rows than one pass (rows > 128): 5 x 40 rows."""
    docs, offsets = ragged_fixture(64, 28, lo=1, hi=40)
    q = np.random.default_rng(29).standard_normal((5, 40, 128)).astype(np.float32)
    qbits = oracle.pack_signs(q.reshape(-1, 128)).reshape(5, 40, 16)
    codes, h = _binary_handle(oracle, docs, offsets)
    np.testing.assert_array_equal(h.hamming_batch(qbits), oracle.binary_hamming_maxsim(qbits, codes, offsets, 128))


@pytest.mark.parametrize("dim", [16, 64])
def test_binary_small_dim(gpu, oracle, dim):
    docs, offsets = ragged_fixture(30, 30, lo=1, hi=12, dim=dim)
    query = np.random.default_rng(31).standard_normal((2, 4, dim)).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    got = h.maxsim_batch(query)
    exp = np.stack([oracle.binary_lut_maxsim(qb, codes, offsets, dim) for qb in query])
    _close(got, exp)


def test_score_async_weights_ordered_on_side_stream(gpu):
    """Back-to-back msim_int4_score_async calls with different reducer weights
    on a non-blocking stream: each call's weights are uploaded on that stream,
    after the previous call's kernel, so every output equals the synchronous
    API's scores for its own weights."""
    import torch

    from maxsim_amd import _maxsim_hip, synthetic
    from maxsim_amd._native import check, ptr

    corpus = synthetic.make_corpus(2048, 64, 192, seed=91)
    query = synthetic.make_queries(corpus, 4)
    _, h = _int4_handle(corpus.embeddings, corpus.offsets, "token")
    b, q = query.shape[:2]
    rng = np.random.default_rng(92)
    weights = [rng.uniform(0.5, 1.5, size=(b, q)).astype(np.float32) for _ in range(6)]
    dq = torch.from_numpy(query).cuda()
    outs = [torch.empty((b, 2048), dtype=torch.float32, device="cuda") for _ in weights]
    side = torch.cuda.Stream()
    sptr = _maxsim_hip._stream_ptr(side)
    torch.cuda.synchronize()
    for w, out in zip(weights, outs):
        check(h._lib.msim_int4_score_async(h._h, ptr(dq), b, q, b"weighted_maxsim", ptr(w), 2, b, q, 1.0, 0,
                                           ptr(out), sptr))
    side.synchronize()
    for w, out in zip(weights, outs):
        np.testing.assert_array_equal(out.cpu().numpy(), h.score_batch(query, "weighted_maxsim", w))


def test_maxsim_cuda_free_functions_match_reference_lut(gpu, oracle):
    """maxsim_cuda / maxsim_cuda_batch (cuda_extension.cu:3308-3412), the
    handle module's free functions the reference's _score_binary calls for
    host-resident sign-bit documents (_api.py:357-371): against the oracle
    LUT (pinned to the reference's compiled maxsim_lut), with a scale, and
    equal to the resident handle's scores."""
    from maxsim_amd import _maxsim_hip

    docs, offsets = ragged_fixture(120, 61, lo=1, hi=30)
    query = np.random.default_rng(62).standard_normal((3, 7, 128)).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    one = _maxsim_hip.maxsim_cuda(query[0], codes, offsets, 128, 0.5)
    _close(one, oracle.binary_lut_maxsim(query[0], codes, offsets, 128, 0.5))
    batch = _maxsim_hip.maxsim_cuda_batch(query, codes, offsets, 128)
    _close(batch, np.stack([oracle.binary_lut_maxsim(qb, codes, offsets, 128) for qb in query]))
    np.testing.assert_array_equal(batch, h.maxsim_batch(query))
    np.testing.assert_array_equal(_maxsim_hip.maxsim_cuda(query[1], codes, offsets, 128), batch[1])


@pytest.mark.parametrize("reducer", ["maxsim", "topk2", "topk4", "smoothsim"])
def test_scores_repeat_and_agree_across_row_splits(gpu, reducer):
    """The same documents scored for four batch rows at once (passes of 64 or
    128 query rows) and for one row at a time (passes of 32 rows) run
    different kernel instantiations over identical per-row arithmetic, so the
    scores must agree bit for bit, and repeating a call must reproduce them.
    Multi-tile documents (up to 150 tokens) exercise the tile look-ahead; a
    read of an MFMA accumulator before its result lands shows up here as
    small, run-to-run varying differences."""
    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_score, binres_to_device, pack_binary_residual
    from maxsim_amd.cascade import pack_residual_int4, residual_int4_to_device, residual_score

    c = synthetic.make_corpus(300, 1, 150, seed=77)
    query = synthetic.make_queries(c, 4)
    p = residual_int4_to_device(pack_residual_int4(c.embeddings, c.offsets))
    full = residual_score(query, p, reducer=reducer, temperature=0.7)
    for _ in range(3):
        np.testing.assert_array_equal(residual_score(query, p, reducer=reducer, temperature=0.7), full)
        rows = np.stack([residual_score(query[r:r + 1], p, reducer=reducer, temperature=0.7)[0] for r in range(4)])
        np.testing.assert_array_equal(rows, full)
    if reducer == "maxsim":
        b = binres_to_device(pack_binary_residual(c.embeddings, c.offsets))
        for fused in (False, True):
            ref = binres_score(query, b, fused=fused)
            for _ in range(3):
                rows = np.stack([binres_score(query[r:r + 1], b, fused=fused)[0] for r in range(4)])
                np.testing.assert_array_equal(rows, ref)


@pytest.fixture
def hamming_fp4():
    from maxsim_amd import _maxsim_hip

    yield _maxsim_hip.set_hamming_fp4
    _maxsim_hip.set_hamming_fp4(1)


@pytest.mark.parametrize("mode", [1, 0])
@pytest.mark.parametrize("shape", [(3, 9), (5, 40), (9, 32), (1, 300)])
def test_hamming_fp4_and_int8_forms_bit_exact(gpu, oracle, hamming_fp4, mode, shape):
    """Sign-query MaxSim on the fp4 kernel (mode 1: 256 query rows per pass,
    +-1 fp4 operands) and on the int8 scorer (mode 0) against the oracle's
    Hamming MaxSim, bit for bit: passes that hold whole batch rows (the
    kernel sums them) and passes that do not (rows summed afterwards), short
    and long documents and an empty one."""
    print(f"case: hamming mode={mode} shape={shape}", flush=True)
    hamming_fp4(mode)
    docs, offsets = ragged_fixture(150, 61 + shape[1], lo=1, hi=70)
    q = np.random.default_rng(62 + shape[0]).standard_normal((*shape, 128)).astype(np.float32)
    qbits = oracle.pack_signs(q.reshape(-1, 128)).reshape(*shape, 16)
    codes, h = _binary_handle(oracle, docs, offsets)
    exp = oracle.binary_hamming_maxsim(qbits, codes, offsets, 128)
    np.testing.assert_array_equal(h.hamming_batch(qbits), exp)
    top_s, top_i = h.topk_hamming(qbits, 7)
    ref_s, ref_i = oracle.topk(exp.astype(np.float32), 7)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s, ref_s)
