"""GPU parity of the generalized scorer for dims above 128 (fp32 queries
against int4 and sign-bit documents) against the C oracle.

Dims above 128 are scored in 128-dim chunks whose MFMA dots add up in one
int32 accumulator (2 chunks up to 256 dims, 4 up to 512); the query's three
int8 limbs share one scale over the whole row.  The bar is the fp32 one of
the 128-dim tests: rtol 1e-5 plus atol 1e-5 x the largest |score|.  The
reference scores any dim (cu:1268-1323 int4, cu:171-235 binary); this build
takes up to 512 and says so above that.
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


def _binary_handle(oracle, docs, offsets):
    from maxsim_amd._maxsim_hip import CudaPackedDocs

    codes = oracle.pack_signs(docs)
    return codes, CudaPackedDocs(codes, offsets, docs.shape[1])


# ---------------------------------------------------------------- int4


@pytest.mark.parametrize("dim", [136, 200, 256, 384, 512])
@pytest.mark.parametrize("granularity", ["token", "tensor"])
@pytest.mark.parametrize("shape", [(2, 5), (4, 32)])
def test_int4_fp32_maxsim_wide(gpu, oracle, dim, granularity, shape):
    print(f"case: int4 dim={dim} {granularity} query {shape}", flush=True)
    docs, offsets = ragged_fixture(90, 61 + dim, lo=1, hi=40, dim=dim)
    query = np.random.default_rng(62 + dim).standard_normal((*shape, dim)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, granularity)
    got = h.maxsim_batch(query)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, scale=packed.scale, token_scale=packed.token_scale)
    _close(got, exp)
    empty = np.flatnonzero(np.diff(offsets) == 0)
    assert np.all(got[:, empty] == 0.0)


@pytest.mark.parametrize("reducer", REDUCERS)
@pytest.mark.parametrize("with_candidates", [False, True])
def test_int4_reducers_dim256(gpu, oracle, reducer, with_candidates):
    print(f"case: int4 dim=256 reducer={reducer} candidates={with_candidates}", flush=True)
    docs, offsets = ragged_fixture(70, 63, lo=1, hi=50, dim=256)
    rng = np.random.default_rng(64)
    query = rng.standard_normal((3, 24, 256)).astype(np.float32)
    weights = rng.uniform(0.5, 1.5, size=(3, 24)).astype(np.float32)
    cand = np.array([5, 1, 69, 0, 2, 33, 2], np.int64)
    packed, h = _int4_handle(docs, offsets, "token")
    w = weights if reducer == "weighted_maxsim" else None
    kwargs = dict(reducer=reducer, query_weights=w, temperature=0.35)
    got = h.score_candidates_batch(query, cand, **kwargs) if with_candidates else h.score_batch(query, **kwargs)
    exp = oracle.int4_fp32_scores(query, packed.values, offsets, scale=packed.scale, token_scale=packed.token_scale,
                                  reducer=reducer, weights=w, temperature=0.35,
                                  candidates=cand if with_candidates else None)
    _close(got, exp)


@pytest.mark.parametrize("dim", [256, 512])
def test_int4_topk_wide_is_stable_order(gpu, oracle, dim):
    docs, offsets = ragged_fixture(300, 65, lo=1, hi=30, dim=dim)
    query = np.random.default_rng(66).standard_normal((3, 7, dim)).astype(np.float32)
    packed, h = _int4_handle(docs, offsets, "token")
    scores = h.maxsim_batch(query)
    _close(scores, oracle.int4_fp32_scores(query, packed.values, offsets, token_scale=packed.token_scale))
    top_s, top_i = h.topk_batch(query, 10)
    for row, si, ii in zip(scores, top_s, top_i):
        order = np.lexsort((np.arange(row.shape[0]), -row))[:10]
        np.testing.assert_array_equal(ii, order)
        np.testing.assert_array_equal(si, row[order])


def _residual_handle(oracle, docs, offsets):
    from maxsim_amd._maxsim_hip import CudaInt4PackedDocs

    pcodes, pv, ps = oracle.pack_int4_token(docs)
    prefix = pv.astype(np.float32) * ps[:, None]
    rcodes, rv, rs = oracle.pack_int4_token(docs - prefix)
    h = CudaInt4PackedDocs(pcodes, offsets, docs.shape[1], 1.0)
    h.set_token_scale_vector(ps)
    h.set_residual_int4(rcodes, 1.0, rs)
    return h, prefix + rv.astype(np.float32) * rs[:, None]


@pytest.mark.parametrize("dim", [200, 256, 512])
@pytest.mark.parametrize("reducer", ["maxsim", "topk4", "smoothsim"])
def test_int4_residual_fused_wide(gpu, oracle, dim, reducer):
    print(f"case: int4 residual dim={dim} reducer={reducer}", flush=True)
    docs, offsets = ragged_fixture(60, 67, lo=1, hi=40, dim=dim)
    query = np.random.default_rng(68).standard_normal((2, 9, dim)).astype(np.float32)
    h, recon = _residual_handle(oracle, docs, offsets)
    got = h.score_residual_batch(query, reducer=reducer, temperature=0.5)
    _close(got, oracle.dense_scores(query, recon, offsets, reducer=reducer, temperature=0.5))


def test_int4_residual_cascade_dim256(gpu, oracle):
    """The int4-residual cascade at dim 256: coarse stable top-M of the prefix
    scores, per-row rescoring of the candidates with the fused scores, final
    order by (fused score desc, document id asc), as cascade.py:294-453."""
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4, prefix_score, residual_int4_to_device, residual_score

    docs, offsets = ragged_fixture(400, 69, lo=1, hi=60, dim=256)
    query = np.random.default_rng(70).standard_normal((3, 16, 256)).astype(np.float32)
    packed = residual_int4_to_device(pack_residual_int4(docs, offsets))
    k, m = 10, 64
    top_s, top_i = cascade_topk(query, packed, k, candidates=m)
    coarse = prefix_score(query, packed)
    for b in range(3):
        cands = np.lexsort((np.arange(coarse.shape[1]), -coarse[b]))[:m]
        fine = residual_score(query[b], packed, candidate_indices=cands)
        order = np.lexsort((cands, -fine))[:k]
        np.testing.assert_array_equal(top_i[b], cands[order])
        np.testing.assert_array_equal(top_s[b], fine[order])
    pcodes, pv, ps = oracle.pack_int4_token(docs)
    prefix = pv.astype(np.float32) * ps[:, None]
    _, rv, rs = oracle.pack_int4_token(docs - prefix)
    full = oracle.dense_scores(query, prefix + rv.astype(np.float32) * rs[:, None], offsets)
    _close(top_s, np.take_along_axis(full, top_i, axis=1))


def test_int4_dim_above_512_is_not_supported(gpu):
    docs, offsets = ragged_fixture(10, 71, lo=1, hi=5, dim=520)
    _, h = _int4_handle(docs, offsets, "token")
    with pytest.raises(NotImplementedError, match="dim <= 512"):
        h.maxsim_batch(np.ones((1, 2, 520), np.float32))


# --------------------------------------------------------------- binary


@pytest.mark.parametrize("dim", [136, 256, 392, 512])
@pytest.mark.parametrize("shape", [(2, 5), (4, 32)])
def test_binary_fp32_maxsim_wide(gpu, oracle, dim, shape):
    print(f"case: binary dim={dim} query {shape}", flush=True)
    docs, offsets = ragged_fixture(80, 72 + dim, lo=1, hi=40, dim=dim)
    query = np.random.default_rng(73 + dim).standard_normal((*shape, dim)).astype(np.float32)
    codes, h = _binary_handle(oracle, docs, offsets)
    got = h.maxsim_batch(query, scale=0.5)
    exp = np.stack([oracle.binary_lut_maxsim(qb, codes, offsets, dim, 0.5) for qb in query])
    _close(got, exp)
    top_s, top_i = h.topk_batch(query, 5, scale=0.5)
    for row, si, ii in zip(got, top_s, top_i):
        order = np.lexsort((np.arange(row.shape[0]), -row))[:5]
        np.testing.assert_array_equal(ii, order)
        np.testing.assert_array_equal(si, row[order])


@pytest.mark.parametrize("reducer", REDUCERS)
def test_binary_reducers_with_scales_dim256(gpu, oracle, reducer):
    docs, offsets = ragged_fixture(50, 74, lo=1, hi=30, dim=256)
    rng = np.random.default_rng(75)
    query = rng.standard_normal((2, 5, 256)).astype(np.float32)
    weights = rng.uniform(0.5, 1.5, size=(2, 5)).astype(np.float32)
    cand = np.array([5, 1, 49, 0, 2], np.int64)
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


def test_binary_wide_int8q_and_limits(gpu, oracle):
    """The int8-query and sign-query forms stay dim-128 forms (as the
    reference's quantize_query_int8_seq_dim128 path); dims above 512 are
    refused at handle creation."""
    from maxsim_amd._maxsim_hip import CudaPackedDocs

    docs, offsets = ragged_fixture(20, 76, lo=1, hi=10, dim=256)
    _, h = _binary_handle(oracle, docs, offsets)
    with pytest.raises(ValueError, match="dim=128"):
        h.maxsim_batch_int8q(np.ones((1, 2, 256), np.float32))
    big = oracle.pack_signs(np.ones((4, 520), np.float32))
    with pytest.raises(NotImplementedError, match="dim <= 512"):
        CudaPackedDocs(big, np.array([0, 4], np.int64), 520)
