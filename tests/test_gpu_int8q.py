"""GPU parity: int4 x int8-query MaxSim and top-k against the C oracle.

The oracle restates tests/test_int4_int8q.py:7-26 of the reference; the device
path matches it bit for bit (integer dots exactly, the float64 pairwise sum in
numpy's order), so scores are compared with assert_array_equal and top-k ids
must be identical.
"""
import numpy as np
import pytest

import maxsim_amd as maxsim
from conftest import ragged_fixture
from maxsim_amd import synthetic
from maxsim_amd.experimental import int4_maxsim_int8q, int4_to_device, pack_int4_symmetric

pytestmark = pytest.mark.gpu


def _scores(oracle, packed, query):
    return oracle.int4_int8q_scores(query, packed.values, packed.doc_offsets,
                                    token_scale=packed.token_scale, scale=float(packed.scale))


@pytest.mark.parametrize("granularity", ["token", "tensor"])
@pytest.mark.parametrize("shape", [(2, 5), (1, 1), (3, 8), (4, 32), (1, 32), (3, 32), (5, 24), (9, 16), (2, 130)])
def test_int8q_scores_bit_exact_ragged(gpu, oracle, granularity, shape):
    b, q = shape
    print(f"case granularity={granularity} B={b} Q={q}", flush=True)
    docs, offsets = ragged_fixture(150, seed=71)
    query = np.random.default_rng(73).standard_normal((b, q, 128)).astype(np.float32)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=granularity)
    device = int4_to_device(packed)
    actual = int4_maxsim_int8q(query, device)
    np.testing.assert_array_equal(actual, _scores(oracle, packed, query))


def test_int8q_zero_query_rows_and_empty_docs(gpu, oracle):
    docs, offsets = ragged_fixture(10, seed=79)
    empty = int(np.flatnonzero(np.diff(offsets) == 0)[0])
    query = np.random.default_rng(83).standard_normal((1, 4, 128)).astype(np.float32)
    query[0, -1] = 0.0
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    actual = int4_maxsim_int8q(query, int4_to_device(packed))
    assert actual[0, empty] == 0.0
    np.testing.assert_array_equal(actual, _scores(oracle, packed, query))


def test_int8q_scale_before_max_kat(gpu):
    """tests/test_int4_int8q.py:109-134: the token scale is applied before the max -> 640.0."""
    docs = np.stack([np.ones(128, np.float32),
                     np.concatenate([np.full(64, 10.0, np.float32), np.zeros(64, np.float32)])])
    packed = pack_int4_symmetric(docs, np.array([0, 2], np.int64), scale_granularity="token")
    actual = int4_maxsim_int8q(np.ones((1, 1, 128), np.float32), int4_to_device(packed))
    assert actual.tolist() == [[640.0]]


@pytest.mark.parametrize("granularity", ["token", "tensor"])
def test_int8q_topk_matches_stable_order(gpu, oracle, granularity):
    docs, offsets = ragged_fixture(150, seed=89)
    query = np.random.default_rng(97).standard_normal((2, 4, 128)).astype(np.float32)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=granularity)
    device = int4_to_device(packed)
    scores = int4_maxsim_int8q(query, device)
    top_scores, top_ids = device.data.topk_batch_int8q(query, 10)
    ref_scores, ref_ids = oracle.topk(scores, 10)
    np.testing.assert_array_equal(top_ids, ref_ids)
    np.testing.assert_array_equal(top_scores, ref_scores)


def test_int8q_topk_consecutive_calls_see_their_own_query(gpu, oracle):
    """The synchronous top-k stages the query and its results in one pinned
    host buffer per handle that the kernels read and write directly: calls in
    a row, with different queries, shapes and k (the buffer grows, then is
    reused by a smaller call), each return the oracle's answer for their own
    query."""
    docs, offsets = ragged_fixture(300, seed=31)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    device = int4_to_device(packed)
    rng = np.random.default_rng(37)
    queries = [rng.standard_normal(s).astype(np.float32) for s in [(2, 8, 128), (4, 32, 128), (1, 3, 128)]]
    for i, (query, k) in enumerate([(queries[0], 5), (queries[1], 10), (queries[0], 5), (queries[2], 32),
                                    (queries[1], 1)]):
        print(f"call {i}: query {query.shape} k={k}", flush=True)
        top_scores, top_ids = device.data.topk_batch_int8q(query, k)
        ref_scores, ref_ids = oracle.topk(_scores(oracle, packed, query), k)
        np.testing.assert_array_equal(top_ids, ref_ids)
        np.testing.assert_array_equal(top_scores, ref_scores)


def test_topk_ties_prefer_lower_doc_id(gpu):
    """Equal documents tie; the lower id wins (tests/test_int4_reference.py:129-146)."""
    docs = np.array([[1] * 128, [1] * 128, [-1] * 128, [1] * 128], np.float32)
    packed = pack_int4_symmetric(docs, np.arange(5, dtype=np.int64), scale_granularity="token")
    scores, ids = int4_to_device(packed).data.topk_batch_int8q(np.ones((1, 1, 128), np.float32), 4)
    assert ids.tolist() == [[0, 1, 3, 2]]
    assert scores[0, 0] == scores[0, 1] == scores[0, 2]


def test_config2_full_size_parity(gpu, oracle):
    """BASELINE config 2 at full size: every score bit-exact, top-10 identical."""
    cfg = synthetic.CONFIGS[2]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query = synthetic.make_queries(corpus, cfg["batch"])
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    device = int4_to_device(packed)
    actual = device.data.maxsim_batch_int8q(query)
    expected = _scores(oracle, packed, query)
    np.testing.assert_array_equal(actual, expected)
    top_scores, top_ids = device.data.topk_batch_int8q(query, 10)
    ref_scores, ref_ids = oracle.topk(expected, 10)
    np.testing.assert_array_equal(top_ids, ref_ids)
    np.testing.assert_array_equal(top_scores, ref_scores)


def test_int8q_repeat_is_deterministic(gpu):
    docs, offsets = ragged_fixture(64, seed=5, lo=0, hi=40)
    query = np.random.default_rng(6).standard_normal((4, 32, 128)).astype(np.float32)
    device = int4_to_device(pack_int4_symmetric(docs, offsets, scale_granularity="token"))
    first = device.data.maxsim_batch_int8q(query)
    for _ in range(3):
        np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), first)


def test_int8q_workspace_growth_after_larger_batch(gpu, oracle):
    docs, offsets = ragged_fixture(40, seed=11)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    device = int4_to_device(packed)
    rng = np.random.default_rng(12)
    for shape in [(1, 4), (8, 32), (2, 3)]:
        query = rng.standard_normal((*shape, 128)).astype(np.float32)
        np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), _scores(oracle, packed, query))


@pytest.fixture
def scan_partition():
    from maxsim_amd import _maxsim_hip

    yield _maxsim_hip.set_scan_partition
    _maxsim_hip.set_scan_partition(0)


@pytest.mark.parametrize("lengths", [(0, 40), (60, 200), (1, 3)])
def test_int8q_scan_partitions_agree_with_oracle(gpu, oracle, scan_partition, lengths):
    """Longest-first document assignment (default) and contiguous ranges
    (msim_set_scan_partition(1), the large-corpus path) both equal the oracle
    bit for bit, scores and top-k."""
    lo, hi = lengths
    docs, offsets = ragged_fixture(1500, seed=lo + hi, lo=lo, hi=hi, empty=7)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    query = np.random.default_rng(3).standard_normal((4, 32, 128)).astype(np.float32)
    expected = _scores(oracle, packed, query)
    ref_s, ref_i = oracle.topk(expected, 10)
    for mode in (0, 1):
        print(f"case partition={mode} lengths={lengths}", flush=True)
        scan_partition(mode)
        device = int4_to_device(packed)
        np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), expected)
        top_s, top_i = device.data.topk_batch_int8q(query, 10)
        np.testing.assert_array_equal(top_i, ref_i)
        np.testing.assert_array_equal(top_s, ref_s)


def test_int8q_scan_ring_fill_short_waves(gpu, oracle):
    """One document per wave (docs_per_wave 1) with 1 to 14 tiles each: a
    wave starts with two ring tiles and fills the ring over its first three
    steps, with special cases for one, two and three tiles; scores and the
    fused top-k bit-exact vs the oracle."""
    from maxsim_amd import _maxsim_hip

    base = [1, 15, 16, 17, 31, 32, 33, 47, 48, 49, 64, 65, 80, 96, 112, 128, 144, 160, 200, 224]
    lengths = np.array(base * 16, np.int64)  # 320 documents
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    rng = np.random.default_rng(11)
    docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    query = rng.standard_normal((4, 32, 128)).astype(np.float32)
    expected = _scores(oracle, packed, query)
    ref_s, ref_i = oracle.topk(expected, 10)
    _maxsim_hip.set_docs_per_wave(1)
    try:
        device = int4_to_device(packed)
        np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), expected)
        top_s, top_i = device.data.topk_batch_int8q(query, 10)
        np.testing.assert_array_equal(top_i, ref_i)
        np.testing.assert_array_equal(top_s, ref_s)
    finally:
        _maxsim_hip.set_docs_per_wave(0)


@pytest.mark.parametrize("long_len", [4000, 16])
def test_int8q_scan_one_long_document(gpu, oracle, scan_partition, long_len):
    """One document far longer than the rest (a wave with thousands of tiles,
    the tile table's stride set by it) among 600 short ones, including empty
    documents and documents shorter than a tile; both work splits, scores and
    the fused top-k bit-exact vs the oracle."""
    rng = np.random.default_rng(long_len)
    lengths = rng.integers(0, 40, size=600)
    lengths[17] = long_len
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    docs[offsets[17]:offsets[18]] *= 3.0  # the long document is among the best
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    query = np.random.default_rng(5).standard_normal((3, 32, 128)).astype(np.float32)
    expected = _scores(oracle, packed, query)
    ref_s, ref_i = oracle.topk(expected, 12)
    for mode in (0, 1):
        print(f"case partition={mode} long_len={long_len}", flush=True)
        scan_partition(mode)
        device = int4_to_device(packed)
        np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), expected)
        top_s, top_i = device.data.topk_batch_int8q(query, 12)
        np.testing.assert_array_equal(top_i, ref_i)
        np.testing.assert_array_equal(top_s, ref_s)


@pytest.mark.parametrize("factor", [2.0 ** -120, 2.0 ** 115])
def test_int8q_token_scales_outside_fma_range(gpu, oracle, factor):
    """The scan's one-fma epilogue needs every token scale in [2^-122, 2^109);
    a corpus with scales outside it (here every seventh token's scale times
    2^-120 or 2^115) takes float(dot) * s instead.  Scores and the fused
    top-k stay bit-exact against the oracle."""
    import dataclasses

    docs, offsets = ragged_fixture(400, seed=13, lo=0, hi=40)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    scales = packed.token_scale.copy()
    scales[::7] *= np.float32(factor)
    assert np.all(np.isfinite(scales)) and np.all(scales > 0)
    packed = dataclasses.replace(packed, token_scale=scales)
    query = np.random.default_rng(17).standard_normal((4, 32, 128)).astype(np.float32)
    device = int4_to_device(packed)
    expected = _scores(oracle, packed, query)
    np.testing.assert_array_equal(device.data.maxsim_batch_int8q(query), expected)
    top_s, top_i = device.data.topk_batch_int8q(query, 10)
    ref_s, ref_i = oracle.topk(expected, 10)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s, ref_s)
