"""GPU tests of the fused selection's give-up path and of searches with k
beyond the device selector's limit.

The give-up path is forced from the host: msim_set_fused_wait_ticks(0) makes
every fused selection give up before it reads anything, so each kernel still
ends through its own code path (no wait is cut short on the device).  The
synchronous calls and the SDK must then raise instead of returning id -1,
the device-resident form must leave the documented sentinel (id -1, NaN),
and the handle's give-up counter must count it.  With the default budget
restored, the next search must be exact again: with the batch rows in
another order, so that entries left by the launch that gave up (other
scores in every row) cannot pass for the next launch's.
"""
import numpy as np
import pytest

import maxsim_amd as maxsim
from maxsim_amd import _maxsim_hip, synthetic
from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

pytestmark = pytest.mark.gpu

DEFAULT_TICKS = 10_000_000


@pytest.fixture
def wait_ticks():
    assert _maxsim_hip.get_fused_wait_ticks() == DEFAULT_TICKS
    yield _maxsim_hip.set_fused_wait_ticks
    _maxsim_hip.set_fused_wait_ticks(DEFAULT_TICKS)


def _corpus():
    corpus = synthetic.make_corpus(1024, 16, 48, seed=31)
    query = synthetic.make_queries(corpus, 4, seed=32)
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    return corpus, query, packed


def test_wait_ticks_knob_validates(gpu):
    with pytest.raises(ValueError, match=">= 0"):
        _maxsim_hip.set_fused_wait_ticks(-1)
    assert _maxsim_hip.get_fused_wait_ticks() == DEFAULT_TICKS


def test_given_up_selection_raises_and_counts(gpu, oracle, wait_ticks):
    print("case: fused selection forced to give up (1024 docs, [4,32,128], k=10)", flush=True)
    _, query, packed = _corpus()
    resident = int4_to_device(packed)
    handle = resident.data
    assert handle.fused_giveups() == 0
    wait_ticks(0)
    with pytest.raises(RuntimeError, match="gave up"):
        handle.topk_batch_int8q(query, 10)
    assert handle.fused_giveups() == 4  # one per batch row

    import torch

    dq = torch.from_numpy(query).cuda()
    s = torch.zeros((4, 10), dtype=torch.float32, device="cuda")
    i = torch.zeros((4, 10), dtype=torch.int64, device="cuda")
    handle.topk_int8q_async(dq, 10, s, i)
    torch.cuda.synchronize()
    assert bool((i == -1).all()) and bool(torch.isnan(s).all())
    assert handle.fused_giveups() == 8

    # Default budget again: exact results, no further give-ups.
    wait_ticks(DEFAULT_TICKS)
    rquery = np.ascontiguousarray(query[::-1])
    got_s, got_i = handle.topk_batch_int8q(rquery, 10)
    exp = oracle.int4_int8q_scores(rquery, packed.values, packed.doc_offsets, token_scale=packed.token_scale)
    ref_s, ref_i = oracle.topk(exp, 10)
    np.testing.assert_array_equal(got_i, ref_i)
    np.testing.assert_array_equal(got_s.view(np.uint32), ref_s.view(np.uint32))
    # The device-resident form after its own give-up, rows reversed again.
    wait_ticks(0)
    handle.topk_int8q_async(dq, 10, s, i)
    wait_ticks(DEFAULT_TICKS)
    handle.topk_int8q_async(torch.from_numpy(rquery).cuda(), 10, s, i)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(i.cpu().numpy(), ref_i)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    assert handle.fused_giveups() == 12


def test_sdk_search_raises_when_the_selection_gave_up(gpu, wait_ticks):
    corpus, query, _ = _corpus()
    ids = [f"doc{j}" for j in range(corpus.offsets.shape[0] - 1)]
    index = maxsim.Index.from_embeddings(ids, corpus.embeddings, corpus.offsets, mode="int4_per_token")
    reranker = maxsim.Reranker(index, device="cuda", int4_query="int8")
    wait_ticks(0)
    with pytest.raises(RuntimeError, match="gave up"):
        reranker.search(query, k=10)
    wait_ticks(DEFAULT_TICKS)
    assert len(reranker.search(query, k=10)) == 4


def _many_docs(n, seed):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, 4, size=n)
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    return docs, offsets, rng.standard_normal((2, 5, 128)).astype(np.float32)


def test_residual_search_with_k_above_the_device_limit(gpu, oracle):
    """k > 4096 on an int4_residual index: the reference's route, the stable
    top-k of the full fused scores (sdk.py:523-533), for any k."""
    from maxsim_amd.cascade import residual_score

    docs, offsets, query = _many_docs(5000, 41)
    ids = [f"d{j}" for j in range(5000)]
    index = maxsim.Index.from_embeddings(ids, docs, offsets, mode="int4_residual")
    res = maxsim.Reranker(index, device="cuda").search(query, k=4500)
    scores = residual_score(query, maxsim.Reranker(index, device="cuda").corpus.int4_packed)
    es, ei = oracle.topk(scores, 4500)
    assert [[x.doc_id for x in row] for row in res] == [[ids[j] for j in row] for row in ei]
    assert [[x.score for x in row] for row in res] == es.astype(np.float64).tolist()


def test_binary_residual_search_with_k_above_the_device_limit(gpu, oracle):
    from maxsim_amd.binres import binres_score

    docs, offsets, query = _many_docs(5000, 43)
    ids = [f"d{j}" for j in range(5000)]
    index = maxsim.Index.from_embeddings(ids, docs, offsets, mode="binary_residual")
    reranker = maxsim.Reranker(index, device="cuda")
    res = reranker.search(query, k=4200)
    es, ei = oracle.topk(binres_score(query, reranker.corpus.int4_packed), 4200)
    assert [[x.doc_id for x in row] for row in res] == [[ids[j] for j in row] for row in ei]
    assert [[x.score for x in row] for row in res] == es.astype(np.float64).tolist()
