"""GPU parity at the BASELINE workloads of configs 1, 3, 4 and 5, against the
C oracle on the same seeded corpora (config 2 is tests/test_gpu_int8q.py's
test_config2_full_size_parity).  The reference runs its correctness matrix
through the harness that times 4,096 documents
(benchmarks/run_cuda_step1.py:189-408 and :598-659); these tests do the same
at each configuration's own size.

Bars: integer paths (int8-query MaxSim, Hamming scores) bit-exact; fp32-query
scores rtol 1e-5 with atol 1e-5 x the row's largest |score| (the scores of
one row share one scale; the reference's own GPU bar, tests/test_cuda_reducers.py,
is atol 2e-3); top-k ids identical, except that a document may trade places
with one whose oracle score lies within that tolerance of it.

The oracle is scalar C; calls over a large corpus are split into document
ranges run on threads (ctypes releases the GIL)."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from maxsim_amd import synthetic

pytestmark = pytest.mark.gpu

RTOL = 1e-5
THREADS = 16


def _row_tol(expected):
    """Per-row absolute tolerance: RTOL x max(1, the row's largest |score|)."""
    return RTOL * np.maximum(1.0, np.max(np.abs(expected), axis=-1, keepdims=True))


def _close_rows(actual, expected):
    tol = _row_tol(expected)
    bad = np.abs(actual - expected) > tol + RTOL * np.abs(expected)
    assert not bad.any(), (f"{int(bad.sum())} scores outside rtol {RTOL} / row atol; worst at "
                           f"{np.unravel_index(np.argmax(np.abs(actual - expected)), actual.shape)}")


def _split_docs(fn, offsets, per_token_arrays=(), threads=THREADS, **kw):
    """fn(..., offsets=rebased slice) over `threads` document ranges, joined on the last axis."""
    n = offsets.shape[0] - 1
    bounds = np.linspace(0, n, threads + 1).astype(np.int64)

    def part(i):
        a, b = int(bounds[i]), int(bounds[i + 1])
        t0, t1 = int(offsets[a]), int(offsets[b])
        tok = [x[t0:t1] for x in per_token_arrays]
        return fn(*tok, offsets[a:b + 1] - t0, **kw)

    with ThreadPoolExecutor(threads) as pool:
        parts = list(pool.map(part, range(threads)))
    return np.concatenate(parts, axis=-1)


def _assert_topk_equivalent(ids, scores_ref, k, tie_ids=None):
    """ids [B, k] equal the stable top-k of scores_ref, except near-ties.

    Every returned id must be one the reference order would place in the
    top-k once scores within the row tolerance count as equal, and the
    returned ids must be distinct."""
    tol = _row_tol(scores_ref)
    for b in range(ids.shape[0]):
        row = scores_ref[b]
        order_ids = np.arange(row.shape[0]) if tie_ids is None else tie_ids[b]
        ref = order_ids[np.lexsort((order_ids, -row))[:k]]
        if np.array_equal(ids[b], ref):
            continue
        assert len(set(ids[b].tolist())) == k, f"row {b}: repeated ids {ids[b]}"
        pos = {int(d): i for i, d in enumerate(order_ids)}
        kth = row[pos[int(ref[-1])]]
        for d in ids[b]:
            assert row[pos[int(d)]] >= kth - tol[b, 0], f"row {b}: id {d} is not a near-tie of the top-{k}"
        differing = [int(d) for d in ref if d not in set(ids[b].tolist())]
        for d in differing:
            assert row[pos[d]] <= kth + tol[b, 0], f"row {b}: missing id {d} is above the near-tie band"


# ------------------------------------------------------------------ config 1


@pytest.mark.parametrize("route", ["fp32", "int8"])
def test_config1_both_query_routes(gpu, oracle, route):
    """512 docs x U{32..64} tokens, one [1,32,128] fp32 query, top-10: the
    fp32-query route within tolerance, the int8-query route bit-exact, and
    Reranker.search returning the same documents in the same order."""
    import maxsim_amd as maxsim
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    cfg = synthetic.CONFIGS[1]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query = synthetic.make_queries(corpus, cfg["batch"])
    print(f"config 1 route={route}: {int(corpus.offsets[-1])} tokens", flush=True)
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    handle = int4_to_device(packed).data
    if route == "int8":
        expected = oracle.int4_int8q_scores(query, packed.values, packed.doc_offsets, token_scale=packed.token_scale)
        got = handle.maxsim_batch_int8q(query)
        np.testing.assert_array_equal(got, expected)
        top_s, top_i = handle.topk_batch_int8q(query, 10)
        ref_s, ref_i = oracle.topk(expected, 10)
        np.testing.assert_array_equal(top_i, ref_i)
        np.testing.assert_array_equal(top_s, ref_s)
    else:
        expected = oracle.int4_fp32_scores(query, packed.values, packed.doc_offsets, token_scale=packed.token_scale)
        _close_rows(handle.maxsim_batch(query), expected)
        top_s, top_i = handle.topk_batch(query, 10)
        _assert_topk_equivalent(top_i, expected, 10)
    ids = [f"doc{i}" for i in range(cfg["num_docs"])]
    index = maxsim.Index.from_embeddings(ids, corpus.embeddings, corpus.offsets, mode="int4_per_token")
    res = maxsim.Reranker(index, device="cuda", int4_query=route).search(query[0], k=10)
    assert [r.doc_id for r in res] == [ids[i] for i in top_i[0]]
    assert [r.rank for r in res] == list(range(1, 11))


# ------------------------------------------------------------------ config 3


@pytest.fixture(scope="module")
def config3():
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    cfg = synthetic.CONFIGS[3]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query = synthetic.make_queries(corpus, cfg["batch"])
    weights = synthetic.query_weights(cfg["batch"], 32)
    packed = pack_int4_symmetric(corpus.embeddings, corpus.offsets, scale_granularity="token")
    return packed, int4_to_device(packed).data, query, weights


@pytest.mark.parametrize("reducer", ["maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"])
def test_config3_full_size_each_reducer(gpu, oracle, config3, reducer):
    """4,096 docs x U{64..192} tokens, fp32 query [4,32,128]: every reducer's
    full scan against the oracle, and the device top-10 against the oracle's
    stable top-10 (weights U[0.5,1.5], SmoothSim tau 0.7)."""
    packed, handle, query, weights = config3
    w = weights if reducer == "weighted_maxsim" else None
    tau = 0.7 if reducer == "smoothsim" else 1.0
    print(f"config 3 reducer={reducer}", flush=True)
    got = handle.score_batch(query, reducer, w, tau)

    def part(values, scales, offs):
        return oracle.int4_fp32_scores(query, values, offs, reducer=reducer, weights=w, temperature=tau,
                                       token_scale=scales)

    expected = _split_docs(part, packed.doc_offsets, per_token_arrays=(packed.values, packed.token_scale))
    _close_rows(got, expected)
    top_s, top_i = handle.topk_score_batch(query, 10, reducer, w, tau)
    _assert_topk_equivalent(top_i, expected, 10)


# ------------------------------------------------------------------ config 4


def test_config4_full_corpus_hamming(gpu, oracle):
    """10,240 binary docs x U{256..1024} tokens, 256 sign queries of 32
    tokens through one device call; the first 8 queries' Hamming MaxSim
    scores bit-exact against the oracle over the whole corpus, and their
    top-10 ids identical (integer scores: ties by document id)."""
    import torch

    from maxsim_amd import _maxsim_hip
    from maxsim_amd._api import pack_query_signs

    cfg = synthetic.CONFIGS[4]
    lengths = synthetic.doc_lengths(cfg["num_docs"], cfg["lo"], cfg["hi"])
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    codes = np.empty((int(offsets[-1]), 16), np.uint8)
    query = None
    for first, lens, emb in synthetic.iter_blocks(cfg["num_docs"], cfg["lo"], cfg["hi"]):
        s0 = int(offsets[first])
        codes[s0:s0 + emb.shape[0]] = oracle.pack_signs(emb)
        if query is None:
            rng = np.random.default_rng(synthetic.SEED + 4)
            loc = np.concatenate([[0], np.cumsum(lens)])
            query = np.empty((cfg["batch"], 32, 128), np.float32)
            for i in range(cfg["batch"]):
                d = int(rng.integers(0, len(lens)))
                tok = emb[loc[d]:loc[d + 1]][rng.choice(int(lens[d]), 32, replace=lens[d] < 32)]
                query[i] = tok + rng.standard_normal(tok.shape).astype(np.float32) * np.float32(0.1)
    qbits = pack_query_signs(query)
    print(f"config 4: {int(offsets[-1])} tokens, 256 queries", flush=True)
    h = _maxsim_hip.CudaPackedDocs(codes, offsets, 128)
    stream = torch.cuda.current_stream()
    ts = torch.empty((cfg["batch"], 10), dtype=torch.float32, device="cuda")
    ti = torch.empty((cfg["batch"], 10), dtype=torch.int64, device="cuda")
    h.topk_hamming_async(torch.from_numpy(qbits).cuda(), 10, ts, ti, stream)
    torch.cuda.synchronize()
    sub = qbits[:8]
    got = h.hamming_batch(sub)
    expected = _split_docs(lambda c, offs: oracle.binary_hamming_maxsim(sub, c, offs, 128), offsets,
                           per_token_arrays=(codes,))
    np.testing.assert_array_equal(got, expected)
    ref_s, ref_i = oracle.topk(expected.astype(np.float32), 10)
    np.testing.assert_array_equal(ti.cpu().numpy()[:8], ref_i)
    np.testing.assert_array_equal(ts.cpu().numpy()[:8], ref_s)


# ------------------------------------------------------------------ config 5


def test_config5_cascade_full_size(gpu, oracle):
    """4,096 docs in the binary-prefix + int4-residual format, query
    [4,32,128], 512 candidates, top-10: coarse and fused scores against the
    oracle; the cascade's candidates and result equal the host procedure
    (stable coarse top-512, fused rescoring, order by fused score then id)
    applied to the device's scores; and the top-10 equals the oracle-only
    pipeline up to near-ties."""
    from maxsim_amd.binres import binres_cascade_topk, binres_score, binres_to_device, pack_binary_residual

    cfg = synthetic.CONFIGS[5]
    corpus = synthetic.make_corpus(cfg["num_docs"], cfg["lo"], cfg["hi"])
    query = synthetic.make_queries(corpus, cfg["batch"])
    host = pack_binary_residual(corpus.embeddings, corpus.offsets)
    packed = binres_to_device(host)
    k, m = 10, 512
    print("config 5: coarse, fused, cascade", flush=True)
    top_s, top_i = binres_cascade_topk(query, packed, k, candidates=m)
    coarse = binres_score(query, packed, fused=False)
    coarse_ref = _split_docs(lambda s, a, offs: oracle.binres_prefix_scores(query, s, a, offs), host.doc_offsets,
                             per_token_arrays=(host.sign_data, host.prefix_scale))
    _close_rows(coarse, coarse_ref)
    cands = np.stack([np.lexsort((np.arange(coarse.shape[1]), -coarse[b]))[:m] for b in range(cfg["batch"])])
    fine = binres_score(query, packed, fused=True, candidate_indices=cands)
    fine_ref = oracle.binres_fused_scores(query, host.sign_data, host.prefix_scale, host.residual_values,
                                          host.residual_token_scale, host.doc_offsets, candidates=cands)
    _close_rows(fine, fine_ref)
    for b in range(cfg["batch"]):
        order = np.lexsort((cands[b], -fine[b]))[:k]
        np.testing.assert_array_equal(top_i[b], cands[b][order])
        np.testing.assert_array_equal(top_s[b], fine[b][order])
    # the oracle-only pipeline: its own coarse top-512, its fused scores, top-10
    ref_cands = np.stack([np.lexsort((np.arange(coarse_ref.shape[1]), -coarse_ref[b]))[:m]
                          for b in range(cfg["batch"])])
    ref_fine = oracle.binres_fused_scores(query, host.sign_data, host.prefix_scale, host.residual_values,
                                          host.residual_token_scale, host.doc_offsets, candidates=ref_cands)
    _assert_topk_equivalent(top_i, ref_fine, k, tie_ids=ref_cands)
