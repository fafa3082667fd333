"""Seeded random sweeps on the GPU, one test per case (pytest -x stops at the
first mismatch and names it):

* int8-query MaxSim + top-k over random ragged corpora (empty and very long
  documents, 1 to 6,000 documents), both work splits and all three top-k
  modes: bit-exact against the C oracle;
* fp32-query int4 scoring, every reducer, token or tensor scales, full corpus
  or candidate lists: within rtol 1e-5 plus atol 1e-5 x the row's largest
  |score| (the bar of the fp32 tests; element-wise relative error is
  unbounded where a score cancels toward zero);
* both cascades (int4 residual, binary prefix + int4 residual): the device
  result equals the reference's host procedure (cascade.py:294-453) applied
  to the device's own coarse and fused scores.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REDUCERS = ["maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim"]


@pytest.fixture
def knobs():
    from maxsim_amd import _maxsim_hip

    yield _maxsim_hip
    _maxsim_hip.set_scan_partition(0)
    _maxsim_hip.set_fused_topk(1)


@pytest.mark.parametrize("seed", range(36))
def test_int8q_random_case_bit_exact(gpu, oracle, knobs, seed):
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    rng = np.random.default_rng(1000 + seed)
    nd = int(rng.choice([1, 5, 255, 256, 300, 1000, 4096, 4097, 6000]))
    hi = int(rng.choice([1, 3, 16, 17, 40, 200]))
    lengths = rng.integers(0, hi + 1, size=nd)
    if rng.random() < 0.5:
        lengths[rng.integers(0, nd)] = int(rng.integers(300, 3000))
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    gran = str(rng.choice(["token", "tensor"]))
    b = int(rng.integers(1, 9))
    q = int(rng.choice([1, 4, 8, 16, 31, 32, 33, 64, 128, 130]))
    k = int(min(nd, rng.choice([1, 10, 32, 33])))
    part, fused = int(rng.integers(0, 2)), int(rng.integers(0, 3))
    print(f"int8q case {seed}: docs={nd} tokens={int(offsets[-1])} {gran} B={b} Q={q} k={k} "
          f"partition={part} fused={fused}", flush=True)
    knobs.set_scan_partition(part)
    knobs.set_fused_topk(fused)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=gran)
    query = rng.standard_normal((b, q, 128)).astype(np.float32)
    expected = oracle.int4_int8q_scores(query, packed.values, packed.doc_offsets, token_scale=packed.token_scale,
                                        scale=float(packed.scale))
    device = int4_to_device(packed).data
    np.testing.assert_array_equal(device.maxsim_batch_int8q(query), expected)
    top_s, top_i = device.topk_batch_int8q(query, k)
    ref_s, ref_i = oracle.topk(expected, k)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s, ref_s)


@pytest.mark.parametrize("seed", range(36))
def test_fp32_reducer_random_case(gpu, oracle, seed):
    from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

    rng = np.random.default_rng(2000 + seed)
    nd = int(rng.choice([1, 7, 300, 1000, 4096]))
    hi = int(rng.choice([1, 16, 17, 60, 200]))
    lengths = rng.integers(0, hi + 1, size=nd)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    docs = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    gran = str(rng.choice(["token", "tensor"]))
    red = str(rng.choice(REDUCERS))
    b = int(rng.integers(1, 6))
    q = int(rng.choice([1, 5, 32, 33, 64]))
    w = rng.uniform(0.5, 1.5, size=(b, q)).astype(np.float32) if red == "weighted_maxsim" else None
    tau = float(rng.choice([0.1, 0.7, 5.0])) if red == "smoothsim" else 1.0
    cand = None
    if rng.random() < 0.4 and nd > 1:
        cand = rng.choice(nd, size=int(rng.integers(1, nd + 1)), replace=False).astype(np.int64)
    print(f"fp32 case {seed}: docs={nd} {gran} {red} B={b} Q={q} tau={tau} "
          f"candidates={None if cand is None else len(cand)}", flush=True)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=gran)
    query = rng.standard_normal((b, q, 128)).astype(np.float32)
    expected = oracle.int4_fp32_scores(query, packed.values, packed.doc_offsets, scale=float(packed.scale),
                                       token_scale=packed.token_scale, reducer=red, weights=w, temperature=tau,
                                       candidates=cand)
    device = int4_to_device(packed).data
    got = device.score_batch(query, red, w, tau) if cand is None else \
        device.score_candidates_batch(query, cand, red, w, tau)
    row_atol = 1e-5 * np.maximum(1.0, np.max(np.abs(expected), axis=1, keepdims=True))
    bad = np.abs(got - expected) > row_atol + 1e-5 * np.abs(expected)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} scores outside the bar"


@pytest.mark.parametrize("seed", range(24))
def test_cascade_random_case_equals_host_procedure(gpu, seed):
    from maxsim_amd import synthetic
    from maxsim_amd.binres import binres_cascade_topk, binres_score, binres_to_device, pack_binary_residual
    from maxsim_amd.cascade import (cascade_topk, pack_residual_int4, prefix_score, residual_int4_to_device,
                                    residual_score)

    def stable(s, k, ids=None):
        ids = np.arange(s.shape[0]) if ids is None else ids
        return np.lexsort((ids, -s))[:k]

    rng = np.random.default_rng(3000 + seed)
    n = int(rng.choice([40, 300, 1000, 4096, 5000]))
    hi = int(rng.choice([8, 60, 150]))
    c = synthetic.make_corpus(n, 1, hi, seed=int(rng.integers(1 << 30)))
    b = int(rng.integers(1, 5))
    query = synthetic.make_queries(c, b)
    m = int(min(n, rng.choice([16, 64, 512, 1000])))
    k = int(min(m, rng.choice([1, 10, 32])))
    kind = str(rng.choice(["int4", "binres"]))
    print(f"cascade case {seed}: {kind} docs={n} hi={hi} B={b} M={m} k={k}", flush=True)
    if kind == "int4":
        red = str(rng.choice(["maxsim", "topk2", "smoothsim"]))
        p = residual_int4_to_device(pack_residual_int4(c.embeddings, c.offsets))
        ts, ti = cascade_topk(query, p, k, candidates=m, reducer=red, temperature=0.7)
        coarse = prefix_score(query, p, reducer=red, temperature=0.7)
        for r in range(b):
            cands = stable(coarse[r], m)
            fine = residual_score(query[r], p, reducer=red, temperature=0.7, candidate_indices=cands)
            order = stable(fine, k, np.asarray(cands))
            np.testing.assert_array_equal(ti[r], cands[order])
            np.testing.assert_array_equal(ts[r], fine[order])
    else:
        p = binres_to_device(pack_binary_residual(c.embeddings, c.offsets))
        ts, ti = binres_cascade_topk(query, p, k, candidates=m)
        coarse = binres_score(query, p, fused=False)
        cands = np.stack([stable(coarse[r], m) for r in range(b)])
        fine = binres_score(query, p, fused=True, candidate_indices=cands)
        for r in range(b):
            order = stable(fine[r], k, cands[r])
            np.testing.assert_array_equal(ti[r], cands[r][order])
            np.testing.assert_array_equal(ts[r], fine[r][order])
