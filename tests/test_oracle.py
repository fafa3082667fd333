"""Pins of the C oracle (oracle/maxsim_oracle.c) before it is trusted as the checker.

Each test checks one oracle function against a known answer from the
reference's own tests, against the reference's compiled CPU extension
(oracle/_ref, built from cpp/maxsim/cpu_extension.cpp), or against an
independent NumPy statement of the closed form the reference's tests use.
No GPU is needed.
"""
import numpy as np
import pytest

from conftest import ragged_fixture

REDUCERS = ("maxsim", "weighted_maxsim", "topk2", "topk4", "smoothsim")


# ------------------------------------------------------------------ helpers


def _np_int8q_scores(values, offsets, query, token_scale=None, scale=1.0):
    """Closed form of tests/test_int4_int8q.py:7-26 in NumPy (float64 sum of
    the per-row maxima times the row scales, numpy's own pairwise order)."""
    values = values.astype(np.float32)
    n = offsets.shape[0] - 1
    out = np.empty((query.shape[0], n), np.float32)
    for b, qm in enumerate(query):
        max_abs = np.max(np.abs(qm), axis=1)
        qs = np.where(max_abs == 0.0, 1.0, max_abs / 127.0).astype(np.float32)
        qi = np.clip(np.rint(qm / qs[:, None]), -127, 127).astype(np.float32)
        for d in range(n):
            s, e = int(offsets[d]), int(offsets[d + 1])
            if s == e:
                out[b, d] = 0.0
                continue
            dots = qi @ values[s:e].T
            if token_scale is not None:
                dots = dots * token_scale[s:e][None, :]
            best = dots.max(axis=1).astype(np.float64)
            out[b, d] = np.float32(float((best * qs).sum()) * scale)
    return out


def _np_reduce(query, docs, offsets, reducer, *, weights=None, temperature=1.0, candidates=None):
    """Closed form of the reducers (tests/test_reducers.py:20-44, _api.py:558-585)."""
    selected = np.arange(offsets.shape[0] - 1) if candidates is None else np.asarray(candidates)
    out = np.empty((query.shape[0], selected.shape[0]), np.float32)
    for b, qm in enumerate(query):
        for j, d in enumerate(selected):
            doc = docs[offsets[d]:offsets[d + 1]]
            if doc.shape[0] == 0:
                out[b, j] = 0.0
                continue
            sims = qm @ doc.T
            if reducer in ("maxsim", "weighted_maxsim"):
                pooled = sims.max(axis=1)
                if reducer == "weighted_maxsim":
                    pooled = pooled * weights[b]
            elif reducer in ("topk2", "topk4"):
                c = min(2 if reducer == "topk2" else 4, doc.shape[0])
                pooled = np.sort(sims, axis=1)[:, -c:].mean(axis=1)
            else:
                m = sims.max(axis=1)
                pooled = m + temperature * np.log(np.exp((sims - m[:, None]) / temperature).sum(axis=1))
            out[b, j] = pooled.sum(dtype=np.float32)
    return out


# ---------------------------------------------------------------- a1 packing


def test_pack_int4_token_kat_scales_and_codes(oracle):
    """Per-token scales [1, 2, 0.1] (tests/test_int4_reference.py:28-49)."""
    docs = np.array(
        [
            [0.0] * 8,
            [-14.0, -7.0, 0.0, 2.0, 4.0, 6.0, 10.0, 14.0],
            [-0.7, -0.5, -0.3, -0.1, 0.1, 0.3, 0.5, 0.7],
        ],
        np.float32,
    )
    codes, values, scales = oracle.pack_int4_token(docs)
    expected_scales = np.array([1.0, 2.0, 0.1], np.float32)
    np.testing.assert_allclose(scales, expected_scales, rtol=1e-6, atol=0)
    np.testing.assert_array_equal(values, np.clip(np.rint(docs / expected_scales[:, None]), -7, 7).astype(np.int8))
    assert codes.shape == (3, 4)


def test_pack_int4_nibble_order_closed_form(oracle):
    """byte i = (v[2i] & 0xF) | (v[2i+1] & 0xF) << 4 (experimental.py:604-609), and
    unpack inverts it for every code pair in [-7, 7]^2 (sdk.py:1085-1093)."""
    pairs = np.array([(a, b) for a in range(-7, 8) for b in range(-7, 8)], np.int8)
    values = pairs.reshape(-1, 2)
    values = np.concatenate([values, np.zeros((values.shape[0], 6), np.int8)], axis=1)  # dim 8
    # Pack through the tensor path with scale 1: x = values exactly, max|x| = 7 -> scale 1.
    codes, got_values, scale = oracle.pack_int4_tensor(values.astype(np.float32))
    assert scale == 1.0
    np.testing.assert_array_equal(got_values, values)
    lo = codes[:, 0] & 0xF
    hi = codes[:, 0] >> 4
    np.testing.assert_array_equal(lo, (values[:, 0].astype(np.int16) & 0xF).astype(np.uint8))
    np.testing.assert_array_equal(hi, (values[:, 1].astype(np.int16) & 0xF).astype(np.uint8))
    np.testing.assert_array_equal(oracle.unpack_int4(codes, 8), values)
    assert np.all(codes[:, 1:] == 0)


def test_pack_int4_tensor_scale_and_range(oracle):
    """Tensor scale = max|x| / 7; codes within [-7, 7]; all-zero input -> scale 1
    (tests/test_int4_reference.py:5-26, experimental.py:246-258)."""
    docs = np.array(
        [
            [-2.0, -1.1, -0.2, 0.0, 0.4, 1.0, 1.6, 2.2],
            [2.1, 1.4, 0.9, 0.1, -0.6, -1.2, -1.8, -2.4],
        ],
        np.float32,
    )
    codes, values, scale = oracle.pack_int4_tensor(docs)
    assert scale == pytest.approx(2.4 / 7.0, rel=1e-6)
    assert codes.shape == (2, 4) and values.min() >= -7 and values.max() <= 7
    np.testing.assert_array_equal(values, np.clip(np.rint(docs / np.float32(scale)), -7, 7).astype(np.int8))
    _, _, zero_scale = oracle.pack_int4_tensor(np.zeros((2, 8), np.float32))
    assert zero_scale == 1.0


def test_pack_signs_bit_order_kat(oracle):
    """LSB-first, x >= 0 -> 1 (tests/test_api_reference.py:43-52)."""
    docs = np.array([[-1, 0, 2, -3, 4, -5, 6, -7]], np.float32)
    assert oracle.pack_signs(docs).tolist() == [[0b01010110]]


# ------------------------------------------------------- a3 + a4 int8 query


def test_quantize_int8_closed_form(oracle):
    """sigma = max|q| / 127 (0 -> 1); q8 = clip(rint(q / sigma), +-127)
    (tests/test_int4_int8q.py:11-14)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((3, 7, 128)).astype(np.float32)
    q[1, 2] = 0.0
    q8, qs = oracle.quantize_int8(q)
    max_abs = np.max(np.abs(q), axis=2)
    exp_s = np.where(max_abs == 0.0, 1.0, max_abs / 127.0).astype(np.float32)
    np.testing.assert_array_equal(qs, exp_s)
    np.testing.assert_array_equal(q8, np.clip(np.rint(q / exp_s[..., None]), -127, 127).astype(np.int8))
    assert qs[1, 2] == 1.0 and np.all(q8[1, 2] == 0)


def test_int8_dots_brute_force(oracle):
    """Integer dots are exact: oracle == int64 NumPy product."""
    rng = np.random.default_rng(6)
    q8 = rng.integers(-127, 128, size=(5, 128)).astype(np.int8)
    v = rng.integers(-7, 8, size=(33, 128)).astype(np.int8)
    np.testing.assert_array_equal(oracle.int8_dots(q8, v), q8.astype(np.int64) @ v.astype(np.int64).T)


@pytest.mark.parametrize("seeds", [(71, 73), (89, 97)])
@pytest.mark.parametrize("granularity", ["token", "tensor"])
def test_int8q_scores_match_reference_closed_form(oracle, seeds, granularity):
    """Seeded ragged fixtures of tests/test_int4_int8q.py:29-35 and 56-69; the
    oracle reproduces the closed form bit for bit (same float64 pairwise sum)."""
    docs, offsets = ragged_fixture(150, seeds[0])
    query = np.random.default_rng(seeds[1]).standard_normal((2, 5, 128)).astype(np.float32)
    if granularity == "token":
        _, values, ts = oracle.pack_int4_token(docs)
        scale = 1.0
    else:
        _, values, scale = oracle.pack_int4_tensor(docs)
        ts = None
    got = oracle.int4_int8q_scores(query, values, offsets, token_scale=ts, scale=scale)
    np.testing.assert_array_equal(got, _np_int8q_scores(values, offsets, query, ts, scale))


def test_int8q_zero_row_and_empty_doc(oracle):
    """Padded zero query row and empty document -> 0.0 (tests/test_int4_int8q.py:73-87)."""
    docs, offsets = ragged_fixture(10, 79)
    query = np.random.default_rng(83).standard_normal((1, 4, 128)).astype(np.float32)
    query[0, -1] = 0.0
    _, values, ts = oracle.pack_int4_token(docs)
    got = oracle.int4_int8q_scores(query, values, offsets, token_scale=ts)
    empty = int(np.flatnonzero(np.diff(offsets) == 0)[0])
    assert got[0, empty] == 0.0
    np.testing.assert_array_equal(got, _np_int8q_scores(values, offsets, query, ts))


def test_int8q_scale_before_max_kat_640(oracle):
    """Token scale applied before the max: exactly 640.0 (tests/test_int4_int8q.py:109-134)."""
    docs = np.stack([np.ones(128, np.float32),
                     np.concatenate([np.full(64, 10.0, np.float32), np.zeros(64, np.float32)])])
    _, values, ts = oracle.pack_int4_token(docs)
    got = oracle.int4_int8q_scores(np.ones((1, 1, 128), np.float32), values, np.array([0, 2]), token_scale=ts)
    assert got.tolist() == [[640.0]]


def test_pairwise_sums_match_numpy(oracle):
    """numpy add.reduce order for contiguous vectors, all lengths up to 300."""
    rng = np.random.default_rng(7)
    for n in range(0, 300):
        a = rng.standard_normal(n) * 10 ** rng.uniform(-3, 3, size=n)
        assert oracle.pairwise_sum_f64(a) == float(np.add.reduce(a))
        f = a.astype(np.float32)
        assert oracle.pairwise_sum_f32(f) == np.add.reduce(f)


# ------------------------------------------------------------------ a6 top-k


def test_topk_ties_prefer_lower_id(oracle):
    """(score desc, id asc) (tests/test_int4_reference.py:129-146; _api.py:732-735)."""
    scores = np.array([[1.0, 3.0, 3.0, 2.0, 3.0, -np.inf]], np.float32)
    s, i = oracle.topk(scores, 4)
    assert i.tolist() == [[1, 2, 4, 3]] and s.tolist() == [[3.0, 3.0, 3.0, 2.0]]


def test_topk_equals_stable_lexsort(oracle):
    rng = np.random.default_rng(8)
    scores = rng.integers(0, 20, size=(3, 500)).astype(np.float32)  # many ties
    s, i = oracle.topk(scores, 37)
    for row, si, ii in zip(scores, s, i):
        order = np.lexsort((np.arange(row.shape[0]), -row))[:37]
        np.testing.assert_array_equal(ii, order)
        np.testing.assert_array_equal(si, row[order])


# -------------------------------------------------- a8 / a9 fp32 + reducers


def _cuda_reducer_fixture(dim=128):
    """tests/test_cuda_reducers.py:18-29: lengths [0,1,2,3,4,7], duplicate candidates."""
    rng = np.random.default_rng(20260713)
    lengths = np.array([0, 1, 2, 3, 4, 7], np.int64)
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int64)
    docs = rng.normal(size=(int(offsets[-1]), dim)).astype(np.float32)
    query = rng.normal(size=(2, 5, dim)).astype(np.float32)
    weights = np.array([[1.0, 0.25, 1.5, 0.0, 0.75], [0.5, 2.0, 0.125, 1.0, 0.25]], np.float32)
    candidates = np.array([5, 1, 5, 0, 2], np.int64)
    return docs, offsets, query, weights, candidates


@pytest.mark.parametrize("reducer", REDUCERS)
@pytest.mark.parametrize("with_candidates", [False, True])
def test_dense_reducers_match_closed_form(oracle, reducer, with_candidates):
    docs, offsets, query, weights, cand = _cuda_reducer_fixture()
    cand = cand if with_candidates else None
    w = weights if reducer == "weighted_maxsim" else None
    got = oracle.dense_scores(query, docs, offsets, reducer=reducer, weights=w, temperature=0.7, candidates=cand)
    exp = _np_reduce(query, docs, offsets, reducer, weights=w, temperature=0.7, candidates=cand)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("reducer", REDUCERS)
@pytest.mark.parametrize("granularity", ["token", "tensor"])
def test_int4_fp32_reducers_match_closed_form(oracle, reducer, granularity):
    """CPU semantics of experimental.py:403-420: q @ (v * scale * s_t).T, then the reducer
    (tests/test_reducers.py:73-98)."""
    docs, offsets, query, weights, cand = _cuda_reducer_fixture()
    if granularity == "token":
        _, values, ts = oracle.pack_int4_token(docs)
        scale = 1.0
    else:
        _, values, scale = oracle.pack_int4_tensor(docs)
        ts = None
    deq = values.astype(np.float32) * np.float32(scale)
    if ts is not None:
        deq = deq * ts[:, None]
    w = weights if reducer == "weighted_maxsim" else None
    got = oracle.int4_fp32_scores(query, values, offsets, scale=scale, token_scale=ts, reducer=reducer,
                                  weights=w, temperature=0.35, candidates=cand)
    exp = _np_reduce(query, deq, offsets, reducer, weights=w, temperature=0.35, candidates=cand)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5)


def test_int4_fp32_scale_before_max_kat_10(oracle):
    """tests/test_int4_reference.py:105-126: the token scale decides the max -> 10.0."""
    docs = np.array([[1.0] * 8, [10.0] + [0.0] * 7], np.float32)
    _, values, ts = oracle.pack_int4_token(docs)
    got = oracle.int4_fp32_scores(np.ones((1, 1, 8), np.float32), values, np.array([0, 2]), token_scale=ts)
    np.testing.assert_allclose(got, [[10.0]], rtol=1e-6)


def test_candidates_are_exact_gather_of_full(oracle):
    """tests/test_cuda_reducers.py:131: candidate scores == full scores gathered (atol 0)."""
    docs, offsets, query, weights, cand = _cuda_reducer_fixture()
    _, values, ts = oracle.pack_int4_token(docs)
    for reducer in REDUCERS:
        w = weights if reducer == "weighted_maxsim" else None
        full = oracle.int4_fp32_scores(query, values, offsets, token_scale=ts, reducer=reducer, weights=w)
        part = oracle.int4_fp32_scores(query, values, offsets, token_scale=ts, reducer=reducer, weights=w,
                                       candidates=cand)
        np.testing.assert_array_equal(part, full[:, cand])


def test_smoothsim_overflow_safe(oracle):
    """Large similarities with a small temperature stay finite (tests/test_cuda_reducers.py:382-427,
    tests/test_reducers.py:138-140)."""
    docs, offsets, query, _, _ = _cuda_reducer_fixture()
    got = oracle.dense_scores(query * np.float32(1e5), docs, offsets, reducer="smoothsim", temperature=0.125)
    assert np.all(np.isfinite(got))
    got = oracle.dense_scores(query * np.float32(1e6), docs, offsets, reducer="smoothsim", temperature=0.01)
    assert np.all(np.isfinite(got))


def test_smoothsim_reduces_to_maxsim_plus_log_count_for_constant_rows(oracle):
    """Math pin: a document whose tokens are identical gives max + tau * log(len) per query row."""
    d = np.random.default_rng(9).standard_normal((1, 16)).astype(np.float32)
    docs = np.repeat(d, 5, axis=0)
    q = np.random.default_rng(10).standard_normal((1, 3, 16)).astype(np.float32)
    got = oracle.dense_scores(q, docs, np.array([0, 5]), reducer="smoothsim", temperature=0.5)
    exp = float((q[0] @ d[0]).sum()) + 3 * 0.5 * np.log(5.0)
    np.testing.assert_allclose(got, [[exp]], rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- a10 binary


def test_binary_lut_matches_reference_extension(oracle):
    """oracle/_ref is the reference's own cpu_extension.cpp compiled here; the
    restatement must agree on its fixture (tests/test_cpu_extension.py:8-31) and on random docs."""
    ref = oracle.reference_cpu_extension()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference source absent)")
    docs = np.array(
        [
            [1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -16],
            [-1, 2, -3, 4, -5, 6, -7, 8, -9, 10, -11, 12, -13, 14, -15, 16],
            [1, 2, 3, 4, -5, -6, -7, -8, 9, 10, 11, 12, -13, -14, -15, -16],
            [-1, -2, -3, -4, 5, 6, 7, 8, -9, -10, -11, -12, 13, 14, 15, 16],
        ],
        np.float32,
    )
    offsets = np.array([0, 2, 4], np.int64)
    query = np.array(
        [
            [3, -1, 2, -4, 5, -6, 7, -8, 1, -3, 5, -7, 2, -4, 6, -8],
            [-2, 4, -6, 8, -1, 3, -5, 7, -8, 6, -4, 2, 7, -5, 3, -1],
        ],
        np.float32,
    )
    codes = oracle.pack_signs(docs)
    np.testing.assert_array_equal(oracle.binary_lut_maxsim(query, codes, offsets, 16),
                                  ref.maxsim_lut(query, codes, offsets, 16, 1.0))
    rng = np.random.default_rng(11)
    d2, o2 = ragged_fixture(40, 12)
    q2 = rng.standard_normal((9, 128)).astype(np.float32)
    c2 = oracle.pack_signs(d2)
    np.testing.assert_array_equal(oracle.binary_lut_maxsim(q2, c2, o2, 128, 0.5),
                                  ref.maxsim_lut(q2, c2, o2, 128, 0.5))


def test_binary_lut_matches_sign_closed_form(oracle):
    """maxsim_lut == sum_q max_t q . sign(d_t) (cpu_extension.cpp:59-126)."""
    docs, offsets = ragged_fixture(30, 13)
    q = np.random.default_rng(14).standard_normal((6, 128)).astype(np.float32)
    codes = oracle.pack_signs(docs)
    signs = np.where(docs >= 0, 1.0, -1.0).astype(np.float32)
    exp = _np_reduce(q[None], signs, offsets, "maxsim")[0]
    np.testing.assert_allclose(oracle.binary_lut_maxsim(q, codes, offsets, 128), exp, rtol=1e-5, atol=1e-4)


def test_hamming_equals_lut_for_sign_queries(oracle):
    """dim - 2 popcount(q ^ d) is exactly the LUT sum for a +-1 query."""
    docs, offsets = ragged_fixture(30, 15)
    q = np.random.default_rng(16).standard_normal((2, 7, 128)).astype(np.float32)
    qsign = np.where(q >= 0, 1.0, -1.0).astype(np.float32)
    qbits = oracle.pack_signs(q.reshape(-1, 128)).reshape(2, 7, 16)
    codes = oracle.pack_signs(docs)
    ham = oracle.binary_hamming_maxsim(qbits, codes, offsets, 128)
    for b in range(2):
        np.testing.assert_array_equal(ham[b].astype(np.float32), oracle.binary_lut_maxsim(qsign[b], codes, offsets, 128))


# ---------------------------------------------------- a11 residual / a12 binres


def test_fused_residual_is_not_sum_of_separate_reductions(oracle):
    """tests/test_cascade.py:242-275: the fused similarity is reduced once."""
    docs = np.array(
        [
            [0, 20, 13, 12, 8, 5, -7, 20],
            [-1, -12, 14, -14, 15, 5, -16, -19],
            [-2, -19, -15, 1, 19, -1, 13, 17],
        ],
        np.float32,
    )
    offsets = np.array([0, 3], np.int64)
    query = np.array([[[2, 1, 0, 0, -2, 0, -1, -2]]], np.float32)
    _, pv, ps = oracle.pack_int4_token(docs)
    prefix = pv.astype(np.float32) * ps[:, None]
    _, rv, rs = oracle.pack_int4_token(docs - prefix)
    residual = rv.astype(np.float32) * rs[:, None]
    fused = oracle.dense_scores(query, prefix + residual, offsets)
    separate = oracle.dense_scores(query, prefix, offsets) + oracle.dense_scores(query, residual, offsets)
    np.testing.assert_allclose(fused, _np_reduce(query, prefix + residual, offsets, "maxsim"), rtol=1e-5, atol=1e-5)
    assert not np.allclose(fused, separate, rtol=0, atol=1e-6)


def test_binary_residual_pack_closed_form(oracle):
    """Binary prefix + int4 residual: a_t = mean|x_t|, prefix = a_t * sign(x),
    residual = per-token int4 of x - prefix (the format's definition)."""
    x = np.random.default_rng(17).standard_normal((20, 128)).astype(np.float32)
    x[3] = 0.0
    signs, a, _, rvalues, rscale = oracle.pack_binary_residual(x)
    np.testing.assert_array_equal(signs, oracle.pack_signs(x))
    np.testing.assert_allclose(a, np.mean(np.abs(x), axis=1), rtol=1e-6)
    pre = a[:, None] * np.where(x >= 0, 1.0, -1.0).astype(np.float32)
    _, v_exp, s_exp = oracle.pack_int4_token((x - pre).astype(np.float32))
    np.testing.assert_array_equal(rvalues, v_exp)
    np.testing.assert_array_equal(rscale, s_exp)
    # Reconstruction error is within half a residual step per coordinate.
    rec = pre + rvalues.astype(np.float32) * rscale[:, None]
    assert np.all(np.abs(rec - x) <= 0.5 * rscale[:, None] + 1e-6)


def _np_binres(query, signs_pm, a, rvalues, rscale, offsets, fused, candidates=None):
    """Closed form of the binary-prefix (+ int4 residual) int8-query score:
    sim_t = f32(a_t * (q8 . sign_t)) [+ f32(s_t * (q8 . r_t))], then the int8q reduction."""
    n = offsets.shape[0] - 1
    out = []
    for b, qm in enumerate(query):
        max_abs = np.max(np.abs(qm), axis=1)
        qs = np.where(max_abs == 0.0, 1.0, max_abs / 127.0).astype(np.float32)
        qi = np.clip(np.rint(qm / qs[:, None]), -127, 127).astype(np.int64)
        docs = range(n) if candidates is None else candidates[b]
        row = []
        for d in docs:
            s, e = int(offsets[d]), int(offsets[d + 1])
            if s == e:
                row.append(np.float32(0.0))
                continue
            sim = a[s:e][None, :] * (qi @ signs_pm[s:e].T).astype(np.float32)
            if fused:
                sim = sim + rscale[s:e][None, :] * (qi @ rvalues[s:e].astype(np.int64).T).astype(np.float32)
            best = sim.max(axis=1).astype(np.float64)
            row.append(np.float32(float((best * qs).sum())))
        out.append(row)
    return np.array(out, np.float32)


def test_binres_prefix_and_fused_closed_form(oracle):
    docs, offsets = ragged_fixture(60, 18)
    query = np.random.default_rng(19).standard_normal((3, 6, 128)).astype(np.float32)
    signs, a, _, rvalues, rscale = oracle.pack_binary_residual(docs)
    pm = np.where(docs >= 0, 1, -1).astype(np.int64)
    np.testing.assert_array_equal(oracle.binres_prefix_scores(query, signs, a, offsets),
                                  _np_binres(query, pm, a, rvalues, rscale, offsets, False))
    np.testing.assert_array_equal(oracle.binres_fused_scores(query, signs, a, rvalues, rscale, offsets),
                                  _np_binres(query, pm, a, rvalues, rscale, offsets, True))
    cand = np.array([[5, 2, 2, 59], [0, 1, 2, 3], [58, 57, 2, 0]], np.int64)
    np.testing.assert_array_equal(
        oracle.binres_fused_scores(query, signs, a, rvalues, rscale, offsets, candidates=cand),
        _np_binres(query, pm, a, rvalues, rscale, offsets, True, cand))
