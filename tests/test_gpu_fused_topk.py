"""GPU parity: the int8-query search's top-k selected in the scan's last
workgroup, against the C oracle's stable top-k (score descending, document id
ascending; reference order cu:1629-1692, _api.py:732-735).

Every case runs in the three modes of msim_set_fused_topk: 1 = fused, register
path; 2 = fused with the k-round path forced; 0 = separate selection launch.
Scores and ids must equal the oracle's bit for bit in each.
"""
import numpy as np
import pytest

from conftest import ragged_fixture
from maxsim_amd import _maxsim_hip
from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

pytestmark = pytest.mark.gpu

MODES = [1, 2, 0]


@pytest.fixture
def fused_mode():
    yield _maxsim_hip.set_fused_topk
    _maxsim_hip.set_fused_topk(1)


def _oracle_topk(oracle, packed, query, k):
    scores = oracle.int4_int8q_scores(query, packed.values, packed.doc_offsets,
                                      token_scale=packed.token_scale, scale=float(packed.scale))
    return oracle.topk(scores, k)


def _check(device, oracle, packed, query, k):
    top_s, top_i = device.data.topk_batch_int8q(query, k)
    ref_s, ref_i = _oracle_topk(oracle, packed, query, k)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s.view(np.uint32), ref_s.view(np.uint32))


# (documents, token lengths lo..hi, batch, query tokens, k, scale granularity)
CASES = [
    (4096, 0, 24, 4, 32, 10, "token"),   # the config-2 shape (shorter documents): rows of 4096 scores
    (1000, 0, 30, 3, 8, 32, "token"),    # padding past the last document, k at its limit
    (5, 1, 20, 2, 4, 5, "tensor"),       # k == n, fewer documents than the tail takes: separate launch
    (257, 0, 10, 2, 8, 32, "tensor"),    # the fewest documents the tail takes, k at its limit
    (300, 0, 20, 8, 16, 1, "token"),     # 8 batch rows in one pass: two rows per wave
    (700, 0, 20, 5, 64, 17, "token"),    # passes of 2, 2 and 1 batch rows
    (64, 0, 20, 130, 1, 7, "token"),     # 128 rows per pass: the separate launch in every mode
    (5000, 0, 6, 2, 32, 10, "token"),    # more documents than the tail takes: separate launch
]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("case", CASES, ids=[f"n{c[0]}_b{c[3]}_q{c[4]}_k{c[5]}" for c in CASES])
def test_fused_topk_matches_oracle(gpu, oracle, fused_mode, mode, case):
    n, lo, hi, b, q, k, gran = case
    print(f"case mode={mode} n={n} B={b} Q={q} k={k} {gran}", flush=True)
    fused_mode(mode)
    docs, offsets = ragged_fixture(n, seed=n + q, lo=lo, hi=hi)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=gran)
    query = np.random.default_rng(k + b).standard_normal((b, q, 128)).astype(np.float32)
    _check(int4_to_device(packed), oracle, packed, query, k)


@pytest.mark.parametrize("mode", MODES)
def test_fused_topk_ties_take_lower_ids(gpu, oracle, fused_mode, mode):
    """Every document appears three times (equal scores), empty documents
    score 0: ties must resolve to the lowest ids."""
    print(f"case ties mode={mode}", flush=True)
    fused_mode(mode)
    docs, offsets = ragged_fixture(400, seed=3, lo=0, hi=12, empty=5)
    lens = np.diff(offsets)
    order = np.repeat(np.arange(400), 3)
    rep_lens = lens[order]
    rep_offsets = np.concatenate([[0], np.cumsum(rep_lens)]).astype(np.int64)
    rep_docs = np.concatenate([docs[offsets[d]:offsets[d + 1]] for d in order])
    packed = pack_int4_symmetric(rep_docs, rep_offsets, scale_granularity="token")
    query = np.random.default_rng(4).standard_normal((3, 16, 128)).astype(np.float32)
    _check(int4_to_device(packed), oracle, packed, query, 32)


@pytest.mark.parametrize("mode", MODES)
def test_fused_topk_all_scores_equal(gpu, oracle, fused_mode, mode):
    """One document repeated 4096 times: every score ties, ids 0..k-1 win."""
    print(f"case all-equal mode={mode}", flush=True)
    fused_mode(mode)
    tok = np.random.default_rng(8).standard_normal((3, 128)).astype(np.float32)
    docs = np.tile(tok, (4096, 1))
    offsets = np.arange(0, 3 * 4096 + 1, 3, dtype=np.int64)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity="token")
    query = np.random.default_rng(9).standard_normal((4, 32, 128)).astype(np.float32)
    top_s, top_i = int4_to_device(packed).data.topk_batch_int8q(query, 20)
    assert top_i.tolist() == [list(range(20))] * 4
    ref_s, ref_i = _oracle_topk(oracle, packed, query, 20)
    np.testing.assert_array_equal(top_i, ref_i)
    np.testing.assert_array_equal(top_s, ref_s)


def test_fused_topk_repeated_calls_and_two_handles(gpu, oracle):
    """The ticket returns to zero after every launch: repeated calls on two
    handles, interleaved, keep selecting correctly."""
    packs, devices = [], []
    for seed in (21, 22):
        docs, offsets = ragged_fixture(2048, seed=seed, lo=0, hi=20)
        packs.append(pack_int4_symmetric(docs, offsets, scale_granularity="token"))
        devices.append(int4_to_device(packs[-1]))
    rng = np.random.default_rng(23)
    for it in range(6):
        h = it % 2
        query = rng.standard_normal((1 + it % 4, 32, 128)).astype(np.float32)
        print(f"case repeat it={it} handle={h} B={query.shape[0]}", flush=True)
        _check(devices[h], oracle, packs[h], query, 10)

