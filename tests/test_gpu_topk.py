"""Device top-k (msim_topk_async) against the oracle's stable order for every
selector: threshold filter (n <= 4096, k <= 32), register selector
(n <= 16384), radix (larger k or n)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 100, 1000, 4096, 4097, 10000, 16384, 20000])
@pytest.mark.parametrize("k", [1, 10, 32, 33, 500])
def test_topk_matches_oracle_with_ties(gpu, oracle, n, k):
    import torch

    from maxsim_amd._maxsim_hip import _stream_ptr
    from maxsim_amd._native import check, ptr

    if k > n:
        pytest.skip("k must not exceed n")
    rng = np.random.default_rng(n * 131 + k)
    scores = rng.integers(-50, 50, size=(3, n)).astype(np.float32) * np.float32(0.25)  # many ties
    scores[1, : n // 2] = -np.inf
    scores[2, 0] = -0.0
    d = torch.from_numpy(scores).cuda()
    s = torch.empty((3, k), dtype=torch.float32, device="cuda")
    i = torch.empty((3, k), dtype=torch.int64, device="cuda")
    check(gpu.msim_topk_async(ptr(d), 3, n, n, k, ptr(s), ptr(i), _stream_ptr(None)))
    torch.cuda.synchronize()
    es, ei = oracle.topk(scores, k)
    np.testing.assert_array_equal(i.cpu().numpy(), ei)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
