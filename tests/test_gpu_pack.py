"""GPU parity: the device int4 packer (msim_pack_int4 / msim_pack_int4_async)
against the host packer, which the CPU suite pins to the reference's KATs
(tests/test_int4_reference.py:5-49 of the reference).  Codes, values, token
scales and the tensor scale must be identical bit for bit.
"""
import numpy as np
import pytest

import maxsim_amd as maxsim
from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric, pack_int4_symmetric_device

pytestmark = pytest.mark.gpu


def _same(a, b):
    np.testing.assert_array_equal(a.data, b.data)
    np.testing.assert_array_equal(a.values, b.values)
    np.testing.assert_array_equal(a.doc_offsets, b.doc_offsets)
    assert a.dim == b.dim and a.num_docs == b.num_docs
    assert a.scale == b.scale
    if b.token_scale is None:
        assert a.token_scale is None
    else:
        np.testing.assert_array_equal(a.token_scale.view(np.uint32), b.token_scale.view(np.uint32))


def _embeddings(t, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((t, d)).astype(np.float32) * rng.uniform(0.01, 10, size=(t, 1)).astype(np.float32)
    if t > 3:
        x[1] = 0.0                                      # zero row: scale 1.0
        x[2, :] = np.float32(1e-30)                     # tiny values
        x[3, :8] = np.array([7, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], np.float32)  # ties at .5 after /1
        x[3, 8:] = 0.0
    return x


@pytest.mark.parametrize("granularity", ["token", "tensor"])
@pytest.mark.parametrize("shape", [(1000, 128), (257, 64), (130, 96), (77, 256), (5, 8), (0, 128)])
def test_device_pack_matches_host(gpu, granularity, shape):
    t, d = shape
    print(f"case pack {granularity} T={t} dim={d}", flush=True)
    x = _embeddings(t, d, seed=t + d)
    offsets = np.array([0, t // 2, t], np.int64)
    _same(pack_int4_symmetric_device(x, offsets, scale_granularity=granularity),
          pack_int4_symmetric(x, offsets, scale_granularity=granularity))


def test_device_pack_given_tensor_scale(gpu):
    x = _embeddings(300, 128, seed=5)
    _same(pack_int4_symmetric_device(x, scale=0.37), pack_int4_symmetric(x, scale=0.37))


def test_device_pack_from_torch_cuda(gpu):
    import torch

    x = _embeddings(700, 128, seed=6)
    xt = torch.from_numpy(x).cuda()
    for granularity in ("token", "tensor"):
        print(f"case torch pack {granularity}", flush=True)
        _same(pack_int4_symmetric_device(xt, scale_granularity=granularity),
              pack_int4_symmetric(x, scale_granularity=granularity))
    no_values = pack_int4_symmetric_device(xt, scale_granularity="token", values=False)
    assert no_values.values is None
    np.testing.assert_array_equal(no_values.data, pack_int4_symmetric(x, scale_granularity="token").data)


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_device_pack_rejects_non_finite(gpu, bad):
    x = _embeddings(64, 128, seed=7)
    x[10, 3] = bad
    for granularity in ("token", "tensor"):
        with pytest.raises(ValueError, match="finite"):
            pack_int4_symmetric_device(x, scale_granularity=granularity)
    import torch

    with pytest.raises(ValueError, match="finite"):
        pack_int4_symmetric_device(torch.from_numpy(x).cuda(), scale_granularity="token")
    # Finiteness is checked before the scale arguments (experimental.py:233-240).
    with pytest.raises(ValueError, match="finite"):
        pack_int4_symmetric_device(x, scale=1.0, scale_granularity="token")


def test_device_pack_argument_errors(gpu):
    x = _embeddings(16, 128, seed=8)
    with pytest.raises(ValueError, match="scale cannot be provided"):
        pack_int4_symmetric_device(x, scale=1.0, scale_granularity="token")
    with pytest.raises(ValueError, match="scale_granularity"):
        pack_int4_symmetric_device(x, scale_granularity="row")
    with pytest.raises(ValueError, match="finite and > 0"):
        pack_int4_symmetric_device(x, scale=0.0)
    with pytest.raises(ValueError, match="divisible by 8"):
        pack_int4_symmetric_device(np.zeros((4, 12), np.float32))


def test_device_packed_corpus_searches_like_host_packed(gpu):
    rng = np.random.default_rng(9)
    lengths = rng.integers(1, 20, size=300)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    x = rng.standard_normal((int(offsets[-1]), 128)).astype(np.float32)
    query = rng.standard_normal((2, 16, 128)).astype(np.float32)
    host = int4_to_device(pack_int4_symmetric(x, offsets, scale_granularity="token"))
    dev = int4_to_device(pack_int4_symmetric_device(x, offsets, scale_granularity="token"))
    np.testing.assert_array_equal(maxsim.int4_maxsim_int8q(query, dev), maxsim.int4_maxsim_int8q(query, host))
