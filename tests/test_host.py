"""Host-side checks that need no GPU: the C ABI library loads and exports what
include/maxsim_hip.h declares, the host packers equal the oracle bit for bit,
and the Python layer raises the reference's errors before touching a device."""
import ctypes
import os
import re
from dataclasses import replace

import numpy as np
import pytest

import maxsim_amd
from maxsim_amd import _native, synthetic
from maxsim_amd.experimental import int4_maxsim, int4_maxsim_int8q, int4_to_device, pack_int4_symmetric

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "maxsim_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msim_[a-z0-9_]+)\s*\(", text)))


# ------------------------------------------------------------------ C ABI


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert "msim_int4_topk_int8q_async" in names and "msim_last_error" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    """dlopen the in-tree library (no device call) and resolve every declared name."""
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail("maxsim_amd/libmaxsim_hip.so is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_signatures_cover_the_header():
    assert sorted(_native.SIGNATURES) == _declared_functions()


def test_abi_version_and_error_string_without_device():
    lib = _native.load()
    assert lib.msim_abi_version() >= 100
    assert isinstance(lib.msim_last_error(), bytes)


def test_docs_per_wave_knob_validation():
    lib = _native.load()
    assert lib.msim_set_docs_per_wave(-1) == _native.MSIM_EINVAL
    assert b"docs per wave" in lib.msim_last_error()
    assert lib.msim_set_docs_per_wave(0) == _native.MSIM_OK
    assert lib.msim_get_docs_per_wave() == 0


def test_fused_topk_knob_validation():
    lib = _native.load()
    assert lib.msim_set_fused_topk(3) == _native.MSIM_EINVAL
    assert b"fused top-k mode" in lib.msim_last_error()
    assert lib.msim_get_fused_topk() == 1
    assert lib.msim_set_fused_topk(1) == _native.MSIM_OK


def test_pack_int4_shape_errors_without_device():
    """Shape checks of the device packer run before any device call
    (messages of experimental.py:226-232)."""
    lib = _native.load()
    assert lib.msim_pack_int4(None, 4, 12, 0, 0.0, None, None, None, None) == _native.MSIM_EINVAL
    assert b"divisible by 8" in lib.msim_last_error()
    assert lib.msim_pack_int4(None, 4, 7, 0, 0.0, None, None, None, None) == _native.MSIM_EINVAL
    assert b"divisible by 2" in lib.msim_last_error()
    assert lib.msim_pack_int4_async(None, 4, 0, 1, 0.0, None, None, None, None, None) == _native.MSIM_EINVAL
    assert b"dim must be positive" in lib.msim_last_error()


def test_product_never_imports_the_oracle():
    """The checker lives in oracle/; nothing under maxsim_amd/ may load it."""
    pkg = os.path.join(ROOT, "maxsim_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"import\s+oracle|from\s+oracle|liboracle|maxsim_oracle", text), f


# ---------------------------------------------------------- host packers


@pytest.mark.parametrize("granularity", ["token", "tensor"])
def test_pack_int4_symmetric_matches_oracle(oracle, granularity):
    docs, offsets = synthetic.make_corpus(64, 1, 40).embeddings, synthetic.make_corpus(64, 1, 40).offsets
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=granularity)
    if granularity == "token":
        codes, values, ts = oracle.pack_int4_token(docs)
        np.testing.assert_array_equal(packed.token_scale, ts)
        assert packed.scale == 1.0
    else:
        codes, values, scale = oracle.pack_int4_tensor(docs)
        assert packed.scale == scale and packed.token_scale is None
    np.testing.assert_array_equal(packed.data, codes)
    np.testing.assert_array_equal(packed.values, values)


def test_pack_signs_matches_oracle(oracle):
    docs, offsets = synthetic.make_corpus(32, 1, 20).embeddings, synthetic.make_corpus(32, 1, 20).offsets
    packed = maxsim_amd.pack_signs(docs, offsets)
    np.testing.assert_array_equal(packed.data, oracle.pack_signs(docs))
    assert maxsim_amd.pack_signs(np.array([[-1, 0, 2, -3, 4, -5, 6, -7]], np.float32)).data.tolist() == [[0b01010110]]


def test_pack_int4_token_kat_through_product():
    docs = np.array(
        [[0.0] * 8, [-14.0, -7.0, 0.0, 2.0, 4.0, 6.0, 10.0, 14.0], [-0.7, -0.5, -0.3, -0.1, 0.1, 0.3, 0.5, 0.7]],
        np.float32,
    )
    packed = pack_int4_symmetric(docs, scale_granularity="token")
    np.testing.assert_allclose(packed.token_scale, [1.0, 2.0, 0.1], rtol=1e-6, atol=0)
    assert packed.token_scale.dtype == np.float32 and packed.token_scale.flags.c_contiguous


# ------------------------------------------------ validation (no device)


@pytest.mark.parametrize("bad", ["doc", "channel", ""])
def test_rejects_unknown_scale_granularity(bad):
    with pytest.raises(ValueError, match="scale_granularity"):
        pack_int4_symmetric(np.ones((1, 8), np.float32), scale_granularity=bad)


def test_rejects_explicit_scale_in_token_mode():
    with pytest.raises(ValueError, match="scale"):
        pack_int4_symmetric(np.ones((1, 8), np.float32), scale=1.0, scale_granularity="token")


def test_rejects_negative_eight_code():
    """tests/test_int4_reference.py:265-278."""
    packed = pack_int4_symmetric(np.ones((1, 8), np.float32))
    values = packed.values.copy()
    values[0, 0] = -8
    with pytest.raises(ValueError, match="symmetric int4"):
        int4_maxsim(np.ones((1, 8), np.float32), replace(packed, values=values))


def test_rejects_data_that_does_not_encode_values():
    """tests/test_int4_reference.py:249-262 (raised before any upload)."""
    packed = pack_int4_symmetric(np.arange(16, dtype=np.float32).reshape(2, 8), scale_granularity="token")
    corrupt = packed.data.copy()
    corrupt[0, 0] ^= np.uint8(1)
    with pytest.raises(ValueError, match="does not encode"):
        int4_to_device(replace(packed, data=corrupt))


def test_int8q_empty_queries_return_without_device():
    """tests/test_int4_int8q.py:38-53."""
    packed = pack_int4_symmetric(np.ones((3, 128), np.float32), np.arange(4, dtype=np.int64),
                                 scale_granularity="token")
    assert int4_maxsim_int8q(np.empty((0, 2, 128), np.float32), packed).shape == (0, 3)
    np.testing.assert_array_equal(int4_maxsim_int8q(np.empty((0, 128), np.float32), packed), np.zeros(3, np.float32))


def test_cpu_device_is_rejected():
    packed = pack_int4_symmetric(np.ones((2, 8), np.float32))
    with pytest.raises(NotImplementedError):
        int4_maxsim(np.ones((1, 8), np.float32), packed, device="cpu")


@pytest.mark.parametrize(
    "kwargs,match",
    [
        ({"reducer": "mean"}, "reducer must be one of"),
        ({"reducer": "smoothsim", "temperature": 0.0}, "temperature"),
        ({"reducer": "smoothsim", "temperature": float("nan")}, "temperature"),
        ({"reducer": "maxsim", "query_weights": [1.0]}, "only supported"),
        ({"reducer": "weighted_maxsim"}, "required"),
        ({"reducer": "weighted_maxsim", "query_weights": [1.0, 2.0]}, "shape"),
        ({"candidate_indices": [5]}, "between 0"),
        ({"candidate_indices": [[0]]}, "one-dimensional"),
    ],
)
def test_reducer_and_candidate_validation(kwargs, match):
    packed = pack_int4_symmetric(np.ones((2, 8), np.float32), np.array([0, 1, 2]))
    with pytest.raises(ValueError, match=match):
        int4_maxsim(np.ones((1, 8), np.float32), packed, **kwargs)


def test_query_dim_mismatch():
    packed = pack_int4_symmetric(np.ones((2, 8), np.float32))
    with pytest.raises(ValueError, match="does not match"):
        int4_maxsim(np.ones((1, 16), np.float32), packed)


@pytest.mark.parametrize("offsets,match", [([1, 2], "start at 0"), ([0, 1], "end at"), ([0, 2, 1, 2], "nondecreasing")])
def test_offsets_validation(offsets, match):
    with pytest.raises(ValueError, match=match):
        pack_int4_symmetric(np.ones((2, 8), np.float32), np.array(offsets))


# ------------------------------------------------------- synthetic data


def test_synthetic_generator_is_deterministic_and_normalised():
    a = synthetic.make_corpus(40, 3, 9)
    b = synthetic.make_corpus(40, 3, 9)
    np.testing.assert_array_equal(a.embeddings, b.embeddings)
    np.testing.assert_array_equal(a.offsets, b.offsets)
    assert a.lengths.min() >= 3 and a.lengths.max() <= 9
    np.testing.assert_allclose(np.linalg.norm(a.embeddings, axis=1), 1.0, rtol=1e-5)
    q = synthetic.make_queries(a, 3)
    assert q.shape == (3, 32, 128)
    np.testing.assert_allclose(np.linalg.norm(q, axis=2), 1.0, rtol=1e-5)


def test_config2_token_count():
    cfg = synthetic.CONFIGS[2]
    lengths = synthetic.doc_lengths(cfg["num_docs"], cfg["lo"], cfg["hi"])
    assert lengths.shape == (4096,) and int(lengths.sum()) == 523330


def test_pack_binary_residual_matches_oracle(oracle):
    from maxsim_amd.binres import pack_binary_residual

    corpus = synthetic.make_corpus(40, 1, 30)
    packed = pack_binary_residual(corpus.embeddings, corpus.offsets)
    signs, a, rcodes, rvalues, rscale = oracle.pack_binary_residual(corpus.embeddings)
    np.testing.assert_array_equal(packed.sign_data, signs)
    np.testing.assert_array_equal(packed.prefix_scale, a)
    np.testing.assert_array_equal(packed.residual_data, rcodes)
    np.testing.assert_array_equal(packed.residual_values, rvalues)
    np.testing.assert_array_equal(packed.residual_token_scale, rscale)
    assert packed.storage_bytes == packed.num_tokens * 88


def test_pack_residual_int4_two_stream_reconstruction():
    """cascade.py:60-93: prefix = token int4 of x, residual = token int4 of x - prefix."""
    from maxsim_amd.cascade import _reconstruct_int4, pack_residual_int4

    corpus = synthetic.make_corpus(30, 1, 20)
    packed = pack_residual_int4(corpus.embeddings, corpus.offsets)
    prefix = _reconstruct_int4(packed.prefix_values, packed.prefix_scale, packed.prefix_token_scale)
    res = pack_int4_symmetric(corpus.embeddings - prefix, corpus.offsets, scale_granularity="token")
    np.testing.assert_array_equal(packed.residual_values, res.values)
    recon = prefix + _reconstruct_int4(packed.residual_values, packed.residual_scale, packed.residual_token_scale)
    assert np.max(np.abs(recon - corpus.embeddings)) < np.max(np.abs(prefix - corpus.embeddings))


@pytest.mark.parametrize("kwargs,match", [({"candidates": 3, "k": 4}, "cascade sizes"),
                                          ({"candidates": 99, "k": 1}, "cascade sizes")])
def test_cascade_size_validation(kwargs, match):
    from maxsim_amd.cascade import cascade_topk, pack_residual_int4

    corpus = synthetic.make_corpus(10, 1, 5)
    packed = pack_residual_int4(corpus.embeddings, corpus.offsets)
    with pytest.raises(ValueError, match=match):
        cascade_topk(np.ones((2, 128), np.float32), packed, kwargs["k"], candidates=kwargs["candidates"])


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says so
    (before touching a GPU)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


@pytest.mark.parametrize("args, match", [
    ((np.zeros((2, 2, 8), np.float32), np.zeros((3, 1), np.uint8), [0, 3], 8), r"query must have shape \[query_tokens, dim\]"),
    ((np.zeros((2, 8), np.float32), np.zeros(3, np.uint8), [0, 3], 8), r"packed must have shape \[num_doc_tokens, dim / 8\]"),
    ((np.zeros((2, 8), np.float32), np.zeros((3, 1), np.uint8), [[0, 3]], 8), "offsets must be a 1-D array"),
    ((np.zeros((2, 8), np.float32), np.zeros((3, 1), np.uint8), [0, 3], 12), "dim must be positive and divisible by 8"),
    ((np.zeros((2, 16), np.float32), np.zeros((3, 1), np.uint8), [0, 3], 8), "query/packed shapes do not match dim"),
])
def test_maxsim_cuda_validation_without_device(args, match):
    """maxsim_cuda's argument checks in the reference's order and wording
    (validate_inputs, cuda_extension.cu:1826-1847), before any device work."""
    from maxsim_amd import _maxsim_hip

    with pytest.raises(ValueError, match=match):
        _maxsim_hip.maxsim_cuda(*args)


def test_maxsim_cuda_batch_requires_3d_query():
    from maxsim_amd import _maxsim_hip

    with pytest.raises(ValueError, match=r"query must have shape \[batch, query_tokens, dim\]"):
        _maxsim_hip.maxsim_cuda_batch(np.zeros((2, 8), np.float32), np.zeros((3, 1), np.uint8), [0, 3], 8)


def test_reference_routing_knobs_validate_like_the_reference():
    """The reference module's launch-shape knobs (cuda_extension.cu:3482-3513):
    same defaults, accepted values and ValueError texts; a rejected value
    leaves the setting unchanged (tests/test_cuda_reducers.py:519-528)."""
    from maxsim_amd import _maxsim_hip as h

    assert (h.get_shared_reducer_warps(), h.get_residual_reducer_warps(), h.get_residual_reducer_force_warps()) == (
        4, 8, -1)
    assert h.get_dim128_unrolled_min_avg_tokens() == 256
    assert h.get_dim128_qtile_min_packed_bytes() == 2**64 - 1
    for setter, getter, good, bad, msg in [
        (h.set_shared_reducer_warps, h.get_shared_reducer_warps, (0, 4, 8), (-1, 1, 2, 16), "one of 0, 4, or 8"),
        (h.set_residual_reducer_warps, h.get_residual_reducer_warps, (0, 4, 8), (-1, 1, 2, 16), "one of 0, 4, or 8"),
        (h.set_residual_reducer_force_warps, h.get_residual_reducer_force_warps, (-1, 0, 4, 8), (-2, 1, 16),
         "one of -1, 0, 4, or 8"),
    ]:
        prior = getter()
        try:
            for v in good:
                setter(v)
                assert getter() == v
            for v in bad:
                before = getter()
                with pytest.raises(ValueError, match=msg):
                    setter(v)
                assert getter() == before
        finally:
            setter(prior)
    # The residual policy of cu:58-76.
    prior = (h.get_residual_reducer_warps(), h.get_residual_reducer_force_warps())
    try:
        assert [h.get_effective_residual_reducer_warps(q) for q in (1, 7, 8, 32)] == [4, 4, 8, 8]
        h.set_residual_reducer_warps(4)
        assert [h.get_effective_residual_reducer_warps(q) for q in (1, 3, 4, 32)] == [0, 0, 4, 4]
        h.set_residual_reducer_force_warps(0)
        assert h.get_effective_residual_reducer_warps(32) == 0
        with pytest.raises(ValueError, match="query tokens must be positive"):
            h.get_effective_residual_reducer_warps(0)
    finally:
        h.set_residual_reducer_warps(prior[0])
        h.set_residual_reducer_force_warps(prior[1])
    prior_q = h.get_dim128_qtile_min_packed_bytes()
    try:
        h.set_dim128_qtile_min_packed_bytes(1 << 62)
        assert h.get_dim128_qtile_min_packed_bytes() == 1 << 62
        with pytest.raises(TypeError):
            h.set_dim128_qtile_min_packed_bytes(-1)
    finally:
        h.set_dim128_qtile_min_packed_bytes(prior_q)


def test_routing_knobs_are_per_thread_like_the_reference():
    """The warp knobs are thread_local in the reference (cu:44-56)."""
    import threading

    from maxsim_amd import _maxsim_hip as h

    prior = h.get_shared_reducer_warps()
    seen = []
    try:
        h.set_shared_reducer_warps(8)
        t = threading.Thread(target=lambda: seen.append(h.get_shared_reducer_warps()))
        t.start()
        t.join()
        assert seen == [4] and h.get_shared_reducer_warps() == 8
    finally:
        h.set_shared_reducer_warps(prior)
