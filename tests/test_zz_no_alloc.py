"""GPU test of msim_int4_topk_int8q_noalloc, called through the C ABI: its
top-k equals msim_int4_topk_int8q_async's bit for bit, and the C oracle's
stable top-k of its int8-query scores, on two calls in a row, the second with
a smaller input, and the call allocates nothing (the handle's workspace,
torch's allocations and the device's free memory stay as they were).  Both
entry points captured in a HIP graph and replayed match the oracle.
"""
import ctypes

import numpy as np
import pytest

from conftest import ragged_fixture
from maxsim_amd import _maxsim_hip
from maxsim_amd._native import Int4Props, check, ptr
from maxsim_amd.experimental import int4_to_device, pack_int4_symmetric

pytestmark = pytest.mark.gpu


def _setup(n, lo, hi, batch, qtok, seed, gran="token"):
    import torch

    docs, offsets = ragged_fixture(n, seed=seed, lo=lo, hi=hi)
    packed = pack_int4_symmetric(docs, offsets, scale_granularity=gran)
    handle = int4_to_device(packed).data
    rng = np.random.default_rng(seed + 1)
    query = torch.from_numpy(rng.standard_normal((batch, qtok, 128)).astype(np.float32)).cuda()
    return handle, query, packed


def _workspace_bytes(lib, handle):
    props = Int4Props()
    check(lib.msim_int4_get_props(handle._h, ctypes.byref(props)))
    return props.workspace_bytes


def _free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _run(lib, entry, handle, query, k, scores, ids):
    import torch

    batch, qtok = query.shape[:2]
    scores.fill_(float("nan"))
    ids.fill_(-1)
    stream = _maxsim_hip._stream_ptr(torch.cuda.current_stream())
    check(getattr(lib, entry)(handle._h, ptr(query), batch, qtok, k, ptr(scores), ptr(ids), stream))
    torch.cuda.synchronize()
    return scores.cpu().numpy(), ids.cpu().numpy()


def _compare(lib, handle, query, k, oracle=None, packed=None):
    import torch

    batch = query.shape[0]
    scores = torch.empty((batch, k), device="cuda")
    ids = torch.empty((batch, k), dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    before_ws, before_free = _workspace_bytes(lib, handle), _free_device_bytes()
    before_torch = torch.cuda.memory_allocated()
    got_s, got_i = _run(lib, "msim_int4_topk_int8q_noalloc", handle, query, k, scores, ids)
    # Nothing grows: the handle's workspaces, torch's allocations, free device memory.
    assert _workspace_bytes(lib, handle) == before_ws
    assert torch.cuda.memory_allocated() == before_torch
    assert _free_device_bytes() == before_free
    ref_s, ref_i = _run(lib, "msim_int4_topk_int8q_async", handle, query, k, scores, ids)
    np.testing.assert_array_equal(got_i, ref_i)
    np.testing.assert_array_equal(got_s.view(np.uint32), ref_s.view(np.uint32))
    if oracle is not None:
        exp = oracle.int4_int8q_scores(query.cpu().numpy(), packed.values, packed.doc_offsets,
                                       token_scale=packed.token_scale, scale=float(packed.scale))
        orc_s, orc_i = oracle.topk(exp, k)
        np.testing.assert_array_equal(got_i, orc_i)
        np.testing.assert_array_equal(got_s.view(np.uint32), orc_s.view(np.uint32))


@pytest.fixture
def fused_mode():
    yield _maxsim_hip.set_fused_topk
    _maxsim_hip.set_fused_topk(1)


# Two calls in a row, the second smaller: (docs, lo, hi, batch, query tokens, k, granularity)
PAIRS = [
    ((4096, 64, 192, 4, 32, 10, "token"), (1500, 8, 40, 2, 16, 7, "token")),   # config-2 shape, then smaller
    ((3000, 0, 60, 8, 16, 32, "tensor"), (300, 0, 20, 3, 8, 5, "tensor")),    # 8 batch rows, k at its limit
    ((900, 1, 30, 2, 64, 12, "token"), (100, 1, 10, 1, 32, 3, "token")),      # second call below 256 docs
    ((4096, 16, 64, 8, 16, 32, "token"), (2000, 4, 30, 5, 16, 9, "token")),   # the fused limits: 8 rows, 4096 docs, k 32
]


@pytest.mark.parametrize("mode", [1, 2, 0])
@pytest.mark.parametrize("pair", PAIRS, ids=["config2_then_small", "b8_then_small", "then_lt256", "limits_then_small"])
def test_noalloc_matches_async(gpu, oracle, fused_mode, mode, pair):
    import torch

    fused_mode(mode)
    # The first call on the device looks the scratch array up (its code object
    # may load then): make one before any memory is compared.
    handle, query, _ = _setup(300, 1, 4, 1, 1, seed=3)
    out_s = torch.empty((1, 1), device="cuda")
    out_i = torch.empty((1, 1), dtype=torch.int64, device="cuda")
    _run(gpu, "msim_int4_topk_int8q_noalloc", handle, query, 1, out_s, out_i)
    for i, (n, lo, hi, b, q, k, gran) in enumerate(pair):
        print(f"noalloc mode={mode} call={i} n={n} B={b} Q={q} k={k} {gran}", flush=True)
        handle, query, packed = _setup(n, lo, hi, b, q, seed=7 * n + q, gran=gran)
        _compare(gpu, handle, query, k, oracle, packed)


def test_noalloc_same_handle_shrinking_batch(gpu, oracle):
    import torch

    handle, query, packed = _setup(2048, 16, 80, 4, 32, seed=11)
    out_s = torch.empty((4, 10), device="cuda")
    out_i = torch.empty((4, 10), dtype=torch.int64, device="cuda")
    _run(gpu, "msim_int4_topk_int8q_noalloc", handle, query, 10, out_s, out_i)
    print("noalloc same handle B=4 then B=1", flush=True)
    _compare(gpu, handle, query, 10)
    _compare(gpu, handle, query[:1].contiguous(), 10, oracle, packed)


def test_noalloc_rejects_sizes_beyond_its_limits(gpu):
    import torch

    handle, query, _ = _setup(5000, 1, 6, 2, 32, seed=5)
    print("noalloc limits", flush=True)
    scores = torch.empty((8, 64), device="cuda")
    ids = torch.empty((8, 64), dtype=torch.int64, device="cuda")
    lib = gpu

    def call(q, k):
        return lib.msim_int4_topk_int8q_noalloc(handle._h, ptr(q), q.shape[0], q.shape[1], k, ptr(scores),
                                                ptr(ids), None)

    big = torch.zeros((5, 32, 128), device="cuda")  # 160 query rows
    with pytest.raises(ValueError, match="1 to 128 query rows"):
        check(call(big, 10))
    with pytest.raises(ValueError, match="k <= 32"):
        check(call(query, 33))
    # 5000 documents: no fused selection, and 8 x 5000 scores exceed the array.
    with pytest.raises(ValueError, match="32768 scores"):
        check(call(torch.zeros((8, 16, 128), device="cuda"), 10))
    with pytest.raises(ValueError, match="k must be between"):
        check(call(query, 0))


@pytest.mark.parametrize("entry", ["msim_int4_topk_int8q_noalloc", "msim_int4_topk_int8q_async"])
def test_captured_call_replays_match_the_oracle(gpu, oracle, entry):
    """The call captured in a HIP graph (the callers the no-alloc entry point
    is for) and replayed six times over three queries, with an eager call
    of the same entry point between replays: every replay and every eager
    call equals the oracle's top-k.  The fused selection's launch counter
    lives on the device, so replays, which the host does not see, still
    tag each launch apart."""
    import torch

    lib, k = gpu, 10
    handle, _, packed = _setup(2048, 8, 40, 4, 32, seed=41)
    rng = np.random.default_rng(42)
    queries = [torch.from_numpy(rng.standard_normal((4, 32, 128)).astype(np.float32)).cuda() for _ in range(3)]
    expected = []
    for q in queries:
        exp = oracle.int4_int8q_scores(q.cpu().numpy(), packed.values, packed.doc_offsets,
                                       token_scale=packed.token_scale, scale=float(packed.scale))
        expected.append(oracle.topk(exp, k))
    static_q = queries[0].clone()
    scores = torch.empty((4, k), device="cuda")
    ids = torch.empty((4, k), dtype=torch.int64, device="cuda")

    def call(stream):
        check(getattr(lib, entry)(handle._h, ptr(static_q), 4, 32, k, ptr(scores), ptr(ids),
                                  _maxsim_hip._stream_ptr(stream)))

    # A first call with these shapes outside the capture (workspaces, tables,
    # the scratch array's address).
    call(torch.cuda.current_stream())
    torch.cuda.synchronize()
    print(f"graph capture of {entry}", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(torch.cuda.current_stream())
    torch.cuda.synchronize()
    eager_s = torch.empty_like(scores)
    eager_i = torch.empty_like(ids)
    for r in range(6):
        print(f"replay {r}", flush=True)
        static_q.copy_(queries[r % 3])
        graph.replay()
        torch.cuda.synchronize()
        ref_s, ref_i = expected[r % 3]
        np.testing.assert_array_equal(ids.cpu().numpy(), ref_i)
        np.testing.assert_array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
        got_s, got_i = _run(lib, entry, handle, queries[(r + 1) % 3], k, eager_s, eager_i)
        ref_s, ref_i = expected[(r + 1) % 3]
        np.testing.assert_array_equal(got_i, ref_i)
        np.testing.assert_array_equal(got_s.view(np.uint32), ref_s.view(np.uint32))


def test_replays_across_the_key_tag_period(gpu, oracle):
    """More than 2^19 - 1 fused launches on the device's counter (1,025
    replays of a graph of 512 captured no-alloc calls): the launch whose tag
    closes the key-tag period zeroes the key rows on the device, and the
    replays and calls after it stay exact."""
    import torch

    lib, k = gpu, 5
    handle, query, packed = _setup(300, 1, 6, 2, 8, seed=51)
    rng = np.random.default_rng(52)
    others = [torch.from_numpy(rng.standard_normal((2, 8, 128)).astype(np.float32)).cuda() for _ in range(2)]

    def expect(q):
        exp = oracle.int4_int8q_scores(q.cpu().numpy(), packed.values, packed.doc_offsets,
                                       token_scale=packed.token_scale, scale=float(packed.scale))
        return oracle.topk(exp, k)

    scores = torch.empty((2, k), device="cuda")
    ids = torch.empty((2, k), dtype=torch.int64, device="cuda")

    def call(stream):
        check(lib.msim_int4_topk_int8q_noalloc(handle._h, ptr(query), 2, 8, k, ptr(scores), ptr(ids),
                                               _maxsim_hip._stream_ptr(stream)))

    call(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(512):
            call(torch.cuda.current_stream())
    torch.cuda.synchronize()
    for r in range(1025):
        graph.replay()
        if r % 256 == 255:
            torch.cuda.synchronize()
            print(f"replays {r + 1} ({(r + 1) * 512} launches)", flush=True)
    torch.cuda.synchronize()
    ref_s, ref_i = expect(query)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_i)
    np.testing.assert_array_equal(scores.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))
    for q in others:
        ref_s, ref_i = expect(q)
        for entry in ("msim_int4_topk_int8q_noalloc", "msim_int4_topk_int8q_async"):
            got_s, got_i = _run(lib, entry, handle, q, k, scores, ids)
            np.testing.assert_array_equal(got_i, ref_i)
            np.testing.assert_array_equal(got_s.view(np.uint32), ref_s.view(np.uint32))
