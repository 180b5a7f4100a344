"""q3_cuda_q4k_linear under HIP graph capture.

The reference's contract for the call (src/q3_q4_linear.h:99-106) is
enqueue-only: no host synchronisation, no allocation, no copies. Capture in
global mode fails on any of those, so a clean capture checks the contract.
Replays must give the eager result bit for bit, several times in a row with
eager work (including other calls through the same arena) between them: the
split-K and stream-K counters are reset by the kernels themselves, so a
replay finds them at zero as an eager call does. Stats are NULL, as a
captured caller passes them (event records are for eager timing only).
"""
import ctypes
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    if not _t.cuda.is_available():
        pytest.fail("gpu test without a visible HIP device")
    q3q4.load()
    return _t


@pytest.fixture(scope="module")
def linear(torch):
    return q3q4.Linear(device=0, max_tokens=2048, max_features=151936, max_k=25600)


def weights(rng, qtype, N, K):
    if qtype == q3q4.QTYPE_Q4_K:
        return oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    if qtype == q3q4.QTYPE_Q4K_TILED:
        gguf = oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        return q3q4.q4k_tiled_bytes(gguf, N, K)
    return oracle.q6k_weights(rng, N, K)


def call(torch, geo, W, x, y):
    """One q3_cuda_q4k_linear on torch's current stream, stats NULL."""
    L = q3q4.load()
    err = ctypes.create_string_buffer(512)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ok = L.q3_cuda_q4k_linear(ctypes.byref(geo), ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                              x.shape[0], ctypes.c_void_p(y.data_ptr()), stream, None, err, 512)
    assert ok, err.value.decode()


def kernel_of(qtype, M, N, K):
    """The kernel the boundary runs for this call, from the library's own
    dispatch queries."""
    L = q3q4.load()
    if qtype in (q3q4.QTYPE_Q4_K, q3q4.QTYPE_Q4K_TILED):
        if M <= 8:
            return "fewtok" if L.sera_q4k_vec_uses_fewtok_qt(qtype, M, N, K) else "dot4"
        if L.sera_q4k_mmq_uses_fewtok(M, N, K):
            return "fewtok-mmq"
        return {1: "mmq-streamk", 2: "mmq-tail"}.get(L.sera_q4k_mmq_schedule(M, N, K), "mmq")
    return "q6k-tile" if M > 8 or L.sera_q6k_vec_uses_tile_qt(qtype, M, N, K) else "q6k-mmvq"


# (qtype, M, N, K, kernel): dot4 MMVQ; the few-token kernel with in-kernel
# split K on the row stage (form 0: a 4096-row matrix from 5 tokens, a tall
# one from 3) and on the MMQ stage (form 1, 9 tokens); the paired MMQ tile
# with split-K + reduce; stream-K (32-token tiles over a 131328-row matrix);
# the 64-token tile with split-K + reduce and under the tail schedule (whole
# tiles, then split tiles handed off through counters);
# Q6_K MMVQ and the Q6_K tile kernel on the row-formula stage, with split-K
# and under its tail schedule (also on the MMQ stage at 64 tokens); the few-token
# kernel's persistent grid (more 16-row tiles than resident workgroups); the
# same kernels on Q4_K weights in the tiled layout (268), where the few-token
# kernel takes tall matrices from 2 tokens
CASES = [
    (12, 1, 4096, 5120, "dot4"),
    (12, 6, 2048, 5120, "dot4"),
    (12, 8, 4096, 5120, "fewtok"),
    (12, 3, 16384, 5120, "fewtok"),
    (12, 9, 1000, 25600, "fewtok-mmq"),
    (12, 10, 1000, 2560, "mmq"),
    (12, 20, 131328, 256, "mmq-streamk"),
    (12, 64, 8192, 2048, "mmq"),
    (12, 100, 4096, 5120, "mmq"),
    (12, 200, 25600, 2048, "mmq-tail"),
    (12, 600, 25600, 1024, "mmq-tail"),
    (14, 1, 2048, 5120, "q6k-mmvq"),
    (14, 8, 2048, 5120, "q6k-mmvq"),
    (14, 8, 4096, 5120, "q6k-tile"),
    (14, 8, 5120, 25600, "q6k-tile+tail"),
    (14, 64, 5120, 25600, "q6k-tile+tail"),
    (12, 16, 70001, 512, "fewtok-mmq-persistent"),
    (268, 1, 4096, 5120, "dot4"),
    (268, 2, 16384, 5120, "fewtok"),
    (268, 20, 131328, 256, "mmq-streamk"),
    (268, 64, 8192, 2048, "mmq"),
    (268, 200, 25600, 2048, "mmq-tail"),
    (268, 16, 70000, 512, "fewtok-mmq-persistent"),
]


@pytest.mark.parametrize("qtype,M,N,K,kernel", CASES)
def test_graph_replay_matches_eager(torch, linear, qtype, M, N, K, kernel):
    say(f"case graph qtype={qtype} M={M} N={N} K={K} kernel={kernel}")
    persistent = kernel.endswith("-persistent")
    tail = kernel.endswith("+tail")
    kernel = kernel.replace("-persistent", "").replace("+tail", "")
    assert kernel_of(qtype, M, N, K) == kernel, "dispatch moved: choose a case that reaches this kernel"
    if tail:
        assert q3q4.q6k_mmq_tail_plan(M, N, K) is not None, "case meant for the Q6_K tail schedule"
    if persistent:
        form = 1 if kernel == "fewtok-mmq" else 0
        assert q3q4.fewtok_splits(M, N, K) == 1 and q3q4.fewtok_grid(form, M, N, K) < q3q4.fewtok_groups(M, N, K), \
            "case meant to run the few-token kernel's persistent grid"
    elif kernel.startswith("fewtok"):
        assert q3q4.fewtok_splits(M, N, K) > 1, "case meant to split K inside the few-token kernel"
    rng = np.random.default_rng(1000 * M + qtype)
    Wd = torch.from_numpy(weights(rng, qtype, N, K)).cuda()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    x_other = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    geo = q3q4.bind_geometry(qtype, K, N)
    y_ref = torch.empty((M, N), dtype=torch.float32, device="cuda")
    call(torch, geo, Wd, x, y_ref)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y_ref).all())

    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    y_other = torch.empty_like(y)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(torch, geo, Wd, x, y)          # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(torch, geo, Wd, x, y)
    for rep in range(3):
        y.fill_(float("nan"))
        call(torch, geo, Wd, x_other, y_other)  # eager call through the same arena
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f"  replay {rep}: equal={bool(torch.equal(y, y_ref))}")
        assert torch.equal(y, y_ref), f"replay {rep} differs from the eager result"
    del graph
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K", [(8, 5120, 25600), (1, 4096, 5120)])
def test_graph_replay_static_entry(torch, linear, M, N, K):
    """sera_q4k_dense_vec_static (the decode path on the library's static
    scratch) captured into a graph: replays equal the eager call bit for bit,
    with eager static calls on other inputs between them."""
    L = q3q4.load()
    kern = "few-token" if L.sera_q4k_vec_uses_fewtok(M, N, K) else "dot4"
    say(f"case graph static M={M} N={N} K={K} ({kern}, splits {q3q4.fewtok_splits(M, N, K)})")
    rng = np.random.default_rng(31 * M + N)
    Wd = torch.from_numpy(weights(rng, q3q4.QTYPE_Q4_K, N, K)).cuda()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    x_other = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()

    def static_call(xx, yy):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = L.sera_q4k_dense_vec_static(ctypes.c_void_p(Wd.data_ptr()), ctypes.c_void_p(xx.data_ptr()),
                                         ctypes.c_void_p(yy.data_ptr()), M, N, K, stream)
        assert rc == 0, L.sera_q4k_last_error().decode()

    y_ref = torch.empty((M, N), dtype=torch.float32, device="cuda")
    static_call(x, y_ref)               # eager; also sets the scratch up on this device
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y_ref).all())
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    y_other = torch.empty_like(y)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        static_call(x, y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        static_call(x, y)
    for rep in range(3):
        y.fill_(float("nan"))
        static_call(x_other, y_other)   # eager call on the same static scratch
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f"  replay {rep}: equal={bool(torch.equal(y, y_ref))}")
        assert torch.equal(y, y_ref), f"replay {rep} differs from the eager result"
    del graph
    torch.cuda.synchronize()
