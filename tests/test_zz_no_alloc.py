"""sera_q4k_dense_vec_static: the decode path on the library's static
scratch, allocating nothing and needing no attached workspace.

It runs the same kernels as sera_q4k_dense_vec, so its outputs must equal
that entry point's bit for bit (the parity bar for the same integer and fp32
arithmetic). Two calls in a row share the one static scratch: the first
(8 tokens on the 25600 -> 5120 down shape) runs the few-token kernel with K
split in five and uses the split slots and row-group counters, the second
(3 tokens, 5120 -> 2048) is smaller and runs the dot4 kernel; both must
match. Device memory in use does not change across the static calls, and a
shape that needs more than the static scratch is rejected with a message.

The first static call on a device sets the scratch up itself (looks up its
address and clears its counters on the caller's stream) unless the
library's init already did. In this test process other tests have called
init first, so a second test runs the static calls in a fresh child
process that calls nothing else in the library, and compares its outputs
with sera_q4k_dense_vec's here.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import q3q4

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_static_entry_point_matches_dense_vec():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible HIP device")
    L = q3q4.load()
    cases = [(8, 5120, 25600), (3, 2048, 5120)]
    rng = np.random.default_rng(2024)
    data = []
    for M, N, K in cases:
        g = torch.Generator(device="cuda").manual_seed(N + K)
        wf = torch.randn((N, K), generator=g, device="cuda", dtype=torch.float32) * 0.02
        W = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
        q3q4.quantize_weights(wf, W)
        del wf
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
        data.append((M, N, K, W, x))
    torch.cuda.synchronize()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def static_call(M, N, K, W, x, y):
        rc = L.sera_q4k_dense_vec_static(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                         ctypes.c_void_p(y.data_ptr()), M, N, K, stream)
        assert rc == 0, L.sera_q4k_last_error().decode()

    got = [torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda") for M, N, K, _, _ in data]
    warm = [torch.empty_like(y) for y in got]
    # one-time set-up: in a fresh process the first call looks up and clears
    # the static scratch itself, and the runtime prepares each kernel on its
    # first launch; neither is the entry point allocating per call
    for d, w in zip(data[::-1], warm[::-1]):
        static_call(*d[:5], w)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for (M, N, K, W, x), y in zip(data, got):
        kern = "few-token" if L.sera_q4k_vec_uses_fewtok(M, N, K) else "dot4"
        say(f"case static M={M} N={N} K={K} ({kern}, splits {q3q4.fewtok_splits(M, N, K)}, "
            f"scratch {L.sera_q4k_dense_vec_static_bytes(M, N, K)} B)")
        static_call(M, N, K, W, x, y)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 == free1, "the static entry point changed device memory in use"

    # the existing entry point, on a workspace the caller attaches
    lin = q3q4.Linear(device=0, max_tokens=8, max_features=5120, max_k=25600)
    for (M, N, K, W, x), ys in zip(data, got):
        yv = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        rc = L.sera_q4k_dense_vec(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                  ctypes.c_void_p(yv.data_ptr()), M, N, K, stream, 0)
        assert rc == 0, L.sera_q4k_last_error().decode()
        torch.cuda.synchronize()
        a, b = ys.cpu().numpy(), yv.cpu().numpy()
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"M={M} N={N} K={K}"
        say(f"  M={M} N={N} K={K}: bit-identical to sera_q4k_dense_vec")
    del lin

    # beyond the static scratch: rejected before anything is enqueued
    M, N, K = 8, 65536, 25600
    assert L.sera_q4k_dense_vec_static_bytes(M, N, K) > 8 << 20
    W, x = data[0][3], data[0][4]
    rc = L.sera_q4k_dense_vec_static(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                     ctypes.c_void_p(got[0].data_ptr()), M, N, K, stream)
    assert rc == -1 and b"static" in L.sera_q4k_last_error()


CHILD = r"""
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[2])
import q3q4
L = q3q4.load()
d = sys.argv[1]
stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
for i, (M, N, K) in enumerate([(8, 5120, 25600), (3, 2048, 5120)]):
    W = torch.from_numpy(np.load(f"{d}/w{i}.npy")).cuda()
    x = torch.from_numpy(np.load(f"{d}/x{i}.npy")).cuda()
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    print(f"child static call M={M} N={N} K={K}", flush=True)
    rc = L.sera_q4k_dense_vec_static(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                     ctypes.c_void_p(y.data_ptr()), M, N, K, stream)
    assert rc == 0, L.sera_q4k_last_error().decode()
    torch.cuda.synchronize()
    np.save(f"{d}/y{i}.npy", y.cpu().numpy())
print("child done", flush=True)
"""


def test_static_entry_point_in_a_fresh_process(tmp_path):
    """The static calls of a process that never initialised the library:
    the first one sets the scratch up on the caller's stream."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible HIP device")
    L = q3q4.load()
    rng = np.random.default_rng(77)
    cases = [(8, 5120, 25600), (3, 2048, 5120)]
    data = []
    for i, (M, N, K) in enumerate(cases):
        g = torch.Generator(device="cuda").manual_seed(3 * N + K)
        wf = torch.randn((N, K), generator=g, device="cuda", dtype=torch.float32) * 0.02
        W = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
        q3q4.quantize_weights(wf, W)
        del wf
        x = rng.standard_normal((M, K)).astype(np.float32)
        np.save(tmp_path / f"w{i}.npy", W.cpu().numpy())
        np.save(tmp_path / f"x{i}.npy", x)
        data.append((M, N, K, W, torch.from_numpy(x).cuda()))
    torch.cuda.synchronize()
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sera.c_amd")
    say("starting the child process")
    r = subprocess.run([sys.executable, "-c", CHILD, str(tmp_path), pkg], capture_output=True, text=True,
                       timeout=240)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().splitlines()[-1] == "child done"
    lin = q3q4.Linear(device=0, max_tokens=8, max_features=5120, max_k=25600)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, (M, N, K, W, x) in enumerate(data):
        yv = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        rc = L.sera_q4k_dense_vec(ctypes.c_void_p(W.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                  ctypes.c_void_p(yv.data_ptr()), M, N, K, stream, 0)
        assert rc == 0, L.sera_q4k_last_error().decode()
        torch.cuda.synchronize()
        a = np.load(tmp_path / f"y{i}.npy")
        b = yv.cpu().numpy()
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"M={M} N={N} K={K}"
        say(f"  fresh process M={M} N={N} K={K}: bit-identical to sera_q4k_dense_vec")
    del lin
