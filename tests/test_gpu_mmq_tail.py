"""MMQ under the tail schedule (whole tiles, then the last round's tiles cut
along K), through the C ABI.

The schedule changes only which workgroup computes which (tile, K range)
and how split tiles are summed; the per-32 int32 dots and the fp32 terms
are the MMQ kernel's own (cuda/mmq/mmq.cuh:1440-1472,2269-2283). So:

  * on the exact-input construction of test_gpu_exact (every partial sum an
    exact fp32 value) the output equals the dequant GEMM bit for bit, for
    any split: whole tiles only, a split tail after whole tiles, everything
    split, one piece per super-block, on all three token tiles (16, 32, 64;
    the 64-token tile at 128 and 256 weight rows)
    and on the tiled weight layout;
  * on random inputs it sits within 2e-5 * rms of the MMQ oracle (the same
    terms summed in another order), repeats bit for bit, leaves its
    counters at zero, and accumulate adds exactly the product;
  * the boundary (q3_cuda_q4k_linear) runs it for M > 32 on more than P/8
    tiles with the plan sera_q4k_mmq_tail_plan gives, and is bit-identical
    to the kernel entry point called with that plan.
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle
from test_gpu_exact import assert_bits, dev, exact_inputs, expected, mmq_stage, nan_out

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


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
    return q3q4.Linear(device=0, max_tokens=2048, max_features=25600, max_k=25600)


def run_tail(torch, Wd, st, M, N, K, dp, pieces, y=None, accum=False, qtype=q3q4.QTYPE_Q4_K):
    L = q3q4.load()
    T = L.sera_q4k_mmq_tiles(M, N)
    nslot = q3q4.mmq_tail_slot_floats(M, N, dp, pieces)
    slots = torch.empty(max(nslot, 1), dtype=torch.float32, device="cuda")
    counters = torch.zeros(max(T - dp, 1), dtype=torch.int32, device="cuda")
    if y is None:
        y = nan_out(torch, M, N)
    q3q4.mmq_tail(Wd, st, y, M, N, K, dp, pieces, slots=slots, counters=counters, accum=accum, qtype=qtype)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0, "tile counters not reset"
    return y


def tail_cases(M, N, K):
    """(dp_tiles, pieces): whole tiles only; everything split in 2 and in
    nkb pieces; half the tiles whole with the rest in 3 (or nkb) pieces."""
    T = q3q4.load().sera_q4k_mmq_tiles(M, N)
    nkb = K // 256
    out = [(T, 1), (0, min(2, nkb)), (0, nkb), (T // 2, min(3, nkb)), (T - 1, nkb)]
    return sorted(set(out))


# (M, N, K): paired 16-token tile, 32-token tile, 64-token tile of 128 rows
# (up to 64 tiles of 256 rows) and of 256 rows (the last), ragged M and N
EXACT = [(16, 512, 5120), (20, 300, 2304), (33, 384, 5120), (100, 256, 2048), (200, 640, 1024), (64, 64, 25600),
         (65, 16640, 1024)]


@pytest.mark.parametrize("M,N,K", EXACT)
def test_tail_exact(torch, M, N, K):
    rng = np.random.default_rng(M * 13 + N + K)
    W, X = exact_inputs(rng, M, N, K)
    ref = expected(W, X, N, K)
    Wd = dev(torch, W)
    st = mmq_stage(torch, X)
    for dp, pieces in tail_cases(M, N, K):
        say(f"case exact mmq tail M={M} N={N} K={K} dp_tiles={dp} pieces={pieces}")
        y = run_tail(torch, Wd, st, M, N, K, dp, pieces)
        assert_bits(y, ref, f"tail M={M} N={N} K={K} dp={dp} pieces={pieces}")
    if N % 16 == 0:
        T = q3q4.QTYPE_Q4K_TILED
        Wt = dev(torch, q3q4.q4k_tiled_bytes(W, N, K))
        dp, pieces = tail_cases(M, N, K)[-1]
        say(f"case exact mmq tail tiled M={M} N={N} K={K} dp_tiles={dp} pieces={pieces}")
        y = run_tail(torch, Wt, st, M, N, K, dp, pieces, qtype=T)
        assert_bits(y, ref, f"tail tiled M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K", [(512, 1024, 5120), (96, 2048, 2560), (40, 1000, 8192)])
def test_tail_parity_repeat_accumulate(torch, M, N, K):
    rng = np.random.default_rng(M + N + K)
    W = oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    X = rng.standard_normal((M, K)).astype(np.float32)
    xq, xd, xs = oracle.q8_1_mmq(X)
    ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
    rms = float(np.sqrt(np.mean(ref * ref)))
    Wd = dev(torch, W)
    st = mmq_stage(torch, X)
    for dp, pieces in tail_cases(M, N, K):
        say(f"case mmq tail M={M} N={N} K={K} dp_tiles={dp} pieces={pieces}")
        y = run_tail(torch, Wd, st, M, N, K, dp, pieces)
        err = float(np.max(np.abs(y.cpu().numpy().astype(np.float64) - ref)))
        say(f"  max|err| / rms = {err / rms:.2e}")
        assert err <= TIGHT * rms
        y2 = run_tail(torch, Wd, st, M, N, K, dp, pieces)
        assert torch.equal(y, y2), "repeat differs"
        base = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
        acc = base.clone()
        run_tail(torch, Wd, st, M, N, K, dp, pieces, y=acc, accum=True)
        assert torch.equal(acc, base + y), "accumulate is not y + product"


def test_schedule_rule(torch, linear):
    """The tail schedule takes the 64-token tile from more than P/8 tiles
    (P = 2 * CUs resident workgroups); split-K below that, and stream-K /
    split-K for the 16- and 32-token tiles."""
    L = q3q4.load()
    P = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    for M, N, K in [(512, 25600, 5120), (512, 1024, 5120), (128, 8192, 5120), (256, 5120, 8192), (64, 25600, 5120),
                    (33, 4096, 5120), (32, 151936, 5120), (16, 4096, 5120)]:
        T = L.sera_q4k_mmq_tiles(M, N)
        got = L.sera_q4k_mmq_schedule(M, N, K)
        if M > 32:
            assert got == (2 if 8 * T > P else 0), (M, N, K, T)
        else:
            assert got in (0, 1), (M, N, K, T)


@pytest.mark.parametrize("M,N,K", [(512, 25600, 5120), (512, 5120, 25600), (2048, 5120, 25600), (256, 5120, 8192),
                                   (64, 25600, 5120)])
def test_boundary_runs_the_planned_tail(torch, linear, M, N, K):
    """The boundary's MMQ call for M > 32 on more than P/8 tiles is the tail
    schedule with the plan's (dp_tiles, pieces); checked bit for bit against
    the kernel entry point with that plan, and on sampled rows against the
    oracle."""
    L = q3q4.load()
    assert L.sera_q4k_mmq_schedule(M, N, K) == 2
    dp, pieces = q3q4.mmq_tail_plan(M, N, K)
    T = L.sera_q4k_mmq_tiles(M, N)
    say(f"case boundary mmq tail M={M} N={N} K={K} tiles={T} plan dp_tiles={dp} pieces={pieces}")
    assert 0 <= dp <= T and 1 <= pieces <= K // 256
    gen = torch.Generator(device="cuda").manual_seed(M + N + K)
    wf = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    Wd = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
    q3q4.quantize_weights(wf, Wd)
    del wf
    rng = np.random.default_rng(N)
    X = rng.standard_normal((M, K)).astype(np.float32)
    y = nan_out(torch, M, N)
    linear(q3q4.bind_geometry(12, K, N), Wd, dev(torch, X), y)
    torch.cuda.synchronize()
    st = mmq_stage(torch, X)
    y2 = run_tail(torch, Wd, st, M, N, K, dp, pieces)
    assert torch.equal(y, y2), "boundary differs from the planned tail call"
    rows = np.sort(rng.choice(N, min(N, 256), replace=False))
    W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
    xq, xd, xs = oracle.q8_1_mmq(X)
    ref = oracle.gemm_mmq(W, xq, xd, xs, len(rows), K)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.cpu().numpy()[:, rows].astype(np.float64) - ref)))
    say(f"  max|err| / rms = {err / rms:.2e} on {len(rows)} rows")
    assert err <= 1e-3 * rms
