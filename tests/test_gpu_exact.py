"""Bit-exact integer dots inside the production Q4_K kernels.

The reference computes each per-32 dot I_b = sum q4 * q8 exactly (dp4a,
cuda/mmq/vecdotq.cuh:516-520; the int32 MMA result C.x[l],
cuda/mmq/mmq.cuh:1470). These tests feed every production Q4_K kernel
inputs on which all arithmetic after the integer dot is exact:

  * weights with d = 2^-8 and dmin = 2^-9, so d*sc and dmin*m are exact in
    fp16 and fp32 for every 6-bit sc and m (the fp16 products of the MMQ
    scale store equal the exact ones);
  * activations x = q * 2^-5 with q = +127 and -127 at positions 0 and 1 of
    every 32-block, so both quantizers give d8 = 2^-5 exactly and q8 = q;
    the weight nibbles at those two positions are equal, so the pair adds
    nothing to I_b and the sums stay small;
  * every term d*sc*d8*I_b and dmin*m*d8*S_b (or fp16 sum s8) is then a
    multiple of 2^-14, and the test asserts on the CPU that the sum of their
    magnitudes is below 2^10 for every output: every partial sum in any
    order is an integer multiple of 2^-14 below 2^24 units, so fp32 holds
    it exactly.

Then the output of any correct kernel equals the plain dequant GEMM
(oracle.gemm_dequant) bit for bit, whatever its summation order; a wrong
integer dot (a dropped or doubled term, a wrong nibble plane or sub-block,
a wrong scale or min field) changes it by at least 2^-14. Covered: the
dot4 MMVQ kernel at every rows-per-tile choice and the 8-wave plan of long
K, the few-token kernel (both formulas, split K), the MMQ paired 16-token,
32-token and 64-token tiles under plain, split-K and stream-K schedules,
and the q3_cuda_q4k_linear boundary on every kernel it dispatches to.
"""
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
    return q3q4.Linear(device=0, max_tokens=512, max_features=25600, max_k=25600)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def exact_inputs(rng, M, N, K, qmax=2):
    """Q4_K bytes and fp32 activations of the exact construction above."""
    W = np.zeros((N, K // 256, 144), np.uint8)
    W[:, :, 0:2] = np.frombuffer(np.float16(2.0 ** -8).tobytes(), np.uint8)
    W[:, :, 2:4] = np.frombuffer(np.float16(2.0 ** -9).tobytes(), np.uint8)
    W[:, :, 4:16] = rng.integers(0, 256, (N, K // 256, 12))      # every 6-bit sc / m field
    qs = rng.integers(0, 256, (N, K // 256, 128)).astype(np.uint8)
    for j2 in range(4):                        # positions 0 and 1 of sub-blocks 2*j2, 2*j2+1
        qs[:, :, 32 * j2 + 1] = qs[:, :, 32 * j2]
    W[:, :, 16:] = qs
    q = rng.integers(-qmax, qmax + 1, (M, K // 32, 32))
    q[:, :, 0] = 127
    q[:, :, 1] = -127
    X = (q.reshape(M, K) * 2.0 ** -5).astype(np.float32)
    return W.reshape(N, -1), X


def expected(W, X, N, K):
    """gemm_dequant, after checking the exactness precondition and that both
    path formulas agree with it on these inputs."""
    M = X.shape[0]
    xq, xd, _ = oracle.q8_1_row(X)
    assert np.all(xd == np.float16(2.0 ** -5).view(np.uint16))
    assert np.array_equal(xq.astype(np.float64), X.astype(np.float64) * 32.0)
    I = oracle.subblock_dots(W, xq, N, K).astype(np.float64)            # [M, N, K/32]
    S = oracle.q8_sums(xq).astype(np.float64)                          # [M, K/32]
    bound = (63 * np.abs(I).sum(axis=2) * 2.0 ** -13
             + 63 * np.abs(S).sum(axis=1)[:, None] * 2.0 ** -14)
    assert float(bound.max()) < 2.0 ** 10, f"exactness bound {bound.max()}"
    ref = oracle.gemm_dequant(W, X, N, K)
    assert np.array_equal(oracle.gemm_mmvq(W, xq, xd, N, K), ref)
    mq, md, ms = oracle.q8_1_mmq(X)
    assert np.array_equal(oracle.gemm_mmq(W, mq, md, ms, N, K), ref)
    assert ref.shape == (M, N)
    return ref


def assert_bits(y, ref, what):
    got = y.cpu().numpy().astype(np.float64)
    bad = int(np.count_nonzero(got != ref))
    say(f"  {what}: {bad} of {ref.size} outputs differ")
    assert bad == 0, what


def row_stage(torch, X):
    M, K = X.shape
    st = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(dev(torch, X), st)
    return st


def mmq_stage(torch, X):
    M, K = X.shape
    st = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(dev(torch, X), st)
    return st


def nan_out(torch, M, N):
    return torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")


# ---------------------------------------------------------------------------
# dot4 MMVQ kernel
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(300, 5120), (203, 2304), (64, 25600), (1, 256)])
def test_mmvq_dot4_exact(torch, N, K):
    """Every rows-per-tile choice (and the built-in plan, 8 waves per
    workgroup at one token and K = 25600) at 1-8 tokens."""
    rng = np.random.default_rng(N * 7 + K)
    W, X8 = exact_inputs(rng, 8, N, K)
    Wd = dev(torch, W)
    for M in range(1, 9):
        X = X8[:M]
        ref = expected(W, X, N, K)
        st = row_stage(torch, X)
        for rows in (0, 2, 4, 8, 16):
            say(f"case exact mmvq M={M} N={N} K={K} rows={rows}")
            y = nan_out(torch, M, N)
            q3q4.mmvq(Wd, st, y, M, N, K, rows_per_tile=rows)
            torch.cuda.synchronize()
            assert_bits(y, ref, f"mmvq M={M} N={N} K={K} rows={rows}")


# ---------------------------------------------------------------------------
# few-token MFMA kernel
# ---------------------------------------------------------------------------

def run_fewtok(torch, Wd, stage, M, N, K, chunk, form):
    s = q3q4.fewtok_splits(M, N, K, chunk)
    slots = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
    counters = (torch.zeros(q3q4.fewtok_groups(M, N, K), dtype=torch.int32, device="cuda")
                if s > 1 else None)
    y = nan_out(torch, M, N)
    q3q4.fewtok(Wd, stage, y, M, N, K, chunk=chunk, slots=slots, counters=counters, form=form)
    torch.cuda.synchronize()
    if counters is not None:
        assert int(counters.abs().sum()) == 0
    return y, s


@pytest.mark.parametrize("N,K", [(1000, 512), (300, 5120), (64, 25600), (16500, 1024)])
def test_fewtok_exact(torch, N, K):
    """Form 0 (row stage, MMVQ formula) at 1-8 tokens and form 1 (MMQ stage,
    MMQ formula) at 1-16 tokens, with K chunkings that split K inside the
    launch (the last split of a row group sums the partials)."""
    rng = np.random.default_rng(N * 3 + K)
    W, X16 = exact_inputs(rng, 16, N, K)
    Wd = dev(torch, W)
    nkb = K // 256
    for M in range(1, 17):
        X = X16[:M]
        ref = expected(W, X, N, K)
        forms = (0, 1) if M <= 8 else (1,)
        for form in forms:
            st = row_stage(torch, X) if form == 0 else mmq_stage(torch, X)
            for chunk in sorted({0, 1, 3, min(20 if M <= 8 else 10, nkb)}):
                if chunk > nkb:
                    continue
                y, s = run_fewtok(torch, Wd, st, M, N, K, chunk, form)
                assert_bits(y, ref, f"fewtok form={form} M={M} N={N} K={K} chunk={chunk} splits={s}")


# ---------------------------------------------------------------------------
# MMQ tiles and schedules
# ---------------------------------------------------------------------------

# M <= 16: paired 16-token tile; 17-32: 32-token tile; above: 64-token
# tile, of 128 weight rows up to 64 tiles of 256 rows (the shapes up to
# (64, 64, 25600)) and of 256 rows past that (the last two)
MMQ_EXACT = [(1, 700, 5120), (7, 300, 2304), (16, 512, 5120), (20, 300, 2304), (32, 640, 1024),
             (33, 384, 5120), (100, 256, 2048), (200, 640, 1024), (64, 64, 25600), (64, 16640, 512),
             (130, 8448, 256)]


@pytest.mark.parametrize("M,N,K", MMQ_EXACT)
def test_mmq_exact_plain_and_splitk(torch, M, N, K):
    rng = np.random.default_rng(M * 5 + N + K)
    W, X = exact_inputs(rng, M, N, K)
    ref = expected(W, X, N, K)
    Wd = dev(torch, W)
    st = mmq_stage(torch, X)
    nkb = K // 256
    for s in sorted({1, 2, min(4, nkb)}):
        if s > nkb or (s > 1 and (M * N) % 4):
            continue
        say(f"case exact mmq M={M} N={N} K={K} splits={s}")
        y = nan_out(torch, M, N)
        partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        q3q4.mmq(Wd, st, y, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        assert_bits(y, ref, f"mmq M={M} N={N} K={K} splits={s}")


@pytest.mark.parametrize("M,N,K,wgs", [(1, 700, 5120, 8), (16, 512, 5120, 24), (20, 300, 2304, 8),
                                       (32, 640, 1024, 8), (100, 256, 2048, 8), (200, 640, 1024, 40)])
def test_mmq_exact_streamk(torch, M, N, K, wgs):
    rng = np.random.default_rng(M * 11 + N + K + wgs)
    W, X = exact_inputs(rng, M, N, K)
    ref = expected(W, X, N, K)
    Wd = dev(torch, W)
    st = mmq_stage(torch, X)
    L = q3q4.load()
    assert L.sera_q4k_mmq_tiles(M, N) * (K // 256) >= wgs
    slots = torch.empty(2 * wgs * L.sera_q4k_mmq_slot_floats(M), dtype=torch.float32, device="cuda")
    counters = torch.zeros(L.sera_q4k_mmq_tiles(M, N), dtype=torch.int32, device="cuda")
    say(f"case exact mmq stream-K M={M} N={N} K={K} wgs={wgs}")
    y = nan_out(torch, M, N)
    q3q4.mmq_streamk(Wd, st, y, M, N, K, slots, counters, wgs=wgs)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    assert_bits(y, ref, f"mmq stream-K M={M} N={N} K={K} wgs={wgs}")


# ---------------------------------------------------------------------------
# the boundary, on each kernel it dispatches to
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 25600, 512), (4, 25600, 512), (8, 4096, 1024), (5, 2048, 1024),
                                   (9, 2048, 1024), (16, 2048, 1024), (40, 1024, 1024)])
def test_linear_boundary_exact(torch, linear, M, N, K):
    """q3_cuda_q4k_linear: dot4 MMVQ, the few-token kernel (tall and
    4096-row matrices), the MMQ-path few-token kernel (9 tokens), the paired
    tile and the 64-token tile, each bit-exact on exact inputs; and the same
    on the tiled layout, with its own few-token rule."""
    L = q3q4.load()
    rng = np.random.default_rng(M * 17 + N + K)
    W, X = exact_inputs(rng, M, N, K)
    ref = expected(W, X, N, K)
    kern = ("fewtok" if L.sera_q4k_vec_uses_fewtok(M, N, K) else "dot4") if M <= 8 else "mmq-path"
    say(f"case exact linear M={M} N={N} K={K} ({kern})")
    y = nan_out(torch, M, N)
    linear(q3q4.bind_geometry(12, K, N), dev(torch, W), dev(torch, X), y)
    torch.cuda.synchronize()
    assert_bits(y, ref, f"linear M={M} N={N} K={K} ({kern})")
    # the same bytes in the tiled layout (its own kernel choice at M <= 8)
    T = q3q4.QTYPE_Q4K_TILED
    kern_t = ("fewtok" if L.sera_q4k_vec_uses_fewtok_qt(T, M, N, K) else "dot4") if M <= 8 else "mmq-path"
    say(f"case exact linear tiled M={M} N={N} K={K} ({kern_t})")
    y = nan_out(torch, M, N)
    linear(q3q4.bind_geometry(T, K, N), dev(torch, q3q4.q4k_tiled_bytes(W, N, K)), dev(torch, X), y)
    torch.cuda.synchronize()
    assert_bits(y, ref, f"linear tiled M={M} N={N} K={K} ({kern_t})")
