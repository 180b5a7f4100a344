"""The few-token kernel (q4k_fewtok.hip) through the C ABI.

Bars: fp32 outputs within max |y - y_oracle| <= 1e-3 * rms(y_oracle) of the
path-faithful oracle: the MMVQ formula (vecdotq.cuh:505-527) on a row stage
for 1-8 tokens, the MMQ formula (mmq.cuh:2269-2283,1440-1472) on an MMQ
stage for 1-16 tokens. The kernel sums the same fp32 terms as the oracle in
another order, so it also sits within 2e-5 * rms, far inside the gap between
the two formulas (the fp16 rounding of d*sc alone moves y by ~1e-4 * rms):
that pins which formula runs. Split-K results repeat bit for bit and leave
the row-group counters at zero; accumulate adds exactly the product; the
persistent grid (more tiles than resident workgroups) matches the oracle and
repeats; the boundary (q3_cuda_q4k_linear) runs this kernel where
sera_q4k_vec_uses_fewtok says so (2-8 tokens) and at 9 tokens.
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3
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
    return q3q4.Linear(device=0, max_tokens=2048, max_features=151936, max_k=25600)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def outlier_activations(rng, M, K, frac=0.01, gain=20.0):
    x = rng.standard_normal((M, K)).astype(np.float32)
    ch = rng.choice(K, max(1, int(np.ceil(frac * K))), replace=False)
    x[:, ch] *= gain
    return x


def rand_weights(rng, N, K, scale=0.02):
    return oracle.quantize_q4k((rng.standard_normal((N, K)) * scale).astype(np.float32))


def check_close(y, ref, what, tol=TOL):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}, ratio = {err / max(rms, 1e-30):.2e}")
    assert np.all(np.isfinite(y)), what
    assert err <= tol * rms, what


def run_fewtok(torch, Wd, stage, M, N, K, chunk, y=None, accum=False, form=0):
    s = q3q4.fewtok_splits(M, N, K, chunk)
    slots = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
    counters = (torch.zeros(q3q4.fewtok_groups(M, N, K), dtype=torch.int32, device="cuda")
                if s > 1 else None)
    if y is None:
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.fewtok(Wd, stage, y, M, N, K, chunk=chunk, slots=slots, counters=counters, accum=accum, form=form)
    torch.cuda.synchronize()
    if counters is not None:
        assert int(counters.abs().sum()) == 0, "row-group counters not reset"
    return y, s


# (N, K): ragged N (not a multiple of 64 or 128 rows), one super-block, K
# below and above the 20-super-block chunk limit, the wide-N plan (8 waves)
# (64, 25600) and (100, 25600): 8-wave workgroups with staged weights whose
# last waves own no rows (and, at 100, a ragged last tile); they read the last
# tile's rows and store nothing
FEWTOK_SHAPES = [(16, 256), (1000, 512), (300, 5120), (64, 25600), (100, 25600), (203, 2304), (16500, 1024)]


@pytest.mark.parametrize("N,K", FEWTOK_SHAPES)
def test_fewtok_parity(torch, N, K):
    """Every batch 1..8 and several K chunkings against the MMVQ-formula oracle."""
    rng = np.random.default_rng(11 * N + K)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    nkb = K // 256
    for M in range(1, 9):
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(dev(torch, x), stage)
        xq, xd, _ = oracle.q8_1_row(x)
        ref = oracle.gemm_mmvq(W, xq, xd, N, K)
        for chunk in sorted({0, 1, 3, 7, min(20, nkb), min(40, nkb)}):
            if chunk > nkb:
                continue
            say(f"case fewtok M={M} N={N} K={K} chunk={chunk} "
                f"splits={q3q4.fewtok_splits(M, N, K, chunk)}")
            y, _ = run_fewtok(torch, Wd, stage, M, N, K, chunk)
            check_close(y.cpu().numpy(), ref, f"fewtok M={M} N={N} K={K} chunk={chunk}", TIGHT)


@pytest.mark.parametrize("N,K", FEWTOK_SHAPES)
def test_fewtok_mmq_formula_parity(torch, N, K):
    """form 1 (MMQ stage) for 1-16 tokens against the MMQ-formula oracle."""
    rng = np.random.default_rng(13 * N + K)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    nkb = K // 256
    for M in (1, 4, 8, 9, 13, 16):
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_mmq(dev(torch, x), stage)
        xq, xd, xs = oracle.q8_1_mmq(x)
        ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
        for chunk in sorted({0, 1, 3, min(10, nkb), min(20 if M > 8 else 40, nkb)}):
            if chunk > nkb:
                continue
            say(f"case fewtok form=1 M={M} N={N} K={K} chunk={chunk} "
                f"splits={q3q4.fewtok_splits(M, N, K, chunk)}")
            y, _ = run_fewtok(torch, Wd, stage, M, N, K, chunk, form=1)
            check_close(y.cpu().numpy(), ref, f"fewtok form 1 M={M} N={N} K={K} chunk={chunk}", TIGHT)


def test_fewtok_split_repeats_and_accumulates(torch):
    """Split-K sums in split order: two runs agree bit for bit; accumulate
    adds exactly the product to what Y held."""
    rng = np.random.default_rng(5)
    M, N, K = 8, 1000, 5120
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    x = outlier_activations(rng, M, K)
    stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(dev(torch, x), stage)
    for chunk in (3, 0):
        say(f"case fewtok repeat M={M} N={N} K={K} chunk={chunk}")
        a, s = run_fewtok(torch, Wd, stage, M, N, K, chunk)
        b, _ = run_fewtok(torch, Wd, stage, M, N, K, chunk)
        assert s > 1 or chunk == 0
        assert torch.equal(a, b)
        base = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
        acc = base.clone()
        run_fewtok(torch, Wd, stage, M, N, K, chunk, y=acc, accum=True)
        assert torch.equal(acc, base + a), "accumulate is not y + product"


# (N, K): more 16-row tiles than the device's resident workgroups take in
# one pass, so the launch is persistent when the K chunk is one even split
# (ragged N; 2 and 10 super-blocks); the odd 3-super-block K keeps one tile
# per wave
# chunks of 2 and 10 super-blocks (one super-block in flight per wave), 4 and
# 12 (two to four in flight), and an odd count (no persistent grid)
PERSIST_SHAPES = [(70001, 512), (40000, 2560), (40000, 1024), (40000, 3072), (70001, 768)]


@pytest.mark.parametrize("N,K", PERSIST_SHAPES)
def test_fewtok_persistent_grid(torch, N, K):
    """Workgroups that stage the activations once and walk a range of tiles
    (results held in LDS, written out at the end): both formulas against the
    oracle, repeats bit for bit, accumulate adds exactly the product."""
    rng = np.random.default_rng(17 * N + K)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    nkb = K // 256
    ran_persistent = False
    for form, M in ((0, 4), (0, 8), (1, 4), (1, 9), (1, 16)):
        x = outlier_activations(rng, M, K)
        if form == 0:
            stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
            q3q4.quantize_row(dev(torch, x), stage)
            xq, xd, _ = oracle.q8_1_row(x)
            ref = oracle.gemm_mmvq(W, xq, xd, N, K)
        else:
            stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
            q3q4.quantize_mmq(dev(torch, x), stage)
            xq, xd, xs = oracle.q8_1_mmq(x)
            ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
        grid, groups = q3q4.fewtok_grid(form, M, N, K), q3q4.fewtok_groups(M, N, K)
        persistent = q3q4.fewtok_splits(M, N, K) == 1 and grid < groups
        ran_persistent |= persistent
        assert persistent or nkb % 2 or q3q4.fewtok_splits(M, N, K) > 1 or grid == groups
        say(f"case fewtok persistent={persistent} form={form} M={M} N={N} K={K} grid={grid} groups={groups}")
        y, _ = run_fewtok(torch, Wd, stage, M, N, K, 0, form=form)
        check_close(y.cpu().numpy(), ref, f"fewtok form {form} M={M} N={N} K={K}", TIGHT)
        b, _ = run_fewtok(torch, Wd, stage, M, N, K, 0, form=form)
        assert torch.equal(y, b), "repeat differs"
        base = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
        acc = base.clone()
        run_fewtok(torch, Wd, stage, M, N, K, 0, y=acc, accum=True, form=form)
        assert torch.equal(acc, base + y), "accumulate is not y + product"
    assert ran_persistent == (nkb % 2 == 0), "the persistent grid was not exercised"


def test_fewtok_persistent_grid_beyond_the_lds_of_one_range(torch, linear):
    """A head tall enough that one resident workgroup per CU cannot hold its
    range's results in LDS (262144 rows at 16 tokens: 256 ranges of 64
    tiles would need 175,632 bytes): the launcher takes more, shorter ranges
    instead of failing, and the outputs match the oracle on sampled rows,
    through the kernel entry point and the boundary."""
    N, K, M = 262144, 5120, 16
    L = q3q4.load()
    grid, groups = q3q4.fewtok_grid(1, M, N, K), q3q4.fewtok_groups(M, N, K)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    say(f"case fewtok LDS-capped persistent grid M={M} N={N} K={K} grid={grid} groups={groups} cus={cus}")
    assert q3q4.fewtok_splits(M, N, K) == 1
    assert cus < grid < groups, "the ranges should be shortened to fit LDS, not left at one per CU"
    gen = torch.Generator(device="cuda").manual_seed(262144)
    wf = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    Wd = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
    q3q4.quantize_weights(wf, Wd)
    del wf
    rng = np.random.default_rng(5)
    x = outlier_activations(rng, M, K)
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(dev(torch, x), stage)
    y, _ = run_fewtok(torch, Wd, stage, M, N, K, 0, form=1)
    yb = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    linear(q3q4.bind_geometry(12, K, N), Wd, dev(torch, x), yb)
    torch.cuda.synchronize()
    assert torch.equal(y, yb), "the boundary's result differs from the kernel entry point's"
    rows = np.unique(np.concatenate([np.arange(256), np.arange(N - 256, N),
                                     rng.choice(N, 512, replace=False)]))
    W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
    xq, xd, xs = oracle.q8_1_mmq(x)
    ref = oracle.gemm_mmq(W, xq, xd, xs, len(rows), K)
    check_close(y.cpu().numpy()[:, rows], ref, f"LDS-capped persistent grid ({len(rows)} rows)", TIGHT)
    del Wd


def test_fewtok_matches_dot4_mmvq(torch):
    """The two MMVQ-path kernels agree within the tolerance at every batch
    they share (1-8 tokens) on a Qwen3-32B-width matrix."""
    rng = np.random.default_rng(9)
    N, K = 2048, 5120
    Wd = dev(torch, rand_weights(rng, N, K))
    for M in range(1, 9):
        x = dev(torch, outlier_activations(rng, M, K))
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(x, stage)
        say(f"case fewtok vs mmvq M={M} N={N} K={K}")
        y_mmvq = torch.empty((M, N), dtype=torch.float32, device="cuda")
        q3q4.mmvq(Wd, stage, y_mmvq, M, N, K)
        y, _ = run_fewtok(torch, Wd, stage, M, N, K, 0)
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), y_mmvq.cpu().numpy().astype(np.float64), f"fewtok vs mmvq M={M}")


@pytest.mark.parametrize("N,K", [(25600, 5120), (5120, 25600), (1024, 5120)])
def test_boundary_vec_dispatch(torch, linear, N, K):
    """q3_cuda_q4k_linear at 2-8 tokens gives, bit for bit, the result of the
    kernel sera_q4k_vec_uses_fewtok names: the few-token kernel (its planned
    chunk) or the dot4 MMVQ kernel."""
    rng = np.random.default_rng(21 + N)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    geo = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
    L = q3q4.load()
    for M in (2, 3, 4, 5, 8):
        x = dev(torch, outlier_activations(rng, M, K))
        few = L.sera_q4k_vec_uses_fewtok(M, N, K)
        say(f"case boundary vec M={M} N={N} K={K} fewtok={few}")
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        linear(geo, Wd, x, y)
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(x, stage)
        if few:
            ref, _ = run_fewtok(torch, Wd, stage, M, N, K, 0)
        else:
            ref = torch.empty((M, N), dtype=torch.float32, device="cuda")
            q3q4.mmvq(Wd, stage, ref, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(y, ref)


@pytest.mark.parametrize("N,K", [(1000, 25600), (1000, 2048)])
def test_boundary_mmq_path_at_nine_to_sixteen_tokens(torch, linear, N, K):
    """q3_cuda_q4k_linear at 9-16 tokens gives, bit for bit, the kernel that
    sera_q4k_mmq_uses_fewtok names: the few-token kernel's MMQ-formula result
    on a K >= 16384 matrix, the paired MMQ tile's on a small one; both stay
    within the tolerance of the MMQ oracle."""
    rng = np.random.default_rng(23 + K)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    geo = q3q4.bind_geometry(q3q4.QTYPE_Q4_K, K, N)
    L = q3q4.load()
    for M in (9, 10, 16):
        few = L.sera_q4k_mmq_uses_fewtok(M, N, K)
        assert few == (K >= 16384)
        xh = outlier_activations(rng, M, K)
        x = dev(torch, xh)
        say(f"case boundary MMQ formula M={M} N={N} K={K} fewtok={few}")
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        linear(geo, Wd, x, y)
        stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_mmq(x, stage)
        if few:
            ref, _ = run_fewtok(torch, Wd, stage, M, N, K, 0, form=1)
        else:
            s = q3q4.mmq_splits(M, N, K)
            ref = torch.empty((M, N), dtype=torch.float32, device="cuda")
            partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
            q3q4.mmq(Wd, stage, ref, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        assert torch.equal(y, ref)
        xq, xd, xs = oracle.q8_1_mmq(xh)
        check_close(y.cpu().numpy(), oracle.gemm_mmq(W, xq, xd, xs, N, K), f"boundary M={M}", TIGHT)
