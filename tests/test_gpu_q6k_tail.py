"""The Q6_K tile kernel under the tail schedule (whole tiles, then the
other tiles cut along K and handed off through counters), through the C ABI.

The schedule changes only which workgroup computes which (tile, K range)
and how a split tile's range sums are added; the per-sub-block exact
integers and the fp32 terms are the tile kernel's own (cuda/mmq/mmq.cuh:
2687-2786 for the arithmetic, :3641-4352 for the decomposition's role). So:

  * on exact inputs (every partial sum an exact fp32 value) the output
    equals the dequant GEMM bit for bit for any (dp_tiles, pieces): whole
    tiles only, everything split, one piece per super-block, whole tiles
    then a split rest; on the 32- and 64-token tiles, GGUF bytes and the
    split layout;
  * on random inputs it sits within 1e-3 * rms of the MMQ oracle, repeats
    bit for bit, leaves its counters at zero, and accumulate adds exactly
    the product;
  * the dense paths take it where sera_q6k_mmq_tail_plan says so, and are
    then bit-identical to the kernel entry point called with that plan.
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle
from test_gpu_q6k import _exact_inputs, check_close, dev, outlier_activations, q6k_weights_with_edges

pytestmark = pytest.mark.gpu
SPLIT = q3q4.QTYPE_Q6K_SPLIT


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


def to_split(torch, W, N, K):
    src = dev(torch, W)
    dst = torch.empty(q3q4.weight_bytes(SPLIT, N, K), dtype=torch.uint8, device="cuda")
    q3q4.weight_to_device_layout(SPLIT, N, K, src, dst)
    torch.cuda.synchronize()
    return dst


def stage_of(torch, x, M, K, row_formula=False):
    st = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    (q3q4.quantize_row_q6k if row_formula else q3q4.quantize_mmq_d4)(dev(torch, x), st)
    return st


def run_tail(torch, Wd, st, M, N, K, dp, pieces, qtype=14, y=None, accum=False):
    L = q3q4.load()
    T = L.sera_q6k_mmq_tiles(M, N, K)
    nslot = q3q4.q6k_mmq_tail_slot_floats(M, N, K, dp, pieces)
    slots = torch.empty(max(nslot, 1), dtype=torch.float32, device="cuda")
    counters = torch.zeros(max(T - dp, 1), dtype=torch.int32, device="cuda")
    if y is None:
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.q6k_mmq_tail(Wd, st, y, M, N, K, dp, pieces, slots=slots, counters=counters, accum=accum, qtype=qtype)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0, "tile counters not reset"
    return y


def tail_cases(M, N, K):
    """(dp_tiles, pieces): whole tiles only; everything in 2 and in K/256
    pieces; half the tiles whole and the rest in 3; all but one whole."""
    T = q3q4.load().sera_q6k_mmq_tiles(M, N, K)
    nkb = K // 256
    out = [(T, 1), (0, min(2, nkb)), (0, nkb), (T // 2, min(3, nkb)), (T - 1, nkb)]
    return sorted(set(out))


# (M, N, K): 32-token tiles (ragged M and N); 64-token tiles (the tile rule's
# 1024 (tile, super-block) pairs: 2 x 16 x 32)
EXACT = [(9, 200, 768), (40, 77, 2304), (100, 2046, 8192)]


@pytest.mark.parametrize("M,N,K", EXACT)
def test_q6k_tail_exact(torch, M, N, K):
    L = q3q4.load()
    rng = np.random.default_rng(M * 7 + N + K)
    W, x = _exact_inputs(rng, M, N, K)
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    st = stage_of(torch, x, M, K)
    tile = L.sera_q6k_mmq_tile_tokens(M, N, K)
    for qt, Wd in ((14, dev(torch, W)), (SPLIT, to_split(torch, W, N, K))):
        for dp, pieces in tail_cases(M, N, K):
            say(f"case exact q6k tail qtype={qt} M={M} N={N} K={K} tile={tile} dp_tiles={dp} pieces={pieces}")
            y = run_tail(torch, Wd, st, M, N, K, dp, pieces, qtype=qt)
            assert np.array_equal(y.cpu().numpy().astype(np.float64), ref), (qt, dp, pieces)


@pytest.mark.parametrize("M,N,K", [(8, 5120, 25600), (64, 640, 5120), (128, 2048, 8192)])
def test_q6k_tail_parity_repeat_accumulate(torch, M, N, K):
    """Random rows with edge blocks: within 1e-3 * rms of the oracle (the MMQ
    formula; the MMVQ formula's row stage at 8 tokens), bit-identical on a
    repeat and on the split layout, and accumulate == y + product."""
    rng = np.random.default_rng(M + N + K)
    W = q6k_weights_with_edges(rng, N, K)
    x = outlier_activations(rng, M, K)
    row = M <= 8
    st = stage_of(torch, x, M, K, row_formula=row)
    if row:
        ref = oracle.linear_reference_q6k(W, x, N, K)
    else:
        xq, d = oracle.q8_1_mmq_d4(x)
        ref = oracle.gemm_q6k(W, xq, d, N, K)
    Wg, Ws = dev(torch, W), to_split(torch, W, N, K)
    for dp, pieces in tail_cases(M, N, K):
        say(f"case q6k tail M={M} N={N} K={K} dp_tiles={dp} pieces={pieces}")
        y = run_tail(torch, Wg, st, M, N, K, dp, pieces)
        check_close(y.cpu().numpy(), ref, f"tail M={M} N={N} K={K} dp={dp} pieces={pieces}")
        y2 = run_tail(torch, Wg, st, M, N, K, dp, pieces)
        assert torch.equal(y, y2), "repeat differs"
        ys = run_tail(torch, Ws, st, M, N, K, dp, pieces, qtype=SPLIT)
        assert torch.equal(y, ys), "split layout differs"
        base = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
        acc = base.clone()
        run_tail(torch, Wg, st, M, N, K, dp, pieces, y=acc, accum=True)
        assert torch.equal(acc, base + y), "accumulate is not y + product"


def test_q6k_tail_plan_rule(torch, linear):
    """The dense paths take the tail when one round of resident workgroups
    (2 per CU) gives every tile at least 4 K pieces of at least 5
    super-blocks; split-K otherwise."""
    P = 2 * torch.cuda.get_device_properties(0).multi_processor_count
    L = q3q4.load()
    for M, N, K in [(8, 5120, 25600), (64, 5120, 25600), (128, 5120, 25600), (512, 5120, 25600),
                    (2048, 5120, 25600), (8, 8192, 5120), (512, 1024, 5120), (512, 151936, 5120)]:
        T = L.sera_q6k_mmq_tiles(M, N, K)
        p = P // T
        plan = q3q4.q6k_mmq_tail_plan(M, N, K)
        want = p >= 4 and K // 256 >= 5 * p
        say(f"case q6k tail plan M={M} N={N} K={K} tiles={T} plan={plan}")
        assert (plan is not None) == want, (M, N, K, T, plan)
        if plan:
            assert plan == (0, min(p, 63))


@pytest.mark.parametrize("M,N,K", [(8, 5120, 25600), (64, 5120, 25600)])
def test_dense_paths_run_the_planned_tail(torch, linear, M, N, K):
    """q3_cuda_q4k_linear with a Q6_K geometry (the tile kernel at 8 tokens on
    the MMVQ path, the MMQ path at 64) on a shape the plan cuts into pieces:
    bit-identical to the kernel entry point with that plan, on both
    layouts, and the stats' launch count is 2 (no reduce)."""
    L = q3q4.load()
    plan = q3q4.q6k_mmq_tail_plan(M, N, K)
    assert plan is not None
    say(f"case dense q6k tail M={M} N={N} K={K} plan={plan}")
    rng = np.random.default_rng(N + M)
    W = oracle.q6k_weights(rng, N, K)
    x = outlier_activations(rng, M, K)
    st = stage_of(torch, x, M, K, row_formula=M <= 8)
    for qt, Wd in ((14, dev(torch, W)), (SPLIT, to_split(torch, W, N, K))):
        if M <= 8:
            assert L.sera_q6k_vec_uses_tile_qt(qt, M, N, K)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        stt = linear(q3q4.bind_geometry(qt, K, N), Wd, dev(torch, x), y)
        torch.cuda.synchronize()
        assert stt.kernel_launches == 2 == L.sera_q6k_kernel_launches_qt(qt, M, N, K)
        y2 = run_tail(torch, Wd, st, M, N, K, plan[0], plan[1], qtype=qt)
        assert torch.equal(y, y2), f"qtype {qt}: the dense path differs from the planned tail call"
