"""The fused linear group (sera_linear_group) through the C ABI.

Bars:
  * grouped products equal the path-faithful oracle within 1e-3 * rms(y);
  * SERA_LIN_ACCUMULATE is bit-identical to product-then-add in fp32, for
    every kernel variant (grouped MMVQ, few-token, split-K, stream-K, Q6_K
    MMVQ and tile kernel);
  * SERA_LIN_RMSNORM is bit-identical to the unfused group on the oracle's
    RMSNorm (same sum order, IEEE sqrt/div);
  * SERA_LIN_SILU_MUL is within 1e-3 * rms of the oracle (the device expf
    and numpy's float32 exp may differ in the last place).
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3


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


def weights(rng, qtype, N, K):
    if qtype == 12:
        return oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    return oracle.q6k_weights(rng, N, K)


def path_oracle(qtype, W, x, N, K):
    return oracle.linear_reference(W, x, N, K) if qtype == 12 else oracle.linear_reference_q6k(W, x, N, K)


def check_close(y, ref, what):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}")
    assert np.all(np.isfinite(y)), what
    assert err <= TOL * rms, what


def run_group(torch, qtype, Ws, Ns, K, x, flags=0, x2=None, gamma=None, eps=0.0, y0=None):
    M = x.shape[0]
    geos = [q3q4.bind_geometry(qtype, K, n) for n in Ns]
    Wd = [dev(torch, w) for w in Ws]
    ys = [dev(torch, y0[i]) if y0 is not None else torch.full((M, n), float("nan"), device="cuda")
          for i, n in enumerate(Ns)]
    q3q4.linear_group(geos, Wd, ys, dev(torch, x), None if x2 is None else dev(torch, x2),
                      None if gamma is None else dev(torch, gamma), eps, flags)
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys]


CASES = [(12, 1), (12, 4), (12, 6), (12, 9), (12, 64), (14, 1), (14, 3), (14, 6), (14, 40)]


@pytest.mark.parametrize("qtype,M", CASES)
def test_group_products_and_accumulate(torch, linear, qtype, M):
    K = 2048
    Ns = [1024, 256, 512] if qtype == 12 else [768, 256]
    rng = np.random.default_rng(qtype * 100 + M)
    Ws = [weights(rng, qtype, n, K) for n in Ns]
    x = rng.standard_normal((M, K)).astype(np.float32)
    say(f"case group qtype={qtype} M={M}")
    ys = run_group(torch, qtype, Ws, Ns, K, x)
    for i, n in enumerate(Ns):
        check_close(ys[i], path_oracle(qtype, Ws[i], x, n, K), f"group[{i}] N={n}")
    y0 = [rng.standard_normal((M, n)).astype(np.float32) for n in Ns]
    ya = run_group(torch, qtype, Ws, Ns, K, x, flags=q3q4.LIN_ACCUMULATE, y0=y0)
    for i in range(len(Ns)):
        assert np.array_equal(ya[i].view(np.uint32), (y0[i] + ys[i]).astype(np.float32).view(np.uint32)), i


@pytest.mark.parametrize("M,N,K,kind", [(9, 256, 2048, "split"), (64, 16384, 2048, "split"),
                                          (100, 4096, 5120, "split"), (20, 131328, 256, "streamk"),
                                          (20, 4096, 1024, "split"), (13, 1000, 2304, "split"),
                                          (16, 131328, 256, "fewtok"), (12, 1000, 16384, "fewtok")])
def test_accumulate_on_split_and_streamk_schedules(torch, linear, M, N, K, kind):
    """Q4_K MMQ path under split-K, stream-K (a full round or more of
    32-token tiles) and the few-token kernel
    it runs at 9-16 tokens on tall or long matrices: the accumulating store
    stays bit-identical to product + add."""
    L = q3q4.load()
    got = ("fewtok" if L.sera_q4k_mmq_uses_fewtok(M, N, K)
           else "streamk" if L.sera_q4k_mmq_schedule(M, N, K) == 1 else "split")
    say(f"case accumulate schedules M={M} N={N} K={K} kernel={got}")
    assert got == kind
    rng = np.random.default_rng(M + N)
    W = weights(rng, 12, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = run_group(torch, 12, [W], [N], K, x)[0]
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    ya = run_group(torch, 12, [W], [N], K, x, flags=q3q4.LIN_ACCUMULATE, y0=[y0])[0]
    assert np.array_equal(ya.view(np.uint32), (y0 + y).astype(np.float32).view(np.uint32))
    idx = np.random.default_rng(3).choice(N, 64, replace=False)
    check_close(y[:, idx], oracle.linear_reference(W[idx], x, 64, K), "sampled rows")


@pytest.mark.parametrize("M,N,K,tile", [(100, 1000, 2304, 32), (128, 2048, 8192, 64), (512, 16384, 2048, 64)])
def test_q6k_accumulate_on_both_token_tiles(torch, linear, M, N, K, tile):
    """Q6_K tile kernel on its 32- and 64-token tiles, split-K (the first
    two) and whole K (the last, 1024 tiles): the accumulating store stays
    bit-identical to product + add."""
    L = q3q4.load()
    say(f"case q6k accumulate M={M} N={N} K={K} tile={tile} splits={L.sera_q6k_mmq_splits_for(M, N, K)}")
    assert L.sera_q6k_mmq_tile_tokens(M, N, K) == tile
    rng = np.random.default_rng(M + N + K)
    W = weights(rng, 14, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = run_group(torch, 14, [W], [N], K, x)[0]
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    ya = run_group(torch, 14, [W], [N], K, x, flags=q3q4.LIN_ACCUMULATE, y0=[y0])[0]
    assert np.array_equal(ya.view(np.uint32), (y0 + y).astype(np.float32).view(np.uint32))
    idx = np.sort(np.random.default_rng(4).choice(N, 64, replace=False))
    check_close(y[:, idx], path_oracle(14, W[idx], x, 64, K), "sampled rows")


@pytest.mark.parametrize("qtype,M", [(12, 1), (12, 5), (12, 33), (14, 2), (14, 7), (14, 40)])
def test_rmsnorm_producer_is_bit_identical_to_unfused(torch, linear, qtype, M):
    K = 5120
    Ns = [512, 256]
    rng = np.random.default_rng(7 * M + qtype)
    Ws = [weights(rng, qtype, n, K) for n in Ns]
    h = (rng.standard_normal((M, K)) * 2.5).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, K).astype(np.float32)
    say(f"case rmsnorm producer qtype={qtype} M={M}")
    fused = run_group(torch, qtype, Ws, Ns, K, h, flags=q3q4.LIN_RMSNORM, gamma=gamma, eps=1e-6)
    xn = oracle.rmsnorm_fused_order(h, gamma, 1e-6)
    plain = run_group(torch, qtype, Ws, Ns, K, xn)
    for i in range(len(Ns)):
        assert np.array_equal(fused[i].view(np.uint32), plain[i].view(np.uint32)), i


def test_rmsnorm_producer_rows_in_decode_batches(torch, linear):
    """The RMSNorm producer on the row stage over 33 rows, in MMVQ-path
    batches of up to 8: bit-identical to the unfused path fed with the
    oracle's RMSNorm. Row 8 of this input is one whose block sums changed
    when the compiler fused the producer's last multiply into the quantizer's
    sum (the quantizer files are compiled without contraction)."""
    K = 5120
    Ns = [512, 256]
    M = 33
    rng = np.random.default_rng(7 * M + 12)
    h = (rng.standard_normal((M, K)) * 2.5).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, K).astype(np.float32)
    Ws = [weights(np.random.default_rng(99), 12, n, K) for n in Ns]
    xn = oracle.rmsnorm_fused_order(h, gamma, 1e-6)
    for r0 in range(0, M, 8):
        hb, xb = h[r0:r0 + 8], xn[r0:r0 + 8]
        say(f"case rmsnorm producer rows {r0}..{r0 + len(hb) - 1}")
        fused = run_group(torch, 12, Ws, Ns, K, hb, flags=q3q4.LIN_RMSNORM, gamma=gamma, eps=1e-6)
        plain = run_group(torch, 12, Ws, Ns, K, xb)
        for i in range(len(Ns)):
            assert np.array_equal(fused[i].view(np.uint32), plain[i].view(np.uint32)), (r0, i)


@pytest.mark.parametrize("qtype,M", [(12, 1), (12, 8), (12, 40), (14, 1), (14, 6), (14, 64)])
def test_silu_mul_producer_with_residual(torch, linear, qtype, M):
    """The down projection step: y += (silu(g) * u) . W^T."""
    K, N = 3072, 512
    rng = np.random.default_rng(11 * M + qtype)
    W = weights(rng, qtype, N, K)
    g = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    u = rng.standard_normal((M, K)).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    say(f"case silu producer qtype={qtype} M={M}")
    y = run_group(torch, qtype, [W], [N], K, g, flags=q3q4.LIN_SILU_MUL | q3q4.LIN_ACCUMULATE, x2=u, y0=[y0])[0]
    ref = path_oracle(qtype, W, oracle.silu_mul(g, u), N, K)
    check_close(y - y0, ref, "silu*up product")


@pytest.mark.parametrize("M,Ns", [(3, [16384, 1024]), (6, [4096, 1024, 256]), (8, [4096, 1024])])
def test_q4k_group_mixes_grouped_dot4_and_fewtok(torch, linear, M, Ns):
    """A Q4_K group at decode whose matrices split between the kernels: the
    ones dot4 takes share one grouped launch, the tall ones run the
    few-token kernel one by one (split K through the shared arena slots).
    Products against the MMVQ-formula oracle, accumulate bit-identical to
    product + add."""
    K = 4096
    L = q3q4.load()
    kinds = [bool(L.sera_q4k_vec_uses_fewtok(M, n, K)) for n in Ns]
    say(f"case mixed q4k group M={M} Ns={Ns} fewtok={kinds}")
    assert any(kinds) and not all(kinds), "case meant to mix the two kernels"
    assert all(q3q4.fewtok_splits(M, n, K) > 1 for n, f in zip(Ns, kinds) if f), "case meant to split K"
    rng = np.random.default_rng(500 + M)
    Ws = [weights(rng, 12, n, K) for n in Ns]
    x = rng.standard_normal((M, K)).astype(np.float32)
    ys = run_group(torch, 12, Ws, Ns, K, x)
    for i, n in enumerate(Ns):
        idx = np.sort(rng.choice(n, min(n, 256), replace=False))
        check_close(ys[i][:, idx], oracle.linear_reference(Ws[i][idx], x, len(idx), K), f"group[{i}] N={n}")
    y0 = [rng.standard_normal((M, n)).astype(np.float32) for n in Ns]
    ya = run_group(torch, 12, Ws, Ns, K, x, flags=q3q4.LIN_ACCUMULATE, y0=y0)
    for i in range(len(Ns)):
        assert np.array_equal(ya[i].view(np.uint32), (y0[i] + ys[i]).astype(np.float32).view(np.uint32)), i


@pytest.mark.parametrize("M", [6, 8])
def test_q6k_group_on_the_tile_branch(torch, linear, M):
    """A Q6_K group whose largest matrix has 4096+ rows at 6-8 tokens: the
    whole group runs the tile kernel on one row-formula stage. Products
    against the oracle and accumulate bit-identical to product + add; the
    RMSNorm producer bit-identical to the unfused group on the oracle's
    norm; the SiLU*up producer within tolerance of the oracle."""
    K = 2048
    Ns = [4096, 1024]
    L = q3q4.load()
    assert L.sera_q6k_vec_uses_tile(M, max(Ns), K)
    say(f"case q6k group tile branch M={M} Ns={Ns}")
    rng = np.random.default_rng(600 + M)
    Ws = [weights(rng, 14, n, K) for n in Ns]
    x = rng.standard_normal((M, K)).astype(np.float32)
    ys = run_group(torch, 14, Ws, Ns, K, x)
    for i, n in enumerate(Ns):
        idx = np.sort(rng.choice(n, 256, replace=False))
        check_close(ys[i][:, idx], oracle.linear_reference_q6k(np.ascontiguousarray(Ws[i][idx]), x, 256, K),
                    f"group[{i}] N={n}")
    y0 = [rng.standard_normal((M, n)).astype(np.float32) for n in Ns]
    ya = run_group(torch, 14, Ws, Ns, K, x, flags=q3q4.LIN_ACCUMULATE, y0=y0)
    for i in range(len(Ns)):
        assert np.array_equal(ya[i].view(np.uint32), (y0[i] + ys[i]).astype(np.float32).view(np.uint32)), i
    h = (rng.standard_normal((M, K)) * 2.5).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, K).astype(np.float32)
    fused = run_group(torch, 14, Ws, Ns, K, h, flags=q3q4.LIN_RMSNORM, gamma=gamma, eps=1e-6)
    plain = run_group(torch, 14, Ws, Ns, K, oracle.rmsnorm_fused_order(h, gamma, 1e-6))
    for i in range(len(Ns)):
        assert np.array_equal(fused[i].view(np.uint32), plain[i].view(np.uint32)), i
    g = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    u = rng.standard_normal((M, K)).astype(np.float32)
    ysil = run_group(torch, 14, Ws, Ns, K, g, flags=q3q4.LIN_SILU_MUL, x2=u)
    xs = oracle.silu_mul(g, u)
    for i, n in enumerate(Ns):
        idx = np.sort(rng.choice(n, 256, replace=False))
        check_close(ysil[i][:, idx], oracle.linear_reference_q6k(np.ascontiguousarray(Ws[i][idx]), xs, 256, K),
                    f"silu group[{i}] N={n}")
