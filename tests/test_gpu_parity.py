"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bars (from the path's contract):
  * Q8_1 blocks (quants, fp16 scale, fp16 sum), per-32 int32 dots, device
    dequant and the weight quantizer: bit-exact.
  * fp32 outputs: max |y - y_oracle| <= 1e-3 * rms(y_oracle), against the
    path-faithful oracle (MMVQ formula for M <= 8, MMQ formula above).
  * the reference test's own gates against the plain dequant oracle:
    cos > 0.999 and relL2 < 1% (tests/test_q3_q4_linear.cu:374,379), and a
    bit-exact repeat (:382-396).
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


def outlier_activations(rng, M, K, frac=0.01, gain=20.0):
    x = rng.standard_normal((M, K)).astype(np.float32)
    ch = rng.choice(K, max(1, int(np.ceil(frac * K))), replace=False)
    x[:, ch] *= gain
    return x


def rand_weights(rng, N, K, scale=0.02):
    return oracle.quantize_q4k((rng.standard_normal((N, K)) * scale).astype(np.float32))


def decode_row_stage(stage, M, K):
    lay = q3q4.row_stage_layout(M, K)
    b = stage.cpu().numpy()
    qs = b[lay["qs"]:lay["qs"] + M * K].view(np.int8).reshape(M, K)
    ds = b[lay["ds"]:lay["ds"] + M * K // 32 * 4].view(np.uint32).reshape(M, K // 32)
    dsf = b[lay["dsf"]:lay["dsf"] + M * K // 64 * 16].view(np.float32).reshape(M, K // 64, 4)
    return qs, (ds & 0xFFFF).astype(np.uint16), (ds >> 16).astype(np.uint16), dsf


def decode_mmq_stage(stage, M, K):
    lay = q3q4.mmq_stage_layout(M, K)
    R = lay["rows"]
    b = stage.cpu().numpy()
    qs = b[lay["qs"]:lay["qs"] + R * K].view(np.int8).reshape(R, K)
    ds = b[lay["ds"]:lay["ds"] + R * K // 32 * 4].view(np.uint32).reshape(R, K // 32)
    return qs, (ds & 0xFFFF).astype(np.uint16), (ds >> 16).astype(np.uint16)


def check_close(y, ref, what, tol=TOL):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}, ratio = {err / max(rms, 1e-30):.2e}")
    assert np.all(np.isfinite(y)), what
    assert err <= tol * rms, what


# ---------------------------------------------------------------------------
# Q8_1 quantizers: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(1, 256), (3, 5120), (8, 25600)])
def test_q8_row_bit_exact(torch, M, K):
    say(f"case q8_row M={M} K={K}")
    rng = np.random.default_rng(M * 1000 + K)
    x = outlier_activations(rng, M, K)
    x[0, 32:64] = 0.0                         # an all-zero block
    stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(dev(torch, x), stage)
    torch.cuda.synchronize()
    qs, d, s, dsf = decode_row_stage(stage, M, K)
    eq, ed, es = oracle.q8_1_row(x)
    assert np.array_equal(qs, eq)
    assert np.array_equal(d, ed)
    assert np.array_equal(s, es)
    d8 = oracle.h2f(ed).reshape(M, K // 64, 2)
    S = oracle.q8_sums(eq).reshape(M, K // 64, 2).astype(np.float32)
    assert np.array_equal(dsf[..., 0:2], d8)
    assert np.array_equal(dsf[..., 2:4], (d8 * S).astype(np.float32))


@pytest.mark.parametrize("M,K", [(9, 256), (33, 5120), (100, 1024), (512, 5120)])
def test_q8_mmq_bit_exact(torch, M, K):
    say(f"case q8_mmq M={M} K={K}")
    rng = np.random.default_rng(M * 7 + K)
    x = outlier_activations(rng, M, K)
    x[-1, :32] = -0.0
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    stage.fill_(0x5A)                          # poison: padding rows must be rewritten
    q3q4.quantize_mmq(dev(torch, x), stage)
    torch.cuda.synchronize()
    qs, d, s = decode_mmq_stage(stage, M, K)
    eq, ed, es = oracle.q8_1_mmq(x)
    assert np.array_equal(qs[:M], eq)
    assert np.array_equal(d[:M], ed)
    assert np.array_equal(s[:M], es)
    assert not qs[M:].any() and not d[M:].any() and not s[M:].any()


def test_q8_hand_cases_on_device(torch):
    """Same known answers as the oracle checks: sum trees 30 (row) and 27
    (DS4), roundf half away from zero."""
    say("case q8 hand cases")
    x = np.ones((1, 256), np.float32)
    x[0, 0], x[0, 16] = 2.0 ** 24, -(2.0 ** 24)
    x[0, 32:64] = 0.0
    x[0, 32:38] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]
    xs = dev(torch, x)
    st_r = torch.empty(q3q4.row_stage_layout(1, 256)["total"], dtype=torch.uint8, device="cuda")
    st_m = torch.empty(q3q4.mmq_stage_layout(1, 256)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(xs, st_r)
    q3q4.quantize_mmq(xs, st_m)
    torch.cuda.synchronize()
    qr, _, sr, _ = decode_row_stage(st_r, 1, 256)
    qm, _, sm = decode_mmq_stage(st_m, 1, 256)
    assert sr[0, 0] == np.float16(30.0).view(np.uint16)
    assert sm[0, 0] == np.float16(27.0).view(np.uint16)
    assert list(qr[0, 32:38]) == [127, 3, -3, 1, -1, 2]
    assert list(qm[0, 32:38]) == [127, 3, -3, 1, -1, 2]


# ---------------------------------------------------------------------------
# Integer dots, dequant, weight quantizer: bit-exact
# ---------------------------------------------------------------------------

def test_subblock_dots_bit_exact(torch):
    say("case subblock dots")
    rng = np.random.default_rng(5)
    M, N, K = 4, 48, 1024
    W = rand_weights(rng, N, K)
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    xq[0, :] = 127
    W[0, 16:144] = 0xFF                        # extreme row: |I| = 60960
    out = torch.empty((M, N, K // 32), dtype=torch.int32, device="cuda")
    q3q4.subblock_dots(dev(torch, W), dev(torch, xq), out, M, N, K)
    torch.cuda.synchronize()
    exp = oracle.subblock_dots(W, xq, N, K)
    assert np.array_equal(out.cpu().numpy(), exp)
    assert exp[0, 0, 0] == 60960


def test_dequant_bit_exact(torch, golden_dir):
    """Reference test 1 (tests/test_q3_q4_linear.cu:76-138): device decode of
    the LCG blocks is bit-exact with the CPU dequant (and with the reference's
    own q3_quant.c vectors)."""
    say("case dequant")
    g = np.load(f"{golden_dir}/dequant_ref.npz")
    blocks = [g["lcg_blocks"].reshape(-1)]
    blocks += [g[k].reshape(-1) for k in g.files if k.startswith("w_")]
    W = np.concatenate(blocks)
    nb = W.size // 144
    out = torch.empty(nb * 256, dtype=torch.float32, device="cuda")
    q3q4.dequantize(dev(torch, W), nb, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = oracle.dequant(W.reshape(1, -1), 1, nb * 256).reshape(-1)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    assert np.array_equal(got[:1024].view(np.uint32), g["lcg_deq"].reshape(-1).view(np.uint32))


def test_weight_quantizer_bit_exact(torch, golden_dir):
    say("case weight quantizer")
    g = np.load(f"{golden_dir}/q4k_quantizer.npz")
    cases = [(g["x_" + k[2:]], g["q_" + k[2:]]) for k in g.files if k.startswith("x_")]
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    cases.append((x, oracle.quantize_q4k(x)))
    for x, exp in cases:
        out = torch.empty(exp.shape, dtype=torch.uint8, device="cuda")
        q3q4.quantize_weights(dev(torch, x), out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), exp)


# ---------------------------------------------------------------------------
# MMVQ and MMQ kernels vs the path-faithful oracles
# ---------------------------------------------------------------------------

MMVQ_SHAPES = [(256, 256), (1000, 512), (512, 5120), (64, 25600), (203, 2304), (1, 256), (5, 768)]


@pytest.mark.parametrize("N,K", MMVQ_SHAPES)
def test_mmvq_parity(torch, N, K):
    rng = np.random.default_rng(N + K)
    W = rand_weights(rng, N, K)
    Wd = dev(torch, W)
    for M in range(1, 9):
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(dev(torch, x), stage)
        xq, xd, _ = oracle.q8_1_row(x)
        ref = oracle.gemm_mmvq(W, xq, xd, N, K)
        for rows in (2, 4, 8, 16):
            say(f"case mmvq M={M} N={N} K={K} rows={rows}")
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.mmvq(Wd, stage, y, M, N, K, rows_per_tile=rows)
            torch.cuda.synchronize()
            check_close(y.cpu().numpy(), ref, f"mmvq M={M} N={N} K={K} rows={rows}")


# M <= 16 runs the paired 16-token tile, 17-32 the 32-token tile, more the 64-token tile
MMQ_CASES = [(9, 128, 256), (16, 256, 1024), (13, 1000, 2304), (1, 300, 512), (33, 1000, 512), (64, 384, 5120),
             (100, 256, 2048), (128, 128, 25600), (200, 640, 1024), (512, 256, 5120)]


@pytest.mark.parametrize("M,N,K", MMQ_CASES)
def test_mmq_parity(torch, M, N, K):
    rng = np.random.default_rng(M * 31 + N + K)
    W = rand_weights(rng, N, K)
    x = outlier_activations(rng, M, K)
    Wd = dev(torch, W)
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(dev(torch, x), stage)
    xq, xd, xs = oracle.q8_1_mmq(x)
    ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
    nkb = K // 256
    splits = sorted({1, 2, min(4, nkb), q3q4.mmq_splits(M, N, K)})
    for s in splits:
        if s > nkb or (s > 1 and (M * N) % 4):
            continue
        say(f"case mmq M={M} N={N} K={K} splits={s}")
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        q3q4.mmq(Wd, stage, y, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), ref, f"mmq M={M} N={N} K={K} splits={s}")


STREAMK_CASES = [(512, 256, 5120, 8), (512, 256, 5120, 24), (300, 640, 1024, 16), (128, 128, 25600, 8),
                 (64, 384, 5120, 8), (20, 1000, 2304, 8), (200, 640, 1024, 40), (16, 1000, 2304, 8),
                 (13, 640, 5120, 16), (3, 512, 2048, 8)]


@pytest.mark.parametrize("M,N,K,wgs", STREAMK_CASES)
def test_mmq_streamk_parity(torch, M, N, K, wgs):
    """Stream-K MMQ: split tiles with 2 or more contributors, summed by the
    last one; results against the MMQ oracle, bit-identical on repeat, and
    the tile counters back at zero."""
    rng = np.random.default_rng(M * 13 + N + K + wgs)
    W = rand_weights(rng, N, K)
    x = outlier_activations(rng, M, K)
    Wd = dev(torch, W)
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(dev(torch, x), stage)
    xq, xd, xs = oracle.q8_1_mmq(x)
    ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
    L = q3q4.load()
    slots = torch.empty(2 * wgs * L.sera_q4k_mmq_slot_floats(M), dtype=torch.float32, device="cuda")
    counters = torch.zeros(L.sera_q4k_mmq_tiles(M, N), dtype=torch.int32, device="cuda")
    outs = []
    for rep in range(2):
        say(f"case mmq stream-K M={M} N={N} K={K} wgs={wgs} rep={rep}")
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        q3q4.mmq_streamk(Wd, stage, y, M, N, K, slots, counters, wgs=wgs)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        assert int(counters.abs().sum()) == 0
    check_close(outs[0], ref, f"mmq stream-K M={M} N={N} K={K} wgs={wgs}")
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("M", [1, 7, 13, 16])
def test_mmq_paired_tile_tight(torch, M):
    """The paired 16-token tile sums the MMQ formula's own fp32 terms (even
    and odd sub-blocks in two accumulators): within 2e-5 * rms of the MMQ
    oracle, far inside the ~1e-4 * rms that the fp16 rounding of d*sc alone
    moves y, on the plain grid, split K and stream-K."""
    N, K = 700, 5120
    rng = np.random.default_rng(600 + M)
    W = rand_weights(rng, N, K)
    x = outlier_activations(rng, M, K)
    Wd = dev(torch, W)
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(dev(torch, x), stage)
    assert q3q4.mmq_stage_layout(M, K)["rows"] == 16
    xq, xd, xs = oracle.q8_1_mmq(x)
    ref = oracle.gemm_mmq(W, xq, xd, xs, N, K)
    L = q3q4.load()
    for s in (1, 4):
        say(f"case mmq paired M={M} N={N} K={K} splits={s}")
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        q3q4.mmq(Wd, stage, y, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), ref, f"mmq paired M={M} splits={s}", 2e-5)
    say(f"case mmq paired stream-K M={M} N={N} K={K}")
    slots = torch.empty(2 * 8 * L.sera_q4k_mmq_slot_floats(M), dtype=torch.float32, device="cuda")
    counters = torch.zeros(L.sera_q4k_mmq_tiles(M, N), dtype=torch.int32, device="cuda")
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.mmq_streamk(Wd, stage, y, M, N, K, slots, counters, wgs=8)
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    check_close(y.cpu().numpy(), ref, f"mmq paired stream-K M={M}", 2e-5)


# ---------------------------------------------------------------------------
# The q3_q4_linear boundary end to end
# ---------------------------------------------------------------------------

def fill_activation(M, K):
    """tests/test_q3_q4_linear.cu:226-233."""
    k = np.arange(K)[None, :]
    t = np.arange(M)[:, None]
    a = ((k * 17 + t * 131) % 1009).astype(np.float32) * np.float32(0.1)
    return (np.float32(0.5) * np.sin(a) + np.float32(0.25) * np.cos(a * np.float32(0.37))).astype(np.float32)


@pytest.mark.parametrize("M", [1, 4, 8, 9, 16, 64])
def test_linear_boundary_parity_and_repeat(torch, linear, M):
    """Reference test 2 on a seeded gate-shaped slice (N=2048, K=5120)."""
    say(f"case q3_cuda_q4k_linear M={M}")
    rng = np.random.default_rng(100 + M)
    N, K = 2048, 5120
    W = rand_weights(rng, N, K)
    g = q3q4.bind_geometry(12, K, N)
    x = fill_activation(M, K)
    Wd, xd = dev(torch, W), dev(torch, x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    y.view(torch.int32).fill_(-1)              # poison (NaN pattern)
    st = linear(g, Wd, xd, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    check_close(got, oracle.linear_reference(W, x, N, K), f"linear M={M} vs path oracle")
    ref = oracle.gemm_dequant(W, x, N, K)
    cos = float((got * ref).sum() / np.sqrt((got.astype(np.float64) ** 2).sum() * (ref ** 2).sum()))
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    say(f"  vs dequant oracle: cos={cos:.9f} relL2={rel:.4g}")
    assert cos > 0.999 and rel < 0.01
    assert st.weight_bytes == N * K // 256 * 144
    assert st.activation_read_bytes == M * K * 4 and st.activation_write_bytes == M * N * 4
    y.zero_()
    linear(g, Wd, xd, y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), got.view(np.uint32)), "repeat not bit-exact"


def test_linear_invariants(torch, linear):
    """Reference test 3: no allocation, no change of the resident pointer,
    timing stats readable after the caller's sync."""
    say("case invariants")
    rng = np.random.default_rng(3)
    N, K, M = 4096, 5120, 4
    W = dev(torch, rand_weights(rng, N, K))
    x = dev(torch, fill_activation(M, K))
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    g = q3q4.bind_geometry(12, K, N)
    ptr = W.data_ptr()
    for _ in range(3):
        linear(g, W, x, y)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    st = linear(g, W, x, y)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 == free1
    assert W.data_ptr() == ptr
    assert st.cuda_allocations == 0 and st.host_syncs == 0 and st.kernel_launches >= 2
    q3q4.Linear.read_stats(st)
    assert st.total_ms > 0 and st.kernel_ms > 0 and st.activation_quant_ms > 0


def test_zero_inputs_give_zero_outputs(torch, linear):
    say("case zeros")
    N, K = 256, 512
    rng = np.random.default_rng(9)
    W = dev(torch, rand_weights(rng, N, K))
    g = q3q4.bind_geometry(12, K, N)
    for M in (1, 8, 9, 40):
        x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
        y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
        linear(g, W, x, y)
        torch.cuda.synchronize()
        assert not y.cpu().numpy().any(), M


@pytest.mark.parametrize("M", [1, 512])
def test_full_size_gate_up_sampled_rows(torch, linear, M):
    """BASELINE shape 25600 x 5120 at M=1 (MMVQ) and M=512 (MMQ): weights
    quantized on the device, every output compared for 256 sampled rows."""
    say(f"case full-size gate/up M={M}")
    N, K = 25600, 5120
    gen = torch.Generator(device="cuda").manual_seed(0)
    wf = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    Wd = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
    q3q4.quantize_weights(wf, Wd)
    del wf
    rng = np.random.default_rng(1)
    x = outlier_activations(rng, M, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    linear(q3q4.bind_geometry(12, K, N), Wd, dev(torch, x), y)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(N, 256, replace=False))
    W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = oracle.linear_reference(W, x, 256, K)
    check_close(y.cpu().numpy()[:, rows], ref, f"gate/up M={M} sampled rows")
