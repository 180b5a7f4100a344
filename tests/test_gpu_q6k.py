"""Parity of the HIP Q6_K path (through the C ABI) with the CPU oracle.

Bars: the D4 activation stage is bit-exact; fp32 outputs are within
max |y - y_oracle| <= 1e-3 * rms(y_oracle) of the path-faithful oracle
(row Q8_1 with fp16 d8 for M <= 8, D4 Q8_1 with fp32 d8 above); on inputs
where every product and partial sum is exactly representable the outputs
are bit-exact, which pins the integer group dots inside the production
kernels; the reference test's gates (cos > 0.999, relL2 < 1%) hold against
the plain dequant oracle, and repeats are bit-exact.
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


def q6k_weights_with_edges(rng, N, K):
    """Seeded Q6_K rows; the first rows carry edge blocks: scales -128 and
    127, all quants 0 (-32) and 63 (+31), d = 0, negative d."""
    W = oracle.q6k_weights(rng, N, K).reshape(N, K // 256, 210)
    if N >= 4:
        W[0, :, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
        W[1, 0, 0:192] = 0x00
        W[1, -1, 0:192] = 0xFF
        W[2, 0, 208:210] = 0
        W[3, :, 208:210] = np.frombuffer(np.float16(-3e-5).tobytes(), np.uint8)
    return W.reshape(N, -1)


def check_close(y, ref, what):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}, ratio = {err / max(rms, 1e-30):.2e}")
    assert np.all(np.isfinite(y)), what
    assert err <= TOL * rms, what


def decode_d4_stage(stage, M, K):
    lay = q3q4.q6k_mmq_stage_layout(M, K)
    R = lay["rows"]
    b = stage.cpu().numpy()
    xh = b[lay["qs"]:lay["qs"] + R * K * 2].view(np.float16).reshape(R, K)
    d = b[lay["d"]:lay["d"] + R * K // 32 * 4].view(np.float32).reshape(K // 256, 8, R)
    return xh, d.transpose(2, 0, 1).reshape(R, K // 32)


# ---------------------------------------------------------------------------
# D4 activation stage: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(9, 256), (33, 5120), (100, 1024), (512, 5120)])
def test_q8_mmq_d4_bit_exact(torch, M, K):
    say(f"case q8_mmq_d4 M={M} K={K}")
    rng = np.random.default_rng(M * 13 + K)
    x = outlier_activations(rng, M, K)
    x[-1, :32] = 0.0
    stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    stage.fill_(0x5A)                          # poison: padding rows must be rewritten
    q3q4.quantize_mmq_d4(dev(torch, x), stage)
    torch.cuda.synchronize()
    xh, d = decode_d4_stage(stage, M, K)
    eq, ed = oracle.q8_1_mmq_d4(x)
    assert np.array_equal(xh[:M].astype(np.int32), 16 * eq.astype(np.int32))   # stored as 16 * q
    assert np.array_equal(d[:M].view(np.uint32), ed.view(np.uint32))
    assert not xh[M:].any() and not d[M:].any()


@pytest.mark.parametrize("M,K", [(1, 256), (5, 5120), (8, 25600), (33, 768)])
def test_q8_row_q6k_stage_bit_exact(torch, M, K):
    """The row quantizer's values (MMVQ arithmetic) in the tile-kernel layout:
    16 * quant, and d8 = fp32 of the fp16 scale."""
    say(f"case q8_row_q6k M={M} K={K}")
    rng = np.random.default_rng(M * 5 + K)
    x = outlier_activations(rng, M, K)
    x[0, 32:64] = 0.0
    stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    stage.fill_(0x5A)
    q3q4.quantize_row_q6k(dev(torch, x), stage)
    torch.cuda.synchronize()
    xh, d = decode_d4_stage(stage, M, K)
    eq, ed, _ = oracle.q8_1_row(x)
    assert np.array_equal(xh[:M].astype(np.int32), 16 * eq.astype(np.int32))
    assert np.array_equal(d[:M].view(np.uint32), oracle.h2f(ed).view(np.uint32))
    assert not xh[M:].any() and not d[M:].any()


@pytest.mark.parametrize("N,K", [(256, 256), (515, 5120), (64, 25600), (203, 2304)])
def test_q6k_tile_kernel_mmvq_formula_parity(torch, N, K):
    """The tile kernel on a row-formula stage computes the MMVQ formula
    (what sera_q6k_dense_vec runs at 4-8 tokens where
    sera_q6k_vec_uses_tile says so)."""
    rng = np.random.default_rng(N * 7 + K)
    W = q6k_weights_with_edges(rng, N, K)
    Wd = dev(torch, W)
    for M in (1, 3, 5, 6, 7, 8, 16):
        say(f"case q6k tile mmvq-formula M={M} N={N} K={K}")
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row_q6k(dev(torch, x), stage)
        xq, xd, _ = oracle.q8_1_row(x)
        ref = oracle.gemm_q6k(W, xq, oracle.h2f(xd), N, K)
        s = q3q4.q6k_mmq_splits(M, N, K)
        partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        q3q4.q6k_mmq(Wd, stage, y, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), ref, f"q6k tile mmvq-formula M={M} N={N} K={K} splits={s}")


# ---------------------------------------------------------------------------
# MMVQ (1..8 tokens)
# ---------------------------------------------------------------------------

Q6_MMVQ_SHAPES = [(256, 256), (1000, 512), (515, 5120), (64, 25600), (203, 2304), (1, 256), (7, 768)]


@pytest.mark.parametrize("N,K", Q6_MMVQ_SHAPES)
def test_q6k_mmvq_parity(torch, N, K):
    rng = np.random.default_rng(N * 3 + K)
    W = q6k_weights_with_edges(rng, N, K)
    Wd = dev(torch, W)
    for M in range(1, 9):
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(dev(torch, x), stage)
        xq, xd, _ = oracle.q8_1_row(x)
        ref = oracle.gemm_q6k(W, xq, oracle.h2f(xd), N, K)
        for rows in ((1, 2, 4) if M <= 4 else (1, 2)):
            say(f"case q6k mmvq M={M} N={N} K={K} rows={rows}")
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.q6k_mmvq(Wd, stage, y, M, N, K, rows_per_wave=rows)
            torch.cuda.synchronize()
            check_close(y.cpu().numpy(), ref, f"q6k mmvq M={M} N={N} K={K} rows={rows}")


def _exact_inputs(rng, M, N, K):
    """d = 2^-8, group scales in [-4, 4], activations q * 2^-5 with a +-127 in
    every 32-block: every partial sum is a multiple of 2^-13 below 2^11, so
    fp32 holds it exactly and the outputs are exact."""
    W = oracle.q6k_weights(rng, N, K, scales=None).reshape(N, K // 256, 210)
    W[:, :, 192:208] = rng.integers(-4, 5, (N, K // 256, 16)).astype(np.int8).view(np.uint8)
    W[:, :, 208:210] = np.frombuffer(np.float16(2.0 ** -8).tobytes(), np.uint8)
    q = rng.integers(-20, 21, (M, K // 32, 32))
    q[:, :, 0] = 127
    q[:, :, 1] = -127
    return W.reshape(N, -1), (q.reshape(M, K) * 2.0 ** -5).astype(np.float32)


@pytest.mark.parametrize("M", [1, 3, 8])
def test_q6k_mmvq_exact_integer_dots(torch, M):
    N, K = 130, 768
    say(f"case q6k mmvq exact M={M}")
    rng = np.random.default_rng(77 + M)
    W, x = _exact_inputs(rng, M, N, K)
    stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(dev(torch, x), stage)
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    xq, xd, _ = oracle.q8_1_row(x)
    assert np.array_equal(oracle.gemm_q6k(W, xq, oracle.h2f(xd), N, K), ref)
    for rows in ((1, 2, 4) if M <= 4 else (1, 2)):
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        q3q4.q6k_mmvq(dev(torch, W), stage, y, M, N, K, rows_per_wave=rows)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().astype(np.float64), ref), f"rows={rows}"


# ---------------------------------------------------------------------------
# MMQ (fp16-MFMA tiles)
# ---------------------------------------------------------------------------

# the last two run the 64-token tile (ragged tokens and rows, N % 4 == 2; and
# whole tiles with 16-byte stores); the others the 32-token tile
Q6_MMQ_CASES = [(9, 128, 256), (16, 256, 1024), (33, 1000, 512), (64, 384, 5120), (100, 250, 2048),
                (128, 128, 25600), (200, 640, 1024), (512, 256, 5120), (40, 77, 2304), (100, 2046, 8192),
                (128, 2048, 8192)]


@pytest.mark.parametrize("M,N,K", Q6_MMQ_CASES)
def test_q6k_mmq_parity(torch, M, N, K):
    rng = np.random.default_rng(M * 17 + N + K)
    W = q6k_weights_with_edges(rng, N, K)
    x = outlier_activations(rng, M, K)
    Wd = dev(torch, W)
    stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq_d4(dev(torch, x), stage)
    xq, d = oracle.q8_1_mmq_d4(x)
    ref = oracle.gemm_q6k(W, xq, d, N, K)
    nkb = K // 256
    splits = sorted({1, 2, min(4, nkb), q3q4.q6k_mmq_splits(M, N, K)})
    for s in splits:
        if s > nkb or (s > 1 and (M * N) % 4):
            continue
        say(f"case q6k mmq M={M} N={N} K={K} splits={s}")
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        q3q4.q6k_mmq(Wd, stage, y, M, N, K, splits=s, partial=partial)
        torch.cuda.synchronize()
        check_close(y.cpu().numpy(), ref, f"q6k mmq M={M} N={N} K={K} splits={s}")


@pytest.mark.parametrize("M,N,K", [(9, 200, 768), (64, 200, 768), (100, 200, 768), (100, 2046, 8192)])
def test_q6k_mmq_exact_integer_dots(torch, M, N, K):
    """The fp16-MFMA products carry the exact integers sc * (q - 32) * q8:
    on exact inputs the output equals the exact GEMM bit for bit (32-token
    tiles; the last case the 64-token tile)."""
    say(f"case q6k mmq exact M={M} N={N} K={K} tile={q3q4.load().sera_q6k_mmq_tile_tokens(M, N, K)}")
    rng = np.random.default_rng(91 + M)
    W, x = _exact_inputs(rng, M, N, K)
    stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq_d4(dev(torch, x), stage)
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    xq, d = oracle.q8_1_mmq_d4(x)
    assert np.array_equal(oracle.gemm_q6k(W, xq, d, N, K), ref)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.q6k_mmq(dev(torch, W), stage, y, M, N, K, splits=1)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.float64), ref)


def test_q6k_mmq_exact_full_scale_range(torch):
    """Group scales at the int8 extremes (-128, 127, ...) with d = 2^-14 and
    quants 0..63: the largest fp16 operand parts (16 * 32 * -8) are used;
    one super-block, activations in [-8, 8] plus +-127 per 32-block, so
    every partial sum is an integer multiple of 2^-19 below 2^5."""
    M, N, K = 40, 64, 256
    say("case q6k mmq exact full scale range")
    rng = np.random.default_rng(1234)
    W = oracle.q6k_weights(rng, N, K).reshape(N, 1, 210)
    pattern = np.array([-128, 127, -127, 126, 64, -65, 1, -1, -128, -128, 127, 127, 0, 15, -16, 16], np.int8)
    W[:, 0, 192:208] = np.array([np.roll(pattern, n) for n in range(N)]).view(np.uint8)
    W[:, 0, 208:210] = np.frombuffer(np.float16(2.0 ** -14).tobytes(), np.uint8)
    W = W.reshape(N, -1)
    q = rng.integers(-8, 9, (M, K // 32, 32))
    q[:, :, 0] = 127
    q[:, :, 1] = -127
    x = (q.reshape(M, K) * 2.0 ** -5).astype(np.float32)
    stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq_d4(dev(torch, x), stage)
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.q6k_mmq(dev(torch, W), stage, y, M, N, K, splits=1)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().astype(np.float64), ref)


# ---------------------------------------------------------------------------
# The q3_q4_linear boundary with qtype 14
# ---------------------------------------------------------------------------

def fill_activation(M, K):
    k = np.arange(K)[None, :]
    t = np.arange(M)[:, None]
    a = ((k * 17 + t * 131) % 1009).astype(np.float32) * np.float32(0.1)
    return (np.float32(0.5) * np.sin(a) + np.float32(0.25) * np.cos(a * np.float32(0.37))).astype(np.float32)


@pytest.mark.parametrize("M", [1, 4, 8, 9, 16, 64])
def test_q6k_linear_boundary_parity_and_repeat(torch, linear, M):
    """attn_v shape (N=1024, K=5120) through q3_cuda_q4k_linear."""
    say(f"case q3_cuda_q4k_linear q6k M={M}")
    rng = np.random.default_rng(300 + M)
    N, K = 1024, 5120
    W = oracle.q6k_weights(rng, N, K)
    g = q3q4.bind_geometry(14, K, N)
    x = fill_activation(M, K)
    Wd, xd = dev(torch, W), dev(torch, x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    y.view(torch.int32).fill_(-1)
    st = linear(g, Wd, xd, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    check_close(got, oracle.linear_reference_q6k(W, x, N, K), f"linear q6k M={M} vs path oracle")
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    cos = float((got * ref).sum() / np.sqrt((got.astype(np.float64) ** 2).sum() * (ref ** 2).sum()))
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    say(f"  vs dequant oracle: cos={cos:.9f} relL2={rel:.4g}")
    assert cos > 0.999 and rel < 0.01
    assert st.weight_bytes == N * K // 256 * 210
    assert st.kernel_launches == q3q4.load().sera_q6k_kernel_launches(M, N, K)
    y.zero_()
    linear(g, Wd, xd, y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), got.view(np.uint32)), "repeat not bit-exact"


def test_q6k_zero_inputs_give_zero_outputs(torch, linear):
    say("case q6k zeros")
    N, K = 256, 512
    W = dev(torch, oracle.q6k_weights(np.random.default_rng(5), N, K))
    g = q3q4.bind_geometry(14, K, N)
    for M in (1, 8, 9, 40):
        x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
        y = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
        linear(g, W, x, y)
        torch.cuda.synchronize()
        assert not y.cpu().numpy().any(), M


def device_q6k_weights(torch, N, K, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    W = torch.randint(0, 256, (N, K // 256, 210), generator=gen, device="cuda", dtype=torch.uint8)
    d = (torch.rand((N, K // 256), generator=gen, device="cuda") + 0.5) * 2e-5
    d = d * (torch.randint(0, 2, (N, K // 256), generator=gen, device="cuda") * 2 - 1)
    W[:, :, 208:210] = d.to(torch.float16).view(torch.uint8).view(N, K // 256, 2)
    return W.view(N, -1)


@pytest.mark.parametrize("M", [1, 512])
def test_q6k_full_size_down_sampled_rows(torch, linear, M):
    """ffn_down shape 25600 -> 5120 (a Q6_K tensor of the stock Q4_K_M GGUF)
    at M=1 (MMVQ) and M=512 (MMQ); 256 sampled rows compared."""
    say(f"case q6k full-size down M={M}")
    N, K = 5120, 25600
    Wd = device_q6k_weights(torch, N, K, seed=2)
    rng = np.random.default_rng(4)
    x = outlier_activations(rng, M, K)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    linear(q3q4.bind_geometry(14, K, N), Wd, dev(torch, x), y)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(N, 256, replace=False))
    W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = oracle.linear_reference_q6k(W, x, 256, K)
    check_close(y.cpu().numpy()[:, rows], ref, f"q6k down M={M} sampled rows")
