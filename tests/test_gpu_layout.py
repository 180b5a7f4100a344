"""The Q6_K split device layout (SERA_QTYPE_Q6K_SPLIT) through the C ABI.

Bars:
  * the repack (device GGUF bytes -> split layout) and the chunked host
    upload are byte-exact with the oracle's q6k_split; GGUF-layout uploads
    are plain copies;
  * the split-layout MMVQ kernel is within 1e-3 * rms(y) of the
    path-faithful oracle for 1..8 tokens and bit-exact on exact inputs;
  * the tile kernel (both activation stages, split-K) and the gathered-row
    kernels give bit-identical results on either layout of the same bytes
    (same arithmetic, other addressing);
  * q3_cuda_q4k_linear and sera_linear_group accept the split qtype.
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3
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
    return q3q4.Linear(device=0, max_tokens=2048, max_features=151936, max_k=25600)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def outlier_activations(rng, M, K, frac=0.01, gain=20.0):
    x = rng.standard_normal((M, K)).astype(np.float32)
    ch = rng.choice(K, max(1, int(np.ceil(frac * K))), replace=False)
    x[:, ch] *= gain
    return x


def weights_with_edges(rng, N, K):
    """Seeded GGUF Q6_K rows; the first rows carry edge blocks: scales -128
    and 127, all quants 0 and 63, d = 0, negative d."""
    W = oracle.q6k_weights(rng, N, K).reshape(N, K // 256, 210)
    if N >= 4:
        W[0, :, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
        W[1, 0, 0:192] = 0x00
        W[1, -1, 0:192] = 0xFF
        W[2, 0, 208:210] = 0
        W[3, :, 208:210] = np.frombuffer(np.float16(-3e-5).tobytes(), np.uint8)
    return W.reshape(N, -1)


def to_split(torch, W, N, K):
    """GGUF bytes -> split layout on the device through the library."""
    src = dev(torch, W)
    dst = torch.empty(q3q4.weight_bytes(SPLIT, N, K), dtype=torch.uint8, device="cuda")
    q3q4.weight_to_device_layout(SPLIT, N, K, src, dst)
    torch.cuda.synchronize()
    return dst


def check_close(y, ref, what):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}")
    assert np.all(np.isfinite(y)), what
    assert err <= TOL * rms, what


# ---------------------------------------------------------------------------
# Repack and upload: byte-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(1, 256), (7, 768), (300, 5120), (64, 25600)])
def test_repack_on_device_is_byte_exact(torch, N, K):
    say(f"case repack N={N} K={K}")
    W = weights_with_edges(np.random.default_rng(N + K), N, K)
    got = to_split(torch, W, N, K).cpu().numpy()
    assert np.array_equal(got, oracle.q6k_split(W, N, K))
    assert np.array_equal(oracle.q6k_unsplit(got, N, K), W)


@pytest.mark.parametrize("N,K,staging", [(5, 512, 210 * 3 + 100), (33, 2304, 4096), (257, 5120, 1 << 20)])
def test_host_upload_split_in_passes(torch, N, K, staging):
    """The staging buffer holds whole blocks per pass (3 blocks, then 19,
    then all): every pass lands at its block offset."""
    say(f"case upload split N={N} K={K} staging={staging}")
    W = weights_with_edges(np.random.default_rng(3 * N + K), N, K)
    dst = torch.full((q3q4.weight_bytes(SPLIT, N, K),), 0xA5, dtype=torch.uint8, device="cuda")
    stage = torch.empty(staging, dtype=torch.uint8, device="cuda")
    host = np.ascontiguousarray(W)
    q3q4.weight_upload(SPLIT, N, K, host, dst, stage)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), oracle.q6k_split(W, N, K))


@pytest.mark.parametrize("qtype", [12, 14])
def test_host_upload_gguf_layouts_copy_verbatim(torch, qtype):
    N, K = 40, 1024
    say(f"case upload verbatim qtype={qtype}")
    rng = np.random.default_rng(qtype)
    W = rng.integers(0, 256, q3q4.weight_bytes(qtype, N, K), dtype=np.uint8)
    dst = torch.zeros(W.size, dtype=torch.uint8, device="cuda")
    q3q4.weight_upload(qtype, N, K, W, dst)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), W)


def test_upload_rejects_bad_arguments(torch):
    N, K = 4, 256
    W = np.zeros(q3q4.weight_bytes(14, N, K), np.uint8)
    dst = torch.empty(W.size, dtype=torch.uint8, device="cuda")
    with pytest.raises(q3q4.Q3Q4Error, match="staging"):
        q3q4.weight_upload(SPLIT, N, K, W, dst, None)
    with pytest.raises(q3q4.Q3Q4Error, match="qtype"):
        q3q4.weight_upload(13, N, K, W, dst, None)
    assert q3q4.weight_bytes(SPLIT, N, 300) == 0


# ---------------------------------------------------------------------------
# MMVQ on the split layout
# ---------------------------------------------------------------------------

SHAPES = [(256, 256), (1000, 512), (515, 5120), (64, 25600), (203, 2304), (1, 256), (3, 768), (7, 768)]


@pytest.mark.parametrize("N,K", SHAPES)
def test_split_mmvq_parity(torch, N, K):
    rng = np.random.default_rng(N * 11 + K)
    W = weights_with_edges(rng, N, K)
    Ws = to_split(torch, W, N, K)
    for M in range(1, 9):
        x = outlier_activations(rng, M, K)
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(dev(torch, x), stage)
        xq, xd, _ = oracle.q8_1_row(x)
        ref = oracle.gemm_q6k(W, xq, oracle.h2f(xd), N, K)
        for rows in (0, 2, 4):
            say(f"case split mmvq M={M} N={N} K={K} rows={rows}")
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.q6k_mmvq(Ws, stage, y, M, N, K, rows_per_wave=rows, qtype=SPLIT)
            torch.cuda.synchronize()
            check_close(y.cpu().numpy(), ref, f"split mmvq M={M} N={N} K={K} rows={rows}")


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_split_mmvq_exact_integer_dots(torch, M):
    """d = 2^-8, scales in [-4, 4], activations q * 2^-5 with +-127 per
    32-block: exact partial sums, so the output equals the exact GEMM."""
    N, K = 130, 768
    say(f"case split mmvq exact M={M}")
    rng = np.random.default_rng(700 + M)
    W = oracle.q6k_weights(rng, N, K).reshape(N, K // 256, 210)
    W[:, :, 192:208] = rng.integers(-4, 5, (N, K // 256, 16)).astype(np.int8).view(np.uint8)
    W[:, :, 208:210] = np.frombuffer(np.float16(2.0 ** -8).tobytes(), np.uint8)
    W = W.reshape(N, -1)
    q = rng.integers(-20, 21, (M, K // 32, 32))
    q[:, :, 0] = 127
    q[:, :, 1] = -127
    x = (q.reshape(M, K) * 2.0 ** -5).astype(np.float32)
    stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_row(dev(torch, x), stage)
    ref = oracle.gemm_dequant_q6k(W, x, N, K)
    Ws = to_split(torch, W, N, K)
    for rows in (2, 4):
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        q3q4.q6k_mmvq(Ws, stage, y, M, N, K, rows_per_wave=rows, qtype=SPLIT)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().astype(np.float64), ref), f"rows={rows}"


# ---------------------------------------------------------------------------
# Tile kernel and gathered rows: the same bits on either layout
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(5, 256, 256), (8, 515, 5120), (33, 1000, 512), (64, 384, 5120),
                                   (200, 77, 2304), (128, 128, 25600)])
def test_split_tile_kernel_bit_identical_to_gguf(torch, M, N, K):
    rng = np.random.default_rng(M + 5 * N + K)
    W = weights_with_edges(rng, N, K)
    Wg, Ws = dev(torch, W), to_split(torch, W, N, K)
    x = dev(torch, outlier_activations(rng, M, K))
    for row_formula in (0, 1):
        stage = torch.empty(q3q4.q6k_mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        (q3q4.quantize_row_q6k if row_formula else q3q4.quantize_mmq_d4)(x, stage)
        nkb = K // 256
        for s in sorted({1, min(2, nkb), q3q4.q6k_mmq_splits(M, N, K)}):
            if s > 1 and (M * N) % 4:
                continue
            say(f"case split tile M={M} N={N} K={K} row_formula={row_formula} splits={s}")
            partial = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
            yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            ys = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.q6k_mmq(Wg, stage, yg, M, N, K, splits=s, partial=partial)
            q3q4.q6k_mmq(Ws, stage, ys, M, N, K, splits=s, partial=partial, qtype=SPLIT)
            torch.cuda.synchronize()
            a, b = yg.cpu().numpy(), ys.cpu().numpy()
            assert np.all(np.isfinite(a))
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("N,K", [(300, 256), (1001, 5120), (77, 2304)])
def test_split_gathered_rows_bit_identical_to_gguf(torch, N, K):
    say(f"case split gathered rows N={N} K={K}")
    rng = np.random.default_rng(N * K)
    W = weights_with_edges(rng, N, K)
    Wg, Ws = dev(torch, W), to_split(torch, W, N, K)
    ids = rng.integers(0, N, 41).astype(np.int32)
    ids[3] = N + 1
    idd = dev(torch, ids)
    outs = []
    for qt, Wx in ((14, Wg), (SPLIT, Ws)):
        e = torch.full((len(ids), K), 7.25, dtype=torch.float32, device="cuda")
        q3q4.embedding(qt, Wx, N, K, idd, e)
        hidden = dev(torch, rng.standard_normal((3, K)).astype(np.float32)) if not outs else outs[0][2]
        lg = torch.full((3 * 13,), 3.0, dtype=torch.float32, device="cuda")
        q3q4.candidate_logits(qt, Wx, N, K, hidden, idd[:39], 13, lg)
        torch.cuda.synchronize()
        outs.append((e.cpu().numpy(), lg.cpu().numpy(), hidden))
    (eg, lgg, _), (es, lgs, _) = outs
    assert np.array_equal(eg.view(np.uint32), es.view(np.uint32))
    assert np.array_equal(lgg.view(np.uint32), lgs.view(np.uint32))
    ref = oracle.dequant_q6k(W, N, K)
    assert np.array_equal(es[0].view(np.uint32), ref[ids[0]].view(np.uint32))
    assert np.all(es[3] == 7.25) and np.isnan(lgs[3])


# ---------------------------------------------------------------------------
# The boundary and the fused group with the split qtype
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 4, 5, 8, 9, 64])
def test_split_linear_boundary(torch, linear, M):
    """attn_v shape through q3_cuda_q4k_linear with a geometry bound to the
    split qtype: within 1e-3 * rms of the path oracle; where the tile kernel
    runs on both layouts (sera_q6k_vec_uses_tile_qt, or the MMQ path)
    bit-identical to the GGUF-layout call."""
    say(f"case q3_cuda_q4k_linear split M={M}")
    rng = np.random.default_rng(900 + M)
    N, K = 1024, 5120
    W = oracle.q6k_weights(rng, N, K)
    x = dev(torch, outlier_activations(rng, M, K))
    gs, gg = q3q4.bind_geometry(SPLIT, K, N), q3q4.bind_geometry(14, K, N)
    assert gs.weight_bytes == gg.weight_bytes == N * K // 256 * 210
    ys = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    linear(gs, to_split(torch, W, N, K), x, ys)
    linear(gg, dev(torch, W), x, yg)
    torch.cuda.synchronize()
    a, b = ys.cpu().numpy(), yg.cpu().numpy()
    check_close(a, oracle.linear_reference_q6k(W, x.cpu().numpy(), N, K), f"split linear M={M}")
    L = q3q4.load()
    if M > 8 or (L.sera_q6k_vec_uses_tile_qt(SPLIT, M, N, K) and L.sera_q6k_vec_uses_tile_qt(14, M, N, K)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("M,N", [(4, 16384), (6, 4096), (7, 4096), (8, 5120), (4, 4096)])
def test_q6k_boundary_tile_branch_of_mmvq_path(torch, linear, M, N):
    """q3_cuda_q4k_linear on Q6_K matrices of 4096+ rows at 4-8 tokens, where
    sera_q6k_dense_vec may run the tile kernel on a row-formula stage (stage
    sized from the padded batch, split partials in the arena): sampled rows
    within 1e-3 * rms of the MMVQ-formula oracle, the split layout
    bit-identical to the GGUF bytes whenever both run the tile kernel (at 6
    tokens on 4096 rows only the GGUF bytes do), and the launch count the
    stats report equal to sera_q6k_kernel_launches_qt."""
    L = q3q4.load()
    K = 5120
    tiles = {qt: bool(L.sera_q6k_vec_uses_tile_qt(qt, M, N, K)) for qt in (14, SPLIT)}
    tile = tiles[14] and tiles[SPLIT]
    say(f"case q6k boundary M={M} N={N} K={K} tile={tiles} launches={L.sera_q6k_kernel_launches(M, N, K)}")
    if (M, N) != (4, 4096):
        assert tiles[14], "case meant for the tile branch"
    assert tiles[SPLIT] == ((M, N) not in ((6, 4096), (4, 4096)))
    rng = np.random.default_rng(70 * M + N)
    W = oracle.q6k_weights(rng, N, K)
    xh = outlier_activations(rng, M, K)
    x = dev(torch, xh)
    outs = {}
    for qt, Wx in ((14, dev(torch, W)), (SPLIT, to_split(torch, W, N, K))):
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        st = linear(q3q4.bind_geometry(qt, K, N), Wx, x, y)
        torch.cuda.synchronize()
        assert st.kernel_launches == L.sera_q6k_kernel_launches_qt(qt, M, N, K)
        outs[qt] = y.cpu().numpy()
        del Wx
    rows = np.sort(rng.choice(N, 256, replace=False))
    ref = oracle.linear_reference_q6k(np.ascontiguousarray(W[rows]), xh, len(rows), K)
    for qt, y in outs.items():
        check_close(y[:, rows], ref, f"q6k boundary qtype={qt} M={M} N={N}")
    if tile:
        assert np.array_equal(outs[14].view(np.uint32), outs[SPLIT].view(np.uint32))


@pytest.mark.parametrize("M", [1, 3, 6, 40])
def test_split_linear_group_accumulate(torch, linear, M):
    K = 2048
    Ns = [768, 256]
    rng = np.random.default_rng(40 + M)
    Ws = [oracle.q6k_weights(rng, n, K) for n in Ns]
    x = outlier_activations(rng, M, K)
    say(f"case split group M={M}")
    geos = [q3q4.bind_geometry(SPLIT, K, n) for n in Ns]
    Wd = [to_split(torch, w, n, K) for w, n in zip(Ws, Ns)]
    y0 = [rng.standard_normal((M, n)).astype(np.float32) for n in Ns]
    ys = [dev(torch, a) for a in y0]
    q3q4.linear_group(geos, Wd, ys, dev(torch, x), None, None, 0.0, q3q4.LIN_ACCUMULATE)
    torch.cuda.synchronize()
    for i, n in enumerate(Ns):
        check_close(ys[i].cpu().numpy() - y0[i], oracle.linear_reference_q6k(Ws[i], x, n, K), f"group[{i}]")
