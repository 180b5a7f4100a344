"""The tiled Q4_K device layout (SERA_QTYPE_Q4K_TILED) through the C ABI.

The layout keeps every 144-byte GGUF block and only reorders them (block
(r, b) at ((r/16)*(K/256) + b)*2304 + (r%16)*144), and every kernel does the
same arithmetic on it as on the GGUF bytes, so the bars are exact:
  * the device repack and the chunked host upload give exactly the bytes of
    that offset formula, written out here block by block;
  * every product kernel (dot4 MMVQ at each rows-per-wave, the few-token
    kernel in both formulas with split K and the persistent grid, split-K
    and stream-K MMQ), the boundary, the fused group and the gathered-row
    kernels return bit-identical outputs on the tiled bytes and on the GGUF
    bytes of the same matrix;
  * the GGUF outputs themselves are held to the oracle by the other GPU
    tests; one case here checks the tiled boundary against the oracle too.
"""
import ctypes
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TILED = q3q4.QTYPE_Q4K_TILED


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


def activations(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32)
    ch = rng.choice(K, max(1, K // 100), replace=False)
    x[:, ch] *= 20.0
    return x


def device_blocks(torch, N, K, seed):
    """Random Q4_K blocks made on the device: random quant and scale bytes,
    d and dmin small positive fp16 (every value finite)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    nblk = N * (K // 256)
    W = torch.randint(0, 256, (nblk, 144), dtype=torch.uint8, device="cuda", generator=g)
    dd = (torch.rand((nblk, 2), device="cuda", generator=g) * 1e-3 + 1e-5).half()
    W[:, 0:4] = dd.view(torch.uint8)
    return W.reshape(-1)


def expected_tiled(W, N, K):
    """GGUF bytes -> tiled bytes, one block at a time from the offset formula."""
    nkb = K // 256
    out = np.empty(N * nkb * 144, np.uint8)
    blocks = W.reshape(N, nkb, 144)
    for r in range(N):
        for b in range(nkb):
            o = ((r // 16) * nkb + b) * 2304 + (r % 16) * 144
            out[o:o + 144] = blocks[r, b]
    return out


def to_tiled(torch, Wg, N, K):
    dst = torch.empty(q3q4.weight_bytes(TILED, N, K), dtype=torch.uint8, device="cuda")
    q3q4.weight_to_device_layout(TILED, N, K, Wg, dst)
    torch.cuda.synchronize()
    return dst


def same_bits(a, b, what):
    a, b = a.cpu().numpy(), b.cpu().numpy()
    assert np.all(np.isfinite(a)), what
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), what


def fewtok_once(torch, qtype, form, W, stage, M, N, K, chunk):
    """One few-token launch (sera_q4k_fewtok_qt) with fresh split slots and
    zeroed row-group counters, which must be zero again afterwards."""
    sp = q3q4.fewtok_splits(M, N, K, chunk)
    slots = torch.empty(sp * M * N, dtype=torch.float32, device="cuda") if sp > 1 else None
    counters = torch.zeros(q3q4.fewtok_groups(M, N, K), dtype=torch.int32, device="cuda") if sp > 1 else None
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q3q4.fewtok(W, stage, y, M, N, K, chunk=chunk, slots=slots, counters=counters, form=form, qtype=qtype)
    torch.cuda.synchronize()
    if counters is not None:
        assert int(counters.abs().sum()) == 0, "row-group counters not reset"
    return y


# ---------------------------------------------------------------------------
# The layout: repack, upload, argument checks
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(16, 256), (48, 768), (320, 5120), (64, 25600)])
def test_repack_on_device_is_byte_exact(torch, N, K):
    say(f"case tiled repack N={N} K={K}")
    W = np.random.default_rng(N + K).integers(0, 256, N * K // 256 * 144, dtype=np.uint8)
    got = to_tiled(torch, dev(torch, W), N, K).cpu().numpy()
    assert np.array_equal(got, expected_tiled(W, N, K))


@pytest.mark.parametrize("N,K,groups", [(48, 512, 1), (80, 2304, 3), (272, 5120, 100)])
def test_host_upload_tiled_in_passes(torch, N, K, groups):
    """The staging buffer holds `groups` whole 16-row groups (plus slack):
    every pass lands at its tile offset."""
    gb = 16 * (K // 256) * 144
    staging = groups * gb + 100
    say(f"case tiled upload N={N} K={K} staging={staging}")
    W = np.random.default_rng(3 * N + K).integers(0, 256, N * K // 256 * 144, dtype=np.uint8)
    dst = torch.full((q3q4.weight_bytes(TILED, N, K),), 0xA5, dtype=torch.uint8, device="cuda")
    stage = torch.empty(staging, dtype=torch.uint8, device="cuda")
    q3q4.weight_upload(TILED, N, K, W, dst, stage)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), expected_tiled(W, N, K))


def test_tiled_rejects_bad_arguments(torch):
    N, K = 32, 512
    W = np.zeros(N * K // 256 * 144, np.uint8)
    dst = torch.empty(W.size, dtype=torch.uint8, device="cuda")
    assert q3q4.weight_bytes(TILED, 40, K) == 0
    assert q3q4.weight_bytes(TILED, N, K) == W.size
    with pytest.raises(q3q4.Q3Q4Error, match="staging"):
        q3q4.weight_upload(TILED, N, K, W, dst, torch.empty(16 * 2 * 144 - 1, dtype=torch.uint8, device="cuda"))
    with pytest.raises(q3q4.Q3Q4Error, match="16"):
        q3q4.weight_upload(TILED, 40, K, np.zeros(40 * 2 * 144, np.uint8), dst, None)
    with pytest.raises(q3q4.Q3Q4Error):
        q3q4.bind_geometry(TILED, K, 40)
    g = q3q4.bind_geometry(TILED, K, N)
    assert g.weight_bytes == W.size


# ---------------------------------------------------------------------------
# Kernels one by one: the same bits on either layout
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(16, 256), (1008, 2304), (25600, 5120), (5120, 25600)])
def test_tiled_mmvq_bit_identical(torch, N, K):
    rng = np.random.default_rng(N + K)
    Wg = device_blocks(torch, N, K, N * 7 + K)
    Wt = to_tiled(torch, Wg, N, K)
    for M in (1, 2, 4, 8):
        x = dev(torch, activations(rng, M, K))
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(x, stage)
        for rows in (0, 2, 4, 8, 16):
            say(f"case tiled mmvq M={M} N={N} K={K} rows={rows}")
            yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            yt = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.mmvq(Wg, stage, yg, M, N, K, rows_per_tile=rows)
            q3q4.mmvq(Wt, stage, yt, M, N, K, rows_per_tile=rows, qtype=TILED)
            torch.cuda.synchronize()
            same_bits(yg, yt, f"mmvq M={M} N={N} K={K} rows={rows}")


# (0, 4, 64, 25600): 8-wave workgroups whose last four waves own no tile (the
# tiled bytes load directly, the GGUF bytes through the staged copy)
FEWTOK_CASES = [(0, 2, 25600, 5120), (0, 4, 25600, 5120), (0, 8, 5120, 25600), (0, 8, 1008, 2304),
                (1, 9, 25600, 5120), (1, 16, 151936, 5120), (1, 12, 4096, 25600), (1, 4, 16, 256), (0, 4, 64, 25600)]


@pytest.mark.parametrize("form,M,N,K", FEWTOK_CASES)
def test_tiled_fewtok_bit_identical(torch, form, M, N, K):
    """Planned chunk and a forced short chunk (split K through the slots and
    row-group counters); the 151936-row case runs the persistent grid."""
    rng = np.random.default_rng(M * N + K)
    Wg = device_blocks(torch, N, K, M + N + K)
    Wt = to_tiled(torch, Wg, N, K)
    x = dev(torch, activations(rng, M, K))
    if form == 0:
        stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(x, stage)
    else:
        stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_mmq(x, stage)
    nkb = K // 256
    for chunk in sorted({0, min(2, nkb)}):
        sp = q3q4.fewtok_splits(M, N, K, chunk)
        say(f"case tiled fewtok form={form} M={M} N={N} K={K} chunk={chunk} splits={sp} "
            f"grid={q3q4.fewtok_grid(form, M, N, K, chunk)}")
        yg = fewtok_once(torch, 12, form, Wg, stage, M, N, K, chunk)
        yt = fewtok_once(torch, TILED, form, Wt, stage, M, N, K, chunk)
        same_bits(yg, yt, f"fewtok form={form} M={M} N={N} K={K} chunk={chunk}")


@pytest.mark.parametrize("M,N,K", [(64, 5120, 5120), (200, 1008, 2304), (512, 25600, 5120), (33, 4096, 25600)])
def test_tiled_mmq_bit_identical(torch, linear, M, N, K):
    """Split-K MMQ at 1, 2 and the built-in split count, and stream-K (its
    workgroup count comes from the CU count the initialised library read)."""
    L = q3q4.load()
    rng = np.random.default_rng(M + N + K)
    Wg = device_blocks(torch, N, K, 3 * M + N + K)
    Wt = to_tiled(torch, Wg, N, K)
    x = dev(torch, activations(rng, M, K))
    stage = torch.empty(q3q4.mmq_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
    q3q4.quantize_mmq(x, stage)
    for s in sorted({1, 2, q3q4.mmq_splits(M, N, K)}):
        if s > 1 and (M * N) % 4:
            continue
        say(f"case tiled mmq M={M} N={N} K={K} splits={s}")
        part = torch.empty(s * M * N, dtype=torch.float32, device="cuda") if s > 1 else None
        ys = []
        for qt, W in ((12, Wg), (TILED, Wt)):
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.mmq(W, stage, y, M, N, K, splits=s, partial=part, qtype=qt)
            torch.cuda.synchronize()
            ys.append(y)
        same_bits(ys[0], ys[1], f"mmq M={M} N={N} K={K} splits={s}")
    wgs = L.sera_q4k_mmq_streamk_wgs(M)
    assert wgs >= 8
    if L.sera_q4k_mmq_tiles(M, N) * (K // 256) >= wgs:
        say(f"case tiled mmq stream-K M={M} N={N} K={K} wgs={wgs}")
        slots = torch.empty(2 * wgs * L.sera_q4k_mmq_slot_floats(M), dtype=torch.float32, device="cuda")
        ys = []
        for qt, W in ((12, Wg), (TILED, Wt)):
            counters = torch.zeros(L.sera_q4k_mmq_tiles(M, N), dtype=torch.int32, device="cuda")
            y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            q3q4.mmq_streamk(W, stage, y, M, N, K, slots, counters, wgs=wgs, qtype=qt)
            torch.cuda.synchronize()
            assert int(counters.abs().sum()) == 0, "tile counters not reset"
            ys.append(y)
        same_bits(ys[0], ys[1], f"mmq stream-K M={M} N={N} K={K}")


# ---------------------------------------------------------------------------
# The boundary, the fused group and the gathered rows
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(25600, 5120), (5120, 25600), (1008, 2304)])
def test_tiled_linear_boundary(torch, linear, N, K):
    """q3_cuda_q4k_linear with a tiled geometry, every path the batch size
    picks (MMVQ, few-token in both formulas, MMQ split-K / stream-K), is
    bit-identical to the GGUF geometry where both pick the same kernel.
    Where the tiled rule picks the few-token kernel and the GGUF rule dot4
    (sera_q4k_vec_uses_fewtok_qt), the tiled output is bit-identical to the
    few-token kernel on the GGUF bytes and within 2e-5 * rms of the dot4
    output (the same MMVQ formula summed in another order)."""
    L = q3q4.load()
    rng = np.random.default_rng(N + 3 * K)
    Wg = device_blocks(torch, N, K, 11 * N + K)
    Wt = to_tiled(torch, Wg, N, K)
    gg, gt = q3q4.bind_geometry(12, K, N), q3q4.bind_geometry(TILED, K, N)
    for M in (1, 2, 3, 4, 5, 8, 9, 16, 17, 64, 512):
        say(f"case tiled boundary M={M} N={N} K={K}")
        x = dev(torch, activations(rng, M, K))
        yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        yt = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        linear(gg, Wg, x, yg)
        linear(gt, Wt, x, yt)
        torch.cuda.synchronize()
        if M <= 8 and L.sera_q4k_vec_uses_fewtok_qt(TILED, M, N, K) != L.sera_q4k_vec_uses_fewtok(M, N, K):
            assert L.sera_q4k_vec_uses_fewtok_qt(TILED, M, N, K) == 1
            stage = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
            q3q4.quantize_row(x, stage)
            yk = fewtok_once(torch, 12, 0, Wg, stage, M, N, K, 0)
            same_bits(yk, yt, f"boundary M={M} N={N} K={K} (few-token on both layouts)")
            a, b = yt.cpu().numpy().astype(np.float64), yg.cpu().numpy().astype(np.float64)
            rms = float(np.sqrt(np.mean(b * b)))
            err = float(np.max(np.abs(a - b)))
            say(f"  tiled few-token vs GGUF dot4: max|diff| = {err:.3e}, rms = {rms:.3e}")
            assert err <= 2e-5 * rms
        else:
            same_bits(yg, yt, f"boundary M={M} N={N} K={K}")


def test_tiled_lm_head_boundary(torch, linear):
    """The 151936-row LM head at 1, 4, 8 and 16 tokens (persistent grid)."""
    N, K = 151936, 5120
    rng = np.random.default_rng(99)
    Wg = device_blocks(torch, N, K, 4242)
    Wt = to_tiled(torch, Wg, N, K)
    gg, gt = q3q4.bind_geometry(12, K, N), q3q4.bind_geometry(TILED, K, N)
    for M in (1, 3, 4, 8, 16):
        say(f"case tiled LM head M={M}")
        x = dev(torch, activations(rng, M, K))
        yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        yt = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        linear(gg, Wg, x, yg)
        linear(gt, Wt, x, yt)
        torch.cuda.synchronize()
        same_bits(yg, yt, f"LM head M={M}")


@pytest.mark.parametrize("M", [1, 6, 12, 40])
def test_tiled_boundary_against_oracle(torch, linear, M):
    """The tiled geometry against the oracle of the linear (quantize +
    product in the formula of the batch size's path), as the GGUF geometry
    is held elsewhere."""
    N, K = 272, 2048
    rng = np.random.default_rng(500 + M)
    W = oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    xh = activations(rng, M, K)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    Wt = torch.empty(q3q4.weight_bytes(TILED, N, K), dtype=torch.uint8, device="cuda")
    q3q4.weight_upload(TILED, N, K, np.ascontiguousarray(W.reshape(-1)), Wt,
                       torch.empty(1 << 20, dtype=torch.uint8, device="cuda"))
    linear(q3q4.bind_geometry(TILED, K, N), Wt, dev(torch, xh), y)
    torch.cuda.synchronize()
    ref = oracle.linear_reference(W, xh, N, K)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.cpu().numpy().astype(np.float64) - ref)))
    say(f"case tiled boundary oracle M={M}: max|err| = {err:.3e}, rms = {rms:.3e}")
    assert err <= 1e-3 * rms


@pytest.mark.parametrize("M,flags", [(1, q3q4.LIN_RMSNORM), (4, 0), (8, q3q4.LIN_ACCUMULATE), (12, q3q4.LIN_SILU_MUL),
                                     (64, q3q4.LIN_RMSNORM | q3q4.LIN_ACCUMULATE)])
def test_tiled_linear_group(torch, linear, M, flags):
    """q/k/v-like group of three matrices on either layout: same bits."""
    K = 5120
    Ns = [8192, 1024, 1024]
    rng = np.random.default_rng(60 + M)
    say(f"case tiled group M={M} flags={flags}")
    Wg = [device_blocks(torch, n, K, 70 + i) for i, n in enumerate(Ns)]
    Wt = [to_tiled(torch, w, n, K) for w, n in zip(Wg, Ns)]
    x = dev(torch, activations(rng, M, K))
    x2 = dev(torch, activations(rng, M, K)) if flags & q3q4.LIN_SILU_MUL else None
    gamma = dev(torch, (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)) if flags & q3q4.LIN_RMSNORM else None
    y0 = [rng.standard_normal((M, n)).astype(np.float32) for n in Ns]
    outs = []
    for qt, Ws in ((12, Wg), (TILED, Wt)):
        ys = [dev(torch, a) for a in y0]
        q3q4.linear_group([q3q4.bind_geometry(qt, K, n) for n in Ns], Ws, ys, x, x2, gamma, 1e-6, flags)
        torch.cuda.synchronize()
        outs.append(ys)
    for i in range(len(Ns)):
        same_bits(outs[0][i], outs[1][i], f"group[{i}] M={M} flags={flags}")


@pytest.mark.parametrize("N,K", [(304, 256), (1008, 5120)])
def test_tiled_gathered_rows_bit_identical(torch, N, K):
    say(f"case tiled gathered rows N={N} K={K}")
    rng = np.random.default_rng(N * K)
    Wg = device_blocks(torch, N, K, N + K)
    Wt = to_tiled(torch, Wg, N, K)
    ids = rng.integers(0, N, 41).astype(np.int32)
    ids[3] = N + 1
    ids[5] = N - 1
    idd = dev(torch, ids)
    hidden = dev(torch, rng.standard_normal((3, K)).astype(np.float32))
    outs = []
    for qt, W in ((12, Wg), (TILED, Wt)):
        e = torch.full((len(ids), K), 7.25, dtype=torch.float32, device="cuda")
        q3q4.embedding(qt, W, N, K, idd, e)
        lg = torch.full((3 * 13,), 3.0, dtype=torch.float32, device="cuda")
        q3q4.candidate_logits(qt, W, N, K, hidden, idd[:39], 13, lg)
        torch.cuda.synchronize()
        outs.append((e.cpu().numpy(), lg.cpu().numpy()))
    (eg, lgg), (et, lgt) = outs
    assert np.array_equal(eg.view(np.uint32), et.view(np.uint32))
    assert np.array_equal(lgg.view(np.uint32), lgt.view(np.uint32))
    ref = oracle.dequant(Wg.cpu().numpy(), N, K)
    assert np.array_equal(et[0].view(np.uint32), ref[ids[0]].view(np.uint32))
    assert np.all(et[3] == 7.25) and np.isnan(lgt[3])


def test_tiled_group_gate_up_two_tokens(torch, linear):
    """gate and up at 2 tokens: on the tiled layout both run the few-token
    kernel (the GGUF rule would group them on dot4). The group's outputs are
    bit-identical to one boundary call per matrix on the same tiled bytes,
    and with SERA_LIN_ACCUMULATE add exactly that product."""
    N, K, M = 25600, 5120, 2
    rng = np.random.default_rng(77)
    assert q3q4.load().sera_q4k_vec_uses_fewtok_qt(TILED, M, N, K) == 1
    Wt = [to_tiled(torch, device_blocks(torch, N, K, 90 + i), N, K) for i in range(2)]
    geo = q3q4.bind_geometry(TILED, K, N)
    x = dev(torch, activations(rng, M, K))
    say("case tiled group gate/up M=2")
    ref = []
    for w in Wt:
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        linear(geo, w, x, y)
        ref.append(y)
    ys = [torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda") for _ in Wt]
    q3q4.linear_group([geo, geo], Wt, ys, x)
    torch.cuda.synchronize()
    for a, b in zip(ys, ref):
        same_bits(a, b, "group vs boundary")
    y0 = [rng.standard_normal((M, N)).astype(np.float32) for _ in Wt]
    ya = [dev(torch, a) for a in y0]
    q3q4.linear_group([geo, geo], Wt, ya, x, None, None, 0.0, q3q4.LIN_ACCUMULATE)
    torch.cuda.synchronize()
    for a, b, c in zip(ya, ref, y0):
        want = (torch.from_numpy(c).cuda() + b)
        same_bits(a, want, "group accumulate")


@pytest.mark.parametrize("N,K", [(16, 256), (48, 768), (272, 2304)])
def test_tiled_small_matrices_boundary(torch, linear, N, K):
    """One to 17 tiles: the dot4 kernel's shifted last tile, the MMQ row
    clamp and the few-token row clamp all stay inside whole 16-row tiles;
    every batch size is bit-identical to the GGUF bytes."""
    rng = np.random.default_rng(N * 7 + K)
    Wg = device_blocks(torch, N, K, 5 * N + K)
    Wt = to_tiled(torch, Wg, N, K)
    gg, gt = q3q4.bind_geometry(12, K, N), q3q4.bind_geometry(TILED, K, N)
    for M in (1, 2, 3, 5, 8, 9, 16, 33, 100):
        say(f"case tiled small boundary N={N} K={K} M={M}")
        x = dev(torch, activations(rng, M, K))
        yg = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        yt = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        linear(gg, Wg, x, yg)
        linear(gt, Wt, x, yt)
        torch.cuda.synchronize()
        same_bits(yg, yt, f"small boundary N={N} K={K} M={M}")


@pytest.mark.parametrize("N,K", [(16, 256), (272, 2304), (1008, 5120)])
def test_tiled_dequant_row_major(torch, N, K):
    """sera_q4k_dequantize_qt on the tiled bytes gives the row-major matrix
    the oracle dequantizes from the GGUF bytes, bit for bit; on GGUF bytes
    the same as sera_q4k_dequantize."""
    say(f"case tiled dequant N={N} K={K}")
    Wg = device_blocks(torch, N, K, 3 * N + K)
    Wt = to_tiled(torch, Wg, N, K)
    ref = oracle.dequant(Wg.cpu().numpy(), N, K)
    for qt, W in ((TILED, Wt), (12, Wg)):
        out = torch.full((N, K), float("nan"), dtype=torch.float32, device="cuda")
        q3q4.dequantize_matrix(qt, W, N, K, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32)), qt
