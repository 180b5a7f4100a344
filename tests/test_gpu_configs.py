"""Every BASELINE configuration at its full Qwen3-32B shape, through the
q3_q4_linear boundary (the reference runs its parity at the production
shape too: tests/test_q3_q4_linear.cu:279-408 on the 25600 x 5120 gate).

Weights are seeded N(0, 0.02) fp32 matrices quantized to Q4_K on the device
(sera_q4k_quantize, bit-exact with the reference quantizer); activations are
N(0, 1), with 1% of channels x20 for the decode sweep (config 2). Outputs are
compared with the path-faithful oracle (MMVQ formula at M <= 8, MMQ formula
above) within max |err| <= 1e-3 * rms(ref): all outputs where the oracle is
cheap (config 1), sampled weight rows elsewhere (Q4_K rows are independent,
so a sampled row is a full check of that row).

Config 5 runs the whole decode pass (64 layers x 7 projections + the LM
head, 449 calls on ~18 GB of resident weights) and checks it bit-identical
to the same calls issued one at a time, eagerly and as a HIP graph replay,
with oracle checks on sampled rows of four layers.
"""
import ctypes
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3
SHAPES = {"q": (8192, 5120), "k": (1024, 5120), "v": (1024, 5120), "o": (5120, 8192),
          "gate": (25600, 5120), "up": (25600, 5120), "down": (5120, 25600), "lm_head": (151936, 5120)}


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


def quantized(torch, N, K, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    wf = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    Wd = torch.empty((N, K // 256 * 144), dtype=torch.uint8, device="cuda")
    q3q4.quantize_weights(wf, Wd)
    del wf
    return Wd


def activations(rng, M, K, outliers):
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        ch = rng.choice(K, int(np.ceil(0.01 * K)), replace=False)
        x[:, ch] *= 20.0
    return x


def check_close(y, ref, what):
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y.astype(np.float64) - ref)))
    say(f"  {what}: max|err| = {err:.3e}, rms = {rms:.3e}, ratio = {err / max(rms, 1e-30):.2e}")
    assert np.all(np.isfinite(y)), what
    assert err <= TOL * rms, what


def run_and_check(torch, linear, Wd, x, N, K, nrows, seed, what):
    M = x.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    linear(q3q4.bind_geometry(12, K, N), Wd, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    if nrows >= N:
        rows = np.arange(N)
    else:
        rows = np.sort(np.random.default_rng(seed).choice(N, nrows, replace=False))
    W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = oracle.linear_reference(W, x, len(rows), K)
    check_close(y.cpu().numpy()[:, rows], ref, f"{what} ({len(rows)} of {N} rows)")
    return y


def test_config1_q_proj_m1_all_outputs(torch, linear):
    """Config 1: M=1, 8192 x 5120 (q_proj), seed 0 weights, every output."""
    say("case config 1: q_proj 8192x5120 M=1")
    N, K = SHAPES["q"]
    Wd = quantized(torch, N, K, 0)
    x = activations(np.random.default_rng(1), 1, K, False)
    run_and_check(torch, linear, Wd, x, N, K, N, 0, "config 1 q_proj M=1")


@pytest.mark.parametrize("name", ["gate", "down"])
def test_config2_decode_sweep(torch, linear, name):
    """Config 2: M in {1, 2, 4, 8} on gate/up 5120->25600 and down
    25600->5120 with 1% outlier channels x20; the row-layout Q8_1 stage of
    each batch bit-exact with the oracle."""
    N, K = SHAPES[name]
    Wd = quantized(torch, N, K, 100 if name == "down" else 0)
    rng = np.random.default_rng(2)
    for M in (1, 2, 4, 8):
        L = q3q4.load()
        kern = "few-token" if L.sera_q4k_vec_uses_fewtok(M, N, K) else "dot4"
        say(f"case config 2: {name} {N}x{K} M={M} ({kern})")
        x = activations(rng, M, K, True)
        run_and_check(torch, linear, Wd, x, N, K, 512, M, f"config 2 {name} M={M} ({kern})")
        st = torch.empty(q3q4.row_stage_layout(M, K)["total"], dtype=torch.uint8, device="cuda")
        q3q4.quantize_row(torch.from_numpy(x).cuda(), st)
        torch.cuda.synchronize()
        lay = q3q4.row_stage_layout(M, K)
        b = st.cpu().numpy()
        qs = b[lay["qs"]:lay["qs"] + M * K].view(np.int8).reshape(M, K)
        ds = b[lay["ds"]:lay["ds"] + M * K // 32 * 4].view(np.uint32).reshape(M, K // 32)
        eq, ed, es = oracle.q8_1_row(x)
        assert np.array_equal(qs, eq)
        assert np.array_equal((ds & 0xFFFF).astype(np.uint16), ed)
        assert np.array_equal((ds >> 16).astype(np.uint16), es)


@pytest.mark.parametrize("name", ["q", "k", "v", "o", "gate", "up", "down"])
def test_config3_prefill_m512(torch, linear, name):
    """Config 3: M=512 on each of the seven projections of one layer."""
    N, K = SHAPES[name]
    say(f"case config 3: {name} {N}x{K} M=512 (schedule "
        f"{'stream-K' if q3q4.load().sera_q4k_mmq_schedule(512, N, K) == 1 else 'tiles/split-K'})")
    Wd = quantized(torch, N, K, 300 + list(SHAPES).index(name))
    x = activations(np.random.default_rng(3), 512, K, False)
    run_and_check(torch, linear, Wd, x, N, K, 128, 3, f"config 3 {name} M=512")


@pytest.mark.parametrize("name", ["gate", "down"])
def test_config4_packed_prefix_m2048(torch, linear, name):
    """Config 4: the packed shared-prefix batch, M=2048 rows (1536 prefix +
    16 x 32 suffix tokens; row order is immaterial to the product)."""
    N, K = SHAPES[name]
    say(f"case config 4: {name} {N}x{K} M=2048")
    Wd = quantized(torch, N, K, 400 + list(SHAPES).index(name))
    x = activations(np.random.default_rng(4), 2048, K, False)
    run_and_check(torch, linear, Wd, x, N, K, 32, 4, f"config 4 {name} M=2048")


def test_config4_lm_head_m16(torch, linear):
    """Config 4: the LM head 5120 -> 151936 at M=16 (one candidate row per
    branch), Q4_K."""
    N, K = SHAPES["lm_head"]
    say(f"case config 4: lm_head {N}x{K} M=16")
    Wd = quantized(torch, N, K, 500)
    x = activations(np.random.default_rng(5), 16, K, False)
    run_and_check(torch, linear, Wd, x, N, K, 1024, 5, "config 4 lm_head M=16")


def test_config5_decode_pass(torch, linear):
    """Config 5: one token through 64 layers x 7 projections + the LM head
    (449 calls, every weight resident). The pass issued from C back to back
    (sera_q4k_bench_stream), and the same pass captured into a HIP graph and
    replayed, equal the per-call results bit for bit; sampled rows of layers
    0, 21, 42 and 63 and of the LM head match the oracle."""
    order = ["q", "k", "v", "o", "gate", "up", "down"]
    L = q3q4.load()
    rng = np.random.default_rng(6)
    calls = []
    say("case config 5: building 448 projection weights + LM head")
    for layer in range(64):
        for name in order:
            N, K = SHAPES[name]
            calls.append((layer, name, quantized(torch, N, K, 10_000 + 7 * layer + order.index(name)),
                          activations(rng, 1, K, False)))
        if layer % 16 == 15:
            torch.cuda.synchronize()
            say(f"  weights of layers 0-{layer} ready")
    calls.append((64, "lm_head", quantized(torch, *SHAPES["lm_head"], 99_999),
                  activations(rng, 1, SHAPES["lm_head"][1], False)))
    torch.cuda.synchronize()
    n = len(calls)
    assert n == 449
    geos = {nm: q3q4.bind_geometry(12, SHAPES[nm][1], SHAPES[nm][0]) for nm in SHAPES}
    xs = [torch.from_numpy(c[3]).cuda() for c in calls]
    say("case config 5: per-call reference pass")
    ref = []
    for (layer, name, Wd, _), x in zip(calls, xs):
        y = torch.empty((1, SHAPES[name][0]), dtype=torch.float32, device="cuda")
        linear(geos[name], Wd, x, y)
        ref.append(y)
    torch.cuda.synchronize()
    g_arr = (ctypes.c_void_p * n)(*[ctypes.addressof(geos[c[1]]) for c in calls])
    w_arr = (ctypes.c_void_p * n)(*[c[2].data_ptr() for c in calls])
    x_arr = (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs])
    m_arr = (ctypes.c_size_t * n)(*([1] * n))
    side = torch.cuda.Stream()
    for use_graph in (0, 1):
        say(f"case config 5: 449-call pass from C (graph={use_graph})")
        ys = [torch.full_like(r, float("nan")) for r in ref]
        y_arr = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        ms = ctypes.c_double()
        strm = ctypes.c_void_p(side.cuda_stream)
        torch.cuda.synchronize()
        rc = L.sera_q4k_bench_stream(g_arr, w_arr, x_arr, m_arr, y_arr, n, strm, 0, 1, use_graph,
                                     ctypes.byref(ms))
        assert rc == 0, L.sera_q4k_last_error().decode()
        torch.cuda.synchronize()
        bad = [i for i in range(n) if not torch.equal(ys[i], ref[i])]
        say(f"  {n - len(bad)} of {n} outputs bit-identical to the per-call pass ({ms.value:.3f} ms)")
        assert not bad, f"calls differ: {bad[:8]}"
    for i, (layer, name, Wd, x) in enumerate(calls):
        if layer not in (0, 21, 42, 63, 64):
            continue
        N, K = SHAPES[name]
        rows = np.sort(np.random.default_rng(i).choice(N, 64, replace=False))
        W = Wd[torch.from_numpy(rows).cuda()].cpu().numpy()
        check_close(ref[i].cpu().numpy()[:, rows], oracle.linear_reference(W, x, 64, K),
                    f"config 5 layer {layer} {name}")
    del calls, xs, ref
    torch.cuda.empty_cache()
