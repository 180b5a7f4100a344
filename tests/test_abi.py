"""Host-side checks of the C ABI (no GPU): the library loads, exports every
function that include/*.h declares, and the host-only argument handling
follows the reference's contracts (src/q3_q4_linear.cu:48-91,93-228)."""
import ctypes
import os
import subprocess

import pytest

import q3q4


@pytest.fixture(scope="module")
def L():
    return q3q4.load()


def test_library_exports_every_header_symbol(L):
    names = q3q4.header_symbols()
    assert len(names) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", q3q4.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(L, n)


def test_reference_boundary_symbols_present():
    """The seven entry points of src/q3_q4_linear.h:65-116 that a caller binds."""
    names = set(q3q4.header_symbols())
    for n in ["q3_q4_linear_bind_geometry", "q3_cuda_q4k_linear_init",
              "q3_cuda_q4k_linear_workspace_bytes", "q3_cuda_q4k_linear_set_workspace",
              "q3_cuda_q4k_linear_path_for_batch", "q3_cuda_q4k_linear",
              "q3_cuda_q4k_linear_read_stats"]:
        assert n in names


def test_struct_layouts_match_reference():
    assert ctypes.sizeof(q3q4.Stats) == 3 * 8 + 6 * 8
    assert ctypes.sizeof(q3q4.Geometry) == 24
    assert q3q4.Geometry.weight_bytes.offset == 16


@pytest.mark.parametrize("qtype,dim0,dim1,wbytes", [
    (12, 5120, 25600, 73_728_000),     # gate/up
    (12, 25600, 5120, 73_728_000),     # down
    (12, 5120, 151936, 437_575_680),   # LM head
    (14, 5120, 1024, 1024 * 20 * 210), # Q6_K: 210-byte blocks, run by the same call
    (268, 5120, 151936, 437_575_680),  # Q4_K tiled: the same bytes reordered
])
def test_bind_geometry(qtype, dim0, dim1, wbytes):
    g = q3q4.bind_geometry(qtype, dim0, dim1)
    assert (g.M, g.N, g.K, g.qtype, g.weight_bytes) == (0, dim1, dim0, qtype, wbytes)


@pytest.mark.parametrize("qtype,dim0,dim1,msg", [
    (2, 5120, 100, "not Q4_K/Q6_K"),
    (12, 0, 100, "degenerate"),
    (12, 512, 0, "degenerate"),
    (12, 5000, 100, "multiple of 256"),
    (12, 2 ** 31 + 256, 4, "exceeds int32"),
    (268, 5120, 100, "divisible by 16"),
])
def test_bind_geometry_errors(qtype, dim0, dim1, msg):
    with pytest.raises(q3q4.Q3Q4Error, match=msg):
        q3q4.bind_geometry(qtype, dim0, dim1)


def test_tiled_layout_host_statement_and_sizes(L):
    """q3q4.q4k_tiled_bytes against the offset formula written block by
    block, and sera_weight_bytes for the tiled qtype (pure host)."""
    import numpy as np
    rng = np.random.default_rng(5)
    for N, K in ((16, 256), (48, 768), (32, 2304)):
        W = rng.integers(0, 256, N * K // 256 * 144, dtype=np.uint8)
        want = np.empty_like(W)
        for r in range(N):
            for b in range(K // 256):
                o = ((r // 16) * (K // 256) + b) * 2304 + (r % 16) * 144
                want[o:o + 144] = W[(r * (K // 256) + b) * 144:(r * (K // 256) + b + 1) * 144]
        assert np.array_equal(q3q4.q4k_tiled_bytes(W, N, K), want)
        assert L.sera_weight_bytes(q3q4.QTYPE_Q4K_TILED, N, K) == W.size
    assert L.sera_weight_bytes(q3q4.QTYPE_Q4K_TILED, 40, 256) == 0


def test_tiled_kernel_calls_reject_bad_layouts(L):
    """The _qt kernel calls check the qtype and the tiled row count on the
    host, before any launch."""
    d = ctypes.c_void_p(256)
    assert L.sera_q4k_mmvq_qt(q3q4.QTYPE_Q4K_TILED, d, d, d, 1, 40, 256, 0, None) == -1
    assert b"16" in L.sera_q4k_last_error()
    assert L.sera_q4k_mmvq_qt(14, d, d, d, 1, 48, 256, 0, None) == -1
    assert b"qtype" in L.sera_q4k_last_error()
    assert L.sera_q4k_mmq_qt(q3q4.QTYPE_Q4K_TILED, d, d, d, None, 16, 40, 256, 1, None) == -1
    assert L.sera_q4k_fewtok_qt(q3q4.QTYPE_Q4K_TILED, 0, d, d, d, None, None, 4, 40, 256, 0, 0, None) == -1
    assert L.sera_q4k_mmq_streamk_qt(q3q4.QTYPE_Q4K_TILED, d, d, d, d, ctypes.c_void_p(512), 64, 40, 5120, 8,
                                     None) == -1


def test_bind_geometry_null_out(L):
    assert not L.q3_q4_linear_bind_geometry(12, 256, 4, None, None, 0)


def test_path_for_batch(L):
    assert L.q3_cuda_q4k_linear_path_for_batch(1) == b"MMVQ"
    assert L.q3_cuda_q4k_linear_path_for_batch(8) == b"MMVQ"
    assert L.q3_cuda_q4k_linear_path_for_batch(9) == b"MMQ"
    assert L.q3_cuda_q4k_linear_path_for_batch(2048) == b"MMQ"


# Runs in a child process that has initialised nothing: with the library
# initialised (as in a process that ran GPU tests first) the call with
# placeholder pointers would pass the init check and launch on them.
_UNINIT_CHILD = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import q3q4
L = q3q4.load()
err = ctypes.create_string_buffer(256)
assert not L.q3_cuda_q4k_linear_init(-1, 16, 1024, 5120, err, 256)
assert b"invalid device" in err.value, err.value
g = q3q4.bind_geometry(12, 256, 4)
st = q3q4.Stats()
# null arguments are rejected before anything else
assert not L.q3_cuda_q4k_linear(ctypes.byref(g), None, None, 1, None, None, ctypes.byref(st), err, 256)
assert b"null argument" in err.value, err.value
# nothing initialised in this process
dummy = ctypes.c_void_p(16)
assert not L.q3_cuda_q4k_linear(ctypes.byref(g), dummy, dummy, 1, dummy, None, ctypes.byref(st), err, 256)
assert b"not initialized" in err.value, err.value
assert not L.q3_cuda_q4k_linear_set_workspace(None, 0, err, 256)
assert b"workspace too small" in err.value, err.value
print("ok")
"""


def test_host_error_paths_without_device():
    import sys as _sys
    pkg = os.path.dirname(q3q4.__file__)
    r = subprocess.run([_sys.executable, "-c", _UNINIT_CHILD, pkg], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_kernel_entry_points_validate_on_host(L):
    d = ctypes.c_void_p(256)
    assert L.sera_q4k_mmvq(d, d, d, 9, 128, 256, 0, None) == -1
    assert b"outside 1..8" in L.sera_q4k_last_error()
    assert L.sera_q4k_mmvq(d, d, d, 1, 128, 256, 3, None) == -1
    assert L.sera_q4k_dense(d, d, d, 16, 128, 300, None, 0) == -1
    assert b"multiple of 256" in L.sera_q4k_last_error()
    assert L.sera_q4k_dense(None, d, d, 16, 128, 256, None, 0) == -1
    assert L.sera_q4k_dense(d, ctypes.c_void_p(258), d, 16, 128, 256, None, 0) == -1
    assert b"16-byte aligned" in L.sera_q4k_last_error()
    assert L.sera_q4k_mmq(d, d, d, None, 64, 128, 1024, 2, None) == -1
    assert b"partial" in L.sera_q4k_last_error()
    assert L.sera_q4k_set_arena(ctypes.c_void_p(100), 1024) == -1
    assert L.sera_q4k_fewtok(0, d, d, d, None, None, 9, 128, 256, 0, 0, None) == -1
    assert b"outside 1..8" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(1, d, d, d, None, None, 17, 128, 256, 0, 0, None) == -1
    assert b"outside 1..16" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(2, d, d, d, None, None, 4, 128, 256, 0, 0, None) == -1
    assert L.sera_q4k_fewtok(0, d, d, d, None, None, 4, 128, 300, 0, 0, None) == -1
    assert L.sera_q4k_fewtok(0, d, ctypes.c_void_p(264), d, None, None, 4, 128, 256, 0, 0, None) == -1
    assert b"16-byte aligned" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(0, d, d, d, None, None, 4, 128, 5120, 41, 0, None) == -1
    assert b"chunk" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(1, d, d, d, None, None, 12, 128, 5120, 21, 0, None) == -1
    assert b"chunk" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(0, d, d, d, None, None, 4, 128, 5120, 3, 0, None) == -1
    assert b"slots" in L.sera_q4k_last_error()
    # the bench kernel loop refuses scratch shorter than its path writes,
    # before any launch: the tail schedule's slots and counters, split-K sums
    ws = (ctypes.c_void_p * 1)(256)
    avg, tot = ctypes.c_double(), ctypes.c_double()
    need = q3q4.mmq_tail_slot_floats(512, 1024, 0, 4) + L.sera_q4k_mmq_tiles(512, 1024)
    assert L.sera_q4k_bench_kernel(15, ws, 1, d, d, d, need - 1, 512, 1024, 5120, 4, None, 0, 1,
                                   ctypes.byref(avg), ctypes.byref(tot)) == -2
    assert f"needs {need} floats".encode() in L.sera_q4k_last_error()
    assert L.sera_q4k_bench_kernel(1, ws, 1, d, d, None, 0, 64, 128, 1024, 2, None, 0, 1,
                                   ctypes.byref(avg), ctypes.byref(tot)) == -2


def test_offset_and_grid_limits_rejected_on_host(L):
    """Shapes past the kernels' 32-bit stage offsets (Mpad*K >= 2^31), the
    quantizers' 65535-row grid or K > 2^24 fail with a message before any
    launch (the reference indexes its quantizers in int64,
    cuda/mmq/quantize.cu:9,28; here they are rejected, never wrapped)."""
    d = ctypes.c_void_p(256)
    # 60000 tokens x K=40960: Mpad*K = 60032*40960 > 2^31
    assert L.sera_q4k_dense(d, d, d, 60000, 128, 40960, None, 0) == -1
    assert b"2^31" in L.sera_q4k_last_error()
    # just under the bound is not rejected by the shape check (it fails later: no arena)
    assert L.sera_q4k_dense(d, d, d, 52416, 128, 40960, None, 0) == -1
    assert b"arena" in L.sera_q4k_last_error()
    # 84000 tokens: more rows than one quantize grid holds
    assert L.sera_q4k_dense(d, d, d, 84000, 128, 5120, None, 0) == -1
    assert b"65535" in L.sera_q4k_last_error()
    big_k = (1 << 24) + 256
    assert L.sera_q4k_dense_vec(d, d, d, 1, 128, big_k, None, 0) == -1
    assert b"exceeds" in L.sera_q4k_last_error()
    assert L.sera_q4k_dense_vec_static(d, d, d, 1, 128, big_k, None) == -1
    assert b"exceeds" in L.sera_q4k_last_error()
    assert L.sera_q8_1_quantize_mmq(d, 60000, 40960, d, None) == -1
    assert b"2^31" in L.sera_q4k_last_error()
    assert L.sera_q8_1_quantize_row(d, 1, big_k, d, None) == -1
    assert L.sera_q4k_mmq_qt(12, d, d, d, d, 60000, 128, 40960, 1, None) == -1
    assert b"2^31" in L.sera_q4k_last_error()
    assert L.sera_q4k_mmq_streamk_qt(12, d, d, d, d, d, 60000, 128, 40960, 8, None) == -1
    assert b"2^31" in L.sera_q4k_last_error()
    assert L.sera_q4k_fewtok(1, d, d, d, None, None, 16, 128, big_k, 0, 0, None) == -1
    assert b"exceeds" in L.sera_q4k_last_error()
    assert L.sera_q6k_dense(14, d, d, d, 60000, 128, 40960, None, 0) == -1
    assert b"2^31" in L.sera_q4k_last_error()
    assert L.sera_q8_1_quantize_mmq_d4(d, 60000, 40960, d, None) == -1
    assert b"2^31" in L.sera_q4k_last_error()


def test_fewtok_plan(L):
    """Planned chunks cover K in at most 20 super-blocks each; explicit
    chunks go up to 40 (20 above 8 tokens); row groups cover N."""
    for M in range(1, 17):
        for N, K in ((1024, 5120), (5120, 25600), (25600, 5120), (151936, 5120), (8192, 5120), (5120, 8192),
                     (16, 256), (203, 2304), (100, 128 * 1024)):
            nkb = K // 256
            cmax = 40 if M <= 8 else 20
            s = L.sera_q4k_fewtok_splits(M, N, K, 0)
            assert 1 <= s <= max(16, -(-nkb // 20)), (M, N, K, s)
            chunk = -(-nkb // s)
            assert chunk <= 20 and -(-nkb // chunk) == s, (M, N, K, s)
            g = L.sera_q4k_fewtok_groups(M, N, K)
            assert g in (-(-N // 64), -(-N // 128)), (N, g)     # 4 or 8 waves of 16 rows
            for c in (1, 3, cmax):
                assert L.sera_q4k_fewtok_splits(M, N, K, c) == -(-nkb // c)
    # the tall Qwen3-32B matrices need no split up to 8 tokens
    assert L.sera_q4k_fewtok_splits(8, 25600, 5120, 0) == 1
    assert L.sera_q4k_fewtok_splits(8, 151936, 5120, 0) == 1


def test_stage_layouts_and_workspace_sizing():
    r = q3q4.row_stage_layout(8, 25600)
    assert r["qs"] == 0 and r["ds"] >= 8 * 25600 and r["dsf"] >= r["ds"] + 8 * 800 * 4
    assert r["total"] >= r["dsf"] + 8 * 400 * 16 and r["total"] % 256 == 0
    m = q3q4.mmq_stage_layout(100, 5120)
    assert m["rows"] == 128 and m["ds"] >= 128 * 5120 and m["total"] >= m["ds"] + 128 * 160 * 4
    L = q3q4.load()
    small = L.sera_q4k_arena_bytes(16, 25600, 25600)
    big = L.sera_q4k_arena_bytes(2048, 25600, 25600)
    assert big > small > q3q4.mmq_stage_layout(16, 25600)["total"]
    # every split-K choice for shapes the arena was sized for fits in it
    for M in (9, 16, 64, 100, 512, 2048):
        for N, K in ((1024, 5120), (5120, 25600), (25600, 5120), (151936, 5120)):
            s = q3q4.mmq_splits(M, N, K)
            need = q3q4.mmq_stage_layout(M, K)["total"] + (s * M * N * 4 if s > 1 else 0)
            assert need <= L.sera_q4k_arena_bytes(2048, 151936, 25600), (M, N, K, s)
    # arenas sized down to 16 or 32 tokens hold every split-K choice of the
    # 16- and 32-token tiles, and the stream-K slots of the LM head at 16
    # tokens (P = 2 x 256 CUs on MI355X), so the boundary takes the planned
    # schedule there instead of falling back
    for mt in (16, 32):
        room = L.sera_q4k_arena_bytes(mt, 151936, 25600) - (256 << 10)
        for M in sorted({10, 13, 16, mt}):
            for N, K in ((1024, 5120), (5120, 25600), (25600, 5120), (151936, 5120), (8192, 5120)):
                s = q3q4.mmq_splits(M, N, K)
                need = q3q4.mmq_stage_layout(M, K)["total"] + (s * M * N * 4 if s > 1 else 0)
                assert need <= room, (mt, M, N, K, s)
        slots = 2 * 512 * L.sera_q4k_mmq_slot_floats(16) * 4
        assert L.sera_q4k_mmq_slot_floats(16) == 32 * 256   # the paired tile keeps 32 MFMA rows
        assert q3q4.mmq_stage_layout(16, 5120)["total"] + slots <= room, mt
    # and every few-token split, for arenas sized down to the batch (row
    # stage on the MMVQ path up to 8 tokens, MMQ stage on the MMQ path up
    # to 16)
    for mt in (1, 4, 8, 9, 12, 16, 2048):
        for M in range(1, min(mt, 16) + 1):
            for N, K in ((1024, 5120), (5120, 25600), (25600, 5120), (151936, 5120), (100, 128 * 1024)):
                s = L.sera_q4k_fewtok_splits(M, N, K, 0)
                stage = q3q4.mmq_stage_layout(M, K)["total"]
                if M <= 8:
                    stage = max(stage, q3q4.row_stage_layout(M, K)["total"])
                need = stage + (s * M * N * 4 if s > 1 else 0)
                assert need <= L.sera_q4k_arena_bytes(mt, 151936, 128 * 1024) - (256 << 10), (mt, M, N, K, s)


def test_mmq_split_rule_picks_measured_best():
    """The split-K cost model picks, on Qwen3-32B shapes, the split count
    that measured fastest on MI355X (q, k/v, o, gate/up, down at 64-2048
    tokens; 128-row tiles where 256-row ones would leave at most 64), and
    keeps every choice within its bounds: at least 2 super-blocks per split,
    at most 2048 workgroups, 16 splits at most."""
    measured_best = {(64, 8192, 5120): 4, (128, 8192, 5120): 4, (512, 8192, 5120): 1,
                     (512, 1024, 5120): 4, (1024, 1024, 5120): 4, (256, 1024, 5120): 8,
                     (256, 5120, 8192): 8, (1024, 5120, 8192): 4,
                     (512, 25600, 5120): 1, (2048, 25600, 5120): 1,
                     (128, 5120, 25600): 16, (512, 5120, 25600): 8, (1024, 5120, 25600): 4,
                     (2048, 5120, 25600): 2}
    for (M, N, K), s in measured_best.items():
        assert q3q4.mmq_splits(M, N, K) == s, (M, N, K)
    L = q3q4.load()
    for M in (9, 16, 17, 32, 33, 64, 100, 256, 777, 2048, 8192):
        for N in (256, 1000, 5120, 25600, 151936):
            for K in (256, 512, 2304, 5120, 25600):
                s = q3q4.mmq_splits(M, N, K)
                assert s in (1, 2, 4, 8, 16), (M, N, K, s)
                if s > 1:
                    assert K // 256 // s >= 2 and L.sera_q4k_mmq_tiles(M, N) * s <= 2048, (M, N, K, s)


def test_kernel_launch_counts(L):
    """quantize + matmul (+ the split-K reduce when an MMQ launch splits K)."""
    assert L.sera_q4k_kernel_launches(1, 25600, 5120) == 2          # dot4 MMVQ
    for N, K in ((25600, 5120), (5120, 25600)):                     # few-token kernel,
        assert L.sera_q4k_kernel_launches(8, N, K) == 2             # split K summed inside
    assert L.sera_q4k_kernel_launches(9, 5120, 25600) == 2          # few-token kernel, MMQ formula
    assert L.sera_q4k_kernel_launches(10, 25600, 5120) == 2         # few-token kernel on a tall matrix
    assert L.sera_q4k_kernel_launches(16, 5120, 25600) == 2         # few-token kernel on a long K
    assert L.sera_q4k_kernel_launches(10, 8192, 5120) == 3          # paired MMQ tile, split K
    assert L.sera_q4k_kernel_launches(512, 25600, 5120) == 2        # MMQ, enough tiles
    assert L.sera_q4k_kernel_launches(0, 5120, 25600) == 0
    assert L.sera_q4k_kernel_launches(4, 5120, 300) == 0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits non-zero with a message
    (before anything touches a GPU)."""
    import sys as _sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([_sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_vec_dispatch_rule(L):
    """The MMVQ path's kernel choice by shape: the few-token kernel on tall
    matrices from 3 tokens, on 4096-16383 rows from 6 (from 5 with K >=
    16384), never below 4096 rows."""
    f = L.sera_q4k_vec_uses_fewtok
    assert [f(M, 25600, 5120) for M in range(1, 9)] == [0, 0, 1, 1, 1, 1, 1, 1]
    assert [f(M, 151936, 5120) for M in range(1, 9)] == [0, 0, 1, 1, 1, 1, 1, 1]
    for N in (5120, 8192):
        assert [f(M, N, 25600) for M in range(1, 9)] == [0, 0, 0, 0, 1, 1, 1, 1]
        assert [f(M, N, 5120) for M in range(1, 9)] == [0, 0, 0, 0, 0, 1, 1, 1]
    assert [L.sera_q4k_mmvq_rows_per_tile(M, 25600, 5120) for M in range(1, 9)] == [4, 4, 8, 8, 4, 2, 2, 2]
    assert [L.sera_q4k_mmvq_rows_per_tile(M, 5120, 25600) for M in range(1, 9)] == [4, 8, 8, 8, 4, 2, 2, 2]
    assert L.sera_q4k_mmvq_rows_per_tile(2, 151936, 5120) == 8
    assert [L.sera_q4k_mmvq_rows_per_tile(M, 8192, 5120) for M in range(1, 6)] == [4, 4, 8, 8, 4]
    assert [L.sera_q4k_mmvq_rows_per_tile(M, 5120, 8192) for M in range(1, 6)] == [4, 4, 4, 4, 4]
    assert [f(M, 1024, 5120) for M in range(1, 9)] == [0] * 8
    assert f(0, 25600, 5120) == 0 and f(9, 25600, 5120) == 0


def test_vec_dispatch_rule_tiled_layout(L):
    """On the tiled layout the few-token kernel takes over earlier: tall
    matrices from 2 tokens, down (K 25600) from 3, q (8192 rows) from 5, o
    (5120 rows, K 8192) from 6, k/v never; qtype 12 answers as the GGUF
    query and other qtypes 0."""
    T = q3q4.QTYPE_Q4K_TILED
    f = L.sera_q4k_vec_uses_fewtok_qt
    assert [f(T, M, 25600, 5120) for M in range(1, 9)] == [0, 1, 1, 1, 1, 1, 1, 1]
    assert [f(T, M, 151936, 5120) for M in range(1, 9)] == [0, 1, 1, 1, 1, 1, 1, 1]
    assert [f(T, M, 5120, 25600) for M in range(1, 9)] == [0, 0, 1, 1, 1, 1, 1, 1]
    assert [f(T, M, 8192, 5120) for M in range(1, 9)] == [0, 0, 0, 0, 1, 1, 1, 1]
    assert [f(T, M, 5120, 8192) for M in range(1, 9)] == [0, 0, 0, 0, 0, 1, 1, 1]
    assert [f(T, M, 1024, 5120) for M in range(1, 9)] == [0] * 8
    for M in range(0, 10):
        for N, K in ((25600, 5120), (5120, 25600), (8192, 5120), (1024, 5120)):
            assert f(12, M, N, K) == L.sera_q4k_vec_uses_fewtok(M, N, K)
    assert f(14, 4, 25600, 5120) == 0 and f(T, 9, 25600, 5120) == 0


def test_q6k_mmq_token_tile_rule(L):
    """The Q6_K tile kernel takes 64 tokens per tile when the padded rows
    divide by 64 and the 64-token grid holds >= 1024 (tile, super-block)
    pairs, else 32; the built-in K split counts the tiles of that choice
    (down 5120 x 25600 at 512 tokens: 320 tiles, 4 splits)."""
    f = L.sera_q6k_mmq_tile_tokens
    assert f(512, 5120, 25600) == 64 and f(2048, 5120, 25600) == 64 and f(64, 5120, 25600) == 64
    assert f(512, 151936, 5120) == 64 and f(64, 151936, 5120) == 64
    assert f(512, 1024, 5120) == 64 and f(2048, 1024, 5120) == 64     # 64 x 20, 256 x 20 pairs
    assert f(256, 1024, 5120) == 32 and f(64, 1024, 5120) == 32       # 32 x 20, 8 x 20 pairs
    assert f(100, 2046, 8192) == 64 and f(128, 2048, 8192) == 64      # 2 x 16 x 32 = 1024
    assert f(96, 5120, 25600) == 32 and f(40, 77, 2304) == 32 and f(8, 5120, 25600) == 32
    assert L.sera_q6k_mmq_splits_for(512, 5120, 25600) == 4
    assert L.sera_q6k_mmq_splits_for(2048, 5120, 25600) == 1
    assert L.sera_q6k_mmq_splits_for(256, 5120, 25600) == 8


def test_q6k_vec_dispatch_rule(L):
    """Q6_K on the MMVQ path: the tile kernel on tall matrices from 4 tokens,
    on 4096-16383 rows from 6 (GGUF bytes) or 7 (split layout), one token
    earlier when K >= 16384 (down), never below 4096 rows; launch counts
    follow."""
    f = L.sera_q6k_vec_uses_tile
    assert [f(M, 151936, 5120) for M in range(1, 9)] == [0, 0, 0, 1, 1, 1, 1, 1]
    assert [f(M, 8192, 5120) for M in range(1, 9)] == [0, 0, 0, 0, 0, 1, 1, 1]
    assert [f(M, 5120, 25600) for M in range(1, 9)] == [0, 0, 0, 0, 1, 1, 1, 1]   # down: tail schedule
    assert [f(M, 1024, 5120) for M in range(1, 9)] == [0] * 8
    g = L.sera_q6k_vec_uses_tile_qt
    S = q3q4.QTYPE_Q6K_SPLIT
    for N, K in ((151936, 5120), (5120, 25600), (8192, 5120), (1024, 5120)):
        assert [g(14, M, N, K) for M in range(0, 10)] == [f(M, N, K) for M in range(0, 10)]
    assert [g(S, M, 151936, 5120) for M in range(1, 9)] == [0, 0, 0, 1, 1, 1, 1, 1]
    assert [g(S, M, 8192, 5120) for M in range(1, 9)] == [0, 0, 0, 0, 0, 0, 1, 1]
    assert [g(S, M, 5120, 25600) for M in range(1, 9)] == [0, 0, 0, 0, 0, 1, 1, 1]
    assert [g(S, M, 1024, 5120) for M in range(1, 9)] == [0] * 8
    assert g(12, 8, 151936, 5120) == 0 and g(S, 9, 151936, 5120) == 0
    assert L.sera_q6k_kernel_launches_qt(S, 6, 8192, 5120) == 2      # MMVQ on the split layout
    assert L.sera_q6k_kernel_launches_qt(14, 6, 8192, 5120) == L.sera_q6k_kernel_launches(6, 8192, 5120)
    assert L.sera_q6k_kernel_launches(8, 1024, 5120) == 2          # MMVQ
    assert L.sera_q6k_kernel_launches(4, 5120, 25600) == 2         # MMVQ
