"""Python binding of libsera_q4k.so (ctypes), the host-side mirror of the
reference's q3_q4_linear interface used by the tests and the bench driver.

The C ABI is the product (include/q3_q4_linear.h, include/sera_q4k.h); this
module only declares its signatures and wraps device buffers that PyTorch
allocates. Import torch before loading the library so that both use the one
HIP runtime in the process (same soname, libamdhip64.so.7).

There is no CPU fallback: load() raises if the library is missing, and the
GPU entry points need a visible device.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsera_q4k.so")
ROOT = os.path.dirname(HERE)
HEADERS = [os.path.join(ROOT, "include", "q3_q4_linear.h"),
           os.path.join(ROOT, "include", "sera_q4k.h")]

QTYPE_Q4_K = 12
QTYPE_Q6_K = 14
MMVQ_MAX_BATCH = 8

_lib = None


class Stats(ctypes.Structure):
    """q3_q4_linear_stats (src/q3_q4_linear.h:32-44)."""
    _fields_ = [("total_ms", ctypes.c_double),
                ("activation_quant_ms", ctypes.c_double),
                ("kernel_ms", ctypes.c_double),
                ("weight_bytes", ctypes.c_uint64),
                ("activation_read_bytes", ctypes.c_uint64),
                ("activation_write_bytes", ctypes.c_uint64),
                ("kernel_launches", ctypes.c_uint64),
                ("cuda_allocations", ctypes.c_uint64),
                ("host_syncs", ctypes.c_uint64)]


class Geometry(ctypes.Structure):
    """q3_q4_linear_geometry (src/q3_q4_linear.h:49-55)."""
    _fields_ = [("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
                ("qtype", ctypes.c_uint32), ("weight_bytes", ctypes.c_uint64)]


class Q3Q4Error(RuntimeError):
    pass


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    """Load libsera_q4k.so and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise Q3Q4Error(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                        "(there is no fallback path)")
    try:  # share torch's HIP runtime when torch is present
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, SZ, B = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t,
                        ctypes.c_bool)
    CP = ctypes.c_char_p
    U32 = ctypes.c_uint32
    sigs = {
        # q3_q4_linear.h
        "q3_q4_linear_bind_geometry": ([ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.POINTER(Geometry), CP, SZ], B),
        "q3_cuda_q4k_linear_init": ([I, SZ, I64, I64, CP, SZ], B),
        "q3_cuda_q4k_linear_workspace_bytes": ([], SZ),
        "q3_cuda_q4k_linear_set_workspace": ([P, SZ, CP, SZ], B),
        "q3_cuda_q4k_linear_path_for_batch": ([SZ], CP),
        "q3_cuda_q4k_linear": ([ctypes.POINTER(Geometry), P, P, SZ, P, P,
                                ctypes.POINTER(Stats), CP, SZ], B),
        "q3_cuda_q4k_linear_read_stats": ([ctypes.POINTER(Stats), P], None),
        # sera_q4k.h
        "sera_q4k_init": ([I], I),
        "sera_q4k_arena_bytes": ([SZ, I64, I64], SZ),
        "sera_q4k_set_arena": ([P, SZ], I),
        "sera_q4k_dense": ([P, P, P, I, I, I, P, I], I),
        "sera_q4k_dense_vec": ([P, P, P, I, I, I, P, I], I),
        "sera_q4k_dense_qt": ([U32, P, P, P, I, I, I, P, I], I),
        "sera_q4k_dense_vec_qt": ([U32, P, P, P, I, I, I, P, I], I),
        "sera_q4k_dense_vec_static": ([P, P, P, I, I, I, P], I),
        "sera_q4k_dense_vec_static_bytes": ([I, I, I], SZ),
        "sera_q4k_read_timings": ([ctypes.POINTER(ctypes.c_double)] * 3, None),
        "sera_q8_1_row_stage_bytes": ([I, I], SZ),
        "sera_q8_1_row_stage_offsets": ([I, I, ctypes.POINTER(SZ), ctypes.POINTER(SZ),
                                         ctypes.POINTER(SZ)], None),
        "sera_q8_1_quantize_row": ([P, I, I, P, P], I),
        "sera_q8_1_mmq_padded_rows": ([I], I),
        "sera_q8_1_mmq_stage_bytes": ([I, I], SZ),
        "sera_q8_1_mmq_stage_offsets": ([I, I, ctypes.POINTER(SZ), ctypes.POINTER(SZ)], None),
        "sera_q8_1_quantize_mmq": ([P, I, I, P, P], I),
        "sera_q4k_mmvq": ([P, P, P, I, I, I, I, P], I),
        "sera_q4k_mmvq_qt": ([U32, P, P, P, I, I, I, I, P], I),
        "sera_q4k_mmq_qt": ([U32, P, P, P, P, I, I, I, I, P], I),
        "sera_q4k_mmq_streamk_qt": ([U32, P, P, P, P, P, I, I, I, I, P], I),
        "sera_q4k_fewtok_qt": ([U32, I, P, P, P, P, P, I, I, I, I, I, P], I),
        "sera_q4k_mmvq_rows_per_tile": ([I, I, I], I),
        "sera_q4k_mmq": ([P, P, P, P, I, I, I, I, P], I),
        "sera_q4k_mmq_splits": ([I, I, I], I),
        "sera_q4k_fewtok": ([I, P, P, P, P, P, I, I, I, I, I, P], I),
        "sera_q4k_fewtok_splits": ([I, I, I, I], I),
        "sera_q4k_fewtok_groups": ([I, I, I], I),
        "sera_q4k_fewtok_grid": ([I, I, I, I, I], I),
        "sera_q4k_kernel_launches": ([I, I, I], I),
        "sera_q4k_vec_uses_fewtok": ([I, I, I], I),
        "sera_q4k_vec_uses_fewtok_qt": ([U32, I, I, I], I),
        "sera_q6k_vec_uses_tile": ([I, I, I], I),
        "sera_q6k_vec_uses_tile_qt": ([U32, I, I, I], I),
        "sera_q4k_mmq_streamk": ([P, P, P, P, P, I, I, I, I, P], I),
        "sera_q4k_mmq_streamk_wgs": ([I], I),
        "sera_q4k_mmq_schedule": ([I, I, I], I),
        "sera_q4k_mmq_tail_qt": ([U32, P, P, P, P, P, I, I, I, I, I, I, P], I),
        "sera_q4k_mmq_tail_plan": ([I, I, I, SZ, ctypes.POINTER(I), ctypes.POINTER(I)], I),
        "sera_q4k_mmq_tail_slot_floats": ([I, I, I, I], SZ),
        "sera_q4k_mmq_uses_fewtok": ([I, I, I], I),
        "sera_q4k_mmq_tiles": ([I, I], I),
        "sera_q4k_mmq_slot_floats": ([I], I),
        "sera_q4k_dequantize": ([P, SZ, P, P], I),
        "sera_q4k_dequantize_qt": ([U32, P, I, I, P, P], I),
        "sera_q4k_subblock_dots": ([P, P, P, I, I, I, P], I),
        "sera_q4k_quantize": ([P, I64, I64, P, P], I),
        "sera_q4k_last_error": ([], CP),
        "sera_q6k_dense": ([U32, P, P, P, I, I, I, P, I], I),
        "sera_q6k_dense_vec": ([U32, P, P, P, I, I, I, P, I], I),
        "sera_q6k_kernel_launches": ([I, I, I], I),
        "sera_q6k_kernel_launches_qt": ([U32, I, I, I], I),
        "sera_q6k_mmvq": ([U32, P, P, P, I, I, I, I, P], I),
        "sera_q6k_mmvq_rows_per_wave": ([I, I], I),
        "sera_q8_1_q6k_mmq_padded_rows": ([I], I),
        "sera_q8_1_q6k_mmq_stage_bytes": ([I, I], SZ),
        "sera_q8_1_q6k_mmq_stage_offsets": ([I, I, ctypes.POINTER(SZ), ctypes.POINTER(SZ)], None),
        "sera_q8_1_quantize_mmq_d4": ([P, I, I, P, P], I),
        "sera_q8_1_quantize_row_q6k": ([P, I, I, P, P], I),
        "sera_q6k_mmq": ([U32, P, P, P, P, I, I, I, I, P], I),
        "sera_weight_bytes": ([U32, I, I], SZ),
        "sera_weight_to_device_layout": ([U32, I, I, P, P, P], I),
        "sera_weight_upload": ([U32, I, I, P, P, P, SZ, P], I),
        "sera_q6k_mmq_splits_for": ([I, I, I], I),
        "sera_q6k_mmq_tile_tokens": ([I, I, I], I),
        "sera_q6k_mmq_tiles": ([I, I, I], I),
        "sera_q6k_mmq_tail": ([U32, P, P, P, P, P, I, I, I, I, I, I, P], I),
        "sera_q6k_mmq_tail_plan": ([I, I, I, SZ, ctypes.POINTER(I), ctypes.POINTER(I)], I),
        "sera_q6k_mmq_tail_slot_floats": ([I, I, I, I, I], SZ),
        "sera_candidate_logits": ([I, P, I, I, P, I, P, I, P, P], I),
        "sera_linear_group": ([I, P, P, P, P, P, P, ctypes.c_float, SZ, ctypes.c_uint, P], I),
        "sera_q4k_bench_group_stream": ([P, I, P, I, I, I, ctypes.POINTER(ctypes.c_double)], I),
        "sera_embedding": ([I, P, I, I, P, I, P, P], I),
        "sera_q4k_bench_linear": ([P, P, I, P, SZ, P, P, I, I, ctypes.POINTER(ctypes.c_double)], I),
        "sera_q4k_bench_stream": ([P, P, P, P, P, I, P, I, I, I, ctypes.POINTER(ctypes.c_double)], I),
        "sera_q4k_bench_kernel": ([I, P, I, P, P, P, SZ, I, I, I, I, P, I, I,
                                   ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], I),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def header_symbols():
    """Function names declared in include/*.h (for the export check)."""
    import re
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            n = m.group(1)
            if n.startswith(("q3_", "sera_")) and n not in names:
                names.append(n)
    return names


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _check(rc, what):
    if rc != 0:
        raise Q3Q4Error(f"{what} failed (rc={rc}): {load().sera_q4k_last_error().decode()}")


# ---------------------------------------------------------------------------
# The q3_q4_linear boundary
# ---------------------------------------------------------------------------

def bind_geometry(qtype, dim0, dim1):
    L = load()
    g = Geometry()
    err = ctypes.create_string_buffer(256)
    ok = L.q3_q4_linear_bind_geometry(qtype, dim0, dim1, ctypes.byref(g), err, 256)
    if not ok:
        raise Q3Q4Error(err.value.decode())
    return g


class Linear:
    """One process-wide q3_q4_linear context: init + caller-owned workspace
    (src/q3_forward.cu:1050-1116 does the same for the reference runtime)."""

    def __init__(self, device=0, max_tokens=16, max_features=25600, max_k=25600):
        import torch
        L = load()
        err = ctypes.create_string_buffer(256)
        if not L.q3_cuda_q4k_linear_init(device, max_tokens, max_features, max_k, err, 256):
            raise Q3Q4Error(err.value.decode())
        nbytes = L.q3_cuda_q4k_linear_workspace_bytes()
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=f"cuda:{device}")
        if not L.q3_cuda_q4k_linear_set_workspace(_ptr(self.workspace), nbytes, err, 256):
            raise Q3Q4Error(err.value.decode())
        self.workspace_bytes = nbytes

    def __call__(self, geometry, weight, x, out, stream=None, stats=None):
        L = load()
        err = ctypes.create_string_buffer(512)
        st = stats if stats is not None else Stats()
        ok = L.q3_cuda_q4k_linear(ctypes.byref(geometry), _ptr(weight), _ptr(x), x.shape[0],
                                  _ptr(out), _stream(stream), ctypes.byref(st), err, 512)
        if not ok:
            raise Q3Q4Error(err.value.decode())
        return st

    @staticmethod
    def read_stats(stats, stream=None):
        load().q3_cuda_q4k_linear_read_stats(ctypes.byref(stats), _stream(stream))
        return stats


# ---------------------------------------------------------------------------
# Building blocks (sera_q4k.h)
# ---------------------------------------------------------------------------

def row_stage_layout(M, K):
    L = load()
    qs, ds, dsf = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    L.sera_q8_1_row_stage_offsets(M, K, ctypes.byref(qs), ctypes.byref(ds), ctypes.byref(dsf))
    return {"qs": qs.value, "ds": ds.value, "dsf": dsf.value,
            "total": L.sera_q8_1_row_stage_bytes(M, K)}


def mmq_stage_layout(M, K):
    L = load()
    qs, ds = ctypes.c_size_t(), ctypes.c_size_t()
    L.sera_q8_1_mmq_stage_offsets(M, K, ctypes.byref(qs), ctypes.byref(ds))
    return {"qs": qs.value, "ds": ds.value, "rows": L.sera_q8_1_mmq_padded_rows(M),
            "total": L.sera_q8_1_mmq_stage_bytes(M, K)}


def quantize_row(x, stage, stream=None):
    M, K = x.shape
    _check(load().sera_q8_1_quantize_row(_ptr(x), M, K, _ptr(stage), _stream(stream)),
           "sera_q8_1_quantize_row")


def quantize_mmq(x, stage, stream=None):
    M, K = x.shape
    _check(load().sera_q8_1_quantize_mmq(_ptr(x), M, K, _ptr(stage), _stream(stream)),
           "sera_q8_1_quantize_mmq")


def mmvq(W, stage, out, M, N, K, rows_per_tile=0, stream=None, qtype=QTYPE_Q4_K):
    """qtype: QTYPE_Q4_K (GGUF bytes) or QTYPE_Q4K_TILED, as for the other
    Q4_K kernel calls below."""
    _check(load().sera_q4k_mmvq_qt(qtype, _ptr(W), _ptr(stage), _ptr(out), M, N, K, rows_per_tile,
                                   _stream(stream)), "sera_q4k_mmvq")


def mmq(W, stage, out, M, N, K, splits=0, partial=None, stream=None, qtype=QTYPE_Q4_K):
    _check(load().sera_q4k_mmq_qt(qtype, _ptr(W), _ptr(stage), _ptr(out), _ptr(partial), M, N, K, splits,
                                  _stream(stream)), "sera_q4k_mmq")


def mmq_splits(M, N, K):
    return load().sera_q4k_mmq_splits(M, N, K)


def mmq_streamk(W, stage, out, M, N, K, slots, counters, wgs=0, stream=None, qtype=QTYPE_Q4_K):
    """MMQ under a stream-K schedule; counters (int32, sera_q4k_mmq_tiles)
    must be zero and are zero again afterwards."""
    _check(load().sera_q4k_mmq_streamk_qt(qtype, _ptr(W), _ptr(stage), _ptr(out), _ptr(slots), _ptr(counters), M,
                                          N, K, wgs, _stream(stream)), "sera_q4k_mmq_streamk")


def mmq_tail(W, stage, out, M, N, K, dp_tiles, pieces, slots=None, counters=None, accum=False, stream=None,
             qtype=QTYPE_Q4_K):
    """MMQ under the tail schedule: dp_tiles whole tiles, the rest cut into
    `pieces` K ranges; slots (mmq_tail_slot_floats float32) and counters
    (tiles - dp_tiles int32, zero before and after) when a tail is split."""
    _check(load().sera_q4k_mmq_tail_qt(qtype, _ptr(W), _ptr(stage), _ptr(out), _ptr(slots), _ptr(counters), M, N,
                                       K, dp_tiles, pieces, 1 if accum else 0, _stream(stream)), "sera_q4k_mmq_tail")


def mmq_tail_plan(M, N, K, max_slot_floats=0):
    """(dp_tiles, pieces) of the tail schedule on the current device (after
    init); max_slot_floats 0: the attached arena's room, as the boundary."""
    dp, pc = ctypes.c_int(), ctypes.c_int()
    _check(load().sera_q4k_mmq_tail_plan(M, N, K, max_slot_floats, ctypes.byref(dp), ctypes.byref(pc)),
           "sera_q4k_mmq_tail_plan")
    return dp.value, pc.value


def mmq_tail_slot_floats(M, N, dp_tiles, pieces):
    return load().sera_q4k_mmq_tail_slot_floats(M, N, dp_tiles, pieces)


def fewtok(W, stage, out, M, N, K, chunk=0, slots=None, counters=None, accum=False, form=0, stream=None,
           qtype=QTYPE_Q4_K):
    """Few-token MFMA kernel: form 0 on a row stage (MMVQ formula, M <= 8),
    form 1 on an MMQ stage (MMQ formula, M <= 16); a split K needs slots
    (splits*M*N float32) and counters (fewtok_groups int32, zero before and
    after)."""
    _check(load().sera_q4k_fewtok_qt(qtype, form, _ptr(W), _ptr(stage), _ptr(out), _ptr(slots), _ptr(counters), M,
                                     N, K, chunk, 1 if accum else 0, _stream(stream)), "sera_q4k_fewtok")


def fewtok_splits(M, N, K, chunk=0):
    return load().sera_q4k_fewtok_splits(M, N, K, chunk)


def fewtok_groups(M, N, K):
    return load().sera_q4k_fewtok_groups(M, N, K)


def fewtok_grid(form, M, N, K, chunk=0):
    """Workgroups along the rows of the launch on the current device (fewer
    than fewtok_groups when the grid is persistent)."""
    return load().sera_q4k_fewtok_grid(form, M, N, K, chunk)


def dequantize(W, nblocks, out, stream=None):
    _check(load().sera_q4k_dequantize(_ptr(W), nblocks, _ptr(out), _stream(stream)),
           "sera_q4k_dequantize")


def dequantize_matrix(qtype, W, N, K, out, stream=None):
    """The N x K matrix in the layout of qtype (QTYPE_Q4_K or QTYPE_Q4K_TILED)
    to row-major fp32 out [N, K]."""
    _check(load().sera_q4k_dequantize_qt(qtype, _ptr(W), N, K, _ptr(out), _stream(stream)),
           "sera_q4k_dequantize")


def subblock_dots(W, stage_qs, out, M, N, K, stream=None):
    _check(load().sera_q4k_subblock_dots(_ptr(W), _ptr(stage_qs), _ptr(out), M, N, K,
                                         _stream(stream)), "sera_q4k_subblock_dots")


def quantize_weights(x, out, stream=None):
    rows, K = x.shape
    _check(load().sera_q4k_quantize(_ptr(x), rows, K, _ptr(out), _stream(stream)),
           "sera_q4k_quantize")


# ---------------------------------------------------------------------------
# Q6_K (GGUF type 14)
# ---------------------------------------------------------------------------

def q6k_mmq_stage_layout(M, K):
    L = load()
    qs, d = ctypes.c_size_t(), ctypes.c_size_t()
    L.sera_q8_1_q6k_mmq_stage_offsets(M, K, ctypes.byref(qs), ctypes.byref(d))
    return {"qs": qs.value, "d": d.value, "rows": L.sera_q8_1_q6k_mmq_padded_rows(M),
            "total": L.sera_q8_1_q6k_mmq_stage_bytes(M, K)}


def quantize_mmq_d4(x, stage, stream=None):
    M, K = x.shape
    _check(load().sera_q8_1_quantize_mmq_d4(_ptr(x), M, K, _ptr(stage), _stream(stream)),
           "sera_q8_1_quantize_mmq_d4")


def quantize_row_q6k(x, stage, stream=None):
    """Row-quantizer values (MMVQ arithmetic) in the Q6_K tile-kernel layout."""
    M, K = x.shape
    _check(load().sera_q8_1_quantize_row_q6k(_ptr(x), M, K, _ptr(stage), _stream(stream)),
           "sera_q8_1_quantize_row_q6k")


QTYPE_Q6K_SPLIT = 270   # SERA_QTYPE_Q6K_SPLIT: Q6_K in the split device layout
QTYPE_Q4K_TILED = 268   # SERA_QTYPE_Q4K_TILED: Q4_K in the 16-row tiled device layout


def q4k_tiled_bytes(gguf, N, K):
    """Host-side statement of the tiled layout (numpy uint8 in, uint8 out):
    block (r, b) of the GGUF rows lands at ((r//16)*(K//256) + b)*2304 +
    (r%16)*144. The device repack must give exactly these bytes."""
    import numpy as np
    nkb = K // 256
    blocks = np.asarray(gguf, dtype=np.uint8).reshape(N // 16, 16, nkb, 144)
    return np.ascontiguousarray(blocks.transpose(0, 2, 1, 3)).reshape(-1)


def q6k_mmvq(W, stage, out, M, N, K, rows_per_wave=0, stream=None, qtype=14):
    """qtype 14: W is GGUF bytes (rows_per_wave in {0,1,2,4}); QTYPE_Q6K_SPLIT:
    W is the split layout (rows per workgroup in {0,2,4})."""
    _check(load().sera_q6k_mmvq(qtype, _ptr(W), _ptr(stage), _ptr(out), M, N, K, rows_per_wave,
                                _stream(stream)), "sera_q6k_mmvq")


def q6k_mmq(W, stage, out, M, N, K, splits=0, partial=None, stream=None, qtype=14):
    _check(load().sera_q6k_mmq(qtype, _ptr(W), _ptr(stage), _ptr(out), _ptr(partial), M, N, K, splits,
                               _stream(stream)), "sera_q6k_mmq")


def weight_bytes(qtype, N, K):
    return load().sera_weight_bytes(qtype, N, K)


def weight_to_device_layout(qtype, N, K, gguf, dst, stream=None):
    """GGUF bytes on the device -> dst in the layout of qtype."""
    _check(load().sera_weight_to_device_layout(qtype, N, K, _ptr(gguf), _ptr(dst), _stream(stream)),
           "sera_weight_to_device_layout")


def weight_upload(qtype, N, K, host_gguf, dst, staging=None, stream=None):
    """host_gguf: a C-contiguous numpy uint8 array of GGUF bytes (kept alive
    until the stream has run the copies); staging: a device uint8 tensor
    (needed for the split layout)."""
    sb = staging.numel() if staging is not None else 0
    _check(load().sera_weight_upload(qtype, N, K, ctypes.c_void_p(host_gguf.ctypes.data), _ptr(dst),
                                     _ptr(staging), sb, _stream(stream)), "sera_weight_upload")


def q6k_mmq_splits(M, N, K):
    return load().sera_q6k_mmq_splits_for(M, N, K)


def q6k_mmq_tail(W, stage, out, M, N, K, dp_tiles, pieces, slots=None, counters=None, accum=False, stream=None,
                 qtype=14):
    """The Q6_K tile kernel under the tail schedule: dp_tiles whole tiles,
    the rest cut into `pieces` K ranges; slots (q6k_mmq_tail_slot_floats
    float32) and counters (tiles - dp_tiles int32, zero before and after)
    when a tail is split."""
    _check(load().sera_q6k_mmq_tail(qtype, _ptr(W), _ptr(stage), _ptr(out), _ptr(slots), _ptr(counters), M, N, K,
                                    dp_tiles, pieces, 1 if accum else 0, _stream(stream)), "sera_q6k_mmq_tail")


def q6k_mmq_tail_plan(M, N, K, max_slot_floats=0):
    """(dp_tiles, pieces) when the dense paths run the tail schedule for this
    shape (after init), else None (split-K)."""
    dp, pc = ctypes.c_int(), ctypes.c_int()
    r = load().sera_q6k_mmq_tail_plan(M, N, K, max_slot_floats, ctypes.byref(dp), ctypes.byref(pc))
    if r < 0:
        raise RuntimeError(f"sera_q6k_mmq_tail_plan: {load().sera_q4k_last_error().decode()}")
    return (dp.value, pc.value) if r else None


def q6k_mmq_tail_slot_floats(M, N, K, dp_tiles, pieces):
    return load().sera_q6k_mmq_tail_slot_floats(M, N, K, dp_tiles, pieces)


# ---------------------------------------------------------------------------
# Gathered rows: selected-row LM head, embedding
# ---------------------------------------------------------------------------

def candidate_logits(qtype, W, N, K, hidden, ids, per_branch, logits, stream=None):
    """hidden [branches, K] fp32, ids uint32/int32 [branches*per_branch] (device)."""
    branches = hidden.shape[0]
    _check(load().sera_candidate_logits(qtype, _ptr(W), N, K, _ptr(hidden), branches, _ptr(ids), per_branch,
                                        _ptr(logits), _stream(stream)), "sera_candidate_logits")


def embedding(qtype, W, N, K, ids, hidden, stream=None):
    _check(load().sera_embedding(qtype, _ptr(W), N, K, _ptr(ids), ids.numel(), _ptr(hidden), _stream(stream)),
           "sera_embedding")


# ---------------------------------------------------------------------------
# Fused linear group
# ---------------------------------------------------------------------------

LIN_ACCUMULATE = 1
LIN_RMSNORM = 2
LIN_SILU_MUL = 4
GROUP_MAX = 4


class GroupCall(ctypes.Structure):
    """sera_linear_group_call (include/sera_q4k.h)."""
    _fields_ = [("count", ctypes.c_int),
                ("geometries", ctypes.c_void_p * GROUP_MAX),
                ("weights", ctypes.c_void_p * GROUP_MAX),
                ("outputs", ctypes.c_void_p * GROUP_MAX),
                ("X", ctypes.c_void_p), ("X2", ctypes.c_void_p), ("gamma", ctypes.c_void_p),
                ("eps", ctypes.c_float), ("M", ctypes.c_size_t), ("flags", ctypes.c_uint)]


def group_call(geometries, weights, outputs, x, x2=None, gamma=None, eps=0.0, flags=0):
    c = GroupCall()
    c.count = len(weights)
    for i, (g, w, y) in enumerate(zip(geometries, weights, outputs)):
        c.geometries[i] = ctypes.addressof(g)
        c.weights[i] = w.data_ptr()
        c.outputs[i] = y.data_ptr()
    c.X = x.data_ptr()
    c.X2 = x2.data_ptr() if x2 is not None else None
    c.gamma = gamma.data_ptr() if gamma is not None else None
    c.eps = eps
    c.M = x.shape[0]
    c.flags = flags
    return c


def linear_group(geometries, weights, outputs, x, x2=None, gamma=None, eps=0.0, flags=0, stream=None):
    """outputs[i] (+)= op(x) . W_i^T for the geometries/weights given (1..4)."""
    n = len(weights)
    G = (ctypes.c_void_p * n)(*[ctypes.addressof(g) for g in geometries])
    Wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in weights])
    Yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in outputs])
    _check(load().sera_linear_group(n, G, Wp, Yp, _ptr(x), _ptr(x2), _ptr(gamma), float(eps), x.shape[0], flags,
                                    _stream(stream)), "sera_linear_group")
