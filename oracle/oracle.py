"""ctypes front-end of the CPU oracle (liborc_q4k.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module as the checker. The product
(sera.c_amd/) never does.

Every function returns numpy arrays in the oracle's layouts:
    W  uint8  [N, K/256*144]   GGUF Q4_K rows
    xq int8   [M, K]           Q8_1 quants
    xd uint16 [M, K/32]        fp16 bits of the Q8_1 scale d
    xs uint16 [M, K/32]        fp16 bits of the Q8_1 sum
The C sources (q4k_oracle.c) cite the reference file:line each one restates.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc_q4k.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libq3quant_ref.so")

_lib = None
_ref = None


def build():
    """Compile the oracle (and the reference dequant when the tree is mounted)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        SZ = ctypes.c_size_t
        for name, args, res in [
            ("orc_h2f_n", [P, SZ, P], None),
            ("orc_f2h_n", [P, SZ, P], None),
            ("orc_np_f32_to_f16_n", [P, SZ, P], None),
            ("orc_np_f16_to_f32_n", [P, SZ, P], None),
            ("orc_dequant_q4k", [P, SZ, P], None),
            ("orc_quantize_q4k", [P, I64, I64, P], ctypes.c_int),
            ("orc_q8_1_row", [P, I64, P, P, P], None),
            ("orc_q8_1_mmq", [P, I64, P, P, P], None),
            ("orc_subblock_dots", [P, P, I64, I64, I64, P], None),
            ("orc_q8_sums", [P, I64, I64, P], None),
            ("orc_gemm_mmvq", [P, P, P, I64, I64, I64, P], None),
            ("orc_gemm_mmq", [P, P, P, P, I64, I64, I64, P], None),
            ("orc_gemm_dequant", [P, P, I64, I64, I64, P], None),
            ("orc_q6k_unpack", [P, P, P, P], None),
            ("orc_dequant_q6k", [P, SZ, P], None),
            ("orc_q8_1_mmq_d4", [P, I64, P, P], None),
            ("orc_q6k_group_dots", [P, P, I64, I64, I64, P], None),
            ("orc_gemm_q6k", [P, P, P, I64, I64, I64, P], None),
            ("orc_gemm_dequant_q6k", [P, P, I64, I64, I64, P], None),
        ]:
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def ref_lib():
    """The reference's own src/q3_quant.c built into _ref/, or None."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        R = ctypes.CDLL(REF_LIB_PATH)
        R.q3_half_to_float.argtypes = [ctypes.c_uint16]
        R.q3_half_to_float.restype = ctypes.c_float
        R.q3_quant_dequantize_row.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t,
                                              ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p,
                                              ctypes.c_size_t]
        R.q3_quant_dequantize_row.restype = ctypes.c_bool
        _ref = R
    return _ref


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def h2f(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_h2f_n(_p(h), h.size, _p(out))
    return out


def f2h(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f2h_n(_p(f), f.size, _p(out))
    return out


def np_f32_to_f16(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_np_f32_to_f16_n(_p(f), f.size, _p(out))
    return out


def np_f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_np_f16_to_f32_n(_p(h), h.size, _p(out))
    return out


def dequant(W, N, K):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size == N * (K // 256) * 144
    out = np.empty((N, K), np.float32)
    lib().orc_dequant_q4k(_p(W), N * (K // 256), _p(out))
    return out


def ref_dequant(W, N, K, qtype=12):
    """Dequant through the reference's compiled q3_quant.c (None if absent);
    qtype 12 = Q4_K, 14 = Q6_K."""
    R = ref_lib()
    if R is None:
        return None
    W = np.ascontiguousarray(W, dtype=np.uint8)
    out = np.empty((N, K), np.float32)
    err = ctypes.create_string_buffer(256)
    ok = R.q3_quant_dequantize_row(qtype, _p(W), N * (K // 256), _p(out), N * K, err, 256)
    assert ok, err.value
    return out


def quantize_q4k(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, K = x.shape
    out = np.empty((rows, K // 256 * 144), np.uint8)
    rc = lib().orc_quantize_q4k(_p(x), rows, K, _p(out))
    if rc != 0:
        raise ValueError("K must be a multiple of 256")
    return out


def _q8(fn, X):
    X = np.ascontiguousarray(X, dtype=np.float32)
    M, K = X.shape
    xq = np.empty((M, K), np.int8)
    xd = np.empty((M, K // 32), np.uint16)
    xs = np.empty((M, K // 32), np.uint16)
    for m in range(M):
        fn(_p(X[m]), K, _p(xq[m]), _p(xd[m]), _p(xs[m]))
    return xq, xd, xs


def q8_1_row(X):
    """MMVQ activation quantizer (cuda/mmq/quantize.cu:4-48)."""
    return _q8(lib().orc_q8_1_row, X)


def q8_1_mmq(X):
    """MMQ DS4 activation quantizer (cuda/mmq/quantize.cu:271-367)."""
    return _q8(lib().orc_q8_1_mmq, X)


def subblock_dots(W, xq, N, K):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    M = xq.shape[0]
    out = np.empty((M, N, K // 32), np.int32)
    lib().orc_subblock_dots(_p(np.ascontiguousarray(W)), _p(xq), M, N, K, _p(out))
    return out


def q8_sums(xq):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    M, K = xq.shape
    out = np.empty((M, K // 32), np.int32)
    lib().orc_q8_sums(_p(xq), M, K, _p(out))
    return out


def gemm_mmvq(W, xq, xd, N, K):
    M = xq.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().orc_gemm_mmvq(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)),
                        _p(np.ascontiguousarray(xd)), M, N, K, _p(Y))
    return Y


def gemm_mmq(W, xq, xd, xs, N, K):
    M = xq.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().orc_gemm_mmq(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)),
                       _p(np.ascontiguousarray(xd)), _p(np.ascontiguousarray(xs)),
                       M, N, K, _p(Y))
    return Y


def gemm_dequant(W, X, N, K):
    X = np.ascontiguousarray(X, dtype=np.float32)
    M = X.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().orc_gemm_dequant(_p(np.ascontiguousarray(W)), _p(X), M, N, K, _p(Y))
    return Y


def linear_reference(W, X, N, K):
    """Output the reference path would produce for X [M,K]: MMVQ formula with
    row-layout Q8_1 when M <= 8, MMQ formula with DS4 Q8_1 otherwise
    (src/q3_q4_linear.cu:198-210)."""
    M = X.shape[0]
    if M <= 8:
        xq, xd, _ = q8_1_row(X)
        return gemm_mmvq(W, xq, xd, N, K)
    xq, xd, xs = q8_1_mmq(X)
    return gemm_mmq(W, xq, xd, xs, N, K)


# ---------------------------------------------------------------------------
# Q6_K (210-byte blocks; layouts: W uint8 [N, K/256*210])
# ---------------------------------------------------------------------------

Q6K_BYTES = 210


def q6k_blocks(rng, nblocks, d_scale=2.0e-5, scales=None):
    """Synthetic Q6_K blocks: uniform ql/qh bytes, int8 group scales uniform
    in [-128, 127] (or the given array), fp16 d of magnitude ~d_scale with a
    random sign. Any such bytes are a valid Q6_K block (the reference repo
    ships no Q6_K quantizer)."""
    b = rng.integers(0, 256, (nblocks, Q6K_BYTES), dtype=np.uint8)
    if scales is not None:
        b[:, 192:208] = np.asarray(scales, np.int8).view(np.uint8)
    d = (rng.uniform(0.5, 1.5, nblocks) * d_scale * rng.choice([-1.0, 1.0], nblocks)).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    return b


def q6k_weights(rng, N, K, **kw):
    return q6k_blocks(rng, N * (K // 256), **kw).reshape(N, K // 256 * Q6K_BYTES)


def q6k_split(W, N, K):
    """GGUF Q6_K bytes [N][K/256][210] -> the split device layout as one flat
    uint8 array: every block's first 208 bytes (ql, qh, sc) in block order,
    then every block's 2-byte d in block order. A byte permutation, nothing
    more (the block fields are those of src/q3_quant.c:78-103)."""
    B = np.ascontiguousarray(W, dtype=np.uint8).reshape(N * (K // 256), Q6K_BYTES)
    return np.concatenate([B[:, :208].reshape(-1), B[:, 208:].reshape(-1)])


def q6k_unsplit(S, N, K):
    """Inverse of q6k_split: split layout -> GGUF bytes [N][K/256*210]."""
    nblk = N * (K // 256)
    S = np.ascontiguousarray(S, dtype=np.uint8).reshape(-1)
    assert S.size == nblk * Q6K_BYTES
    B = np.empty((nblk, Q6K_BYTES), np.uint8)
    B[:, :208] = S[:nblk * 208].reshape(nblk, 208)
    B[:, 208:] = S[nblk * 208:].reshape(nblk, 2)
    return B.reshape(N, (K // 256) * Q6K_BYTES)


def q6k_unpack(block):
    """(q - 32 as int8 [256], int8 scales [16], d as float32) of one block."""
    block = np.ascontiguousarray(block, dtype=np.uint8)
    q = np.empty(256, np.int8)
    sc = np.empty(16, np.int8)
    d = ctypes.c_float()
    lib().orc_q6k_unpack(_p(block), _p(q), _p(sc), ctypes.byref(d))
    return q, sc, np.float32(d.value)


def dequant_q6k(W, N, K):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    assert W.size == N * (K // 256) * Q6K_BYTES
    out = np.empty((N, K), np.float32)
    lib().orc_dequant_q6k(_p(W), N * (K // 256), _p(out))
    return out


def q8_1_mmq_d4(X):
    """MMQ D4 activation quantizer (Q6_K): int8 quants and fp32 d [M, K/32]."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    M, K = X.shape
    xq = np.empty((M, K), np.int8)
    d = np.empty((M, K // 32), np.float32)
    for m in range(M):
        lib().orc_q8_1_mmq_d4(_p(X[m]), K, _p(xq[m]), _p(d[m]))
    return xq, d


def q6k_group_dots(W, xq, N, K):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    M = xq.shape[0]
    out = np.empty((M, N, K // 16), np.int32)
    lib().orc_q6k_group_dots(_p(np.ascontiguousarray(W)), _p(xq), M, N, K, _p(out))
    return out


def gemm_q6k(W, xq, d8, N, K):
    """y = sum_blk d * sum_g sc_g * d8[g/2] * I_g (double); d8 float [M, K/32]."""
    M = xq.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().orc_gemm_q6k(_p(np.ascontiguousarray(W)), _p(np.ascontiguousarray(xq)),
                       _p(np.ascontiguousarray(d8, dtype=np.float32)), M, N, K, _p(Y))
    return Y


def gemm_dequant_q6k(W, X, N, K):
    X = np.ascontiguousarray(X, dtype=np.float32)
    M = X.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().orc_gemm_dequant_q6k(_p(np.ascontiguousarray(W)), _p(X), M, N, K, _p(Y))
    return Y


def linear_reference_q6k(W, X, N, K):
    """Output the reference path produces for Q6_K weights: row Q8_1 with
    fp16 d8 when M <= 8 (MMVQ), D4 Q8_1 with fp32 d8 otherwise (MMQ)
    (src/q3_q4_linear.cu:198-210, cuda/q3_mmq.cu:303-316,408-470)."""
    M = X.shape[0]
    if M <= 8:
        xq, xd, _ = q8_1_row(X)
        return gemm_q6k(W, xq, h2f(xd), N, K)
    xq, d = q8_1_mmq_d4(X)
    return gemm_q6k(W, xq, d, N, K)


# ---------------------------------------------------------------------------
# Producers fused into the quantize (numpy float32, IEEE)
# ---------------------------------------------------------------------------

def rmsnorm_fused_order(H, gamma, eps):
    """RMSNorm of each row in the order the fused quantizer uses: thread t of
    256 sums x[t + 256 i]^2 in i order (square exact in double, each sum
    rounded to float32, as the reference's `float += double` in
    rms_norm_batched_kernel, src/q3_forward.cu:131-132); an xor butterfly
    over each 64-thread wave (offsets 32..1); the four wave sums left to
    right; inv = 1 / sqrt(sum / K + eps) with IEEE float32 division and
    square root (the reference uses rsqrtf, :143); x = (h * inv) * gamma
    (:144-145)."""
    H = np.ascontiguousarray(H, dtype=np.float32)
    gamma = np.asarray(gamma, np.float32)
    M, K = H.shape
    out = np.empty_like(H)
    eps = np.float32(eps)
    for m in range(M):
        h = H[m]
        part = np.zeros(256, np.float32)
        for t in range(256):
            acc = np.float32(0.0)
            for v in h[t::256].astype(np.float64):
                acc = np.float32(np.float64(acc) + v * v)
            part[t] = acc
        waves = part.reshape(4, 64).copy()
        idx = np.arange(64)
        for o in (32, 16, 8, 4, 2, 1):
            waves = (waves + waves[:, idx ^ o]).astype(np.float32)
        tot = np.float32(np.float32(np.float32(waves[0, 0] + waves[1, 0]) + waves[2, 0]) + waves[3, 0])
        inv = np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(tot / np.float32(K)) + eps)))
        out[m] = ((h * inv).astype(np.float32) * gamma).astype(np.float32)
    return out


def silu_mul(G, U):
    """(g / (1 + exp(-g))) * u in float32 (silu_mul_kernel,
    src/q3_forward.cu:154-161); numpy's float32 exp may differ from the
    device expf in the last place."""
    G = np.asarray(G, np.float32)
    U = np.asarray(U, np.float32)
    with np.errstate(over="ignore"):
        den = (np.float32(1.0) + np.exp(-G)).astype(np.float32)
    return ((G / den).astype(np.float32) * U).astype(np.float32)
