"""Writes the golden fixtures under tests/golden/ (run in the build container).

Sources of truth, both from the reference tree /root/reference:
  * tools/qwen3_q4.py (imported here, in the build container only): the
    repo's Q4_K quantizer quantize_q4_k_matrix (:410-481) and its fp16 helpers
    f32_to_f16 / f16_to_f32 (:94-130). Nothing else in the reference pins
    their bytes, so their outputs are recorded as vectors.
  * src/q3_quant.c compiled by oracle/Makefile into oracle/_ref/: the Q4_K
    dequant (:57-76) applied to the LCG blocks of
    tests/test_q3_q4_linear.cu:57-74 and to the quantized matrices.

Outputs (data only: inputs and expected outputs):
  q4k_quantizer.npz  float32 matrices and the Q4_K bytes the reference makes
  fp16_helpers.npz   float32 inputs -> f32_to_f16 bits; all 65536 halves ->
                     f16_to_f32 values
  dequant_ref.npz    Q4_K bytes (LCG blocks + quantized matrices) and the
                     reference dequant of each
  dequant_q6k_ref.npz  seeded Q6_K blocks (plus edge blocks: extreme group
                     scales, all-low / all-high quants, d = 0, negative and
                     subnormal d) and the reference dequant (src/q3_quant.c:78-103,
                     qtype 14) of each; needs only oracle/_ref
Run:  python tests/golden/make_golden.py            (all fixtures)
      python tests/golden/make_golden.py --q6k      (Q6_K fixture only)
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("SERA_REFERENCE", "/root/reference")
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402


def load_ref_quantizer():
    path = os.path.join(REF, "tools", "qwen3_q4.py")
    spec = importlib.util.spec_from_file_location("ref_qwen3_q4", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def lcg_blocks(nblock=4):
    """Input blocks of tests/test_q3_q4_linear.cu:57-74 (seed 0x12345678,
    x = x*1664525 + 1013904223, value = x >> 8)."""
    state = [0x12345678]

    def nxt():
        state[0] = (state[0] * 1664525 + 1013904223) & 0xFFFFFFFF
        return state[0] >> 8

    out = np.zeros((nblock, 144), np.uint8)
    for b in range(nblock):
        d = 0x2000 + (nxt() & 0x0FFF)
        dmin = 0x1800 + (nxt() & 0x0FFF)
        out[b, 0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
        out[b, 2:4] = np.frombuffer(np.uint16(dmin).tobytes(), np.uint8)
        for i in range(12):
            out[b, 4 + i] = nxt() & 0xFF
        for i in range(128):
            lo = nxt() & 0x0F
            hi = nxt() & 0x0F
            out[b, 16 + i] = (hi << 4) | lo
    return out


def quantizer_inputs():
    rng = np.random.default_rng(20240601)
    mats = {}
    mats["normal_0p02_8x512"] = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    mats["normal_1_4x256"] = rng.standard_normal((4, 256)).astype(np.float32)
    # rows whose sub-blocks have very different magnitudes
    x = rng.standard_normal((6, 256)).astype(np.float32)
    x *= np.repeat(np.exp2(rng.integers(-12, 6, (6, 8))).astype(np.float32), 32, axis=1)
    mats["mixed_scale_6x256"] = x
    edge = np.zeros((10, 256), np.float32)
    edge[1, :] = 0.5                                  # constant positive
    edge[2, :] = -0.25                                # constant negative
    edge[3, :] = np.linspace(0.0, 1.0, 256)           # non-negative ramp
    edge[4, 17] = 3.0                                 # single spike
    edge[5, :] = rng.standard_normal(256) * 1e-6      # tiny values
    edge[6, :] = rng.standard_normal(256) * 300.0     # large values
    edge[7, ::2] = 1.0                                # two-level pattern
    edge[7, 1::2] = -1.0
    edge[8, :] = np.abs(rng.standard_normal(256))     # all positive
    edge[9, :] = -np.abs(rng.standard_normal(256))    # all negative
    mats["edge_10x256"] = edge
    return mats


def q6k_vectors():
    """Q6_K blocks and their dequant through the compiled reference."""
    rng = np.random.default_rng(60606)
    blocks = [oracle.q6k_blocks(rng, 24)]
    edge = oracle.q6k_blocks(rng, 8)
    edge[0, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)   # extreme scales
    edge[1, 0:192] = 0x00                                                   # all quants 0 -> -32
    edge[2, 0:192] = 0xFF                                                   # all quants 63 -> +31
    edge[3, 208:210] = np.array([0], np.uint16).view(np.uint8)              # d = 0
    edge[4, 208:210] = np.array([0x8001], np.uint16).view(np.uint8)         # negative subnormal d
    edge[5, 208:210] = np.array([0x7BFF], np.uint16).view(np.uint8)         # largest finite d
    edge[6, 192:208] = np.arange(16, dtype=np.int8).view(np.uint8)          # scale = group index
    blocks.append(edge)
    W = np.concatenate(blocks).reshape(4, -1)                               # 4 rows x 2048 weights
    deq = oracle.ref_dequant(W, 4, 2048, qtype=14)
    assert deq is not None, "oracle/_ref not built (reference tree not mounted?)"
    np.savez_compressed(os.path.join(HERE, "dequant_q6k_ref.npz"), w=W, deq=deq)
    print("dequant_q6k_ref.npz", os.path.getsize(os.path.join(HERE, "dequant_q6k_ref.npz")), "bytes")


def main():
    oracle.build()
    if "--q6k" in sys.argv[1:]:
        q6k_vectors()
        return
    q = load_ref_quantizer()

    # --- quantizer ---
    mats = quantizer_inputs()
    qz = {}
    for name, x in mats.items():
        b = np.frombuffer(q.quantize_q4_k_matrix(x), np.uint8).reshape(x.shape[0], -1)
        qz["x_" + name] = x
        qz["q_" + name] = b.copy()
    np.savez_compressed(os.path.join(HERE, "q4k_quantizer.npz"), **qz)

    # --- fp16 helpers ---
    rng = np.random.default_rng(7)
    f = np.concatenate([
        (rng.standard_normal(3000) * np.exp2(rng.uniform(-30, 20, 3000))).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6,
                  5.96e-8, 2.98e-8, 2.99e-8, 6.1e-5, 6.0e-5, 1e-10, np.inf, -np.inf],
                 np.float32),
        # exact ties between adjacent halves around 1.0 and in the subnormal range
        (np.float32(1.0) + np.arange(1, 64, dtype=np.float32) * np.float32(2.0 ** -11)),
        (np.arange(1, 64, dtype=np.float32) * np.float32(2.0 ** -25)),
    ]).astype(np.float32)
    h_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h_all = h_all[((h_all >> 10) & 0x1F) != 0x1F]  # finite halves
    np.savez_compressed(os.path.join(HERE, "fp16_helpers.npz"),
                        f32_in=f, f32_to_f16=np.asarray(q.f32_to_f16(f), np.uint16),
                        f16_in=h_all, f16_to_f32=np.asarray(q.f16_to_f32(h_all), np.float32))

    # --- dequant through the compiled reference ---
    lcg = lcg_blocks(4)
    dq = {"lcg_blocks": lcg, "lcg_deq": oracle.ref_dequant(lcg.reshape(1, -1), 1, 1024)}
    for name in mats:
        W = qz["q_" + name]
        N, K = mats[name].shape
        dq["w_" + name] = W
        dq["deq_" + name] = oracle.ref_dequant(W, N, K)
    np.savez_compressed(os.path.join(HERE, "dequant_ref.npz"), **dq)
    for fn in ("q4k_quantizer.npz", "fp16_helpers.npz", "dequant_ref.npz"):
        print(fn, os.path.getsize(os.path.join(HERE, fn)), "bytes")
    q6k_vectors()


if __name__ == "__main__":
    main()
