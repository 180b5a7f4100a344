"""The C ABI from a compiled C99 host program on the GPU.

The reference's own linear test is an executable that binds the geometry,
calls q3_cuda_q4k_linear_init, allocates the workspace, attaches it and runs
q3_cuda_q4k_linear on a stream (tests/test_q3_q4_linear.cu:195-408). This
test builds the same caller in C99 with gcc against include/q3_q4_linear.h
and the HIP runtime's C API, links libsera_q4k.so, and runs it on the GPU:

  bind -> init(device 0, 16 tokens) -> workspace_bytes -> hipMalloc ->
  set_workspace -> hipStreamCreate -> for M in {1, 16}: H2D copy of X,
  q3_cuda_q4k_linear on the stream with stats, hipStreamSynchronize,
  read_stats, D2H copy of Y; a repeat call that must match bit for bit.

The weights and activations come from files this test writes (seeded
synthetic Q4_K; the activations are the reference test's fill_activation,
:225-233). Its outputs are checked here against the path-faithful oracle
within 1e-3 * rms(y), and against the reference test's own gates
(cos > 0.999, relative L2 < 1 %, :374,379) on the dequant * fp32 oracle.
"""
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCE = r"""
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>
#include "q3_q4_linear.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void *read_file(const char *path, size_t bytes) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(bytes);
    if (p && fread(p, 1, bytes, f) != bytes) { free(p); p = NULL; }
    fclose(f);
    return p;
}

static int write_file(const char *path, const void *p, size_t bytes) {
    FILE *f = fopen(path, "wb");
    if (!f) return 0;
    const int ok = fwrite(p, 1, bytes, f) == bytes;
    fclose(f);
    return ok;
}

#define HIP_OK(x) do { if ((x) != hipSuccess) { printf("FAIL hip %s\n", #x); fflush(stdout); return 2; } } while (0)

int main(int argc, char **argv) {
    if (argc != 4) return 3;
    const char *dir = argv[1];
    const unsigned N = (unsigned)atoi(argv[2]), K = (unsigned)atoi(argv[3]);
    char path[1024], err[256];
    q3_q4_linear_geometry g;
    if (!q3_q4_linear_bind_geometry(12, K, N, &g, err, sizeof err)) { printf("FAIL bind %s\n", err); return 1; }
    if (!q3_cuda_q4k_linear_init(0, 16, (int64_t)N, (int64_t)K, err, sizeof err)) {
        printf("FAIL init %s\n", err);
        return 1;
    }
    const size_t ws_bytes = q3_cuda_q4k_linear_workspace_bytes();
    void *ws = NULL, *dW = NULL;
    float *dX = NULL, *dY = NULL;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    if (q3_cuda_q4k_linear_set_workspace(ws, ws_bytes / 2, err, sizeof err)) {
        printf("FAIL a half-size workspace was accepted\n");
        return 1;
    }
    if (!q3_cuda_q4k_linear_set_workspace(ws, ws_bytes, err, sizeof err)) {
        printf("FAIL set_workspace %s\n", err);
        return 1;
    }
    snprintf(path, sizeof path, "%s/w.bin", dir);
    void *W = read_file(path, (size_t)g.weight_bytes);
    if (!W) { printf("FAIL reading %s\n", path); return 1; }
    HIP_OK(hipMalloc(&dW, (size_t)g.weight_bytes));
    HIP_OK(hipMemcpy(dW, W, (size_t)g.weight_bytes, hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));
    HIP_OK(hipMalloc((void **)&dX, (size_t)16 * K * sizeof(float)));
    HIP_OK(hipMalloc((void **)&dY, (size_t)16 * N * sizeof(float)));
    const size_t batches[2] = {1, 16};
    for (int bi = 0; bi < 2; bi++) {
        const size_t M = batches[bi];
        printf("call M=%zu N=%u K=%u path=%s\n", M, N, K, q3_cuda_q4k_linear_path_for_batch(M));
        fflush(stdout);
        snprintf(path, sizeof path, "%s/x%zu.bin", dir, M);
        float *x = (float *)read_file(path, M * K * sizeof(float));
        float *y = (float *)malloc(M * N * sizeof(float));
        float *y2 = (float *)malloc(M * N * sizeof(float));
        if (!x || !y || !y2) { printf("FAIL host buffers\n"); return 1; }
        HIP_OK(hipMemcpy(dX, x, M * K * sizeof(float), hipMemcpyHostToDevice));
        HIP_OK(hipMemset(dY, 0xff, M * N * sizeof(float)));   /* poison: Y must be overwritten */
        q3_q4_linear_stats st;
        memset(&st, 0, sizeof st);
        if (!q3_cuda_q4k_linear(&g, dW, dX, M, dY, (void *)stream, &st, err, sizeof err)) {
            printf("FAIL linear M=%zu: %s\n", M, err);
            return 1;
        }
        HIP_OK(hipStreamSynchronize(stream));
        q3_cuda_q4k_linear_read_stats(&st, (void *)stream);
        HIP_OK(hipMemcpy(y, dY, M * N * sizeof(float), hipMemcpyDeviceToHost));
        HIP_OK(hipMemset(dY, 0, M * N * sizeof(float)));
        if (!q3_cuda_q4k_linear(&g, dW, dX, M, dY, (void *)stream, NULL, err, sizeof err)) {
            printf("FAIL repeat M=%zu: %s\n", M, err);
            return 1;
        }
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipMemcpy(y2, dY, M * N * sizeof(float), hipMemcpyDeviceToHost));
        const int same = memcmp(y, y2, M * N * sizeof(float)) == 0;
        printf("stats M=%zu launches=%llu quant_ms=%.4f kernel_ms=%.4f total_ms=%.4f allocs=%llu syncs=%llu "
               "repeat=%d\n", M, (unsigned long long)st.kernel_launches, st.activation_quant_ms, st.kernel_ms,
               st.total_ms, (unsigned long long)st.cuda_allocations, (unsigned long long)st.host_syncs, same);
        fflush(stdout);
        snprintf(path, sizeof path, "%s/y%zu.bin", dir, M);
        if (!write_file(path, y, M * N * sizeof(float))) { printf("FAIL writing %s\n", path); return 1; }
        free(x);
        free(y);
        free(y2);
    }
    HIP_OK(hipStreamDestroy(stream));
    HIP_OK(hipFree(dX));
    HIP_OK(hipFree(dY));
    HIP_OK(hipFree(dW));
    HIP_OK(hipFree(ws));
    free(W);
    printf("done\n");
    return 0;
}
"""


def fill_activation(tokens, K):
    """The reference test's deterministic activation (tests/test_q3_q4_linear.cu:225-233)."""
    k = np.arange(K, dtype=np.uint64)[None, :]
    t = np.arange(tokens, dtype=np.uint64)[:, None]
    a = ((k * 17 + t * 131) % 1009).astype(np.float32) * np.float32(0.1)
    return (np.float32(0.5) * np.sin(a) + np.float32(0.25) * np.cos(a * np.float32(0.37))).astype(np.float32)


def test_c99_host_program_runs_the_linear_on_a_stream(tmp_path):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible HIP device")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.fail("no C compiler in PATH")
    q3q4.load()
    N, K = 2048, 5120
    rng = np.random.default_rng(11)
    W = oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    (tmp_path / "w.bin").write_bytes(W.tobytes())
    xs = {}
    for M in (1, 16):
        xs[M] = fill_activation(M, K)
        (tmp_path / f"x{M}.bin").write_bytes(xs[M].tobytes())

    src = tmp_path / "caller.c"
    src.write_text(SOURCE)
    exe = tmp_path / "caller"
    libdir = os.path.dirname(q3q4.LIB_PATH)
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                        "-I", os.path.join(ROCM, "include"), str(src), "-L", libdir, "-lsera_q4k",
                        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{libdir}",
                        f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-o", str(exe)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    print("running the C caller", flush=True)
    r = subprocess.run([str(exe), str(tmp_path), str(N), str(K)], capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "done"
    stats = {int(l.split()[1][2:]): dict(kv.split("=") for kv in l.split()[2:]) for l in lines if l.startswith("stats")}
    for M in (1, 16):
        st = stats[M]
        assert st["repeat"] == "1", f"M={M}: the repeat call differs"
        assert int(st["launches"]) >= 2
        assert st["allocs"] == "0" and st["syncs"] == "0"
        assert float(st["kernel_ms"]) > 0.0 and float(st["total_ms"]) >= float(st["kernel_ms"])
        y = np.frombuffer((tmp_path / f"y{M}.bin").read_bytes(), dtype=np.float32).reshape(M, N)
        assert np.all(np.isfinite(y))
        ref = oracle.linear_reference(W, xs[M], N, K)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        err = float(np.max(np.abs(y.astype(np.float64) - ref)))
        assert err <= 1e-3 * rms, f"M={M}: max|err| {err:.3e} > 1e-3 * rms {rms:.3e}"
        # the reference test's own gates, against dequant * fp32 activations
        dq = oracle.gemm_dequant(W, xs[M], N, K).astype(np.float64)
        yd = y.astype(np.float64)
        cos = float(np.sum(yd * dq) / (np.sqrt(np.sum(yd * yd)) * np.sqrt(np.sum(dq * dq)) + 1e-30))
        rel_l2 = float(np.sqrt(np.sum((yd - dq) ** 2)) / (np.sqrt(np.sum(dq * dq)) + 1e-30))
        assert cos > 0.999 and rel_l2 < 0.01, (cos, rel_l2)
