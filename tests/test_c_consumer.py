"""The C ABI from a C99 caller, as the reference's C host code would bind it.

A small C program includes both public headers, links libsera_q4k.so and
calls the host-only entry points (geometry binding and its errors, the path
name, weight sizes of every layout, the dispatch queries). It must compile
with -std=c99 -Wall -Wextra -Werror (no C++ in the headers) and print the
expected values. No GPU is touched.
"""
import os
import shutil
import subprocess

import pytest

import q3q4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SOURCE = r"""
#include "q3_q4_linear.h"
#include "sera_q4k.h"
#include <stdio.h>

int main(void) {
    q3_q4_linear_geometry g;
    char err[256];
    int ok = q3_q4_linear_bind_geometry(12, 5120, 25600, &g, err, sizeof err);
    printf("bind12 %d %d %d %u %llu\n", ok, g.N, g.K, g.qtype, (unsigned long long)g.weight_bytes);
    ok = q3_q4_linear_bind_geometry(SERA_QTYPE_Q4K_TILED, 5120, 151936, &g, err, sizeof err);
    printf("bind268 %d %llu\n", ok, (unsigned long long)g.weight_bytes);
    ok = q3_q4_linear_bind_geometry(SERA_QTYPE_Q4K_TILED, 5120, 100, &g, err, sizeof err);
    printf("bind268bad %d %s\n", ok, err);
    ok = q3_q4_linear_bind_geometry(12, 5000, 100, &g, err, sizeof err);
    printf("bindK %d %s\n", ok, err);
    printf("path %s %s\n", q3_cuda_q4k_linear_path_for_batch(8), q3_cuda_q4k_linear_path_for_batch(9));
    printf("bytes %zu %zu %zu %zu\n", sera_weight_bytes(12, 25600, 5120),
           sera_weight_bytes(SERA_QTYPE_Q4K_TILED, 25600, 5120), sera_weight_bytes(14, 1024, 5120),
           sera_weight_bytes(SERA_QTYPE_Q6K_SPLIT, 1024, 5120));
    printf("fewtok %d %d %d\n", sera_q4k_vec_uses_fewtok(2, 25600, 5120),
           sera_q4k_vec_uses_fewtok_qt(SERA_QTYPE_Q4K_TILED, 2, 25600, 5120),
           sera_q4k_mmq_uses_fewtok(16, 151936, 5120));
    return 0;
}
"""


def test_c99_caller_compiles_links_and_runs(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.fail("no C compiler in PATH")
    q3q4.load()   # builds nothing: fails loudly when the library is missing
    src = tmp_path / "caller.c"
    src.write_text(SOURCE)
    exe = tmp_path / "caller"
    libdir = os.path.dirname(q3q4.LIB_PATH)
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                        str(src), "-L", libdir, "-lsera_q4k", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = dict(line.split(" ", 1) for line in r.stdout.strip().splitlines())
    assert out["bind12"] == "1 25600 5120 12 73728000"
    assert out["bind268"] == "1 437575680"
    assert out["bind268bad"].startswith("0 ") and "16" in out["bind268bad"]
    assert out["bindK"].startswith("0 ") and "multiple of 256" in out["bindK"]
    assert out["path"] == "MMVQ MMQ"
    assert out["bytes"] == "73728000 73728000 4300800 4300800"   # 1024 x 20 x 210
    assert out["fewtok"] == "0 1 1"
