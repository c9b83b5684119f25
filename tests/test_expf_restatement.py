"""The device expf (motoria_amd/csrc/expf_glibc.h, compiled here for the
host) returns the host glibc expf's bits for every float.

The softmax and SwiGLU of the reference call glibc's expf
(src/model/forward.c:99,190); the GPU kernels use this restatement."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HARNESS = r"""
#include <math.h>
#include <stdio.h>
#include <string.h>
#include "expf_glibc.h"
int main(void) {
    long mism = 0, n = 0;
#pragma omp parallel for reduction(+ : mism, n) schedule(static)
    for (long long u = 0; u < 0x100000000LL; u++) {
        unsigned b = (unsigned)u;
        float x, r, m;
        memcpy(&x, &b, 4);
        r = expf(x);
        m = mia_expf_glibc(x);
        n++;
        if (memcmp(&r, &m, 4) && !(r != r && m != m)) mism++;
    }
    printf("%ld %ld\n", n, mism);
    return 0;
}
"""


@pytest.mark.timeout(600)
def test_expf_restatement_matches_host_on_every_float(tmp_path):
    src = tmp_path / "expf_sweep.c"
    src.write_text(HARNESS)
    exe = tmp_path / "expf_sweep"
    subprocess.run(["gcc", "-std=gnu99", "-O2", "-ffp-contract=off", "-fopenmp",
                    "-I", os.path.join(ROOT, "motoria_amd", "csrc"), str(src), "-o", str(exe),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    n, mism = int(out[0]), int(out[1])
    assert n == 2 ** 32
    assert mism == 0, "%d floats differ from the host expf" % mism
