"""sw_libm.h (the device restatements of glibc expf / log1pf) against the
host's glibc, on a CPU build of the same header.  Every float input whose
bit pattern is a multiple of SW_LIBM_STRIDE (default 7, about 6e8 inputs
spanning every exponent; SW_LIBM_STRIDE=1 is the exhaustive 2^32 run)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r"""
#include "sw_libm.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
int main(int argc, char **argv) {
    long long stride = atoll(argv[1]);
    long long bad_e = 0, bad_l = 0, bad_sp = 0, n = 0;
    #pragma omp parallel for reduction(+:bad_e,bad_l,bad_sp,n) schedule(static)
    for (long long u = 0; u < 0x100000000ll; u += stride) {
        float x = sw_asf32((uint32_t)u);
        if (x != x) continue;
        n++;
        float a = expf(x), b = sw_expf(x);
        if (sw_asu32(a) != sw_asu32(b)) bad_e++;
        float c = log1pf(x), d = sw_log1pf(x);
        if (sw_asu32(c) != sw_asu32(d) && !(c != c && d != d)) bad_l++;
        if (x <= 20.f) {
            float e = log1pf(expf(x)), f = sw_softplus_ref(x);
            if (sw_asu32(e) != sw_asu32(f)) bad_sp++;
        }
    }
    printf("%lld %lld %lld %lld\n", n, bad_e, bad_l, bad_sp);
    return 0;
}
"""


def test_libm_matches_glibc(tmp_path):
    src = tmp_path / "libm_check.hip"
    src.write_text(SRC)
    exe = tmp_path / "libm_check"
    r = subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-fopenmp", "-ffp-contract=off", "--offload-arch=gfx950",
                        "-I", os.path.join(ROOT, "sabrewing_amd", "csrc"), str(src), "-o", str(exe)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        pytest.fail(r.stdout[-2000:])
    stride = os.environ.get("SW_LIBM_STRIDE", "7")
    out = subprocess.run([str(exe), stride], stdout=subprocess.PIPE, text=True, check=True).stdout.split()
    n, bad_e, bad_l, bad_sp = map(int, out)
    assert n > (1 << 32) // int(stride) - (1 << 24) // int(stride) - 1
    assert (bad_e, bad_l, bad_sp) == (0, 0, 0)
