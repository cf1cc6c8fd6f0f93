"""The reference's own GPU acceptance test, run unmodified on this backend.

oracle/_ref/laguna_hip is the reference engine (c/laguna.c) compiled with
-DCOLI_CUDA, as its Makefile builds `laguna CUDA=1`, but linked against
libsabrewing_loader.so instead of backend_cuda_laguna.o (oracle/Makefile).
With LAG_CUDA_TEST=1 it runs cuda_selftest (c/laguna.c:1554-1666):
random data through its CPU kernels and through lag_cuda_matmul_bf16,
lag_cuda_matmul_q4, lag_cuda_expert_q4, lag_cuda_moe_experts and
lag_cuda_moe_group, with its own bars: bf16 max rel < 5e-3, q4 max rel
< 1e-3, expert max abs < 1e-3, grouped == per-token bit-identical.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE = os.path.join(ROOT, "oracle", "_ref", "laguna_hip")

pytestmark = pytest.mark.gpu


def test_reference_engine_cuda_selftest():
    if not os.path.exists(ENGINE):
        pytest.skip("reference engine binary not built (make -C oracle ref, with the reference sources present)")
    env = dict(os.environ, LAG_CUDA_TEST="1", OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8"))
    r = subprocess.run([ENGINE], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=110)
    print(r.stdout)
    lines = [l for l in r.stdout.splitlines() if l.startswith("[cuda-test]")]
    assert r.returncode == 0 and lines and lines[-1] == "[cuda-test] ALL PASS", r.stdout
    assert any("BIT-IDENTICAL" in l for l in lines)
