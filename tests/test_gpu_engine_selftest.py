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

import numpy as np

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


INKLING = os.path.join(ROOT, "oracle", "_ref", "inkling_hip")


def test_reference_inkling_cuda_q4_test(tmp_path):
    """The Inkling engine (c/inkling.c built with -DCOLI_CUDA against the loader's
    ink_cuda_* table) and its own --cuda-q4-test (c/inkling.c:1789-1862): int4
    GEMM, int8 GEMM and the fused int4 expert at 6144 x 6144 against its CPU
    kernels, each to a scaled error below 1e-3.  IDOT=0 selects the CPU's f32
    activation route, the reference run the test's own comment names."""
    if not os.path.exists(INKLING):
        pytest.skip("inkling engine binary not built (make -C oracle ref, with the reference sources present)")
    env = dict(os.environ, SNAP=str(tmp_path), IDOT="0", OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8"))
    r = subprocess.run([INKLING, "--cuda-q4-test"], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=110)
    print(r.stdout)
    oks = [l for l in r.stdout.splitlines() if l.endswith("[OK]")]
    assert r.returncode == 0 and len(oks) == 3, r.stdout
    assert any(l.startswith("q4 GPU") for l in oks) and any(l.startswith("q8 GPU") for l in oks)
    assert any(l.startswith("fused-expert GPU") for l in oks)


@pytest.mark.parametrize("S_", [1, 5, 150])
def test_reference_engine_moe_rows_on_device(be, orc, S_):
    """The engine's own lag_moe_rows (c/laguna.c:805-824) with a device-resident
    layer, built against this backend's loader: S == 1 goes through moe_block's
    expert_batch hook (lag_cuda_moe_experts), S > 1 through the engine's host
    counting sort and lag_cuda_moe_group (150 rows: two chunks of the engine's
    128), the shared expert through lag_cuda_matmul_bf16.  Against the same
    engine on the CPU: within the benchmark tolerance; grouped and per-token
    device runs bit-identical.  The host copies handed to the device run have
    zero scales and zero shared weights, so a silent fallback to the engine's
    CPU path cannot pass."""
    from dataclasses import replace
    from oracle import synth
    from oracle.oracle import RefLaguna, RefLagunaHip
    from sabrewing_amd import configs as cf
    if not (RefLagunaHip.available() and RefLaguna.available()):
        pytest.skip("reference engine libraries not built")
    cfg = replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), gs=0, router_bf16=False)
    L = synth.make_layer(orc, cfg, 71, corr_bias_sigma=0.01)
    d = synth.desc_of(cfg)
    x = synth.make_x(orc, cfg, 72, S_)
    h0 = synth.make_x(orc, cfg, 73, S_)
    want = RefLaguna().moe_rows(d, L, x, h0, group=1)
    bufs = [be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s, L.sg, L.su, L.sd)]
    poisoned = replace(L, gu_s=np.zeros_like(L.gu_s), dn_s=np.zeros_like(L.dn_s), sg=np.zeros_like(L.sg),
                       su=np.zeros_like(L.su), sd=np.zeros_like(L.sd))
    lag = RefLagunaHip()
    got = lag.moe_rows(d, poisoned, [int(b) for b in bufs], x, h0, group=1)
    got_pt = lag.moe_rows(d, poisoned, [int(b) for b in bufs], x, h0, group=0)
    for b in bufs:
        b.free()
    dg, dw = got - h0, want - h0
    nw = float(np.max(np.abs(dg - dw))) / float(np.max(np.abs(dw)))
    assert nw <= 2e-3, nw
    assert np.array_equal(got.view(np.uint32), got_pt.view(np.uint32))


@pytest.mark.parametrize("S_", [1, 5, 150])
def test_reference_qwen35_moe_rows_on_device(be, orc, S_):
    """The qwen35 engine's moe_forward_rows (c/qwen35.c:595-700), the second caller of
    lag_cuda_moe_group (c/qwen35.c:637-642), built with -DCOLI_CUDA against this
    backend's loader (oracle/ref_qwen35.c): its host router, moe_route and counting
    sort hand all S rows' groups to lag_cuda_moe_group in one call (no 128-row chunks,
    unlike laguna), and its shared expert runs through lag_cuda_matmul_bf16 before the
    engine's sigmoid gate.  Against the same engine on the CPU: within the benchmark
    tolerance.  The host copies handed to the device run have zero scales and zero
    shared weights, so a silent fallback to the engine's CPU path cannot pass."""
    from dataclasses import replace
    from oracle import synth
    from oracle.oracle import RefQwen35Hip
    from sabrewing_amd import configs as cf
    if not RefQwen35Hip.available():
        pytest.skip("qwen35 engine library not built (make -C oracle ref, with the reference sources present)")
    cfg = replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), gs=0, router_bf16=False)
    L = synth.make_layer(orc, cfg, 81)
    x = synth.make_x(orc, cfg, 82, S_)
    sgate = (np.random.default_rng(83).standard_normal(cfg.D) * 0.05).astype(np.float32)
    q = RefQwen35Hip()
    want = q.moe_rows(cfg.E, cfg.K, L, sgate, x)
    bufs = [be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s, L.sg, L.su, L.sd)]
    poisoned = replace(L, gu_s=np.zeros_like(L.gu_s), dn_s=np.zeros_like(L.dn_s), sg=np.zeros_like(L.sg),
                       su=np.zeros_like(L.su), sd=np.zeros_like(L.sd))
    got = q.moe_rows(cfg.E, cfg.K, poisoned, sgate, x, [int(b) for b in bufs])
    for b in bufs:
        b.free()
    assert np.all(np.isfinite(got))
    nw = float(np.max(np.abs(got - want))) / float(np.max(np.abs(want)))
    print(f"S={S_}: normwise {nw:.2e}")
    assert nw <= 2e-3, nw
