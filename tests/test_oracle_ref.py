"""The oracle restatement against the compiled reference (oracle/_ref), bit for bit.

Every kernel of the path on seeded inputs, including the shapes that take the
scalar tails, plus moe_block over laguna-shaped hooks and the reference
engine's own lag_moe_rows (per-token and grouped) at gs = 0.
"""
from dataclasses import replace

import numpy as np
import pytest

from oracle import synth
from oracle.oracle import RefLaguna
from sabrewing_amd import configs as cf


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32); b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(20261201)


@pytest.mark.parametrize("S,I,O", [(1, 2048, 64), (3, 4096, 256), (2, 100, 7), (1, 33, 5), (4, 16, 3)])
def test_router_contracts(orc, ref, rng, S, I, O):
    x = rng.standard_normal((S, I)).astype(np.float32)
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    for exact in (0, 1):
        assert bits_equal(orc.matmul_f32(x, W, exact), ref.matmul_f32(x, W, exact))
        Wb = orc.to_bf16(W)
        assert bits_equal(orc.matmul_bf16(x, Wb, exact), ref.matmul_bf16(x, Wb, exact))


@pytest.mark.parametrize("S,I,O,gs", [(1, 2048, 64, 32), (3, 1024, 96, 32), (2, 512, 8, 64), (2, 200, 4, 64),
                                      (1, 65, 3, 64), (2, 201, 4, 64), (1, 33, 2, 16), (8, 320, 6, 64),
                                      (1, 64, 4, 128)])
def test_i4_grouped(orc, ref, rng, S, I, O, gs):
    x = rng.standard_normal((S, I)).astype(np.float32)
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    p, s = orc.quant_i4(W, gs)
    assert bits_equal(orc.matmul_i4_grouped(x, p, s, gs), ref.matmul_i4_grouped(x, p, s, gs))


@pytest.mark.parametrize("S,I,O", [(1, 2048, 64), (4, 1024, 96), (1, 100, 8), (3, 96, 8), (2, 8192, 4), (1, 8256, 3)])
def test_q4_rows(orc, ref, rng, S, I, O):
    x = rng.standard_normal((S, I)).astype(np.float32)
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    p, s = orc.quant_i4(W, 0)
    for mode, exact in ((0, 0), (1, 0), (0, 1)):
        assert bits_equal(orc.matmul_q4(x, p, s, mode, exact), ref.matmul_q4(x, p, s, mode, exact)), (mode, exact)


@pytest.mark.parametrize("S,I,O", [(1, 64, 5), (3, 4096, 37), (2, 96, 7), (2, 40, 3), (1, 6144, 64)])
def test_bf16_round_x(orc, ref, rng, S, I, O):
    """inkling's matmul_h contract (bf16-rounded activations, vdpbf16ps lanes), with
    denormal, huge and halfway activations and denormal / extreme bf16 weights; I = 40
    takes the reference's f32-activation route"""
    x = rng.standard_normal((S, I)).astype(np.float32)
    x[0, :5] = [1e-39, -1e-40, 3e38, np.float32(1.0000001), -0.0]
    W = orc.to_bf16((rng.standard_normal((O, I)) * 0.05).astype(np.float32))
    W[0, :4] = [0x0001, 0x8003, 0x7F7F, 0x0080]
    assert bits_equal(orc.matmul_bf16_rx(x, W), ref.matmul_bf16(x, W, round_x=1))
    tiny = np.full((1, 64), 1e-20, np.float32)         # products below the normal range: flushed
    Wt = orc.to_bf16(np.full((3, 64), 1e-20, np.float32))
    assert bits_equal(orc.matmul_bf16_rx(tiny, Wt), ref.matmul_bf16(tiny, Wt, round_x=1))


@pytest.mark.parametrize("S,I,O", [(1, 64, 5), (3, 4096, 37), (2, 96, 7), (2, 40, 3), (1, 6144, 64)])
def test_q8_rows(orc, ref, rng, S, I, O):
    """int8 weights with row scales (matmul_q8_k), both activation contracts"""
    x = rng.standard_normal((S, I)).astype(np.float32)
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    sc = (rng.random(O) * 1e-3).astype(np.float32)
    for mode in (0, 1):
        assert bits_equal(orc.matmul_q8(x, q, sc, mode), ref.matmul_q8(x, q, sc, mode)), mode


def test_softmax_topk(orc, ref, rng):
    for n in (8, 64, 256):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        assert bits_equal(orc.softmax_row(v), ref.softmax_row(v))
        for K in (1, 4, min(10, n)):
            assert np.array_equal(orc.topk(v, K), ref.topk(v, K))
            b = (rng.standard_normal(n) * 0.1).astype(np.float32)
            assert np.array_equal(orc.topk(v, K, b), ref.topk(v, K, b))
    # ties, signed zeros, NaN and values at the -1e30 threshold
    v = np.array([0.5, 0.5, -0.0, 0.0, np.nan, -1e30, 0.5, -np.inf], np.float32)
    for K in range(1, 9):
        assert np.array_equal(orc.topk(v, K), ref.topk(v, K))
    v = np.full(6, np.nan, np.float32)
    assert np.array_equal(orc.topk(v, 4), ref.topk(v, 4))


def test_scalar_math(orc, ref):
    xs = np.concatenate([np.linspace(-30, 30, 20001), [-104.0, -88.0, 0.0, -0.0, 20.0, 20.000002, 88.7]]).astype(np.float32)
    f = lambda lib, name: np.array([getattr(lib, name)(float(v)) for v in xs], np.float32)
    assert bits_equal(f(orc.lib, "sw_siluf"), f(ref.lib, "ref_siluf"))
    assert bits_equal(f(orc.lib, "sw_softplusf"), f(ref.lib, "ref_softplusf"))


SMALL = [cf.scaled(cf.C1, D=256, E=16, K=4, I=128),
         cf.scaled(cf.C2_SIGMOID, D=256, E=32, K=6, I=128, Is=128),
         cf.scaled(cf.C5_LAYER, D=256, E=32, K=8, I=384)]


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: c.name)
def test_moe_block_vs_ref(orc, ref, cfg):
    L = synth.make_layer(orc, cfg, 42, corr_bias_sigma=0.01)
    d = synth.desc_of(cfg)
    x = synth.make_x(orc, cfg, 42, 5)
    out0 = synth.make_x(orc, cfg, 43, 5)         # a non-zero residual
    a = orc.moe_block_rows(d, L, x, out0)
    assert bits_equal(a, ref.moe_block_rows(d, L, x, out0))
    assert bits_equal(a, orc.moe_group_rows(d, L, x, out0))          # grouped == per-token


def test_laguna_engine_path(orc):
    if not RefLaguna.available():
        pytest.skip("compiled reference engine not built")
    lag = RefLaguna()
    cfg = replace(cf.scaled(cf.C2_SIGMOID, D=256, E=32, K=6, I=128, Is=128), gs=0, router_bf16=False)
    L = synth.make_layer(orc, cfg, 7, corr_bias_sigma=0.01)
    d = synth.desc_of(cfg)
    x = synth.make_x(orc, cfg, 7, 6)
    h0 = synth.make_x(orc, cfg, 8, 6)
    assert bits_equal(orc.moe_block_rows(d, L, x, h0), lag.moe_rows(d, L, x, h0, group=0))
    assert bits_equal(orc.moe_group_rows(d, L, x, h0), lag.moe_rows(d, L, x, h0, group=1))
    assert bits_equal(orc.moe_block_rows(d, L, x[:1], h0[:1]), lag.moe_rows(d, L, x[:1], h0[:1]))
    for mode in (2,):                                # g_exact: the double-accumulate kernels
        assert bits_equal(orc.moe_block_rows(d, L, x, h0, mode), lag.moe_rows(d, L, x, h0, exact=1, group=0))


_IDOT_CHILD = r"""
import sys
import numpy as np
from dataclasses import replace
from oracle import synth
from oracle.oracle import Oracle, RefLaguna
from sabrewing_amd import configs as cf
orc, lag = Oracle(), RefLaguna()
cfg = replace(cf.scaled(cf.C2_SIGMOID, D=256, E=32, K=6, I=128, Is=128), gs=0, router_bf16=False)
L = synth.make_layer(orc, cfg, 17, corr_bias_sigma=0.01)
d = synth.desc_of(cfg)
x, h0 = synth.make_x(orc, cfg, 18, 5), synth.make_x(orc, cfg, 19, 5)
a = orc.moe_block_rows(d, L, x, h0, 1).view(np.uint32)
b = lag.moe_rows(d, L, x, h0, group=0).view(np.uint32)
c = lag.moe_rows(d, L, x, h0, group=1).view(np.uint32)
f = orc.moe_block_rows(d, L, x, h0, 0).view(np.uint32)
print("IDOT-OK" if np.array_equal(a, b) and np.array_equal(a, c) and not np.array_equal(a, f) else "IDOT-MISMATCH")
"""


def test_laguna_engine_idot():
    """the oracle's IDOT layer (mode 1) against the reference engine's CPU tier under
    LAG_IDOT=1 (c/laguna.c:204-207, read once per process: a child process), per-token
    and grouped (c/laguna.c:739), bit for bit; the f32 contract differs"""
    import os
    import subprocess
    import sys
    if not RefLaguna.available():
        pytest.skip("compiled reference engine not built")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, LAG_IDOT="1", PYTHONPATH=root)
    r = subprocess.run([sys.executable, "-c", _IDOT_CHILD], env=env, cwd=root, capture_output=True, text=True, timeout=300)
    assert "IDOT-OK" in r.stdout, r.stdout + r.stderr


def _logit_sets(rng, E):
    """random rows, rows with exact ties, a NaN row, -inf entries, huge logits"""
    rows = [(rng.standard_normal(E) * s).astype(np.float32) for s in (0.5, 3.0, 30.0)]
    t = (rng.standard_normal(E) * 2).astype(np.float32)
    t[::3] = t[0]                                       # ties of the leading value
    rows.append(t)
    r = rng.standard_normal(E).astype(np.float32); r[E // 2] = np.nan
    rows.append(r)
    r = rng.standard_normal(E).astype(np.float32); r[:E // 4] = -np.inf
    rows.append(r)
    rows.append(np.full(E, -1e31, np.float32))          # below OLMoE's -1e30 start
    rows.append(np.full(E, 5.0, np.float32))            # all equal
    return np.stack(rows)


@pytest.mark.parametrize("E,K", [(64, 8), (256, 8), (60, 6), (8, 8)])
def test_other_callers_routing_vs_ref(orc, rng, E, K):
    """A17: the OLMoE engine's routing (c/olmoe.c:607-632) and qwen35's
    moe_route (c/qwen35.c:558-589), each from its own compiled source"""
    from oracle.oracle import RefCallers
    if not RefCallers.available():
        pytest.skip("compiled reference callers not built")
    rc = RefCallers()
    lg = _logit_sets(rng, E)
    for row in lg:
        assert bits_equal(orc.softmax_row_olmoe(row), rc.olmoe_softmax_row(row))
        for norm in (0, 1):
            d = synth.Desc(E, K, cf.ROUTE_SOFTMAX_OLMOE, 0, norm, 1.0, 0)
            sel, w = orc.route_logits(d, row[None])
            rs, rw = rc.olmoe_route(row, K, norm)
            assert np.array_equal(sel[0], rs) and bits_equal(w[0], rw)
        d = synth.Desc(E, K, cf.ROUTE_SOFTMAX_QWEN, 0, 0, 1.0, 0)
        sel, w = orc.route_logits(d, row[None])
        qs, qw = rc.qwen_route(row, K)
        assert np.array_equal(sel[0], qs) and bits_equal(w[0], qw)


def test_sqrt_softplus_gate(orc, ref, rng):
    """route_act 5: the oracle's scores are the compiled reference's softplusf then an
    IEEE sqrt (c/deepseek.c:854), selected with the correction bias by moe_topk and
    weighted as moe_block's sigmoid scores, renormalised (c/moe_block.h:115-122)"""
    from oracle.oracle import Ref
    cfg = cf.scaled(cf.C2_SQRTSP, D=512, E=64, K=6, I=256, Is=256)
    L = synth.make_layer(orc, cfg, 31, corr_bias_sigma=0.01)
    x = synth.make_x(orc, cfg, 32, 7)
    lg, sel, w = orc.route(synth.desc_of(cfg), L, x)
    for s in range(x.shape[0]):
        sp = np.array([ref.lib.ref_softplusf(float(v)) for v in lg[s]], np.float32)
        sc = np.sqrt(sp)                                   # float32 sqrt: correctly rounded
        choice = sc + L.corr_bias
        order = sorted(range(cfg.E), key=lambda e: (-float(choice[e]), e))[:cfg.K]
        assert list(sel[s]) == order
        want = sc[order] / np.float32(sum(np.float32(v) for v in sc[order]))   # route_scale: after the combine
        assert np.allclose(w[s], want, rtol=2e-7, atol=0)


INK_CHILD = """
import sys, numpy as np
sys.path.insert(0, sys.argv[1])
from oracle.oracle import RefInkling
z = np.load(sys.argv[2])
from types import SimpleNamespace
L = SimpleNamespace(**{k: (z[k] if z[k].size else None) for k in ("router", "corr_bias", "gu_q", "gu_s", "dn_q", "dn_s", "sg", "su", "sd")}, D=int(z["D"]), I=int(z["I"]))
np.save(sys.argv[3], RefInkling().moe(int(z["E"]), int(z["K"]), int(z["ns"]), float(z["rs"]), float(z["gs"]), L, z["x"]))
"""


@pytest.mark.parametrize("S_", [1, 4])
def test_inkling_moe_vs_engine(orc, tmp_path, S_):
    """the oracle's Inkling layer against the engine's own moe() (oracle/_ref,
    compiled from c/inkling.c), bit for bit: the engine's default int8 activation
    route in this process, its f32 route (IDOT=0) in a child process (the engine
    reads IDOT once)"""
    import os, subprocess, sys
    from oracle.oracle import RefInkling
    if not RefInkling.available():
        pytest.skip("compiled Inkling engine (oracle/_ref) not built")
    cfg = cf.scaled(cf.INKLING, D=512, E=64, K=6, I=256, Is=256, name="inkling-pin")
    gsc = 0.75
    L = synth.make_layer(orc, cfg, 131 + S_, corr_bias_sigma=0.02)
    x = synth.make_x(orc, cfg, 132, S_)
    d = synth.desc_of(replace(cfg, route_scale=float(np.float32(cfg.route_scale) * np.float32(gsc))))
    z = np.zeros_like(x)
    if "IDOT" not in os.environ:
        want = RefInkling().moe(cfg.E, cfg.K, cfg.n_shared, cfg.route_scale, gsc, L, x)
        assert bits_equal(orc.moe_block_rows(d, L, x, z, 1), want)
        assert bits_equal(orc.moe_group_rows(d, L, x, z, 1), want)
    f = tmp_path / "layer.npz"
    np.savez(f, x=x, D=L.D, I=L.I, E=cfg.E, K=cfg.K, ns=cfg.n_shared, rs=cfg.route_scale, gs=gsc,
             **{k: getattr(L, k) for k in ("router", "corr_bias", "gu_q", "gu_s", "dn_q", "dn_s", "sg", "su", "sd")})
    env = dict(os.environ, IDOT="0")
    out = tmp_path / "out.npy"
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.run([sys.executable, "-c", INK_CHILD, root, str(f), str(out)], env=env, check=True)
    assert bits_equal(orc.moe_block_rows(d, L, x, z, 0), np.load(out))
