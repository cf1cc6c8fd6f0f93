"""The oracle against the committed golden vectors (tests/golden/), bit for bit.

The fixtures were written by tests/golden/make_golden.py from the compiled
reference: router logits, top-k picks and the moe_block output of seeded
small layers, plus the int4 known answer of c/tests/test_backend_cuda.cu:105-110.
These tests need neither the reference nor a GPU.
"""
import glob
import os

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(os.path.basename(p)[4:-4] for p in glob.glob(os.path.join(GOLD, "moe_*.npz")))


def load_case(orc, name):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec); spec.loader.exec_module(mg)
    cfg, seed, rows, cb = mg.case_config(name)
    g = np.load(os.path.join(GOLD, f"moe_{name}.npz"))
    assert int(g["seed"]) == seed and int(g["rows"]) == rows and float(g["corr_bias_sigma"]) == cb
    L = synth.make_layer(orc, cfg, seed, corr_bias_sigma=cb)
    return cfg, L, g


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fixture_set_complete():
    assert set(CASES) >= {"c1_small", "c2_sigmoid_small", "c5_small", "c2_sigmoid_mid", "c4_zipf_sigmoid_small"}
    assert os.path.exists(os.path.join(GOLD, "kat_q4_rows.npz"))
    assert os.path.exists(os.path.join(GOLD, "route_callers.npz"))


def test_kat_q4_rows(orc):
    k = np.load(os.path.join(GOLD, "kat_q4_rows.npz"))
    p = k["q4"].reshape(2, 2)
    for mode, exact in ((0, 0), (0, 1)):
        assert np.array_equal(orc.matmul_q4(k["x"], p, k["s4"], mode, exact), k["want"])
    # closed form: low nibble first, v = nibble - 8, times the row scale
    lo, hi = (p & 15).astype(np.int32) - 8, (p >> 4).astype(np.int32) - 8
    W = np.stack([lo, hi], axis=-1).reshape(2, 4) * k["s4"][:, None]
    assert np.array_equal(W, [[-8, -1, 0, 7], [0.25, 0.5, 0.75, 1.0]])
    assert np.array_equal((k["x"] @ W.T).astype(np.float32), k["want"])


@pytest.mark.parametrize("name", CASES)
def test_inputs_regenerate(orc, name):
    cfg, L, g = load_case(orc, name)
    rows = int(g["rows"])
    assert np.array_equal(bits(synth.make_x(orc, cfg, int(g["seed"]), rows)), bits(g["x"]))
    assert np.array_equal(bits(synth.make_x(orc, cfg, int(g["seed"]) + 1, rows)), bits(g["out0"]))


@pytest.mark.parametrize("name", CASES)
def test_route_matches_golden(orc, name):
    cfg, L, g = load_case(orc, name)
    lg, sel, _ = orc.route(synth.desc_of(cfg), L, g["x"])
    assert np.array_equal(bits(lg), bits(g["logits"]))
    assert np.array_equal(sel, g["sel"])


@pytest.mark.parametrize("name", CASES)
def test_moe_block_matches_golden(orc, name):
    cfg, L, g = load_case(orc, name)
    d = synth.desc_of(cfg)
    assert np.array_equal(bits(orc.moe_block_rows(d, L, g["x"], g["out0"])), bits(g["out"]))
    assert np.array_equal(bits(orc.moe_group_rows(d, L, g["x"], g["out0"])), bits(g["out"]))


def test_planted_mistake_is_caught(orc):
    """a wrong sign in one expert's down scale changes the output bits: the
    comparison above is sharp enough to see a one-expert slip"""
    cfg, L, g = load_case(orc, "c1_small")
    d = synth.desc_of(cfg)
    sel = g["sel"][0]
    ngI = cfg.I // cfg.gs
    e = int(sel[0])
    L.dn_s = L.dn_s.copy()
    L.dn_s[e * cfg.D * ngI:(e * cfg.D + 1) * ngI] *= -1
    assert not np.array_equal(bits(orc.moe_block_rows(d, L, g["x"][:1], g["out0"][:1])), bits(g["out"][:1]))


def test_callers_routing_golden(orc):
    """A17: OLMoE's and qwen35's routing against the fixtures their own
    compiled sources wrote (tests/golden/route_callers.npz)"""
    g = np.load(os.path.join(GOLD, "route_callers.npz"))
    lg, K = g["logits"], int(g["K"])
    E = lg.shape[1]
    for norm in (0, 1):
        d = synth.Desc(E, K, cf.ROUTE_SOFTMAX_OLMOE, 0, norm, 1.0, 0)
        sel, w = orc.route_logits(d, lg)
        assert np.array_equal(sel, g["olmoe_sel"][norm]) and np.array_equal(bits(w), bits(g["olmoe_w"][norm]))
    d = synth.Desc(E, K, cf.ROUTE_SOFTMAX_QWEN, 0, 0, 1.0, 0)
    sel, w = orc.route_logits(d, lg)
    assert np.array_equal(sel, g["qwen_sel"]) and np.array_equal(bits(w), bits(g["qwen_w"]))
    # closed forms: qwen's weights sum to 1 in double within a float rounding each; picks distinct
    assert all(len(set(r)) == K for r in sel)
    ok = np.isfinite(w).all(axis=1)
    assert np.allclose(w[ok].astype(np.float64).sum(axis=1), 1.0, atol=1e-6)


def test_inkling_layer_golden(orc):
    """The oracle's Inkling contract (route_act 6 + gated shared experts) reproduces the
    Inkling engine's own moe() bit for bit, on both of its activation routes (fixture
    written by tests/golden/make_inkling_golden.py from the compiled engine)"""
    import importlib.util
    from dataclasses import replace
    spec = importlib.util.spec_from_file_location("mig", os.path.join(GOLD, "make_inkling_golden.py"))
    mig = importlib.util.module_from_spec(spec); spec.loader.exec_module(mig)
    g = np.load(os.path.join(GOLD, "inkling_moe.npz"))
    assert int(g["seed"]) == mig.SEED and int(g["rows"]) == mig.ROWS
    cfg, L, x = mig.layer_and_x(orc)
    assert np.array_equal(bits(x), bits(g["x"]))
    # the engine's route_scale * gate.global_scale, formed in float
    d = synth.desc_of(replace(cfg, route_scale=float(np.float32(cfg.route_scale) * g["gscale"])))
    z = np.zeros_like(x)
    for mode, key in ((1, "out_idot"), (0, "out_f32")):
        assert np.array_equal(bits(orc.moe_block_rows(d, L, x, z, mode)), bits(g[key])), key
        assert np.array_equal(bits(orc.moe_group_rows(d, L, x, z, mode)), bits(g[key])), key
    # the routing itself against a brute-force reading of c/inkling.c:1027-1043
    lg, sel, w = orc.route(d, L, x)
    assert lg.shape == (x.shape[0], cfg.E + cfg.n_shared) and w.shape == (x.shape[0], cfg.K + cfg.n_shared)
    sig = lambda v: np.float32(1) / (np.float32(1) + np.exp(-v.astype(np.float64)).astype(np.float32))
    for s in range(x.shape[0]):
        key = sig(lg[s, :cfg.E]) + L.corr_bias
        assert set(sel[s]) == set(np.argsort(-key, kind="stable")[:cfg.K])
        assert abs(float(np.sum(w[s])) - d.route_scale) < 1e-5 * d.route_scale
