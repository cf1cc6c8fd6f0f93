"""The Inkling engine's MoE contract on the device (route_act INKLING + GATED
shared experts, c/inkling.c:1011-1183) against the oracle, whose Inkling layer
equals the engine's own moe() bit for bit (tests/test_oracle_ref.py,
tests/test_oracle_golden.py):

  * routing: logits over E + n_shared router rows, the picks and the K + n_shared
    weights (routed, then the shared gates') bit for bit;
  * the layer in the engine's default int8 activation route (the device's IDOT
    contract) bit for bit, against the oracle and against the compiled engine;
  * the layer in the default dot8 contract within the tolerance, every stream of a
    batch bit-identical to its single-stream call;
  * one full-size Inkling-shaped layer (D=4096, E=256, K=6, I=2048, 2 shared)."""
from dataclasses import replace

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.backend import DeviceLayer, desc_of

pytestmark = pytest.mark.gpu
TOL = 2e-3
GSCALE = np.float32(1.25)


def cfg_small(**kw):
    c = cf.scaled(cf.INKLING, D=512, E=64, K=6, I=256, Is=256, name="inkling-small")
    # the engine's route_scale * gate.global_scale, formed in float
    return replace(c, route_scale=float(np.float32(c.route_scale) * GSCALE), **kw)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def normwise(got, want, base):
    dw = want - base
    return float(np.max(np.abs((got - base) - dw))) / float(np.max(np.abs(dw)))


@pytest.mark.parametrize("S_", [1, 5, 40])
def test_inkling_routing_bits(be, orc, S_):
    cfg = cfg_small()
    L = synth.make_layer(orc, cfg, 201, corr_bias_sigma=0.02)
    x = synth.make_x(orc, cfg, 202, S_)
    dl = DeviceLayer.from_host(be, cfg, L)
    xd = be.upload(x)
    lg, sel, w = be.route(desc_of(cfg), dl.weights(), xd, S_)
    xd.free(); dl.free()
    lg_w, sel_w, w_w = orc.route(synth.desc_of(cfg), L, x)
    assert lg.shape == (S_, cfg.E + cfg.n_shared) and w.shape == (S_, cfg.K + cfg.n_shared)
    assert np.array_equal(bits(lg), bits(lg_w))
    assert np.array_equal(sel, sel_w)
    assert np.array_equal(bits(w), bits(w_w))


@pytest.mark.parametrize("S_", [1, 5, 40])
def test_inkling_layer_idot_bit_exact(be, orc, S_):
    """the device's IDOT contract is the engine's default int8 activation route: the
    whole layer -- routing, routed experts, gated shared experts, combine -- bit for bit"""
    from oracle.oracle import RefInkling
    cfg = cfg_small()
    L = synth.make_layer(orc, cfg, 211, corr_bias_sigma=0.02)
    x = synth.make_x(orc, cfg, 212, S_)
    z = np.zeros_like(x)
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, z, 1)
    if RefInkling.available():
        import os
        if os.environ.get("IDOT", "1") != "0":      # the engine reads IDOT once per process
            eng = RefInkling().moe(cfg.E, cfg.K, cfg.n_shared, cf.INKLING.route_scale, float(GSCALE), L, x)
            assert np.array_equal(bits(eng), bits(want))
    dl = DeviceLayer.from_host(be, cfg, L)
    prev = be.set_q4_mode(be.Q4_IDOT)
    try:
        got = be.moe_block(desc_of(cfg), dl.weights(), x, z)
    finally:
        be.set_q4_mode(prev)
        dl.free()
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("S_", [1, 5, 40])
def test_inkling_layer_dot8(be, orc, S_):
    cfg = cfg_small()
    L = synth.make_layer(orc, cfg, 221, corr_bias_sigma=0.02)
    x = synth.make_x(orc, cfg, 222, S_)
    base = synth.make_x(orc, cfg, 223, S_)
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base, 0)
    dl = DeviceLayer.from_host(be, cfg, L)
    got = be.moe_block(desc_of(cfg), dl.weights(), x, base)
    single = np.stack([be.moe_block(desc_of(cfg), dl.weights(), x[s:s + 1], base[s:s + 1])[0] for s in range(S_)])
    dl.free()
    assert normwise(got, want, base) <= TOL
    assert np.array_equal(bits(got), bits(single))


def test_inkling_routing_only_no_shared(be, orc):
    """INKLING routing with the shared experts left to the caller (shared NONE): the
    routed part of moe() on the device, the gates' weights from lag_hip_route"""
    cfg = cfg_small(shared_mode=cf.SHARED_NONE, Is=0)
    L = synth.make_layer(orc, cfg, 231, corr_bias_sigma=0.02)
    x = synth.make_x(orc, cfg, 232, 3)
    z = np.zeros_like(x)
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, z, 1)
    dl = DeviceLayer.from_host(be, cfg, L)
    prev = be.set_q4_mode(be.Q4_IDOT)
    try:
        got = be.moe_block(desc_of(cfg), dl.weights(), x, z)
    finally:
        be.set_q4_mode(prev)
        dl.free()
    assert np.array_equal(bits(got), bits(want))


def test_inkling_full_size_layer(be, orc):
    """one full-size Inkling-shaped layer (D=4096, E=256, K=6, I=Is=2048, two gated
    shared experts, per-row int4) at S = 4, device-generated, against the oracle"""
    from fullsize import host_layer
    cfg = replace(cf.INKLING, route_scale=float(np.float32(cf.INKLING.route_scale) * GSCALE))
    seed, S_ = 241, 4
    x = synth.make_x(orc, cfg, seed, S_)
    dl = DeviceLayer.generate(be, cfg, seed)
    try:
        L, sel_w = host_layer(be, orc, cfg, dl, seed, x)
        z = np.zeros_like(x)
        xd, od = be.upload(x), be.upload(z)
        _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
        be.moe_forward(desc_of(cfg), dl.weights(), xd, od, S_)
        got = be.d2h(od, x.shape, np.float32)
        prev = be.set_q4_mode(be.Q4_IDOT)
        be.h2d(od, z)
        be.moe_forward(desc_of(cfg), dl.weights(), xd, od, S_)
        got_idot = be.d2h(od, x.shape, np.float32)
        be.set_q4_mode(prev)
        xd.free(); od.free()
    finally:
        dl.free()
    assert np.array_equal(sel, sel_w)
    assert normwise(got, orc.moe_group_rows(synth.desc_of(cfg), L, x, z, 0), z) <= TOL
    assert np.array_equal(bits(got_idot), bits(orc.moe_group_rows(synth.desc_of(cfg), L, x, z, 1)))
