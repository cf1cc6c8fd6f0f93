"""The f16 MFMA grouped GEMMs of prefill (k_mfma.hip) against the dot8 ones
(k_dot8.hip): the same bits for every token, through the device-resident
block (lag_hip_moe_forward) and through the host-grouped entry
(lag_hip_moe_group), plus the oracle's bar (routing identical, normwise
max|a-b|/max|b| <= 2e-3 on the MoE update).

Both kernels form the same exact int32 per (weight row, group of 32 inputs)
and sum the same float terms in the same canonical order, so their outputs
must be equal bit for bit, whatever the tile shapes."""
from dataclasses import replace

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.backend import DeviceLayer, desc_of

pytestmark = pytest.mark.gpu
TOL = 2e-3
AUTO, DOT8, MFMA = 0, 1, 2

SMALL = [cf.scaled(cf.C1, D=512, E=16, K=4, I=256),
         cf.scaled(cf.C2, D=512, E=32, K=6, I=256, Is=256),
         cf.scaled(cf.C5_LAYER, D=512, E=32, K=8, I=384),
         replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), name="C2-small-gs0", gs=0),
         replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), name="C2-small-gs64", gs=64),
         cf.scaled(cf.C2_SIGMOID, D=768, E=32, K=6, I=384, Is=384, name="C2-D768"),     # 24 groups: padded runs
         cf.scaled(cf.C1, D=128, E=8, K=2, I=128, name="C1-D128"),                     # 4 groups: runs of 4
         cf.scaled(cf.C1, D=256, E=8, K=2, I=384, name="C1-D256-I384"),                # 8 and 12 groups
         cf.scaled(cf.QWEN, D=512, E=64, K=8, I=256, name="qwen35-small")]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def errs(got, want, base):
    dg, dw = got - base, want - base
    return float(np.max(np.abs(dg - dw))) / float(np.max(np.abs(dw)))


def block(be, cfg, dl, x, base, mode):
    prev = be.set_grouped_kernel(mode)
    try:
        return be.moe_block(desc_of(cfg), dl.weights(), x, base)
    finally:
        be.set_grouped_kernel(prev)


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: c.name)
@pytest.mark.parametrize("S_", [5, 40, 300])
def test_mfma_equals_dot8_small(be, orc, cfg, S_):
    L = synth.make_layer(orc, cfg, 51, corr_bias_sigma=0.01)
    x = synth.make_x(orc, cfg, 52, S_)
    base = synth.make_x(orc, cfg, 53, S_)
    dl = DeviceLayer.from_host(be, cfg, L)
    got_m = block(be, cfg, dl, x, base, MFMA)
    got_d = block(be, cfg, dl, x, base, DOT8)
    dl.free()
    assert np.array_equal(bits(got_m), bits(got_d))
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base)
    assert errs(got_m, want, base) <= TOL


def test_mfma_multi_tile_groups(be, orc):
    """groups of 100-200 tokens: two to four 64-token tiles each, the last one
    partial, and one group with exactly 64"""
    cfg = cf.scaled(cf.C1, D=512, E=8, K=2, I=256, name="C1-E8")
    L = synth.make_layer(orc, cfg, 61)
    S_ = 400
    x = synth.make_x(orc, cfg, 62, S_)
    base = np.zeros_like(x)
    dl = DeviceLayer.from_host(be, cfg, L)
    got_m = block(be, cfg, dl, x, base, MFMA)
    G, gexp, gbeg, gcnt = be.last_groups()
    got_d = block(be, cfg, dl, x, base, DOT8)
    # per-token (decode path) for a few streams
    single = np.stack([block(be, cfg, dl, x[s:s + 1], base[s:s + 1], AUTO)[0] for s in (0, 199, 399)])
    dl.free()
    assert max(gcnt[:G]) > 64
    assert np.array_equal(bits(got_m), bits(got_d))
    assert np.array_equal(bits(got_m[[0, 199, 399]]), bits(single))
    assert errs(got_m, orc.moe_block_rows(synth.desc_of(cfg), L, x, base), base) <= TOL


@pytest.mark.parametrize("cfg", [cf.C2, cf.C5_LAYER, cf.C1], ids=lambda c: c.name)
def test_mfma_equals_dot8_full_size(be, cfg):
    """full-size layers generated on the device (C2: D=4096 in 128 groups,
    down over 32; C5: I=1536, 48 groups), 256 tokens"""
    dl = DeviceLayer.generate(be, cfg, 71)
    S_ = 256
    rng = np.random.default_rng(72)
    x = rng.standard_normal((S_, cfg.D)).astype(np.float32)
    base = rng.standard_normal((S_, cfg.D)).astype(np.float32)
    got_m = block(be, cfg, dl, x, base, MFMA)
    got_d = block(be, cfg, dl, x, base, DOT8)
    dl.free()
    assert np.isfinite(got_m).all()
    assert np.array_equal(bits(got_m), bits(got_d))


def test_mfma_nan_group_propagates(be, orc):
    """a NaN input poisons exactly the outputs dot8 poisons (its group's factor is NaN)"""
    cfg = SMALL[1]
    L = synth.make_layer(orc, cfg, 81)
    x = synth.make_x(orc, cfg, 82, 64)
    x[5, 40] = np.nan
    base = np.zeros_like(x)
    dl = DeviceLayer.from_host(be, cfg, L)
    got_m = block(be, cfg, dl, x, base, MFMA)
    got_d = block(be, cfg, dl, x, base, DOT8)
    dl.free()
    assert np.array_equal(np.isnan(got_m), np.isnan(got_d))
    ok = ~np.isnan(got_d)
    assert np.array_equal(bits(got_m[ok]), bits(got_d[ok]))
