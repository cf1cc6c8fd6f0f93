"""The allocation-free forward (lag_hip_moe_forward_noalloc) against the arena
forward (lag_hip_moe_forward) through the C ABI: the same bits on two calls in a
row, the second with a smaller input (the static scratch keeps the first call's
contents), no change of free device memory across calls, and a shape whose
scratch does not fit refused before any launch."""
import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.backend import BackendError, DeviceLayer, desc_of

pytestmark = pytest.mark.gpu


def _pair(be, dl, cfg, x):
    """(arena forward, allocation-free forward) of x onto a zero residual"""
    z = np.zeros_like(x)
    xd, oa, on = be.upload(x), be.upload(z), be.upload(z)
    be.moe_forward(desc_of(cfg), dl.weights(), xd, oa, x.shape[0])
    be.moe_forward_noalloc(desc_of(cfg), dl.weights(), xd, on, x.shape[0])
    be.sync()
    a = be.d2h(oa, x.shape, np.float32)
    n = be.d2h(on, x.shape, np.float32)
    for b in (xd, oa, on):
        b.free()
    return a, n


@pytest.mark.parametrize("cfg,sizes", [(cf.C2, (32, 4, 1)), (cf.scaled(cf.C5_LAYER, D=512, E=32, K=8, I=384), (33, 5))],
                         ids=["C2", "C5-small"])
def test_noalloc_equals_arena_forward(be, orc, cfg, sizes):
    dl = DeviceLayer.generate(be, cfg, 8800)
    try:
        for S_ in sizes:                     # a larger call first, then smaller ones over the same scratch
            x = synth.make_x(orc, cfg, 8801 + S_, S_)
            a, n = _pair(be, dl, cfg, x)
            assert np.array_equal(a.view(np.uint32), n.view(np.uint32)), S_
    finally:
        dl.free()


def test_noalloc_allocates_nothing(be, orc):
    cfg = cf.scaled(cf.C2, D=512, E=32, K=6, I=256, Is=256)
    dl = DeviceLayer.generate(be, cfg, 8810)
    x = synth.make_x(orc, cfg, 8811, 16)
    xd, od = be.upload(x), be.upload(np.zeros_like(x))
    try:
        be.moe_forward_noalloc(desc_of(cfg), dl.weights(), xd, od, 16)
        be.sync()
        free0 = be.lib.lag_hip_free_bytes()
        for S_ in (16, 3, 16):
            be.moe_forward_noalloc(desc_of(cfg), dl.weights(), xd, od, S_)
        be.sync()
        assert be.lib.lag_hip_free_bytes() == free0
    finally:
        for b in (xd, od):
            b.free()
        dl.free()


def test_noalloc_refuses_oversized_shapes(be, orc):
    """the C2 layer at S = 128 needs ~36 MiB of scratch: refused with a message, and
    the entry keeps working afterwards"""
    cfg = cf.C2
    dl = DeviceLayer.generate(be, cfg, 8820)
    x = synth.make_x(orc, cfg, 8821, 128)
    xd, od = be.upload(x), be.upload(np.zeros_like(x))
    try:
        with pytest.raises(BackendError, match="scratch"):
            be.moe_forward_noalloc(desc_of(cfg), dl.weights(), xd, od, 128)
        a, n = _pair(be, dl, cfg, x[:2])
        assert np.array_equal(a.view(np.uint32), n.view(np.uint32))
    finally:
        for b in (xd, od):
            b.free()
        dl.free()
