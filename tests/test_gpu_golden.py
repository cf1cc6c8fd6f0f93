"""The device path against the committed golden vectors of the compiled
reference (tests/golden/): top-k picks identical, moe_block output within the
benchmark tolerance (normwise max|a-b|/max|b| of the update <= 2e-3, and
elementwise |a-b|/max(|b|, 1e-3 max|b|) <= 2e-3), and the
grouped batch bit-identical to single-token calls on the same rows."""
import glob
import importlib.util
import os

import numpy as np
import pytest

from fullsize import errs
from oracle import synth
from sabrewing_amd.backend import DeviceLayer, desc_of

pytestmark = pytest.mark.gpu
TOL = 2e-3
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(os.path.basename(p)[4:-4] for p in glob.glob(os.path.join(GOLD, "moe_*.npz")))


def case_config(name):
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec); spec.loader.exec_module(mg)
    return mg.case_config(name)


@pytest.mark.parametrize("name", CASES)
def test_device_matches_golden(be, orc, name):
    cfg, seed, rows, cb = case_config(name)
    g = np.load(os.path.join(GOLD, f"moe_{name}.npz"))
    L = synth.make_layer(orc, cfg, seed, corr_bias_sigma=cb)
    dl = DeviceLayer.from_host(be, cfg, L)
    x, base, want = g["x"], g["out0"], g["out"]
    xd = be.upload(x)
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, rows)
    got = be.moe_block(desc_of(cfg), dl.weights(), x, base)
    single = np.stack([be.moe_block(desc_of(cfg), dl.weights(), x[s:s + 1], base[s:s + 1])[0] for s in range(rows)])
    xd.free(); dl.free()
    assert np.array_equal(sel, g["sel"])
    nw, el = errs(got, want, base)
    print(f"[{name}] normwise {nw:.2e}, elementwise {el:.2e}", flush=True)
    assert nw <= TOL and el <= TOL, (nw, el)
    assert np.array_equal(got.view(np.uint32), single.view(np.uint32))
