"""The parity tests' error measures (tests/fullsize.py) on closed-form cases."""
import numpy as np

from fullsize import ELEM_FLOOR, errs, normwise


def test_errs_closed_form():
    base = np.array([[0.5, -1.0, 2.0, 0.0]], np.float32)
    upd = np.array([[1.0, 1e-4, -2.0, 0.0]])
    want = base + upd
    got = base + upd + np.array([[1e-3, 1e-6, 0.0, 0.0]])
    nw, el = errs(got, want, base)
    assert np.isclose(nw, 1e-3 / 2.0, rtol=1e-3)                 # max|d| / max|want - base|
    # the 1e-4 entry is judged against ELEM_FLOOR * 2 = 2e-3, not its own size
    assert np.isclose(el, max(1e-3 / 1.0, 1e-6 / (ELEM_FLOOR * 2.0)), rtol=1e-3)
    assert np.isclose(normwise(got, want, base), nw, rtol=1e-6)


def test_errs_zero_error_and_floor_bites():
    base = np.zeros((2, 3), np.float32)
    want = np.array([[1.0, 1e-6, -1.0], [0.5, 0.25, 0.0]], np.float32)
    nw, el = errs(want.copy(), want, base)
    assert nw == 0.0 and el == 0.0
    got = want.copy()
    got[0, 1] += np.float32(2e-6)                                # 200 % of its own size, 2e-3 of the floor
    nw, el = errs(got, want, base)
    assert el < 2.1e-3 and el > 1.9e-3


def test_exact_layer_agrees_with_the_reference(orc):
    """exact_layer (float64) against the oracle's f32 moe_block on a small C2 layer
    (shared expert, softplus, gs=32) and a per-row-scale copy: they differ only by the
    f32 rounding, far below the bar; a transposed nibble order would not"""
    from dataclasses import replace
    from oracle import synth
    from sabrewing_amd import configs as cf
    from fullsize import exact_layer
    for cfg in (cf.scaled(cf.C2, D=512, E=32, K=6, I=256, Is=256),
                replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), name="gs0", gs=0)):
        L = synth.make_layer(orc, cfg, 31, corr_bias_sigma=0.01)
        x = synth.make_x(orc, cfg, 32, 3)
        base = synth.make_x(orc, cfg, 33, 3)
        want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base)
        _, sel, w = orc.route(synth.desc_of(cfg), L, x)
        ex = exact_layer(cfg, L, x, base, sel, w)
        nw, el = errs(want, ex, base)
        assert nw < 2e-5 and el < 2e-3, (cfg.name, nw, el)
        # the same with the nibbles of every byte swapped: far off
        Lb = replace(L, gu_q=((L.gu_q >> 4) | (L.gu_q << 4)).astype(np.uint8))
        assert errs(want, exact_layer(cfg, Lb, x, base, sel, w), base)[0] > 1e-2
