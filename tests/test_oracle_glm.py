"""The oracle's GLM routing (oracle/sw_oracle.c sw_glm_*, oracle.py glm_select),
the contract of coli_hip_pipe_router, pinned on the CPU:

  * the logits GEMV equals the reference's own c/quant.h matmul, compiled from
    the reference (oracle/_ref/libref_glm_avx512.so), bit for bit at every
    input count 1..80 and at the GLM shapes (its vector body and scalar tail),
    and the committed vectors written from it (tests/golden/glm_router.npz);
  * the selection against what the mathematics fixes: a brute-force ranking
    (value descending, then id), ties to the lowest id, NaN and values at or
    below -1e30 never chosen, the fallback of an empty pass, the top-p cut at
    the first cumulative weight >= p * total, the normalisation to 1 and the
    routed scale."""
import numpy as np
import pytest

from oracle.oracle import Oracle, RefGlm


@pytest.fixture(scope="module")
def o():
    return Oracle()


@pytest.mark.skipif(not RefGlm.available(), reason="reference GLM router not built (oracle/_ref)")
def test_logits_equal_compiled_reference(o):
    r = RefGlm()
    rng = np.random.default_rng(1)
    for D in list(range(1, 81)) + [1003, 4096, 5120, 5127, 6144]:
        x = rng.standard_normal((2, D)).astype(np.float32)
        W = (rng.standard_normal((17, D)) * 0.05).astype(np.float32)
        a, b = o.glm_matmul(x, W), r.matmul(x, W)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), D


def test_logits_equal_golden(o):
    """the committed vectors of the compiled c/quant.h matmul (tests/golden/make_glm_golden.py):
    the pin without the reference present"""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "glm_router.npz"))
    for D in (5, 13, 37, 5120, 5127):
        got = o.glm_matmul(g[f"x_{D}"], g[f"w_{D}"])
        assert np.array_equal(got.view(np.uint32), g[f"y_{D}"].view(np.uint32)), D


def test_logits_are_sigmoid_of_the_dot(o):
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((40, 300)) * 0.1).astype(np.float32)
    x = rng.standard_normal(300).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    lg, ch = o.glm_logits(x, W, b)
    dot = o.glm_matmul(x.reshape(1, -1), W)[0].astype(np.float64)
    assert np.allclose(lg, 1 / (1 + np.exp(-dot)), rtol=1e-6, atol=0)
    assert np.array_equal(ch, (lg + b).astype(np.float32))
    # a plain dot of this size agrees with the chain to f32 accuracy (a dropped or
    # transposed operand would not)
    assert np.allclose(dot, W.astype(np.float64) @ x.astype(np.float64), rtol=1e-4, atol=1e-5)


def test_selection_brute_force(o):
    rng = np.random.default_rng(3)
    for trial in range(40):
        E, K = int(rng.integers(8, 300)), int(rng.integers(1, 9))
        lg = rng.random(E).astype(np.float32)
        ch = (lg + rng.standard_normal(E).astype(np.float32) * 0.01).astype(np.float32)
        if trial % 4 == 0:                                   # ties
            ch[rng.integers(0, E, 5)] = ch.max()
        idx, w, ke = o.glm_select(lg, ch, K, 0.0, 0, 1.0)
        order = sorted(range(E), key=lambda e: (-float(ch[e]), e))[:K]
        assert list(idx) == order and ke == K
        assert np.array_equal(w, lg[order])
        idx, w, ke = o.glm_select(lg, ch, K, 0.0, 1, 2.5)   # normalised, then scaled
        assert list(idx) == order
        assert abs(float(w.astype(np.float64).sum()) - 2.5) < 1e-5


def test_selection_special_values(o):
    lg = np.array([0.2, 0.9, 0.5, 0.7, 0.1], np.float32)
    ch = np.array([np.nan, 0.9, -1e30, -np.inf, 0.3], np.float32)
    idx, _, _ = o.glm_select(lg, ch, 4, 0.0, 0, 1.0)
    # 1 and 4 are the only candidates; the empty passes take kk (2, then 3)
    assert list(idx) == [1, 4, 2, 3]
    idx, _, _ = o.glm_select(lg, np.full(5, np.nan, np.float32), 3, 0.0, 0, 1.0)
    assert list(idx) == [0, 1, 2]
    idx, _, _ = o.glm_select(lg[:2], np.array([0.5, 0.4], np.float32), 4, 0.0, 0, 1.0)
    assert list(idx) == [0, 1, 0, 0]                         # more passes than experts: kk < E ? kk : 0


def test_top_p_cut(o):
    # kept weights 0.4 0.3 0.2 0.1 (sorted); tot = 1: p = 0.65 keeps 2, 0.75 keeps 3, 0.95 keeps 4
    lg = np.array([0.1, 0.4, 0.2, 0.3], np.float32)
    ch = np.array([0.35, 0.3, 0.2, 0.1], np.float32)        # selection order 0, 1, 2, 3
    for p, keep in ((0.65, 2), (0.75, 3), (0.95, 4), (0.3, 1)):
        idx, w, ke = o.glm_select(lg, ch, 4, p, 1, 1.0)
        assert ke == keep
        assert list(idx[:keep]) == [1, 3, 2, 0][:keep]       # re-sorted by weight, descending
        assert abs(float(w[:keep].astype(np.float64).sum()) - 1.0) < 1e-6
    idx, w, ke = o.glm_select(lg, ch, 4, 1.0, 0, 1.0)        # p >= 1: no cut, no re-sort
    assert ke == 4 and list(idx) == [0, 1, 2, 3]
