"""The oracle against what the mathematics fixes, independently of the
reference build: known-answer vectors of the reference tests, brute-force
double dequantisation, closed forms of the gate activations, invariants of
top-k and of the counting sort, and the quantiser's error bound."""
import math

import numpy as np
import pytest

from sabrewing_amd import synth as S


def test_nibble_kat(orc):
    # c/tests/test_backend_cuda.cu:105-110: rows [-8,-1,0,7] and [1,2,3,4],
    # packed low nibble first, scales {1, 0.25}, x = {1,-2,3,-4} -> {-34, -2.5}
    q4 = np.array([[0x70, 0xf8], [0xa9, 0xcb]], np.uint8)
    s4 = np.array([1.0, 0.25], np.float32)
    x = np.array([[1, -2, 3, -4]], np.float32)
    for mode, exact in ((0, 0), (0, 1)):
        assert np.allclose(orc.matmul_q4(x, q4, s4, mode, exact), [[-34.0, -2.5]], atol=1e-6)
    # the same rows as group-scaled int4 with one group per row
    assert np.allclose(orc.matmul_i4_grouped(x, q4, s4.reshape(2, 1), 4), [[-34.0, -2.5]], atol=1e-6)


def brute_i4(x, p, s, gs):
    """double dequant reference (c/tests/test_i4_grouped.c:30-54): value, sum of |terms|"""
    S_, I = x.shape; O = p.shape[0]
    ng = (I + gs - 1) // gs if gs > 0 else 1
    nib = np.empty((O, I), np.int64)
    nib[:, 0::2] = (p[:, : (I + 1) // 2] & 0xF)[:, : (I + 1) // 2]
    nib[:, 1::2] = (p[:, : I // 2] >> 4)
    sc = s.reshape(O, ng).astype(np.float64)
    gi = (np.arange(I) // gs) if gs > 0 else np.zeros(I, np.int64)
    w = (nib - 8) * sc[:, gi]
    terms = x.astype(np.float64)[:, None, :] * w[None, :, :]
    return terms.sum(-1), np.abs(terms).sum(-1)


@pytest.mark.parametrize("S_,I,O,gs,edges", [(2, 512, 8, 64, 0), (1, 256, 4, 64, 1), (2, 200, 4, 64, 0),
                                            (1, 65, 3, 64, 0), (2, 201, 4, 64, 0), (1, 33, 2, 16, 0),
                                            (8, 320, 6, 64, 0), (1, 4096, 16, 32, 0)])
def test_i4_grouped_vs_brute(orc, S_, I, O, gs, edges):
    rng = np.random.default_rng(I * 31 + O)
    p = rng.integers(0, 256, size=(O, (I + 1) // 2), dtype=np.uint8)
    if I % 2:
        p[:, -1] &= 0x0F
    if edges:
        p.reshape(-1)[:64] = np.where(np.arange(64) % 2 == 1, 0x00, 0xFF)
    ng = (I + gs - 1) // gs
    s = ((0.001 + rng.integers(0, 1000, size=(O, ng)) / 1000.0) * rng.choice([-1, 1], size=(O, ng))).astype(np.float32)
    x = (rng.integers(0, 2001, size=(S_, I)) / 1000.0 - 1.0).astype(np.float32)
    y = orc.matmul_i4_grouped(x, p, s, gs)
    want, mag = brute_i4(x, p, s, gs)
    rel = np.abs(y - want) / np.maximum(mag, 1e-30)
    assert rel.max() < 1e-6                     # c/tests/test_i4_grouped.c:84 bound


def test_q4_rows_vs_brute(orc):
    rng = np.random.default_rng(5)
    I, O = 2048, 64
    W = rng.standard_normal((O, I)).astype(np.float32)
    p, s = orc.quant_i4(W, 0)
    x = rng.standard_normal((3, I)).astype(np.float32)
    want, mag = brute_i4(x, p, s, 0)
    assert np.array_equal(orc.matmul_q4(x, p, s, 0, 1), want.astype(np.float32))   # exact path: double sum
    assert (np.abs(orc.matmul_q4(x, p, s, 0, 0) - want) / mag).max() < 1e-6
    # IDOT: int8 activations per 32-block are lossy but bounded (tools/kernel_check.c:115)
    yi = orc.matmul_q4(x, p, s, 1, 0)
    assert np.linalg.norm(yi - want) / np.linalg.norm(want) < 3e-2


def test_quantiser_bounds(orc):
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    W[3] = 0.0                                  # all-zero row: scale floor 1e-8, nibbles 8
    for gs in (0, 32, 64):
        p, s = orc.quant_i4(W, gs)
        ng = s.shape[1]
        nib = np.empty(W.shape, np.int64)
        nib[:, 0::2] = p & 0xF
        nib[:, 1::2] = p >> 4
        gi = np.arange(256) // (gs if gs else 256)
        deq = (nib - 8) * s[:, gi]
        amax = np.abs(W).reshape(16, ng, -1).max(-1)
        assert np.allclose(s, np.maximum(amax / np.float32(7), np.float32(1e-8)), rtol=0, atol=0)
        assert np.all(np.abs(deq - W) <= s[:, gi] * 0.5 * (1 + 1e-6) + 1e-12)   # round to nearest, no clipping
        assert np.all(nib[3] == 8)


def test_gate_closed_forms(orc):
    xs = np.linspace(-25, 25, 5001).astype(np.float32)
    sig = np.array([orc.lib.sw_sigmoidf(float(v)) for v in xs])
    assert np.allclose(sig, 1 / (1 + np.exp(-xs.astype(np.float64))), rtol=2e-7, atol=1e-30)
    sp = np.array([orc.lib.sw_softplusf(float(v)) for v in xs])
    want = np.where(xs > 20, xs, np.log1p(np.exp(xs.astype(np.float64))))
    assert np.allclose(sp, want, rtol=3e-7, atol=1e-30)
    assert orc.lib.sw_softplusf(20.5) == np.float32(20.5)                # identity branch above 20
    si = np.array([orc.lib.sw_siluf(float(v)) for v in xs])
    assert np.allclose(si, xs / (1 + np.exp(-xs.astype(np.float64))), rtol=3e-7, atol=1e-30)
    v = np.random.default_rng(3).standard_normal(256).astype(np.float32) * 4
    sm = orc.softmax_row(v)
    e = np.exp(v.astype(np.float64) - v.max())
    assert np.allclose(sm, e / e.sum(), rtol=1e-6, atol=1e-12)
    assert abs(float(sm.astype(np.float64).sum()) - 1.0) < 1e-5


def test_topk_rules(orc):
    rng = np.random.default_rng(11)
    for _ in range(200):
        E = int(rng.integers(4, 80)); K = int(rng.integers(1, E + 1))
        v = np.round(rng.standard_normal(E) * 2, 1).astype(np.float32)     # many ties
        b = (rng.standard_normal(E) * 0.3).astype(np.float32) if rng.random() < 0.5 else None
        key = v + (b if b is not None else np.float32(0))
        want = sorted(range(E), key=lambda e: (-float(key[e]), e))[:K]
        assert list(orc.topk(v, K, b)) == want
    # non-finite: NaN never wins; all-invalid falls back to the lowest unselected id
    v = np.array([np.nan, 1.0, np.nan, 2.0], np.float32)
    assert list(orc.topk(v, 4)) == [3, 1, 0, 2]
    v = np.array([-1e31, -np.inf, -1e30, 5.0], np.float32)
    assert list(orc.topk(v, 3)) == [3, 0, 1]


def test_bucket_invariants(orc):
    rng = np.random.default_rng(13)
    for S_, K, E in ((1, 10, 256), (4, 3, 6), (32, 10, 256), (7, 8, 16), (128, 4, 64)):
        sel = np.stack([rng.choice(E, K, replace=False) for _ in range(S_)]).astype(np.int32)
        G, gexp, gbeg, gcnt, grow, rowof = orc.bucket(sel, S_, K, E)
        assert G == len(np.unique(sel)) and np.all(np.diff(gexp) > 0)
        assert np.array_equal(gbeg, np.concatenate([[0], np.cumsum(gcnt)[:-1]]))
        T = S_ * K
        assert sorted(rowof.tolist()) == list(range(T))
        for p in range(T):
            s_, slot = p // K, rowof[p]
            g = np.searchsorted(gbeg, slot, side="right") - 1
            assert gexp[g] == sel.reshape(-1)[p] and grow[slot] == s_
        for g in range(G):                      # stable: rows of a group ascend in (s, a) order
            assert np.all(np.diff(grow[gbeg[g]:gbeg[g] + gcnt[g]]) >= 0)


def test_generator(orc):
    # the documented stream: element i of a tensor = Box-Muller of draws (2p, 2p+1)
    seed = S.tensor_seed(7, 0, S.T_ROUTER)
    assert orc.tensor_seed(7, 0, S.T_ROUTER) == seed
    assert orc.lib.sw_u64(seed, 5) == S.u64(seed, 5)
    z = orc.normal(8, seed, 1.0)
    for i in range(8):
        p = i // 2
        u1 = ((S.u64(seed, 2 * p) >> 11) + 1) * 2.0 ** -53
        u2 = (S.u64(seed, 2 * p + 1) >> 11) * 2.0 ** -53
        r = math.sqrt(-2 * math.log(u1))
        want = r * (math.cos if i % 2 == 0 else math.sin)(2 * math.pi * u2)
        assert abs(float(z[i]) - want) < 1e-6 * max(1.0, abs(want))
    big = orc.normal(1 << 20, seed, 0.02)
    assert abs(big.mean()) < 1e-4 and abs(big.std() - 0.02) < 1e-4
    assert abs(float(((big / 0.02) ** 4).mean()) - 3.0) < 0.05             # normal kurtosis
    assert np.array_equal(orc.normal(100, seed, 0.02, offset=50), big[50:150])


def test_rmsnorm_and_argmax(orc):
    """A18 glue: rmsnorm_row (c/moe_math.h:58-62) bit-exact against the
    compiled reference when built, and against its closed form in double
    within one float rounding; argmax (c/laguna.c:1159) against a brute-force
    strict scan, ties, signed zeros and NaN included"""
    from oracle.oracle import Ref
    rng = np.random.default_rng(58)
    for D in (64, 512, 4096):
        x = (rng.standard_normal((3, D)) * rng.choice([1e-3, 1.0, 1e3], (3, 1))).astype(np.float32)
        w = (1 + rng.standard_normal(D) * 0.02).astype(np.float32)
        got = orc.rmsnorm_rows(x, w, 1e-6)
        inv = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
        assert np.allclose(got, x * inv * w, rtol=4e-7, atol=0)
        if Ref.available():
            r = Ref()
            for s in range(3):
                assert np.array_equal(got[s].view(np.uint32), r.rmsnorm_row(x[s], w, 1e-6).view(np.uint32))

    def scan(v):
        b = 0
        for i in range(1, len(v)):
            if v[i] > v[b]:
                b = i
        return b
    cases = [rng.standard_normal(100).astype(np.float32),
             np.array([1, 3, 3, 2, 3], np.float32),
             np.array([-0.0, 0.0, -1.0], np.float32),
             np.array([0.0, -0.0, -1.0], np.float32),
             np.array([np.nan, 5, 7], np.float32),
             np.array([1, np.nan, 7, 7, np.nan], np.float32),
             np.array([-np.inf, -np.inf], np.float32)]
    for v in cases:
        assert orc.argmax_rows(v[None])[0] == scan(list(v))
