"""The GLM engine's coli_cuda_* table on the device (include/sabrewing_coli.h,
sabrewing_amd/csrc/coli_hip.hip) against the oracle and against the lag family.

  * expert groups: each row equals the same expert's lag_hip_expert_q4 output bit
    for bit (the same dot8 kernels, or for prefill-sized groups the f16 MFMA
    GEMMs, reading the group's three tensors through a per-group table) and the
    oracle's int4 expert (c/moe_quant.h / c/quant.h numerics) within the lag
    family's bounds;
  * issue/take, expert_mlp and the shared MLP are the same computation;
  * the resident pair: one fma per expert in call order, slots summed in order;
  * the router: idx, weights and the kept count equal the oracle's restatement of
    c/colibri.c:2871-2999 bit for bit (its logits are pinned to the compiled
    c/quant.h matmul in tests/test_oracle_glm.py);
  * validation, fault injection and the "unavailable" slots return 0."""
import os

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.coli import Coli, ColiError

pytestmark = pytest.mark.gpu

D, I, E = 1024, 512, 6


@pytest.fixture(scope="module")
def coli():
    c = Coli([0])
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def normwise(a, b):
    return float(np.max(np.abs(a - b))) / max(float(np.max(np.abs(b))), 1e-30)


def layer(orc, gs, seed=5):
    from dataclasses import replace
    cfg = replace(cf.scaled(cf.C2_SIGMOID, D=D, E=E, K=3, I=I, Is=128), gs=gs)
    return synth.make_layer(orc, cfg, seed)


def parts(L, e, gs):
    """expert e's gate, up, down (bytes, scales) out of the fused layer tensors"""
    ngD, ngI = (D // gs, I // gs) if gs else (1, 1)
    gq, gsc = L.gu_q.reshape(-1, D // 2), L.gu_s.reshape(-1, ngD)
    dq, dsc = L.dn_q.reshape(-1, I // 2), L.dn_s.reshape(-1, ngI)
    r = e * 2 * I
    return ((gq[r:r + I], gsc[r:r + I]), (gq[r + I:r + 2 * I], gsc[r + I:r + 2 * I]),
            (dq[e * D:(e + 1) * D], dsc[e * D:(e + 1) * D]))


class Experts:
    def __init__(self, coli, L, gs):
        self.t = []
        for e in range(E):
            (g, gsc), (u, usc), (d, dsc) = parts(L, e, gs)
            self.t.append((coli.upload(g, gsc, D, I, 0, gs), coli.upload(u, usc, D, I, 0, gs),
                           coli.upload(d, dsc, I, D, 0, gs)))

    def lists(self, ids):
        return [self.t[e][0] for e in ids], [self.t[e][1] for e in ids], [self.t[e][2] for e in ids]

    def free(self):
        for ts in self.t:
            for t in ts:
                t.free()


def cpu_expert(orc, L, e, x, gs):
    (g, gsc), (u, usc), (d, dsc) = parts(L, e, gs)
    mm = (lambda x_, p, s: orc.matmul_i4_grouped(x_, p, s, gs)) if gs else (lambda x_, p, s: orc.matmul_q4(x_, p, s))
    gg = mm(x.reshape(1, -1), g, gsc)[0]
    uu = mm(x.reshape(1, -1), u, usc)[0]
    h = np.array([orc.lib.sw_siluf(float(v)) for v in gg], np.float32) * uu
    return mm(h.reshape(1, -1), d, dsc)[0]


def lag_expert(be, dev, L, e, x, gs):
    ngD, ngI = (D // gs, I // gs) if gs else (1, 1)
    off = lambda buf, nbytes: type("P", (), {"__int__": lambda s_: int(buf) + nbytes})()
    return be.expert_q4(x, off(dev[0], e * 2 * I * D // 2), off(dev[1], e * 2 * I * ngD * 4),
                        off(dev[2], e * D * I // 2), off(dev[3], e * D * ngI * 4), I, D, gs)


@pytest.mark.parametrize("gs", [0, 32])
def test_expert_group_equals_lag_and_oracle(coli, be, orc, gs):
    L = layer(orc, gs)
    ex = Experts(coli, L, gs)
    ids, rows = [2, 0, 5, 2, 3], [1, 3, 2, 7, 1]
    T = sum(rows)
    x = np.random.default_rng(3).standard_normal((T, D)).astype(np.float32)
    y = coli.expert_group(*ex.lists(ids), rows, x)
    dev = [be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s)]
    r = 0
    for e, n in zip(ids, rows):
        for _ in range(n):
            assert np.array_equal(bits(y[r]), bits(lag_expert(be, dev, L, e, x[r], gs))), (e, r)
            if r % 3 == 0:
                assert normwise(y[r], cpu_expert(orc, L, e, x[r], gs)) < (2e-4 if gs == 0 else 2e-3)
            r += 1
    for b in dev:
        b.free()
    # the group statistics count calls, experts and rows (c/backend_cuda.cu:935-937)
    import ctypes as C
    n = (C.c_uint64 * 3)()
    coli.f.group_stats(C.addressof(n), C.addressof(n) + 8, C.addressof(n) + 16, None, None, None)
    assert n[0] >= 1 and n[1] >= 5 and n[2] >= T
    ex.free()


@pytest.mark.parametrize("gs", [0, 32])
def test_expert_group_one_row_each(coli, be, orc, gs):
    """groups of one row each (decode) take the one-token weight passes; each row
    still equals the same expert's lag_hip_expert_q4 output bit for bit and the
    oracle's expert within the lag family's bounds"""
    L = layer(orc, gs, seed=7)
    ex = Experts(coli, L, gs)
    ids, rows = [2, 0, 5, 3], [1, 1, 1, 1]
    x = np.random.default_rng(11).standard_normal((4, D)).astype(np.float32)
    y = coli.expert_group(*ex.lists(ids), rows, x)
    dev = [be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s)]
    for r, e in enumerate(ids):
        assert np.array_equal(bits(y[r]), bits(lag_expert(be, dev, L, e, x[r], gs))), (e, r)
        assert normwise(y[r], cpu_expert(orc, L, e, x[r], gs)) < (2e-4 if gs == 0 else 2e-3)
    for b in dev:
        b.free()
    ex.free()


@pytest.mark.parametrize("gs", [0, 32])
def test_prefill_group_on_the_mfma(coli, be, orc, gs):
    """groups averaging >= 8 rows take the f16 MFMA GEMMs (64-token tiles, partial tiles,
    one group over two tiles): still each row's lag expert output bit for bit"""
    L = layer(orc, gs, seed=21)
    ex = Experts(coli, L, gs)
    ids, rows = [3, 1, 4, 0], [40, 70, 9, 130]
    T = sum(rows)
    x = np.random.default_rng(7).standard_normal((T, D)).astype(np.float32)
    y = coli.expert_group(*ex.lists(ids), rows, x)
    dev = [be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s)]
    owner = np.repeat(ids, rows)
    for r in list(range(0, T, 7)) + [39, 40, 109, 110, 118, 119, 182, 183, T - 1]:
        e = int(owner[r])
        assert np.array_equal(bits(y[r]), bits(lag_expert(be, dev, L, e, x[r], gs))), (e, r)
        if r % 35 == 0:
            assert normwise(y[r], cpu_expert(orc, L, e, x[r], gs)) < (2e-4 if gs == 0 else 2e-3)
    for b in dev:
        b.free()
    ex.free()


@pytest.mark.parametrize("gs", [0, 64])
def test_mlp_issue_take_are_the_group(coli, orc, gs):
    L = layer(orc, gs, seed=8)
    ex = Experts(coli, L, gs)
    x = np.random.default_rng(4).standard_normal((6, D)).astype(np.float32)
    g, u, d = ex.t[4]
    want = coli.expert_group([g], [u], [d], [6], x)
    assert np.array_equal(bits(coli.expert_mlp(g, u, d, x)), bits(want))
    if gs == 0:
        assert np.array_equal(bits(coli.expert_mlp(g, u, d, x, shared=True)), bits(want))
    else:                                   # the W4A16 shared entry takes per-row int4 only
        with pytest.raises(ColiError):
            coli.expert_mlp(g, u, d, x, shared=True)
    # issue/take: <= 8 rows, one outstanding per device
    ids, rows = [1, 4, 0], [2, 1, 3]
    xs = x[:6]
    want = coli.expert_group(*ex.lists(ids), rows, xs)
    assert coli.issue(*ex.lists(ids), rows, xs)
    assert not coli.issue(*ex.lists(ids), rows, xs)         # one outstanding
    got = coli.take(0, (6, D))
    assert np.array_equal(bits(got), bits(want))
    assert coli.take(0, (6, D)) is None                     # nothing pending
    assert not coli.issue(*ex.lists([1, 2]), [5, 4], np.zeros((9, D), np.float32))   # > 8 rows
    ex.free()


def test_resident_issue_take(coli, orc):
    L = layer(orc, 0, seed=11)
    ex = Experts(coli, L, 0)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(D).astype(np.float32)
    sets = ([3, 1, 4], [0, 5])
    ws = (np.array([0.5, 0.3, 0.2], np.float32), np.array([1.25, -0.75], np.float32))
    xd = coli.dev_put(x)
    slots = coli.f.pipe_alloc(0, 2 * D * 4)
    acc = coli.f.pipe_alloc(0, D * 4)
    for k, (ids, w) in enumerate(zip(sets, ws)):
        assert coli.resident_issue(*ex.lists(ids), w, 0, xd, slots + k * D * 4)
    assert coli.resident_take(0, [0, 0], slots, acc, D)
    got_slots = coli.dev_get(slots, (2, D))
    got_acc = coli.dev_get(acc, (D,))
    for k, (ids, w) in enumerate(zip(sets, ws)):
        y = coli.expert_group(*ex.lists(ids), [1] * len(ids), np.tile(x, (len(ids), 1)))
        want = np.zeros(D, np.float64)
        for c in range(len(ids)):                          # one fma per expert, in call order
            want = np.float32(np.float64(w[c]) * y[c].astype(np.float64) + want).astype(np.float64)
        assert normwise(got_slots[k], want.astype(np.float32)) < 1e-6
    assert np.array_equal(bits(got_acc), bits(got_slots[0] + got_slots[1]))   # slots summed in issue order
    # group-scaled tensors are refused, as the reference's per-row-only resident path
    Lg = layer(orc, 32, seed=12)
    exg = Experts(coli, Lg, 32)
    assert not coli.resident_issue(*exg.lists([0]), np.ones(1, np.float32), 0, xd, slots)
    for p in (xd, slots, acc):
        coli.dev_free(p)
    ex.free(); exg.free()


ROUTER_CASES = [(160, 5120, 8, 0.0, 1, 2.5), (256, 4096, 8, 0.0, 1, 1.0), (64, 1003, 6, 0.7, 1, 2.5),
                (128, 6144, 8, 0.9, 0, 1.0), (96, 37, 5, 0.5, 1, 1.5), (16, 2048, 16, 0.0, 1, 1.0)]


@pytest.mark.parametrize("E_,D_,Ksel,topp,norm,scale", ROUTER_CASES)
def test_router_bit_exact(coli, orc, E_, D_, Ksel, topp, norm, scale):
    rng = np.random.default_rng(E_ * 7 + D_)
    W = (rng.standard_normal((E_, D_)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(E_) * 0.01).astype(np.float32)
    x = rng.standard_normal(D_).astype(np.float32)
    if E_ == 128:                                       # ties: duplicated rows and biases -> lowest id
        W[77] = W[12]; b[77] = b[12]; W[100] = W[12]; b[100] = b[12]
    if E_ == 96:
        b[[3, 9, 40]] = -np.inf                         # never above -1e30: never chosen
    pw, pb, px = coli.dev_put(W), coli.dev_put(b), coli.dev_put(x)
    idx, w, ke = coli.router(0, px, pw, pb, D_, E_, Ksel, topp, norm, scale)
    widx, ww, wke = orc.glm_route(x, W, b, Ksel, topp, norm, scale)
    assert np.array_equal(idx, widx) and ke == wke and np.array_equal(bits(w), bits(ww)), (idx, widx, ke, wke)
    for p in (pw, pb, px):
        coli.dev_free(p)


def test_router_nonfinite_fallback(coli, orc):
    """NaN logits never win; a pass with no candidate takes expert kk (c/colibri.c:2776-2782)"""
    E_, D_, K_ = 32, 256, 4
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((E_, D_)) * 0.02).astype(np.float32)
    b = np.zeros(E_, np.float32)
    x = rng.standard_normal(D_).astype(np.float32)
    x[17] = np.nan
    pw, pb, px = coli.dev_put(W), coli.dev_put(b), coli.dev_put(x)
    idx, w, ke = coli.router(0, px, pw, pb, D_, E_, K_, 0.0, 1, 1.0)
    widx, ww, wke = orc.glm_route(x, W, b, K_, 0.0, 1, 1.0)
    assert list(idx) == [0, 1, 2, 3] and np.array_equal(idx, widx) and ke == wke
    assert np.isnan(w).all() and np.isnan(ww).all()      # NaN weights (their payload is not part of the contract)
    for p in (pw, pb, px):
        coli.dev_free(p)


@pytest.mark.parametrize("gs", [0, 32, 512])
def test_matmul_and_pipe_gemm(coli, be, orc, gs):
    L = layer(orc, gs, seed=13)
    (g, gsc), _, _ = parts(L, 1, gs)
    t = coli.upload(g, gsc, D, I, 0, gs)
    x = np.random.default_rng(6).standard_normal((5, D)).astype(np.float32)
    y = coli.matmul(t, x)
    # the GLM engine's int4 matmul has two CPU routes chosen at run time (IDOT and f32):
    # the device follows the f32 route's lanes (matmul_q4_k per row, matmul_i4_grouped
    # with group scales, c/backend_cuda.cu:128-160 names the latter) bit for bit
    want = orc.matmul_i4_grouped(x, g, gsc, gs) if gs else orc.matmul_q4(x, g, gsc)
    assert np.array_equal(bits(y), bits(want))
    xd, yd = coli.dev_put(x), coli.f.pipe_alloc(0, 5 * I * 4)
    assert coli.f.pipe_gemm(t.ptr, yd, xd, 5)
    assert np.array_equal(bits(coli.dev_get(yd, (5, I))), bits(y))
    coli.dev_free(xd); coli.dev_free(yd)
    t.free()


def test_pipe_data_plane(coli, orc):
    rng = np.random.default_rng(9)
    n = 3000
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    pa, pb = coli.dev_put(a), coli.dev_put(b)
    assert coli.f.pipe_add(0, pa, pb, n) and np.array_equal(coli.dev_get(pa, (n,)), a + b)
    assert coli.f.pipe_silu_mul(0, pb, pa, n)
    want = np.array([orc.lib.sw_siluf(float(v)) for v in b], np.float32) * (a + b)
    assert np.array_equal(bits(coli.dev_get(pb, (n,))), bits(want))
    # rows_add: x[rows[b]] += partial[b]
    X = rng.standard_normal((6, 40)).astype(np.float32)
    Pp = rng.standard_normal((3, 40)).astype(np.float32)
    rows = np.array([4, 0, 2], np.int32)
    pX, pP, pr = coli.dev_put(X), coli.dev_put(Pp), coli.dev_put(rows)
    assert coli.f.pipe_rows_add(0, pX, pP, pr, 3, 40)
    want = X.copy(); want[rows] += Pp
    assert np.array_equal(coli.dev_get(pX, (6, 40)), want)
    # copy2d (pitches in floats) and the same-device peer copy
    Y = coli.f.pipe_alloc(0, 6 * 64 * 4)
    assert coli.f.pipe_copy2d(0, Y, 64, pX, 40, 40, 6) and coli.f.pipe_sync(0)
    assert np.array_equal(coli.dev_get(Y, (6, 64))[:, :40], want)
    Z = coli.f.pipe_alloc(0, 6 * 40 * 4)
    assert coli.f.pipe_peer_copy(0, Z, 0, pX, 6 * 40 * 4)
    assert np.array_equal(coli.dev_get(Z, (6, 40)), want)
    # scratch slots grow and are reused
    s1 = coli.f.pipe_scratch(0, 3, 1024)
    assert s1 and coli.f.pipe_scratch(0, 3, 512) == s1 and coli.f.pipe_scratch(0, 27, 16) is None
    for p in (pa, pb, pX, pP, pr, Y, Z):
        coli.dev_free(p)


def test_validation_and_unavailable(coli, orc):
    import ctypes as C
    L = layer(orc, 0, seed=14)
    ex = Experts(coli, L, 0)
    g, u, d = ex.t[0]
    x = np.zeros((2, D), np.float32)
    with pytest.raises(ColiError):                       # down of the wrong shape
        coli.expert_group([g], [u], [g], [2], x)
    with pytest.raises(ColiError):                       # 65 groups
        coli.expert_group([g] * 65, [u] * 65, [d] * 65, [1] * 65, np.zeros((65, D), np.float32))
    with pytest.raises(ColiError):                       # a row count < 1
        coli.expert_group([g, g], [u, u], [d, d], [1, 0], np.zeros((1, D), np.float32))
    with pytest.raises(ColiError):                       # I not a multiple of 32
        coli.upload(np.zeros((4, 24), np.uint8), np.ones(4, np.float32), 48, 4)
    with pytest.raises(ColiError):                       # gs not a power of two
        coli.upload(np.zeros((4, 48), np.uint8), np.ones(8, np.float32), 96, 4, gs=48)
    h = C.c_void_p(0)                                    # formats other than int4: unavailable
    assert not coli.f.tensor_upload(C.addressof(h), np.zeros(64, np.float32).ctypes.data,
                                    np.ones(1, np.float32).ctypes.data, 0, 64, 1, 0)
    # a cached tensor answers 1 for its own (fmt, I, O, device, gs), 0 otherwise
    h = C.c_void_p(g.ptr)
    assert coli.f.tensor_upload(C.addressof(h), None, None, 2, D, I, 0)
    assert not coli.f.tensor_upload(C.addressof(h), None, None, 2, D, I + 1, 0)
    assert coli.f.tensor_bytes(g.ptr) == I * D // 2 + I * 4 and coli.f.tensor_device(g.ptr) == 0
    n, b = C.c_size_t(0), C.c_size_t(0)
    coli.f.stats(-1, C.addressof(n), C.addressof(b))
    assert n.value >= 3 * E and b.value >= 3 * E * (I * D // 2)
    fr, to = C.c_size_t(0), C.c_size_t(0)
    assert coli.f.mem_info(0, C.addressof(fr), C.addressof(to)) and 0 < fr.value <= to.value
    assert not coli.f.mem_info(5, C.addressof(fr), C.addressof(to))            # not configured
    assert coli.f.device_count() == 1 and coli.f.device_at(0) == 0 and coli.f.device_at(1) == -1
    # tensor_update replaces the contents in place
    (g1, g1s), _, _ = parts(L, 1, 0)
    y0 = coli.matmul(g, x[:1] + 1)
    assert coli.f.tensor_update(g.ptr, np.ascontiguousarray(g1).ctypes.data, np.ascontiguousarray(g1s).ctypes.data)
    t1 = coli.upload(g1, g1s, D, I)
    assert np.array_equal(bits(coli.matmul(g, x[:1] + 1)), bits(coli.matmul(t1, x[:1] + 1)))
    assert not np.array_equal(bits(y0), bits(coli.matmul(t1, x[:1] + 1)))
    t1.free()
    # the attention / norm / RoPE slots answer "unavailable"
    assert coli.f.attention_absorb(g.ptr, None, None, None, None, 1, 1, 1, 1, 1, 1, 1.0) == 0
    assert coli.f.pipe_rmsnorm(0, None, None, None, 1, 1, 1e-6) == 0
    assert coli.f.pipe_rope_base(0, None, 0, 1, 1, 0, 2, 1, 1e4) == 0
    ex.free()


def test_fault_injection(coli, orc):
    """COLI_GPU_FAIL_AFTER=N: compute entries fail after N calls (c/backend_cuda.cu:667-677)"""
    L = layer(orc, 0, seed=15)
    ex = Experts(coli, L, 0)
    g, u, d = ex.t[2]
    x = np.ones((1, D), np.float32)
    os.environ["COLI_GPU_FAIL_AFTER"] = "0"
    try:
        with pytest.raises(ColiError):
            coli.expert_group([g], [u], [d], [1], x)
        with pytest.raises(ColiError):
            coli.matmul(g, x)
    finally:
        del os.environ["COLI_GPU_FAIL_AFTER"]
    assert np.all(np.isfinite(coli.expert_group([g], [u], [d], [1], x)))
    ex.free()
