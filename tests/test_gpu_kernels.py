"""The Laguna-ABI entries (lag_hip_*) against the CPU reference contract,
and the reference backend self-test's invariants (c/laguna.c:1560-1666)."""
import os

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf

pytestmark = pytest.mark.gpu


def normwise(got, want):
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def q4_case(orc, O, I, gs, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    p, s = orc.quant_i4(W, gs)
    return p, s


@pytest.mark.parametrize("gs", [0, 32, 64, 256, 512, 2048])
@pytest.mark.parametrize("S_", [1, 3, 17, 70])
def test_matmul_q4(be, orc, gs, S_):
    O, I = 512, 2048
    p, s = q4_case(orc, O, I, gs, 11 + gs)
    x = np.random.default_rng(S_).standard_normal((S_, I)).astype(np.float32)
    want = orc.matmul_i4_grouped(x, p, s, gs) if gs else orc.matmul_q4(x, p, s)
    dp, ds = be.upload(p), be.upload(s)
    got = be.matmul_q4(x, dp, ds, O, gs)
    dp.free(); ds.free()
    # per-row scales: matmul_q4_k's F32 lanes; group scales: matmul_i4_grouped's lanes with
    # the scales applied in f32 per group (groups wider than the kernel's 256-column tile
    # too) -- bit for bit at every S
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_nibble_kat(be):
    # c/tests/test_backend_cuda.cu:105-110, padded to the kernel's K granularity
    I = 128
    q4 = np.full((16, I // 2), 0x88, np.uint8)          # nibble 8 -> 0
    q4[0, :2] = [0x70, 0xf8]
    q4[1, :2] = [0xa9, 0xcb]
    s4 = np.ones(16, np.float32); s4[1] = 0.25
    x = np.zeros((1, I), np.float32); x[0, :4] = [1, -2, 3, -4]
    dp, ds = be.upload(q4), be.upload(s4)
    y = be.matmul_q4(x, dp, ds, 16, 0)
    dp.free(); ds.free()
    assert y[0, 0] == -34.0 and y[0, 1] == -2.5 and np.all(y[0, 2:] == 0)


@pytest.mark.parametrize("S_", [1, 4, 40, 64, 65, 130])
def test_matmul_bf16(be, orc, S_):
    """every row count reproduces the CPU's 16-lane f32-activation contract bit for
    bit (the 16-lane kernel takes up to 16 tokens per weight pass, so 65 and 130 rows
    run several passes), |x| up to 1e5 and tiny values included"""
    O, I = 256, 1024
    rng = np.random.default_rng(3)
    Wb = orc.to_bf16((rng.standard_normal((O, I)) * 0.02).astype(np.float32))
    x = rng.standard_normal((S_, I)).astype(np.float32)
    x[0, :8] *= 1e5
    x[-1, 8:16] *= 1e-30
    want = orc.matmul_bf16(x, Wb)
    dW = be.upload(Wb)
    got = be.matmul_bf16(x, dW, O)
    dW.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("S_,I,O", [(1, 1024, 256), (5, 4096, 100), (3, 40, 17), (9, 6144, 64)])
def test_matmul_bf16_round_x(be, orc, S_, I, O):
    """inkling's matmul_h contract (ink_cuda_matmul_bf16): bf16-rounded activations in
    the vdpbf16ps lane order, bit for bit, denormals and huge values included; I = 40
    takes the f32-activation lanes, as the CPU does"""
    rng = np.random.default_rng(I + S_)
    Wb = orc.to_bf16((rng.standard_normal((O, I)) * 0.05).astype(np.float32))
    Wb[0, :4] = [0x0001, 0x8003, 0x7F7F, 0x0080]
    x = rng.standard_normal((S_, I)).astype(np.float32)
    x[0, :5] = [1e-39, -1e-40, 3e38, np.float32(1.0000001), -0.0]
    want = orc.matmul_bf16_rx(x, Wb)
    dW = be.upload(Wb)
    got = be.matmul_bf16_rx(x, dW, O)
    dW.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("S_,I,O", [(1, 6144, 64), (4, 1000, 33), (2, 40, 7)])
def test_matmul_q8(be, orc, S_, I, O):
    """int8 weights + row scales (lag/ink matmul_q8): matmul_q8_k's F32 lanes, bit for bit"""
    rng = np.random.default_rng(I)
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    sc = (rng.random(O) * 1e-3).astype(np.float32)
    x = rng.standard_normal((S_, I)).astype(np.float32)
    want = orc.matmul_q8(x, q, sc, 0)
    dq, ds = be.upload(q), be.upload(sc)
    got = be.matmul_q8(x, dq, ds, O)
    dq.free(); ds.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def layer_small(orc, gs, seed=5, E=6, D=1024, I=512):
    cfg = cf.scaled(cf.C2_SIGMOID, D=D, E=E, K=3, I=I, Is=128)
    from dataclasses import replace
    cfg = replace(cfg, gs=gs)
    return cfg, synth.make_layer(orc, cfg, seed)


class DevExperts:
    def __init__(self, be, L):
        self.D, self.I = L.D, L.I
        self.gu_q, self.gu_s, self.dn_q, self.dn_s = (be.upload(a) for a in (L.gu_q, L.gu_s, L.dn_q, L.dn_s))

    def free(self):
        for b in (self.gu_q, self.gu_s, self.dn_q, self.dn_s):
            b.free()


def cpu_expert(orc, L, e, x, gs):
    D, I = L.D, L.I
    ngD, ngI = (D // gs, I // gs) if gs else (1, 1)
    p13 = L.gu_q.reshape(-1, D // 2)[e * 2 * I:(e + 1) * 2 * I]; s13 = L.gu_s.reshape(-1, ngD)[e * 2 * I:(e + 1) * 2 * I]
    p2 = L.dn_q.reshape(-1, I // 2)[e * D:(e + 1) * D]; s2 = L.dn_s.reshape(-1, ngI)[e * D:(e + 1) * D]
    mm = (lambda x_, p, s: orc.matmul_i4_grouped(x_, p, s, gs)) if gs else (lambda x_, p, s: orc.matmul_q4(x_, p, s))
    gu = mm(x.reshape(1, -1), p13, s13)[0]
    glu = np.array([orc.lib.sw_siluf(float(g)) for g in gu[:I]], np.float32) * gu[I:]
    return mm(glu.reshape(1, -1), p2, s2)[0]


@pytest.mark.parametrize("gs", [0, 32])
def test_expert_and_moe_experts(be, orc, gs):
    cfg, L = layer_small(orc, gs)
    dev = DevExperts(be, L)
    x = synth.make_x(orc, cfg, 9, 1)[0]
    # single expert through lag_hip_expert_q4: pointers offset to expert 2
    e = 2
    D, I = cfg.D, cfg.I
    ngD, ngI = (D // gs, I // gs) if gs else (1, 1)
    off = lambda buf, nbytes: type("P", (), {"__int__": lambda s_: int(buf) + nbytes})()
    got = be.expert_q4(x, off(dev.gu_q, e * 2 * I * D // 2), off(dev.gu_s, e * 2 * I * ngD * 4),
                       off(dev.dn_q, e * D * I // 2), off(dev.dn_s, e * D * ngI * 4), I, D, gs)
    want = cpu_expert(orc, L, e, x, gs)
    # activations enter the int4 GEMV as one exact integer per input (2^-21 of its
    # 32-input group's max); the rest is the f32 sum order
    assert normwise(got, want) < (2e-4 if gs == 0 else 2e-3)
    # K experts in one submission: out = sum_k w_k expert(sel_k)
    sel = np.array([4, 0, 5], np.int32); w = np.array([0.5, 0.3, 0.2], np.float32)
    got = be.moe_experts(x, dev, sel, w, gs)
    want = np.zeros(D, np.float32)
    for a in range(3):
        want = np.float32(w[a]) * cpu_expert(orc, L, int(sel[a]), x, gs) + want
    assert normwise(got, want) < (2e-4 if gs == 0 else 2e-3)
    dev.free()


@pytest.mark.parametrize("gs", [0, 32])
def test_group_bit_identical_to_per_token(be, orc, gs):
    """c/laguna.c:1623-1662: grouped experts == per-token path, max|abs| == 0"""
    cfg, L = layer_small(orc, gs)
    dev = DevExperts(be, L)
    S_, K, E = 4, 3, 6
    sel = np.array([[0, 1, 2], [1, 2, 3], [0, 2, 4], [2, 3, 5]], np.int32)
    rng = np.random.default_rng(1234)
    w = (0.05 + rng.random((S_, K)) * 0.3).astype(np.float32)
    x = synth.make_x(orc, cfg, 17, S_)
    ref = np.stack([be.moe_experts(x[s], dev, sel[s], w[s], gs) for s in range(S_)])
    G, gexp, gbeg, gcnt, grow, rowof = orc.bucket(sel, S_, K, E)
    grp = be.moe_group(x, dev, gexp, gbeg, gcnt, grow, rowof, w, K, gs)
    assert np.array_equal(grp.view(np.uint32), ref.view(np.uint32))
    dev.free()


def test_fault_injection(be, orc):
    """COLI_GPU_FAIL_AFTER=0 fails every compute entry; unset, the next call works
    (c/backend_cuda.cu:684-693; used at c/tests/test_backend_cuda.cu:93-98)."""
    p, s = q4_case(orc, 16, 128, 0, 1)
    dp, ds = be.upload(p), be.upload(s)
    x = np.ones((1, 128), np.float32)
    os.environ["COLI_GPU_FAIL_AFTER"] = "0"
    try:
        with pytest.raises(Exception):
            be.matmul_q4(x, dp, ds, 16, 0)
    finally:
        del os.environ["COLI_GPU_FAIL_AFTER"]
    y = be.matmul_q4(x, dp, ds, 16, 0)
    assert np.allclose(y, orc.matmul_q4(x, p, s), rtol=1e-5, atol=1e-6)
    dp.free(); ds.free()


@pytest.mark.parametrize("D,I", [(4096, 256), (1024, 1536)])
def test_group_large_groups_chunked(be, orc, D, I):
    """groups of 8 tokens: the activation staging no longer fits LDS whole and
    runs in chunks (D=4096: K-split 2 with two chunks per slice; I=1536 down:
    a last chunk shorter than the others), still bit-identical per token"""
    from dataclasses import replace
    cfg = replace(cf.scaled(cf.C2_SIGMOID, D=D, E=4, K=2, I=I, Is=128), gs=32)
    L = synth.make_layer(orc, cfg, 77)
    dev = DevExperts(be, L)
    S_, K, E = 8, 2, 4
    sel = np.tile(np.array([[1, 3]], np.int32), (S_, 1))
    w = np.full((S_, K), 0.5, np.float32)
    x = synth.make_x(orc, cfg, 78, S_)
    ref = np.stack([be.moe_experts(x[s], dev, sel[s], w[s], 32) for s in range(S_)])
    G, gexp, gbeg, gcnt, grow, rowof = orc.bucket(sel, S_, K, E)
    assert list(gcnt[:G]) == [8, 8]
    grp = be.moe_group(x, dev, gexp, gbeg, gcnt, grow, rowof, w, K, 32)
    assert np.array_equal(grp.view(np.uint32), ref.view(np.uint32))
    want = np.zeros((S_, D), np.float32)
    for s in range(S_):
        for a in range(K):
            want[s] = np.float32(w[s, a]) * cpu_expert(orc, L, int(sel[s, a]), x[s], 32) + want[s]
    assert normwise(grp, want) < 2e-3
    dev.free()
