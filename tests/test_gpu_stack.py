"""The stack glue on the device (A18): RMSNorm rows, the bf16 head's logits
and the greedy pick, and a small stack of MoE layers end to end, against the
oracle: RMSNorm, head logits and the pick bit for bit; the stack's residual
stream within the benchmark tolerance and its greedy tokens identical."""
import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.stack import DeviceStack, NORM_EPS, head_bf16, norm_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [512, 4096])
def test_rmsnorm_bits(be, orc, D):
    rng = np.random.default_rng(D)
    x = (rng.standard_normal((5, D)) * np.array([[1e-3], [1.0], [30.0], [1.0], [1e3]])).astype(np.float32)
    w = (1 + rng.standard_normal(D) * 0.02).astype(np.float32)
    xd, wd, od = be.upload(x), be.upload(w), be.upload(np.zeros_like(x))
    be.rmsnorm(xd, wd, od, 5, D, NORM_EPS)
    got = be.d2h(od, x.shape, np.float32)
    for b in (xd, wd, od):
        b.free()
    assert np.array_equal(got.view(np.uint32), orc.rmsnorm_rows(x, w, NORM_EPS).view(np.uint32))


def test_head_logits_and_pick(be, orc):
    cfg = cf.scaled(cf.C5_LAYER, D=512)
    V, S = 1000, 4
    head = head_bf16(orc, cfg, 5, V)
    x = np.random.default_rng(2).standard_normal((S, cfg.D)).astype(np.float32)
    Wc = be.router_upload(head, True)
    xd, ld, td = be.upload(x), be.alloc(S * V * 4), be.alloc(S * 4)
    be.head_argmax(Wc, True, xd, S, cfg.D, V, ld, td)
    logits = be.d2h(ld, (S, V), np.float32)
    tok = be.d2h(td, (S,), np.int32)
    want = orc.matmul_bf16(x, head)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(tok, orc.argmax_rows(want))
    # the pick's rules on planted rows: ties to the lowest index, -0.0 == +0.0, NaN
    rows = np.full((4, V), -1.0, np.float32)
    rows[0, [7, 3, 900]] = 5.0
    rows[1, :] = -2.0; rows[1, 10] = -0.0; rows[1, 4] = 0.0
    rows[2, 0] = np.nan; rows[2, 5] = 9.0
    rows[3, 1] = np.nan; rows[3, 600] = 2.0
    be.h2d(ld, rows)
    be.argmax(ld, S, V, td)
    assert np.array_equal(be.d2h(td, (S,), np.int32), [3, 4, 0, 600])
    assert np.array_equal(orc.argmax_rows(rows), [3, 4, 0, 600])
    for b in (Wc, xd, ld, td):
        b.free()


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("S,V", [(2, 4099), (8, 4132), (13, 5000), (600, 1026)])
def test_tiled_head_bits(be, orc, bf16, S, V):
    """Heads of >= 4096 rows, and any head at >= 512 tokens, take the token-tiled router
    (tiles of 8 or 16 tokens, two groups of 4 rows per wave for bf16 weights): logits
    bit-exact for ragged token tiles and row counts whose last block holds fewer groups
    than a block's waves take (the clamped loads), the pick of every row (V % 4 != 0: the
    argmax's scalar path)."""
    D = 512
    rng = np.random.default_rng(S * 7 + V)
    Wf = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    W = (Wf.view(np.uint32) >> 16).astype(np.uint16) if bf16 else Wf
    x = rng.standard_normal((S, D)).astype(np.float32)
    Wc = be.router_upload(W, bf16)
    xd, ld, td = be.upload(x), be.alloc(S * V * 4), be.alloc(S * 4)
    be.head_argmax(Wc, bf16, xd, S, D, V, ld, td)
    logits = be.d2h(ld, (S, V), np.float32)
    tok = be.d2h(td, (S,), np.int32)
    want = orc.matmul_bf16(x, W) if bf16 else orc.matmul_f32(x, W)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(tok, orc.argmax_rows(want))
    for b in (Wc, xd, ld, td):
        b.free()


@pytest.mark.parametrize("V", [40004, 40001])
def test_pick_long_rows(be, orc, V):
    """Rows longer than one pass of the argmax block (32768 values as float4, 1024 as
    scalars): ties between passes go to the lowest index, -0.0 == +0.0 across passes, a
    maximum in the last partial float4 or scalar pass."""
    rows = np.full((4, V), -3.0, np.float32)
    rows[0, [33000, 100, 39999]] = 7.0                   # tie across passes
    rows[1, V - 1] = 1.0                                 # the last value
    rows[2, :] = -1.0; rows[2, 35000] = -0.0; rows[2, 20] = 0.0
    rows[3, 0] = 2.0; rows[3, 32768] = np.nan; rows[3, 32769] = 2.5
    want = [100, V - 1, 20, 32769]
    assert np.array_equal(orc.argmax_rows(rows), want)
    ld, td = be.upload(rows), be.alloc(4 * 4)
    be.argmax(ld, 4, V, td)
    assert np.array_equal(be.d2h(td, (4,), np.int32), want)
    # rows starting 4 bytes past a 16-byte boundary (the scalar path)
    lo = be.upload(np.concatenate([np.zeros(1, np.float32), rows.reshape(-1)]))
    be.argmax(int(lo) + 4, 4, V, td)
    assert np.array_equal(be.d2h(td, (4,), np.int32), want)
    for b in (ld, td, lo):
        b.free()


@pytest.mark.parametrize("S_", [1, 4])
def test_small_stack(be, orc, S_):
    cfg = cf.scaled(cf.C5_LAYER, D=512, E=32, K=8, I=384)
    n_layers, V, seed = 3, 1000, 77
    layers = [synth.make_layer(orc, cfg, seed, layer=l) for l in range(n_layers)]
    nw = norm_weights(orc, cfg, seed, n_layers)
    head = head_bf16(orc, cfg, seed, V)
    h0 = synth.make_x(orc, cfg, seed, S_)
    wh, wlog, wtok = orc.stack(synth.desc_of(cfg), layers, nw[:n_layers], nw[n_layers], head, h0, NORM_EPS)
    st = DeviceStack.from_host(be, cfg, layers, nw[:n_layers], nw[n_layers], head)
    hd, xn, ld, td = be.upload(h0), be.alloc(S_ * cfg.D * 4), be.alloc(S_ * V * 4), be.alloc(S_ * 4)
    st.step(hd, xn, ld, td, S_)
    h = be.d2h(hd, h0.shape, np.float32)
    logits = be.d2h(ld, (S_, V), np.float32)
    tok = be.d2h(td, (S_,), np.int32)
    st.free()
    for b in (hd, xn, ld, td):
        b.free()
    dw = wh - h0
    assert float(np.max(np.abs((h - h0) - dw))) / float(np.max(np.abs(dw))) <= 2e-3
    err = float(np.max(np.abs(logits - wlog)))
    srt = np.sort(wlog, axis=1)
    margin = srt[:, -1] - srt[:, -2]
    clear = margin > 20 * err
    assert clear.sum() >= max(1, S_ - 1), (margin, err)
    assert np.array_equal(tok[clear], wtok[clear])


NORM_CASES = [(cf.scaled(cf.C5_LAYER, D=512, E=32, K=8, I=384), s) for s in (1, 4, 40)] + \
             [(cf.scaled(cf.C2, D=512, E=32, K=6, I=256, Is=256, name="C2-small-shared"), 4)]


@pytest.mark.parametrize("cfg,S_", NORM_CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_layer_norm_fused_bits(be, orc, cfg, S_):
    """lag_hip_moe_forward_rmsnorm against lag_hip_rmsnorm then lag_hip_moe_forward: the
    normalised rows and the updated residual bit for bit -- with the norm applied by the
    router blocks as they stage x (one expert group per block at S <= 4, one token per
    block at 40) and on the two-launch path a shared expert takes"""
    from sabrewing_amd.backend import DeviceLayer, desc_of
    L = synth.make_layer(orc, cfg, 91)
    dl = DeviceLayer.from_host(be, cfg, L)
    h0 = (synth.make_x(orc, cfg, 92, S_) * np.float32(3.0)).astype(np.float32)
    w = norm_weights(orc, cfg, 93, 1)[0]
    wd = be.upload(w)
    h1, xn1 = be.upload(h0), be.alloc(S_ * cfg.D * 4)
    be.rmsnorm(h1, wd, xn1, S_, cfg.D, NORM_EPS)
    be.moe_forward(desc_of(cfg), dl.weights(), xn1, h1, S_)
    h2, xn2 = be.upload(h0), be.alloc(S_ * cfg.D * 4)
    be.moe_forward_rmsnorm(desc_of(cfg), dl.weights(), wd, NORM_EPS, xn2, h2, S_)
    got = [be.d2h(b, h0.shape, np.float32) for b in (h1, xn1, h2, xn2)]
    for b in (wd, h1, xn1, h2, xn2):
        b.free()
    dl.free()
    assert np.array_equal(got[3].view(np.uint32), got[1].view(np.uint32))      # xn
    assert np.array_equal(got[2].view(np.uint32), got[0].view(np.uint32))      # h
    assert np.array_equal(got[1].view(np.uint32), orc.rmsnorm_rows(h0, w, NORM_EPS).view(np.uint32))
