"""The router over token tiles (a prefill-sized batch, or a head-sized router):
each weight slice is loaded once per tile of tokens, and every logit keeps the
16-lane FMA-chain contract of the per-token router (c/moe_matmul.h:25-43,
92-110), so the logits equal the oracle's bit for bit, and so do the scores,
the picks and the weights built on them."""
import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.backend import DeviceLayer, desc_of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("S,V", [(2, 4100), (8, 4096), (11, 5003)])
def test_head_tiles_bits(be, orc, S, V, bf16):
    """head-sized rows (>= 4096: the tiled path), a ragged last group of four rows and
    a partial token tile"""
    D = 512
    rng = np.random.default_rng(V + S)
    W = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    if bf16:
        W = orc.to_bf16(W)
    x = (rng.standard_normal((S, D)) * np.logspace(-3, 3, S)[:, None]).astype(np.float32)
    Wc = be.router_upload(W, bf16)
    xd, ld, td = be.upload(x), be.alloc(S * V * 4), be.alloc(S * 4)
    be.head_argmax(Wc, bf16, xd, S, D, V, ld, td)
    logits = be.d2h(ld, (S, V), np.float32)
    tok = be.d2h(td, (S,), np.int32)
    want = orc.matmul_bf16(x, W) if bf16 else orc.matmul_f32(x, W)
    for b in (Wc, xd, ld, td):
        b.free()
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(tok, orc.argmax_rows(want))


@pytest.mark.parametrize("act", [cf.ROUTE_SOFTMAX, cf.ROUTE_SIGMOID, cf.ROUTE_SOFTPLUS])
def test_batch_route_tiles_bits(be, orc, act):
    """S = 600 (the tiled path: 16-token tiles on four waves), E = 72 (a partial block of
    16 experts), the bf16 router; the logits bit for bit and the routing exact"""
    cfg = cf.scaled(cf.C2, D=512, E=72, K=6, I=128, Is=128)
    cfg = cf.replace(cfg, route_act=act, use_corr_bias=int(act != cf.ROUTE_SOFTMAX))
    L = synth.make_layer(orc, cfg, 31, corr_bias_sigma=0.01)
    dl = DeviceLayer.from_host(be, cfg, L)
    S = 600
    x = np.random.default_rng(act).standard_normal((S, cfg.D)).astype(np.float32)
    xd = be.upload(x)
    lg, sel, w = be.route(desc_of(cfg), dl.weights(), xd, S)
    xd.free()
    dl.free()
    lg_o, sel_o, w_o = orc.route(synth.desc_of(cfg), L, x)
    assert np.array_equal(lg.view(np.uint32), lg_o.view(np.uint32))
    assert np.array_equal(sel, sel_o)
    assert np.array_equal(w.view(np.uint32), w_o.view(np.uint32))
