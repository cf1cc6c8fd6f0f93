"""The whole MoE block on the device (lag_hip_moe_block / moe_forward) against
the CPU reference contract: routing identical, layer output within the
benchmark tolerance (normwise max|a-b|/max|b| <= 2e-3 against the reference, and
elementwise |a-b|/max(|b|, 1e-3 max|b|) <= 2e-3 against the reference at full size
and against the exact float64 layer at reduced sizes), grouped batches
bit-identical per token to single-token calls."""
from dataclasses import replace

import numpy as np
import pytest

from fullsize import errs, exact_layer
from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd import synth as S
from sabrewing_amd.backend import DeviceLayer, desc_of, gen_x

pytestmark = pytest.mark.gpu
TOL = 2e-3




SMALL = [cf.scaled(cf.C1, D=512, E=16, K=4, I=256),
         cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256),
         cf.scaled(cf.C2, D=512, E=32, K=6, I=256, Is=256),
         cf.scaled(cf.C4_ZIPF, D=512, E=32, K=6, I=256, Is=256),
         cf.scaled(cf.C5_LAYER, D=512, E=32, K=8, I=384),
         replace(cf.scaled(cf.C2_SIGMOID, D=512, E=32, K=6, I=256, Is=256), name="C2-small-gs0", gs=0),
         cf.scaled(cf.C2_SIGMOID, D=768, E=32, K=6, I=384, Is=384, name="C2-D768"),     # 24 groups: padded runs of 16
         cf.scaled(cf.C1_OLMOE, D=512, E=64, K=8, I=256, name="C1-olmoe-engine"),
         cf.scaled(cf.QWEN, D=512, E=64, K=8, I=256, name="qwen35-small"),
         cf.scaled(cf.C2_SQRTSP, D=512, E=32, K=6, I=256, Is=256, name="C2-sqrt-softplus-small")]


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: c.name)
@pytest.mark.parametrize("S_", [1, 3, 33])
def test_layer_small(be, orc, cfg, S_):
    L = synth.make_layer(orc, cfg, 31, corr_bias_sigma=0.01)
    x = synth.make_x(orc, cfg, 32, S_)
    base = synth.make_x(orc, cfg, 33, S_)               # residual stream
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base)
    dl = DeviceLayer.from_host(be, cfg, L)
    got = be.moe_block(desc_of(cfg), dl.weights(), x, base)
    _, sel_w, _ = orc.route(synth.desc_of(cfg), L, x)
    xd = be.upload(x)
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
    xd.free(); dl.free()
    assert np.array_equal(sel, sel_w)
    check_small(orc, cfg, L, x, base, got, want, S_)


def check_small(orc, cfg, L, x, base, got, want, S_):
    """a reduced-size layer: normwise against the f32 reference (<= TOL), and elementwise
    against the exact (float64) layer on the same picks, within TOL or within twice the
    f32 reference's own elementwise error against that layer, whichever is larger.  At
    these sizes f32 rounding alone can reach the bar where outputs cancel to near the
    floor (C1-small, f32 activations: the reference is 2.3e-3 from exact arithmetic at
    the 1e-3 floor), so the device is held to the reference's own accuracy there."""
    _, sel_w, w_w = orc.route(synth.desc_of(cfg), L, x)
    ex = exact_layer(cfg, L, x, base, sel_w, w_w)
    nw, el_ref = errs(got, want, base)
    _, el = errs(got, ex, base)
    _, el_cpu = errs(want, ex, base)
    print(f"[{cfg.name} S={S_}] normwise {nw:.2e}; elementwise vs exact {el:.2e} (the f32 reference's own "
          f"{el_cpu:.2e}), vs the reference {el_ref:.2e}", flush=True)
    assert nw <= TOL and el <= max(TOL, 2 * el_cpu), (nw, el, el_cpu)


@pytest.mark.parametrize("cfg", [SMALL[1], SMALL[4]], ids=lambda c: c.name)
@pytest.mark.parametrize("S_", [5, 32, 40])
def test_grouped_equals_per_token(be, orc, cfg, S_):
    """every stream of a batch gets the same bits as its own single-token call -- at 5
    tokens (gate + top-k and bucketing in one launch), 32 (the shared expert's blocks in
    the grouped gate_up and the combine launches) and 40 (in the routing and grouped
    gate_up launches)"""
    L = synth.make_layer(orc, cfg, 41)
    dl = DeviceLayer.from_host(be, cfg, L)
    x = synth.make_x(orc, cfg, 42, S_)
    base = np.zeros_like(x)
    batched = be.moe_block(desc_of(cfg), dl.weights(), x, base)
    single = np.stack([be.moe_block(desc_of(cfg), dl.weights(), x[s:s + 1], base[s:s + 1])[0] for s in range(S_)])
    dl.free()
    assert np.array_equal(batched.view(np.uint32), single.view(np.uint32))


def host_layer_for(orc, cfg, seed, x):
    """the full-size host layer with only the experts x routes to generated
    (the rest stay zero: moe_block never reads them)"""
    D, I, E, gs = cfg.D, cfg.I, cfg.E, cfg.gs
    ts = lambda tid: S.tensor_seed(seed, 0, tid)
    r = orc.normal(E * D, ts(S.T_ROUTER), 0.02).reshape(E, D)
    router = orc.to_bf16(r) if cfg.router_bf16 else r
    corr = np.zeros(E, np.float32) if cfg.use_corr_bias else None
    lb = S.zipf_bias(E, cfg.zipf, ts(S.T_ROUTER) ^ 0x5A5A) if cfg.zipf > 0 else None
    ngD, ngI = D // gs, I // gs
    gu_q = np.zeros((E * 2 * I, D // 2), np.uint8); gu_s = np.zeros((E * 2 * I, ngD), np.float32)
    dn_q = np.zeros((E * D, I // 2), np.uint8); dn_s = np.zeros((E * D, ngI), np.float32)
    sg = su = sd = None
    if cfg.shared_mode:
        sg = orc.to_bf16(orc.normal(cfg.Is * D, ts(S.T_SH_GATE), 0.02)).reshape(cfg.Is, D)
        su = orc.to_bf16(orc.normal(cfg.Is * D, ts(S.T_SH_UP), 0.02)).reshape(cfg.Is, D)
        sd = orc.to_bf16(orc.normal(D * cfg.Is, ts(S.T_SH_DOWN), 0.02)).reshape(D, cfg.Is)
    L = synth.Layer(D, I, cfg.Is, E, gs, cfg.router_bf16, router, corr, lb, gu_q.reshape(-1), gu_s.reshape(-1),
                    dn_q.reshape(-1), dn_s.reshape(-1), sg, su, sd)
    _, sel, _ = orc.route(synth.desc_of(cfg), L, x)
    for e in np.unique(sel):
        e = int(e)
        q, s = orc.gen_q4(ts(S.T_GATE_UP), 0.02, 2 * I, D, gs, row0=e * 2 * I)
        gu_q[e * 2 * I:(e + 1) * 2 * I] = q; gu_s[e * 2 * I:(e + 1) * 2 * I] = s
        q, s = orc.gen_q4(ts(S.T_DOWN), 0.02, D, I, gs, row0=e * D)
        dn_q[e * D:(e + 1) * D] = q; dn_s[e * D:(e + 1) * D] = s
    return L, sel


@pytest.mark.parametrize("cfg,S_", [(c, s) for c in (cf.C1, cf.C2, cf.C2_SIGMOID) for s in (1, 4)] + [(cf.C2, 32)],
                         ids=lambda v: v.name if hasattr(v, "name") else str(v))
def test_layer_full_size(be, orc, cfg, S_):
    """benchmark shapes, the bench's B = 1 and B = 32 workloads included: device-generated
    layer vs the oracle on the same bits"""
    seed = 555
    x = synth.make_x(orc, cfg, seed, S_)
    L, sel_w = host_layer_for(orc, cfg, seed, x)
    base = np.zeros_like(x)
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base)
    dl = DeviceLayer.generate(be, cfg, seed)
    xd = be.upload(x)
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
    od = be.upload(base)
    be.moe_forward(desc_of(cfg), dl.weights(), xd, od, S_)
    got = be.d2h(od, x.shape, np.float32)
    xd.free(); od.free(); dl.free()
    assert np.array_equal(sel, sel_w)
    nw, el = errs(got, want, base)
    print(f"[{cfg.name} S={S_}] normwise {nw:.2e}, elementwise {el:.2e}", flush=True)
    assert nw <= TOL and el <= TOL, (nw, el)


def test_device_x_generator(be, orc):
    cfg = cf.C2
    xd = gen_x(be, cfg, 9, 3, stream=2)
    got = be.d2h(xd, (3, cfg.D), np.float32)
    xd.free()
    want = orc.bf16_round(orc.normal(3 * cfg.D, S.tensor_seed(9, 1002, S.T_X), 1.0)).reshape(3, cfg.D)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("S_", [1, 5])
def test_graph_replay_matches_eager(be, orc, S_):
    """a recorded forward replays bit-identical to the eager call, every time,
    with eager work and syncs between replays"""
    cfg = SMALL[2]
    L = synth.make_layer(orc, cfg, 51)
    dl = DeviceLayer.from_host(be, cfg, L)
    x = synth.make_x(orc, cfg, 52, S_)
    zero = np.zeros_like(x)
    xd, oe, og = be.upload(x), be.upload(zero), be.upload(zero)
    be.moe_forward(desc_of(cfg), dl.weights(), xd, oe, S_)       # eager; also sizes the scratch
    be.sync()
    want = be.d2h(oe, x.shape, np.float32)
    be.graph_begin()
    be.moe_forward(desc_of(cfg), dl.weights(), xd, og, S_)
    g = be.graph_end()
    try:
        for rep in range(3):
            be.h2d(og, zero)
            be.graph_launch(g)
            be.sync()
            got = be.d2h(og, x.shape, np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
            be.h2d(oe, zero)                                        # eager work between replays
            be.moe_forward(desc_of(cfg), dl.weights(), xd, oe, S_)
            be.sync()
            assert np.array_equal(be.d2h(oe, x.shape, np.float32).view(np.uint32), want.view(np.uint32))
    finally:
        be.graph_destroy(g)
        for b in (xd, oe, og):
            b.free()
        dl.free()


def test_graph_survives_larger_eager_calls(be, orc):
    """a live recording keeps the scratch it was recorded over: eager calls of a
    larger shape between replays (which need a larger arena) leave its replays
    bit-identical to the eager result"""
    cfg = SMALL[2]
    L = synth.make_layer(orc, cfg, 53)
    dl = DeviceLayer.from_host(be, cfg, L)
    x1 = synth.make_x(orc, cfg, 54, 1)
    xb = synth.make_x(orc, cfg, 55, 300)
    z1, zb = np.zeros_like(x1), np.zeros_like(xb)
    xd, oe, og = be.upload(x1), be.upload(z1), be.upload(z1)
    xbd, obd = be.upload(xb), be.upload(zb)
    be.moe_forward(desc_of(cfg), dl.weights(), xd, oe, 1)
    be.sync()
    want = be.d2h(oe, x1.shape, np.float32)
    be.graph_begin()
    be.moe_forward(desc_of(cfg), dl.weights(), xd, og, 1)
    g = be.graph_end()
    try:
        for rep in range(3):
            be.h2d(obd, zb)                                         # a larger eager call first
            be.moe_forward(desc_of(cfg), dl.weights(), xbd, obd, 300 - 50 * rep)
            be.sync()
            be.h2d(og, z1)
            be.graph_launch(g)
            be.sync()
            got = be.d2h(og, x1.shape, np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
    finally:
        be.graph_destroy(g)
    # after the graph is gone the eager path still works
    be.h2d(oe, z1)
    be.moe_forward(desc_of(cfg), dl.weights(), xd, oe, 1)
    be.sync()
    assert np.array_equal(be.d2h(oe, x1.shape, np.float32).view(np.uint32), want.view(np.uint32))
    for b in (xd, oe, og, xbd, obd):
        b.free()
    dl.free()


def test_graphs_recorded_back_to_back(be, orc):
    """two recordings in a row with no eager call between them (one graph per layer,
    the second gets fresh scratch of the first's capacity), and a third graph's
    destroy issued while another recording is open: every replay bit-identical to
    its eager result"""
    cfg = SMALL[2]
    Ls = [synth.make_layer(orc, cfg, 81 + i) for i in range(2)]
    dls = [DeviceLayer.from_host(be, cfg, L) for L in Ls]
    x = synth.make_x(orc, cfg, 83, 4)
    zero = np.zeros_like(x)
    xd = be.upload(x)
    oe = [be.upload(zero) for _ in dls]
    og = [be.upload(zero) for _ in dls]
    want = []
    for dl, o in zip(dls, oe):
        be.moe_forward(desc_of(cfg), dl.weights(), xd, o, 4)
        be.sync()
        want.append(be.d2h(o, x.shape, np.float32))
    gs = []
    try:
        for dl, o in zip(dls, og):
            be.graph_begin()
            be.moe_forward(desc_of(cfg), dl.weights(), xd, o, 4)
            gs.append(be.graph_end())
        be.graph_begin()                                   # destroy graph 0 while recording graph 2
        be.graph_destroy(gs[0])
        be.moe_forward(desc_of(cfg), dls[0].weights(), xd, og[0], 4)
        gs[0] = be.graph_end()
        for rep in range(3):
            for i in (1, 0):
                be.h2d(og[i], zero)
                be.graph_launch(gs[i])
                be.sync()
                got = be.d2h(og[i], x.shape, np.float32)
                assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), (rep, i)
            be.h2d(oe[0], zero)                            # eager work between replays
            be.moe_forward(desc_of(cfg), dls[0].weights(), xd, oe[0], 4)
            be.sync()
    finally:
        for g in gs:
            be.graph_destroy(g)
        for b in [xd] + oe + og:
            b.free()
        for dl in dls:
            dl.free()


@pytest.mark.parametrize("S_", [2, 33, 200])
def test_device_bucket_matches_oracle(be, orc, S_):
    """the device counting sort (A11): groups in ascending expert id, begin
    offsets and counts equal to the CPU sort of the same picks"""
    cfg = SMALL[4]
    L = synth.make_layer(orc, cfg, 61)
    dl = DeviceLayer.from_host(be, cfg, L)
    x = synth.make_x(orc, cfg, 62, S_)
    xd, od = be.upload(x), be.upload(np.zeros_like(x))
    be.moe_forward(desc_of(cfg), dl.weights(), xd, od, S_)
    G, gexp, gbeg, gcnt = be.last_groups()
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
    xd.free(); od.free(); dl.free()
    Gw, gexp_w, gbeg_w, gcnt_w, _, _ = orc.bucket(sel, S_, cfg.K, cfg.E)
    assert G == Gw
    assert np.array_equal(gexp, gexp_w) and np.array_equal(gbeg, gbeg_w) and np.array_equal(gcnt, gcnt_w)


@pytest.mark.parametrize("S_", [1, 2, 5])
def test_layer_1024_experts(be, orc, S_):
    """E = 1024 (the descriptor's limit): the gate/top-k launch and the counting sort
    hold every expert; routing identical and the layer within tolerance at S = 1 and
    on the grouped path"""
    cfg = cf.scaled(cf.C1, D=512, E=1024, K=8, I=256, name="C1-E1024")
    L = synth.make_layer(orc, cfg, 71)
    x = synth.make_x(orc, cfg, 72, S_)
    base = synth.make_x(orc, cfg, 73, S_)
    want = orc.moe_block_rows(synth.desc_of(cfg), L, x, base)
    dl = DeviceLayer.from_host(be, cfg, L)
    got = be.moe_block(desc_of(cfg), dl.weights(), x, base)
    xd = be.upload(x)
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, S_)
    xd.free(); dl.free()
    _, sel_w, _ = orc.route(synth.desc_of(cfg), L, x)
    assert np.array_equal(sel, sel_w)
    check_small(orc, cfg, L, x, base, got, want, S_)
