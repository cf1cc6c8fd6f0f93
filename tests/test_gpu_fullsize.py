"""Parity at the benchmark's full configurations, on
device-generated layers:

  * C3: the C2 layer at batch 4, 8, 32 and 64 -- routing identical to the oracle's,
    the layer within the tolerance, and every stream of the batch bit-identical
    to its own single-stream call;
  * C4: 2048-token prefill (the grouped GEMMs on the f16 MFMA), with the softplus
    gate and with the Zipf(1.1)-skewed router -- all 2048 rows' routing identical,
    all rows within the tolerance, and sampled streams (the hottest expert's
    included) bit-identical to their single-stream calls;
  * C5: one full-shape layer (E=256, top-8 softmax, I=1536) at batch 8;
  * 64 single-token calls queued back to back, bit-identical to one batched call.

The oracle gets a host copy of each device layer with only the experts it routes
to (tests/fullsize.py).  Tolerance (north_star's max-rel-err 2e-3), both on the MoE
update: normwise max|a-b|/max|b| <= 2e-3 and elementwise |a-b|/max(|b|, 1e-3 max|b|)
<= 2e-3; routing exact."""
import sys

import numpy as np
import pytest

from fullsize import ELEM_FLOOR, errs, host_layer
from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd.backend import DeviceLayer, desc_of

pytestmark = pytest.mark.gpu
TOL = 2e-3


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def run_device(be, cfg, dl, x, base):
    xd, od = be.upload(x), be.upload(base)
    _, sel, _ = be.route(desc_of(cfg), dl.weights(), xd, x.shape[0])
    be.moe_forward(desc_of(cfg), dl.weights(), xd, od, x.shape[0])
    out = be.d2h(od, x.shape, np.float32)
    xd.free(); od.free()
    return sel, out


def single_streams(be, cfg, dl, x, rows):
    """each listed row through its own S = 1 forward (the per-token path)"""
    out = []
    xd, od = be.alloc(cfg.D * 4), be.alloc(cfg.D * 4)
    z = np.zeros((1, cfg.D), np.float32)
    for s in rows:
        be.h2d(xd, x[s:s + 1])
        be.h2d(od, z)
        be.moe_forward(desc_of(cfg), dl.weights(), xd, od, 1)
        out.append(be.d2h(od, (cfg.D,), np.float32))
    xd.free(); od.free()
    return np.stack(out)


def check_layer(be, orc, cfg, seed, S_, sample=None):
    x = synth.make_x(orc, cfg, seed, S_)
    base = np.zeros_like(x)
    dl = DeviceLayer.generate(be, cfg, seed)
    try:
        L, sel_w = host_layer(be, orc, cfg, dl, seed, x)
        want = orc.moe_group_rows(synth.desc_of(cfg), L, x, base)
        sel, got = run_device(be, cfg, dl, x, base)
        assert np.array_equal(sel, sel_w), int(np.sum(sel != sel_w))
        nw, el = errs(got, want, base)
        G = len(np.unique(sel))
        hot = np.bincount(sel.reshape(-1), minlength=cfg.E).max() / sel.size
        say(f"[{cfg.name} S={S_}] normwise {nw:.2e}, elementwise (floor {ELEM_FLOOR:g}) {el:.2e}, G={G}, "
            f"hottest expert {hot:.1%} of pairs")
        assert nw <= TOL and el <= TOL, (nw, el)
        rows = range(S_) if sample is None else sample(sel)
        rows = sorted(set(int(r) for r in rows))
        single = single_streams(be, cfg, dl, x, rows)
        assert np.array_equal(single.view(np.uint32), got[rows].view(np.uint32))
        return sel
    finally:
        dl.free()


@pytest.mark.parametrize("B", [4, 8, 32, 64])
def test_c3_batches(be, orc, B):
    """C3: the C2 layer (softplus gate, K=10, shared expert) at B streams; every
    stream checked against its single-stream output.  B = 4 takes the grouped kernels'
    one-token passes (40 pairs of 256 experts) with the shared expert's batch blocks"""
    check_layer(be, orc, cf.C2, 7100 + B, B)


def _sample(sel, n=24, seed=5):
    """n random streams plus the first streams routed to the hottest expert"""
    rng = np.random.default_rng(seed)
    hot = np.bincount(sel.reshape(-1)).argmax()
    on_hot = np.nonzero((sel == hot).any(axis=1))[0][:8]
    return list(rng.choice(sel.shape[0], n, replace=False)) + list(on_hot)


@pytest.mark.parametrize("cfg", [cf.C2, cf.C4_ZIPF], ids=lambda c: c.name)
def test_c4_prefill(be, orc, cfg):
    """C4: 2048 tokens in one chunk; the Zipf(1.1) variant puts a few experts far
    above the mean load"""
    sel = check_layer(be, orc, cfg, 7300, 2048, sample=_sample)
    if cfg.zipf > 0:
        cnt = np.sort(np.bincount(sel.reshape(-1), minlength=cfg.E))[::-1]
        assert cnt[0] > 4 * sel.size / cfg.E          # skewed: the hottest expert far above the mean


def test_c5_layer_b8(be, orc):
    """C5's layer shape (E=256, top-8 softmax, I=1536, no shared) at batch 8"""
    check_layer(be, orc, cf.C5_LAYER, 7500, cf.C5_BATCH)


@pytest.mark.parametrize("cfg", [cf.C2, cf.C5_LAYER], ids=lambda c: c.name)
def test_single_tokens_back_to_back(be, orc, cfg):
    """64 single-token forwards queued back to back with no host synchronisation
    between them (each token's gate + top-k runs in every block of its expert stage)
    against one batched forward (a gate launch and the grouped kernels): every output
    bit-identical to its batched row, with softplus scores (C2) and softmax logits (C5)."""
    S_, seed = 64, 7600
    x = synth.make_x(orc, cfg, seed, S_)
    dl = DeviceLayer.generate(be, cfg, seed)
    xd, ob, o1 = be.upload(x), be.upload(np.zeros_like(x)), be.upload(np.zeros_like(x))
    try:
        be.moe_forward(desc_of(cfg), dl.weights(), xd, ob, S_)
        for s in range(S_):
            off = s * cfg.D * 4
            be.moe_forward(desc_of(cfg), dl.weights(), int(xd) + off, int(o1) + off, 1)
        batch = be.d2h(ob, x.shape, np.float32)
        single = be.d2h(o1, x.shape, np.float32)
        bad = np.nonzero((single.view(np.uint32) != batch.view(np.uint32)).any(axis=1))[0]
        assert bad.size == 0, f"tokens {bad.tolist()} differ"
    finally:
        for b in (xd, ob, o1):
            b.free()
        dl.free()


def test_c5_stack_48_layers(be, orc):
    """C5: the 48-layer resident stack at batch 8 with the 4096 x 32000 bf16 head:
    the device step's greedy tokens equal the oracle's, whose layers are fed one at
    a time (h += MoE(rmsnorm(h)), c/laguna.c:1156-1160; rmsnorm c/moe_math.h:58-62)"""
    from sabrewing_amd.stack import NORM_EPS, DeviceStack, head_bf16, norm_weights
    cfg, nL, V, B, seed = cf.C5_LAYER, cf.C5_LAYERS, cf.C5_VOCAB, cf.C5_BATCH, 7700
    st = DeviceStack.generate(be, cfg, nL, V, seed)
    try:
        h0 = synth.make_x(orc, cfg, seed, B)
        hd, xn, ld, td = be.upload(h0), be.alloc(B * cfg.D * 4), be.alloc(B * V * 4), be.alloc(B * 4)
        st.step(hd, xn, ld, td, B)
        h_dev = be.d2h(hd, h0.shape, np.float32)
        lg_dev = be.d2h(ld, (B, V), np.float32)
        tok_dev = be.d2h(td, (B,), np.int32)
        for b in (hd, xn, ld, td):
            b.free()
        nw = norm_weights(orc, cfg, seed, nL)
        h = h0.copy()
        for l in range(nL):
            x = orc.rmsnorm_rows(h, nw[l], NORM_EPS)
            L, _ = host_layer(be, orc, cfg, st.layers[l], seed, x, layer=l)
            h = orc.moe_group_rows(synth.desc_of(cfg), L, x, h)
            del L
            if l % 8 == 7:
                say(f"[C5 stack] oracle through layer {l + 1} of {nL}")
        logits = orc.matmul_bf16(orc.rmsnorm_rows(h, nw[nL], NORM_EPS), head_bf16(orc, cfg, seed, V))
        tok = orc.argmax_rows(logits)
    finally:
        st.free()
    srt = np.sort(logits, axis=1)
    err = float(np.max(np.abs(lg_dev - logits)))
    nw, el = errs(h_dev, h, h0)
    say(f"[C5 stack] tokens dev {tok_dev.tolist()} oracle {tok.tolist()}; residual normwise {nw:.2e}, elementwise "
        f"{el:.2e}; logit max|err| {err:.2e}; top-2 margins {np.round(srt[:, -1] - srt[:, -2], 4).tolist()}")
    assert nw <= TOL and el <= TOL, (nw, el)
    assert np.array_equal(tok_dev, tok)
