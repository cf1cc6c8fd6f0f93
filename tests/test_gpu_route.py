"""Routing on the device against the CPU reference contract, bit for bit:
router logits (16-lane FMA chains + the GCC reduction tree), gate scores
(glibc-exact expf/log1pf), top-k selection and renormalised weights."""
from dataclasses import replace

import numpy as np
import pytest

from oracle import synth
from sabrewing_amd import configs as cf
from sabrewing_amd import synth as S
from sabrewing_amd.backend import LagHipMoeWeights, desc_of
import ctypes as C

pytestmark = pytest.mark.gpu


def router_layer(orc, cfg, seed, corr_sigma=0.0):
    """a host layer with only the routing tensors filled in"""
    E, D = cfg.E, cfg.D
    r = orc.normal(E * D, S.tensor_seed(seed, 0, S.T_ROUTER), 0.02).reshape(E, D)
    router = orc.to_bf16(r) if cfg.router_bf16 else r
    corr = None
    if cfg.use_corr_bias:
        corr = orc.normal(E, S.tensor_seed(seed, 0, S.T_CORR_BIAS), corr_sigma) if corr_sigma else np.zeros(E, np.float32)
    lb = S.zipf_bias(E, cfg.zipf, 77) if cfg.zipf > 0 else None
    z8 = np.zeros(8, np.uint8); z4 = np.zeros(2, np.float32)
    return synth.Layer(D, cfg.I, cfg.Is, E, cfg.gs, cfg.router_bf16, router, corr, lb, z8, z4, z8, z4, None, None, None)


def device_route(be, cfg, L, x):
    keep = [be.router_upload(L.router, cfg.router_bf16)]
    dummy = be.alloc(256); keep.append(dummy)
    cb = lb = None
    if L.corr_bias is not None:
        cb = be.upload(L.corr_bias); keep.append(cb)
    if L.logit_bias is not None:
        lb = be.upload(L.logit_bias); keep.append(lb)
    p = lambda b: C.c_void_p(int(b)) if b is not None else None
    d = dummy
    w = LagHipMoeWeights(p(keep[0]), p(cb), p(lb), p(d), p(d), p(d), p(d), p(d), p(d), p(d))
    xd = be.upload(np.ascontiguousarray(x, np.float32)); keep.append(xd)
    out = be.route(desc_of(cfg), w, xd, x.shape[0])
    for b in keep:
        b.free()
    return out


CASES = [
    (cf.C1, 0.0),                                                  # f32 router, softmax, no bias
    (cf.C2_SIGMOID, 0.01),                                         # bf16 router, sigmoid + correction bias
    (cf.C2, 0.01),                                                 # softplus, renormalised
    (cf.C4_ZIPF, 0.0),                                             # skew: logit bias
    (cf.C5_LAYER, 0.0),                                            # softmax over 256
    (replace(cf.C2_SIGMOID, name="C2-sigmoid-nonorm", norm_topk=0), 0.02),
    (cf.C1_OLMOE, 0.0),                                            # OLMoE engine: float-sum softmax, divide
    (replace(cf.C1_OLMOE, name="C1-olmoe-nonorm", norm_topk=0), 0.0),
    (cf.QWEN, 0.0),                                                # qwen35: double softmax, double renorm
    (cf.C2_SQRTSP, 0.01),                                          # DeepSeek-V4's sqrt(softplus) + correction bias
]


@pytest.mark.parametrize("cfg,corr", CASES, ids=[c[0].name for c in CASES])
@pytest.mark.parametrize("S_", [1, 5, 64])
def test_route_bit_exact(be, orc, cfg, corr, S_):
    L = router_layer(orc, cfg, 2024, corr)
    x = synth.make_x(orc, cfg, 2024 + S_, S_)
    lg_w, sel_w, w_w = orc.route(synth.desc_of(cfg), L, x)
    lg, sel, w = device_route(be, cfg, L, x)
    assert np.array_equal(lg.view(np.uint32), lg_w.view(np.uint32))
    assert np.array_equal(sel, sel_w)
    assert np.array_equal(w.view(np.uint32), w_w.view(np.uint32))


def test_route_ties_and_nonfinite(be, orc):
    """Crafted logits through the device top-k: exact ties (lowest id wins),
    a NaN-scoring expert, and correction-bias ties."""
    cfg = replace(cf.C2_SIGMOID, name="tie", E=64, K=8, D=128)
    E, D = cfg.E, cfg.D
    # router rows that give identical logits to pairs of experts
    rng = np.random.default_rng(5)
    base = (rng.standard_normal((E // 2, D)) * 0.02).astype(np.float32)
    Wf = np.repeat(base, 2, axis=0)
    L = router_layer(orc, cfg, 1)
    L.router = orc.to_bf16(Wf)
    L.corr_bias = np.zeros(E, np.float32)
    x = synth.make_x(orc, cfg, 3, 4)
    x[1, 0] = np.nan                      # a poisoned token: every logit NaN -> fallback ids
    lg_w, sel_w, w_w = orc.route(synth.desc_of(cfg), L, x)
    lg, sel, w = device_route(be, cfg, L, x)
    assert np.array_equal(sel, sel_w)
    ok = (w.view(np.uint32) == w_w.view(np.uint32)) | (np.isnan(w) & np.isnan(w_w))
    assert ok.all()
    assert list(sel_w[1]) == list(range(cfg.K))


SOFTMAX = [cf.C1, cf.C5_LAYER, cf.QWEN]


@pytest.mark.parametrize("cfg", SOFTMAX, ids=[c.name for c in SOFTMAX])
@pytest.mark.parametrize("xscale", [1.0, 8.0])
def test_route_softmax_sum_paths(be, orc, cfg, xscale):
    """The softmax's double sum takes a wave tree when every nonzero term is at least
    2^-19 (then every partial sum is exact, so any order gives the expert-order sum) and
    the expert-order scan otherwise.  x as drawn keeps every token on the tree; x * 8
    spreads the logits so that every token has terms below 2^-19 and takes the scan.
    Both must give the reference's bits."""
    L = router_layer(orc, cfg, 77)
    x = synth.make_x(orc, cfg, 78, 16) * np.float32(xscale)
    lg_w, sel_w, w_w = orc.route(synth.desc_of(cfg), L, x)
    lg64 = lg_w[:, :cfg.E].astype(np.float64)
    p = np.exp(lg64 - lg64.max(1, keepdims=True)).astype(np.float32)
    tiny = ((p > 0) & (p < 2.0 ** -19)).any(1)
    assert (not tiny.any()) if xscale == 1.0 else tiny.all()      # the path each token takes
    lg, sel, w = device_route(be, cfg, L, x)
    assert np.array_equal(lg.view(np.uint32), lg_w.view(np.uint32))
    assert np.array_equal(sel, sel_w)
    assert np.array_equal(w.view(np.uint32), w_w.view(np.uint32))
