"""Helpers of the full-size parity tests: host copies of device-generated layers.

A full-size layer is generated in HBM by the device generator (bit-identical to
the host generator: tests/test_gpu_kernels.py pins it), and the oracle gets a
host copy of it one layer at a time.  Only the experts the oracle's own routing
picks are copied back (moe_block never reads the others), into zero-filled
arrays whose untouched pages cost no host memory.  The router, the correction
and Zipf biases and the norms are small and regenerated on the host."""
import ctypes as C

import numpy as np

from oracle import synth
from sabrewing_amd import synth as S


def _d2h_into(be, dst, src, src_off):
    """dst[:] <- device bytes at int(src) + src_off"""
    dst = np.ascontiguousarray(dst)
    be.check(be.lib.lag_hip_d2h(dst.ctypes.data_as(C.c_void_p), C.c_void_p(int(src) + src_off), dst.nbytes), "d2h")


def host_layer(be, orc, cfg, dl, seed, x, layer=0):
    """(host Layer with the experts routed by x copied from device layer dl, sel [S, K])"""
    D, I, E, gs = cfg.D, cfg.I, cfg.E, cfg.gs
    ngD, ngI = (D // gs, I // gs) if gs else (1, 1)
    ts = lambda tid: S.tensor_seed(seed, layer, tid)
    R, ns = cfg.router_rows, cfg.n_shared_experts
    r = orc.normal(R * D, ts(S.T_ROUTER), 0.02).reshape(R, D)
    router = orc.to_bf16(r) if cfg.router_bf16 else r
    corr = np.zeros(E, np.float32) if cfg.use_corr_bias else None
    lb = S.zipf_bias(E, cfg.zipf, ts(S.T_ROUTER) ^ 0x5A5A) if cfg.zipf > 0 else None
    gu_q = np.zeros((E * 2 * I, D // 2), np.uint8)
    gu_s = np.zeros((E * 2 * I, ngD), np.float32)
    dn_q = np.zeros((E * D, I // 2), np.uint8)
    dn_s = np.zeros((E * D, ngI), np.float32)
    sg = su = sd = None
    if cfg.shared_mode:
        sg = be.d2h(dl.sg, (ns * cfg.Is, D), np.uint16)
        su = be.d2h(dl.su, (ns * cfg.Is, D), np.uint16)
        sd = be.d2h(dl.sd, (ns * D, cfg.Is), np.uint16)
    L = synth.Layer(D, I, cfg.Is, E, gs, cfg.router_bf16, router, corr, lb, gu_q.reshape(-1), gu_s.reshape(-1),
                    dn_q.reshape(-1), dn_s.reshape(-1), sg, su, sd)
    _, sel, _ = orc.route(synth.desc_of(cfg), L, x)
    for e in np.unique(sel):
        e = int(e)
        r0, r1 = e * 2 * I, (e + 1) * 2 * I
        _d2h_into(be, gu_q[r0:r1], dl.gu_q, r0 * (D // 2))
        _d2h_into(be, gu_s[r0:r1], dl.gu_s, r0 * ngD * 4)
        r0, r1 = e * D, (e + 1) * D
        _d2h_into(be, dn_q[r0:r1], dl.dn_q, r0 * (I // 2))
        _d2h_into(be, dn_s[r0:r1], dl.dn_s, r0 * ngI * 4)
    return L, sel


def normwise(got, want, base):
    """max |(got - base) - (want - base)| / max |want - base|: the MoE update's error"""
    dw = want - base
    return float(np.max(np.abs((got - base) - dw))) / float(np.max(np.abs(dw)))


# Elementwise errors are taken relative to max(|want|, ELEM_FLOOR * max|want|): an
# output that the experts' sum cancels to near zero is judged against a thousandth of
# the layer's largest output instead of its own magnitude.
ELEM_FLOOR = 1e-3


def errs(got, want, base):
    """(normwise, floored elementwise) relative errors of the MoE update d = out - base:
    max|d_got - d_want| / max|d_want|, and max_i |d_got - d_want|_i / max(|d_want|_i,
    ELEM_FLOOR * max|d_want|)"""
    dg, dw = (got - base).astype(np.float64), (want - base).astype(np.float64)
    m = float(np.max(np.abs(dw)))
    d = np.abs(dg - dw)
    return float(np.max(d)) / m, float(np.max(d / np.maximum(np.abs(dw), ELEM_FLOOR * m)))


def dequant_q4(q, s, rows, K, gs):
    """float64 [rows, K] of an int4 container (low nibble = even input, value n - 8) times
    its f32 scales (one per row, or one per gs inputs)"""
    q = np.asarray(q, np.uint8).reshape(rows, K // 2)
    n = np.empty((rows, K), np.float64)
    n[:, 0::2] = (q & 15).astype(np.float64) - 8.0
    n[:, 1::2] = (q >> 4).astype(np.float64) - 8.0
    s = np.asarray(s, np.float32).astype(np.float64)
    return n * (np.repeat(s.reshape(rows, K // gs), gs, axis=1) if gs > 0 else s.reshape(rows, 1))


def bf16_f64(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def exact_layer(cfg, L, x, base, sel, w):
    """The MoE block in float64 on the same weights, picks and weights (moe_block's
    arithmetic, c/moe_block.h:18-54, without f32 rounding): out = base + route_scale *
    sum_a w_a down_e(silu(gate_e x) * up_e x) + shared(x).  The yardstick for the
    reduced-size layers, where the f32 reference's own rounding is near the bar."""
    D, I, Is, E, gs = cfg.D, cfg.I, cfg.Is, cfg.E, cfg.gs
    x = np.asarray(x, np.float64)
    out = np.asarray(base, np.float64).copy()
    silu_glu = lambda g, u: g / (1.0 + np.exp(-g)) * u
    sh = cfg.shared_mode == 1
    if sh:
        Wsg, Wsu, Wsd = bf16_f64(L.sg), bf16_f64(L.su), bf16_f64(L.sd)
    for s in range(x.shape[0]):
        acc = np.zeros(D)
        for a in range(cfg.K):
            e = int(sel[s, a])
            gu = dequant_q4(L.gu_q[e * 2 * I * D // 2:(e + 1) * 2 * I * D // 2],
                            L.gu_s[e * 2 * I * (D // gs if gs else 1):(e + 1) * 2 * I * (D // gs if gs else 1)],
                            2 * I, D, gs) @ x[s]
            h = silu_glu(gu[:I], gu[I:])
            dn = dequant_q4(L.dn_q[e * D * I // 2:(e + 1) * D * I // 2],
                            L.dn_s[e * D * (I // gs if gs else 1):(e + 1) * D * (I // gs if gs else 1)], D, I, gs)
            acc += float(w[s, a]) * (dn @ h)
        out[s] += acc * cfg.route_scale
        if sh:
            out[s] += Wsd @ silu_glu(Wsg @ x[s], Wsu @ x[s])
    return out
