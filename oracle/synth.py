"""Host-side synthetic MoE layers for the CPU checker (test infrastructure).

Builds every tensor of one layer from the workload config and a base seed with
the oracle's generator; the device generator produces the same bits.
"""
from dataclasses import dataclass
from typing import Optional
import numpy as np

from sabrewing_amd.configs import WEIGHT_SIGMA
from sabrewing_amd import synth as S


@dataclass
class Desc:
    E: int
    K: int
    route_act: int
    use_corr_bias: int
    norm_topk: int
    route_scale: float
    shared_mode: int
    n_shared: int = 0


@dataclass
class Layer:
    D: int
    I: int
    Is: int
    E: int
    gs: int
    router_bf16: bool
    router: np.ndarray            # f32 [E,D] or u16 (bf16) [E,D]
    corr_bias: Optional[np.ndarray]
    logit_bias: Optional[np.ndarray]
    gu_q: np.ndarray
    gu_s: np.ndarray
    dn_q: np.ndarray
    dn_s: np.ndarray
    sg: Optional[np.ndarray]
    su: Optional[np.ndarray]
    sd: Optional[np.ndarray]

    def router_f32(self):
        if not self.router_bf16:
            return self.router
        return (self.router.astype(np.uint32) << 16).view(np.float32)


def desc_of(cfg):
    return Desc(cfg.E, cfg.K, cfg.route_act, cfg.use_corr_bias, cfg.norm_topk, cfg.route_scale, cfg.shared_mode,
                cfg.n_shared)


def make_layer(orc, cfg, base_seed, layer=0, corr_bias_sigma=0.0):
    D, I, Is, E, gs = cfg.D, cfg.I, cfg.Is, cfg.E, cfg.gs
    ts = lambda tid: S.tensor_seed(base_seed, layer, tid)
    R, ns = cfg.router_rows, cfg.n_shared_experts
    r = orc.normal(R * D, ts(S.T_ROUTER), WEIGHT_SIGMA).reshape(R, D)
    router = orc.to_bf16(r) if cfg.router_bf16 else r
    gu_q, gu_s = orc.gen_q4(ts(S.T_GATE_UP), WEIGHT_SIGMA, E * 2 * I, D, gs)
    dn_q, dn_s = orc.gen_q4(ts(S.T_DOWN), WEIGHT_SIGMA, E * D, I, gs)
    sg = su = sd = None
    if cfg.shared_mode:                  # ns experts stacked: [ns*Is, D], [ns*Is, D], [ns*D, Is]
        sg = orc.to_bf16(orc.normal(ns * Is * D, ts(S.T_SH_GATE), WEIGHT_SIGMA)).reshape(ns * Is, D)
        su = orc.to_bf16(orc.normal(ns * Is * D, ts(S.T_SH_UP), WEIGHT_SIGMA)).reshape(ns * Is, D)
        sd = orc.to_bf16(orc.normal(ns * D * Is, ts(S.T_SH_DOWN), WEIGHT_SIGMA)).reshape(ns * D, Is)
    corr = None
    if cfg.use_corr_bias:
        corr = (orc.normal(E, ts(S.T_CORR_BIAS), corr_bias_sigma) if corr_bias_sigma > 0
                else np.zeros(E, np.float32))
    lb = S.zipf_bias(E, cfg.zipf, ts(S.T_ROUTER) ^ 0x5A5A) if cfg.zipf > 0 else None
    return Layer(D, I, Is, E, gs, cfg.router_bf16, router, corr, lb,
                 gu_q.reshape(-1), gu_s.reshape(-1), dn_q.reshape(-1), dn_s.reshape(-1), sg, su, sd)


def make_x(orc, cfg, base_seed, S_rows, stream=0):
    """S_rows tokens of N(0,1) activations (bf16-valued when cfg.x_bf16)."""
    x = orc.normal(S_rows * cfg.D, S.tensor_seed(base_seed, 1000 + stream, S.T_X), 1.0).reshape(S_rows, cfg.D)
    return orc.bf16_round(x).reshape(S_rows, cfg.D) if cfg.x_bf16 else x
