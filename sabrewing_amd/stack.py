"""A stack of MoE layers on the device, the shape of the reference engines'
decode step: for every layer h += MoE(rmsnorm(h, w_l)), then rmsnorm(h, w_f),
the bf16 head and a greedy pick (c/laguna.c forward_span / argmax_logits,
c/laguna.c:1156-1160; rmsnorm_row c/moe_math.h:58-62).

Synthetic stacks are seeded like the layers: norm weights 1 + N(0, 0.02)
(tensor T_NORM of layer l, the final norm as layer L), the head N(0, 0.02)
bf16 [V, D] (tensor T_HEAD).
"""
import numpy as np

from . import synth
from .backend import DeviceLayer, desc_of
from .configs import WEIGHT_SIGMA

NORM_EPS = 1e-6


class DeviceStack:
    def __init__(self, be, cfg, V):
        self.be, self.cfg, self.V = be, cfg, V
        self.layers, self.norms, self.bufs = [], [], []
        self.final_norm = self.head = None

    @classmethod
    def from_host(cls, be, cfg, host_layers, norms, final_norm, head_bf16):
        """host_layers: oracle.synth.Layer list; norms: [L, D] f32; head_bf16: u16 [V, D]"""
        self = cls(be, cfg, head_bf16.shape[0])
        self.layers = [DeviceLayer.from_host(be, cfg, L) for L in host_layers]
        self.norms = [self._keep(be.upload(np.ascontiguousarray(n, np.float32))) for n in norms]
        self.final_norm = self._keep(be.upload(np.ascontiguousarray(final_norm, np.float32)))
        self.head = self._keep(be.router_upload(head_bf16, True))
        return self

    @classmethod
    def generate(cls, be, cfg, n_layers, V, seed):
        """Everything generated on the device (the bits of norm_weights / head_bf16)."""
        self = cls(be, cfg, V)
        self.layers = [DeviceLayer.generate(be, cfg, seed, layer=l) for l in range(n_layers)]
        D = cfg.D
        for l in range(n_layers + 1):
            g = be.alloc(D * 4)
            be.gen_normal(g, D, synth.tensor_seed(seed, l, synth.T_NORM), WEIGHT_SIGMA)
            w = (np.float32(1.0) + be.d2h(g, (D,), np.float32)).astype(np.float32)
            g.free()
            b = self._keep(be.upload(w))
            if l < n_layers:
                self.norms.append(b)
            else:
                self.final_norm = b
        tmp = be.alloc(V * D * 2)
        be.gen_bf16(tmp, V * D, synth.tensor_seed(seed, 0, synth.T_HEAD), WEIGHT_SIGMA)
        self.head = self._keep(be.alloc((V + 3) // 4 * 4 * D * 2))
        be.check(be.lib.lag_hip_router_chain(int(tmp), int(self.head), V, D, 1), "head chain")
        be.sync()
        tmp.free()
        return self

    def _keep(self, b):
        self.bufs.append(b)
        return b

    def step(self, h, xn, logits, tok, S, fused=True):
        """h [S, D] (device, updated in place), xn [S, D] scratch, logits [S, V], tok [S] int32;
        fused: each layer's RMSNorm inside its routing launch (lag_hip_moe_forward_rmsnorm,
        the same bits as the separate rmsnorm + forward)"""
        be, D = self.be, self.cfg.D
        desc = desc_of(self.cfg)
        for l, dl in enumerate(self.layers):
            if fused:
                be.moe_forward_rmsnorm(desc, dl.weights(), self.norms[l], NORM_EPS, xn, h, S)
            else:
                be.rmsnorm(h, self.norms[l], xn, S, D, NORM_EPS)
                be.moe_forward(desc, dl.weights(), xn, h, S)
        be.rmsnorm(h, self.final_norm, xn, S, D, NORM_EPS)
        be.head_argmax(self.head, True, xn, S, D, self.V, logits, tok)

    def free(self):
        for dl in self.layers:
            dl.free()
        for b in self.bufs:
            b.free()
        self.layers, self.bufs = [], []


def norm_weights(orc, cfg, seed, n_layers):
    """[n_layers + 1, D] f32: 1 + N(0, 0.02) per layer, the final norm last"""
    return np.stack([1.0 + orc.normal(cfg.D, synth.tensor_seed(seed, l, synth.T_NORM), WEIGHT_SIGMA)
                     for l in range(n_layers + 1)]).astype(np.float32)


def head_bf16(orc, cfg, seed, V):
    return orc.to_bf16(orc.normal(V * cfg.D, synth.tensor_seed(seed, 0, synth.T_HEAD), WEIGHT_SIGMA)).reshape(V, cfg.D)
