"""Workload configurations of the MoE-block benchmark.

C1  OLMoE-1B-7B-shaped layer: D=2048, E=64, top-8 softmax, I=1024, no shared
    expert, f32 router, f32 activations.
C2  Laguna-style layer: D=4096, E=256, top-10 + 1 always-on shared expert,
    I=1024, Is=1024 (shared width not stated by the benchmark; Laguna's own
    shared expert is as wide as a routed one), bf16 router and shared expert,
    bf16-valued activations.  Gate "softplus" with renormalised top-k weights
    (the benchmark's wording), plus the Laguna-faithful "sigmoid" variant
    (e_score_correction_bias for selection, norm_topk, route_scale 2.5;
    c/laguna.c:819) used for engine-level parity.
C3  C2 at batch 1/8/32/64 (batched decode through the grouped path).
C4  C2 prefill, 2048 tokens, plus a Zipf(1.1)-skewed router variant.
C5  48 resident layers of D=4096, E=256, top-8 softmax, I=1536, batch 8,
    RMSNorm + residual between layers, bf16 4096x32000 head + greedy argmax.
All int4 experts use group-32 f32 scales (moe_quant.h nibbles, quant.h fmt=4
scale layout).  Weights N(0, 0.02), activations N(0, 1).
"""
from dataclasses import dataclass, replace

ROUTE_SIGMOID, ROUTE_SOFTMAX, ROUTE_SOFTPLUS = 0, 1, 2
# other callers' routing contracts (c/olmoe.c:607-632; c/qwen35.c:558-589)
ROUTE_SOFTMAX_OLMOE, ROUTE_SOFTMAX_QWEN = 3, 4
# DeepSeek-V4's router score sqrtf(softplusf(x)) (c/deepseek.c:854) as a moe_block gate
ROUTE_SQRT_SOFTPLUS = 5
# the Inkling engine's routing (c/inkling.c:1027-1043): sigmoid + bias selection, weights
# normalised over the K picks and the n_shared shared-expert gates, x route_scale
ROUTE_INKLING = 6
# Inkling's shared experts, weighted from that pool (c/inkling.c:1166-1183)
SHARED_NONE, SHARED_UNSCALED, SHARED_GATED = 0, 1, 3
WEIGHT_SIGMA = 0.02


@dataclass(frozen=True)
class MoeConfig:
    name: str
    D: int
    E: int
    K: int
    I: int
    Is: int
    route_act: int
    use_corr_bias: int
    norm_topk: int
    route_scale: float
    shared_mode: int
    gs: int = 32
    router_bf16: bool = True
    x_bf16: bool = True
    zipf: float = 0.0          # >0: per-expert logit bias -zipf*ln(rank) (skew variant)
    n_shared: int = 0          # ROUTE_INKLING: shared gate rows after the E routed ones; SHARED_GATED: experts

    @property
    def ngD(self):
        return (self.D + self.gs - 1) // self.gs if self.gs > 0 else 1

    @property
    def ngI(self):
        return (self.I + self.gs - 1) // self.gs if self.gs > 0 else 1

    def expert_bytes(self):
        """int4 nibbles + f32 scales of one routed expert (gate_up + down)."""
        nib = 2 * self.I * ((self.D + 1) // 2) + self.D * ((self.I + 1) // 2)
        sc = 4 * (2 * self.I * self.ngD + self.D * self.ngI)
        return nib + sc

    @property
    def router_rows(self):
        return self.E + (self.n_shared if self.route_act == ROUTE_INKLING else 0)

    @property
    def n_shared_experts(self):
        return self.n_shared if self.shared_mode == SHARED_GATED else (1 if self.shared_mode else 0)

    def router_bytes(self):
        return self.router_rows * self.D * (2 if self.router_bf16 else 4)

    def shared_bytes(self):
        return 3 * self.D * self.Is * 2 * self.n_shared_experts

    def step_bytes(self, S, G):
        """Algorithmic HBM bytes of one layer pass over S tokens touching G
        distinct experts: each expert, the router and the shared expert read
        once, activations in (f32) and out (f32 read-modify-write)."""
        return G * self.expert_bytes() + self.router_bytes() + self.shared_bytes() + 3 * S * self.D * 4

    def flops(self, S):
        return 2 * S * (self.K * 3 * self.D * self.I + (3 * self.D * self.Is if self.shared_mode else 0) + self.D * self.E)


C1 = MoeConfig("C1-olmoe", D=2048, E=64, K=8, I=1024, Is=0, route_act=ROUTE_SOFTMAX, use_corr_bias=0,
               norm_topk=0, route_scale=1.0, shared_mode=SHARED_NONE, router_bf16=False, x_bf16=False)
C2 = MoeConfig("C2-laguna-softplus", D=4096, E=256, K=10, I=1024, Is=1024, route_act=ROUTE_SOFTPLUS,
               use_corr_bias=1, norm_topk=1, route_scale=2.5, shared_mode=SHARED_UNSCALED)
C2_SIGMOID = replace(C2, name="C2-laguna-sigmoid", route_act=ROUTE_SIGMOID)
C4_ZIPF = replace(C2, name="C4-laguna-zipf", zipf=1.1)
C5_LAYER = MoeConfig("C5-inkling-small", D=4096, E=256, K=8, I=1536, Is=0, route_act=ROUTE_SOFTMAX,
                     use_corr_bias=0, norm_topk=0, route_scale=1.0, shared_mode=SHARED_NONE)
C5_LAYERS, C5_BATCH, C5_VOCAB = 48, 8, 32000

# C1 routed as the OLMoE engine routes it; a qwen35-style layer (int4 experts through
# lag_cuda_moe_group, softmax top-8 renormalised in double, c/qwen35.c:600-640)
# a DeepSeek-V4-shaped gate (c/deepseek.c:854): sqrt(softplus) scores with the correction
# bias in the selection, on the C2 layer shape (a parity case, not a bench config)
C2_SQRTSP = replace(C2, name="C2-sqrt-softplus", route_act=ROUTE_SQRT_SOFTPLUS)
C1_OLMOE = replace(C1, name="C1-olmoe-engine-routing", route_act=ROUTE_SOFTMAX_OLMOE, norm_topk=1)
QWEN = MoeConfig("qwen35-moe", D=2048, E=256, K=8, I=512, Is=0, route_act=ROUTE_SOFTMAX_QWEN,
                 use_corr_bias=0, norm_topk=0, route_scale=1.0, shared_mode=SHARED_NONE, router_bf16=False,
                 x_bf16=False)
# an Inkling-shaped layer (c/inkling.c:1011-1183; docs/inkling.md): f32 router over E + 2 rows,
# sigmoid + correction-bias selection, 2 gated bf16 shared experts, per-row int4 experts,
# route_scale 8 x a gate.global_scale of 1 (a parity case, not a bench config)
INKLING = MoeConfig("inkling-gated", D=4096, E=256, K=6, I=2048, Is=2048, route_act=ROUTE_INKLING,
                    use_corr_bias=1, norm_topk=0, route_scale=8.0, shared_mode=SHARED_GATED, gs=0,
                    router_bf16=False, x_bf16=False, n_shared=2)
CONFIGS = {c.name: c for c in (C1, C2, C2_SIGMOID, C4_ZIPF, C5_LAYER, C1_OLMOE, QWEN, INKLING)}


def scaled(cfg, D=None, E=None, K=None, I=None, Is=None, name=None):
    """A reduced-size copy of a config (same contracts) for quick parity runs."""
    kw = {}
    for k, v in dict(D=D, E=E, K=K, I=I, Is=Is).items():
        if v is not None:
            kw[k] = v
    if cfg.shared_mode == SHARED_NONE:
        kw["Is"] = 0
    return replace(cfg, name=name or (cfg.name + "-small"), **kw)
