"""Seeded synthetic-workload helpers shared by the host and the device generator.

The element stream is SplitMix64 (a counter-based draw per element pair) fed
through Box-Muller in double; the device generator (csrc/k_gen.hip) and the
CPU checker evaluate the same fixed sequence of IEEE operations, so a tensor
generated on the GPU is bit-identical to the same tensor generated on the host.
This module holds the small host-side pieces: per-tensor seeds and the
Zipf-skew router bias of the prefill skew variant.
"""
import math
import numpy as np

M64 = (1 << 64) - 1
T_ROUTER, T_GATE_UP, T_DOWN, T_SH_GATE, T_SH_UP, T_SH_DOWN, T_X, T_CORR_BIAS, T_NORM, T_HEAD = range(1, 11)


def mix64(z):
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def u64(seed, i):
    return mix64((seed + (i + 1) * 0x9E3779B97F4A7C15) & M64)


def tensor_seed(base, layer, tensor_id):
    k = ((layer & 0xFFFFFFFF) << 8) | (tensor_id & 0xFFFFFFFF)
    return mix64((base & M64) ^ mix64((k + 0x632BE59BD9B4E019) & M64))


def zipf_bias(E, alpha, seed):
    """Per-expert additive router-logit bias b_e = -alpha * ln(rank_e), with
    rank_e in 1..E a seeded permutation (experts ordered by their u64 draw).
    Applied after the router GEMV and before the gate activation, on both the
    CPU reference and the device path (a router-hook wrapper, c/moe_arch.h:47)."""
    keys = [u64(seed, e) for e in range(E)]
    order = sorted(range(E), key=lambda e: keys[e])
    rank = np.empty(E, np.int64)
    for r, e in enumerate(order):
        rank[e] = r + 1
    return np.array([-alpha * math.log(float(r)) for r in rank], dtype=np.float32)
