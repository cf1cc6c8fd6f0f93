"""MoE-layer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B] [--config NAME]

A step is one pass of the MoE block (router -> gate -> top-k -> group-by-expert
-> int4 SwiGLU experts -> combine -> shared expert -> residual) over one batch
of synthetic tokens already resident in HBM, through lag_hip_moe_forward.
Weights are seeded N(0, 0.02) int4 group-32 (generated on the device); every
step takes fresh N(0,1) tokens and steps rotate over `--layers` distinct layers
so that the 256 MB Infinity Cache cannot hold what a step reads.

Prints one JSON line: tokens/s of the whole job, the roofline of the dominant
kernel (algorithmic bytes / average launch time, from HIP events on the
backend stream), the layer's HBM fraction, and the reference CPU path timed
on this host's cores on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# MI355X dense bf16 MFMA (the peak BASELINE prices the prefill at; the kernels issue f16
# MFMAs, 2 per int4 multiply-add of the layer (one per 12-bit digit), against the same
# 2.5 P flop/s dense f16 peak)
MFMA_PEAK_TFS = 2500.0
# what the kernels compute in: int4 weights and their f32 group scales against the
# activations written per 32 inputs as integers of 7 signed base-8 digits (held as 6
# base-16 limbs) under a power-of-two factor (exact integer dots, |input error| <= 2^-21
# of the group's largest input);
# f32 accumulation; the router and the shared expert in f32 fma chains on bf16 weights
DTYPE = ("int4 weights x activation integers of 7 base-8 digits per 32 inputs (2^-21 of the group max, held as 6 base-16 limbs), "
         "exact int32 dots, f32 scales and accumulation; router f32 FMA chains on bf16 weights; "
         "shared expert bf16 weights x f32 inputs split exactly into three bf16 parts on the MFMA")
# the reference CPU baseline's OpenMP placement (c/moe_util.h:78-86 sets one thread per
# physical core; the pinning is the reference's measured setting); read when the
# OpenMP runtime first starts, so set before any OpenMP library loads
os.environ.setdefault("OMP_PROC_BIND", "spread")
os.environ.setdefault("OMP_PLACES", "cores")


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def kernel_bytes(cfg, S, G):
    """algorithmic HBM bytes per launch of each kernel of the forward pass:
    every weight byte the launch needs once, activations in and out once
    (dot8 limbs: 6 x 16 bytes + one f32 factor per 32 inputs)"""
    D, I, Is, E, K = cfg.D, cfg.I, cfg.Is, cfg.E, cfg.K
    ngD, ngI = (D // cfg.gs, I // cfg.gs) if cfg.gs else (1, 1)
    T = S * K
    limb = lambda n: n // 32 * (6 * 16 + 4)
    gu_w = G * (2 * I * D // 2 + 2 * I * ngD * 4)
    dn_w = G * (D * I // 2 + D * ngI * 4)
    sh_gu = 2 * Is * D * 2 if cfg.shared_mode else 0
    sh_dn = D * Is * 2 if cfg.shared_mode else 0
    route = cfg.router_bytes() + S * D * 4 + 2 * S * E * 4 + S * limb(D)
    if S == 1:        # the shared expert rides in stages 1 and 2
        b = {"stage_route": route + sh_gu + S * Is * 4,
             "stage_experts": gu_w + S * limb(D) + T * limb(I) + sh_dn + S * Is * 4 + S * D * 4,
             "q4_down_combine": dn_w + T * limb(I) + T * 8 + 2 * D * 4 + (D * 4 if cfg.shared_mode else 0)}
    else:             # its own kernels over token tiles
        b = {"stage_route": route, "router_tiles": cfg.router_bytes() + S * D * 4 + 2 * S * E * 4,
             "limbs": S * D * 4 + S * limb(D), "gate_topk": 2 * S * E * 4 + T * 8, "bucket": T * 4 * 3 + E * 12,
             "stage_experts": gu_w + S * limb(D) + T * limb(I),
             "q4_down": dn_w + T * limb(I) + T * D * 4,
             "combine": T * D * 4 + 2 * S * D * 4 + (S * D * 4 if cfg.shared_mode else 0) + T * 8}
        b["gate_bucket"] = b["gate_topk"] + b["bucket"]      # (one launch up to 8 tokens)
        # prefill-sized batches: the grouped GEMMs on the f16 MFMA over MFMA digits (128
        # bytes + one f32 factor per 32 inputs)
        dig = lambda n: n // 32 * (128 + 4)
        b["digits"] = S * D * 4 + S * dig(D)
        b["mf_glu"] = gu_w + S * dig(D) + T * dig(I)
        b["mf_down"] = dn_w + T * dig(I) + T * D * 4
        if cfg.shared_mode:
            b["shared_glu"] = sh_gu + S * D * 4 + S * Is * 6
            b["shared_down"] = sh_dn + S * Is * 6 + S * D * 4
            # decode-sized batches: the shared expert's blocks ride in other launches (h as
            # three bf16 parts, 6 bytes per value)
            if S <= 32:
                b["stage_experts"] += b["shared_glu"]
                b["shared_down_combine"] = b["combine"] + sh_dn + S * Is * 6
            elif S <= 128:
                b["stage_route"] += sh_gu + S * Is * 6
                b["stage_experts"] += b["shared_down"]
    return b


def kernel_flops(cfg, S):
    """algorithmic flops (2 per multiply-add of the layer's own arithmetic) per launch of
    the kernels that run on the MFMA"""
    D, I, Is, E, K = cfg.D, cfg.I, cfg.Is, cfg.E, cfg.K
    T = S * K
    f = {"mf_glu": 2 * T * 2 * I * D, "mf_down": 2 * T * D * I, "router_tiles": 2 * S * E * D}
    if cfg.shared_mode:
        f["shared_glu"] = 2 * S * 2 * Is * D
        f["shared_down"] = 2 * S * D * Is
    return f


def cpu_baseline(be, cfg, dl, xs, seconds):
    """The reference CPU moe_block (oracle/_ref, compiled from the reference
    sources: moe_block.h + matmul_i4_grouped + matmul_bf16_k) over the same
    layer, one token at a time, for about `seconds` of host time."""
    from oracle.oracle import Ref
    from oracle import synth as osyn
    isa = "avx512" if "avx512f" in open("/proc/cpuinfo").read() else "avx2"
    if not Ref.available(isa):
        return None
    ref = Ref(isa)
    ref.lib.ref_omp_autotune()                       # one OpenMP thread per physical core (c/moe_util.h:78-86)
    cores = ref.lib.ref_physical_cores()
    D, I, E, gs = cfg.D, cfg.I, cfg.E, cfg.gs
    ngD, ngI = D // gs, I // gs
    get = lambda b, shape, dt: be.d2h(b, shape, dt)
    # host copy of the layer (router back in natural order from its seed)
    from sabrewing_amd import synth as S
    from oracle.oracle import Oracle
    orc = Oracle()
    r = orc.normal(E * D, S.tensor_seed(dl.seed, dl.layer, S.T_ROUTER), 0.02).reshape(E, D)
    router = orc.to_bf16(r) if cfg.router_bf16 else r
    L = osyn.Layer(D, I, cfg.Is, E, gs, cfg.router_bf16, router,
                   np.zeros(E, np.float32) if cfg.use_corr_bias else None, None,
                   get(dl.gu_q, E * 2 * I * D // 2, np.uint8), get(dl.gu_s, E * 2 * I * ngD, np.float32),
                   get(dl.dn_q, E * D * I // 2, np.uint8), get(dl.dn_s, E * D * ngI, np.float32),
                   get(dl.sg, (cfg.Is, D), np.uint16) if cfg.shared_mode else None,
                   get(dl.su, (cfg.Is, D), np.uint16) if cfg.shared_mode else None,
                   get(dl.sd, (D, cfg.Is), np.uint16) if cfg.shared_mode else None)
    d = osyn.desc_of(cfg)
    if cfg.route_act == 2:                         # softplus is the descriptor extension: time the
        from dataclasses import replace            # reference block with its sigmoid gate (same work)
        d = osyn.desc_of(replace(cfg, route_act=0))
    out = np.zeros((1, D), np.float32)
    ref.moe_block_rows(d, L, xs[0:1], out)           # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and n < 1000000:
        ref.moe_block_rows(d, L, xs[n % len(xs):n % len(xs) + 1], out)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "tokens/s", "cores": int(cores), "kind": "reference",
            "sample": f"{n} single-token moe_block calls ({cfg.name}, B=1, gs={gs}) on one layer, "
                      f"{isa} build, {dt:.1f} s"}


def per_row_modes(be, cfg, dl, xs, seconds, steps):
    """Side figures for the per-row-scale (gs = 0) contracts: the reference CPU moe_block
    in its F32 and IDOT activation modes (c/moe_quant.h:45-125; LAG_IDOT), and the device
    layer at B = 1 in its default and IDOT modes, on one per-row-quantised copy of the
    workload's layer (generated on the device)."""
    from dataclasses import replace
    from oracle.oracle import Ref
    from oracle import synth as osyn
    isa = "avx512" if "avx512f" in open("/proc/cpuinfo").read() else "avx2"
    if not Ref.available(isa):
        return None
    from sabrewing_amd.backend import DeviceLayer
    c0 = replace(cfg, gs=0, name=cfg.name + "-gs0")
    seed0 = dl.seed + 7
    d0 = DeviceLayer.generate(be, c0, seed0)
    ref = Ref(isa)
    ref.lib.ref_omp_autotune()
    D, I, E = c0.D, c0.I, c0.E
    get = lambda b, shape, dt: be.d2h(b, shape, dt)
    from sabrewing_amd import synth as S
    from oracle.oracle import Oracle
    r = Oracle().normal(E * D, S.tensor_seed(seed0, 0, S.T_ROUTER), 0.02).reshape(E, D)
    L = osyn.Layer(D, I, c0.Is, E, 0, c0.router_bf16, Oracle().to_bf16(r) if c0.router_bf16 else r,
                   np.zeros(E, np.float32) if c0.use_corr_bias else None, None,
                   get(d0.gu_q, E * 2 * I * D // 2, np.uint8), get(d0.gu_s, E * 2 * I, np.float32),
                   get(d0.dn_q, E * D * I // 2, np.uint8), get(d0.dn_s, E * D, np.float32),
                   get(d0.sg, (c0.Is, D), np.uint16) if c0.shared_mode else None,
                   get(d0.su, (c0.Is, D), np.uint16) if c0.shared_mode else None,
                   get(d0.sd, (D, c0.Is), np.uint16) if c0.shared_mode else None)
    d = osyn.desc_of(replace(c0, route_act=0) if c0.route_act == 2 else c0)
    out = {}
    xb, ob = be.upload(xs[:1]), be.alloc(D * 4)
    for name, mode in (("device", be.Q4_DOT8), ("device_idot", be.Q4_IDOT)):
        prev = be.set_q4_mode(mode)
        try:
            for _ in range(10):
                be.moe_forward(d0.desc(), d0.weights(), xb, ob, 1)
            be.sync()
            e0, e1 = be.event(), be.event()
            be.record(e0)
            for _ in range(steps):
                be.moe_forward(d0.desc(), d0.weights(), xb, ob, 1)
            be.record(e1)
            be.sync()
            out[name] = round(steps / (be.elapsed_ms(e0, e1) * 1e-3), 1)
        finally:
            be.set_q4_mode(prev)
    # the CPU modes after the device ones (the OpenMP team pins the host thread)
    o = np.zeros((1, D), np.float32)
    for name, mode in (("cpu_f32", 0), ("cpu_idot", 1)):
        ref.moe_block_rows(d, L, xs[0:1], o, mode)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds and n < 100000:
            ref.moe_block_rows(d, L, xs[n % len(xs):n % len(xs) + 1], o, mode)
            n += 1
        out[name] = round(n / (time.perf_counter() - t0), 1)
    xb.free(); ob.free(); d0.free()
    out["unit"] = "tokens/s (B=1, eager)"
    out["sample"] = f"{c0.name}: per-row int4, {isa} reference with one thread per physical core, ~{seconds:.0f} s per CPU mode"
    return out


def stack_result(be, args, steps, warmup):
    """The Config-5 decode step -- 48 resident MoE layers (D=4096, E=256, top-8
    softmax, I=1536, no shared expert), h += MoE(rmsnorm(h)) each, then rmsnorm,
    the bf16 4096x32000 head and the greedy pick, for a batch of C5_BATCH streams:
    W eager warmup steps, K timed steps (eager, then recorded as one graph and
    replayed), per-kernel launch times; the stack is freed before returning."""
    from sabrewing_amd import configs as cf
    from sabrewing_amd.backend import gen_x
    from sabrewing_amd.stack import DeviceStack
    cfg, L, V = cf.C5_LAYER, args.layers_stack, cf.C5_VOCAB
    B = args.batch if args.config == "C5-stack" and args.batch else cf.C5_BATCH
    t0 = time.time()
    st = DeviceStack.generate(be, cfg, L, V, args.seed)
    log(f"generated the {L}-layer stack ({L * cfg.expert_bytes() * cfg.E / 1e9:.1f} GB of experts) in {time.time() - t0:.1f}s")
    D = cfg.D
    nx = warmup + steps
    xs = gen_x(be, cfg, args.seed, B * nx)
    h, xn, lg, tok = be.alloc(B * D * 4), be.alloc(B * D * 4), be.alloc(B * V * 4), be.alloc(B * 4)
    try:
        def step(i):
            be.check(be.lib.lag_hip_d2d(int(h), int(xs) + i * B * D * 4, B * D * 4), "d2d")
            st.step(h, xn, lg, tok, B)

        for i in range(warmup):
            step(i)
        be.sync()
        ev0, ev1 = be.event(), be.event()
        be.record(ev0)
        for i in range(steps):
            step(warmup + i)
        be.record(ev1)
        be.sync()
        ms_eager = be.elapsed_ms(ev0, ev1) / steps
        ms = ms_eager
        if not args.eager:
            # the same K steps recorded once and replayed with one submission (as the B=1
            # line): the device time of the steps without the host's per-launch cost
            be.graph_begin()
            for i in range(steps):
                step(warmup + i)
            g = be.graph_end()
            be.graph_launch(g)
            be.sync()
            be.record(ev0)
            be.graph_launch(g)
            be.record(ev1)
            be.sync()
            be.graph_destroy(g)
            ms = be.elapsed_ms(ev0, ev1) / steps
        log(f"C5 stack B={B}: {ms * 1e3:.0f} us/step ({'eager' if args.eager else 'graph replay'}; eager {ms_eager * 1e3:.0f})")
        be.profile_reset(); be.profile(True)
        step(0); be.sync()
        prof = be.profile_read(); be.profile(False)
        kern = {k: {"avg_us": round(1e3 * v[0] / max(v[1], 1), 2), "launches": v[1]} for k, v in prof.items()}
        # algorithmic bytes of a step: each layer's distinct experts (counted on the
        # profiled step), its router, the head, the activations
        head = V * D * 2
        G_mean = cfg.E * (1.0 - (1.0 - 1.0 / cfg.E) ** (B * cfg.K))         # expected distinct experts per layer
        step_bytes = L * (G_mean * cfg.expert_bytes() + cfg.router_bytes() + 4 * B * D * 4) + head
        gbs = step_bytes / (ms * 1e-3) / 1e9
        return {"workload": "C5-stack", "batch": B, "layers": L, "hidden": D, "experts": cfg.E, "topk": cfg.K,
                "moe_inter": cfg.I, "vocab": V, "ms_per_step": round(ms, 4), "eager_ms_per_step": round(ms_eager, 4),
                "tokens_per_s": round(B / (ms * 1e-3), 1), "steps": steps, "warmup": warmup,
                "submission": "eager" if args.eager else "graph replay of the timed steps",
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": int(step_bytes),
                             "bytes_note": "48 x (expected distinct experts E(1-(1-1/E)^(B K)) x expert bytes + router) "
                                           "+ the bf16 head + activations"},
                "kernels": kern}
    finally:
        for b_ in (h, xn, lg, tok, xs):
            b_.free()
        st.free()


def run_stack(args):
    """--config C5-stack: the stack step alone, as its own JSON line."""
    from sabrewing_amd.backend import Backend
    be = Backend(0)
    be.set_grouped_kernel({"auto": 0, "dot8": 1, "mfma": 2}[args.grouped])
    r = stack_result(be, args, args.steps, args.warmup)
    res = {"metric": "Config-5 stack decode tokens/s (48 int4 MoE layers + RMSNorm + bf16 head + greedy pick)",
           "value": r["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": DTYPE, "submission": r["submission"],
           "eager_ms_per_step": r["eager_ms_per_step"],
           "data": "synthetic: seeded N(0,0.02) weights generated on device, N(0,1) bf16-valued tokens",
           "config": {k: r[k] for k in ("workload", "batch", "layers", "hidden", "experts", "topk", "moe_inter", "vocab")},
           "roofline": r["roofline"], "kernels": r["kernels"]}
    print(json.dumps(res), flush=True)


def run_coli(args):
    """--config GLM-coli: the GLM engine's coli_cuda_expert_group on GLM-4.5-shaped experts
    (D=5120, I=1536, per-row int4, separate gate/up/down tensors), a side figure: decode
    (8 experts x 1 row) and prefill (8 experts x 256 rows).  Four sets of 8 experts (378 MB)
    rotate so the Infinity Cache cannot serve a call's weights.  Device time is the
    reference's own COLI_CUDA_PROFILE accounting (events around the launches,
    c/backend_cuda.cu:822-940); the host figure includes the PCIe copies and the sync."""
    import ctypes as C
    os.environ["COLI_CUDA_PROFILE"] = "1"
    from sabrewing_amd.coli import Coli
    D, I, NE, NSET = 5120, 1536, 8, 4
    c = Coli([0])
    rng = np.random.default_rng(args.seed)
    sets = []
    for _ in range(NSET):
        ts = []
        for _ in range(NE):
            g = rng.integers(0, 256, (I, D // 2), dtype=np.uint8)
            u = rng.integers(0, 256, (I, D // 2), dtype=np.uint8)
            d = rng.integers(0, 256, (D, I // 2), dtype=np.uint8)
            ts.append((c.upload(g, np.full(I, 2e-3, np.float32), D, I), c.upload(u, np.full(I, 2e-3, np.float32), D, I),
                       c.upload(d, np.full(D, 2e-3, np.float32), I, D)))
        sets.append(([t[0] for t in ts], [t[1] for t in ts], [t[2] for t in ts]))
    wbytes = NE * (3 * I * D // 2 + (2 * I + D) * 4)

    def stats():
        v = (C.c_uint64 * 3)(); f = (C.c_double * 3)()
        c.f.group_stats(C.addressof(v), C.addressof(v) + 8, C.addressof(v) + 16, C.addressof(f), C.addressof(f) + 8,
                        C.addressof(f) + 16)
        return v[0], f[1]

    res = {}
    for name, rows, n in (("decode", 1, max(args.steps, 40)), ("prefill", 256, max(args.steps // 10, 8))):
        x = rng.standard_normal((NE * rows, D)).astype(np.float32)
        for i in range(4):
            c.expert_group(*sets[i % NSET], [rows] * NE, x)
        c0, k0 = stats()
        t0 = time.perf_counter()
        for i in range(n):
            c.expert_group(*sets[i % NSET], [rows] * NE, x)
        dt = (time.perf_counter() - t0) / n
        c1, k1 = stats()
        kern_us = 1e3 * (k1 - k0) / max(c1 - c0, 1)
        res[name] = {"experts": NE, "rows_per_expert": rows, "calls": n, "host_us_per_call": round(dt * 1e6, 1),
                     "device_us_per_call": round(kern_us, 1), "weight_bytes": wbytes,
                     "weight_GBs_device": round(wbytes / (kern_us * 1e-6) / 1e9, 1),
                     "expert_rows_per_s_host": round(NE * rows / dt, 1),
                     "tera_ops_device": round(2 * 3 * I * D * NE * rows / (kern_us * 1e-6) / 1e12, 2),
                     "kernel": "f16 MFMA" if rows >= 8 else "dot8 grouped"}
        log(f"GLM-coli {name}: {dt * 1e6:.1f} us/call host, {kern_us:.1f} us device "
            f"({wbytes / (kern_us * 1e-6) / 1e9:.0f} GB/s of expert weights)")
    print(json.dumps({"metric": "coli_cuda_expert_group (GLM-4.5-shaped experts) side figure", "unit": "us/call",
                      "n_gpus": 1, "higher_is_better": False, "dtype": "int4 per-row weights x f32 activations",
                      "data": "synthetic: uniform random int4 bytes, N(0,1) rows",
                      "config": {"workload": "GLM-coli", "hidden": D, "moe_inter": I, "sets_rotated": NSET}, **res}),
          flush=True)
    for st in sets:
        for ts in st:
            for t in ts:
                t.free()
    c.close()


def host_facts():
    """the CPU baseline's host: model, sockets, NUMA nodes, CPUs, glibc (read before
    any OpenMP team binds the process's threads)"""
    import glob
    info = open("/proc/cpuinfo").read().splitlines()
    model = next((l.split(":", 1)[1].strip() for l in info if l.startswith("model name")), "unknown")
    sockets = len({l.split(":", 1)[1].strip() for l in info if l.startswith("physical id")}) or 1
    try:
        glibc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        glibc = None
    return {"cpu_model": model, "sockets": sockets,
            "numa_nodes": len(glob.glob("/sys/devices/system/node/node[0-9]*")) or 1,
            "logical_cpus": os.cpu_count(), "cpus_allowed": len(os.sched_getaffinity(0)), "glibc": glibc,
            "omp": {k: os.environ.get(k) for k in ("OMP_PROC_BIND", "OMP_PLACES")}}


def measure(be, cfg, layers, B, args, seed, profile=True):
    """One batch size: W eager warmup steps, K timed steps (eager, then the same
    steps recorded as one graph and replayed), then the distinct experts per step
    and, with profile, each kernel's average launch time from HIP events."""
    from sabrewing_amd.backend import desc_of, gen_x
    nx = args.warmup + args.steps
    xbuf = gen_x(be, cfg, seed, B * nx)
    outs = [be.alloc(B * cfg.D * 4) for _ in layers]
    for o in outs:
        be.lib.lag_hip_memset(int(o), 0, B * cfg.D * 4)
    desc = desc_of(cfg)
    wts = [dl.weights() for dl in layers]
    xptr = lambda i: int(xbuf) + i * B * cfg.D * 4

    def step(i):
        l = i % len(layers)
        be.moe_forward(desc, wts[l], xptr(i), outs[l], B)

    r = {"B": B}
    try:
        for i in range(args.warmup):
            step(i)
        be.sync()
        ev0, ev1 = be.event(), be.event()
        be.record(ev0)
        h0 = time.perf_counter()
        for i in range(args.steps):
            step(args.warmup + i)
        r["host_us"] = (time.perf_counter() - h0) * 1e6 / args.steps
        be.record(ev1)
        be.sync()
        r["ms_eager"] = be.elapsed_ms(ev0, ev1) / args.steps
        log(f"{cfg.name} B={B} eager: {r['ms_eager'] * 1e3:.1f} us/step, {B / (r['ms_eager'] * 1e-3):.0f} tokens/s "
            f"(host enqueue {r['host_us']:.1f} us/step)")
        r["ms"] = r["ms_eager"]
        if not args.eager:
            # the same K steps recorded once and replayed with one submission: the
            # device time of the steps without the host's per-launch cost
            be.graph_begin()
            for i in range(args.steps):
                step(args.warmup + i)
            g = be.graph_end()
            be.graph_launch(g)
            be.sync()
            be.record(ev0)
            be.graph_launch(g)
            be.record(ev1)
            be.sync()
            be.graph_destroy(g)
            r["ms"] = be.elapsed_ms(ev0, ev1) / args.steps
        r["tok_s"] = B / (r["ms"] * 1e-3)
        log(f"{cfg.name} B={B}: {r['ms'] * 1e3:.1f} us/step, {r['tok_s']:.0f} tokens/s "
            f"({'eager' if args.eager else 'graph replay'})")
        if not profile:
            return r
        # distinct experts per step (the bytes a step must read)
        G_sum, nG = 0, min(args.steps, 20)
        for i in range(nG):
            step(args.warmup + i)
            if B > 1:
                G_sum += be.last_groups()[0]
        G = G_sum / nG if B > 1 and G_sum > 0 else cfg.K
        # per-kernel times: the same steps again, each launch bracketed by HIP events
        # on the backend stream
        be.profile_reset()
        be.profile(True)
        for i in range(args.steps):
            step(args.warmup + i)
        be.sync()
        prof = be.profile_read()
        be.profile(False)
        kb = kernel_bytes(cfg, B, G)
        kf = kernel_flops(cfg, B) if B > 1 else {}
        kern = {k: {"avg_us": 1e3 * v[0] / max(v[1], 1), "launches": v[1]} for k, v in prof.items()}
        for k, v in kern.items():
            if k in kb:
                v["bytes"] = kb[k]
                v["GBs"] = kb[k] / (v["avg_us"] * 1e-6) / 1e9 if v["avg_us"] > 0 else 0.0
            if k in kf:
                v["flops"] = kf[k]
                v["TFs"] = kf[k] / (v["avg_us"] * 1e-6) / 1e12 if v["avg_us"] > 0 else 0.0
        dom = max(kern, key=lambda k: kern[k]["avg_us"] * kern[k]["launches"])
        dk = kern[dom]
        # HBM bytes per launch of that kernel as rocprofv3 counted them (FETCH_SIZE x2 + WRITE_SIZE,
        # calibrated on a device copy; profiles/decode_kernels_*.md), when a profile covers this workload
        traffic = None
        try:
            with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
                traffic = json.load(f).get(cfg.name, {}).get(str(B), {}).get(dom, {}).get("traffic_bytes")
        except (OSError, ValueError):
            pass
        r["G"] = G
        r["layer_bytes"] = cfg.step_bytes(B, G)
        r["layer_gbs"] = r["layer_bytes"] / (r["ms"] * 1e-3) / 1e9
        if dom.startswith("mf_"):
            # the prefill's grouped GEMMs on the MFMA: useful flops over the launch time
            r["roofline"] = {"bound": "mfma", "kernel": dom, "achieved": round(dk["TFs"], 1), "peak": MFMA_PEAK_TFS,
                             "unit": "TFLOP/s", "frac": round(dk["TFs"] / MFMA_PEAK_TFS, 4), "traffic": traffic,
                             "flops_per_launch": dk["flops"], "bytes_per_launch": dk.get("bytes"),
                             "hbm_GBs": round(dk.get("GBs", 0.0), 1), "avg_launch_us": round(dk["avg_us"], 2)}
        else:
            r["roofline"] = {"bound": "hbm", "kernel": dom, "achieved": round(dk.get("GBs", 0.0), 1),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dk.get("GBs", 0.0) / HBM_PEAK_GBS, 4),
                             "traffic": traffic, "bytes_per_launch": dk.get("bytes"), "avg_launch_us": round(dk["avg_us"], 2)}
        # the layer's own floor: its flops at the MFMA peak or its bytes at the HBM peak
        r["layer_flops"] = cfg.flops(B)
        r["floor_us"] = max(cfg.flops(B) / (MFMA_PEAK_TFS * 1e12), r["layer_bytes"] / (HBM_PEAK_GBS * 1e9)) * 1e6
        r["kernels"] = {k: {kk: (round(vv, 2) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                        for k, v in kern.items()}
        log(f"B={B} kernels:", json.dumps(r["kernels"]))
        if B == args.batch:
            # the host-buffer boundary (lag_hip_moe_block: x and out in host memory, copied
            # over PCIe each call, synchronous): a side figure, never `value`
            hx = be.d2h(xbuf, (B, cfg.D), np.float32)
            hout = np.zeros((B, cfg.D), np.float32)
            for i in range(5):
                be.moe_block(desc, wts[i % len(wts)], hx, hout)
            nh = max(20, min(args.steps, 200))
            h0 = time.perf_counter()
            for i in range(nh):
                be.moe_block(desc, wts[i % len(wts)], hx, hout)
            r["pcie_ms"] = (time.perf_counter() - h0) * 1e3 / nh
            log(f"host-buffer entry (PCIe-inclusive, synchronous): {r['pcie_ms'] * 1e3:.1f} us/step, "
                f"{B / (r['pcie_ms'] * 1e-3):.0f} tokens/s")
        return r
    finally:
        for o in outs:
            o.free()
        xbuf.free()


def extra_objects(be, args):
    """C1 at batch 1, C4's 2048-token prefill (softplus and Zipf(1.1) routers) and the
    C5 48-layer stack at batch 8, measured in the same run as the headline line (the
    same timing: eager warmup, then the timed steps as one graph replay)."""
    from argparse import Namespace
    from sabrewing_amd import configs as cf
    from sabrewing_amd.backend import DeviceLayer
    out = {}

    def layers_of(cfg, n, seed):
        ls = []
        for l in range(n):
            dl = DeviceLayer.generate(be, cfg, seed, layer=l)
            dl.seed, dl.layer = seed, l
            ls.append(dl)
        return ls

    # C1: the OLMoE-shaped layer, one token per step, 12 layers rotated (each step reads
    # 8 of a layer's 64 experts; 12 layers hold 3 GB)
    ls = layers_of(cf.C1, args.layers, args.seed + 11)
    try:
        r = measure(be, cf.C1, ls, 1, args, args.seed + 13)
        out["c1_b1"] = {"workload": cf.C1.name, "hidden": cf.C1.D, "experts": cf.C1.E, "topk": cf.C1.K,
                        "moe_inter": cf.C1.I, "gs": cf.C1.gs, "router": "f32", **batch_summary(cf.C1, r),
                        "kernels": r["kernels"]}
    finally:
        for dl in ls:
            dl.free()
    # C4: 2048 tokens in one chunk; every step reads all 256 experts (2 GB), two layers rotated
    pa = Namespace(**{**vars(args), "steps": min(args.steps, 20), "warmup": min(args.warmup, 5)})
    pre = {}
    for cfg in (cf.C2, cf.C4_ZIPF):
        ls = layers_of(cfg, 2, args.seed + 17)
        try:
            r = measure(be, cfg, ls, 2048, pa, args.seed + 19)
            pre[cfg.name] = {"workload": cfg.name, "tokens": 2048, "zipf": cfg.zipf, **batch_summary(cfg, r),
                             "layer_flops": r["layer_flops"], "floor_us": round(r["floor_us"], 1),
                             "layer_roofline_frac": round(r["floor_us"] * 1e-3 / r["ms"], 4), "kernels": r["kernels"]}
        finally:
            for dl in ls:
                dl.free()
    out["prefill"] = {"steps": pa.steps, "warmup": pa.warmup,
                      "note": "layer_roofline_frac = max(layer flops at the 2.5 PF/s bf16 MFMA peak, layer bytes at "
                              "8 TB/s) / measured step time; roofline = the dominant kernel",
                      **pre}
    # C5: the 48-layer stack (145 GB of experts), batch 8
    out["stack"] = stack_result(be, args, min(args.steps, 20), min(args.warmup, 5))
    return out


def batch_summary(cfg, r):
    return {"batch": r["B"], "ms_per_step": round(r["ms"], 5), "tokens_per_s": round(r["tok_s"], 1),
            "distinct_experts_per_step": round(r["G"], 2), "layer_bytes_per_step": int(r["layer_bytes"]),
            "layer_hbm_GBs": round(r["layer_gbs"], 1), "layer_hbm_frac": round(r["layer_gbs"] / HBM_PEAK_GBS, 4),
            "roofline": r["roofline"]}


def run(args):
    from sabrewing_amd import configs as cf
    from sabrewing_amd.backend import Backend, DeviceLayer, gen_x

    cfg = cf.CONFIGS[args.config]
    B = args.batch
    facts = host_facts()
    be = Backend(0)
    be.set_grouped_kernel({"auto": 0, "dot8": 1, "mfma": 2}[args.grouped])
    t0 = time.time()
    layers = []
    for l in range(args.layers):
        dl = DeviceLayer.generate(be, cfg, args.seed, layer=l)
        dl.seed, dl.layer = args.seed, l
        layers.append(dl)
    log(f"generated {args.layers} x {cfg.name} layers in {time.time() - t0:.1f}s")

    if args.calib_copy_mb:
        # a plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters
        n = args.calib_copy_mb << 20
        a_, b_ = be.alloc(n), be.alloc(n)
        be.lib.lag_hip_memset(int(a_), 1, n)
        be.lib.lag_hip_d2d(int(b_), int(a_), n)
        be.sync()
        a_.free(); b_.free()
        log(f"calibration copy: {args.calib_copy_mb} MiB device-to-device")

    main_r = measure(be, cfg, layers, B, args, args.seed, profile=not args.timed_only)
    if args.timed_only:
        return
    # the batched-decode sweep of the same layer: B = 8, 32, 64
    sweep = {}
    if not args.no_sweep and B == 1:
        for b in (8, 32, 64):
            sweep[b] = measure(be, cfg, layers, b, args, args.seed + 101 * b)

    # the other BASELINE configurations, each on device layers of its own (freed before
    # the next; the first C2 layer stays for the CPU baseline below)
    extra = {}
    if not args.no_extra and B == 1 and cfg.name == "C2-laguna-softplus":
        for dl in layers[1:]:
            dl.free()
        layers = layers[:1]
        extra = extra_objects(be, args)

    # the CPU side last: the OpenMP team it starts pins the host thread (OMP_PROC_BIND)
    cpu = None
    modes = None
    if not args.no_cpu:
        rng_x = gen_x(be, cfg, args.seed + 1, 64)
        xs = be.d2h(rng_x, (64, cfg.D), np.float32)
        rng_x.free()
        if B == 1 and cfg.gs > 0:
            try:
                modes = per_row_modes(be, cfg, layers[0], xs, args.cpu_seconds / 3, args.steps)
                log("per-row (gs=0) contracts:", json.dumps(modes))
            except Exception as e:
                log("per-row modes failed:", repr(e))
        try:
            cpu = cpu_baseline(be, cfg, layers[0], xs, args.cpu_seconds)
            if cpu:
                cpu["host"] = facts
        except Exception as e:                      # the baseline is reported, never required
            log("cpu baseline failed:", repr(e))

    r = main_r
    res = {
        "metric": "MoE-layer tokens/s + % peak HBM GB/s, int4 experts, batch 1 and batch 32",
        "value": round(r["tok_s"], 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "submission": "eager" if args.eager else "graph replay of the timed steps",
        "eager_value": round(B / (r["ms_eager"] * 1e-3), 1), "eager_host_enqueue_us": round(r["host_us"], 1),
        "host_buffer_value": round(B / (r["pcie_ms"] * 1e-3), 1) if "pcie_ms" in r else None,
        "dtype": DTYPE,
        "data": "synthetic: seeded N(0,0.02) int4 weights generated on device, N(0,1) bf16-valued tokens",
        "config": {"workload": cfg.name, "batch": B, "hidden": cfg.D, "experts": cfg.E, "topk": cfg.K,
                   "moe_inter": cfg.I, "shared_inter": cfg.Is, "gs": cfg.gs,
                   "gate": ["sigmoid", "softmax", "softplus", "softmax-olmoe", "softmax-qwen", "sqrt-softplus"][cfg.route_act],
                   "layers_rotated": args.layers, "distinct_experts_per_step": round(r["G"], 2),
                   "layer_bytes_per_step": int(r["layer_bytes"]), "layer_hbm_GBs": round(r["layer_gbs"], 1),
                   "layer_hbm_frac": round(r["layer_gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "per_row_modes": modes,
        "kernels": r["kernels"],
    }
    if 32 in sweep:
        b32 = sweep[32]
        per_tok1 = r["layer_bytes"] / B
        per_tok32 = b32["layer_bytes"] / 32
        res["batch32"] = {**batch_summary(cfg, b32), "kernels": b32["kernels"],
                          "tokens_per_s_vs_batch1": round(b32["tok_s"] / r["tok_s"], 3),
                          # bytes per token fall only this much with G distinct experts, so
                          # this is the ratio at equal HBM efficiency; F7's ceiling puts B=1
                          # at 70 % and B=32 at 100 % of peak
                          "ratio_at_equal_hbm_frac": round(per_tok1 / per_tok32, 3),
                          "ratio_ceiling_b1_70pct_b32_100pct": round(per_tok1 / per_tok32 / 0.7, 3),
                          "target_ratio": 8.0}
    if sweep:
        res["batch_sweep"] = {str(b): batch_summary(cfg, v) for b, v in sweep.items()}
    res.update(extra)
    print(json.dumps(res), flush=True)
    for dl in layers:
        dl.free()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=None, help="tokens per step (default 1; C5-stack: 8)")
    ap.add_argument("--layers-stack", type=int, default=48, help="C5-stack: resident MoE layers")
    ap.add_argument("--config", default="C2-laguna-softplus")
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--grouped", choices=["auto", "dot8", "mfma"], default="auto",
                    help="grouped expert GEMMs of batches: auto (f16 MFMA at >= 8 tokens per group), dot8, mfma")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="one device-to-device copy of this many MiB before the timed steps (counter calibration)")
    ap.add_argument("--eager", action="store_true",
                    help="time the per-call submission only (default: also record the steps as one graph and time its replay)")
    ap.add_argument("--no-sweep", action="store_true", help="B=1 only (no batch 8/32/64 objects)")
    ap.add_argument("--no-extra", action="store_true",
                    help="no C1 / C4 prefill / C5 stack objects in the headline line")
    ap.add_argument("--timed-only", action="store_true",
                    help="stop after the timed steps (no per-kernel pass, no CPU baseline, no JSON line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the MoE block on one MI355X); "
              "--gpus N > 1 is not supported", file=sys.stderr)
        sys.exit(2)
    if args.config == "C5-stack":
        run_stack(args)
        return
    if args.config == "GLM-coli":
        run_coli(args)
        return
    args.batch = args.batch or 1
    run(args)


if __name__ == "__main__":
    main()
