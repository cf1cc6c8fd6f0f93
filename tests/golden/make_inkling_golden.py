"""Golden vectors of the Inkling engine's MoE layer, made by the compiled engine.

    python tests/golden/make_inkling_golden.py    # needs oracle/_ref (built from /root/reference)

Writes inkling_moe.npz: a seeded small Inkling-shaped layer (f32 router over
E routed + 2 shared gate rows, correction bias, per-row int4 experts, two bf16
gated shared experts; oracle/synth.py regenerates it from the stored seed) and
the engine's own moe() (c/inkling.c:1011-1185, compiled in
oracle/_ref/libref_inkling_avx512.so) over rows of tokens, once with its
default int8 activation route (IDOT) and once with IDOT=0 (the f32 route),
each in a process of its own since the engine reads IDOT once.

Only the compiled engine computes what is stored; the restatement under oracle/
is used for nothing but regenerating the seeded weights.
"""
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import synth                      # noqa: E402
from oracle.oracle import Oracle, RefInkling  # noqa: E402
from sabrewing_amd import configs as cf       # noqa: E402

SEED, ROWS, CORR, GSCALE = 111, 5, 0.01, 1.25


def config():
    return cf.scaled(cf.INKLING, D=512, E=32, K=6, I=256, Is=256, name="inkling-small")


def layer_and_x(orc):
    cfg = config()
    return cfg, synth.make_layer(orc, cfg, SEED, corr_bias_sigma=CORR), synth.make_x(orc, cfg, SEED, ROWS)


def engine_out():
    orc = Oracle()
    cfg, L, x = layer_and_x(orc)
    return RefInkling().moe(cfg.E, cfg.K, cfg.n_shared, cfg.route_scale, GSCALE, L, x)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--child":
        np.save(sys.argv[2], engine_out())
        return
    if not RefInkling.available():
        raise SystemExit("oracle/_ref is not built (make -C oracle ref, with /root/reference present)")
    outs = {}
    for name, idot in (("out_idot", None), ("out_f32", "0")):
        env = dict(os.environ)
        env.pop("IDOT", None)
        if idot is not None:
            env["IDOT"] = idot
        tmp = os.path.join(HERE, f".{name}.npy")
        subprocess.run([sys.executable, __file__, "--child", tmp], env=env, check=True)
        outs[name] = np.load(tmp)
        os.remove(tmp)
    orc = Oracle()
    cfg, L, x = layer_and_x(orc)
    np.savez(os.path.join(HERE, "inkling_moe.npz"), seed=np.int64(SEED), rows=np.int64(ROWS),
             corr_bias_sigma=np.float64(CORR), gscale=np.float32(GSCALE), x=x, **outs)
    print("inkling_moe:", {k: v.shape for k, v in outs.items()})


if __name__ == "__main__":
    main()
