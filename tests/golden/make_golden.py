"""Writes the golden fixture of the full-size RF run (the benchmark configuration) with the CPU
oracle (f32 arithmetic, the NdArray<f32> analogue): 40 Joint-CFG Euler steps (scale 3,
min_t 0, max_t 1) of the 12-layer d=1024 DiT on seeded synthetic inputs.

Inputs are regenerated from their seeds by irodori_hip.synthetic (weights seed 0,
context seed 1, noise seed 2), so only the [1, 750, 32] output is stored.  Run from the
repository root:  python tests/golden/make_golden.py   (several minutes on 8 cores).
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "irodori-tts-burn_amd")]

import irodori_hip as ih  # noqa: E402
from oracle.oracle import Oracle, get_threads  # noqa: E402


def main():
    cfg = ih.cfg_full_rf()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 256, 375, seed=1)
    x0 = ih.make_noise(1, 750, cfg.latent_dim, 2)
    c, u = ctx.rows([0]), ctx.rows([1])
    t0 = time.time()
    out, run = Oracle("f32").sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask),
                                              40, 3.0, 0.0, 1.0)
    dt = time.time() - t0
    here = os.path.dirname(os.path.abspath(__file__))
    np.save(os.path.join(here, "cfg4_joint40_final_latent.npy"), out)
    meta = {"config": "BASELINE config 4", "oracle": "orc_f32 (C, float arithmetic)",
            "weights_seed": 0, "weight_std": 0.02, "context_seed": 1, "text": 256,
            "speaker": 375, "noise_seed": 2, "steps": run, "cfg_scale": 3.0, "min_t": 0.0,
            "max_t": 1.0, "norm_eps": cfg.norm_eps, "t_dim": cfg.timestep_embed_dim,
            "adaln_rank": cfg.adaln_rank, "seconds": round(dt, 1), "threads": get_threads(),
            "text_valid": int(ctx.mask[0, :256].sum())}
    with open(os.path.join(here, "cfg4_joint40_final_latent.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(json.dumps(meta))


if __name__ == "__main__":
    main()
