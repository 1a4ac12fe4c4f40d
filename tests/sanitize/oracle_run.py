"""Drives the CPU oracle's entry points on small inputs, for the AddressSanitizer / UBSan
build of the oracle (tests/sanitize/Makefile: _build/liboracle_asan.so, selected with
IRODORI_ORACLE_LIB and run with the ASan runtime preloaded; test_sanitize.py).  Imports
numpy, the irodori_hip Python package (configs and seeded synthetic weights; it does not
load the HIP library here) and the oracle only.  Prints "ok" when every call returned
finite values; a sanitizer report aborts the process first."""
import dataclasses
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (ROOT, os.path.join(ROOT, "irodori-tts-burn_amd")):
    sys.path.insert(0, p)

import irodori_hip as ih  # noqa: E402
from oracle.oracle import Oracle, mx_dequantize_rows, mx_quantize_rows, sampler_struct  # noqa: E402


def finite(*arrays):
    for a in arrays:
        assert np.all(np.isfinite(a)), "non-finite oracle output"


def main():
    rng = np.random.default_rng(0)
    for prec in ("f32", "f64"):
        orc = Oracle(prec)
        for cfg, S in ((ih.cfg_tiny(), 37),
                       (dataclasses.replace(ih.cfg_tiny(), model_dim=256, num_heads=2, mlp_hidden=512,
                                            latent_dim=200), 21)):
            w = ih.DitWeights.random(cfg, 0, std=0.05, norm_jitter=0.1)
            ctx = ih.make_context_kv(cfg, 1, 9, 7, seed=1)
            x = ih.make_noise(2, S, cfg.latent_dim, 2)
            t = np.array([0.9, 0.3], np.float32)
            lat = np.ones((2, S), np.uint8)
            lat[1, S - 5:] = 0
            v, dbg = orc.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True, latent_mask=lat)
            finite(v, dbg)
            c, u = ctx.rows([0]), ctx.rows([1])
            out, _ = orc.sample_joint_cfg(cfg, w, x[:1], (c.k, c.v, c.mask), (u.k, u.v, u.mask), 3, 3.0)
            finite(out)
        cfg = ih.cfg_tiny()
        w = ih.DitWeights.random(cfg, 1, std=0.05)
        for method in (0, 1, 2):
            for mode in (0, 1, 2):
                if mode == 2 and method == 2:
                    continue
                roles = 2 if mode == 1 else 3
                ctx = ih.make_context_kv(cfg, roles - 1, 6, 5, seed=3)
                ctx = ctx.rows(list(range(ctx.k.shape[1])) + [0] * (roles - ctx.k.shape[1]))
                sp = sampler_struct(num_steps=3, method=method, cfg_mode=mode, scale_text=2.0,
                                    scale_speaker=2.0 if mode == 1 else 3.0, has_speaker=1,
                                    # (Heun's last corrector meets t = 0, where the rescale is
                                    # NaN as in the reference: no rescale with Heun here.)
                                    has_temporal_rescale=int(method != 1), rescale_k=1.2, rescale_sigma=0.5,
                                    ctx_aux_start=6)
                out, _ = orc.sample_rf(cfg, w, ih.make_noise(1, 12, cfg.latent_dim, 4),
                                       (ctx.k, ctx.v, ctx.mask), sp)
                finite(out)
        for ecfg, inp in ((ih.enc_text_tiny(), "ids"), (ih.enc_speaker_tiny(), "latent")):
            ew = ih.EncoderWeights.random(ecfg, 2, std=0.05, norm_jitter=0.1)
            mask = np.ones((2, 11), np.uint8)
            mask[1, 7:] = 0
            kw = ({"ids": rng.integers(0, ecfg.vocab_size, (2, 11)).astype(np.int32)} if inp == "ids" else
                  {"latent": rng.standard_normal((2, 11, ecfg.in_dim)).astype(np.float32)})
            st, _ = orc.encoder_forward(ecfg, ew, mask, **kw)
            finite(st)
        cc = ih.codec_tiny()
        cw = ih.CodecWeights.random(cc, 1)
        wav = orc.codec_decode(cc, cw, rng.standard_normal((1, 5, cc.latent_dim)).astype(np.float32))
        finite(wav)
    f8 = Oracle("f32", gemm_fp8=True)
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 2, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 9, 7, seed=1)
    v = f8.forward(cfg, w, ih.make_noise(2, 16, cfg.latent_dim, 2), np.array([0.5, 0.5], np.float32),
                   ctx.k, ctx.v, ctx.mask)
    finite(v)
    xq = rng.standard_normal((5, 64)).astype(np.float32)
    q, sc = mx_quantize_rows(xq)
    finite(mx_dequantize_rows(q, sc))
    print("ok")


if __name__ == "__main__":
    main()
