"""GPU parity of BASELINE config 1 as one chain, from token ids to the sampled latent:
text token ids U[0, 1000) and 32 reference latent frames through the GPU text and speaker
encoders (text_encoder.rs:17-148, speaker_encoder.rs:85-162), the device context-KV build of
the conditioned row and the unconditioned bundle (attention.rs:431-501, condition.rs:144-154)
and 4 Joint-CFG Euler steps (euler_sampler.rs:167-252), against the oracle's chain on the
same seeded inputs (encoder_forward -> build_kv_cache -> sample_joint_cfg).

Bars: f32 1e-4 and bf16 2e-2 relative L2 on the sampled latent (test_gpu_model.py's), with
the encoded states also checked on the way (1e-4 / 2e-2, test_gpu_encoder.py's).
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL_STATE = {F32: 1e-4, BF16: 2e-2}
TOL_FINAL = {F32: 1e-4, BF16: 2e-2}


def encode(ecfg, ew, backend, mask, **inp):
    B, S = mask.shape
    with ih.HipEncoder(ecfg, backend, max_rows=B, max_seq=S) as enc:
        enc.load_weights(ew)
        return enc.forward(mask, **inp)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_config1_chain_from_token_ids(oracle64, backend):
    cfg = ih.cfg_cpu_plumbing()  # 4 layers, d 256, 4 x 64 heads, SwiGLU 704, latent 32
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()  # vocab 1000; 32-channel latents
    assert te.vocab_size == 1000 and se.in_dim == cfg.latent_dim
    w = ih.DitWeights.random(cfg, 0)
    tw, sw = ih.EncoderWeights.random(te, 1, std=0.05), ih.EncoderWeights.random(se, 2, std=0.05)
    proj = ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3, std=0.05)
    rng = np.random.default_rng(4)
    Tt, Tr, S = 16, 32, 64
    ids = rng.integers(0, 1000, (1, Tt)).astype(np.int32)
    tmask = np.ones((1, Tt), np.uint8)
    ref_lat = rng.standard_normal((1, Tr, cfg.latent_dim)).astype(np.float32)
    rmask = np.ones((1, Tr), np.uint8)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 5)

    # GPU chain
    ts, tmo = encode(te, tw, backend, tmask, ids=ids)
    ss, smo = encode(se, sw, backend, rmask, latent=ref_lat)
    T = ts.shape[1] + ss.shape[1]
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=3.0, scale_speaker=3.0, min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=4, guidance=g)
    with ih.HipInferenceEngine(cfg, backend, max_rows=2, max_seq=S, max_ctx=T) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        e.build_context_kv(0, ts[0], tmo[0], ss[0], smo[0])
        e.build_context_kv(1, np.zeros_like(ts[0]), np.zeros_like(tmo[0]), np.zeros_like(ss[0]),
                           np.zeros_like(smo[0]))
        got = e.sample(x0, p)

    # Oracle chain
    ts_ref, tmo_ref = oracle64.encoder_forward(te, tw, tmask, ids=ids)
    ss_ref, smo_ref = oracle64.encoder_forward(se, sw, rmask, latent=ref_lat)
    assert np.array_equal(tmo, tmo_ref) and np.array_equal(smo, smo_ref)
    e_t, e_s = rel_l2(ts, ts_ref), rel_l2(ss, ss_ref)
    ks, vs = {0: [], 1: []}, {0: [], 1: []}
    masks = {}
    for row, (tst, tm, sst, sm) in enumerate([(ts_ref, tmo, ss_ref, smo),
                                              (np.zeros_like(ts_ref), np.zeros_like(tmo),
                                               np.zeros_like(ss_ref), np.zeros_like(smo))]):
        for l in range(cfg.num_layers):
            lw = proj.layers[l]
            ck, cv, cm = oracle64.build_kv_cache(cfg, w.blocks[l]["k_norm"], tst, tm, lw["wk_text"], lw["wv_text"],
                                                 sst, sm, lw["wk_aux"], lw["wv_aux"])
            ks[row].append(ck)
            vs[row].append(cv)
            masks[row] = cm
    cond = (np.stack(ks[0]), np.stack(vs[0]), masks[0])
    unc = (np.stack(ks[1]), np.stack(vs[1]), masks[1])
    ref, _ = oracle64.sample_joint_cfg(cfg, w, x0, cond, unc, 4, 3.0)
    err = rel_l2(got, ref)
    print(backend.value, "config-1 chain: text state %.2e, speaker state %.2e, sampled latent %.2e"
          % (e_t, e_s, err))
    assert e_t < TOL_STATE[backend] and e_s < TOL_STATE[backend]
    assert err < TOL_FINAL[backend]
