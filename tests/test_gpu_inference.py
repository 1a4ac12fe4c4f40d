"""GPU parity of the request-level API (InferenceBuilder -> InferenceEngine.sample,
src/inference.rs:91-255; SamplingRequest, src/rf/params.rs:234-247): text tokens and a
reference latent (or caption tokens) through the GPU encoders, every CFG role's context
bundle built on the device and the RF loop, against the oracle's chain on the same inputs
(encoder_forward -> build_kv_cache per role bundle -> sample_rf).

Bars: f32 1e-4 and bf16 2e-2 relative L2 on the sampled latent (test_gpu_model.py's).
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2
from test_gpu_sampler import orc_params

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL = {F32: 1e-4, BF16: 2e-2}
M, SM = ih.CfgGuidanceMode, ih.SamplerMethod


def speaker_model():
    cfg = ih.cfg_cpu_plumbing()  # 4 layers, d 256, 4 x 64 heads, latent 32
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()
    mc = ih.ModelConfig(dit=cfg, text=te, aux=se)
    mw = ih.ModelWeights(dit=ih.DitWeights.random(cfg, 0), text=ih.EncoderWeights.random(te, 1, std=0.05),
                         ctx_proj=ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3, std=0.05),
                         aux=ih.EncoderWeights.random(se, 2, std=0.05))
    return mc, mw


def caption_model():
    cfg = ih.cfg_cpu_plumbing()
    te = ih.enc_text_tiny()
    ce = ih.EncoderConfig(dim=te.dim, num_layers=1, num_heads=te.num_heads, mlp_hidden=te.mlp_hidden,
                          vocab_size=500)
    mc = ih.ModelConfig(dit=cfg, text=te, aux=ce)
    mw = ih.ModelWeights(dit=ih.DitWeights.random(cfg, 0), text=ih.EncoderWeights.random(te, 1, std=0.05),
                         ctx_proj=ih.CtxProjWeights.random(cfg, te.dim, ce.dim, seed=3, std=0.05),
                         aux=ih.EncoderWeights.random(ce, 4, std=0.05))
    return mc, mw


def oracle_chain(oracle, mc, mw, req, p, has_speaker, has_caption):
    """The request on the oracle: encoders, the role bundles' K / V caches, sample_rf."""
    cfg = mc.dit
    ts, tm = oracle.encoder_forward(mc.text, mw.text, req.text_mask, ids=req.text_ids)
    aux = am = None
    if has_speaker:
        rm = req.ref_mask if req.ref_mask is not None else np.ones(req.ref_latent.shape[:2], np.uint8)
        aux, am = oracle.encoder_forward(mc.aux, mw.aux, rm, latent=req.ref_latent)
    elif has_caption:
        aux, am = oracle.encoder_forward(mc.aux, mw.aux, req.caption_mask, ids=req.caption_ids)
    roles = p.cfg_roles(has_speaker=has_speaker, has_caption=has_caption)
    ks, vs, ms = [], [], []
    for role in roles:
        keep_text, keep_aux = role in ("cond", "no_aux"), role in ("cond", "no_text")
        t_s, t_m = (ts, tm) if keep_text else (np.zeros_like(ts), np.zeros_like(tm))
        a_s, a_m = (aux, am) if keep_aux or aux is None else (np.zeros_like(aux), np.zeros_like(am))
        kl, vl = [], []
        for l in range(cfg.num_layers):
            lw = mw.ctx_proj.layers[l]
            ck, cv, cm = oracle.build_kv_cache(cfg, mw.dit.blocks[l]["k_norm"], t_s, t_m, lw["wk_text"], lw["wv_text"],
                                               a_s, a_m, lw.get("wk_aux"), lw.get("wv_aux"))
            kl.append(ck)
            vl.append(cv)
        ks.append(np.stack(kl))
        vs.append(np.stack(vl))
        ms.append(cm)
    ctx = (np.concatenate(ks, axis=1), np.concatenate(vs, axis=1), np.concatenate(ms, axis=0))
    op = orc_params(p, has_speaker=has_speaker, aux_start=req.text_ids.shape[1], has_caption=has_caption)
    ref, _ = oracle.sample_rf(cfg, mw.dit, req.initial_noise, ctx, op)
    return ref


def request(mc, B=1, Tt=16, Tr=32, S=64, seed=4, text_valid=None, caption=False):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, mc.text.vocab_size, (B, Tt)).astype(np.int32)
    tmask = np.ones((B, Tt), np.uint8)
    if text_valid is not None:
        for b, n in enumerate(text_valid):
            tmask[b, n:] = 0
    x0 = rng.standard_normal((B, S, mc.dit.latent_dim)).astype(np.float32)
    if caption:
        cids = rng.integers(0, mc.aux.vocab_size, (B, 12)).astype(np.int32)
        return ih.SamplingRequest(text_ids=ids, text_mask=tmask, sequence_length=S, caption_ids=cids,
                                  caption_mask=np.ones((B, 12), np.uint8), initial_noise=x0)
    lat = rng.standard_normal((B, Tr, mc.dit.latent_dim)).astype(np.float32)
    return ih.SamplingRequest(text_ids=ids, text_mask=tmask, sequence_length=S, ref_latent=lat,
                              ref_mask=np.ones((B, Tr), np.uint8), initial_noise=x0)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_joint_cfg_request_matches_oracle_chain(oracle64, backend):
    # Config 1 through the request API: 16 text tokens and 32 reference frames, Joint CFG,
    # 4 Euler steps.
    mc, mw = speaker_model()
    g = ih.GuidanceConfig(mode=M.JOINT, scale_text=3.0, scale_speaker=3.0, min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=4, guidance=g)
    req = request(mc)
    with ih.InferenceBuilder(0, backend).load_weights(mc, mw).with_sampling(p).build(max_seq=64, max_text=16,
                                                                                      max_aux=32) as eng:
        got = eng.sample(req)
    ref = oracle_chain(oracle64, mc, mw, req, p, True, False)
    print(backend.value, "joint request rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_default_sampling_two_utterances(oracle64, backend):
    # The reference's default sampler (Independent CFG, text 3 / speaker 5, CFG for t >= 0.5;
    # 6 of its 40 steps here) on two utterances with padded text: three role bundles each.
    mc, mw = speaker_model()
    b = ih.InferenceBuilder(0, backend).load_weights(mc, mw).with_default_sampling()
    assert b.model_config() is mc
    p = ih.SamplerParams(num_steps=6)
    req = request(mc, B=2, Tt=20, Tr=24, S=40, seed=7, text_valid=[20, 11])
    with b.with_sampling(p).build(max_batch=2, max_seq=64, max_text=32, max_aux=32) as eng:
        assert eng.sampling_params() is p
        got = eng.sample(req)
    ref = oracle_chain(oracle64, mc, mw, req, p, True, False)
    print(backend.value, "independent request rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL[backend]


def test_with_sampling_shares_the_model(oracle64):
    # with_sampling returns an engine over the same GPU objects; requests of another text
    # length on the same engine rebuild the bundles; every result equals a fresh engine's.
    mc, mw = speaker_model()
    pj = ih.SamplerParams(num_steps=3, guidance=ih.GuidanceConfig(mode=M.JOINT, scale_text=2.0, scale_speaker=2.0,
                                                                  min_t=0.0))
    pi = ih.SamplerParams(num_steps=3, method=SM.HEUN)
    r1, r2 = request(mc, Tt=16, S=48, seed=1), request(mc, Tt=9, S=48, seed=2)
    kw = dict(max_seq=48, max_text=16, max_aux=32)
    eng = ih.InferenceBuilder(0, F32).load_weights(mc, mw).with_sampling(pj).build(**kw)
    try:
        e2 = eng.with_sampling(pi)
        assert e2.model() is eng.model()
        seq = [eng.sample(r1), e2.sample(r1), eng.sample(r2), e2.sample(r2)]
    finally:
        eng.close()
    for (p, r), got in zip([(pj, r1), (pi, r1), (pj, r2), (pi, r2)], seq):
        with ih.InferenceBuilder(0, F32).load_weights(mc, mw).with_sampling(p).build(**kw) as fresh:
            assert np.array_equal(got, fresh.sample(r))
    assert rel_l2(seq[0], oracle_chain(oracle64, mc, mw, r1, pj, True, False)) < TOL[F32]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_caption_request_matches_oracle_chain(oracle64, backend):
    # A caption model: the auxiliary segment holds the caption encoder's keys (has_caption),
    # Independent CFG over text and caption.
    mc, mw = caption_model()
    g = ih.GuidanceConfig(mode=M.INDEPENDENT, scale_text=2.0, scale_caption=4.0, min_t=0.0)
    p = ih.SamplerParams(num_steps=4, guidance=g)
    req = request(mc, S=40, seed=9, caption=True)
    with ih.InferenceBuilder(0, backend).load_weights(mc, mw).with_sampling(p).build(max_seq=40, max_text=16,
                                                                                      max_aux=12) as eng:
        got = eng.sample(req)
    ref = oracle_chain(oracle64, mc, mw, req, p, False, True)
    print(backend.value, "caption request rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL[backend]


def test_request_errors():
    mc, mw = speaker_model()
    p = ih.SamplerParams(num_steps=2)
    with ih.InferenceBuilder(0, F32).load_weights(mc, mw).with_sampling(p).build(max_seq=32, max_text=16,
                                                                                  max_aux=16) as eng:
        with pytest.raises(ih.IrodoriError) as ei:
            eng.sample(request(mc, Tt=16, Tr=16, S=33))
        assert ei.value.kind == "Shape"  # more frames than the engine holds
        r = request(mc, Tt=16, Tr=16, S=32)
        r.caption_ids = np.zeros((1, 4), np.int32)
        with pytest.raises(ih.IrodoriError) as ei:
            eng.sample(r)
        assert ei.value.kind == "UnsupportedMode"  # no caption conditioner
        bad = ih.SamplerParams(num_steps=2, guidance=ih.GuidanceConfig(mode=M.JOINT, scale_text=2.0,
                                                                       scale_speaker=3.0))
        with pytest.raises(ih.IrodoriError) as ei:
            eng.with_sampling(bad).sample(request(mc, Tt=16, Tr=16, S=32))
        assert ei.value.kind == "Config"  # Joint CFG with unequal scales (euler_sampler.rs:209-228)
