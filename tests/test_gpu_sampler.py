"""GPU parity of the HIP RF sampler in every CFG mode and integrator (sample_euler_rf_cfg,
euler_sampler.rs:132-718) against the oracle's sample_rf, whose loop is pinned on the CPU
(test_oracle_sampler.py), through the C ABI on the same seeded inputs.

Bars: f32 path 1e-4 relative L2 on the final latent, bf16 2e-2.
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2
from oracle.oracle import sampler_struct

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL = {BF16: 2e-2, F32: 1e-4}
M = ih.CfgGuidanceMode
SM = ih.SamplerMethod
TT, TA, S = 10, 9, 24  # text keys, aux keys, latent frames


def params(mode, method, steps=4, scale_text=2.0, scale_speaker=3.0, min_t=0.0, **kw):
    if mode is M.JOINT:
        scale_speaker = scale_text
    g = ih.GuidanceConfig(mode=mode, scale_text=scale_text, scale_speaker=scale_speaker,
                          scale_caption=0.0, min_t=min_t, max_t=1.0)
    return ih.SamplerParams(num_steps=steps, method=method, guidance=g, **kw)


def orc_params(p, has_speaker=True, aux_start=TT, has_caption=False):
    g = p.guidance
    tr, skv = p.temporal_rescale, p.speaker_kv
    return sampler_struct(
        num_steps=p.num_steps, method={SM.EULER: 0, SM.HEUN: 1, SM.PLMS4: 2}[p.method],
        cfg_mode={M.INDEPENDENT: 0, M.JOINT: 1, M.ALTERNATING: 2}[g.mode],
        scale_text=g.scale_text, scale_caption=g.scale_caption, scale_speaker=g.scale_speaker,
        min_t=g.min_t, max_t=g.max_t, has_truncation=int(p.truncation_factor is not None),
        truncation_factor=p.truncation_factor or 1.0, has_speaker=int(has_speaker), has_caption=int(has_caption),
        has_temporal_rescale=int(tr is not None), rescale_k=tr.k if tr else 1.0,
        rescale_sigma=tr.sigma if tr else 1.0, has_speaker_kv=int(skv is not None),
        speaker_kv_scale=skv.scale if skv else 1.0,
        speaker_kv_max_layers=skv.max_layers if skv and skv.max_layers is not None else -1,
        speaker_kv_has_min_t=int(skv is not None and skv.min_t is not None),
        speaker_kv_min_t=skv.min_t if skv is not None and skv.min_t is not None else 0.0,
        ctx_aux_start=aux_start)


@pytest.fixture(scope="module")
def model():
    cfg = ih.cfg_tiny()
    return cfg, ih.DitWeights.random(cfg, 21, std=0.05, norm_jitter=0.1)


def run(oracle64, model, backend, p, U=1, seed=3, lengths=None):
    cfg, w = model
    roles = p.cfg_roles(has_speaker=True)
    ctx = ih.make_role_context(cfg, U, TT, TA, roles, seed=seed)
    x0 = ih.make_noise(U, S, cfg.latent_dim, seed + 1)
    e = ih.HipInferenceEngine(cfg, backend, max_rows=len(roles) * U, max_seq=S, max_ctx=ctx.t_ctx)
    try:
        e.load_weights(w)
        e.set_context_kv(ctx)
        got = e.sample(x0, p, ctx_aux_start=TT, lengths=lengths)
        again = e.sample(x0, p, ctx_aux_start=TT, lengths=lengths)
    finally:
        e.close()
    lat = None
    if lengths is not None:
        lat = np.zeros((U, S), np.uint8)
        for u, n in enumerate(lengths):
            lat[u, :n] = 1
    ref, _ = oracle64.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), orc_params(p), latent_mask=lat)
    return got, again, ref


CASES = [(mode, method) for mode in (M.INDEPENDENT, M.JOINT, M.ALTERNATING)
         for method in (SM.EULER, SM.HEUN, SM.PLMS4)
         if not (mode is M.ALTERNATING and method is SM.PLMS4)]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("mode,method", CASES, ids=["%s-%s" % (a.value, b.value) for a, b in CASES])
def test_mode_and_method(oracle64, model, backend, mode, method):
    # min_t 0.5: the CFG window closes half way (the later steps run the conditioned role
    # alone; PLMS-4 restarts its history there).
    p = params(mode, method, steps=5, min_t=0.5)
    got, again, ref = run(oracle64, model, backend, p)
    print(mode.value, method.value, backend.value, "rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL[backend]
    assert np.array_equal(got, again)  # replays of the captured evaluations are deterministic


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("method", [SM.EULER, SM.PLMS4], ids=["euler", "plms4"])
def test_temporal_rescale(oracle64, model, backend, method):
    p = params(M.INDEPENDENT, method, steps=4,
               temporal_rescale=ih.config.TemporalRescaleConfig(k=2.0, sigma=0.8))
    got, _, ref = run(oracle64, model, backend, p)
    plain, _, _ = run(oracle64, model, backend, params(M.INDEPENDENT, method, steps=4))
    assert rel_l2(got, ref) < TOL[backend]
    assert rel_l2(got, plain) > 1e-3


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("mode", [M.INDEPENDENT, M.JOINT], ids=["independent", "joint"])
def test_speaker_kv_scaling_with_revert(oracle64, model, backend, mode):
    # Scaled in the first layer only, reverted once t drops below 0.6 (step 2 of 4).
    skv = ih.config.SpeakerKvConfig(scale=1.8, max_layers=1, min_t=0.6)
    p = params(mode, SM.EULER, steps=4, speaker_kv=skv)
    got, again, ref = run(oracle64, model, backend, p)
    plain, _, _ = run(oracle64, model, backend, params(mode, SM.EULER, steps=4))
    assert rel_l2(got, ref) < TOL[backend]
    assert rel_l2(got, plain) > 1e-4
    assert np.array_equal(got, again)  # the context copies are rebuilt for every call


def test_speaker_kv_layer_count_changes_between_calls(oracle64, model):
    # One context sampled with speaker-KV scaling in the first layer, then in both layers,
    # then without, then in the first layer again: the captured evaluations must follow the
    # layer count of each call (each result equals a fresh context's, bit for bit, and the
    # oracle's).
    cfg, w = model
    runs = [ih.config.SpeakerKvConfig(scale=1.8, max_layers=1), ih.config.SpeakerKvConfig(scale=1.8, max_layers=2),
            None, ih.config.SpeakerKvConfig(scale=1.8, max_layers=1)]
    ps = [params(M.JOINT, SM.EULER, steps=3, speaker_kv=skv) for skv in runs]
    roles = ps[0].cfg_roles(has_speaker=True)
    ctx = ih.make_role_context(cfg, 1, TT, TA, roles, seed=3)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 4)

    def engine():
        e = ih.HipInferenceEngine(cfg, F32, max_rows=len(roles), max_seq=S, max_ctx=ctx.t_ctx)
        e.load_weights(w)
        e.set_context_kv(ctx)
        return e

    with engine() as e:
        seq = [e.sample(x0, p, ctx_aux_start=TT) for p in ps]
    for p, got in zip(ps, seq):
        with engine() as fresh:
            alone = fresh.sample(x0, p, ctx_aux_start=TT)
        ref, _ = oracle64.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), orc_params(p))
        assert np.array_equal(got, alone)
        assert rel_l2(got, ref) < TOL[F32]
    assert rel_l2(seq[0], seq[1]) > 1e-5  # the layer count matters


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_two_utterances_independent_padded(oracle64, model, backend):
    # Role-major rows with U = 2 (conditioned 0-1, text dropped 2-3, speaker dropped 4-5),
    # the second utterance padded from 17 frames.
    p = params(M.INDEPENDENT, SM.HEUN, steps=3)
    got, _, ref = run(oracle64, model, backend, p, U=2, lengths=[S, 17])
    assert rel_l2(got[0], ref[0]) < TOL[backend]
    assert rel_l2(got[1, :17], ref[1, :17]) < TOL[backend]


def test_heun_rescale_reaches_t_zero_as_the_reference(oracle64, model):
    # The last Heun corrector evaluates at t_N = 0, where the rescale's snr = (1-t)^2 / t^2
    # is infinite and the ratio inf / inf is NaN (math.rs:38-53): the reference's latent is
    # NaN, and so is this one.
    p = params(M.JOINT, SM.HEUN, steps=3, temporal_rescale=ih.config.TemporalRescaleConfig(k=2.0, sigma=0.8))
    got, _, ref = run(oracle64, model, F32, p)
    assert np.isnan(ref).all() and np.isnan(got).all()


# ---- caption-conditioned CFG (euler_sampler.rs:186-195, :205, :314-321, :490) -------------
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("mode,method", [(M.INDEPENDENT, SM.EULER), (M.ALTERNATING, SM.HEUN), (M.JOINT, SM.PLMS4)],
                         ids=["indep-euler", "alt-heun", "joint-plms4"])
def test_caption_cfg_matches_oracle(oracle64, model, backend, mode, method):
    # A caption model: the aux segment holds caption keys, has_caption = 1, has_speaker = 0;
    # the caption signal follows text and takes scale_caption (the speaker scale is ignored).
    cfg, w = model
    s_cap = 2.0 if mode is M.JOINT else 3.5
    g = ih.GuidanceConfig(mode=mode, scale_text=2.0, scale_caption=s_cap, scale_speaker=9.0,
                          min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=4, method=method, guidance=g)
    roles = p.cfg_roles(has_speaker=False, has_caption=True)
    assert roles == (["cond", "uncond"] if mode is M.JOINT else ["cond", "no_text", "no_aux"])
    ctx = ih.make_role_context(cfg, 1, TT, TA, roles, seed=13)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 14)
    with ih.HipInferenceEngine(cfg, backend, max_rows=len(roles), max_seq=S, max_ctx=ctx.t_ctx) as e:
        e.load_weights(w)
        e.set_context_kv(ctx)
        got = e.sample(x0, p, has_speaker=False, has_caption=True, ctx_aux_start=TT)
        with pytest.raises(ih.IrodoriError, match="exclusive"):
            e.sample(x0, p, has_speaker=True, has_caption=True, ctx_aux_start=TT)
    ref, _ = oracle64.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                                orc_params(p, has_speaker=False, has_caption=True))
    err = rel_l2(got, ref)
    print(mode, method, backend.value, "caption CFG rel L2 %.2e" % err)
    assert err < TOL[backend]


# ---- the published model's width in the A6000 benchmark's sampler configuration -----------
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_published_width_independent_cfg(oracle64, backend):
    # d 1280, 20 x 64 heads, SwiGLU 3680 (two layers); Independent CFG with three roles, text
    # scale 3, speaker scale 5, min_t 0.5 (CFG only on the steps with t >= 0.5), 4 text keys,
    # 9 speaker keys (docs/benchmarks/rtx-a6000.md:24-36); 6 Euler steps over 48 frames.
    import dataclasses
    cfg = dataclasses.replace(ih.cfg_published_500m(), num_layers=2)
    w = ih.DitWeights.random(cfg, 31, norm_jitter=0.05)
    p = params(M.INDEPENDENT, SM.EULER, steps=6, scale_text=3.0, scale_speaker=5.0, min_t=0.5)
    roles = p.cfg_roles(has_speaker=True)
    assert roles == ["cond", "no_text", "no_aux"]
    tt, ta, s = 4, 9, 48
    ctx = ih.make_role_context(cfg, 1, tt, ta, roles, seed=32)
    x0 = ih.make_noise(1, s, cfg.latent_dim, 33)
    with ih.HipInferenceEngine(cfg, backend, max_rows=3, max_seq=s, max_ctx=ctx.t_ctx) as e:
        e.load_weights(w)
        e.set_context_kv(ctx)
        got = e.sample(x0, p, ctx_aux_start=tt)
    ref, _ = oracle64.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), orc_params(p, aux_start=tt))
    err = rel_l2(got, ref)
    print(backend.value, "published width Independent CFG rel L2 %.2e" % err)
    assert err < TOL[backend]
