"""CPU pins of the oracle's general RF sampler (euler_sampler.rs:132-718).

Every check reaches the sampler's result by a route independent of sample_rf's loop:
exact equalities with the already pinned Joint sampler, compositions of single oracle
forwards (whose parity is pinned in test_oracle.py) following the reference's update
rules, limits of the temporal score rescale that fix its formula, and equalities with a
context scaled by hand for the speaker-KV option.
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, ".."))
sys.path.insert(0, os.path.join(HERE, "..", "irodori-tts-burn_amd"))

import irodori_hip as ih  # noqa: E402
from conftest import rel_l2  # noqa: E402
from oracle.oracle import Oracle, sampler_struct  # noqa: E402

EULER, HEUN, PLMS = 0, 1, 2
INDEP, JOINT, ALT = 0, 1, 2
TT, TA = 10, 9  # text / aux context keys


@pytest.fixture(scope="module")
def orc():
    return Oracle("f64")


@pytest.fixture(scope="module")
def orc32():
    # exact equalities are checked in f32, where every operator rounds as the reference's
    return Oracle("f32")


@pytest.fixture(scope="module")
def model():
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 11, std=0.05, norm_jitter=0.1)
    return cfg, w


def _ctx(cfg, roles, U=1, seed=5):
    return ih.make_role_context(cfg, U, TT, TA, roles, seed=seed)


def _rows(ctx, r, U):
    c = ctx.rows([r * U + u for u in range(U)])
    return c.k, c.v, c.mask


def _sched(n):
    return [np.float32(0.999) * (np.float32(1.0) - np.float32(i) / np.float32(n)) for i in range(n + 1)]


def _fwd(orc, cfg, w, x, t, ctx, r, U):
    k, v, m = _rows(ctx, r, U)
    return orc.forward(cfg, w, x, np.full(U, t, np.float32), k, v, m).astype(np.float64)


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def test_joint_equals_the_joint_sampler(orc32, model):
    orc = orc32
    cfg, w = model
    U, S = 2, 20
    ctx = _ctx(cfg, ["cond", "uncond"], U)
    x0 = ih.make_noise(U, S, cfg.latent_dim, 3)
    sp = sampler_struct(num_steps=3, cfg_mode=JOINT, scale_text=2.5, min_t=0.0, max_t=1.0)
    got, run = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp)
    ref, _ = orc.sample_joint_cfg(cfg, w, x0, _rows(ctx, 0, U), _rows(ctx, 1, U), 3, 2.5, 0.0, 1.0)
    assert run == 3
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("mode", [INDEP, ALT])
def test_one_signal_modes_equal_joint(orc32, model, mode):
    orc = orc32
    # With only text guidance, dropping the text signal is the role the Joint sampler
    # uses as unconditioned when the aux segment is absent from the context.
    cfg, w = model
    ctx = ih.make_role_context(cfg, 1, TT, 0, ["cond", "no_text"], seed=6)
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 4)
    kw = dict(num_steps=3, scale_text=2.0, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(cfg_mode=mode, **kw))
    ref, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(cfg_mode=JOINT, **kw))
    assert np.array_equal(got, ref)


def test_independent_two_signals_one_step(orc, model):
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "no_text", "no_aux"])
    x0 = ih.make_noise(1, 18, cfg.latent_dim, 7)
    sp = sampler_struct(num_steps=2, cfg_mode=INDEP, scale_text=3.0, scale_speaker=5.0,
                        has_speaker=1, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp, max_steps_run=1)
    t = _sched(2)
    vc, v1, v2 = (_fwd(orc, cfg, w, x0, t[0], ctx, r, 1) for r in range(3))
    v = vc + (vc - v1) * 3.0 + (vc - v2) * 5.0
    assert rel(got, x0 + v * (t[1] - t[0])) < 1e-6


def test_alternating_drops_the_signals_in_turn(orc, model):
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "no_text", "no_aux"])
    x0 = ih.make_noise(1, 18, cfg.latent_dim, 8)
    sp = sampler_struct(num_steps=2, cfg_mode=ALT, scale_text=3.0, scale_speaker=5.0,
                        has_speaker=1, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp)
    t = _sched(2)
    x = x0.astype(np.float64)
    for i, (role, s) in enumerate([(1, 3.0), (2, 5.0)]):  # step 0 drops text, step 1 speaker
        vc = _fwd(orc, cfg, w, x, t[i], ctx, 0, 1)
        va = _fwd(orc, cfg, w, x, t[i], ctx, role, 1)
        x = x + (vc + (vc - va) * s) * (t[i + 1] - t[i])
    assert rel(got, x) < 1e-6


def test_heun_one_step(orc, model):
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "uncond"])
    x0 = ih.make_noise(1, 18, cfg.latent_dim, 9)
    sp = sampler_struct(num_steps=3, method=HEUN, cfg_mode=JOINT, scale_text=2.0, scale_speaker=2.0,
                        has_speaker=1, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp, max_steps_run=1)
    t = _sched(3)
    dt = t[1] - t[0]

    def guided(x, tt):
        vc = _fwd(orc, cfg, w, x, tt, ctx, 0, 1)
        return vc + (vc - _fwd(orc, cfg, w, x, tt, ctx, 1, 1)) * 2.0

    v1 = guided(x0, t[0])
    v2 = guided(x0 + v1 * dt, t[1])
    assert rel(got, x0 + (v1 + v2) / 2 * dt) < 1e-6


def test_plms_startup_orders(orc, model):
    # AB-1, AB-2, AB-3 on the first three steps (euler_sampler.rs:98-117).
    cfg, w = model
    ctx = _ctx(cfg, ["cond"])
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 10)
    sp = sampler_struct(num_steps=5, method=PLMS, cfg_mode=JOINT, scale_text=0.0, scale_speaker=0.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp, max_steps_run=3)
    t = _sched(5)
    coef = [[1.0], [1.5, -0.5], [23 / 12, -16 / 12, 5 / 12]]
    x, hist = x0.astype(np.float64), []
    for i in range(3):
        hist.insert(0, _fwd(orc, cfg, w, x, t[i], ctx, 0, 1))
        x = x + sum(c * h for c, h in zip(coef[i], hist)) * (t[i + 1] - t[i])
    assert rel(got, x) < 1e-6


def test_plms_history_restarts_when_cfg_switches_off(orc, model):
    # N = 4: t = 0.999, 0.749, 0.4995, 0.2497; CFG window [0.6, 1] covers steps 0-1 only, so
    # step 2 restarts at AB-1 and step 3 runs AB-2 over steps 2-3 (euler_sampler.rs:383-390).
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "uncond"])
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 12)
    sp = sampler_struct(num_steps=4, method=PLMS, cfg_mode=JOINT, scale_text=2.0, scale_speaker=2.0,
                        has_speaker=1, min_t=0.6, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp)
    t = _sched(4)
    x, hist = x0.astype(np.float64), []
    for i in range(4):
        vc = _fwd(orc, cfg, w, x, t[i], ctx, 0, 1)
        on = 0.6 <= t[i] <= 1.0
        v = vc + (vc - _fwd(orc, cfg, w, x, t[i], ctx, 1, 1)) * 2.0 if on else vc
        if i == 2:
            hist = []
        hist.insert(0, v)
        c = [[1.0], [1.5, -0.5], [23 / 12, -16 / 12, 5 / 12]][len(hist) - 1]
        x = x + sum(a * h for a, h in zip(c, hist)) * (t[i + 1] - t[i])
    assert rel(got, x) < 1e-6


def test_temporal_rescale_limits(orc, model):
    # ratio = (snr s^2 + 1) / (snr s^2 / k + 1), snr = (1-t)^2 / t^2 (math.rs:38-53):
    # k = 1 is the identity; at t = 0.999 with s = 1 (snr s^2 ~ 1e-6) it is ~1; with
    # s = 1e6 (snr s^2 ~ 1e6) it is ~k, giving v' = (v (1-t) + x) k / (1-t) - x / (1-t).
    cfg, w = model
    ctx = _ctx(cfg, ["cond"])
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 13)
    base = dict(num_steps=4, cfg_mode=JOINT, scale_text=0.0, scale_speaker=0.0)
    ref, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(**base), max_steps_run=1)
    # k = 1: ratio exactly 1.  k = 3, s = 1: ratio - 1 ~ 7e-7, amplified by 1 / (1 - t) =
    # 1e3 into a ~1e-4 change (an inverted snr would give ratio ~ k, an O(1) change).
    for k_, s_, bound in ((1.0, 0.37, 1e-5), (3.0, 1.0, 1e-3)):
        got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                               sampler_struct(has_temporal_rescale=1, rescale_k=k_, rescale_sigma=s_, **base),
                               max_steps_run=1)
        assert rel(got, ref) < bound, (k_, s_)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                           sampler_struct(has_temporal_rescale=1, rescale_k=2.0, rescale_sigma=1e6, **base),
                           max_steps_run=1)
    t = _sched(4)
    v = _fwd(orc, cfg, w, x0, t[0], ctx, 0, 1)
    omt = 1.0 - t[0]
    v_r = (v * omt + x0) * 2.0 / omt - x0 / omt
    assert rel(got, x0 + v_r * (t[1] - t[0])) < 1e-5
    assert rel(got, ref) > 1e-3  # the rescale changed the step


def _prescaled(ctx, roles_scaled, layers, s, U=1):
    k, v = ctx.k.copy(), ctx.v.copy()
    for r in roles_scaled:
        for u in range(U):
            k[:layers, r * U + u, TT:] *= np.float32(s)
            v[:layers, r * U + u, TT:] *= np.float32(s)
    return k, v


@pytest.mark.parametrize("mode,roles,scaled", [
    (JOINT, ["cond", "uncond"], [0]),
    (INDEP, ["cond", "no_text", "no_aux"], [0, 1, 2]),
    (ALT, ["cond", "no_text", "no_aux"], [0]),
])
def test_speaker_kv_scaling_equals_a_prescaled_context(orc32, model, mode, roles, scaled):
    orc = orc32
    # kv_scaling.rs:10-60: the aux keys of the conditioned cache (and, in Independent
    # mode, of the batched cache) times the scale in the first max_layers layers.
    cfg, w = model
    ctx = _ctx(cfg, roles)
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 14)
    kw = dict(num_steps=3, cfg_mode=mode, scale_text=2.0, scale_speaker=2.0, has_speaker=1,
              min_t=0.0, max_t=1.0, ctx_aux_start=TT)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                           sampler_struct(has_speaker_kv=1, speaker_kv_scale=1.7, speaker_kv_max_layers=1, **kw))
    k, v = _prescaled(ctx, scaled, 1, 1.7)
    ref, _ = orc.sample_rf(cfg, w, x0, (k, v, ctx.mask), sampler_struct(**kw))
    assert np.array_equal(got, ref)
    plain, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(**kw))
    assert rel(got, plain) > 1e-4
    # not applied when the condition holds no speaker state (euler_sampler.rs:258-264)
    kw_ns = dict(kw, has_speaker=0)
    a, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                         sampler_struct(has_speaker_kv=1, speaker_kv_scale=1.7, **kw_ns))
    b, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(**kw_ns))
    assert np.array_equal(a, b)


def test_speaker_kv_reverts_below_min_t(orc, model):
    # t = 0.999, 0.666: with min_t = 0.8 the scaling holds for step 0 and is undone (times
    # 1 / scale, euler_sampler.rs:533-545) before step 1.
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "uncond"])
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 15)
    kw = dict(num_steps=3, cfg_mode=JOINT, scale_text=2.0, scale_speaker=2.0, has_speaker=1,
              min_t=0.0, max_t=1.0, ctx_aux_start=TT)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                           sampler_struct(has_speaker_kv=1, speaker_kv_scale=2.5, speaker_kv_has_min_t=1,
                                          speaker_kv_min_t=0.8, **kw), max_steps_run=2)
    t = _sched(3)
    k, v = _prescaled(ctx, [0], cfg.num_layers, 2.5)
    scaled = ih.ContextKV(k, v, ctx.mask)
    x = x0.astype(np.float64)
    for i, c in enumerate([scaled, ctx]):
        vc = _fwd(orc, cfg, w, x, t[i], c, 0, 1)
        vu = _fwd(orc, cfg, w, x, t[i], c, 1, 1)
        x = x + (vc + (vc - vu) * 2.0) * (t[i + 1] - t[i])
    assert rel(got, x) < 1e-6


# ---- caption-conditioned CFG (euler_sampler.rs:186-195, :205, :314-321, :490) ----------------
# A caption model's aux segment holds the caption keys; its CFG signal comes last in the
# order (text, speaker, caption), takes scale_caption, and dropping it zeroes the aux
# segment like dropping a speaker (make_aux_uncond, euler_sampler.rs:59-82).  The speaker
# scale is ignored there (cfg_scale_speaker = 0 without speaker conditioning, :162-166).

def test_caption_independent_one_step(orc, model):
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "no_text", "no_aux"])
    x0 = ih.make_noise(1, 18, cfg.latent_dim, 17)
    sp = sampler_struct(num_steps=2, cfg_mode=INDEP, scale_text=3.0, scale_caption=4.0, scale_speaker=9.0,
                        has_speaker=0, has_caption=1, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp, max_steps_run=1)
    t = _sched(2)
    vc, v1, v2 = (_fwd(orc, cfg, w, x0, t[0], ctx, r, 1) for r in range(3))
    v = vc + (vc - v1) * 3.0 + (vc - v2) * 4.0
    assert rel(got, x0 + v * (t[1] - t[0])) < 1e-6


def test_caption_alternating_drops_text_then_caption(orc, model):
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "no_text", "no_aux"])
    x0 = ih.make_noise(1, 18, cfg.latent_dim, 18)
    sp = sampler_struct(num_steps=2, cfg_mode=ALT, scale_text=3.0, scale_caption=4.0, has_speaker=0,
                        has_caption=1, min_t=0.0, max_t=1.0)
    got, _ = orc.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sp)
    t = _sched(2)
    x = x0.astype(np.float64)
    for i, (role, s) in enumerate([(1, 3.0), (2, 4.0)]):  # step 0 drops text, step 1 the caption
        vc = _fwd(orc, cfg, w, x, t[i], ctx, 0, 1)
        va = _fwd(orc, cfg, w, x, t[i], ctx, role, 1)
        x = x + (vc + (vc - va) * s) * (t[i + 1] - t[i])
    assert rel(got, x) < 1e-6


def test_caption_joint_equals_speaker_joint(orc32, model):
    # Joint mode with text + caption at one scale runs the same two roles as text + speaker.
    cfg, w = model
    ctx = _ctx(cfg, ["cond", "uncond"], 2)
    x0 = ih.make_noise(2, 16, cfg.latent_dim, 19)
    kw = dict(num_steps=3, cfg_mode=JOINT, scale_text=2.5, min_t=0.0, max_t=1.0)
    cap, _ = orc32.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                             sampler_struct(scale_caption=2.5, scale_speaker=7.0, has_caption=1, **kw))
    spk, _ = orc32.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                             sampler_struct(scale_speaker=2.5, has_speaker=1, **kw))
    assert np.array_equal(cap, spk)


def test_caption_without_valid_token_is_no_signal(orc32, model):
    # has_caption = 0 (no caption token is valid, euler_sampler.rs:186-195): text guidance
    # only, whatever scale_caption says.
    cfg, w = model
    ctx = ih.make_role_context(cfg, 1, TT, TA, ["cond", "no_text"], seed=20)
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 21)
    kw = dict(num_steps=3, cfg_mode=INDEP, scale_text=2.0, min_t=0.0, max_t=1.0, has_speaker=0)
    a, _ = orc32.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask),
                           sampler_struct(scale_caption=4.0, has_caption=0, **kw))
    b, _ = orc32.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), sampler_struct(**kw))
    assert np.array_equal(a, b)


def test_speaker_and_caption_flags_are_exclusive():
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.INDEPENDENT, scale_text=2.0, scale_caption=3.0)
    p = ih.SamplerParams(num_steps=4, guidance=g)
    with pytest.raises(ih.IrodoriError, match="exclusive"):
        p.validate(has_speaker=True, has_caption=True)
    p.validate(has_speaker=False, has_caption=True)


def _joint_run(orc, cfg, w, ctx, x0, steps=3):
    c, u = ctx.rows([0]), ctx.rows([1])
    out, _ = orc.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), steps, 3.0)
    return out


def test_folded_adaln_is_the_same_function_in_exact_arithmetic():
    # The folded adaLN of the bf16 sampler chains (h W = r (x (1 + scale)) W + shift W,
    # norm.rs:160-169) is an algebraic identity: in float64 arithmetic it reproduces the
    # unfolded sampler to rounding (both store their intermediates as f32, so to f32
    # rounding: ~1e-7 over three steps; a dropped shift or a misplaced r costs ~1e-1).
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 4, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 1, 9, 7, seed=2)
    x0 = ih.make_noise(1, 20, cfg.latent_dim, 3)
    plain = _joint_run(Oracle("f64"), cfg, w, ctx, x0)
    folded = _joint_run(Oracle("f64", fused_adaln=True), cfg, w, ctx, x0)
    assert rel_l2(folded, plain) < 1e-6
