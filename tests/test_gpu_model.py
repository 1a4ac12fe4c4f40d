"""GPU parity of the whole RF-step DiT path (libirodori_hip through the C ABI) against the
CPU oracle, on identical seeded inputs and random-init weights.

Bars: f32 HIP path within 1e-4 relative L2 per block, bf16 within
1e-2 per block and 2e-2 on the final sampled latent.
"""
import dataclasses
import os

import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL_BLOCK = {BF16: 1e-2, F32: 1e-4}
TOL_FINAL = {BF16: 2e-2, F32: 1e-4}


def joint_params(steps, scale=3.0, **kw):
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=scale, scale_speaker=scale,
                          min_t=kw.pop("min_t", 0.0), max_t=kw.pop("max_t", 1.0))
    return ih.SamplerParams(num_steps=steps, guidance=g, **kw)


def make_engine(cfg, backend, w, ctx, rows, seq):
    e = ih.HipInferenceEngine(cfg, backend, max_rows=rows, max_seq=seq, max_ctx=max(ctx.t_ctx, 1))
    e.load_weights(w)
    e.set_context_kv(ctx)
    return e


SMALL = {
    # name: (cfg factory, seq, text, speaker, weight std, norm jitter)
    "tiny": (ih.cfg_tiny, 40, 20, 13, 0.05, 0.1),
    # odd S: the V^T token pair at the batch-row boundary straddles two rows
    "tiny_odd": (ih.cfg_tiny, 37, 11, 9, 0.05, 0.1),
    "cfg1": (ih.cfg_cpu_plumbing, 64, 16, 32, 0.02, 0.0),
    # a 48-channel latent takes the output head's 64-wide tile path (more staged outputs
    # than threads)
    "tiny_p48": (lambda: dataclasses.replace(ih.cfg_tiny(), latent_dim=48), 40, 20, 13, 0.05, 0.1),
    # a 120-channel latent: the output head's 128-wide W' rows (8 zero columns), in_proj over
    # two 64-channel chunks
    "tiny_p120": (lambda: dataclasses.replace(ih.cfg_tiny(), latent_dim=120), 40, 20, 13, 0.05, 0.1),
    # patched latents wider than 128 (latent_patch_size > 1: model.rs:231-233): the output
    # head's 256-wide W' rows, one frame per block; 200 channels leave 56 zero columns
    "tiny_p200": (lambda: dataclasses.replace(ih.cfg_tiny(), latent_dim=200), 40, 20, 13, 0.05, 0.1),
    "tiny_p256": (lambda: dataclasses.replace(ih.cfg_tiny(), latent_dim=256), 37, 20, 13, 0.05, 0.1),
    # the published 500M-v2 width (d 1280, 20 x 64 heads, SwiGLU 3680 padded to 3712 on the
    # device, norms unfused) with two of its twelve layers; 4 text + 9 speaker keys as the
    # A6000 benchmark's request (text_len 4, 8 reference frames + the mean token)
    "pub500m": (lambda: dataclasses.replace(ih.cfg_published_500m(), num_layers=2), 64, 4, 9, 0.02, 0.05),
    # an odd head count (3 x 64, D = 192): the 128-column QKV+gate tile at column D - 64
    # holds the last q head (no RoPE) and k head 0 (RoPE), so the tile must load the RoPE
    # rows although its first head does not rotate
    "h3": (lambda: dataclasses.replace(ih.cfg_tiny(), model_dim=192, num_heads=3, mlp_hidden=320), 40, 20, 13,
           0.05, 0.1),
    # 4000 latent + 250 context keys: 67 key tiles per row, past the 64 one word of the
    # bf16 attention's tile list holds
    "long_keys": (ih.cfg_tiny, 4000, 150, 100, 0.05, 0.1),
    # one and three latent frames: every token pair of the V^T scatter crosses a batch row
    # (S = 1), the QKV+gate RoPE rows step through fewer tokens than one load covers (S < 4),
    # and the output head's frame blocks are mostly past S
    "one_frame": (ih.cfg_tiny, 1, 20, 13, 0.05, 0.1),
    "three_frames": (ih.cfg_tiny, 3, 20, 13, 0.05, 0.1),
}


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(SMALL))
def test_forward_per_block(oracle64, name, backend):
    make_cfg, S, tt, ts, std, jit = SMALL[name]
    cfg = make_cfg()
    w = ih.DitWeights.random(cfg, 0, std=std, norm_jitter=jit)
    ctx = ih.make_context_kv(cfg, 1, tt, ts, seed=1)
    x = ih.make_noise(2, S, cfg.latent_dim, 2)
    t = np.array([0.9, 0.35], np.float32)
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    print(name, backend.value, "per-block rel L2:", ["%.2e" % x for x in errs],
          "v: %.2e" % rel_l2(v, v_ref))
    assert max(errs) < TOL_BLOCK[backend]
    assert rel_l2(v, v_ref) < TOL_BLOCK[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_block_forward_matches_oracle(oracle64, backend):
    cfg = ih.cfg_cpu_plumbing()
    w = ih.DitWeights.random(cfg, 5, norm_jitter=0.05)
    ctx = ih.make_context_kv(cfg, 1, 16, 32, seed=6)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 64, cfg.model_dim)).astype(np.float32)
    cond = (0.5 * rng.standard_normal((2, 3 * cfg.model_dim))).astype(np.float32)
    with make_engine(cfg, backend, w, ctx, 2, 64) as e:
        got = e.block_forward(1, x, cond)
    ref = oracle64.block_forward(cfg, w.blocks[1], x, cond, ctx.k[1], ctx.v[1], ctx.mask)
    assert rel_l2(got, ref) < TOL_BLOCK[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_sample_joint_cfg_cfg1(oracle64, backend):
    # The CPU-plumbing configuration sampled for 4 Euler steps (Joint CFG, scale 3, min_t 0).
    cfg = ih.cfg_cpu_plumbing()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 16, 32, seed=1)
    x0 = ih.make_noise(1, 64, cfg.latent_dim, 2)
    p = joint_params(4)
    with make_engine(cfg, backend, w, ctx, 2, 64) as e:
        got = e.sample(x0, p)
        again = e.sample(x0, p)
    c, u = ctx.rows([0]), ctx.rows([1])
    ref, _ = oracle64.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 4, 3.0)
    print(backend.value, "final rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL_FINAL[backend]
    assert np.array_equal(got, again)  # graph replay is deterministic


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("P", [120, 256])
def test_sample_joint_cfg_wide_latent(oracle64, backend, P):
    # A 120-channel latent through the sampler: the fused head + update with 128-wide W'
    # rows and two frames per block; a 256-channel one with 256-wide rows and one frame per
    # block.  4 Euler steps of Joint CFG against the oracle.
    cfg = dataclasses.replace(ih.cfg_tiny(), latent_dim=P)
    w = ih.DitWeights.random(cfg, 0, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 20, 13, seed=1)
    x0 = ih.make_noise(1, 40, cfg.latent_dim, 2)
    p = joint_params(4)
    with make_engine(cfg, backend, w, ctx, 2, 40) as e:
        got = e.sample(x0, p)
    c, u = ctx.rows([0]), ctx.rows([1])
    ref, _ = oracle64.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 4, 3.0)
    print(backend.value, "latent %d: final rel L2 %.2e" % (P, rel_l2(got, ref)))
    assert rel_l2(got, ref) < TOL_FINAL[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("S", [1, 3])
def test_sample_joint_cfg_few_frames(oracle64, backend, S):
    # Utterances of one and three latent frames through the graph-captured sampler: 4 Euler
    # steps of Joint CFG against the oracle.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 0, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 20, 13, seed=1)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 2)
    p = joint_params(4)
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        got = e.sample(x0, p)
    c, u = ctx.rows([0]), ctx.rows([1])
    ref, _ = oracle64.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 4, 3.0)
    print(backend.value, "S = %d: final rel L2 %.2e" % (S, rel_l2(got, ref)))
    assert rel_l2(got, ref) < TOL_FINAL[backend]


def test_sample_two_utterances_rows_independent(oracle64):
    # Two utterances in one batch (role-major rows: conditioned 0, 1; unconditioned 2, 3)
    # equal each utterance sampled alone.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 2, 12, 9, seed=4)
    x0 = ih.make_noise(2, 24, cfg.latent_dim, 5)
    p = joint_params(3, scale=2.0)
    with make_engine(cfg, F32, w, ctx, 4, 24) as e:
        both = e.sample(x0, p)
    for u in range(2):
        c, un = ctx.rows([u]), ctx.rows([2 + u])
        ref, _ = oracle64.sample_joint_cfg(cfg, w, x0[u:u + 1], (c.k, c.v, c.mask),
                                           (un.k, un.v, un.mask), 3, 2.0)
        assert rel_l2(both[u:u + 1], ref) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("S", [37, 41, 64])
def test_forward_identical_rows_are_bit_identical(backend, S):
    # Every batch row computes the same function of its own inputs, so identical rows give
    # identical outputs in any precision.  Odd S puts odd batch rows on odd token offsets
    # (the V^T pair stores of the QKV epilogue once scrambled them there).
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 6, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 1, 12, 9, seed=7).rows([0, 0, 0])
    x = np.repeat(ih.make_noise(1, S, cfg.latent_dim, 8), 3, axis=0)
    t = np.full(3, 0.6, np.float32)
    with make_engine(cfg, backend, w, ctx, 3, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    for b in (1, 2):
        assert np.array_equal(dbg[:, b], dbg[:, 0]), f"row {b} differs from row 0"
        assert np.array_equal(v[b], v[0])


def test_sample_cfg_window_off_equals_scale_zero():
    # min_t above every t_i disables CFG (euler_sampler.rs:379) == scale 0.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 8, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 8, 8, seed=9)
    x0 = ih.make_noise(1, 16, cfg.latent_dim, 10)
    with make_engine(cfg, F32, w, ctx, 2, 16) as e:
        a = e.sample(x0, joint_params(3, min_t=1.0, max_t=1.0))
        b = e.sample(x0, joint_params(3, scale=0.0))
        c = e.sample(x0, joint_params(3))
    assert np.array_equal(a, b)
    assert rel_l2(c, b) > 1e-3


def test_forward_errors_are_reported():
    cfg = ih.cfg_tiny()
    e = ih.HipInferenceEngine(cfg, F32, max_rows=2, max_seq=16, max_ctx=8)
    x = np.zeros((2, 16, cfg.latent_dim), np.float32)
    with pytest.raises(ih.IrodoriError) as ei:
        e.forward_with_cond_cached(x, np.zeros(2, np.float32))
    assert ei.value.kind == "NotLoaded"
    e.load_weights(ih.DitWeights.random(cfg, 0))
    with pytest.raises(ih.IrodoriError) as ei:
        e.forward_with_cond_cached(np.zeros((2, 17, cfg.latent_dim), np.float32),
                                   np.zeros(2, np.float32))
    assert ei.value.kind == "Shape"
    with pytest.raises(ih.IrodoriError) as ei:
        e.sample(x[:1], joint_params(0))
    assert ei.value.kind == "Config"
    e.close()


# ---- the benchmark configuration (12 layers, d=1024, 750 frames, 631 context keys) ------------------
def cfg4_inputs():
    cfg = ih.cfg_full_rf()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 256, 375, seed=1)
    x0 = ih.make_noise(1, 750, cfg.latent_dim, 2)
    return cfg, w, ctx, x0


@pytest.fixture(scope="module")
def cfg4():
    return cfg4_inputs()


def test_cfg4_forward_per_block_bf16(oracle32, cfg4):
    cfg, w, ctx, x0 = cfg4
    x = np.concatenate([x0, x0])
    t = np.array([0.999, 0.999], np.float32)
    with make_engine(cfg, BF16, w, ctx, 2, 750) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle32.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    # The block increments are ~8 % of the stream: bound them on their own too.
    inc = [rel_l2(a, b) for a, b in zip(_increments(dbg), _increments(dbg_ref))]
    print("cfg4 bf16 per-block rel L2:", ["%.2e" % e_ for e_ in errs], "increments:",
          ["%.1e" % e_ for e_ in inc], "v %.2e" % rel_l2(v, v_ref))
    assert max(errs) < 1e-2 and max(inc) < 2e-2 and rel_l2(v, v_ref) < 1e-2


def _increments(dbg):
    # Each block's own contribution x_{l+1} - x_l (the residual stream is ~12x larger).
    return [dbg[i + 1].astype(np.float64) - dbg[i] for i in range(dbg.shape[0] - 1)]


def test_cfg4_forward_per_block_f32(oracle64, cfg4):
    # Config 4 at the north-star f32 bar: 1e-4 relative L2 per block, the stream and each
    # block's increment, both CFG rows (conditioned with 631 context keys, unconditioned).
    cfg, w, ctx, x0 = cfg4
    x = np.concatenate([x0, x0])
    t = np.array([0.999, 0.6], np.float32)
    with make_engine(cfg, F32, w, ctx, 2, 750) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    inc = [rel_l2(a, b) for a, b in zip(_increments(dbg), _increments(dbg_ref))]
    print("cfg4 f32 per-block rel L2:", ["%.1e" % e_ for e_ in errs], "increments:", ["%.1e" % e_ for e_ in inc])
    assert max(errs) < 1e-4 and max(inc) < 1e-4 and rel_l2(v, v_ref) < 1e-4


@pytest.mark.parametrize("row", [0, 1], ids=["cond", "uncond"])
def test_cfg4_forward_increments_bf16(oracle32, cfg4, row):
    # bf16 at config 4, one CFG row per forward (the sampler's chain: every row on one
    # modulation vector, so the adaLN runs fused into the GEMMs): each block's stream within
    # 1e-2 and each block's own increment within 2e-2 of the f32 oracle.
    cfg, w, ctx, x0 = cfg4
    one = ctx.rows([row])
    t = np.array([0.75], np.float32)
    with make_engine(cfg, BF16, w, one, 1, 750) as e:
        v, dbg = e.forward_with_cond_cached(x0, t, debug=True)
    v_ref, dbg_ref = oracle32.forward(cfg, w, x0, t, one.k, one.v, one.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    inc = [rel_l2(a, b) for a, b in zip(_increments(dbg), _increments(dbg_ref))]
    print("cfg4 bf16 row %d per-block:" % row, ["%.1e" % e_ for e_ in errs], "increments:",
          ["%.1e" % e_ for e_ in inc])
    assert max(errs) < 1e-2 and max(inc) < 2e-2 and rel_l2(v, v_ref) < 1e-2


def test_cfg4_sampler_is_deterministic_across_many_runs(cfg4):
    """Twelve 40-step RF runs of the benchmark configuration, with forward calls of another
    batch shape between them (other graphs, other cache contents), all bit-identical to the
    first: the step counter on the device, the last-workgroup step advance and the forked
    role chains leave no run-to-run state."""
    cfg, w, ctx, x0 = cfg4
    xb = np.concatenate([x0, x0])
    with make_engine(cfg, BF16, w, ctx, 2, 750) as e:
        first = e.sample(x0, joint_params(40))
        for i in range(11):
            if i % 3 == 0:
                e.forward_with_cond_cached(xb, np.array([0.8, 0.3], np.float32))
            assert np.array_equal(e.sample(x0, joint_params(40)), first), i


def test_cfg4_sample_40_steps_bf16_vs_golden(cfg4):
    # Final 40-step latent against the f32 oracle's, committed by tests/golden/make_golden.py.
    path = os.path.join(HERE, "golden", "cfg4_joint40_final_latent.npy")
    if not os.path.exists(path):
        pytest.skip("golden fixture not generated")
    cfg, w, ctx, x0 = cfg4
    with make_engine(cfg, BF16, w, ctx, 2, 750) as e:
        got = e.sample(x0, joint_params(40))
        again = e.sample(x0, joint_params(40))  # graph replays are bit-identical
    assert np.array_equal(got, again)
    ref = np.load(path)
    err = rel_l2(got, ref)
    print("cfg4 bf16 40-step final latent rel L2 %.3e" % err)
    assert err < 2e-2


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_large_batch_tile_shapes_are_bit_identical(cfg4, backend):
    # At 12 rows x 750 frames the W_o / W2 projections switch from 64x64 to 128x128 tiles;
    # both run the same MFMA sequence over k, so rows shared with a 2-row forward (64x64
    # tiles, checked against the oracle above) must agree to the bit.
    cfg, w, _, _ = cfg4
    ctx = ih.make_context_kv(cfg, 6, 256, 375, seed=3)
    x = ih.make_noise(12, 750, cfg.latent_dim, 4)
    t = np.linspace(0.1, 0.9, 12).astype(np.float32)
    with make_engine(cfg, backend, w, ctx, 12, 750) as e:
        v12 = e.forward_with_cond_cached(x, t)
        v2 = e.forward_with_cond_cached(x[:2], t[:2])
    assert np.all(np.isfinite(v12))
    assert np.array_equal(v12[:2], v2)


# ---- latent key mask (attention.rs:730-750; config 5's padded batches) -------------------

def _latent_mask(B, S, lengths, holes=()):
    m = np.zeros((B, S), np.uint8)
    for b, n in enumerate(lengths):
        m[b, :n] = 1
    for b, s in holes:
        m[b, s] = 0
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", ["tiny", "cfg1"])
def test_forward_latent_mask_vs_oracle(oracle64, name, backend):
    make_cfg, S, tt, ts, std, jit = SMALL[name]
    cfg = make_cfg()
    w = ih.DitWeights.random(cfg, 3, std=std, norm_jitter=jit)
    ctx = ih.make_context_kv(cfg, 1, tt, ts, seed=4)
    x = ih.make_noise(2, S, cfg.latent_dim, 5)
    t = np.array([0.8, 0.45], np.float32)
    # row 0: isolated masked keys (first, middle, last tile positions); row 1: a masked
    # tail of 19 keys plus one hole
    m = _latent_mask(2, S, [S, S - 19], holes=[(0, 1), (0, S // 2), (0, S - 1), (1, 7)])
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True, latent_mask=m)
        v_plain = e.forward_with_cond_cached(x, t)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True, latent_mask=m)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    print(name, backend.value, "masked per-block rel L2:", ["%.2e" % x for x in errs])
    assert max(errs) < TOL_BLOCK[backend]
    assert rel_l2(v, v_ref) < TOL_BLOCK[backend]
    assert rel_l2(v, v_plain) > 1e-3  # the mask reached the attention


@pytest.mark.gpu
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_forward_row_without_any_valid_key(oracle64, backend):
    # Row 1 is the unconditioned bundle (every context key masked); with its latent keys
    # masked too, no key of that row attends: its attention output is 0 in every block
    # (attention.rs:770-787) and the forward still matches the oracle.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 1, 12, 9, seed=4)
    S = 40
    x = ih.make_noise(2, S, cfg.latent_dim, 5)
    t = np.array([0.7, 0.7], np.float32)
    m = _latent_mask(2, S, [S, 0])
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True, latent_mask=m)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True, latent_mask=m)
    assert np.all(np.isfinite(v))
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    assert max(errs) < TOL_BLOCK[backend], errs
    assert rel_l2(v, v_ref) < TOL_BLOCK[backend]


@pytest.mark.gpu
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_sample_padded_batch_matches_unpadded(backend):
    # Two utterances padded to 64 frames, the second only 41 long: its first 41 frames
    # equal an unpadded 41-frame run of that utterance alone.
    cfg = ih.cfg_cpu_plumbing()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 2, 16, 32, seed=1)
    x0 = ih.make_noise(2, 64, cfg.latent_dim, 2)
    p = joint_params(4)
    n = 41
    with make_engine(cfg, backend, w, ctx, 4, 64) as e:
        padded = e.sample(x0, p, lengths=[64, n])
        full = e.sample(x0, p)
    with make_engine(cfg, backend, w, ctx.rows([1, 3]), 2, 64) as e:  # utterance 1's roles
        short = e.sample(x0[1:2, :n], p)
    assert rel_l2(padded[1:2, :n], short) < 1e-6
    assert rel_l2(padded[0:1], full[0:1]) < 1e-6  # full-length utterance unaffected
    import torch
    d_x0 = torch.from_numpy(x0).to("cuda")
    d_out = torch.empty_like(d_x0)
    with make_engine(cfg, backend, w, ctx, 4, 64) as e:  # device-pointer variant
        e.sample_device(d_x0.data_ptr(), d_out.data_ptr(), 2, 64, p, lengths=[64, n])
        torch.cuda.synchronize()
    assert np.array_equal(d_out.cpu().numpy(), padded)
    with pytest.raises(ih.IrodoriError):
        with make_engine(cfg, backend, w, ctx, 4, 64) as e:
            e.sample(x0, p, lengths=[64, 65])


@pytest.mark.parametrize("backend", [BF16, ih.InferenceBackendKind.HIP_FP8], ids=["bf16", "fp8"])
def test_profile_layer_reports_every_kernel(backend):
    # irodori_profile_layer on the configuration-1 model (bf16, and its fp8 GEMM mode): one
    # positive, finite time per kernel of the block and the output head; an f32 context is
    # refused with a dtype error.
    cfg = ih.cfg_cpu_plumbing()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 16, 32, seed=1)
    with make_engine(cfg, backend, w, ctx, 2, 64) as e:
        kt = e.profile_layer(1, 64, 3)
    assert set(kt) == {"norm_mod_us", "qkvg_gemm_us", "attention_us", "wo_gemm_us", "w13_gemm_us",
                       "w2_gemm_us", "final_us"}
    assert all(np.isfinite(v) and v > 0 for v in kt.values()), kt
    with make_engine(cfg, F32, w, ctx, 2, 64) as e:
        with pytest.raises(ih.IrodoriError, match="Dtype"):
            e.profile_layer(1, 64, 3)


def test_device_allocation_limit_reports_out_of_memory(monkeypatch):
    # IRODORI_DEVICE_ALLOC_LIMIT turns a context's, encoder's or codec's persistent
    # allocations past the limit into IRODORI_ERR_OOM (OutOfMemory) before hipMalloc runs; the
    # partly built object is released, and objects created without the limit work.
    cfg = ih.cfg_tiny()
    monkeypatch.setenv("IRODORI_DEVICE_ALLOC_LIMIT", "4096")
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipInferenceEngine(cfg, F32, max_rows=2, max_seq=40, max_ctx=33)
    assert ei.value.kind == "OutOfMemory" and "IRODORI_DEVICE_ALLOC_LIMIT" in str(ei.value)
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipEncoder(ih.enc_text_tiny(), F32, max_rows=2, max_seq=20)
    assert ei.value.kind == "OutOfMemory"
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipDacVaeCodec(ih.codec_tiny(), F32, max_frames=16)
    assert ei.value.kind == "OutOfMemory"
    monkeypatch.delenv("IRODORI_DEVICE_ALLOC_LIMIT")
    w = ih.DitWeights.random(cfg, 0, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 20, 13, seed=1)
    x = ih.make_noise(2, 40, cfg.latent_dim, 2)
    with make_engine(cfg, F32, w, ctx, 2, 40) as e:
        v = e.forward_with_cond_cached(x, np.array([0.9, 0.35], np.float32))
    assert np.all(np.isfinite(v))



def test_graph_cache_eviction_keeps_results():
    """The sampler keeps at most 64 captured graphs, least recently used out first.  70
    distinct sequence lengths evict the first ones; running the first length again re-captures
    its graph and gives the same bits as its first run."""
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 6, 2, seed=1)
    x0 = ih.make_noise(1, 72, cfg.latent_dim, 4)
    p = joint_params(1)
    with make_engine(cfg, ih.InferenceBackendKind.HIP_BF16, w, ctx, 2, 72) as e:
        first = {S: e.sample(x0[:, :S].copy(), p, has_speaker=True) for S in (3, 4)}
        for S in range(5, 73):
            e.sample(x0[:, :S].copy(), p, has_speaker=True)
        for S, ref in first.items():
            again = e.sample(x0[:, :S].copy(), p, has_speaker=True)
            assert np.array_equal(again, ref), S
