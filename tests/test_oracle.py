"""Pins of the CPU oracle (CPU only).

The reference ships no golden vectors for this path (its Python fixtures are generated
on demand from an absent upstream), so each oracle function is pinned by the
reference's own closed-form unit tests, by special cases the mathematics fixes, by
library routines (torch.nn.functional) and by brute force on tiny inputs.  Each check is
chosen so that a plausible slip — wrong chunk order, wrong RoPE sign or pairing, a
transposed weight, an inverted mask, a dropped norm weight — fails it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import irodori_hip as ih
from conftest import rel_l2
import torch_reference as tref


# ---- RMSNorm / adaLN --------------------------------------------------------------------
def test_rms_norm_ones_is_one(oracle32):
    # norm.rs:193-203 (rms_norm_unit_scale_preserves_magnitude)
    y = oracle32.rms_norm(np.ones((1, 8), np.float32), np.ones(8, np.float32), 1e-6)
    assert np.allclose(y, 1.0, atol=1e-3)


def test_rms_norm_closed_form(oracle64):
    # x = [3, 4] -> rms = sqrt(12.5 + eps); weight applied per column.
    x = np.array([[3.0, 4.0]], np.float32)
    w = np.array([2.0, -1.0], np.float32)
    y = oracle64.rms_norm(x, w, 0.0)
    r = math.sqrt(12.5)
    assert np.allclose(y, [[6.0 / r, -4.0 / r]], rtol=1e-6)


def test_fused_adaln_chunk_order_and_gate(oracle64):
    # norm.rs:135-173 with zero up-projections (norm.rs:226-244 generalised): with x = ones
    # (x/rms = 1), h = 1 * (1 + raw_scale) + raw_shift and gate = tanh(raw_gate), where
    # (shift, scale, gate) are chunks 0, 1, 2 of cond.  Distinct chunk values pin the order.
    cfg = ih.DitConfig(latent_dim=4, model_dim=64, num_layers=1, num_heads=1, mlp_hidden=64,
                       adaln_rank=4, timestep_embed_dim=8)
    w = ih.DitWeights.random(cfg, 0)
    blk = w.blocks[0]
    for i in range(2):
        for ch in range(3):
            blk["ada_up"][i][ch][:] = 0
            blk["ada_up_b"][i][ch][:] = 0
    D = cfg.model_dim
    cond = np.concatenate([np.full(D, 0.25), np.full(D, -0.5), np.full(D, 0.5)]).astype(np.float32)[None]
    sh, sc, g = oracle64.adaln_vectors(cfg, blk, 0, cond)
    assert np.allclose(sh, 0.25) and np.allclose(sc, -0.5)
    assert np.allclose(g, math.tanh(0.5), atol=1e-7)
    h = oracle64.fused_adaln(np.ones((1, D), np.float32), sc, sh, 1, 1, 1e-12)
    assert np.allclose(h, 1.0 * (1 - 0.5) + 0.25, atol=1e-6)


def test_adaln_low_rank_residual_brute_force(oracle64):
    # shift = raw + up(down(silu(raw))) + b_up, checked against an f64 numpy loop.
    cfg = ih.DitConfig(latent_dim=4, model_dim=64, num_layers=1, num_heads=1, mlp_hidden=64,
                       adaln_rank=8, timestep_embed_dim=8)
    w = ih.DitWeights.random(cfg, 3, std=0.3)
    blk = w.blocks[0]
    rng = np.random.default_rng(0)
    cond = rng.standard_normal((2, 3 * 64)).astype(np.float32)
    outs = oracle64.adaln_vectors(cfg, blk, 1, cond)
    for ch in range(3):
        raw = cond[:, ch * 64:(ch + 1) * 64].astype(np.float64)
        silu = raw / (1 + np.exp(-raw))
        v = raw.copy()
        for b in range(2):
            mid = [sum(silu[b, d] * blk["ada_down"][1][ch][d, j] for d in range(64)) for j in range(8)]
            for n in range(64):
                v[b, n] += sum(mid[j] * blk["ada_up"][1][ch][j, n] for j in range(8)) + blk["ada_up_b"][1][ch][n]
        want = np.tanh(v) if ch == 2 else v
        assert np.allclose(outs[ch], want, rtol=1e-5, atol=1e-6)


# ---- RoPE / timestep embedding -----------------------------------------------------------
def test_rope_tables_closed_form(oracle64):
    cs, sn = oracle64.rope_tables(5, 64, 10000.0)
    s, i = np.meshgrid(np.arange(5), np.arange(32), indexing="ij")
    ang = s * 10000.0 ** (-2.0 * i / 64)
    assert np.allclose(cs, np.cos(ang), atol=1e-6) and np.allclose(sn, np.sin(ang), atol=1e-6)


def test_rope_position_zero_identity_and_passthrough(oracle64):
    # rope.rs:183 (pos 0 = identity) and :230 (heads >= H/2 untouched).
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 3, 4, 64)).astype(np.float32)
    cs, sn = oracle64.rope_tables(3, 64)
    y = oracle64.rope_half(x, cs, sn)
    assert np.array_equal(y[:, 0], x[:, 0])
    assert np.array_equal(y[:, :, 2:], x[:, :, 2:])
    assert not np.allclose(y[:, 1, :2], x[:, 1, :2])


def test_rope_sign_and_interleaved_pairs(oracle64):
    # Unit vector on the odd element of pair 0 at position 1 (angle 1 rad for k = 0):
    # complex (0 + 1i) * (cos1 + i sin1) = -sin1 + i cos1, landing on elements (0, 1).
    x = np.zeros((1, 2, 2, 64), np.float32)
    x[0, 1, 0, 1] = 1.0
    cs, sn = oracle64.rope_tables(2, 64)
    y = oracle64.rope_half(x, cs, sn)
    assert np.allclose(y[0, 1, 0, :2], [-math.sin(1.0), math.cos(1.0)], atol=1e-7)
    assert np.allclose(y[0, 1, 0, 2:], 0.0)


def test_rope_matches_complex_library_rotation(oracle64):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 7, 4, 64)).astype(np.float32)
    cs, sn = oracle64.rope_tables(7, 64)
    y = oracle64.rope_full(x, cs, sn)
    want = tref.rope(tref.T(x), tref.T(cs), tref.T(sn)).numpy()
    assert np.allclose(y, want, atol=1e-6)


def test_timestep_embedding(oracle64):
    # rope.rs:141-165: cos half first; t = 0 -> [1...1, 0...0].
    e0 = oracle64.timestep_embedding(np.zeros(1, np.float32), 8)
    assert np.array_equal(e0, [[1, 1, 1, 1, 0, 0, 0, 0]])
    t = np.array([0.37], np.float32)
    e = oracle64.timestep_embedding(t, 8)
    f = 1000.0 * np.exp(-np.log(10000.0) * np.arange(4) / 4)
    assert np.allclose(e[0, :4], np.cos(0.37 * f), atol=1e-5)
    assert np.allclose(e[0, 4:], np.sin(0.37 * f), atol=1e-5)


# ---- SwiGLU --------------------------------------------------------------------------------
def test_swiglu_zero_input(oracle32):
    # feed_forward.rs:157 (SwiGLU(0) = 0)
    rng = np.random.default_rng(0)
    w13 = rng.standard_normal((16, 64)).astype(np.float32)
    w2 = rng.standard_normal((32, 16)).astype(np.float32)
    assert np.array_equal(oracle32.swiglu(np.zeros((3, 16), np.float32), w13, w2), np.zeros((3, 16)))


def test_swiglu_gate_is_first_half(oracle64):
    # One-hot input selects row 0 of W13: u1 = a (W1 half), u3 = b (W3 half); with W2 = I
    # the output is silu(a) * b — swapping the halves would give silu(b) * a.
    Fh = 4
    w13 = np.zeros((2, 2 * Fh), np.float32)
    a = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    b = np.array([2.0, 1.0, -1.0, 0.25], np.float32)
    w13[0, :Fh], w13[0, Fh:] = a, b
    w2 = np.zeros((Fh, 2), np.float32)
    w2[0, 0] = w2[1, 1] = 1.0
    out = oracle64.swiglu(np.array([[1.0, 0.0]], np.float32), w13, w2)
    silu = a / (1 + np.exp(-a.astype(np.float64)))
    assert np.allclose(out[0], (silu * b)[:2], atol=1e-7)


# ---- SDPA ------------------------------------------------------------------------------------
def _ref_inputs(B, H, Sq, Skv, Dh):
    # Deterministic sin/cos inputs of the reference's kernel tests (fused_sdpa_native.rs:397-405).
    nq, nk = B * H * Sq * Dh, B * H * Skv * Dh
    q = (np.sin(np.arange(nq, dtype=np.float32) * 0.01) * 0.5).reshape(B, H, Sq, Dh)
    k = (np.cos(np.arange(nk, dtype=np.float32) * 0.013 + 1.0) * 0.5).reshape(B, H, Skv, Dh)
    v = (np.sin(np.arange(nk, dtype=np.float32) * 0.007 + 2.0) * 0.5).reshape(B, H, Skv, Dh)
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)


# Shapes of the reference's native FA tests (fused_sdpa_native.rs:465-611), incl. the
# non-divisible edge case and the masked case, plus the hot path's head_dim 64.
SDPA_CASES = [
    (1, 2, 4, 6, 128, None),
    (1, 2, 4, 8, 128, [1, 1, 1, 1, 1, 0, 0, 0]),
    (1, 16, 32, 48, 128, None),
    (1, 1, 17, 9, 128, None),
    (2, 3, 33, 70, 64, "random"),
]


@pytest.mark.parametrize("B,H,Sq,Skv,Dh,mask", SDPA_CASES)
def test_sdpa_matches_torch(oracle64, oracle32, B, H, Sq, Skv, Dh, mask):
    q, k, v = _ref_inputs(B, H, Sq, Skv, Dh)
    if mask is None:
        m = np.ones((B, Skv), np.float32)
    elif mask == "random":
        m = (np.random.default_rng(0).random((B, Skv)) > 0.4).astype(np.float32)
        m[:, 0] = 1
    else:
        m = np.tile(np.asarray(mask, np.float32), (B, 1))
    scale = Dh ** -0.5
    want = F.scaled_dot_product_attention(tref.T(q), tref.T(k), tref.T(v),
                                          attn_mask=(tref.T(m) > 0.5)[:, None, None, :]).numpy()
    assert np.allclose(oracle64.sdpa(q, k, v, m, scale), want, rtol=1e-6, atol=1e-8)  # f32 output rounding
    assert np.allclose(oracle32.sdpa(q, k, v, m, scale), want, atol=1e-5)  # reference tol 1e-5


def test_sdpa_all_masked_is_zero(oracle32):
    # attention.rs:770-787 (sdpa_all_masked_gives_zero)
    q = np.ones((1, 2, 3, 4), np.float32)
    k = np.ones((1, 2, 4, 4), np.float32)
    out = oracle32.sdpa(q, k, k, np.zeros((1, 4), np.float32), 0.5)
    assert np.array_equal(out, np.zeros_like(out))


def test_sdpa_masked_keys_values_irrelevant(oracle64):
    q, k, v = _ref_inputs(1, 2, 5, 12, 64)
    m = np.ones((1, 12), np.float32)
    m[0, 7:] = 0
    a = oracle64.sdpa(q, k, v, m, 0.125)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 7:] = 1e3
    v2[:, :, 7:] = -1e3
    assert np.array_equal(a, oracle64.sdpa(q, k2, v2, m, 0.125))


# ---- context KV cache --------------------------------------------------------------------
def test_build_kv_cache_matches_library(oracle64):
    # attention.rs:431-501: k = k_norm(text @ Wk_text) ++ k_norm(aux @ Wk_aux) (not rotated),
    # v = text @ Wv_text ++ aux @ Wv_aux, mask = text_mask ++ aux_mask.
    cfg = ih.cfg_tiny()
    H, Dh, HD = cfg.num_heads, cfg.head_dim, cfg.num_heads * cfg.head_dim
    rng = np.random.default_rng(5)
    text = rng.standard_normal((2, 5, 24)).astype(np.float32)
    aux = rng.standard_normal((2, 3, 16)).astype(np.float32)
    tm = np.array([[1, 1, 1, 0, 0], [1, 1, 1, 1, 1]], np.uint8)
    am = np.array([[1, 1, 1], [1, 0, 0]], np.uint8)
    wkt, wvt = (rng.standard_normal((24, HD)).astype(np.float32) for _ in range(2))
    wka, wva = (rng.standard_normal((16, HD)).astype(np.float32) for _ in range(2))
    kn = (1 + 0.1 * rng.standard_normal((H, Dh))).astype(np.float32)
    ck, cv, cm = oracle64.build_kv_cache(cfg, kn, text, tm, wkt, wvt, aux, am, wka, wva)
    def kproj(s, w):
        k = tref.lin(tref.T(s), w).reshape(s.shape[0], s.shape[1], H, Dh)
        return (k / tref.rms(k, cfg.norm_eps) * tref.T(kn)).numpy()
    assert np.allclose(ck, np.concatenate([kproj(text, wkt), kproj(aux, wka)], 1), atol=1e-9)
    vv = np.concatenate([(text.astype(np.float64) @ wvt), (aux.astype(np.float64) @ wva)], 1)
    assert np.allclose(cv, vv.reshape(cv.shape), atol=1e-9)
    assert np.array_equal(cm, np.concatenate([tm, am], 1))


# ---- whole model --------------------------------------------------------------------------
def _tiny_setup(seed=0, utter=1, S=16, tt=8, ts=8):
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, seed, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, utter, tt, ts, seed=seed + 1)
    x = ih.make_noise(2 * utter, S, cfg.latent_dim, seed + 2)
    return cfg, w, ctx, x


def test_forward_matches_torch_library_composition(oracle64, oracle32):
    cfg, w, ctx, x = _tiny_setup()
    t = np.array([0.8, 0.8], np.float32)
    v64, d64 = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    vt, dt = tref.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    # The f64 oracle keeps f32 storage between operators: agreement is at f32 rounding.
    assert rel_l2(d64, dt) < 1e-6
    assert rel_l2(v64, vt) < 1e-6
    v32 = oracle32.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask)
    assert rel_l2(v32, vt) < 1e-5


def test_forward_rows_independent(oracle32):
    # B=2 batched forward == two B=1 forwards (the property that makes the batched Joint
    # CFG forward equal to the reference's two sequential passes).
    cfg, w, ctx, x = _tiny_setup(seed=4)
    t = np.array([0.5, 0.5], np.float32)
    both = oracle32.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask)
    for r in range(2):
        c = ctx.rows([r])
        one = oracle32.forward(cfg, w, x[r:r + 1], t[r:r + 1], c.k, c.v, c.mask)
        assert rel_l2(one, both[r:r + 1]) < 1e-6


def test_sampler_constant_velocity_closed_form(oracle64):
    # out_proj weight = 0 => v == out_b for every row and step, so CFG combine gives out_b
    # and Euler telescopes: x_N = x_0 + out_b * (t_N - t_0) = x_0 - 0.999 * out_b.
    cfg, w, ctx, x = _tiny_setup(seed=6)
    w.io["out_w"][:] = 0
    x0 = x[:1]
    cond, unc = ctx.rows([0]), ctx.rows([1])
    out, run = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                         (unc.k, unc.v, unc.mask), 5, 3.0)
    assert run == 5
    assert np.allclose(out, x0 - 0.999 * w.io["out_b"][None, None, :], atol=1e-6)


def test_sampler_cfg_window_and_zero_scale(oracle64):
    # min_t > every t_i disables CFG (euler_sampler.rs:379): identical to scale 0.
    cfg, w, ctx, x = _tiny_setup(seed=7)
    x0 = x[:1]
    cond, unc = ctx.rows([0]), ctx.rows([1])
    a, _ = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                     (unc.k, unc.v, unc.mask), 3, 3.0, min_t=1.0, max_t=1.0)
    b, _ = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                     (unc.k, unc.v, unc.mask), 3, 0.0)
    assert np.array_equal(a, b)
    c, _ = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                     (unc.k, unc.v, unc.mask), 3, 3.0)
    assert rel_l2(c, b) > 1e-3


def test_sampler_one_step_is_cfg_euler(oracle64):
    # One step from t0 = 0.999 to t1 = 0: x1 = x0 + (v_c + s (v_c - v_u)) * (0 - 0.999),
    # with v_c / v_u the conditioned / unconditioned forwards at t0.
    cfg, w, ctx, x = _tiny_setup(seed=8)
    x0 = x[:1]
    cond, unc = ctx.rows([0]), ctx.rows([1])
    t = np.array([0.999], np.float32)
    vc = oracle64.forward(cfg, w, x0, t, cond.k, cond.v, cond.mask).astype(np.float64)
    vu = oracle64.forward(cfg, w, x0, t, unc.k, unc.v, unc.mask).astype(np.float64)
    out, _ = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                       (unc.k, unc.v, unc.mask), 1, 2.0)
    want = x0 + (vc + 2.0 * (vc - vu)) * (0.0 - 0.999)
    assert np.allclose(out, want, atol=1e-6)


# ---- latent key mask (build_joint_mask, attention.rs:730-750) ---------------------------

def _latent_mask(B, S, lengths, holes=()):
    m = np.zeros((B, S), np.uint8)
    for b, n in enumerate(lengths):
        m[b, :n] = 1
    for b, s in holes:
        m[b, s] = 0
    return m


def test_latent_mask_matches_torch_library(oracle64):
    # Masked latent keys via torch's scaled_dot_product_attention attn_mask (an independent
    # library route) — a dropped or inverted mask fails here.
    cfg, w, ctx, x = _tiny_setup(seed=11, S=24)
    t = np.array([0.7, 0.3], np.float32)
    m = _latent_mask(2, 24, [24, 17], holes=[(0, 3), (0, 20), (1, 5)])
    v64 = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, latent_mask=m)
    vt = tref.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, latent_mask=m)
    assert rel_l2(v64, vt) < 1e-6
    # and it changes the result (the mask is not ignored)
    v_nomask = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask)
    assert rel_l2(v64, v_nomask) > 1e-3


def test_latent_mask_equals_dropping_the_padding(oracle64):
    # A padded row with its padding masked equals the unpadded row on its valid frames:
    # masked keys contribute exp(-inf) = 0 exactly, every other operator is per frame.
    cfg, w, ctx, x = _tiny_setup(seed=12, S=24)
    t = np.array([0.6, 0.6], np.float32)
    n = 15
    m = _latent_mask(2, 24, [24, n])
    padded = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, latent_mask=m)
    c = ctx.rows([1])
    short = oracle64.forward(cfg, w, x[1:2, :n], t[1:2], c.k, c.v, c.mask)
    assert np.array_equal(padded[1:2, :n], short)


def test_sampler_latent_mask_equals_unpadded(oracle64):
    cfg, w, ctx, x = _tiny_setup(seed=13, S=20)
    cond, unc = ctx.rows([0]), ctx.rows([1])
    n = 13
    m = _latent_mask(1, 20, [n])
    x0 = x[:1]
    padded, _ = oracle64.sample_joint_cfg(cfg, w, x0, (cond.k, cond.v, cond.mask),
                                          (unc.k, unc.v, unc.mask), 4, 2.0, latent_mask=m)
    short, _ = oracle64.sample_joint_cfg(cfg, w, x0[:, :n], (cond.k, cond.v, cond.mask),
                                         (unc.k, unc.v, unc.mask), 4, 2.0)
    assert np.array_equal(padded[:, :n], short)
