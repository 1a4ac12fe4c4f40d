"""GPU parity of the DiT path with 128-dim attention heads (the reference's default
ModelConfig: d 2048, 16 heads of 128, latent 128; config/model.rs:46-82, head_dim :226-228)
against the CPU oracle, through the C ABI on seeded inputs and random-init weights.

128-dim heads take the QKV+gate GEMM with 4 x 1 waves (one whole head per wave: head
RMSNorm over 128 columns, half RoPE, V^T in the 16x16 attention's key order), the 16x16
joint attention with 128-dim fragments, and the same 4 x 1 tile for the context-KV build.

Bars as in test_gpu_model.py: f32 1e-4 relative L2 per block and on the sampled latent,
bf16 1e-2 per block and 2e-2 on the sampled latent; context K / V as in
test_gpu_ctx_build.py (f32 1e-5, bf16 1e-2).
"""
import dataclasses

import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2
from test_gpu_ctx_build import build_rows, check_readback, oracle_ctx, states
from test_gpu_model import TOL_BLOCK, TOL_FINAL, joint_params, make_engine

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32


def cfg_dh128_tiny():
    # d 256 = 2 heads of 128 (head 0 rotated, head 1 not); fused adaLN on the bf16 path.
    return dataclasses.replace(ih.cfg_tiny(), model_dim=256, num_heads=2, mlp_hidden=512)


def cfg_dh128_h3():
    # 3 heads of 128 (D = 384): only head 0 rotates; the q / k boundary falls inside a tile.
    return dataclasses.replace(ih.cfg_tiny(), model_dim=384, num_heads=3, mlp_hidden=640)


def cfg_reference_default(layers=2):
    # The reference's default DiT width (d 2048, 16 x 128 heads, SwiGLU 2048 * 2.875 = 5888,
    # latent 128, adaLN rank 256, timestep embedding 512, eps 1e-5) with `layers` layers.
    return dataclasses.replace(ih.cfg_full_rf(), latent_dim=128, model_dim=2048, num_layers=layers, num_heads=16,
                               mlp_hidden=5888, adaln_rank=256, timestep_embed_dim=512, norm_eps=1e-5)


def cfg_d4096(layers=1):
    # Wider than the reference's default: d 4096 = 32 x 128 heads, SwiGLU 4096 * 2.875 (the
    # unfused adaLN, 16 float4 chunks per lane in its norm kernel; the output head stages at
    # most six rows).
    return dataclasses.replace(cfg_reference_default(layers), model_dim=4096, num_heads=32, mlp_hidden=11776)


CASES = {
    # name: (cfg factory, seq, text, speaker, weight std, norm jitter)
    "tiny": (cfg_dh128_tiny, 40, 20, 13, 0.05, 0.1),
    "tiny_odd": (cfg_dh128_tiny, 37, 11, 9, 0.05, 0.1),
    "h3": (cfg_dh128_h3, 40, 20, 13, 0.05, 0.1),
    "ref_default": (cfg_reference_default, 48, 16, 20, 0.02, 0.05),
    "d4096": (cfg_d4096, 24, 8, 9, 0.02, 0.05),
    # 512 frames: the output head takes two frames per block (enough blocks to fill the chip)
    "d4096_s512": (cfg_d4096, 512, 8, 9, 0.02, 0.05),
}


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(CASES))
def test_forward_per_block_dh128(oracle64, oracle32, name, backend):
    make_cfg, S, tt, ts, std, jit = CASES[name]
    if name == "d4096_s512":
        oracle64 = oracle32  # 1024 rows at d 4096: the f32 oracle (per-block bars unchanged)
    cfg = make_cfg()
    assert cfg.head_dim == 128
    w = ih.DitWeights.random(cfg, 0, std=std, norm_jitter=jit)
    ctx = ih.make_context_kv(cfg, 1, tt, ts, seed=1)
    x = ih.make_noise(2, S, cfg.latent_dim, 2)
    t = np.array([0.9, 0.35], np.float32)
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    print(name, backend.value, "per-block rel L2:", ["%.2e" % a for a in errs], "v: %.2e" % rel_l2(v, v_ref))
    assert max(errs) < TOL_BLOCK[backend]
    assert rel_l2(v, v_ref) < TOL_BLOCK[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", ["tiny", "ref_default", "d4096"])
def test_sample_joint_cfg_dh128(oracle64, name, backend):
    # 4 Euler steps of Joint CFG (scale 3) through the captured step graphs.
    make_cfg, S, tt, ts, std, jit = CASES[name]
    cfg = make_cfg()
    w = ih.DitWeights.random(cfg, 0, std=std, norm_jitter=jit)
    ctx = ih.make_context_kv(cfg, 1, tt, ts, seed=1)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 2)
    p = joint_params(4)
    with make_engine(cfg, backend, w, ctx, 2, S) as e:
        got = e.sample(x0, p)
        again = e.sample(x0, p)
    c, u = ctx.rows([0]), ctx.rows([1])
    ref, _ = oracle64.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 4, 3.0)
    print(name, backend.value, "final rel L2 %.2e" % rel_l2(got, ref))
    assert rel_l2(got, ref) < TOL_FINAL[backend]
    assert np.array_equal(got, again)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_context_kv_build_dh128(oracle64, backend):
    # The device context-KV build with 128-dim heads (ragged input dims 40 / 72 padded on
    # the device, an unconditioned second row), read back and attended to.
    tol_kv = {BF16: 1e-2, F32: 1e-5}
    cfg = cfg_dh128_tiny()
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    proj = ih.CtxProjWeights.random(cfg, 40, 72, seed=4, std=0.1)
    rng = np.random.default_rng(5)
    text, tm = states(rng, 10, 40, 7)
    aux, am = states(rng, 9, 72, 9)
    rows = [(text, tm, aux, am),
            (np.zeros_like(text), np.zeros_like(tm), np.zeros_like(aux), np.zeros_like(am))]
    ref = oracle_ctx(oracle64, cfg, w, proj, rows)
    S = 40
    x = ih.make_noise(2, S, cfg.latent_dim, 6)
    t = np.array([0.8, 0.8], np.float32)
    with ih.HipInferenceEngine(cfg, backend, max_rows=2, max_seq=S, max_ctx=19) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        build_rows(e, rows)
        for l in range(cfg.num_layers):
            k, v, m = e.read_context_kv(l, 0, ref.t_ctx)
            assert rel_l2(k, ref.k[l, 0]) < tol_kv[backend] and rel_l2(v, ref.v[l, 0]) < tol_kv[backend]
        check_readback(e, cfg, ref, backend)
        v_dev, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ref.k, ref.v, ref.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    assert max(errs) < TOL_BLOCK[backend], errs
    assert rel_l2(v_dev, v_ref) < TOL_BLOCK[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_speaker_kv_scaling_dh128(oracle64, backend):
    # Speaker-KV scaling of the aux keys in the first layer, reverted below t = 0.6, with
    # 128-dim heads (the device copies of K and of V^T in the 16x16 attention's key order).
    from test_gpu_sampler import orc_params, params
    cfg = cfg_dh128_tiny()
    w = ih.DitWeights.random(cfg, 21, std=0.05, norm_jitter=0.1)
    TT, TA, S = 10, 9, 24
    skv = ih.config.SpeakerKvConfig(scale=1.8, max_layers=1, min_t=0.6)
    p = params(ih.CfgGuidanceMode.JOINT, ih.SamplerMethod.EULER, steps=4, speaker_kv=skv)
    roles = p.cfg_roles(has_speaker=True)
    ctx = ih.make_role_context(cfg, 1, TT, TA, roles, seed=3)
    x0 = ih.make_noise(1, S, cfg.latent_dim, 4)
    with ih.HipInferenceEngine(cfg, backend, max_rows=len(roles), max_seq=S, max_ctx=ctx.t_ctx) as e:
        e.load_weights(w)
        e.set_context_kv(ctx)
        got = e.sample(x0, p, ctx_aux_start=TT)
        plain = e.sample(x0, params(ih.CfgGuidanceMode.JOINT, ih.SamplerMethod.EULER, steps=4), ctx_aux_start=TT)
    ref, _ = oracle64.sample_rf(cfg, w, x0, (ctx.k, ctx.v, ctx.mask), orc_params(p, aux_start=TT))
    assert rel_l2(got, ref) < TOL_FINAL[backend]
    assert rel_l2(got, plain) > 1e-4


def test_dh128_refusals():
    # fp8 compute keeps 64-dim heads (refused at create); the isolated joint-attention
    # operator stages 64-dim heads only (refused at the call, not at launch).
    cfg = cfg_dh128_tiny()
    with pytest.raises(ih.IrodoriError):
        ih.HipInferenceEngine(cfg, ih.InferenceBackendKind.HIP_FP8, max_rows=2, max_seq=16, max_ctx=8)
    w = ih.DitWeights.random(cfg, 0, std=0.05)
    ctx = ih.make_context_kv(cfg, 1, 5, 3, seed=1)
    import torch
    with make_engine(cfg, BF16, w, ctx, 2, 16) as e:
        buf = torch.zeros(2 * 16 * cfg.model_dim, dtype=torch.float32, device="cuda")
        p = buf.data_ptr()
        with pytest.raises(ih.IrodoriError):
            e.joint_attention(0, 2, 16, p, p, p, p, p)
        torch.cuda.synchronize()
