"""The block's hot kernels in isolation (irodori_op_joint_attention / irodori_op_swiglu_mlp)
at the isolated-kernel configurations, through the C ABI, against oracle compositions of
the pinned operators (head RMSNorm, half RoPE, SDPA with the joint key mask, adaLN,
SwiGLU) in float64.

- Joint attention, B = 2 x 16 heads x 64, 750 latent queries; keys = 750 latent (RoPE'd
  and head-normed with the layer's weights) + 256 text (valid length U[32, 256] per row) +
  375 speaker, Q/K/V ~ N(0, 1), sigmoid output gate (attention.rs:328-425).
- SwiGLU MLP half of a block, 1500 tokens (B = 2 x 750) x 1024 -> 2816 -> 1024, weights
  N(0, 0.02), activations N(0, 1), shift / scale / gate per batch row ~ N(0, 0.1), RMSNorm
  eps 1e-6 (diffusion.rs:101-104).
Bars: f32 1e-4 relative L2; bf16 1e-2 (the MLP's increment on its own 2e-2).
"""
import dataclasses

import numpy as np
import pytest
import torch

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL = {BF16: 1e-2, F32: 1e-4}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda")


def one_layer(eps=1e-5):
    return dataclasses.replace(ih.cfg_full_rf(), num_layers=1, norm_eps=eps)


def joint_attention_ref(orc, cfg, blk, q, k, v, gate, ck, cv, cmask):
    """attention.rs:328-425 composed from the oracle's pinned operators."""
    B, S, H, Dh = q.shape
    qn = orc.head_rms_norm(q, blk["q_norm"], cfg.norm_eps)
    kn = orc.head_rms_norm(k, blk["k_norm"], cfg.norm_eps)
    cs, sn = orc.rope_tables(S, Dh, cfg.rope_theta)
    qr, kr = orc.rope_half(qn, cs, sn), orc.rope_half(kn, cs, sn)
    K = np.concatenate([kr, ck], axis=1).transpose(0, 2, 1, 3)
    V = np.concatenate([v, cv], axis=1).transpose(0, 2, 1, 3)
    mask = np.concatenate([np.ones((B, S), np.float32), cmask.astype(np.float32)], axis=1)
    o = orc.sdpa(qr.transpose(0, 2, 1, 3), K, V, mask, Dh ** -0.5).transpose(0, 2, 1, 3)
    g = 1.0 / (1.0 + np.exp(-gate.astype(np.float64)))
    return (o.reshape(B, S, H * Dh) * g).astype(np.float64)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("roles", [["cond"], ["cond", "uncond"]], ids=["two-utterances", "cond+uncond"])
def test_joint_attention_op_config2(oracle64, backend, roles):
    cfg = one_layer()
    w = ih.DitWeights.random(cfg, 7, norm_jitter=0.1)
    U = 2 if roles == ["cond"] else 1
    ctx = ih.make_role_context(cfg, U, 256, 375, roles, seed=8)  # 2 rows either way
    B, S, H, Dh = 2, 750, cfg.num_heads, cfg.head_dim
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((B, S, H, Dh)).astype(np.float32) for _ in range(3))
    gate = rng.standard_normal((B, S, H * Dh)).astype(np.float32)
    out = torch.empty((B, S, H * Dh), dtype=torch.float32, device="cuda")
    with ih.HipInferenceEngine(cfg, backend, max_rows=B, max_seq=S, max_ctx=ctx.t_ctx) as e:
        e.load_weights(w)
        e.set_context_kv(ctx)
        dq, dk, dv, dg = dev(q), dev(k), dev(v), dev(gate)
        e.joint_attention(0, B, S, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), out.data_ptr())
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        # No gate: sigmoid(gate) replaced by 1.
        e.joint_attention(0, B, S, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), 0, out.data_ptr())
        torch.cuda.synchronize()
        got_ng = out.cpu().numpy()
    ref = joint_attention_ref(oracle64, cfg, w.blocks[0], q, k, v, gate, ctx.k[0], ctx.v[0], ctx.mask)
    ref_ng = joint_attention_ref(oracle64, cfg, w.blocks[0], q, k, v, np.full_like(gate, 60.0), ctx.k[0],
                                 ctx.v[0], ctx.mask)
    err, err_ng = rel_l2(got, ref), rel_l2(got_ng, ref_ng)
    print(backend.value, roles, "joint attention op rel L2 %.2e / ungated %.2e" % (err, err_ng))
    assert err < TOL[backend] and err_ng < TOL[backend]


def test_joint_attention_op_rejects_missing_context():
    cfg = one_layer()
    with ih.HipInferenceEngine(cfg, BF16, max_rows=2, max_seq=64, max_ctx=16) as e:
        e.load_weights(ih.DitWeights.random(cfg, 1))
        ctx = ih.make_context_kv(cfg, 1, 8, 8, seed=2)
        e.set_context_kv(ih.ContextKV(ctx.k[:, :1], ctx.v[:, :1], ctx.mask[:1]))  # row 0 only
        z = torch.zeros((2, 64, cfg.model_dim), device="cuda")
        with pytest.raises(ih.IrodoriError) as ei:
            e.joint_attention(0, 2, 64, z.data_ptr(), z.data_ptr(), z.data_ptr(), 0, z.data_ptr())
        assert ei.value.kind == "NotLoaded"


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("B", [2, 1])
def test_swiglu_mlp_op_config3(oracle64, backend, B):
    cfg = one_layer(eps=1e-6)
    w = ih.DitWeights.random(cfg, 3)
    S, D = 750, cfg.model_dim
    rng = np.random.default_rng(4)
    x = rng.standard_normal((B, S, D)).astype(np.float32)
    shift, scale, gate = ((0.1 * rng.standard_normal((B, D))).astype(np.float32) for _ in range(3))
    # Keep every device tensor referenced until the call completes (a temporary's block
    # would go back to torch's cache and be handed to the next allocation).
    dx, dsh, dsc, dg = dev(x), dev(shift), dev(scale), dev(gate)
    with ih.HipInferenceEngine(cfg, backend, max_rows=B, max_seq=S, max_ctx=1) as e:
        e.load_weights(w)
        e.swiglu_mlp(0, B, S, dx.data_ptr(), dsh.data_ptr(), dsc.data_ptr(), dg.data_ptr())
        torch.cuda.synchronize()
    got = dx.cpu().numpy()
    h = oracle64.fused_adaln(x.reshape(B * S, D), scale, shift, B, S, 1e-6)
    m = oracle64.swiglu(h, w.blocks[0]["w13"], w.blocks[0]["w2"]).reshape(B, S, D).astype(np.float64)
    ref = x + gate[:, None, :].astype(np.float64) * m
    err, inc = rel_l2(got, ref), rel_l2(got - x, ref - x)
    print(backend.value, "B=%d swiglu mlp op rel L2 %.2e, increment %.2e" % (B, err, inc))
    assert err < TOL[backend] and inc < 2 * TOL[backend]
