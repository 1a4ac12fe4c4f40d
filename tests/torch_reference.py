"""Independent restatement of the RF-step DiT forward with torch.nn.functional library
routines (F.linear, F.silu, F.scaled_dot_product_attention, torch.tanh/sigmoid/rsqrt),
in float64 on the CPU.  Test infrastructure: it pins the C oracle's composition (index
order, transposes, chunk order, mask polarity) against code that shares none of its
loops.  Follows the reference's structure: src/model/dit/model.rs:354-393 (backbone),
src/model/diffusion.rs:62-105 (block), src/model/attention.rs:272-425 (joint attention),
src/model/norm.rs:25-173, src/model/rope.rs:24-165, src/model/feed_forward.rs:76-85.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

DT = torch.float64


def T(a):
    return torch.as_tensor(np.asarray(a), dtype=DT)


def lin(x, w, b=None):
    # Burn row layout w [d_in, d_out]: y = x @ w + b == F.linear(x, w^T, b)
    return F.linear(x, T(w).t(), None if b is None else T(b))


def rms(x, eps):
    return torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def timestep_embedding(t, dim):
    half = dim // 2
    i = torch.arange(half, dtype=DT)
    f = 1000.0 * torch.exp(-math.log(10000.0) * i / half)
    a = T(t)[:, None] * f[None]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=1)


def rope_tables(S, Dh, theta=10000.0):
    half = Dh // 2
    freq = 1.0 / theta ** (2.0 * torch.arange(half, dtype=DT) / Dh)
    ang = torch.arange(S, dtype=DT)[:, None] * freq[None]
    return torch.cos(ang), torch.sin(ang)


def rope(x, cos, sin):
    # x [B, S, H, Dh]: complex rotation of interleaved pairs via torch.view_as_complex.
    B, S, H, Dh = x.shape
    xc = torch.view_as_complex(x.reshape(B, S, H, Dh // 2, 2).contiguous())
    rot = torch.polar(torch.ones_like(cos), torch.atan2(sin, cos))  # cos + i sin
    y = xc * rot[None, :, None, :]
    return torch.view_as_real(y).reshape(B, S, H, Dh)


def adaln(x, cond_chunks, blk, which, eps):
    outs = []
    for ch in range(3):
        raw = cond_chunks[ch]
        v = lin(lin(F.silu(raw), blk["ada_down"][which][ch]), blk["ada_up"][which][ch],
                blk["ada_up_b"][which][ch]) + raw
        outs.append(v)
    shift, scale, gate = outs
    h = x / rms(x, eps) * (1 + scale[:, None, :]) + shift[:, None, :]
    return h, torch.tanh(gate)[:, None, :]


def joint_attention(h, blk, ctx_k, ctx_v, ctx_mask, cos, sin, H, Dh, eps, latent_mask=None):
    B, S, D = h.shape
    HD = H * Dh
    qkv = lin(h, blk["w_qkv"])
    q, k, v = qkv[..., :HD], qkv[..., HD:2 * HD], qkv[..., 2 * HD:]
    q = q.reshape(B, S, H, Dh)
    k = k.reshape(B, S, H, Dh)
    v = v.reshape(B, S, H, Dh)
    qn = T(blk["q_norm"])
    kn = T(blk["k_norm"])
    q = q / rms(q, eps) * qn
    k = k / rms(k, eps) * kn
    hh = H // 2
    q = torch.cat([rope(q[:, :, :hh], cos, sin), q[:, :, hh:]], dim=2)
    k = torch.cat([rope(k[:, :, :hh], cos, sin), k[:, :, hh:]], dim=2)
    K = torch.cat([k, T(ctx_k)], dim=1).transpose(1, 2)
    V = torch.cat([v, T(ctx_v)], dim=1).transpose(1, 2)
    lat = torch.ones(B, S, dtype=torch.bool) if latent_mask is None else T(latent_mask) > 0
    valid = torch.cat([lat, T(ctx_mask) > 0], dim=1)
    o = F.scaled_dot_product_attention(q.transpose(1, 2), K, V,
                                       attn_mask=valid[:, None, None, :])
    o = o.transpose(1, 2).reshape(B, S, HD)
    return lin(torch.sigmoid(lin(h, blk["w_gate"])) * o, blk["w_o"])


def swiglu(h, w13, w2):
    Fh = np.asarray(w2).shape[0]
    u = lin(h, w13)
    return lin(F.silu(u[..., :Fh]) * u[..., Fh:], w2)


def forward(cfg, weights, x_t, t, ctx_k, ctx_v, ctx_mask, debug=False, latent_mask=None):
    io = weights.io
    D, H, Dh, eps = cfg.model_dim, cfg.num_heads, cfg.head_dim, cfg.norm_eps
    x_t = T(x_t)
    B, S, _ = x_t.shape
    cos, sin = rope_tables(S, Dh, cfg.rope_theta)
    c = lin(F.silu(lin(F.silu(lin(timestep_embedding(t, cfg.timestep_embed_dim), io["cond_w0"])),
                       io["cond_w1"])), io["cond_w2"])
    chunks = [c[:, 0:D], c[:, D:2 * D], c[:, 2 * D:3 * D]]
    x = lin(x_t, io["in_w"], io["in_b"])
    outs = [x.clone()]
    for l, blk in enumerate(weights.blocks):
        h1, g1 = adaln(x, chunks, blk, 0, eps)
        x = x + g1 * joint_attention(h1, blk, ctx_k[l], ctx_v[l], ctx_mask, cos, sin, H, Dh, eps,
                                     latent_mask)
        h2, g2 = adaln(x, chunks, blk, 1, eps)
        x = x + g2 * swiglu(h2, blk["w13"], blk["w2"])
        outs.append(x.clone())
    v = lin(x / rms(x, eps) * T(io["out_norm_w"]), io["out_w"], io["out_b"])
    if debug:
        return v.numpy(), torch.stack(outs).numpy()
    return v.numpy()


# ---- condition encoders (text_encoder.rs:17-148, speaker_encoder.rs:85-162,
# attention.rs:52-127, aux_conditioner.rs:150-185) ------------------------------------------
def text_block(x, blk, mask, cos, sin, H, eps):
    B, S, E = x.shape
    Dh = E // H
    h = x / rms(x, eps) * T(blk["attn_norm"])
    q = lin(h, blk["wq"]).reshape(B, S, H, Dh)
    k = lin(h, blk["wk"]).reshape(B, S, H, Dh)
    v = lin(h, blk["wv"]).reshape(B, S, H, Dh)
    q = rope(q / rms(q, eps) * T(blk["q_norm"]), cos, sin)
    k = rope(k / rms(k, eps) * T(blk["k_norm"]), cos, sin)
    valid = T(mask) > 0
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                       attn_mask=valid[:, None, None, :])
    o = torch.nan_to_num(o)  # a row with no valid key: 0 (attention.rs:686-716)
    o = o.transpose(1, 2).reshape(B, S, E)
    x = x + lin(torch.sigmoid(lin(h, blk["w_gate"])) * o, blk["wo"])
    h2 = x / rms(x, eps) * T(blk["mlp_norm"])
    return x + swiglu(h2, blk["w13"], blk["w2"])


def encoder_forward(ecfg, ew, mask, ids=None, latent=None):
    m = T(mask)[..., None]
    if ids is not None:
        x = T(ew.io["embedding"])[torch.as_tensor(np.asarray(ids), dtype=torch.long)]
    else:
        x = lin(T(latent), ew.io["in_w"], ew.io["in_b"]) / 6.0
    x = x * m
    S = x.shape[1]
    cos, sin = rope_tables(S, ecfg.dim // ecfg.num_heads)
    for blk in ew.blocks:
        x = text_block(x, blk, mask, cos, sin, ecfg.num_heads, ecfg.norm_eps) * m
    st = x / rms(x, ecfg.norm_eps) * T(ew.io["out_norm"])
    mo = torch.as_tensor(np.asarray(mask, np.uint8))
    if ecfg.mean_token:
        cnt = m.sum(1, keepdim=True)
        mean = (st * m).sum(1, keepdim=True) / cnt.clamp(min=1.0)
        st = torch.cat([mean, st], 1)
        mo = torch.cat([(cnt[:, 0, 0] > 0).to(torch.uint8)[:, None], mo], 1)
    return st.numpy(), mo.numpy()


# ---- DACVAE decoder (codec/model.rs:60-65, decoder.rs, layers.rs, bottleneck.rs) ----------
def snake(x, alpha):
    a = T(alpha)[None, :, None]
    return x + torch.sin(a * x).pow(2) / (a + 1e-9)


def _b(v):
    return None if v is None else T(v)


def codec_decode(ccfg, cw, latent):
    """latent [B, T, latent_dim] -> wav [B, 1, T * hop] with F.conv1d / F.conv_transpose1d
    (PyTorch's ConvTranspose1d padding rule of layers.rs:62-65)."""
    x = T(latent).transpose(1, 2)
    io = cw.io
    x = F.conv1d(x, T(io["out_proj_w"]), _b(io["out_proj_b"]))
    x = F.conv1d(x, T(io["stem_w"]), _b(io["stem_b"]), padding=3)
    for blk, r in zip(cw.blocks, ccfg.rates):
        x = snake(x, blk["alpha"])
        x = F.conv_transpose1d(x, T(blk["convt_w"]), _b(blk["convt_b"]), stride=r, padding=(r + 1) // 2,
                               output_padding=r % 2)
        for u, d in enumerate((1, 3, 9)):
            y = snake(x, blk["res_alpha0"][u])
            y = F.conv1d(y, T(blk["res_conv_w"][u]), _b(blk["res_conv_b"][u]), padding=3 * d, dilation=d)
            y = snake(y, blk["res_alpha1"][u])
            y = F.conv1d(y, T(blk["res_pw_w"][u]), _b(blk["res_pw_b"][u]))
            x = x + y
    x = snake(x, io["head_alpha"])
    return torch.tanh(F.conv1d(x, T(io["head_w"]), _b(io["head_b"]), padding=3)).numpy()
