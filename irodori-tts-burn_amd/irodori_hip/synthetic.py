"""Seeded synthetic inputs for the RF-step DiT: random-init weights, context KV, noise.

The reference's random-init constructors zero out_proj and every adaLN up-projection
(src/model/dit/model.rs:28-43, src/model/norm.rs:107-119), which would make v == 0; the
benchmark configurations instead draw EVERY Linear weight and bias from N(0, std) and
set norm weights to 1 (optionally 1 + N(0, norm_jitter) so tests see the norm weights).
Arrays are float32 in Burn row layout [d_in, d_out] (src/weights/record_builders.rs:37-66).
Draw order is fixed, so a (cfg, seed) pair always yields the same arrays.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .config import DitConfig


class _Draw:
    def __init__(self, seed: int, std: float, norm_jitter: float):
        self.rng = np.random.default_rng(seed)
        self.std = np.float32(std)
        self.jit = np.float32(norm_jitter)

    def lin(self, *shape):
        return (self.rng.standard_normal(shape, dtype=np.float32) * self.std).astype(np.float32)

    def norm(self, *shape):
        w = np.ones(shape, np.float32)
        if self.jit:
            w += self.rng.standard_normal(shape, dtype=np.float32) * self.jit
        return w


@dataclass
class DitWeights:
    io: dict
    blocks: list

    @staticmethod
    def random(cfg: DitConfig, seed: int = 0, std: float = 0.02,
               norm_jitter: float = 0.0) -> "DitWeights":
        d = _Draw(seed, std, norm_jitter)
        D, P, F, r, H, Dh = (cfg.model_dim, cfg.latent_dim, cfg.mlp_hidden, cfg.adaln_rank,
                             cfg.num_heads, cfg.head_dim)
        HD = H * Dh
        io = {
            "cond_w0": d.lin(cfg.timestep_embed_dim, D),
            "cond_w1": d.lin(D, D),
            "cond_w2": d.lin(D, 3 * D),
            "in_w": d.lin(P, D),
            "in_b": d.lin(D),
            "out_norm_w": d.norm(D),
            "out_w": d.lin(D, P),
            "out_b": d.lin(P),
        }
        blocks = []
        for _ in range(cfg.num_layers):
            b = {
                "w_qkv": d.lin(D, 3 * HD),
                "w_gate": d.lin(D, D),
                "w_o": d.lin(HD, D),
                "q_norm": d.norm(H, Dh),
                "k_norm": d.norm(H, Dh),
                "w13": d.lin(D, 2 * F),
                "w2": d.lin(F, D),
                "ada_down": [[d.lin(D, r) for _ in range(3)] for _ in range(2)],
                "ada_up": [[d.lin(r, D) for _ in range(3)] for _ in range(2)],
                "ada_up_b": [[d.lin(D) for _ in range(3)] for _ in range(2)],
            }
            blocks.append(b)
        return DitWeights(io, blocks)

    def nbytes(self) -> int:
        n = sum(a.nbytes for a in self.io.values())
        for b in self.blocks:
            for k, v in b.items():
                if isinstance(v, list):
                    n += sum(x.nbytes for row in v for x in row)
                else:
                    n += v.nbytes
        return n


@dataclass
class EncoderWeights:
    """Weights of a condition encoder (EncoderConfig), Burn [d_in, d_out] layouts:
    io: embedding [vocab, E] (token input) or in_w [in_dim, E] + in_b [E] (latent input),
    out_norm [E] (the conditioner norm); blocks: per TextBlock attn_norm, wq / wk / wv
    [E, E], wo [E, E], w_gate [E, E], q_norm / k_norm [H, Dh], mlp_norm, w13 [E, 2F] =
    [W1 | W3], w2 [F, E]."""

    io: dict
    blocks: list

    @staticmethod
    def random(cfg, seed: int = 0, std: float = 0.02, norm_jitter: float = 0.0) -> "EncoderWeights":
        d = _Draw(seed, std, norm_jitter)
        E, F, H, Dh = cfg.dim, cfg.mlp_hidden, cfg.num_heads, cfg.head_dim
        io = {}
        if cfg.vocab_size:
            io["embedding"] = d.rng.standard_normal((cfg.vocab_size, E), dtype=np.float32)
        if cfg.in_dim:
            io["in_w"] = d.lin(cfg.in_dim, E)
            io["in_b"] = d.lin(E)
        io["out_norm"] = d.norm(E)
        blocks = []
        for _ in range(cfg.num_layers):
            blocks.append({
                "attn_norm": d.norm(E), "wq": d.lin(E, E), "wk": d.lin(E, E), "wv": d.lin(E, E),
                "wo": d.lin(E, E), "w_gate": d.lin(E, E), "q_norm": d.norm(H, Dh),
                "k_norm": d.norm(H, Dh), "mlp_norm": d.norm(E), "w13": d.lin(E, 2 * F),
                "w2": d.lin(F, E),
            })
        return EncoderWeights(io, blocks)


@dataclass
class CtxProjWeights:
    """Per-layer context projections of JointAttention (attention.rs:142-147): wk_text /
    wv_text [text_dim, H*Dh] and, when aux_dim > 0, wk_aux / wv_aux [aux_dim, H*Dh] (the
    speaker or caption pair), Burn row layout, no bias."""

    layers: list
    text_dim: int
    aux_dim: int

    @staticmethod
    def random(cfg: DitConfig, text_dim: int, aux_dim: int, seed: int = 0,
               std: float = 0.02) -> "CtxProjWeights":
        d = _Draw(seed, std, 0.0)
        HD = cfg.num_heads * cfg.head_dim
        layers = []
        for _ in range(cfg.num_layers):
            w = {"wk_text": d.lin(text_dim, HD), "wv_text": d.lin(text_dim, HD)}
            if aux_dim:
                w["wk_aux"] = d.lin(aux_dim, HD)
                w["wv_aux"] = d.lin(aux_dim, HD)
            layers.append(w)
        return CtxProjWeights(layers, text_dim, aux_dim)


@dataclass
class ContextKV:
    """Per-layer cached context K/V for every batch row (CondKvCache, attention.rs:24-45):
    k, v [L, B, T, H, Dh] (k already k-normed, not rotated), mask [B, T] (1 = attend)."""

    k: np.ndarray
    v: np.ndarray
    mask: np.ndarray

    @property
    def t_ctx(self) -> int:
        return self.k.shape[2]

    def rows(self, idx) -> "ContextKV":
        return ContextKV(np.ascontiguousarray(self.k[:, idx]), np.ascontiguousarray(self.v[:, idx]),
                         np.ascontiguousarray(self.mask[idx]))


# Context bundles of the CFG roles (euler_sampler.rs:41-85, condition.rs:144-154): the
# conditioned bundle, the fully unconditioned one (Joint), and the bundles with the text or
# the aux (speaker / caption) signal dropped.  A dropped signal has zero states, which
# project to zero K/V, and every one of its keys masked out.
ROLE_COND, ROLE_UNCOND, ROLE_NO_TEXT, ROLE_NO_AUX = "cond", "uncond", "no_text", "no_aux"


def make_role_context(cfg: DitConfig, utterances: int, t_text: int, t_aux: int, roles,
                      seed: int = 1, text_valid=None, kv_std: float = 1.0) -> ContextKV:
    """Synthetic cached context for the CFG roles of `utterances` utterances, role-major:
    role r of utterance u is row r * U + u (the row layout of irodori_sample).

    Utterance u draws text and aux K/V ~ N(0, kv_std) once; its text keys are valid up to
    a per-utterance length (default uniform in [min(32, t_text), t_text]) and its aux keys
    are all valid.  Each role keeps or drops the two segments (see the ROLE_* names)."""
    rng = np.random.default_rng(seed)
    L, H, Dh = cfg.num_layers, cfg.num_heads, cfg.head_dim
    T, U, R = t_text + t_aux, utterances, len(roles)
    k = np.zeros((L, R * U, T, H, Dh), np.float32)
    v = np.zeros_like(k)
    mask = np.zeros((R * U, T), np.uint8)
    for u in range(U):
        ku = rng.standard_normal((L, T, H, Dh), dtype=np.float32) * np.float32(kv_std)
        vu = rng.standard_normal((L, T, H, Dh), dtype=np.float32) * np.float32(kv_std)
        if text_valid is not None:
            tv = int(text_valid[u])
        else:
            tv = int(rng.integers(min(32, t_text), t_text + 1)) if t_text > 0 else 0
        for r, role in enumerate(roles):
            row = r * U + u
            keep_text = role in (ROLE_COND, ROLE_NO_AUX)
            keep_aux = role in (ROLE_COND, ROLE_NO_TEXT)
            if role not in (ROLE_COND, ROLE_UNCOND, ROLE_NO_TEXT, ROLE_NO_AUX):
                raise ValueError("unknown role %r" % (role,))
            if keep_text:
                k[:, row, :t_text] = ku[:, :t_text]
                v[:, row, :t_text] = vu[:, :t_text]
                mask[row, :tv] = 1
            if keep_aux:
                k[:, row, t_text:] = ku[:, t_text:]
                v[:, row, t_text:] = vu[:, t_text:]
                mask[row, t_text:] = 1
    return ContextKV(k, v, mask)


def make_context_kv(cfg: DitConfig, utterances: int, t_text: int, t_spk: int, seed: int = 1,
                    text_valid=None, joint_cfg: bool = True, kv_std: float = 1.0) -> ContextKV:
    """Synthetic cached context for `utterances` utterances: with joint_cfg the Joint-CFG
    roles (rows [0, U) conditioned, rows [U, 2U) the unconditioned bundle of
    EncodedCondition::zeros_like: zero K/V, every key masked out), else the conditioned
    rows only.  Text keys are valid up to a per-utterance length (default uniform in
    [min(32, t_text), t_text]); speaker keys are all valid."""
    roles = (ROLE_COND, ROLE_UNCOND) if joint_cfg else (ROLE_COND,)
    return make_role_context(cfg, utterances, t_text, t_spk, roles, seed=seed,
                             text_valid=text_valid, kv_std=kv_std)


def make_noise(utterances: int, seq: int, latent_dim: int, seed: int = 2) -> np.ndarray:
    """Initial RF noise x_0 ~ N(0, 1), [U, S, P] (euler_sampler.rs:146-152)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((utterances, seq, latent_dim), dtype=np.float32)


@dataclass
class CodecWeights:
    """DACVAE decoder weights (CodecConfig), Burn layouts (codec/weights.rs): out_proj_w
    [proj, latent, 1], stem_w [dim, proj, 7], per block alpha [in], convt_w [in, out, 2r],
    convt_b [out], res_alpha0 / res_conv_w [out, out, 7] / res_conv_b / res_alpha1 /
    res_pw_w [out, out, 1] / res_pw_b (lists of three), head_alpha [C], head_w [1, C, 7],
    head_b [1].  Random draws keep the activations of order one: conv weights
    N(0, gain^2 / fan_in) (residual units 0.5 gain, the head 0.3 gain, so tanh mostly stays
    off saturation), Snake alphas U(0.5, 2), biases N(0, 0.05^2)."""

    io: dict
    blocks: list

    @staticmethod
    def random(cfg, seed: int = 0, gain: float = 1.0, bias: bool = True) -> "CodecWeights":
        rng = np.random.default_rng(seed)

        def conv(o, i, k, g=gain):
            return (rng.standard_normal((o, i, k), dtype=np.float32) * np.float32(g / np.sqrt(i * k))).astype(np.float32)

        def vec(n):
            return (rng.standard_normal(n, dtype=np.float32) * np.float32(0.05)).astype(np.float32) if bias else None

        def alpha(n):
            return rng.uniform(0.5, 2.0, n).astype(np.float32)

        io = {"out_proj_w": conv(cfg.proj_dim, cfg.latent_dim, 1), "out_proj_b": vec(cfg.proj_dim),
              "stem_w": conv(cfg.decoder_dim, cfg.proj_dim, 7), "stem_b": vec(cfg.decoder_dim),
              "head_alpha": alpha(cfg.head_dim), "head_w": conv(1, cfg.head_dim, 7, 0.3 * gain),
              "head_b": vec(1)}
        blocks = []
        for i, r in enumerate(cfg.rates):
            cin, cout = cfg.block_dims(i)
            blk = {"alpha": alpha(cin),
                   "convt_w": (rng.standard_normal((cin, cout, 2 * r), dtype=np.float32)
                               * np.float32(gain / np.sqrt(2 * cin))).astype(np.float32),
                   "convt_b": vec(cout)}
            for k in ("res_alpha0", "res_conv_w", "res_conv_b", "res_alpha1", "res_pw_w", "res_pw_b"):
                blk[k] = []
            for _ in range(3):
                blk["res_alpha0"].append(alpha(cout))
                blk["res_conv_w"].append(conv(cout, cout, 7, 0.5 * gain))
                blk["res_conv_b"].append(vec(cout))
                blk["res_alpha1"].append(alpha(cout))
                blk["res_pw_w"].append(conv(cout, cout, 1, 0.5 * gain))
                blk["res_pw_b"].append(vec(cout))
            blocks.append(blk)
        return CodecWeights(io, blocks)
