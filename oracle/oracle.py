"""ctypes wrapper for the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, as the checker and as the timed CPU baseline.  The product path
(libirodori_hip.so and the irodori_hip package) never imports it.

`Oracle("f32")` mirrors the reference's Burn NdArray<f32> arithmetic;
`Oracle("f64")` is the same restatement in double precision.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)


class OrcCfg(C.Structure):
    _fields_ = [
        ("latent_dim", C.c_int32), ("model_dim", C.c_int32), ("num_layers", C.c_int32),
        ("num_heads", C.c_int32), ("head_dim", C.c_int32), ("mlp_hidden", C.c_int32),
        ("adaln_rank", C.c_int32), ("t_dim", C.c_int32), ("norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("gemm_fp8", C.c_int32), ("fused_adaln", C.c_int32),
    ]


class OrcBlock(C.Structure):
    _fields_ = [
        ("w_qkv", _f32p), ("w_gate", _f32p), ("w_o", _f32p), ("q_norm", _f32p),
        ("k_norm", _f32p), ("w13", _f32p), ("w2", _f32p),
        ("ada_down", (_f32p * 3) * 2), ("ada_up", (_f32p * 3) * 2), ("ada_up_b", (_f32p * 3) * 2),
    ]


class OrcIo(C.Structure):
    _fields_ = [
        ("cond_w0", _f32p), ("cond_w1", _f32p), ("cond_w2", _f32p), ("in_w", _f32p),
        ("in_b", _f32p), ("out_norm_w", _f32p), ("out_w", _f32p), ("out_b", _f32p),
    ]


class OrcEncCfg(C.Structure):
    _fields_ = [("dim", C.c_int32), ("num_layers", C.c_int32), ("num_heads", C.c_int32),
                ("mlp_hidden", C.c_int32), ("norm_eps", C.c_float)]


class OrcEncBlock(C.Structure):
    _fields_ = [(n, _f32p) for n in ("attn_norm", "wq", "wk", "wv", "wo", "w_gate", "q_norm",
                                     "k_norm", "mlp_norm", "w13", "w2")]


class OrcCodecBlock(C.Structure):
    _fields_ = [("alpha", _f32p), ("convt_w", _f32p), ("convt_b", _f32p),
                ("res_alpha0", _f32p * 3), ("res_conv_w", _f32p * 3), ("res_conv_b", _f32p * 3),
                ("res_alpha1", _f32p * 3), ("res_pw_w", _f32p * 3), ("res_pw_b", _f32p * 3)]


class OrcCodec(C.Structure):
    _fields_ = [("latent_dim", C.c_int32), ("proj_dim", C.c_int32), ("decoder_dim", C.c_int32),
                ("num_blocks", C.c_int32), ("rates", C.c_int32 * 8), ("out_proj_w", _f32p),
                ("out_proj_b", _f32p), ("stem_w", _f32p), ("stem_b", _f32p),
                ("blocks", C.POINTER(OrcCodecBlock)), ("head_alpha", _f32p), ("head_w", _f32p),
                ("head_b", _f32p)]


class OrcSampler(C.Structure):
    """orc_sampler (oracle.h): the sampler parameters and request facts."""
    _fields_ = [
        ("num_steps", C.c_int32), ("method", C.c_int32), ("cfg_mode", C.c_int32),
        ("scale_text", C.c_float), ("scale_caption", C.c_float), ("scale_speaker", C.c_float),
        ("min_t", C.c_float), ("max_t", C.c_float), ("has_truncation", C.c_int32),
        ("truncation_factor", C.c_float), ("has_speaker", C.c_int32), ("has_caption", C.c_int32),
        ("has_temporal_rescale", C.c_int32), ("rescale_k", C.c_float), ("rescale_sigma", C.c_float),
        ("has_speaker_kv", C.c_int32), ("speaker_kv_scale", C.c_float),
        ("speaker_kv_max_layers", C.c_int32), ("speaker_kv_has_min_t", C.c_int32),
        ("speaker_kv_min_t", C.c_float), ("ctx_aux_start", C.c_int32),
    ]


# Defaults of a sampler request: Independent CFG, Euler, scales 3/3/5 over [0.5, 1]
# (params.rs:22-33), no truncation, rescale or speaker-KV scaling.
SAMPLER_DEFAULTS = dict(num_steps=40, method=0, cfg_mode=0, scale_text=3.0, scale_caption=3.0,
                        scale_speaker=5.0, min_t=0.5, max_t=1.0, has_truncation=0,
                        truncation_factor=1.0, has_speaker=0, has_caption=0,
                        has_temporal_rescale=0, rescale_k=1.0, rescale_sigma=1.0,
                        has_speaker_kv=0, speaker_kv_scale=1.0, speaker_kv_max_layers=-1,
                        speaker_kv_has_min_t=0, speaker_kv_min_t=0.0, ctx_aux_start=0)


def sampler_struct(**kw) -> OrcSampler:
    """OrcSampler from SAMPLER_DEFAULTS overridden by keyword arguments."""
    unknown = set(kw) - set(SAMPLER_DEFAULTS)
    if unknown:
        raise TypeError("unknown sampler fields: %s" % sorted(unknown))
    d = dict(SAMPLER_DEFAULTS, **kw)
    return OrcSampler(**d)


def build() -> None:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def _load():
    """The oracle library; IRODORI_ORACLE_LIB names another build of the same source (the
    sanitizer build of tests/sanitize/)."""
    global _lib
    if _lib is None:
        path = os.environ.get("IRODORI_ORACLE_LIB")
        if not path:
            path = _LIB_PATH
            if not os.path.exists(path):
                build()
        _lib = C.CDLL(path)
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def _lat(mask):
    """Optional latent key mask -> uint8 pointer (None = every latent key attends)."""
    return None if mask is None else _u8(np.ascontiguousarray(mask, np.uint8))


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    _load().orc_set_threads(int(n))


def get_threads() -> int:
    return int(_load().orc_get_threads())


def e4m3_encode(x) -> np.ndarray:
    """float32 array -> e4m3fn codes (uint8), round to nearest even, saturating at 448."""
    lib = _load()
    lib.orc_e4m3_encode.restype = C.c_uint8
    lib.orc_e4m3_encode.argtypes = [C.c_float]
    x = _c32(x)
    return np.array([lib.orc_e4m3_encode(float(v)) for v in x.ravel()], np.uint8).reshape(x.shape)


def e4m3_decode(b) -> np.ndarray:
    lib = _load()
    lib.orc_e4m3_decode.restype = C.c_float
    lib.orc_e4m3_decode.argtypes = [C.c_uint8]
    b = np.ascontiguousarray(b, np.uint8)
    return np.array([lib.orc_e4m3_decode(int(v)) for v in b.ravel()], np.float32).reshape(b.shape)


def mx_scale_exp(amax: float) -> int:
    lib = _load()
    lib.orc_mx_scale_exp.restype = C.c_int
    lib.orc_mx_scale_exp.argtypes = [C.c_float]
    return int(lib.orc_mx_scale_exp(float(amax)))


def mx_quantize_rows(x):
    """x [M, K] (K % 32 == 0) -> (codes uint8 [M, K], E8M0 scale bytes uint8 [M, K/32])."""
    x = _c32(x)
    M, K = x.shape
    q = np.empty((M, K), np.uint8)
    sc = np.empty((M, K // 32), np.uint8)
    _load().orc_mx_quantize_rows(_f(x), M, K, _u8(q), _u8(sc))
    return q, sc


def mx_dequantize_rows(q, sc) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    sc = np.ascontiguousarray(sc, np.uint8)
    M, K = q.shape
    y = np.empty((M, K), np.float32)
    _load().orc_mx_dequantize_rows(_u8(q), _u8(sc), M, K, _f(y))
    return y


def quant_weight_cols(w):
    """Burn w [K, N] -> (codes uint8 [K, N], per-output-channel f32 scales [N])."""
    w = _c32(w)
    K, N = w.shape
    q = np.empty((K, N), np.uint8)
    sc = np.empty(N, np.float32)
    _load().orc_quant_weight_cols(_f(w), K, N, _u8(q), _f(sc))
    return q, sc


class Oracle:
    """Oracle entry points; arrays are numpy float32 (masks uint8), shapes as in oracle.h.
    gemm_fp8: the block GEMMs take fp8 operands (the HIP path's fp8 compute mode).
    fused_adaln: the samplers' forwards fold the adaLN into the GEMMs that read its output,
    the algebra of the HIP path's bf16 sampler chains (orc_cfg.fused_adaln).  Every row of a
    sampler evaluation shares one modulation vector; the plain forward and block entry
    points, whose rows may carry different t, keep the unfolded adaLN unless asked."""

    def __init__(self, precision: str = "f32", gemm_fp8: bool = False, fused_adaln: bool = False):
        assert precision in ("f32", "f64")
        self.lib = _load()
        self.p = "orc_%s_" % precision
        self.fp8 = bool(gemm_fp8)
        self.fused = bool(fused_adaln)

    def _fn(self, name):
        return getattr(self.lib, self.p + name)

    # ---- structs -------------------------------------------------------------------
    def cfg_struct(self, cfg, sampler: bool = False) -> OrcCfg:
        return OrcCfg(cfg.latent_dim, cfg.model_dim, cfg.num_layers, cfg.num_heads,
                      cfg.head_dim, cfg.mlp_hidden, cfg.adaln_rank, cfg.timestep_embed_dim,
                      cfg.norm_eps, cfg.rope_theta, int(self.fp8), int(sampler and self.fused))

    @staticmethod
    def block_struct(b) -> OrcBlock:
        s = OrcBlock()
        for k in ("w_qkv", "w_gate", "w_o", "q_norm", "k_norm", "w13", "w2"):
            setattr(s, k, _f(b[k]))
        for w in range(2):
            for ch in range(3):
                s.ada_down[w][ch] = _f(b["ada_down"][w][ch])
                s.ada_up[w][ch] = _f(b["ada_up"][w][ch])
                s.ada_up_b[w][ch] = _f(b["ada_up_b"][w][ch])
        return s

    @staticmethod
    def io_struct(io) -> OrcIo:
        return OrcIo(*[_f(io[k]) for k in ("cond_w0", "cond_w1", "cond_w2", "in_w", "in_b",
                                            "out_norm_w", "out_w", "out_b")])

    # ---- operators -----------------------------------------------------------------
    def timestep_embedding(self, t, t_dim):
        t = _c32(t)
        out = np.empty((t.shape[0], t_dim), np.float32)
        self._fn("timestep_embedding")(_f(t), t.shape[0], t_dim, _f(out))
        return out

    def rope_tables(self, S, Dh, theta=10000.0):
        cs = np.empty((S, Dh // 2), np.float32)
        sn = np.empty((S, Dh // 2), np.float32)
        self._fn("rope_tables")(S, Dh, C.c_float(theta), _f(cs), _f(sn))
        return cs, sn

    def linear(self, x, w, b=None):
        x, w = _c32(x), _c32(w)
        M, K = x.shape
        N = w.shape[1]
        y = np.empty((M, N), np.float32)
        bb = _c32(b) if b is not None else None
        self._fn("linear")(_f(x), _f(w), _f(bb) if bb is not None else None, M, K, N, _f(y))
        return y

    def rms_norm(self, x, w, eps):
        x, w = _c32(x), _c32(w)
        y = np.empty_like(x)
        rows, D = x.reshape(-1, x.shape[-1]).shape
        self._fn("rms_norm")(_f(x), _f(w), rows, D, C.c_float(eps), _f(y))
        return y

    def fused_adaln(self, x, scale, shift, B, S, eps):
        x, scale, shift = _c32(x), _c32(scale), _c32(shift)
        D = x.shape[-1]
        y = np.empty_like(x)
        self._fn("fused_adaln")(_f(x), _f(scale), _f(shift), B, S, D, C.c_float(eps), _f(y))
        return y

    def head_rms_norm(self, x, w, eps):
        x, w = _c32(x), _c32(w)
        H, Dh = w.shape
        N = x.size // (H * Dh)
        y = np.empty_like(x)
        self._fn("head_rms_norm")(_f(x), _f(w), N, H, Dh, C.c_float(eps), _f(y))
        return y

    def rope_half(self, x, cs, sn):
        x = _c32(x)
        B, S, H, Dh = x.shape
        y = np.empty_like(x)
        self._fn("rope_half")(_f(x), _f(_c32(cs)), _f(_c32(sn)), B, S, H, Dh, _f(y))
        return y

    def rope_full(self, x, cs, sn):
        x = _c32(x)
        B, S, H, Dh = x.shape
        y = np.empty_like(x)
        self._fn("rope_full")(_f(x), _f(_c32(cs)), _f(_c32(sn)), B, S, H, Dh, _f(y))
        return y

    def sdpa(self, q, k, v, mask, scale):
        q, k, v = _c32(q), _c32(k), _c32(v)
        B, H, Sq, Dh = q.shape
        Skv = k.shape[2]
        m = _c32(mask) if mask is not None else None
        out = np.empty_like(q)
        self._fn("sdpa")(_f(q), _f(k), _f(v), _f(m) if m is not None else None, B, H, Sq, Skv,
                         Dh, C.c_float(scale), _f(out))
        return out

    def cond_module(self, cfg, io, t):
        t = _c32(t)
        out = np.empty((t.shape[0], 3 * cfg.model_dim), np.float32)
        self._fn("cond_module")(C.byref(self.cfg_struct(cfg)), C.byref(self.io_struct(io)),
                                _f(t), t.shape[0], _f(out))
        return out

    def adaln_vectors(self, cfg, blk, which, cond):
        cond = _c32(cond)
        B, D = cond.shape[0], cfg.model_dim
        sh, sc, g = (np.empty((B, D), np.float32) for _ in range(3))
        self._fn("adaln_vectors")(C.byref(self.cfg_struct(cfg)), C.byref(self.block_struct(blk)),
                                  which, _f(cond), B, _f(sh), _f(sc), _f(g))
        return sh, sc, g

    def gemm_fp8(self, x, w):
        """The fp8-operand block GEMM: x [M, K] @ w [K, N] (oracle.h gemm_fp8)."""
        x, w = _c32(x), _c32(w)
        M, K = x.shape
        N = w.shape[1]
        y = np.empty((M, N), np.float32)
        self._fn("gemm_fp8")(_f(x), _f(w), M, K, N, _f(y))
        return y

    # ---- condition encoders --------------------------------------------------------
    @staticmethod
    def enc_cfg_struct(ecfg) -> OrcEncCfg:
        return OrcEncCfg(ecfg.dim, ecfg.num_layers, ecfg.num_heads, ecfg.mlp_hidden, ecfg.norm_eps)

    @staticmethod
    def enc_block_struct(b) -> OrcEncBlock:
        return OrcEncBlock(*[_f(b[k]) for k in ("attn_norm", "wq", "wk", "wv", "wo", "w_gate",
                                                 "q_norm", "k_norm", "mlp_norm", "w13", "w2")])

    def encoder_forward(self, ecfg, ew, mask, ids=None, latent=None):
        """Condition encoder + conditioner norm (+ the speaker mean token): ids [B, S] int32
        or latent [B, S, in_dim]; mask [B, S] -> (state [B, S + mean_token, E],
        mask_out [B, S + mean_token])."""
        mask = np.ascontiguousarray(mask, np.uint8)
        B, S = mask.shape
        Tn = S + (1 if ecfg.mean_token else 0)
        out = np.empty((B, Tn, ecfg.dim), np.float32)
        mo = np.empty((B, Tn), np.uint8)
        blocks = (OrcEncBlock * ecfg.num_layers)(*[self.enc_block_struct(b) for b in ew.blocks])
        keep = [ew.blocks, ew.io]
        idp = None
        if ids is not None:
            ids = np.ascontiguousarray(ids, np.int32)
            idp = ids.ctypes.data_as(C.POINTER(C.c_int32))
        lat = _c32(latent) if latent is not None else None
        self._fn("encoder_forward")(
            C.byref(self.enc_cfg_struct(ecfg)), blocks,
            _f(ew.io["embedding"]) if ids is not None else None,
            _f(ew.io["in_w"]) if lat is not None else None,
            _f(ew.io["in_b"]) if lat is not None else None, ecfg.in_dim,
            _f(ew.io["out_norm"]), int(ecfg.mean_token), B, S, idp,
            _f(lat) if lat is not None else None, _u8(mask), _f(out), _u8(mo))
        del keep
        return out, mo

    # ---- DACVAE decoder -------------------------------------------------------------
    def conv1d(self, x, w, b=None, dilation=1, padding=0):
        """Conv1d, stride 1: x [C, L], w [O, C, k] (Burn layout), b [O] -> [O, L_out]."""
        x, w = _c32(x), _c32(w)
        Cc, L = x.shape
        O, _, k = w.shape
        Lo = L + 2 * padding - dilation * (k - 1)
        y = np.empty((O, Lo), np.float32)
        bb = _c32(b) if b is not None else None
        self._fn("conv1d")(_f(x), Cc, L, _f(w), _f(bb) if bb is not None else None, O, k, dilation,
                           padding, _f(y))
        return y

    def conv_transpose1d(self, x, w, b=None, stride=1, padding=0, output_padding=0):
        """ConvTranspose1d: x [C, L], w [C, O, k] (Burn layout), b [O] -> [O, L_out]."""
        x, w = _c32(x), _c32(w)
        Cc, L = x.shape
        _, O, k = w.shape
        Lo = (L - 1) * stride - 2 * padding + k + output_padding
        y = np.empty((O, Lo), np.float32)
        bb = _c32(b) if b is not None else None
        self._fn("conv_transpose1d")(_f(x), Cc, L, _f(w), _f(bb) if bb is not None else None, O, k,
                                     stride, padding, output_padding, _f(y))
        return y

    def snake(self, x, alpha):
        """Snake1d: x [C, L], alpha [C]."""
        x, alpha = _c32(x), _c32(alpha)
        y = np.empty_like(x)
        self._fn("snake")(_f(x), _f(alpha), x.shape[0], x.shape[1], _f(y))
        return y

    def codec_decode(self, ccfg, cw, latent):
        """DacVaeCodec::decode: latent [B, T, latent_dim] -> wav [B, 1, T * hop]."""
        lat = _c32(latent)
        B, T, _ = lat.shape

        def p(a):
            return _f(_c32(a)) if a is not None else None

        keep = []

        def q(a):
            if a is None:
                return None
            a = _c32(a)
            keep.append(a)
            return _f(a)

        blocks = (OrcCodecBlock * ccfg.num_blocks)()
        for i, b in enumerate(cw.blocks):
            s = blocks[i]
            s.alpha, s.convt_w, s.convt_b = q(b["alpha"]), q(b["convt_w"]), q(b["convt_b"])
            for k in ("res_alpha0", "res_conv_w", "res_conv_b", "res_alpha1", "res_pw_w", "res_pw_b"):
                arr = getattr(s, k)
                for u in range(3):
                    arr[u] = q(b[k][u])
        io = cw.io
        cd = OrcCodec(ccfg.latent_dim, ccfg.proj_dim, ccfg.decoder_dim, ccfg.num_blocks,
                      (C.c_int32 * 8)(*ccfg.rates), q(io["out_proj_w"]), q(io["out_proj_b"]),
                      q(io["stem_w"]), q(io["stem_b"]), blocks, q(io["head_alpha"]), q(io["head_w"]),
                      q(io["head_b"]))
        wav = np.empty((B, 1, T * ccfg.hop_length), np.float32)
        self._fn("codec_decode")(C.byref(cd), B, T, _f(lat), _f(wav))
        del keep, p
        return wav

    def swiglu(self, h, w13, w2):
        h = _c32(h)
        M, D = h.shape
        F = w2.shape[0]
        out = np.empty((M, D), np.float32)
        self._fn("swiglu")(_f(h), _f(_c32(w13)), _f(_c32(w2)), M, D, F, _f(out))
        return out

    def joint_attention(self, cfg, blk, h, ctx_k, ctx_v, ctx_mask, cs, sn, latent_mask=None):
        h = _c32(h)
        B, S, _ = h.shape
        T = ctx_k.shape[1]
        out = np.empty_like(h)
        self._fn("joint_attention")(C.byref(self.cfg_struct(cfg)), C.byref(self.block_struct(blk)),
                                    _f(h), B, S, T, _f(_c32(ctx_k)), _f(_c32(ctx_v)),
                                    _u8(np.ascontiguousarray(ctx_mask, np.uint8)), _lat(latent_mask),
                                    _f(_c32(cs)), _f(_c32(sn)), _f(out))
        return out

    def build_kv_cache(self, cfg, k_norm, text, text_mask, wk_text, wv_text,
                       aux=None, aux_mask=None, wk_aux=None, wv_aux=None):
        text = _c32(text)
        B, Tt, Dt = text.shape
        Ta, Da = (aux.shape[1], aux.shape[2]) if aux is not None else (0, 0)
        T = Tt + Ta
        HD = cfg.num_heads * cfg.head_dim
        ck = np.empty((B, T, cfg.num_heads, cfg.head_dim), np.float32)
        cv = np.empty_like(ck)
        cm = np.empty((B, T), np.uint8)
        auxp = _f(_c32(aux)) if aux is not None else None
        amp = _u8(np.ascontiguousarray(aux_mask, np.uint8)) if aux_mask is not None else None
        self._fn("build_kv_cache")(
            C.byref(self.cfg_struct(cfg)), _f(_c32(k_norm)), B, _f(text),
            _u8(np.ascontiguousarray(text_mask, np.uint8)), Tt, Dt, _f(_c32(wk_text)),
            _f(_c32(wv_text)), auxp, amp, Ta, Da,
            _f(_c32(wk_aux)) if wk_aux is not None else None,
            _f(_c32(wv_aux)) if wv_aux is not None else None, _f(ck), _f(cv), _u8(cm))
        assert HD == cfg.num_heads * cfg.head_dim
        return ck, cv, cm

    def block_forward(self, cfg, blk, x, cond, ctx_k, ctx_v, ctx_mask, latent_mask=None):
        """One DiffusionBlock on x [B,S,D] with cond [B,3D]; ctx_* of this layer [B,T,H,Dh]."""
        x = _c32(x).copy()
        B, S, _ = x.shape
        T = ctx_k.shape[1]
        cs, sn = self.rope_tables(S, cfg.head_dim, cfg.rope_theta)
        self._fn("block_forward")(C.byref(self.cfg_struct(cfg)), C.byref(self.block_struct(blk)),
                                  _f(x), _f(_c32(cond)), B, S, T, _f(_c32(ctx_k)), _f(_c32(ctx_v)),
                                  _u8(np.ascontiguousarray(ctx_mask, np.uint8)), _lat(latent_mask),
                                  _f(cs), _f(sn))
        return x

    # ---- model ---------------------------------------------------------------------
    def forward(self, cfg, weights, x_t, t, ctx_k, ctx_v, ctx_mask, debug=False, latent_mask=None,
                folded=False):
        """x_t [B,S,P]; t [B]; ctx_k/ctx_v [L,B,T,H,Dh]; ctx_mask [B,T] -> v [B,S,P]
        (and [L+1,B,S,D] block outputs when debug).  latent_mask [B,S] (nonzero = key
        attends) masks latent keys (attention.rs:730-750).  folded: the adaLN folded into
        the GEMMs as in the samplers (with this oracle's fused_adaln), for a forward whose
        rows share one t."""
        x_t = _c32(x_t)
        B, S, Pd = x_t.shape
        T = ctx_k.shape[2]
        blocks = (OrcBlock * cfg.num_layers)(*[self.block_struct(b) for b in weights.blocks])
        v = np.empty_like(x_t)
        dbg = np.empty((cfg.num_layers + 1, B, S, cfg.model_dim), np.float32) if debug else None
        self._fn("forward")(C.byref(self.cfg_struct(cfg, sampler=folded)), C.byref(self.io_struct(weights.io)),
                            blocks, B, S, _f(x_t), _f(_c32(t)), T, _f(_c32(ctx_k)),
                            _f(_c32(ctx_v)), _u8(np.ascontiguousarray(ctx_mask, np.uint8)),
                            _lat(latent_mask), _f(v), _f(dbg) if debug else None)
        return (v, dbg) if debug else v

    def sample_rf(self, cfg, weights, x0, ctx, sampler, max_steps_run=0, latent_mask=None):
        """x0 [U,S,P]; ctx = (k [L,R*U,T,H,Dh], v, mask [R*U,T]) role-major (row r*U + u);
        sampler: an OrcSampler (sampler_struct); latent_mask [U,S] or None.
        Returns (x_out, steps_run)."""
        x0 = _c32(x0)
        U, S, Pd = x0.shape
        k, v, m = ctx
        T = k.shape[2]
        blocks = (OrcBlock * cfg.num_layers)(*[self.block_struct(b) for b in weights.blocks])
        out = np.empty_like(x0)
        run = self._fn("sample_rf")(
            C.byref(self.cfg_struct(cfg, sampler=True)), C.byref(self.io_struct(weights.io)), blocks, U, S,
            _f(x0), T, _f(_c32(k)), _f(_c32(v)), _u8(np.ascontiguousarray(m, np.uint8)),
            _lat(latent_mask), C.byref(sampler), max_steps_run, _f(out))
        return out, int(run)

    def sample_joint_cfg(self, cfg, weights, x0, ctx_cond, ctx_unc, num_steps, scale,
                         min_t=0.0, max_t=1.0, max_steps_run=0, latent_mask=None):
        """x0 [U,S,P]; ctx_* = (k [L,U,T,H,Dh], v, mask [U,T]); latent_mask [U,S] or None.
        Returns (x_out, steps_run)."""
        x0 = _c32(x0)
        U, S, Pd = x0.shape
        kc, vc, mc = ctx_cond
        ku, vu, mu = ctx_unc
        T = kc.shape[2]
        blocks = (OrcBlock * cfg.num_layers)(*[self.block_struct(b) for b in weights.blocks])
        out = np.empty_like(x0)
        run = self._fn("sample_joint_cfg")(
            C.byref(self.cfg_struct(cfg, sampler=True)), C.byref(self.io_struct(weights.io)), blocks, U, S,
            _f(x0), T, _f(_c32(kc)), _f(_c32(vc)), _u8(np.ascontiguousarray(mc, np.uint8)),
            _f(_c32(ku)), _f(_c32(vu)), _u8(np.ascontiguousarray(mu, np.uint8)),
            _lat(latent_mask), num_steps,
            C.c_float(scale), C.c_float(min_t), C.c_float(max_t), max_steps_run, _f(out))
        return out, int(run)
