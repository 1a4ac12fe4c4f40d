"""HipInferenceEngine: the HIP backend's InferenceEngine over libirodori_hip.so.

Mirrors the reference's API for the hot path:
  - construction + load_weights  ~ InferenceBuilder -> InferenceEngine
    (src/inference.rs:83-196) with InferenceOptimizedModel fusion (optimized.rs:37-62);
  - set_context_kv               ~ build_kv_caches / CondKvCache (dit/model.rs:444-472);
  - forward_with_cond_cached     ~ optimized.rs:102-113 (one DiT forward);
  - sample                       ~ InferenceEngine::sample -> sample_euler_rf_cfg
    (inference.rs:222-227, euler_sampler.rs:132-718), Joint CFG.
Errors map the C status codes onto IrodoriError variants (src/error.rs:4-60).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L
from .config import (CfgGuidanceMode, CodecConfig, DitConfig, EncoderConfig, InferenceBackendKind,
                     IrodoriError, SamplerMethod, SamplerParams)
from .synthetic import CodecWeights, ContextKV, CtxProjWeights, DitWeights, EncoderWeights

_f32p = C.POINTER(C.c_float)


def _check(rc: int) -> None:
    if rc != L.OK:
        raise IrodoriError(L.ERR_NAMES.get(rc, "Unknown(%d)" % rc), L.last_error())


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _shaped(a, shape, what: str, dtype=np.float32) -> np.ndarray:
    """a as a C-contiguous array of dtype with exactly `shape`: the library reads that many
    elements through the pointer, so any other shape is refused before the call."""
    if a is None:
        raise IrodoriError("InvalidArg", "%s is missing" % what)
    arr = np.ascontiguousarray(a, dtype)
    if arr.shape != tuple(shape):
        raise IrodoriError("Shape", "%s must be %s, got %s" % (what, tuple(shape), arr.shape))
    return arr


def dit_weight_shapes(cfg: DitConfig):
    """Shapes of DitWeights (Burn [d_in, d_out] layouts): io and per-block entries; the
    ada_* entries are [2 norms][3 chunks] lists of the given shape."""
    D, P, F, r, HD = cfg.model_dim, cfg.latent_dim, cfg.mlp_hidden, cfg.adaln_rank, cfg.num_heads * cfg.head_dim
    io = {"cond_w0": (cfg.timestep_embed_dim, D), "cond_w1": (D, D), "cond_w2": (D, 3 * D), "in_w": (P, D),
          "in_b": (D,), "out_norm_w": (D,), "out_w": (D, P), "out_b": (P,)}
    block = {"w_qkv": (D, 3 * HD), "w_gate": (D, D), "w_o": (HD, D), "q_norm": (cfg.num_heads, cfg.head_dim),
             "k_norm": (cfg.num_heads, cfg.head_dim), "w13": (D, 2 * F), "w2": (F, D),
             "ada_down": (D, r), "ada_up": (r, D), "ada_up_b": (D,)}
    return io, block


def codec_weight_shapes(cfg: CodecConfig):
    """Shapes of CodecWeights (Burn layouts, codec/weights.rs): io entries and, per decoder
    block, its entries (the res_* ones per residual unit).  Biases may also be None."""
    C0, hd, P = cfg.decoder_dim, cfg.head_dim, cfg.proj_dim
    io = {"out_proj_w": (P, cfg.latent_dim, 1), "out_proj_b": (P,), "stem_w": (C0, P, 7), "stem_b": (C0,),
          "head_alpha": (hd,), "head_w": (1, hd, 7), "head_b": (1,)}
    blocks = []
    for i, r in enumerate(cfg.rates):
        cin, cout = cfg.block_dims(i)
        blocks.append({"alpha": (cin,), "convt_w": (cin, cout, 2 * r), "convt_b": (cout,), "res_alpha0": (cout,),
                       "res_conv_w": (cout, cout, 7), "res_conv_b": (cout,), "res_alpha1": (cout,),
                       "res_pw_w": (cout, cout, 1), "res_pw_b": (cout,)})
    return io, blocks


def encoder_weight_shapes(cfg: EncoderConfig):
    """Shapes of EncoderWeights: io (the input embedding or projection, the output norm) and
    per-block entries."""
    E, F, H = cfg.dim, cfg.mlp_hidden, cfg.num_heads
    io = {"out_norm": (E,)}
    if cfg.vocab_size:
        io["embedding"] = (cfg.vocab_size, E)
    if cfg.in_dim:
        io["in_w"] = (cfg.in_dim, E)
        io["in_b"] = (E,)
    block = {"attn_norm": (E,), "wq": (E, E), "wk": (E, E), "wv": (E, E), "wo": (E, E), "w_gate": (E, E),
             "q_norm": (H, E // H), "k_norm": (H, E // H), "mlp_norm": (E,), "w13": (E, 2 * F), "w2": (F, E)}
    return io, block


def sampler_params_c(p: SamplerParams, has_speaker: bool = True, has_caption: bool = False,
                     ctx_aux_start: int = 0) -> L.SamplerParamsC:
    """irodori_sampler_params from the params and the request facts: whether the condition
    holds a speaker state (and the model uses it) or a caption with a valid token, and the
    first aux key of the cached context (the text key count)."""
    mode = {CfgGuidanceMode.INDEPENDENT: L.CFG_INDEPENDENT, CfgGuidanceMode.JOINT: L.CFG_JOINT,
            CfgGuidanceMode.ALTERNATING: L.CFG_ALTERNATING}[p.guidance.mode]
    method = {SamplerMethod.EULER: L.METHOD_EULER, SamplerMethod.HEUN: L.METHOD_HEUN,
              SamplerMethod.PLMS4: L.METHOD_PLMS4}[p.method]
    g = p.guidance
    tr, skv = p.temporal_rescale, p.speaker_kv
    return L.SamplerParamsC(
        num_steps=p.num_steps, method=method, cfg_mode=mode, scale_text=g.scale_text,
        scale_caption=g.scale_caption, scale_speaker=g.scale_speaker, min_t=g.min_t, max_t=g.max_t,
        has_truncation=1 if p.truncation_factor is not None else 0,
        truncation_factor=p.truncation_factor if p.truncation_factor is not None else 0.0,
        has_speaker=1 if has_speaker else 0, has_caption=1 if has_caption else 0,
        has_temporal_rescale=1 if tr is not None else 0, rescale_k=tr.k if tr else 1.0,
        rescale_sigma=tr.sigma if tr else 1.0, has_speaker_kv=1 if skv is not None else 0,
        speaker_kv_scale=skv.scale if skv else 1.0,
        speaker_kv_max_layers=skv.max_layers if skv and skv.max_layers is not None else -1,
        speaker_kv_has_min_t=1 if skv is not None and skv.min_t is not None else 0,
        speaker_kv_min_t=skv.min_t if skv is not None and skv.min_t is not None else 0.0,
        ctx_aux_start=ctx_aux_start)


def validate_sampler_params(p: SamplerParams, has_speaker: bool = True, has_caption: bool = False) -> None:
    """SamplerParams::validate (params.rs:99-183), evaluated by the library."""
    c = sampler_params_c(p, has_speaker, has_caption)
    _check(L.load().irodori_sampler_params_validate(C.byref(c)))


class HipInferenceEngine:
    def __init__(self, cfg: DitConfig, backend: InferenceBackendKind = InferenceBackendKind.HIP_BF16,
                 max_rows: int = 2, max_seq: int = 750, max_ctx: int = 631, device: int = 0):
        cfg.validate()
        self.cfg = cfg
        self.backend = backend
        self.lib = L.load()
        c = L.DitConfigC(cfg.latent_dim, cfg.model_dim, cfg.num_layers, cfg.num_heads,
                         cfg.head_dim, cfg.mlp_hidden, cfg.adaln_rank, cfg.timestep_embed_dim,
                         cfg.norm_eps, cfg.rope_theta,
                         {InferenceBackendKind.HIP_BF16: L.DTYPE_BF16,
                          InferenceBackendKind.HIP_F32: L.DTYPE_F32,
                          InferenceBackendKind.HIP_FP8: L.DTYPE_FP8}[backend],
                         max_rows, max_seq, max_ctx)
        h = C.c_void_p()
        _check(self.lib.irodori_ctx_create(device, C.byref(c), C.byref(h)))
        self.ctx = h
        self.max_rows, self.max_seq, self.max_ctx = max_rows, max_seq, max_ctx

    def close(self) -> None:
        if getattr(self, "ctx", None):
            self.lib.irodori_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_bytes(self) -> int:
        n = C.c_uint64()
        _check(self.lib.irodori_ctx_device_bytes(self.ctx, C.byref(n)))
        return int(n.value)

    # ---- weights / context --------------------------------------------------------------
    def load_weights(self, w: DitWeights) -> None:
        ios, bs = dit_weight_shapes(self.cfg)
        if len(w.blocks) != self.cfg.num_layers:
            raise IrodoriError("Shape", "%d blocks of weights for %d layers" % (len(w.blocks), self.cfg.num_layers))
        # Every array is checked before the first upload, so a refusal loads nothing.
        io_arrs = [_shaped(w.io.get(k), ios[k], "io." + k) for k in ("cond_w0", "cond_w1", "cond_w2", "in_w",
                                                                     "in_b", "out_norm_w", "out_w", "out_b")]
        plain = ("w_qkv", "w_gate", "w_o", "q_norm", "k_norm", "w13", "w2")
        blocks = []
        for l, b in enumerate(w.blocks):
            arrs = {k: _shaped(b.get(k), bs[k], "blocks[%d].%s" % (l, k)) for k in plain}
            for k in ("ada_down", "ada_up", "ada_up_b"):
                rows = b.get(k)
                if rows is None or len(rows) != 2 or any(len(r) != 3 for r in rows):
                    raise IrodoriError("Shape", "blocks[%d].%s must be 2 x 3 arrays" % (l, k))
                arrs[k] = [[_shaped(rows[i][ch], bs[k], "blocks[%d].%s[%d][%d]" % (l, k, i, ch)) for ch in range(3)]
                           for i in range(2)]
            blocks.append(arrs)
        io = L.IoWeightsC(*[_fp(a) for a in io_arrs])
        _check(self.lib.irodori_load_io_weights(self.ctx, C.byref(io)))
        for l, arrs in enumerate(blocks):
            s = L.BlockWeightsC()
            for k in plain:
                setattr(s, k, _fp(arrs[k]))
            for k in ("ada_down", "ada_up", "ada_up_b"):
                for i in range(2):
                    for ch in range(3):
                        getattr(s, k)[i][ch] = _fp(arrs[k][i][ch])
            _check(self.lib.irodori_load_block_weights(self.ctx, l, C.byref(s)))

    def set_context_kv(self, ctx: ContextKV) -> None:
        _check(self.lib.irodori_clear_ctx_kv(self.ctx))
        Lc, B, T = ctx.k.shape[:3]
        kv = (Lc, B, T, self.cfg.num_heads, self.cfg.head_dim)
        ks, vs = _shaped(ctx.k, kv, "context k"), _shaped(ctx.v, kv, "context v")
        ms = _shaped(ctx.mask, (B, T), "context mask", np.uint8)
        for l in range(Lc):
            for r in range(B):
                k = ks[l, r]
                v = vs[l, r]
                m = ms[r]
                _check(self.lib.irodori_set_ctx_kv(self.ctx, l, r, T, _fp(k), _fp(v),
                                                   m.ctypes.data_as(C.POINTER(C.c_uint8))))

    def load_ctx_proj_weights(self, w: CtxProjWeights) -> None:
        """Upload every layer's context projections (wk/wv_text, wk/wv_speaker|caption)."""
        if len(w.layers) != self.cfg.num_layers:
            raise IrodoriError("Shape", "%d layers of context projections for %d layers"
                               % (len(w.layers), self.cfg.num_layers))
        HD = self.cfg.num_heads * self.cfg.head_dim
        keys = ("wk_text", "wv_text", "wk_aux", "wv_aux") if w.aux_dim else ("wk_text", "wv_text")
        layers = [{k: _shaped(lw.get(k), (w.text_dim if k.endswith("text") else w.aux_dim, HD),
                              "layers[%d].%s" % (l, k)) for k in keys} for l, lw in enumerate(w.layers)]
        for l, a in enumerate(layers):
            s = L.CtxProjWeightsC(_fp(a["wk_text"]), _fp(a["wv_text"]),
                                  _fp(a["wk_aux"]) if w.aux_dim else None,
                                  _fp(a["wv_aux"]) if w.aux_dim else None)
            _check(self.lib.irodori_load_ctx_proj_weights(self.ctx, l, w.text_dim, w.aux_dim,
                                                          C.byref(s)))
        self._ctx_dims = (w.text_dim, w.aux_dim)

    def build_context_kv(self, row: int, text_state: np.ndarray, text_mask: np.ndarray,
                         aux_state: np.ndarray = None, aux_mask: np.ndarray = None) -> None:
        """build_kv_cache (attention.rs:431-501) of batch row `row` on the device, every layer:
        text_state [t_text, text_dim], aux_state [t_aux, aux_dim] (None: no aux keys)."""
        text_dim, aux_dim = getattr(self, "_ctx_dims", (None, None))
        if text_dim is None:
            raise IrodoriError("NotLoaded", "load_ctx_proj_weights first")
        ts = _c32(text_state)
        if ts.ndim != 2:
            raise IrodoriError("Shape", "text_state must be [tokens, %d]" % text_dim)
        ts = _shaped(ts, (ts.shape[0], text_dim), "text_state")
        tm = _shaped(text_mask, (ts.shape[0],), "text_mask", np.uint8)
        t_aux = 0 if aux_state is None else aux_state.shape[0]
        if t_aux and not aux_dim:
            raise IrodoriError("NotLoaded", "no auxiliary context projection is loaded")
        a = _shaped(aux_state, (t_aux, aux_dim), "aux_state") if t_aux else None
        am = _shaped(aux_mask, (t_aux,), "aux_mask", np.uint8) if t_aux else None
        u8 = C.POINTER(C.c_uint8)
        _check(self.lib.irodori_build_ctx_kv(
            self.ctx, row, ts.shape[0], _fp(ts), tm.ctypes.data_as(u8), t_aux,
            _fp(a) if t_aux else None, am.ctypes.data_as(u8) if t_aux else None))

    def clear_context_kv(self) -> None:
        """Forget every row's cached context (irodori_clear_ctx_kv), so that the next bundle
        may have another length."""
        _check(self.lib.irodori_clear_ctx_kv(self.ctx))

    def read_context_kv(self, layer: int, row: int, t_ctx: int):
        """The cached context of (layer, row): k, v [t_ctx, H, Dh], mask [t_ctx]."""
        H, Dh = self.cfg.num_heads, self.cfg.head_dim
        k = np.empty((t_ctx, H, Dh), np.float32)
        v = np.empty_like(k)
        m = np.empty(t_ctx, np.uint8)
        _check(self.lib.irodori_read_ctx_kv(self.ctx, layer, row, _fp(k), _fp(v),
                                            m.ctypes.data_as(C.POINTER(C.c_uint8))))
        return k, v, m

    # ---- compute ------------------------------------------------------------------------
    def forward_with_cond_cached(self, x_t: np.ndarray, t: np.ndarray, debug: bool = False,
                                 latent_mask: np.ndarray = None):
        """x_t [B,S,P], t [B] -> v [B,S,P] (and [L+1,B,S,D] block outputs if debug).
        latent_mask [B,S] (nonzero = the latent key attends) masks latent keys
        (optimized.rs:102-113, attention.rs:730-750); None = every key attends."""
        x_t = _c32(x_t)
        if x_t.ndim != 3:
            raise IrodoriError("Shape", "x_t must be [B, S, latent_dim]")
        B, S, P = x_t.shape
        x_t = _shaped(x_t, (B, S, self.cfg.latent_dim), "x_t")
        t = _shaped(t, (B,), "t")
        v = np.empty_like(x_t)
        dbg = (np.empty((self.cfg.num_layers + 1, B, S, self.cfg.model_dim), np.float32)
               if debug else None)
        if latent_mask is None:
            _check(self.lib.irodori_forward(self.ctx, B, S, _fp(x_t), _fp(t), _fp(v),
                                            _fp(dbg) if debug else None))
        else:
            m = np.ascontiguousarray(latent_mask, np.uint8)
            if m.shape != (B, S):
                raise IrodoriError("Shape", "latent_mask must be [B, S]")
            _check(self.lib.irodori_forward_masked(self.ctx, B, S, _fp(x_t), _fp(t),
                                                   m.ctypes.data_as(C.POINTER(C.c_uint8)), _fp(v),
                                                   _fp(dbg) if debug else None))
        return (v, dbg) if debug else v

    def block_forward(self, layer: int, x: np.ndarray, cond: np.ndarray) -> np.ndarray:
        """One DiffusionBlock::forward_fused on x [B,S,D] with cond_module output [B,3D]."""
        x = _c32(x).copy()
        if x.ndim != 3:
            raise IrodoriError("Shape", "x must be [B, S, model_dim]")
        B, S, _ = x.shape
        D = self.cfg.model_dim
        x = _shaped(x, (B, S, D), "x")
        cond = _shaped(cond, (B, 3 * D), "cond")
        _check(self.lib.irodori_block_forward(self.ctx, layer, B, S, _fp(x), _fp(cond)))
        return x

    def sample(self, x0: np.ndarray, params: SamplerParams, has_speaker: bool = True,
               lengths=None, has_caption: bool = False, ctx_aux_start: int = 0) -> np.ndarray:
        """RF sampling of U utterances (sample_euler_rf_cfg): x0 [U,S,P] -> x [U,S,P], any
        CFG mode and method.  The context rows must hold params.cfg_roles(has_speaker,
        has_caption) role-major (row r * U + u).  lengths [U] (optional): utterance u
        attends to its first lengths[u] latent frames (padded variable-length batch).
        ctx_aux_start: first aux key of the context (used by speaker-KV scaling)."""
        x0 = _c32(x0)
        if x0.ndim != 3:
            raise IrodoriError("Shape", "x0 must be [utterances, S, latent_dim]")
        U, S, P = x0.shape
        x0 = _shaped(x0, (U, S, self.cfg.latent_dim), "x0")
        out = np.empty_like(x0)
        pc = sampler_params_c(params, has_speaker, has_caption, ctx_aux_start)
        if lengths is None:
            _check(self.lib.irodori_sample(self.ctx, C.byref(pc), U, S, _fp(x0), _fp(out)))
        else:
            ln = np.ascontiguousarray(lengths, np.int32)
            if ln.shape != (U,):
                raise IrodoriError("Shape", "lengths must be [U]")
            _check(self.lib.irodori_sample_masked(self.ctx, C.byref(pc), U, S,
                                                  ln.ctypes.data_as(C.POINTER(C.c_int32)),
                                                  _fp(x0), _fp(out)))
        return out

    def sample_device(self, d_x0: int, d_out: int, utterances: int, seq: int,
                      params: SamplerParams, has_speaker: bool = True, has_caption: bool = False,
                      ctx_aux_start: int = 0, lengths=None) -> None:
        """Same as sample() on device pointers (inputs/outputs resident in HBM)."""
        pc = sampler_params_c(params, has_speaker, has_caption, ctx_aux_start)
        if lengths is None:
            _check(self.lib.irodori_sample_device(self.ctx, C.byref(pc), utterances, seq,
                                                  C.c_void_p(d_x0), C.c_void_p(d_out)))
            return
        ln = np.ascontiguousarray(lengths, np.int32)
        if ln.shape != (utterances,):
            raise IrodoriError("Shape", "lengths must be [utterances]")
        _check(self.lib.irodori_sample_device_masked(
            self.ctx, C.byref(pc), utterances, seq, ln.ctypes.data_as(C.POINTER(C.c_int32)),
            C.c_void_p(d_x0), C.c_void_p(d_out)))


    def joint_attention(self, layer: int, batch: int, seq: int, d_q: int, d_k: int, d_v: int, d_gate: int,
                        d_out: int, stream: int = 0) -> None:
        """irodori_op_joint_attention on device pointers: q, k, v [batch, seq, H, 64] f32, gate
        logits [batch, seq, H*64] (0: none) -> out [batch, seq, H*64] f32, with this layer's head
        norms and cached context of rows 0..batch-1."""
        _check(self.lib.irodori_op_joint_attention(self.ctx, layer, batch, seq, d_q, d_k, d_v, d_gate or None,
                                                   d_out, stream or None))

    def swiglu_mlp(self, layer: int, batch: int, seq: int, d_x: int, d_shift: int, d_scale: int, d_gate: int,
                   stream: int = 0) -> None:
        """irodori_op_swiglu_mlp on device pointers: x [batch, seq, D] f32 += gate * SwiGLU(adaLN(x))
        with modulation vectors [batch, D] f32."""
        _check(self.lib.irodori_op_swiglu_mlp(self.ctx, layer, batch, seq, d_x, d_shift, d_scale, d_gate,
                                              stream or None))

    def profile_layer(self, batch: int, seq: int, iters: int = 20) -> dict:
        """Average microseconds per kernel of one block (HIP events on the context stream)."""
        kt = L.KernelTimesC()
        _check(self.lib.irodori_profile_layer(self.ctx, batch, seq, iters, C.byref(kt)))
        return {n: float(getattr(kt, n)) for n, _ in L.KernelTimesC._fields_}


class HipEncoder:
    """A condition encoder on the GPU (irodori_encoder_*): TextEncoder / ReferenceLatentEncoder
    + the conditioner norm (+ the speaker mean token), i.e. EncodedCondition's text_state or
    aux state (dit/model.rs:182-205)."""

    def __init__(self, cfg: EncoderConfig, backend: InferenceBackendKind = InferenceBackendKind.HIP_BF16,
                 max_rows: int = 2, max_seq: int = 512, device: int = 0):
        if backend not in (InferenceBackendKind.HIP_BF16, InferenceBackendKind.HIP_F32):
            raise IrodoriError("Dtype", "the encoders run in bf16 or f32")
        self.cfg = cfg
        self.lib = L.load()
        c = L.EncoderConfigC(cfg.dim, cfg.num_layers, cfg.num_heads, cfg.mlp_hidden, cfg.vocab_size,
                             cfg.in_dim, int(cfg.mean_token), cfg.norm_eps,
                             L.DTYPE_BF16 if backend is InferenceBackendKind.HIP_BF16 else L.DTYPE_F32,
                             max_rows, max_seq)
        h = C.c_void_p()
        _check(self.lib.irodori_encoder_create(device, C.byref(c), C.byref(h)))
        self.enc = h

    def close(self) -> None:
        if getattr(self, "enc", None):
            self.lib.irodori_encoder_destroy(self.enc)
            self.enc = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load_weights(self, w: EncoderWeights) -> None:
        ios, bs = encoder_weight_shapes(self.cfg)
        if len(w.blocks) != self.cfg.num_layers:
            raise IrodoriError("Shape", "%d blocks of weights for %d layers" % (len(w.blocks), self.cfg.num_layers))
        io_arrs = {k: _shaped(w.io.get(k), ios[k], "io." + k) for k in ios}
        blocks = [[_shaped(b.get(k), bs[k], "blocks[%d].%s" % (l, k)) for k in L.ENC_BLOCK_FIELDS]
                  for l, b in enumerate(w.blocks)]
        io = L.EncoderIoWeightsC(*[_fp(io_arrs[k]) if k in io_arrs else None
                                   for k in ("embedding", "in_w", "in_b", "out_norm")])
        _check(self.lib.irodori_encoder_load_io_weights(self.enc, C.byref(io)))
        for l, arrs in enumerate(blocks):
            s = L.EncoderBlockWeightsC(*[_fp(a) for a in arrs])
            _check(self.lib.irodori_encoder_load_block_weights(self.enc, l, C.byref(s)))

    def forward(self, mask: np.ndarray, ids: np.ndarray = None, latent: np.ndarray = None):
        """mask [B, S]; ids [B, S] (token encoder) or latent [B, S, in_dim] ->
        (state [B, S + mean_token, dim], mask_out [B, S + mean_token])."""
        mask = np.ascontiguousarray(mask, np.uint8)
        if mask.ndim != 2:
            raise IrodoriError("Shape", "mask must be [B, S]")
        B, S = mask.shape
        if (ids is None) == (latent is None):
            raise IrodoriError("InvalidArg", "give either token ids or latent frames")
        Tn = S + int(self.cfg.mean_token)
        out = np.empty((B, Tn, self.cfg.dim), np.float32)
        mo = np.empty((B, Tn), np.uint8)
        u8 = C.POINTER(C.c_uint8)
        idp = lat = None
        if ids is not None:
            ids = _shaped(ids, (B, S), "ids", np.int32)
            idp = ids.ctypes.data_as(C.POINTER(C.c_int32))
        if latent is not None:
            lat = _shaped(latent, (B, S, self.cfg.in_dim), "latent")
        _check(self.lib.irodori_encoder_forward(self.enc, B, S, idp, _fp(lat) if lat is not None else None,
                                                mask.ctypes.data_as(u8), _fp(out), mo.ctypes.data_as(u8)))
        return out, mo


class HipDacVaeCodec:
    """The DACVAE decoder on the GPU (irodori_codec_*): DacVaeCodec::decode
    (codec/model.rs:60-65) for latents [B, T, latent_dim] -> waveforms [B, 1, T * hop]."""

    def __init__(self, cfg: CodecConfig, backend: InferenceBackendKind = InferenceBackendKind.HIP_BF16,
                 max_frames: int = 750, device: int = 0):
        if backend not in (InferenceBackendKind.HIP_BF16, InferenceBackendKind.HIP_F32):
            raise IrodoriError("Dtype", "the codec runs in bf16 or f32")
        if cfg.num_blocks > L.CODEC_MAX_BLOCKS:
            raise IrodoriError("Config", "at most %d decoder blocks" % L.CODEC_MAX_BLOCKS)
        self.cfg = cfg
        self.lib = L.load()
        rates = (C.c_int32 * L.CODEC_MAX_BLOCKS)(*cfg.rates)
        c = L.CodecConfigC(cfg.latent_dim, cfg.proj_dim, cfg.decoder_dim, cfg.num_blocks, rates,
                           L.DTYPE_BF16 if backend is InferenceBackendKind.HIP_BF16 else L.DTYPE_F32,
                           max_frames)
        h = C.c_void_p()
        _check(self.lib.irodori_codec_create(device, C.byref(c), C.byref(h)))
        self.codec = h

    def close(self) -> None:
        if getattr(self, "codec", None):
            self.lib.irodori_codec_destroy(self.codec)
            self.codec = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sample_rate(self) -> int:
        return self.cfg.sample_rate

    def hop_length(self) -> int:
        return int(self.lib.irodori_codec_hop_length(self.codec))

    def load_weights(self, w: CodecWeights) -> None:
        """Burn layouts (codec/weights.rs); biases may be None (zero)."""
        cfg = self.cfg
        keep = []

        def p(a, shape, what, optional=False):
            if a is None and optional:
                return None
            keep.append(_shaped(a, shape, what))
            return _fp(keep[-1])

        if len(w.blocks) != cfg.num_blocks:
            raise IrodoriError("Shape", "%d decoder blocks of weights for %d" % (len(w.blocks), cfg.num_blocks))
        ios, bss = codec_weight_shapes(cfg)
        blocks = (L.CodecBlockWeightsC * cfg.num_blocks)()
        for i, b in enumerate(w.blocks):
            s, bs = blocks[i], bss[i]
            s.alpha = p(b.get("alpha"), bs["alpha"], "blocks[%d].alpha" % i)
            s.convt_w = p(b.get("convt_w"), bs["convt_w"], "blocks[%d].convt_w" % i)
            s.convt_b = p(b.get("convt_b"), bs["convt_b"], "blocks[%d].convt_b" % i, True)
            for k in ("res_alpha0", "res_conv_w", "res_conv_b", "res_alpha1", "res_pw_w", "res_pw_b"):
                arr = getattr(s, k)
                for u in range(3):
                    arr[u] = p(b[k][u], bs[k], "blocks[%d].%s[%d]" % (i, k, u), k.endswith("_b"))
        io = w.io
        cw = L.CodecWeightsC(*[p(io.get(k), ios[k], "io." + k, k.endswith("_b")) for k in
                               ("out_proj_w", "out_proj_b", "stem_w", "stem_b")],
                             blocks, *[p(io.get(k), ios[k], "io." + k, k.endswith("_b")) for k in
                                       ("head_alpha", "head_w", "head_b")])
        _check(self.lib.irodori_codec_load_weights(self.codec, C.byref(cw)))
        del keep

    def decode(self, latent: np.ndarray) -> np.ndarray:
        """latent [B, T, latent_dim] -> wav [B, 1, T * hop_length] (host arrays)."""
        lat = _c32(latent)
        if lat.ndim != 3:
            raise IrodoriError("Shape", "latent must be [B, T, latent_dim]")
        B, T, _ = lat.shape
        lat = _shaped(lat, (B, T, self.cfg.latent_dim), "latent")
        wav = np.empty((B, 1, T * self.cfg.hop_length), np.float32)
        _check(self.lib.irodori_codec_decode(self.codec, B, T, _fp(lat), _fp(wav)))
        return wav

    def decode_device(self, d_latent: int, batch: int, frames: int, d_wav: int, stream: int = 0) -> None:
        """Device pointers: latent [batch, frames, latent_dim] -> wav [batch, frames * hop]."""
        _check(self.lib.irodori_codec_decode_device(self.codec, batch, frames, d_latent, d_wav,
                                                    stream or None))


class ops:
    """Operator entry points (src/kernels analogues) on device pointers."""

    @staticmethod
    def rms_norm(d_x: int, d_w: int, rows: int, dim: int, eps: float, d_y: int,
                 stream: int = 0) -> None:
        _check(L.load().irodori_op_rms_norm(d_x, d_w, rows, dim, eps, d_y, stream or None))

    @staticmethod
    def fused_adaln(d_x, d_scale, d_shift, batch, seq, dim, eps, d_y, stream: int = 0) -> None:
        _check(L.load().irodori_op_fused_adaln(d_x, d_scale, d_shift, batch, seq, dim, eps, d_y,
                                               stream or None))

    @staticmethod
    def mx_quantize(d_x, rows, dim, d_q, d_s, stream: int = 0) -> None:
        _check(L.load().irodori_op_mx_quantize(d_x, rows, dim, d_q, d_s, stream or None))

    @staticmethod
    def gemm_fp8(d_a, d_as, d_w, d_ws, M, N, K, d_c, stream: int = 0) -> None:
        _check(L.load().irodori_op_gemm_fp8(d_a, d_as, d_w, d_ws, M, N, K, d_c, stream or None))

    @staticmethod
    def sdpa(dtype: int, d_q, d_k, d_v, d_mask, batch, heads, seq_q, seq_kv, head_dim, scale,
             d_out, stream: int = 0) -> None:
        _check(L.load().irodori_op_sdpa(dtype, d_q, d_k, d_v, d_mask or None, batch, heads, seq_q,
                                        seq_kv, head_dim, scale, d_out, stream or None))

    @staticmethod
    def sdpa_noalloc(dtype: int, d_q, d_k, d_v, d_mask, batch, heads, seq_q, seq_kv, head_dim, scale,
                     d_out, stream: int = 0) -> None:
        """sdpa without any device allocation: the staging lives in the library's fixed
        per-GPU buffer (SDPA_SCRATCH_BYTES); overlapping calls on one GPU race."""
        _check(L.load().irodori_op_sdpa_noalloc(dtype, d_q, d_k, d_v, d_mask or None, batch, heads, seq_q,
                                                seq_kv, head_dim, scale, d_out, stream or None))
