"""InferenceBuilder / InferenceEngine: the reference's builder and request-level engine
(src/inference.rs:83-255) with its SamplingRequest (src/rf/params.rs:234-247), over the HIP
library.  One request runs end to end on the GPU:

  - the text tokens, and the reference latent or the caption tokens, through the condition
    encoders (irodori_encoder_*; text_encoder.rs, speaker_encoder.rs);
  - every CFG role's context bundle projected into each layer's K / V cache on the device
    (irodori_build_ctx_kv; attention.rs:431-501): the conditioned bundle, and per role the
    dropped signals as EncodedCondition::zeros_like (zero states, every key masked;
    condition.rs:144-154);
  - the graph-captured RF loop (irodori_sample; euler_sampler.rs:132-718).

The reference's builder is a typestate (Unconfigured -> Loaded -> Ready): calling a method
in the wrong state does not compile there, and raises IrodoriError("Config") here.  The
reference reads its weights from a safetensors checkpoint (load_model); here they are handed
over already loaded as host arrays (ModelWeights), the checkpoint format staying with the
caller.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from typing import Optional

import numpy as np

from .config import DitConfig, EncoderConfig, InferenceBackendKind, IrodoriError, SamplerParams
from .engine import HipEncoder, HipInferenceEngine
from .synthetic import CtxProjWeights, DitWeights, EncoderWeights


@dataclass
class ModelConfig:
    """The model's shapes (config/model.rs:8-82): the DiT, the text encoder and the optional
    auxiliary conditioner, a speaker encoder over reference latents (in_dim > 0) or a
    caption encoder over tokens (vocab_size > 0)."""

    dit: DitConfig
    text: EncoderConfig
    aux: Optional[EncoderConfig] = None

    @property
    def aux_kind(self) -> Optional[str]:
        if self.aux is None:
            return None
        return "caption" if self.aux.vocab_size else "speaker"


@dataclass
class ModelWeights:
    """Host weights of the whole conditioned model: the DiT, the encoders and every layer's
    context projections (wk / wv of the text and auxiliary segments)."""

    dit: DitWeights
    text: EncoderWeights
    ctx_proj: CtxProjWeights
    aux: Optional[EncoderWeights] = None


@dataclass
class SamplingRequest:
    """Mirror of SamplingRequest (src/rf/params.rs:234-247) on numpy arrays: text_ids /
    text_mask [B, T]; ref_latent [B, Tr, latent_dim] with ref_mask [B, Tr] (speaker models);
    caption_ids / caption_mask [B, Tc] (caption models); initial_noise [B, S, latent_dim]
    (None: drawn from N(0, 1) with the seed given to sample)."""

    text_ids: np.ndarray
    text_mask: np.ndarray
    sequence_length: int
    ref_latent: Optional[np.ndarray] = None
    ref_mask: Optional[np.ndarray] = None
    caption_ids: Optional[np.ndarray] = None
    caption_mask: Optional[np.ndarray] = None
    initial_noise: Optional[np.ndarray] = None


class InferenceBuilder:
    """InferenceBuilder::new(device) -> load_weights -> with_sampling / with_default_sampling
    -> build (src/inference.rs:91-200)."""

    def __init__(self, device: int = 0, backend: InferenceBackendKind = InferenceBackendKind.HIP_BF16):
        self._device, self._backend = device, backend
        self._state = "unconfigured"
        self._config: Optional[ModelConfig] = None
        self._weights: Optional[ModelWeights] = None
        self._params: Optional[SamplerParams] = None

    def _need(self, *states: str) -> None:
        if self._state not in states:
            raise IrodoriError("Config", "builder is %s; this call needs it %s" % (self._state, " or ".join(states)))

    def _next(self, state: str, **kw) -> "InferenceBuilder":
        b = InferenceBuilder(self._device, self._backend)
        b._state, b._config, b._weights, b._params = state, self._config, self._weights, self._params
        for k, v in kw.items():
            setattr(b, "_" + k, v)
        return b

    def load_weights(self, config: ModelConfig, weights: ModelWeights) -> "InferenceBuilder":
        self._need("unconfigured")
        config.dit.validate()
        if (config.aux is None) != (weights.aux is None):
            raise IrodoriError("Config", "the auxiliary conditioner's config and weights come together")
        if weights.ctx_proj.text_dim != config.text.dim or \
                weights.ctx_proj.aux_dim != (config.aux.dim if config.aux else 0):
            raise IrodoriError("Shape", "context projections do not match the encoder widths")
        return self._next("loaded", config=config, weights=weights)

    def model_config(self) -> ModelConfig:
        self._need("loaded", "ready")
        return self._config

    def with_sampling(self, params: SamplerParams) -> "InferenceBuilder":
        self._need("loaded", "ready")
        return self._next("ready", params=params)

    def with_default_sampling(self) -> "InferenceBuilder":
        return self.with_sampling(SamplerParams())

    def build(self, max_batch: int = 1, max_seq: int = 750, max_text: int = 256, max_aux: int = 375) -> "InferenceEngine":
        """The engine, with device buffers sized for requests of at most max_batch utterances
        of max_seq latent frames, max_text text tokens and max_aux reference frames or
        caption tokens."""
        self._need("ready")
        return InferenceEngine(self._config, self._weights, self._params, self._device, self._backend,
                               max_batch, max_seq, max_text, max_aux)


class _Model:
    """The GPU objects an engine and the engines derived from it by with_sampling share."""

    def __init__(self, config: ModelConfig, weights: ModelWeights, device: int, backend: InferenceBackendKind,
                 max_batch: int, max_seq: int, max_text: int, max_aux: int):
        enc_backend = InferenceBackendKind.HIP_F32 if backend is InferenceBackendKind.HIP_F32 \
            else InferenceBackendKind.HIP_BF16
        self.max_batch, self.max_seq, self.max_text, self.max_aux = max_batch, max_seq, max_text, max_aux
        self.text = HipEncoder(config.text, enc_backend, max_rows=max_batch, max_seq=max_text, device=device)
        self.text.load_weights(weights.text)
        self.aux = None
        max_ctx = max_text
        if config.aux is not None:
            self.aux = HipEncoder(config.aux, enc_backend, max_rows=max_batch, max_seq=max_aux, device=device)
            self.aux.load_weights(weights.aux)
            max_ctx += max_aux + int(config.aux.mean_token)
        # Up to three role bundles per utterance (Independent CFG with two signals).
        self.dit = HipInferenceEngine(config.dit, backend, max_rows=3 * max_batch, max_seq=max_seq,
                                      max_ctx=max_ctx, device=device)
        self.dit.load_weights(weights.dit)
        self.dit.load_ctx_proj_weights(weights.ctx_proj)

    def close(self) -> None:
        for m in (self.dit, self.text, self.aux):
            if m is not None:
                m.close()


class InferenceEngine:
    """InferenceEngine (src/inference.rs:206-255): sample(request) runs one request on the
    GPU and returns the denoised latent [B, sequence_length, latent_dim]."""

    def __init__(self, config: ModelConfig, weights: ModelWeights, params: SamplerParams, device: int,
                 backend: InferenceBackendKind, max_batch: int, max_seq: int, max_text: int, max_aux: int,
                 _model: Optional[_Model] = None):
        self._config, self._params, self._device, self._backend = config, params, device, backend
        self._m = _model or _Model(config, weights, device, backend, max_batch, max_seq, max_text, max_aux)

    def close(self) -> None:
        self._m.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def with_sampling(self, params: SamplerParams) -> "InferenceEngine":
        """A new engine with the same loaded model and other sampling parameters.  The
        reference's with_sampling consumes the engine; here both stay usable and share the
        GPU model, which close() on either releases."""
        return InferenceEngine(self._config, None, params, self._device, self._backend, 0, 0, 0, 0, _model=self._m)

    def model_config(self) -> ModelConfig:
        return self._config

    def sampling_params(self) -> SamplerParams:
        return self._params

    def device(self) -> int:
        return self._device

    def model(self) -> HipInferenceEngine:
        return self._m.dit

    def sample(self, request: SamplingRequest, seed: int = 0) -> np.ndarray:
        m, cfg, p = self._m, self._config, self._params
        ids = np.ascontiguousarray(request.text_ids, np.int32)
        if ids.ndim != 2:
            raise IrodoriError("Shape", "text_ids must be [batch, tokens]")
        B, Tt = ids.shape
        S = int(request.sequence_length)
        if not (0 < B <= m.max_batch and 0 < S <= m.max_seq and 0 < Tt <= m.max_text):
            raise IrodoriError("Shape", "request of %d utterances x %d frames x %d tokens exceeds the engine's "
                               "%d x %d x %d" % (B, S, Tt, m.max_batch, m.max_seq, m.max_text))
        tmask = np.ascontiguousarray(request.text_mask, np.uint8)
        if tmask.shape != (B, Tt):
            raise IrodoriError("Shape", "text_mask must match text_ids")

        # The auxiliary condition the request carries (aux_conditioner.rs:43-52).
        kind = cfg.aux_kind
        has_speaker = kind == "speaker" and request.ref_latent is not None
        has_caption = kind == "caption" and request.caption_ids is not None
        if request.ref_latent is not None and kind != "speaker":
            raise IrodoriError("UnsupportedMode", "the model has no speaker conditioner")
        if request.caption_ids is not None and kind != "caption":
            raise IrodoriError("UnsupportedMode", "the model has no caption conditioner")
        p.validate(has_speaker=has_speaker, has_caption=has_caption)

        aux_job = None
        if has_speaker:
            lat = np.ascontiguousarray(request.ref_latent, np.float32)
            rm = request.ref_mask if request.ref_mask is not None else np.ones(lat.shape[:2], np.uint8)
            if lat.shape[0] != B or lat.shape[1] > m.max_aux:
                raise IrodoriError("Shape", "ref_latent must be [batch, <= %d frames, latent_dim]" % m.max_aux)
            aux_job = lambda: m.aux.forward(np.ascontiguousarray(rm, np.uint8), latent=lat)  # noqa: E731
        elif has_caption:
            cids = np.ascontiguousarray(request.caption_ids, np.int32)
            cm = request.caption_mask if request.caption_mask is not None else np.ones(cids.shape, np.uint8)
            if cids.shape[0] != B or cids.shape[1] > m.max_aux:
                raise IrodoriError("Shape", "caption_ids must be [batch, <= %d tokens]" % m.max_aux)
            aux_job = lambda: m.aux.forward(np.ascontiguousarray(cm, np.uint8), ids=cids)  # noqa: E731
        # The two encoders are independent objects with streams of their own, and the library
        # calls release the GIL: the auxiliary one runs on a second host thread beside the text one.
        aux_state = aux_m = None
        if aux_job is None:
            text_state, text_m = m.text.forward(tmask, ids=ids)
        else:
            with ThreadPoolExecutor(max_workers=1) as pool:
                fut = pool.submit(aux_job)
                text_state, text_m = m.text.forward(tmask, ids=ids)
                aux_state, aux_m = fut.result()

        # One bundle per CFG role and utterance, role-major (row r * B + u): the role keeps or
        # drops the text and the auxiliary segment.
        roles = p.cfg_roles(has_speaker=has_speaker, has_caption=has_caption)
        m.dit.clear_context_kv()
        for r, role in enumerate(roles):
            keep_text = role in ("cond", "no_aux")
            keep_aux = role in ("cond", "no_text")
            for u in range(B):
                ts, tm = text_state[u], text_m[u]
                if not keep_text:
                    ts, tm = np.zeros_like(ts), np.zeros_like(tm)
                a_s = a_m = None
                if aux_state is not None:
                    a_s, a_m = aux_state[u], aux_m[u]
                    if not keep_aux:
                        a_s, a_m = np.zeros_like(a_s), np.zeros_like(a_m)
                m.dit.build_context_kv(r * B + u, ts, tm, a_s, a_m)

        P = cfg.dit.latent_dim
        if request.initial_noise is not None:
            x0 = np.ascontiguousarray(request.initial_noise, np.float32)
            if x0.shape != (B, S, P):
                raise IrodoriError("Shape", "initial_noise must be [batch, sequence_length, latent_dim]")
        else:
            x0 = np.random.default_rng(seed).standard_normal((B, S, P), dtype=np.float32)
        return m.dit.sample(x0, p, has_speaker=has_speaker, has_caption=has_caption, ctx_aux_start=Tt)
