"""Model / sampler configuration, mirroring the reference's Rust types.

`DitConfig` carries the ModelConfig fields the DiT forward uses
(src/config/model.rs:8-44, head_dim :226-228, patched_latent_dim :231-233).
`GuidanceConfig` / `SamplerParams` mirror src/rf/params.rs:9-35 and :61-92, and
`SamplerParams.validate` restates params.rs:99-183 plus the Joint-mode scale check of
src/rf/euler_sampler.rs:209-228.  `InferenceBackendKind` mirrors
src/backend_config.rs:319-365 with the two HIP variants this library adds.
"""
from __future__ import annotations

import enum
import math
from dataclasses import dataclass, field


class IrodoriError(Exception):
    """Mirror of IrodoriError (src/error.rs:4-60); `kind` names the variant."""

    def __init__(self, kind: str, msg: str):
        super().__init__("%s: %s" % (kind, msg))
        self.kind = kind


class InferenceBackendKind(enum.Enum):
    """Runtime backend selector (src/backend_config.rs:319-365) — HIP variants only here."""

    HIP_BF16 = "hip-bf16"
    HIP_F32 = "hip-f32"
    # bf16 activations with the block GEMMs on e4m3 operands (no reference counterpart).
    HIP_FP8 = "hip-fp8"

    @property
    def label(self) -> str:
        return {"hip-bf16": "HIP bf16 (gfx950)", "hip-f32": "HIP f32 (gfx950)",
                "hip-fp8": "HIP fp8 GEMMs + bf16 (gfx950)"}[self.value]

    @property
    def is_reduced_precision(self) -> bool:
        return self is not InferenceBackendKind.HIP_F32


class CfgGuidanceMode(enum.Enum):
    """src/config/sampling.rs:100-108."""

    INDEPENDENT = "independent"
    JOINT = "joint"
    ALTERNATING = "alternating"


class SamplerMethod(enum.Enum):
    """src/config/sampling.rs:8-20."""

    EULER = "euler"
    HEUN = "heun"
    PLMS4 = "plms4"


@dataclass
class DitConfig:
    latent_dim: int = 32          # patched latent dim (latent_dim * latent_patch_size)
    model_dim: int = 1024
    num_layers: int = 12
    num_heads: int = 16
    mlp_hidden: int = 2816
    adaln_rank: int = 256
    timestep_embed_dim: int = 512
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.model_dim // self.num_heads

    def validate(self) -> None:
        if self.model_dim % self.num_heads:
            raise IrodoriError("Config", "model_dim must be divisible by num_heads")
        if self.head_dim % 2:
            raise IrodoriError("Config", "head_dim must be even for RoPE")
        if not (self.norm_eps > 0):
            raise IrodoriError("Config", "norm_eps must be > 0")


def cfg_cpu_plumbing() -> DitConfig:
    """The CPU-plumbing configuration: 4 layers, d=256, 4x64 heads, SwiGLU 704, latent 32."""
    return DitConfig(latent_dim=32, model_dim=256, num_layers=4, num_heads=4, mlp_hidden=704,
                     adaln_rank=64, timestep_embed_dim=256, norm_eps=1e-5)


def cfg_full_rf() -> DitConfig:
    """The benchmark configuration: 12 layers, d=1024, 16x64 heads, SwiGLU 2816, latent 32."""
    return DitConfig(latent_dim=32, model_dim=1024, num_layers=12, num_heads=16,
                     mlp_hidden=2816, adaln_rank=256, timestep_embed_dim=512, norm_eps=1e-5)


def cfg_published_500m() -> DitConfig:
    """The shape of the published Irodori-TTS-500M-v2 checkpoint (docs/benchmarks/rtx-a6000.md:13-21:
    d 1280, 12 layers, 20 heads) with ModelConfig's default mlp_ratio 2.875
    (src/config/model.rs:54): SwiGLU hidden floor(1280 * 2.875) = 3680 (src/model/diffusion.rs:32);
    latents of the DACVAE codebook width 32 (src/codec/weights.rs:213)."""
    return DitConfig(latent_dim=32, model_dim=1280, num_layers=12, num_heads=20, mlp_hidden=3680,
                     adaln_rank=256, timestep_embed_dim=512, norm_eps=1e-5)


def cfg_tiny() -> DitConfig:
    """Shape of the reference's tiny_model_config (src/config/model.rs:285-313) with
    head_dim 64: small enough for brute-force checks."""
    return DitConfig(latent_dim=8, model_dim=128, num_layers=2, num_heads=2, mlp_hidden=256,
                     adaln_rank=16, timestep_embed_dim=32, norm_eps=1e-5)


@dataclass
class EncoderConfig:
    """A condition encoder and its conditioner norm: TextEncoder (text / caption,
    text_encoder.rs:64-148) when vocab_size > 0, ReferenceLatentEncoder (speaker,
    speaker_encoder.rs:85-162) when in_dim > 0; TextBlocks of width dim, num_heads heads of
    dim / num_heads (64 or 128), SwiGLU hidden floor(dim * mlp_ratio) (text_encoder.rs:36).
    mean_token: prepend the speaker conditioner's masked-mean token
    (aux_conditioner.rs:150-185)."""

    dim: int
    num_layers: int
    num_heads: int
    mlp_hidden: int
    norm_eps: float = 1e-5
    vocab_size: int = 0
    in_dim: int = 0
    mean_token: bool = False

    @property
    def head_dim(self) -> int:
        return self.dim // self.num_heads


def enc_text_default() -> EncoderConfig:
    """The reference's default text encoder (config/model.rs:46-80): 1280 wide, 14 layers,
    10 heads, mlp ratio 2.6, vocab 102400."""
    return EncoderConfig(dim=1280, num_layers=14, num_heads=10, mlp_hidden=int(1280 * 2.6),
                         vocab_size=102400)


def enc_speaker_default(latent_dim: int = 32) -> EncoderConfig:
    """The default speaker encoder over latent_dim-channel reference latents (patch 1)."""
    return EncoderConfig(dim=1280, num_layers=14, num_heads=10, mlp_hidden=int(1280 * 2.6),
                         in_dim=latent_dim, mean_token=True)


def enc_text_tiny() -> EncoderConfig:
    return EncoderConfig(dim=256, num_layers=2, num_heads=2, mlp_hidden=640, vocab_size=1000)


def enc_speaker_tiny() -> EncoderConfig:
    return EncoderConfig(dim=256, num_layers=2, num_heads=4, mlp_hidden=640, in_dim=32,
                         mean_token=True)


@dataclass
class CodecConfig:
    """The DACVAE decoder (codec/weights.rs:225-292): quantizer.out_proj latent_dim ->
    proj_dim (k 1), the stem proj_dim -> decoder_dim (k 7), one DecoderBlock per rate (the
    channels halve, ConvTranspose1d kernel 2 * rate), the watermark head to one channel.
    hop_length = prod(rates) waveform samples per latent frame (codec/model.rs)."""

    latent_dim: int = 32
    proj_dim: int = 1024
    decoder_dim: int = 1536
    rates: tuple = (12, 10, 8, 2)
    sample_rate: int = 48000

    @property
    def num_blocks(self) -> int:
        return len(self.rates)

    @property
    def hop_length(self) -> int:
        return int(math.prod(self.rates))

    def block_dims(self, i: int):
        """(in, out) channels of DecoderBlock i."""
        return self.decoder_dim >> i, self.decoder_dim >> (i + 1)

    @property
    def head_dim(self) -> int:
        return self.decoder_dim >> self.num_blocks


def codec_default() -> CodecConfig:
    """DACVAE as loaded by load_codec (weights.rs:268-292): 1536 -> 96 over rates 12/10/8/2."""
    return CodecConfig()


def codec_tiny() -> CodecConfig:
    """Small decoder for parity tests: an odd and an even rate, channels 192 -> 96 -> 48
    (both padded to a multiple of 64 on the GPU)."""
    return CodecConfig(latent_dim=8, proj_dim=64, decoder_dim=192, rates=(3, 4))


@dataclass
class GuidanceConfig:
    """src/rf/params.rs:9-35 (defaults :23-34)."""

    mode: CfgGuidanceMode = CfgGuidanceMode.INDEPENDENT
    scale_text: float = 3.0
    scale_caption: float = 3.0
    scale_speaker: float = 5.0
    min_t: float = 0.5
    max_t: float = 1.0


@dataclass
class TemporalRescaleConfig:
    """src/rf/params.rs:37-45 (arxiv:2510.01184); k and sigma are set together."""

    k: float
    sigma: float


@dataclass
class SpeakerKvConfig:
    """src/rf/params.rs:47-58: scale the speaker K/V of the context cache."""

    scale: float
    max_layers: int | None = None   # None = every layer
    min_t: float | None = None      # revert once t drops below it; None = never


@dataclass
class SamplerParams:
    """src/rf/params.rs:61-92 (defaults :77-90)."""

    num_steps: int = 40
    method: SamplerMethod = SamplerMethod.EULER
    guidance: GuidanceConfig = field(default_factory=GuidanceConfig)
    truncation_factor: float | None = None
    temporal_rescale: TemporalRescaleConfig | None = None
    speaker_kv: SpeakerKvConfig | None = None
    use_context_kv_cache: bool = True

    def validate(self, has_speaker: bool = True, has_caption: bool = False) -> None:
        """params.rs:99-183 and the Joint equal-scale rule (euler_sampler.rs:209-228)."""
        if self.num_steps == 0:
            raise IrodoriError("Config", "num_steps must be > 0")
        g = self.guidance
        for name, s in (("guidance.scale_text", g.scale_text),
                        ("guidance.scale_caption", g.scale_caption),
                        ("guidance.scale_speaker", g.scale_speaker)):
            if not math.isfinite(s):
                raise IrodoriError("Config", "%s must be finite, got %s" % (name, s))
        for name, t in (("guidance.min_t", g.min_t), ("guidance.max_t", g.max_t)):
            if not (math.isfinite(t) and 0.0 <= t <= 1.0):
                raise IrodoriError("Config", "%s must be finite and in [0, 1], got %s" % (name, t))
        if g.min_t > g.max_t:
            raise IrodoriError("Config", "guidance.min_t (%s) must not exceed guidance.max_t (%s)"
                               % (g.min_t, g.max_t))
        if self.truncation_factor is not None and not (
                math.isfinite(self.truncation_factor) and self.truncation_factor > 0):
            raise IrodoriError("Config", "truncation_factor must be finite and > 0")
        if self.temporal_rescale is not None:
            if not math.isfinite(self.temporal_rescale.k):
                raise IrodoriError("Config", "temporal_rescale.k must be finite")
            if self.temporal_rescale.sigma == 0.0:
                raise IrodoriError("Config", "temporal_rescale.sigma must not be zero")
        if self.speaker_kv is not None:
            skv = self.speaker_kv
            if not (math.isfinite(skv.scale) and skv.scale > 0):
                raise IrodoriError("Config", "speaker_kv.scale must be finite and > 0")
            if skv.min_t is not None and not (math.isfinite(skv.min_t) and 0.0 <= skv.min_t <= 1.0):
                raise IrodoriError("Config", "speaker_kv.min_t must be finite and in [0, 1]")
        if has_speaker and has_caption:
            # AuxConditioner is a speaker or a caption conditioner (aux_conditioner.rs:43-52).
            raise IrodoriError("Config", "has_speaker and has_caption are exclusive: the auxiliary "
                                         "condition is a speaker or a caption")
        if self.method is SamplerMethod.PLMS4 and g.mode is CfgGuidanceMode.ALTERNATING:
            raise IrodoriError("Config", "sampler PLMS4 is not compatible with "
                                         "cfg_guidance_mode=Alternating; use Independent or Joint instead")
        if g.mode is CfgGuidanceMode.JOINT:
            active = self.cfg_scales(has_speaker, has_caption)
            if active and max(active) - min(active) >= 1e-6:
                raise IrodoriError(
                    "Config",
                    "cfg_guidance_mode=Joint requires all active cfg scales to be equal, but got "
                    "text=%s, speaker=%s, caption=%s" % (g.scale_text, g.scale_speaker,
                                                        g.scale_caption))

    def cfg_signals(self, has_speaker: bool = True, has_caption: bool = False) -> list[str]:
        """Active CFG signals in the sampler's order (euler_sampler.rs:163-200): text if its
        scale is > 0, speaker if the condition holds a speaker state and its scale is > 0,
        caption if the condition holds a caption with a valid token and its scale is > 0."""
        g = self.guidance
        out = []
        if g.scale_text > 0:
            out.append("text")
        if has_speaker and g.scale_speaker > 0:
            out.append("speaker")
        if has_caption and g.scale_caption > 0:
            out.append("caption")
        return out

    def cfg_scales(self, has_speaker: bool = True, has_caption: bool = False) -> list[float]:
        g = self.guidance
        by = {"text": g.scale_text, "speaker": g.scale_speaker, "caption": g.scale_caption}
        return [by[n] for n in self.cfg_signals(has_speaker, has_caption)]

    def joint_scale(self, has_speaker: bool = True, has_caption: bool = False) -> float:
        sc = self.cfg_scales(has_speaker, has_caption)
        return sc[0] if sc else 0.0

    def cfg_roles(self, has_speaker: bool = True, has_caption: bool = False) -> list[str]:
        """The context bundles irodori_sample reads, in role order (row r * U + u): the
        conditioned bundle, then for Joint the fully unconditioned one, for Independent and
        Alternating one bundle per active signal with that signal dropped (text ->
        "no_text", speaker / caption -> "no_aux", euler_sampler.rs:41-85)."""
        sig = self.cfg_signals(has_speaker, has_caption)
        if self.guidance.mode is CfgGuidanceMode.JOINT:
            return ["cond", "uncond"] if sig else ["cond"]
        return ["cond"] + ["no_text" if s == "text" else "no_aux" for s in sig]

    def t_schedule(self) -> list[float]:
        """euler_sampler.rs:325-328, computed in f32: t_i = 0.999 * (1 - i/N), i = 0..N."""
        import numpy as np
        n = np.float32(self.num_steps)
        return [float(np.float32(0.999) * (np.float32(1.0) - np.float32(i) / n))
                for i in range(self.num_steps + 1)]
