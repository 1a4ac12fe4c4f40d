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

    @property
    def label(self) -> str:
        return {"hip-bf16": "HIP bf16 (gfx950)", "hip-f32": "HIP f32 (gfx950)"}[self.value]

    @property
    def is_reduced_precision(self) -> bool:
        return self is InferenceBackendKind.HIP_BF16


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
    """4 layers, d=256, 4x64 heads, SwiGLU 704, latent 32."""
    return DitConfig(latent_dim=32, model_dim=256, num_layers=4, num_heads=4, mlp_hidden=704,
                     adaln_rank=64, timestep_embed_dim=256, norm_eps=1e-5)


def cfg_full_rf() -> DitConfig:
    """12 layers, d=1024, 16x64 heads, SwiGLU 2816, latent 32."""
    return DitConfig(latent_dim=32, model_dim=1024, num_layers=12, num_heads=16,
                     mlp_hidden=2816, adaln_rank=256, timestep_embed_dim=512, norm_eps=1e-5)


def cfg_tiny() -> DitConfig:
    """Shape of the reference's tiny_model_config (src/config/model.rs:285-313) with
    head_dim 64: small enough for brute-force checks."""
    return DitConfig(latent_dim=8, model_dim=128, num_layers=2, num_heads=2, mlp_hidden=256,
                     adaln_rank=16, timestep_embed_dim=32, norm_eps=1e-5)


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
class SamplerParams:
    """src/rf/params.rs:61-92 (defaults :77-90)."""

    num_steps: int = 40
    method: SamplerMethod = SamplerMethod.EULER
    guidance: GuidanceConfig = field(default_factory=GuidanceConfig)
    truncation_factor: float | None = None
    use_context_kv_cache: bool = True

    def validate(self, has_speaker: bool = True) -> None:
        """params.rs:99-183 and the Joint equal-scale rule (euler_sampler.rs:209-228)."""
        if self.num_steps == 0:
            raise IrodoriError("Config", "num_steps must be > 0")
        g = self.guidance
        for name, s in (("guidance.scale_text", g.scale_text),
                        ("guidance.scale_caption", g.scale_caption),
                        ("guidance.scale_speaker", g.scale_speaker)):
            if not math.isfinite(s):
                raise IrodoriError("Config", "%s must be finite, got %s" % (name, s))
        if not (math.isfinite(g.min_t) and math.isfinite(g.max_t)):
            raise IrodoriError("Config", "guidance min_t/max_t must be finite")
        if g.min_t > g.max_t:
            raise IrodoriError("Config", "guidance.min_t must be <= guidance.max_t")
        if self.truncation_factor is not None and not (
                math.isfinite(self.truncation_factor) and self.truncation_factor > 0):
            raise IrodoriError("Config", "truncation_factor must be finite and > 0")
        if g.mode is CfgGuidanceMode.JOINT:
            active = [s for s in (g.scale_text, g.scale_speaker if has_speaker else 0.0) if s > 0]
            if active and max(active) - min(active) >= 1e-6:
                raise IrodoriError(
                    "Config",
                    "cfg_guidance_mode=Joint requires all active cfg scales to be equal, but got "
                    "text=%s, speaker=%s, caption=%s" % (g.scale_text, g.scale_speaker,
                                                        g.scale_caption))

    def joint_scale(self, has_speaker: bool = True) -> float:
        g = self.guidance
        for s in (g.scale_text, g.scale_speaker if has_speaker else 0.0):
            if s > 0:
                return s
        return 0.0

    def t_schedule(self) -> list[float]:
        """euler_sampler.rs:325-328, computed in f32: t_i = 0.999 * (1 - i/N), i = 0..N."""
        import numpy as np
        n = np.float32(self.num_steps)
        return [float(np.float32(0.999) * (np.float32(1.0) - np.float32(i) / n))
                for i in range(self.num_steps + 1)]
