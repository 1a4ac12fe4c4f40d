"""irodori_hip — MI355X (gfx950) RF-step DiT forward for Irodori-TTS behind a C ABI.

Host-side mirror of the reference's inference API for the HIP backend:
`InferenceBackendKind.HIP_BF16 / HIP_F32`, `SamplerParams`, `GuidanceConfig`, and
`HipInferenceEngine` (forward_with_cond_cached / sample over libirodori_hip.so), and the
request-level `InferenceBuilder` -> `InferenceEngine.sample(SamplingRequest)`.
"""
from .config import (CfgGuidanceMode, CodecConfig, DitConfig, EncoderConfig, GuidanceConfig,
                     InferenceBackendKind, IrodoriError, SamplerMethod, SamplerParams,
                     cfg_cpu_plumbing, cfg_full_rf, cfg_published_500m, cfg_tiny, codec_default, codec_tiny,
                     enc_speaker_default, enc_speaker_tiny, enc_text_default, enc_text_tiny)
from .engine import HipDacVaeCodec, HipEncoder, HipInferenceEngine, ops
from .inference import InferenceBuilder, InferenceEngine, ModelConfig, ModelWeights, SamplingRequest
from .synthetic import (ROLE_COND, ROLE_NO_AUX, ROLE_NO_TEXT, ROLE_UNCOND, CodecWeights, ContextKV,
                        CtxProjWeights, DitWeights, EncoderWeights, make_context_kv, make_noise,
                        make_role_context)

__all__ = [
    "CfgGuidanceMode", "DitConfig", "GuidanceConfig", "InferenceBackendKind", "IrodoriError",
    "SamplerMethod", "SamplerParams", "cfg_cpu_plumbing", "cfg_full_rf", "cfg_published_500m", "cfg_tiny",
    "HipInferenceEngine", "HipEncoder", "ops", "ContextKV", "CtxProjWeights", "DitWeights", "make_context_kv", "make_noise",
    "make_role_context", "ROLE_COND", "ROLE_UNCOND", "ROLE_NO_TEXT", "ROLE_NO_AUX",
    "EncoderConfig", "EncoderWeights", "enc_text_default", "enc_speaker_default", "enc_text_tiny",
    "enc_speaker_tiny", "CodecConfig", "CodecWeights", "HipDacVaeCodec", "codec_default",
    "codec_tiny", "InferenceBuilder", "InferenceEngine", "ModelConfig", "ModelWeights", "SamplingRequest",
]
