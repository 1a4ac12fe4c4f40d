"""ctypes binding of libirodori_hip.so (include/irodori_hip.h).

The library is built in-tree (irodori-tts-burn_amd/_build/libirodori_hip.so) by
`make -C irodori-tts-burn_amd` / __graft_entry__.build().  Loading fails loudly when it
is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "_build", "libirodori_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_ROOT), "include", "irodori_hip.h")

OK = 0
ERR_INVALID_ARG = 1
ERR_SHAPE = 2
ERR_DTYPE = 3
ERR_HIP = 4
ERR_OOM = 5
ERR_NOT_LOADED = 6
ERR_CONFIG = 7
ERR_NAMES = {ERR_INVALID_ARG: "InvalidArg", ERR_SHAPE: "Shape", ERR_DTYPE: "Dtype",
             ERR_HIP: "Hip", ERR_OOM: "OutOfMemory", ERR_NOT_LOADED: "NotLoaded",
             ERR_CONFIG: "Config"}

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_FP8 = 2
DTYPE_F16 = 3  # irodori_op_sdpa operands only (native_fa_sdpa_f16_in)
SDPA_SCRATCH_BYTES = 16 << 20  # IRODORI_SDPA_SCRATCH_BYTES
CFG_INDEPENDENT, CFG_JOINT, CFG_ALTERNATING = 0, 1, 2
METHOD_EULER, METHOD_HEUN, METHOD_PLMS4 = 0, 1, 2

_f32p = C.POINTER(C.c_float)


class DitConfigC(C.Structure):
    _fields_ = [
        ("latent_dim", C.c_int32), ("model_dim", C.c_int32), ("num_layers", C.c_int32),
        ("num_heads", C.c_int32), ("head_dim", C.c_int32), ("mlp_hidden", C.c_int32),
        ("adaln_rank", C.c_int32), ("timestep_embed_dim", C.c_int32), ("norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("compute_dtype", C.c_int32), ("max_rows", C.c_int32),
        ("max_seq", C.c_int32), ("max_ctx", C.c_int32),
    ]


class BlockWeightsC(C.Structure):
    _fields_ = [
        ("w_qkv", _f32p), ("w_gate", _f32p), ("w_o", _f32p), ("q_norm", _f32p),
        ("k_norm", _f32p), ("w13", _f32p), ("w2", _f32p),
        ("ada_down", (_f32p * 3) * 2), ("ada_up", (_f32p * 3) * 2), ("ada_up_b", (_f32p * 3) * 2),
    ]


class IoWeightsC(C.Structure):
    _fields_ = [
        ("cond_w0", _f32p), ("cond_w1", _f32p), ("cond_w2", _f32p), ("in_w", _f32p),
        ("in_b", _f32p), ("out_norm_w", _f32p), ("out_w", _f32p), ("out_b", _f32p),
    ]


class SamplerParamsC(C.Structure):
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


class CtxProjWeightsC(C.Structure):
    _fields_ = [("wk_text", _f32p), ("wv_text", _f32p), ("wk_aux", _f32p), ("wv_aux", _f32p)]


class EncoderConfigC(C.Structure):
    _fields_ = [("dim", C.c_int32), ("num_layers", C.c_int32), ("num_heads", C.c_int32),
                ("mlp_hidden", C.c_int32), ("vocab_size", C.c_int32), ("in_dim", C.c_int32),
                ("mean_token", C.c_int32), ("norm_eps", C.c_float), ("compute_dtype", C.c_int32),
                ("max_rows", C.c_int32), ("max_seq", C.c_int32)]


class EncoderIoWeightsC(C.Structure):
    _fields_ = [("embedding", _f32p), ("in_w", _f32p), ("in_b", _f32p), ("out_norm", _f32p)]


ENC_BLOCK_FIELDS = ("attn_norm", "wq", "wk", "wv", "wo", "w_gate", "q_norm", "k_norm", "mlp_norm",
                    "w13", "w2")


class EncoderBlockWeightsC(C.Structure):
    _fields_ = [(n, _f32p) for n in ENC_BLOCK_FIELDS]


CODEC_MAX_BLOCKS = 8


class CodecConfigC(C.Structure):
    _fields_ = [("latent_dim", C.c_int32), ("proj_dim", C.c_int32), ("decoder_dim", C.c_int32),
                ("num_blocks", C.c_int32), ("rates", C.c_int32 * CODEC_MAX_BLOCKS),
                ("compute_dtype", C.c_int32), ("max_frames", C.c_int32)]


class CodecBlockWeightsC(C.Structure):
    _fields_ = [("alpha", _f32p), ("convt_w", _f32p), ("convt_b", _f32p),
                ("res_alpha0", _f32p * 3), ("res_conv_w", _f32p * 3), ("res_conv_b", _f32p * 3),
                ("res_alpha1", _f32p * 3), ("res_pw_w", _f32p * 3), ("res_pw_b", _f32p * 3)]


class CodecWeightsC(C.Structure):
    _fields_ = [("out_proj_w", _f32p), ("out_proj_b", _f32p), ("stem_w", _f32p), ("stem_b", _f32p),
                ("blocks", C.POINTER(CodecBlockWeightsC)), ("head_alpha", _f32p), ("head_w", _f32p),
                ("head_b", _f32p)]


class KernelTimesC(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("norm_mod_us", "qkvg_gemm_us", "attention_us",
                                          "wo_gemm_us", "w13_gemm_us", "w2_gemm_us", "final_us")]


# name -> (restype, argtypes): every symbol include/irodori_hip.h declares.
_vp = C.c_void_p
SIGNATURES = {
    "irodori_last_error": (C.c_char_p, []),
    "irodori_version": (C.c_char_p, []),
    "irodori_roctx_enabled": (C.c_int, []),
    "irodori_sampler_params_validate": (C.c_int, [C.POINTER(SamplerParamsC)]),
    "irodori_ctx_create": (C.c_int, [C.c_int, C.POINTER(DitConfigC), C.POINTER(_vp)]),
    "irodori_ctx_destroy": (C.c_int, [_vp]),
    "irodori_ctx_device_bytes": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "irodori_load_io_weights": (C.c_int, [_vp, C.POINTER(IoWeightsC)]),
    "irodori_load_block_weights": (C.c_int, [_vp, C.c_int, C.POINTER(BlockWeightsC)]),
    "irodori_set_ctx_kv": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p,
                                     C.POINTER(C.c_uint8)]),
    "irodori_clear_ctx_kv": (C.c_int, [_vp]),
    "irodori_load_ctx_proj_weights": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int,
                                                C.POINTER(CtxProjWeightsC)]),
    "irodori_build_ctx_kv": (C.c_int, [_vp, C.c_int, C.c_int, _f32p, C.POINTER(C.c_uint8),
                                       C.c_int, _f32p, C.POINTER(C.c_uint8)]),
    "irodori_read_ctx_kv": (C.c_int, [_vp, C.c_int, C.c_int, _f32p, _f32p, C.POINTER(C.c_uint8)]),
    "irodori_forward": (C.c_int, [_vp, C.c_int, C.c_int, _f32p, _f32p, _f32p, _f32p]),
    "irodori_forward_masked": (C.c_int, [_vp, C.c_int, C.c_int, _f32p, _f32p,
                                         C.POINTER(C.c_uint8), _f32p, _f32p]),
    "irodori_block_forward": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p]),
    "irodori_sample": (C.c_int, [_vp, C.POINTER(SamplerParamsC), C.c_int, C.c_int, _f32p,
                                 _f32p]),
    "irodori_sample_masked": (C.c_int, [_vp, C.POINTER(SamplerParamsC), C.c_int, C.c_int,
                                        C.POINTER(C.c_int32), _f32p, _f32p]),
    "irodori_sample_device": (C.c_int, [_vp, C.POINTER(SamplerParamsC), C.c_int, C.c_int,
                                        _vp, _vp]),
    "irodori_sample_device_masked": (C.c_int, [_vp, C.POINTER(SamplerParamsC), C.c_int, C.c_int,
                                               C.POINTER(C.c_int32), _vp, _vp]),
    "irodori_profile_layer": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.POINTER(KernelTimesC)]),
    "irodori_encoder_create": (C.c_int, [C.c_int, C.POINTER(EncoderConfigC), C.POINTER(_vp)]),
    "irodori_encoder_destroy": (C.c_int, [_vp]),
    "irodori_encoder_load_io_weights": (C.c_int, [_vp, C.POINTER(EncoderIoWeightsC)]),
    "irodori_encoder_load_block_weights": (C.c_int, [_vp, C.c_int, C.POINTER(EncoderBlockWeightsC)]),
    "irodori_encoder_forward": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(C.c_int32), _f32p,
                                          C.POINTER(C.c_uint8), _f32p, C.POINTER(C.c_uint8)]),
    "irodori_codec_create": (C.c_int, [C.c_int, C.POINTER(CodecConfigC), C.POINTER(_vp)]),
    "irodori_codec_destroy": (C.c_int, [_vp]),
    "irodori_codec_load_weights": (C.c_int, [_vp, C.POINTER(CodecWeightsC)]),
    "irodori_codec_hop_length": (C.c_int, [_vp]),
    "irodori_codec_decode": (C.c_int, [_vp, C.c_int, C.c_int, _f32p, _f32p]),
    "irodori_codec_decode_device": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp, _vp]),
    "irodori_op_rms_norm": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_float, _vp, _vp]),
    "irodori_op_fused_adaln": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_float,
                                         _vp, _vp]),
    "irodori_op_sdpa": (C.c_int, [C.c_int, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_int, C.c_float, _vp, _vp]),
    "irodori_op_sdpa_noalloc": (C.c_int, [C.c_int, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int,
                                          C.c_int, C.c_int, C.c_float, _vp, _vp]),
    "irodori_op_joint_attention": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "irodori_op_swiglu_mlp": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp]),
    "irodori_op_mx_quantize": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp, _vp]),
    "irodori_op_gemm_fp8": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
}

_lib = None


def load():
    """Load libirodori_hip.so; raises FileNotFoundError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                "libirodori_hip.so not built at %s (run __graft_entry__.build() or "
                "make -C irodori-tts-burn_amd)" % LIB_PATH)
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().irodori_last_error().decode("utf-8", "replace")
