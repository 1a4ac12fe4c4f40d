"""C-ABI surface tests that need no GPU: the library loads, exports every symbol the
header declares, validates arguments before touching a device, and maps failures onto
status codes + irodori_last_error() (never aborting)."""
import ctypes as C
import math
import re

import numpy as np
import pytest
import torch

import irodori_hip as ih
from irodori_hip import _lib as L
from irodori_hip.engine import sampler_params_c, validate_sampler_params


def _declared_symbols():
    text = open(L.HEADER_PATH).read()
    return set(re.findall(r"^\s*(?:int|const char\s*\*)\s*(irodori_\w+)\s*\(", text, re.M))


def test_library_exports_every_declared_symbol():
    lib = L.load()
    declared = _declared_symbols()
    assert len(declared) >= 17
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(L.SIGNATURES), declared ^ set(L.SIGNATURES)


def test_version_string():
    assert b"gfx950" in L.load().irodori_version()


def _joint(**kw):
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=3.0, scale_speaker=3.0,
                          min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=40, guidance=g)
    for k, v in kw.items():
        if hasattr(g, k):
            setattr(g, k, v)
        else:
            setattr(p, k, v)
    return p


def test_params_valid_joint():
    validate_sampler_params(_joint())


@pytest.mark.parametrize("kw,msg", [
    ({"num_steps": 0}, "num_steps must be > 0"),
    ({"scale_text": math.nan}, "scale_text must be finite"),
    ({"scale_caption": math.inf}, "scale_caption must be finite"),
    ({"min_t": -0.1}, "min_t must be finite and in [0, 1]"),
    ({"max_t": 1.5}, "max_t must be finite and in [0, 1]"),
    ({"min_t": 0.8, "max_t": 0.2}, "must not exceed"),
    ({"truncation_factor": 0.0}, "truncation_factor"),
    ({"scale_speaker": 5.0}, "Joint requires all active cfg scales to be equal"),
])
def test_params_invalid(kw, msg):
    # params.rs:99-183 and euler_sampler.rs:209-228
    with pytest.raises(ih.IrodoriError) as ei:
        validate_sampler_params(_joint(**kw))
    assert ei.value.kind == "Config" and msg in str(ei.value)


def test_params_joint_scale_ignores_speaker_without_speaker_model():
    validate_sampler_params(_joint(scale_speaker=5.0), has_speaker=False)


def test_params_plms4_alternating_rejected():
    p = _joint(method=ih.SamplerMethod.PLMS4)
    p.guidance.mode = ih.CfgGuidanceMode.ALTERNATING
    with pytest.raises(ih.IrodoriError, match="PLMS4"):
        validate_sampler_params(p)


def test_null_arguments_rejected():
    lib = L.load()
    h = C.c_void_p()
    assert lib.irodori_ctx_create(0, None, C.byref(h)) == L.ERR_INVALID_ARG
    assert "null" in L.last_error()
    assert lib.irodori_sampler_params_validate(None) == L.ERR_INVALID_ARG
    assert lib.irodori_op_rms_norm(None, None, 4, 4, 1e-5, None, None) == L.ERR_INVALID_ARG
    assert lib.irodori_op_sdpa(L.DTYPE_BF16, None, None, None, None, 1, 1, 1, 1, 64, 1.0, None,
                               None) == L.ERR_INVALID_ARG
    assert lib.irodori_forward(None, 1, 1, None, None, None, None) == L.ERR_INVALID_ARG


def test_op_shape_and_dtype_errors_before_any_device_call():
    lib = L.load()
    p = C.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.irodori_op_sdpa(7, p, p, p, None, 1, 1, 1, 1, 64, 1.0, p, None) == L.ERR_DTYPE
    assert lib.irodori_op_sdpa(L.DTYPE_F32, p, p, p, None, 1, 1, 1, 1, 96, 1.0, p, None) == L.ERR_SHAPE
    assert lib.irodori_op_fused_adaln(p, p, p, 0, 4, 4, 1e-5, p, None) == L.ERR_SHAPE


@pytest.mark.parametrize("field,value,code", [
    ("head_dim", 96, L.ERR_SHAPE),
    ("mlp_hidden", 0, L.ERR_SHAPE),
    ("compute_dtype", 9, L.ERR_DTYPE),
    ("norm_eps", 0.0, L.ERR_CONFIG),
    ("latent_dim", 257, L.ERR_SHAPE),
    ("model_dim", 4160, L.ERR_SHAPE),
    ("max_rows", 65536, L.ERR_SHAPE),
])
def test_ctx_create_config_errors(field, value, code):
    lib = L.load()
    cfg = ih.cfg_cpu_plumbing()
    c = L.DitConfigC(cfg.latent_dim, cfg.model_dim, cfg.num_layers, cfg.num_heads, cfg.head_dim,
                     cfg.mlp_hidden, cfg.adaln_rank, cfg.timestep_embed_dim, cfg.norm_eps,
                     cfg.rope_theta, L.DTYPE_BF16, 2, 64, 48)
    setattr(c, field, value)
    h = C.c_void_p()
    assert lib.irodori_ctx_create(0, C.byref(c), C.byref(h)) == code
    assert not h.value
    assert L.last_error()


def _plumbing_cfg_c(dtype, max_seq, max_ctx):
    cfg = ih.cfg_cpu_plumbing()
    return L.DitConfigC(cfg.latent_dim, cfg.model_dim, cfg.num_layers, cfg.num_heads, cfg.head_dim,
                        cfg.mlp_hidden, cfg.adaln_rank, cfg.timestep_embed_dim, cfg.norm_eps,
                        cfg.rope_theta, dtype, 2, max_seq, max_ctx)


@pytest.mark.parametrize("dtype", [L.DTYPE_BF16, L.DTYPE_FP8])
def test_ctx_create_refuses_more_keys_than_the_attention_lists(dtype):
    # 16-bit attention: ceil(max_seq / 64) + ceil(max_ctx / 64) <= 256 key tiles, checked
    # at create (before any device call), so a long request never fails inside a launch.
    lib = L.load()
    h = C.c_void_p()
    c = _plumbing_cfg_c(dtype, 16384 - 64 + 1, 64)  # 256 + 1 tiles
    assert lib.irodori_ctx_create(0, C.byref(c), C.byref(h)) == L.ERR_SHAPE
    assert "16384 keys" in L.last_error() and not h.value


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error path")
def test_ctx_create_key_limit_boundary_reaches_the_device_check():
    # 255 latent tiles + 1 context tile pass the shape checks (the call then fails for want
    # of a device here); so does an f32 context far past the limit (its attention has none).
    lib = L.load()
    h = C.c_void_p()
    for dtype, S, T in ((L.DTYPE_BF16, 16320, 64), (L.DTYPE_F32, 40000, 3000)):
        c = _plumbing_cfg_c(dtype, S, T)
        assert lib.irodori_ctx_create(0, C.byref(c), C.byref(h)) == L.ERR_HIP, L.last_error()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error path")
def test_ctx_create_without_device_fails_cleanly():
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipInferenceEngine(ih.cfg_cpu_plumbing())
    assert ei.value.kind == "Hip" and "no HIP device" in str(ei.value)


def test_sampler_params_struct_roundtrip():
    p = _joint(truncation_factor=0.8)
    c = sampler_params_c(p)
    assert c.num_steps == 40 and c.cfg_mode == L.CFG_JOINT and c.has_truncation == 1
    assert abs(c.truncation_factor - 0.8) < 1e-7 and c.min_t == 0.0 and c.max_t == 1.0


def test_t_schedule_endpoints_and_uniformity():
    # euler_sampler.rs:731-766: t_0 = 0.999, t_N = 0, uniform spacing.
    s = ih.SamplerParams(num_steps=40).t_schedule()
    assert len(s) == 41 and abs(s[0] - 0.999) < 1e-7 and s[-1] == 0.0
    d = np.diff(np.asarray(s, np.float64))
    assert np.allclose(d, -0.999 / 40, atol=1e-6)


@pytest.mark.parametrize("env,expect", [(None, 0), ("0", 0), ("1", 1)])
def test_roctx_ranges_are_opt_in(env, expect):
    # The NVTX-named roctx ranges load the roctx library only with IRODORI_ROCTX=1 (read at
    # the first range); a fresh process per setting, since the choice is made once.
    import os
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); from irodori_hip import _lib as L; "
            "print(L.load().irodori_roctx_enabled())" % os.path.join(os.path.dirname(L.__file__), ".."))
    e = dict(os.environ)
    e.pop("IRODORI_ROCTX", None)
    if env is not None:
        e["IRODORI_ROCTX"] = env
    out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == str(expect)
