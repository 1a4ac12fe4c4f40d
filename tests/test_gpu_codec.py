"""GPU parity of the DACVAE decoder (irodori_codec_*: DacVaeCodec::decode, codec/model.rs:60-65)
against the oracle's codec_decode (pinned in test_oracle_codec.py), through the C ABI on the
same seeded inputs.

Bars (relative L2 on the waveform): f32 1e-4; bf16 2e-2 (bf16 operands for every
convolution of the ~40 in the chain, f32 accumulation and residual stream).  The
benchmark's 750-frame row is tied to the oracle through its prefix: the decoder's receptive
field spans about 8 latent frames (stem +-3, block 0's units +-39 samples at 12 per frame,
the later blocks less), so the first 14 frames' samples of a 750-frame decode equal those
of a 24-frame decode, which the oracle computes in seconds.
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL = {F32: 1e-4, BF16: 2e-2}

CONFIGS = {
    "tiny": ih.codec_tiny,  # rates 3 (odd) and 4; channels 192 -> 96 (K slices straddling taps) -> 48 (padded to 64)
    "even": lambda: ih.CodecConfig(latent_dim=4, proj_dim=32, decoder_dim=64, rates=(2, 4)),
    # out_proj at the latent limit (its 8 staged latent rows fill 32 KB of LDS) onto 40
    # channels padded to 64 (a channel block only partly real).
    "wide_latent": lambda: ih.CodecConfig(latent_dim=1024, proj_dim=40, decoder_dim=64, rates=(2, 4)),
}


def latent(cfg, B, T, seed):
    return np.random.default_rng(seed).standard_normal((B, T, cfg.latent_dim)).astype(np.float32)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(CONFIGS))
def test_codec_vs_oracle(oracle64, name, backend):
    cfg = CONFIGS[name]()
    cw = ih.CodecWeights.random(cfg, 2, bias=name == "tiny")
    lat = latent(cfg, 2, 37, 3)
    with ih.HipDacVaeCodec(cfg, backend, max_frames=40) as codec:
        codec.load_weights(cw)
        assert codec.hop_length() == cfg.hop_length
        got = codec.decode(lat)
        again = codec.decode(lat[1:, :20])  # smaller second call on the same buffers
    ref = oracle64.codec_decode(cfg, cw, lat)
    err = rel_l2(got, ref)
    print(name, backend.value, "rel L2 %.2e" % err)
    assert got.shape == ref.shape and err < TOL[backend]
    ref2 = oracle64.codec_decode(cfg, cw, lat[1:, :20])
    assert rel_l2(again, ref2) < TOL[backend]


@pytest.mark.parametrize("frames", [1, 2])
@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_shortest_latents(oracle64, backend, frames):
    # One and two latent frames: every convolution reads mostly zero padding (the halos),
    # the transposed convolutions' first and last windows are partial.
    cfg = ih.codec_tiny()
    cw = ih.CodecWeights.random(cfg, 11)
    lat = latent(cfg, 2, frames, 12)
    with ih.HipDacVaeCodec(cfg, backend, max_frames=4) as codec:
        codec.load_weights(cw)
        got = codec.decode(lat)
    ref = oracle64.codec_decode(cfg, cw, lat)
    assert got.shape == ref.shape == (2, 1, frames * cfg.hop_length)
    assert rel_l2(got, ref) < TOL[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_reference_widths_short(oracle64, backend):
    # The reference's decoder (1024 -> 1536 -> 768 -> 384 -> 192 -> 96, rates 12/10/8/2) on
    # 6 latent frames (11520 samples).
    cfg = ih.codec_default()
    cw = ih.CodecWeights.random(cfg, 4)
    lat = latent(cfg, 1, 6, 5)
    with ih.HipDacVaeCodec(cfg, backend, max_frames=6) as codec:
        codec.load_weights(cw)
        got = codec.decode(lat)
    ref = oracle64.codec_decode(cfg, cw, lat)
    err = rel_l2(got, ref)
    print("reference widths", backend.value, "rel L2 %.2e" % err)
    assert err < TOL[backend]


def test_full_utterance_prefix_vs_oracle(oracle32):
    # The benchmark's utterance length (750 frames -> 1.44 M samples) in bf16: finite, in [-1, 1],
    # two rows decoded together equal each decoded alone (bit for bit), and the first 14
    # frames match the oracle's 24-frame decode at the bf16 bar.
    cfg = ih.codec_default()
    cw = ih.CodecWeights.random(cfg, 6)
    lat = latent(cfg, 2, 750, 7)
    with ih.HipDacVaeCodec(cfg, BF16, max_frames=750) as codec:
        codec.load_weights(cw)
        both = codec.decode(lat)
        one = codec.decode(lat[1:])
    assert both.shape == (2, 1, 750 * 1920)
    assert np.isfinite(both).all() and np.abs(both).max() <= 1.0
    assert np.array_equal(both[1:], one)
    ref = oracle32.codec_decode(cfg, cw, lat[:1, :24])
    n = 14 * cfg.hop_length
    err = rel_l2(both[0, 0, :n], ref[0, 0, :n])
    print("750-frame prefix vs oracle rel L2 %.2e" % err)
    assert err < TOL[BF16]


def test_device_entry_point_matches_host():
    import torch
    cfg = ih.codec_tiny()
    cw = ih.CodecWeights.random(cfg, 8)
    lat = latent(cfg, 2, 16, 9)
    with ih.HipDacVaeCodec(cfg, BF16, max_frames=16) as codec:
        codec.load_weights(cw)
        host = codec.decode(lat)
        d_lat = torch.from_numpy(lat).cuda()
        d_wav = torch.empty((2, 16 * cfg.hop_length), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        codec.decode_device(d_lat.data_ptr(), 2, 16, d_wav.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    assert np.array_equal(d_wav.cpu().numpy(), host[:, 0])


def test_codec_errors_are_reported():
    cfg = ih.codec_tiny()
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipDacVaeCodec(ih.CodecConfig(latent_dim=4, proj_dim=32, decoder_dim=64, rates=(1, 4)), F32)
    assert ei.value.kind == "Config"  # rate 1
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipDacVaeCodec(ih.CodecConfig(latent_dim=4, proj_dim=32, decoder_dim=72, rates=(2, 2)), F32)
    assert ei.value.kind == "Shape"  # channels do not halve to multiples of 8
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipDacVaeCodec(ih.CodecConfig(latent_dim=1025, proj_dim=32, decoder_dim=64, rates=(2, 4)), F32)
    assert ei.value.kind == "Shape" and "latent_dim" in str(ei.value)
    # At the reference widths the 192-channel stream of 6000 latent frames is 960 x 6000 x 192
    # f32 values (4.4 GB), more than one GEMM operand may span: refused at creation.
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipDacVaeCodec(ih.codec_default(), F32, max_frames=6000)
    assert ei.value.kind == "Shape" and "max_frames" in str(ei.value)
    with ih.HipDacVaeCodec(cfg, F32, max_frames=8) as codec:
        lat = latent(cfg, 1, 8, 0)
        with pytest.raises(ih.IrodoriError) as ei:
            codec.decode(lat)
        assert ei.value.kind == "NotLoaded"
        codec.load_weights(ih.CodecWeights.random(cfg, 0))
        with pytest.raises(ih.IrodoriError) as ei:
            codec.decode(latent(cfg, 1, 9, 0))
        assert ei.value.kind == "Shape"
