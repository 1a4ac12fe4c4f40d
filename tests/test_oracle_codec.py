"""The oracle's DACVAE decoder (oracle_body.h conv1d / conv_transpose1d / snake /
codec_decode; codec/model.rs:60-65, decoder.rs, layers.rs, bottleneck.rs) pinned on the CPU.

The reference's codec tests hold no golden vectors, only properties (layers.rs:108-200:
Snake is 0 at 0 and >= x for x > 0, the ConvTranspose1d padding rule; decoder.rs:74-93:
the head's output lies in [-1, 1] with one channel), which are checked here.  The operators
are pinned against PyTorch's own convolutions (F.conv1d, F.conv_transpose1d, library
routines sharing no loop with the oracle), and the composition against the float64 torch
restatement in torch_reference.codec_decode, so a transposed weight, a wrong tap, padding
or dilation fails.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import irodori_hip as ih
import torch_reference as tr
from conftest import rel_l2


def t64(a):
    return torch.from_numpy(np.asarray(a)).double()


@pytest.mark.parametrize("k,dil,bias", [(7, 1, True), (7, 3, False), (7, 9, True), (1, 1, True)])
def test_conv1d_vs_torch(oracle64, k, dil, bias):
    rng = np.random.default_rng(k * 10 + dil)
    x = rng.standard_normal((6, 61)).astype(np.float32)
    w = rng.standard_normal((5, 6, k)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32) if bias else None
    pad = (k - 1) * dil // 2  # conv_pad(k, 1, dil) (layers.rs:57-59)
    got = oracle64.conv1d(x, w, b, dil, pad)
    ref = F.conv1d(t64(x)[None], t64(w), None if b is None else t64(b), padding=pad, dilation=dil)[0].numpy()
    assert got.shape == ref.shape == (5, 61)
    assert rel_l2(got, ref) < 1e-6


@pytest.mark.parametrize("stride", [2, 3, 4, 5, 8, 10, 12])
def test_conv_transpose1d_vs_torch(oracle64, stride):
    rng = np.random.default_rng(stride)
    x = rng.standard_normal((7, 13)).astype(np.float32)
    w = rng.standard_normal((7, 4, 2 * stride)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    pad, out_pad = (stride + 1) // 2, stride % 2  # conv_transpose_pad (layers.rs:62-65)
    got = oracle64.conv_transpose1d(x, w, b, stride, pad, out_pad)
    ref = F.conv_transpose1d(t64(x)[None], t64(w), t64(b), stride=stride, padding=pad,
                             output_padding=out_pad)[0].numpy()
    assert got.shape == ref.shape == (4, 13 * stride)  # the decoder's exact upsampling
    assert rel_l2(got, ref) < 1e-6


def test_transpose_padding_rule_values():
    # layers.rs:166-178: (12, 10, 8, 2) -> (6, 0), (5, 0), (4, 0), (1, 0); 3 -> (2, 1).
    rule = lambda s: ((s + 1) // 2, s % 2)
    assert [rule(s) for s in (12, 10, 8, 2, 3)] == [(6, 0), (5, 0), (4, 0), (1, 0), (2, 1)]


def test_snake_closed_forms(oracle32):
    a = np.array([1.0, 2.0, 0.5, 1.5], np.float32)
    assert not oracle32.snake(np.zeros((4, 8), np.float32), a).any()  # 0 at 0
    x = np.random.default_rng(0).uniform(0.01, 5.0, (4, 64)).astype(np.float32)
    assert (oracle32.snake(x, a) - x >= -1e-6).all()                     # >= x for x > 0
    # a x = pi / 2: sin^2 = 1, so snake = x + 1 / (a + 1e-9).
    xq = (np.pi / 2 / a)[:, None].astype(np.float32)
    got = oracle32.snake(xq, a)[:, 0]
    assert np.allclose(got, xq[:, 0] + 1.0 / a, rtol=1e-6)


@pytest.mark.parametrize("name", ["tiny", "even", "nobias", "wide_latent"])
def test_codec_decode_vs_torch(oracle64, name):
    # wide_latent: the latent (1024 channels, the library's limit) is the widest array of the
    # decode, so the oracle's scratch must be sized by it too.
    cfg = {"tiny": ih.codec_tiny(), "even": ih.CodecConfig(latent_dim=4, proj_dim=32, decoder_dim=64,
                                                               rates=(2, 4)),
           "nobias": ih.codec_tiny(),
           "wide_latent": ih.CodecConfig(latent_dim=1024, proj_dim=40, decoder_dim=64, rates=(2, 4))}[name]
    cw = ih.CodecWeights.random(cfg, 3, bias=name != "nobias")
    lat = np.random.default_rng(5).standard_normal((2, 11, cfg.latent_dim)).astype(np.float32)
    got = oracle64.codec_decode(cfg, cw, lat)
    ref = tr.codec_decode(cfg, cw, lat)
    assert got.shape == ref.shape == (2, 1, 11 * cfg.hop_length)
    assert rel_l2(got, ref) < 1e-6
    assert np.abs(got).max() <= 1.0  # tanh head (decoder.rs:74-84)
    assert 0.02 < np.abs(got).mean() < 0.9  # not collapsed, not saturated: the bar can see errors


def test_codec_rows_are_independent_and_f32_tracks_f64(oracle32, oracle64):
    cfg = ih.codec_tiny()
    cw = ih.CodecWeights.random(cfg, 4)
    lat = np.random.default_rng(6).standard_normal((3, 7, cfg.latent_dim)).astype(np.float32)
    both = oracle32.codec_decode(cfg, cw, lat)
    one = oracle32.codec_decode(cfg, cw, lat[1:2])
    assert np.array_equal(both[1:2], one)
    assert rel_l2(both, oracle64.codec_decode(cfg, cw, lat)) < 1e-5
