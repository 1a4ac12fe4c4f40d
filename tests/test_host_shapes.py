"""Host-side shape checks of the ctypes wrappers (irodori_hip/engine.py).

The library reads every host array through a bare pointer, so the wrappers refuse any array
whose shape differs from the one the library will read, before the call.  These tests pin
the wrappers' shape tables against the synthetic weight generators (the Burn layouts of
config/model.rs, text_encoder.rs, codec/weights.rs) at the small shipped configs, and at the
published width against the per-block weight volume the sampler streams (27.8 MB of bf16
per DiT block), and check the refusal itself.  No GPU is needed.
"""
import dataclasses

import numpy as np
import pytest

import irodori_hip as ih
from irodori_hip import engine as E


def dit_cfgs():
    tiny = ih.cfg_tiny()
    return {
        "tiny": tiny,
        "cpu_plumbing": ih.cfg_cpu_plumbing(),
        "tiny_dh128": dataclasses.replace(tiny, model_dim=256, num_heads=2),
        "tiny_p120": dataclasses.replace(tiny, latent_dim=120),
    }


@pytest.mark.parametrize("name", list(dit_cfgs()))
def test_dit_weight_shapes_match_the_synthetic_weights(name):
    cfg = dit_cfgs()[name]
    w = ih.DitWeights.random(cfg, 0)
    io, block = E.dit_weight_shapes(cfg)
    assert set(io) == set(w.io)
    for k, shp in io.items():
        assert w.io[k].shape == shp, k
    assert len(w.blocks) == cfg.num_layers
    for b in w.blocks:
        assert set(block) == set(b)
        for k, shp in block.items():
            if k.startswith("ada_"):
                assert len(b[k]) == 2 and all(len(row) == 3 for row in b[k])
                assert all(a.shape == shp for row in b[k] for a in row), k
            else:
                assert b[k].shape == shp, k


def test_dit_block_weights_at_the_published_width_are_27_8_mb_of_bf16():
    # The per-step weight stream of one block at BASELINE config 4 (d 1024, 16 x 64 heads,
    # SwiGLU 2816): QKV 1024 x 3072, gate and W_o 1024 x 1024, W13 1024 x 5632, W2
    # 2816 x 1024 and the two head norms; the adaLN projections are folded into the
    # modulation table at the start of a run and are not part of it.
    _, block = E.dit_weight_shapes(ih.cfg_full_rf())
    n = sum(int(np.prod(s)) for k, s in block.items() if not k.startswith("ada_"))
    assert n == 3 * 1024 * 1024 + 2 * 1024 * 1024 + 2 * 16 * 64 + 1024 * 5632 + 2816 * 1024
    assert abs(2 * n / 1e6 - 27.8) < 0.05


@pytest.mark.parametrize("name", ["text_tiny", "speaker_tiny", "caption"])
def test_encoder_weight_shapes_match_the_synthetic_weights(name):
    te = ih.enc_text_tiny()
    cfg = {"text_tiny": te, "speaker_tiny": ih.enc_speaker_tiny(),
           "caption": ih.EncoderConfig(dim=te.dim, num_layers=1, num_heads=te.num_heads,
                                       mlp_hidden=te.mlp_hidden, vocab_size=500)}[name]
    w = ih.EncoderWeights.random(cfg, 0)
    io, block = E.encoder_weight_shapes(cfg)
    assert set(io) == set(w.io)
    for k, shp in io.items():
        assert w.io[k].shape == shp, k
    for b in w.blocks:
        assert set(block) == set(b)
        for k, shp in block.items():
            assert b[k].shape == shp, k


@pytest.mark.parametrize("cfg", [ih.codec_tiny(), ih.CodecConfig(latent_dim=4, proj_dim=32, decoder_dim=64,
                                                                 rates=(2, 4))], ids=["tiny", "even"])
def test_codec_weight_shapes_match_the_synthetic_weights(cfg):
    w = ih.CodecWeights.random(cfg, 0)
    io, blocks = E.codec_weight_shapes(cfg)
    assert set(io) == set(w.io)
    for k, shp in io.items():
        assert w.io[k].shape == shp, k
    assert len(blocks) == len(w.blocks) == cfg.num_blocks
    for bs, b in zip(blocks, w.blocks):
        assert set(bs) == set(b)
        for k, shp in bs.items():
            arrs = b[k] if isinstance(b[k], list) else [b[k]]
            assert all(a.shape == shp for a in arrs), k


def test_shaped_refuses_other_shapes_and_missing_arrays():
    a = np.arange(6, dtype=np.float64).reshape(2, 3)
    got = E._shaped(a, (2, 3), "a")
    assert got.dtype == np.float32 and got.flags.c_contiguous and np.array_equal(got, a)
    with pytest.raises(ih.IrodoriError) as ei:
        E._shaped(a, (3, 2), "a")
    assert ei.value.kind == "Shape" and "(3, 2)" in str(ei.value)
    with pytest.raises(ih.IrodoriError) as ei:
        E._shaped(a.reshape(6), (2, 3), "a")
    assert ei.value.kind == "Shape"
    with pytest.raises(ih.IrodoriError) as ei:
        E._shaped(None, (2, 3), "a")
    assert ei.value.kind == "InvalidArg"
    ids = E._shaped([[1, 2]], (1, 2), "ids", np.int32)
    assert ids.dtype == np.int32
