"""CPU pins of the oracle's condition encoders (text / caption TextEncoder, speaker
ReferenceLatentEncoder with its mean token, text_encoder.rs:17-148, speaker_encoder.rs:85-162,
aux_conditioner.rs:150-185) against a torch.nn.functional restatement in float64
(tests/torch_reference.py) that shares none of the oracle's loops."""
import numpy as np
import pytest

import irodori_hip as ih
import torch_reference as tref
from conftest import rel_l2


def inputs(ecfg, B, S, seed, valid):
    rng = np.random.default_rng(seed)
    mask = np.zeros((B, S), np.uint8)
    for b, n in enumerate(valid):
        mask[b, :n] = 1
    if ecfg.vocab_size:
        return dict(ids=rng.integers(0, ecfg.vocab_size, (B, S)).astype(np.int32)), mask
    return dict(latent=rng.standard_normal((B, S, ecfg.in_dim)).astype(np.float32)), mask


@pytest.mark.parametrize("kind", ["text", "speaker"])
def test_encoder_matches_torch(oracle64, kind):
    ecfg = ih.enc_text_tiny() if kind == "text" else ih.enc_speaker_tiny()
    ew = ih.EncoderWeights.random(ecfg, 3, std=0.05, norm_jitter=0.1)
    # ragged rows, and a row with no valid frame (the unconditioned bundle's shape)
    inp, mask = inputs(ecfg, 3, 20, 4, [20, 13, 0])
    got, gm = oracle64.encoder_forward(ecfg, ew, mask, **inp)
    ref, rm = tref.encoder_forward(ecfg, ew, mask, **inp)
    assert got.shape == ref.shape
    assert rel_l2(got, ref) < 1e-6  # the oracle stores intermediates as float32
    assert np.array_equal(gm, rm)
    off = 1 if ecfg.mean_token else 0
    assert not got[2].any()                          # nothing valid: exactly zero
    assert not got[1, off + 13:].any()               # masked frames: exactly zero
    if ecfg.mean_token:
        assert np.allclose(got[1, 0], got[1, 1:14].mean(0), atol=1e-6)
        assert gm[2, 0] == 0 and gm[0, 0] == 1


def test_encoder_rows_are_independent(oracle64):
    ecfg = ih.enc_text_tiny()
    ew = ih.EncoderWeights.random(ecfg, 5, std=0.05)
    inp, mask = inputs(ecfg, 2, 16, 6, [16, 9])
    both, _ = oracle64.encoder_forward(ecfg, ew, mask, **inp)
    one, _ = oracle64.encoder_forward(ecfg, ew, mask[1:], ids=inp["ids"][1:])
    assert np.allclose(both[1], one[0], atol=1e-6)
    # masked-out tokens do not matter: change their ids
    ids2 = inp["ids"].copy()
    ids2[1, 9:] = (ids2[1, 9:] + 7) % ecfg.vocab_size
    again, _ = oracle64.encoder_forward(ecfg, ew, mask, ids=ids2)
    assert np.array_equal(again, both)
