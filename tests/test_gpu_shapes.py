"""Wrong-shaped host arrays are refused by the wrappers with IrodoriError("Shape") before the
library reads them, on live GPU objects, and the objects keep working afterwards (the
refusals leave nothing half-loaded)."""
import numpy as np
import pytest

import irodori_hip as ih

pytestmark = pytest.mark.gpu

F32 = ih.InferenceBackendKind.HIP_F32


def refused(fn, kind="Shape"):
    with pytest.raises(ih.IrodoriError) as ei:
        fn()
    assert ei.value.kind == kind, str(ei.value)


def test_dit_engine_refuses_wrong_shapes():
    cfg = ih.cfg_tiny()
    P, D = cfg.latent_dim, cfg.model_dim
    w = ih.DitWeights.random(cfg, 0)
    with ih.HipInferenceEngine(cfg, F32, max_rows=2, max_seq=16, max_ctx=8) as e:
        bad = ih.DitWeights(dict(w.io), [dict(b) for b in w.blocks])
        bad.blocks[1]["w2"] = w.blocks[1]["w2"][:-1]
        refused(lambda: e.load_weights(bad))
        bad = ih.DitWeights(dict(w.io), w.blocks[:-1])
        refused(lambda: e.load_weights(bad))
        e.load_weights(w)
        e.set_context_kv(ih.make_context_kv(cfg, 1, 6, 2, seed=1))  # rows: conditioned, unconditioned
        x = ih.make_noise(2, 12, P, 0)
        t = np.array([0.3, 0.7], np.float32)
        refused(lambda: e.forward_with_cond_cached(x, t[:1]))
        refused(lambda: e.forward_with_cond_cached(x[..., :-1], t))
        refused(lambda: e.forward_with_cond_cached(x[0], t))
        xd = np.random.default_rng(2).standard_normal((2, 12, D)).astype(np.float32)
        cond = np.zeros((2, 3 * D), np.float32)
        refused(lambda: e.block_forward(0, xd, cond[:, :-1]))
        refused(lambda: e.block_forward(0, xd[..., :-1], cond))
        p = ih.SamplerParams(num_steps=2)
        refused(lambda: e.sample(x[..., :-1], p, has_speaker=False))
        v = e.forward_with_cond_cached(x, t)
        assert v.shape == x.shape and np.isfinite(v).all()


def test_context_build_refuses_wrong_shapes():
    cfg = ih.cfg_tiny()
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()
    with ih.HipInferenceEngine(cfg, F32, max_rows=2, max_seq=16, max_ctx=40) as e:
        e.load_weights(ih.DitWeights.random(cfg, 0))
        ts = np.ones((5, te.dim), np.float32)
        refused(lambda: e.build_context_kv(0, ts, np.ones(5, np.uint8)), "NotLoaded")
        pw = ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3)
        bad = ih.CtxProjWeights([dict(l) for l in pw.layers], pw.text_dim, pw.aux_dim)
        bad.layers[0]["wv_aux"] = pw.layers[0]["wv_aux"][:, :-1]
        refused(lambda: e.load_ctx_proj_weights(bad))
        e.load_ctx_proj_weights(pw)
        refused(lambda: e.build_context_kv(0, ts[:, :-1], np.ones(5, np.uint8)))
        refused(lambda: e.build_context_kv(0, ts, np.ones(4, np.uint8)))
        aux = np.ones((3, se.dim), np.float32)
        refused(lambda: e.build_context_kv(0, ts, np.ones(5, np.uint8), aux, np.ones(2, np.uint8)))
        refused(lambda: e.build_context_kv(0, ts, np.ones(5, np.uint8), aux[:, :-1], np.ones(3, np.uint8)))
        e.build_context_kv(0, ts, np.ones(5, np.uint8), aux, np.ones(3, np.uint8))
        k, v, m = e.read_context_kv(0, 0, 8)
        assert m[:8].sum() == 8


def test_encoder_and_codec_refuse_wrong_shapes():
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()
    with ih.HipEncoder(te, F32, max_rows=2, max_seq=16) as enc:
        w = ih.EncoderWeights.random(te, 1)
        bad = ih.EncoderWeights(dict(w.io), [dict(b) for b in w.blocks])
        bad.blocks[0]["w13"] = w.blocks[0]["w13"][:, :-1]
        refused(lambda: enc.load_weights(bad))
        enc.load_weights(w)
        mask = np.ones((2, 6), np.uint8)
        ids = np.arange(12, dtype=np.int32).reshape(2, 6)
        refused(lambda: enc.forward(mask, ids=ids[:, :-1]))
        refused(lambda: enc.forward(mask), "InvalidArg")
        state, _ = enc.forward(mask, ids=ids)
        assert state.shape[:2] == (2, 6 + int(te.mean_token))
    with ih.HipEncoder(se, F32, max_rows=2, max_seq=16) as enc:
        enc.load_weights(ih.EncoderWeights.random(se, 2))
        lat = np.ones((2, 6, se.in_dim), np.float32)
        refused(lambda: enc.forward(np.ones((2, 6), np.uint8), latent=lat[..., :-1]))
    cfg = ih.codec_tiny()
    with ih.HipDacVaeCodec(cfg, F32, max_frames=8) as codec:
        w = ih.CodecWeights.random(cfg, 0)
        bad = ih.CodecWeights(dict(w.io), [dict(b) for b in w.blocks])
        bad.io["head_w"] = w.io["head_w"][:, :-1]
        refused(lambda: codec.load_weights(bad))
        codec.load_weights(w)
        lat = np.random.default_rng(0).standard_normal((1, 4, cfg.latent_dim)).astype(np.float32)
        refused(lambda: codec.decode(lat[..., :-1]))
        wav = codec.decode(lat)
        assert wav.shape == (1, 1, 4 * cfg.hop_length) and np.isfinite(wav).all()
