"""GPU parity of the condition encoders (irodori_encoder_*: TextEncoder / ReferenceLatentEncoder,
the conditioner norm and the speaker mean token; text_encoder.rs:17-148,
speaker_encoder.rs:85-162, aux_conditioner.rs:60-85, :150-185) against the oracle's
encoder_forward (pinned in test_oracle_encoder.py), through the C ABI on the same seeded
inputs.

Bars: f32 1e-4 relative L2 on the encoded state; bf16 2e-2 (bf16 GEMM and attention
operands over two blocks and the norms).
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL = {F32: 1e-4, BF16: 2e-2}


def inputs(ecfg, valid, S, seed):
    rng = np.random.default_rng(seed)
    mask = np.zeros((len(valid), S), np.uint8)
    for b, n in enumerate(valid):
        mask[b, :n] = 1
    if ecfg.vocab_size:
        return dict(ids=rng.integers(0, ecfg.vocab_size, (len(valid), S)).astype(np.int32)), mask
    return dict(latent=rng.standard_normal((len(valid), S, ecfg.in_dim)).astype(np.float32)), mask


def run(ecfg, ew, backend, mask, **inp):
    B, S = mask.shape
    with ih.HipEncoder(ecfg, backend, max_rows=B, max_seq=S) as enc:
        enc.load_weights(ew)
        return enc.forward(mask, **inp)


CASES = {
    # name: (config, rows' valid lengths, seq)
    "text_dh128": (ih.enc_text_tiny, [20, 13, 0], 20),     # a row with no valid token
    "speaker_dh64": (ih.enc_speaker_tiny, [37, 30], 37),    # mean token, odd length
    "text_one_token": (ih.enc_text_tiny, [1, 0], 1),        # one token, and a row with none
    "speaker_one_frame": (ih.enc_speaker_tiny, [1, 1], 1),  # one reference frame + the mean token
}


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("name", list(CASES))
def test_encoder_vs_oracle(oracle64, name, backend):
    make, valid, S = CASES[name]
    ecfg = make()
    ew = ih.EncoderWeights.random(ecfg, 3, std=0.05, norm_jitter=0.1)
    inp, mask = inputs(ecfg, valid, S, 4)
    got, gm = run(ecfg, ew, backend, mask, **inp)
    ref, rm = oracle64.encoder_forward(ecfg, ew, mask, **inp)
    err = rel_l2(got, ref)
    print(name, backend.value, "rel L2 %.2e" % err)
    assert err < TOL[backend]
    assert np.array_equal(gm, rm)
    off = int(ecfg.mean_token)
    for b, n in enumerate(valid):
        assert not got[b, off + n:].any()  # masked positions: exactly zero


def test_reference_width_two_blocks(oracle32):
    # The reference's text-encoder width (1280, 10 heads of 128, SwiGLU 3328) over two
    # blocks and 256 tokens, bf16.
    ecfg = ih.EncoderConfig(dim=1280, num_layers=2, num_heads=10, mlp_hidden=3328, vocab_size=2000)
    ew = ih.EncoderWeights.random(ecfg, 5)
    inp, mask = inputs(ecfg, [256, 181], 256, 6)
    got, _ = run(ecfg, ew, BF16, mask, **inp)
    ref, _ = oracle32.encoder_forward(ecfg, ew, mask, **inp)
    err = rel_l2(got, ref)
    print("1280-wide rel L2 %.2e" % err)
    assert err < TOL[BF16]


def test_encoded_condition_feeds_the_context_build(oracle64):
    # Text and speaker states from the GPU encoders, through the device context-KV build,
    # equal the oracle's chain (encoders -> build_kv_cache) at the f32 bar.
    cfg = ih.cfg_tiny()
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()
    tw, sw = ih.EncoderWeights.random(te, 1, std=0.05), ih.EncoderWeights.random(se, 2, std=0.05)
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    proj = ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=4, std=0.05)
    tin, tm = inputs(te, [11], 11, 5)
    sin_, sm = inputs(se, [9], 9, 6)
    ts, tmo = run(te, tw, F32, tm, **tin)
    ss, smo = run(se, sw, F32, sm, **sin_)
    ts_ref, _ = oracle64.encoder_forward(te, tw, tm, **tin)
    ss_ref, _ = oracle64.encoder_forward(se, sw, sm, **sin_)
    T = ts.shape[1] + ss.shape[1]
    with ih.HipInferenceEngine(cfg, F32, max_rows=1, max_seq=16, max_ctx=T) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        e.build_context_kv(0, ts[0], tmo[0], ss[0], smo[0])
        k, v, m = [], [], None
        for l in range(cfg.num_layers):
            kl, vl, m = e.read_context_kv(l, 0, T)
            k.append(kl)
            v.append(vl)
    for l in range(cfg.num_layers):
        lw = proj.layers[l]
        ck, cv, cm = oracle64.build_kv_cache(cfg, w.blocks[l]["k_norm"], ts_ref, tmo, lw["wk_text"], lw["wv_text"],
                                             ss_ref, smo, lw["wk_aux"], lw["wv_aux"])
        assert rel_l2(k[l], ck[0]) < 1e-4 and rel_l2(v[l], cv[0]) < 1e-4
        assert np.array_equal(m, cm[0])


def test_encoder_errors_are_reported():
    ecfg = ih.enc_text_tiny()
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipEncoder(ih.EncoderConfig(dim=192, num_layers=1, num_heads=3, mlp_hidden=256, vocab_size=10), F32)
    assert ei.value.kind == "Shape"  # dim not a multiple of 128
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipEncoder(ih.EncoderConfig(dim=256, num_layers=1, num_heads=2, mlp_hidden=256), F32)
    assert ei.value.kind == "Config"  # neither tokens nor latent frames
    with ih.HipEncoder(ecfg, F32, max_rows=1, max_seq=8) as enc:
        inp, mask = inputs(ecfg, [8], 8, 0)
        with pytest.raises(ih.IrodoriError) as ei:
            enc.forward(mask, **inp)
        assert ei.value.kind == "NotLoaded"
        enc.load_weights(ih.EncoderWeights.random(ecfg, 0))
        with pytest.raises(ih.IrodoriError) as ei:
            enc.forward(np.ones((1, 9), np.uint8), ids=np.zeros((1, 9), np.int32))
        assert ei.value.kind == "Shape"
        with pytest.raises(ih.IrodoriError) as ei:
            enc.forward(mask, ids=np.full((1, 8), ecfg.vocab_size, np.int32))
        assert ei.value.kind == "InvalidArg"


def test_two_threads_match_sequential_runs():
    # Two host threads, each with its own encoder (the first launches of every kernel
    # variant, whose one-time LDS limit is guarded by a once flag, race between them), give
    # the bits of the same encoders run one after the other.
    import threading
    jobs = []
    for i, (make, valid, S) in enumerate([(ih.enc_text_tiny, [20, 13], 20), (ih.enc_speaker_tiny, [37, 30], 37)]):
        ecfg = make()
        ew = ih.EncoderWeights.random(ecfg, 10 + i, std=0.05, norm_jitter=0.1)
        inp, mask = inputs(ecfg, valid, S, 20 + i)
        jobs.append((ecfg, ew, mask, inp))
    for backend in (BF16, F32):
        out = [None, None]
        errs = []

        def work(k):
            try:
                ecfg, ew, mask, inp = jobs[k]
                out[k] = run(ecfg, ew, backend, mask, **inp)
            except Exception as exc:  # reported below, on the main thread
                errs.append(exc)

        ths = [threading.Thread(target=work, args=(k,)) for k in range(2)]
        for th in ths:
            th.start()
        for th in ths:
            th.join()
        assert not errs, errs
        for k, (ecfg, ew, mask, inp) in enumerate(jobs):
            seq, seq_mask = run(ecfg, ew, backend, mask, **inp)
            assert np.array_equal(out[k][0], seq) and np.array_equal(out[k][1], seq_mask)
