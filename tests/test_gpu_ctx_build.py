"""GPU parity of the device context-KV build (build_kv_cache, attention.rs:431-501) against
the oracle's build_kv_cache (pinned in test_oracle.py against a float64 restatement), read
back through irodori_read_ctx_kv, and of the forward that attends to it.

Bars: the f32 path 1e-5 relative L2 on K and V (one f32 GEMM and a head RMSNorm), bf16 1e-2
(states and weights rounded to bf16, K and V stored in bf16); forwards as in
test_gpu_model.py (1e-4 f32, 1e-2 bf16 per block).
"""
import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16, F32 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32
TOL_KV = {BF16: 1e-2, F32: 1e-5}
TOL_BLOCK = {BF16: 1e-2, F32: 1e-4}


def states(rng, t, dim, valid):
    s = rng.standard_normal((t, dim)).astype(np.float32)
    m = np.zeros(t, np.uint8)
    m[:valid] = 1
    return s, m


def oracle_ctx(oracle, cfg, w, proj, rows):
    """rows: per batch row (text, text_mask, aux, aux_mask) -> ContextKV [L, B, T, H, Dh]."""
    ks, vs, mask = [], [], None
    for l in range(cfg.num_layers):
        lw = proj.layers[l]
        kl, vl, ml = [], [], []
        for text, tm, aux, am in rows:
            ck, cv, cm = oracle.build_kv_cache(
                cfg, w.blocks[l]["k_norm"], text[None], tm[None], lw["wk_text"], lw["wv_text"],
                None if aux is None else aux[None], None if am is None else am[None],
                lw.get("wk_aux"), lw.get("wv_aux"))
            kl.append(ck[0]); vl.append(cv[0]); ml.append(cm[0])
        ks.append(np.stack(kl)); vs.append(np.stack(vl)); mask = np.stack(ml)
    return ih.ContextKV(np.stack(ks), np.stack(vs), mask)


def build_rows(e, rows):
    for r, (text, tm, aux, am) in enumerate(rows):
        e.build_context_kv(r, text, tm, aux, am)


def check_readback(e, cfg, ref, backend):
    for l in range(cfg.num_layers):
        for r in range(ref.k.shape[1]):
            k, v, m = e.read_context_kv(l, r, ref.t_ctx)
            assert np.array_equal(m, ref.mask[r])
            assert rel_l2(k, ref.k[l, r]) < TOL_KV[backend], (l, r)
            assert rel_l2(v, ref.v[l, r]) < TOL_KV[backend], (l, r)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_ragged_dims_and_unconditioned_row(oracle64, backend):
    # Input dims 40 and 72 are padded to 64 and 128 on the device; row 1 is the
    # unconditioned bundle (zero states, every key masked out: condition.rs:144-154).
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    proj = ih.CtxProjWeights.random(cfg, 40, 72, seed=4, std=0.1)
    rng = np.random.default_rng(5)
    text, tm = states(rng, 10, 40, 7)
    aux, am = states(rng, 9, 72, 9)
    rows = [(text, tm, aux, am),
            (np.zeros_like(text), np.zeros_like(tm), np.zeros_like(aux), np.zeros_like(am))]
    ref = oracle_ctx(oracle64, cfg, w, proj, rows)
    S = 40
    x = ih.make_noise(2, S, cfg.latent_dim, 6)
    t = np.array([0.8, 0.8], np.float32)
    with ih.HipInferenceEngine(cfg, backend, max_rows=2, max_seq=S, max_ctx=19) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        build_rows(e, rows)
        check_readback(e, cfg, ref, backend)
        k1, v1, _ = e.read_context_kv(1, 1, 19)
        assert not k1.any() and not v1.any()
        v_dev, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v_ref, dbg_ref = oracle64.forward(cfg, w, x, t, ref.k, ref.v, ref.mask, debug=True)
    errs = [rel_l2(dbg[i], dbg_ref[i]) for i in range(dbg.shape[0])]
    print(backend.value, "per-block rel L2:", ["%.2e" % a for a in errs])
    assert max(errs) < TOL_BLOCK[backend]
    assert rel_l2(v_dev, v_ref) < TOL_BLOCK[backend]


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_reference_lengths_and_dims(oracle32, backend):
    # The reference's default condition widths (text_dim = speaker_dim = 1280,
    # src/config/model.rs:61-72) at the benchmark's 256 text + 375 speaker keys: several
    # row tiles per segment, the last one partial, and the speaker keys at offset 256.
    cfg = ih.cfg_cpu_plumbing()
    w = ih.DitWeights.random(cfg, 7, norm_jitter=0.05)
    proj = ih.CtxProjWeights.random(cfg, 1280, 1280, seed=8, std=0.03)
    rng = np.random.default_rng(9)
    text, tm = states(rng, 256, 1280, 201)
    aux, am = states(rng, 375, 1280, 375)
    rows = [(text, tm, aux, am)]
    ref = oracle_ctx(oracle32, cfg, w, proj, rows)
    with ih.HipInferenceEngine(cfg, backend, max_rows=1, max_seq=64, max_ctx=631) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        build_rows(e, rows)
        check_readback(e, cfg, ref, backend)


@pytest.mark.parametrize("backend", [F32, BF16], ids=["f32", "bf16"])
def test_text_only_rebuild_and_matches_host_upload(oracle64, backend):
    # No aux projection (aux_dim 0); a second build of the same row replaces the first
    # entirely; a forward over the device-built context equals one over the same K / V
    # uploaded from the host.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 11, std=0.05, norm_jitter=0.1)
    proj = ih.CtxProjWeights.random(cfg, 64, 0, seed=12, std=0.1)
    rng = np.random.default_rng(13)
    first, m1 = states(rng, 70, 64, 70)
    second, m2 = states(rng, 70, 64, 33)
    ref = oracle_ctx(oracle64, cfg, w, proj, [(second, m2, None, None)])
    x = ih.make_noise(1, 24, cfg.latent_dim, 14)
    t = np.array([0.6], np.float32)
    with ih.HipInferenceEngine(cfg, backend, max_rows=1, max_seq=24, max_ctx=70) as e:
        e.load_weights(w)
        e.load_ctx_proj_weights(proj)
        e.build_context_kv(0, first, m1)
        e.build_context_kv(0, second, m2)
        check_readback(e, cfg, ref, backend)
        v_built = e.forward_with_cond_cached(x, t)
        kk = np.stack([e.read_context_kv(l, 0, 70)[0] for l in range(cfg.num_layers)])[:, None]
        vv = np.stack([e.read_context_kv(l, 0, 70)[1] for l in range(cfg.num_layers)])[:, None]
        e.set_context_kv(ih.ContextKV(kk, vv, m2[None]))
        v_host = e.forward_with_cond_cached(x, t)
    # The read-back values are exactly the stored ones, so both forwards see the same K / V.
    assert np.array_equal(v_built, v_host)


def test_build_errors_are_reported():
    cfg = ih.cfg_tiny()
    rng = np.random.default_rng(0)
    text, tm = states(rng, 8, 40, 8)
    aux, am = states(rng, 4, 72, 4)
    with ih.HipInferenceEngine(cfg, F32, max_rows=2, max_seq=16, max_ctx=12) as e:
        with pytest.raises(ih.IrodoriError) as ei:
            e.build_context_kv(0, text, tm)
        assert ei.value.kind == "NotLoaded"
        e.load_ctx_proj_weights(ih.CtxProjWeights.random(cfg, 40, 0, seed=1))
        with pytest.raises(ih.IrodoriError) as ei:  # no aux projection loaded
            e.build_context_kv(0, text, tm, aux, am)
        assert ei.value.kind == "NotLoaded"
        with pytest.raises(ih.IrodoriError) as ei:  # input dim differs from the loaded one
            e.load_ctx_proj_weights(ih.CtxProjWeights.random(cfg, 48, 0, seed=1))
        assert ei.value.kind == "Shape"
        with pytest.raises(ih.IrodoriError) as ei:  # 13 keys > max_ctx 12
            e.build_context_kv(0, np.zeros((13, 40), np.float32), np.ones(13, np.uint8))
        assert ei.value.kind == "Shape"
        with pytest.raises(ih.IrodoriError) as ei:  # block weights (k_norm) not loaded
            e.build_context_kv(0, text, tm)
        assert ei.value.kind == "NotLoaded"
        e.load_weights(ih.DitWeights.random(cfg, 0))
        e.build_context_kv(0, text, tm)
        with pytest.raises(ih.IrodoriError) as ei:  # t_ctx differs from the one already set
            e.build_context_kv(1, text[:5], tm[:5])
        assert ei.value.kind == "Shape"
