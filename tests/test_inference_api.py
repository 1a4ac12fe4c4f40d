"""The request-level builder's state machine and argument checks on the CPU (no device
work): the reference's InferenceBuilder typestate (src/inference.rs:83-200) rejects these
calls at compile time; the Python mirror raises IrodoriError("Config" / "Shape")."""
import pytest

import irodori_hip as ih


def model():
    cfg = ih.cfg_cpu_plumbing()
    te, se = ih.enc_text_tiny(), ih.enc_speaker_tiny()
    mc = ih.ModelConfig(dit=cfg, text=te, aux=se)
    mw = ih.ModelWeights(dit=ih.DitWeights.random(cfg, 0), text=ih.EncoderWeights.random(te, 1),
                         ctx_proj=ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3),
                         aux=ih.EncoderWeights.random(se, 2))
    return mc, mw


def test_builder_states():
    mc, mw = model()
    b = ih.InferenceBuilder()
    for call in (lambda: b.with_sampling(ih.SamplerParams()), b.with_default_sampling, b.build, b.model_config):
        with pytest.raises(ih.IrodoriError) as ei:
            call()
        assert ei.value.kind == "Config"
    loaded = b.load_weights(mc, mw)
    assert loaded.model_config() is mc
    with pytest.raises(ih.IrodoriError):
        loaded.build()  # no sampling parameters yet
    with pytest.raises(ih.IrodoriError):
        loaded.load_weights(mc, mw)  # weights are loaded once
    ready = loaded.with_default_sampling()
    assert ready.with_sampling(ih.SamplerParams(num_steps=8))._params.num_steps == 8
    assert ready._params.num_steps == 40  # each transition returns a new builder


def test_load_weights_checks():
    mc, mw = model()
    with pytest.raises(ih.IrodoriError) as ei:
        ih.InferenceBuilder().load_weights(ih.ModelConfig(dit=mc.dit, text=mc.text), mw)
    assert ei.value.kind == "Config"  # aux weights without an aux config
    mc2 = ih.ModelConfig(dit=mc.dit, text=ih.EncoderConfig(dim=128, num_layers=1, num_heads=2, mlp_hidden=256,
                                                           vocab_size=10), aux=mc.aux)
    with pytest.raises(ih.IrodoriError) as ei:
        ih.InferenceBuilder().load_weights(mc2, mw)
    assert ei.value.kind == "Shape"  # projections sized for another text width
