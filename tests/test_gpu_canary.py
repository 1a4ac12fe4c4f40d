"""Out-of-bounds write checks on the GPU: every entry point that writes a caller's device
buffer is given one bordered by canary values on both sides, at ragged shapes (odd
sequence lengths, partial tiles, padded rows), and the borders must come back untouched.
The interior is checked for finiteness (its values are checked against the oracle by the
parity tests)."""
import dataclasses

import numpy as np
import pytest
import torch

import irodori_hip as ih
from irodori_hip import _lib as L
from irodori_hip import ops

pytestmark = pytest.mark.gpu

BF16, F32, FP8 = ih.InferenceBackendKind.HIP_BF16, ih.InferenceBackendKind.HIP_F32, ih.InferenceBackendKind.HIP_FP8
PAD = 4096  # canary elements on each side (16 KB of f32)


def bordered(n, dtype=torch.float32):
    canary = -12345.678 if dtype.is_floating_point else 0xA5
    buf = torch.full((PAD + n + PAD,), canary, dtype=dtype, device="cuda")
    return buf, buf[PAD:PAD + n], canary


def assert_borders(buf, n, canary):
    torch.cuda.synchronize()
    head, tail = buf[:PAD].cpu(), buf[PAD + n:].cpu()
    assert bool((head == canary).all()), "write before the buffer"
    assert bool((tail == canary).all()), "write past the buffer"


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype).contiguous()


@pytest.mark.parametrize("backend", [F32, BF16, FP8], ids=["f32", "bf16", "fp8"])
def test_sampler_writes_only_its_output(backend):
    # Two utterances of 37 frames (one padded to 37 from 29 under the latent mask), 3 Joint-CFG
    # steps through the device entry point.
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 0, std=0.05)
    ctx = ih.make_context_kv(cfg, 2, 20, 13, seed=1)
    U, S, P = 2, 37, cfg.latent_dim
    x0 = dev(ih.make_noise(U, S, P, 2))
    buf, out, canary = bordered(U * S * P)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=3.0, scale_speaker=3.0)
    with ih.HipInferenceEngine(cfg, backend, max_rows=2 * U, max_seq=S, max_ctx=ctx.t_ctx) as e:
        e.load_weights(w)
        e.set_context_kv(ctx)
        torch.cuda.synchronize()
        e.sample_device(x0.data_ptr(), out.data_ptr(), U, S, ih.SamplerParams(num_steps=3, guidance=g),
                        lengths=[S, 29])
    assert_borders(buf, U * S * P, canary)
    assert bool(torch.isfinite(out).all())


@pytest.mark.parametrize("dtype,Dh", [(L.DTYPE_F32, 64), (L.DTYPE_F32, 128), (L.DTYPE_BF16, 64),
                                      (L.DTYPE_F16, 64)], ids=["f32", "f32_dh128", "bf16", "f16"])
def test_sdpa_writes_only_its_output(dtype, Dh):
    B, H, Sq, Skv = 2, 3, 17, 9
    tdt = {L.DTYPE_F32: torch.float32, L.DTYPE_BF16: torch.bfloat16, L.DTYPE_F16: torch.float16}[dtype]
    rng = np.random.default_rng(0)
    q, k, v = (dev(rng.standard_normal((B, H, n, Dh)), tdt) for n in (Sq, Skv, Skv))
    m = np.ones((B, Skv), np.float32)
    m[1, 5:] = 0.0
    n = B * H * Sq * Dh
    buf, out, canary = bordered(n)
    ops.sdpa(dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), dev(m).data_ptr(), B, H, Sq, Skv, Dh,
             Dh ** -0.5, out.data_ptr())
    assert_borders(buf, n, canary)
    assert bool(torch.isfinite(out).all())


def test_norm_ops_write_only_their_outputs():
    rows, dim = 7, 1000
    x = dev(np.random.default_rng(1).standard_normal((rows, dim)))
    buf, y, canary = bordered(rows * dim)
    ops.rms_norm(x.data_ptr(), dev(np.ones(dim)).data_ptr(), rows, dim, 1e-6, y.data_ptr())
    assert_borders(buf, rows * dim, canary)
    B, S, D = 2, 37, 384
    x = dev(np.random.default_rng(2).standard_normal((B * S, D)))
    sc, sh = (dev(0.1 * np.random.default_rng(s).standard_normal((B, D))) for s in (3, 4))
    buf, y, canary = bordered(B * S * D)
    ops.fused_adaln(x.data_ptr(), sc.data_ptr(), sh.data_ptr(), B, S, D, 1e-6, y.data_ptr())
    assert_borders(buf, B * S * D, canary)


def test_fp8_ops_write_only_their_outputs():
    rows, dim = 37, 256
    x = dev(np.random.default_rng(5).standard_normal((rows, dim)))
    qbuf, q, qc = bordered(rows * dim, torch.uint8)
    sbuf, s, sc = bordered(rows * dim // 32, torch.uint8)
    ops.mx_quantize(x.data_ptr(), rows, dim, q.data_ptr(), s.data_ptr())
    assert_borders(qbuf, rows * dim, qc)
    assert_borders(sbuf, rows * dim // 32, sc)
    M, N, K = 300, 256, 384
    rng = np.random.default_rng(6)
    a = dev(rng.integers(0, 0x7F, (M, K)).astype(np.uint8), torch.uint8)
    a_s = dev(np.full((M, K // 32), 127, np.uint8), torch.uint8)
    w = dev(rng.integers(0, 0x7F, (N, K)).astype(np.uint8), torch.uint8)
    w_s = dev(np.full(N, 2.0 ** -8, np.float32))
    cbuf, c, cc = bordered(M * N)
    ops.gemm_fp8(a.data_ptr(), a_s.data_ptr(), w.data_ptr(), w_s.data_ptr(), M, N, K, c.data_ptr())
    assert_borders(cbuf, M * N, cc)
    assert bool(torch.isfinite(c).all())


def test_codec_decode_writes_only_its_output():
    cfg = ih.codec_tiny()
    w = ih.CodecWeights.random(cfg, 0)
    B, T = 2, 11
    lat = dev(np.random.default_rng(7).standard_normal((B, T, cfg.latent_dim)))
    n = B * T * cfg.hop_length
    buf, wav, canary = bordered(n)
    with ih.HipDacVaeCodec(cfg, BF16, max_frames=16) as codec:
        codec.load_weights(w)
        torch.cuda.synchronize()
        codec.decode_device(lat.data_ptr(), B, T, wav.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert_borders(buf, n, canary)
    assert bool(torch.isfinite(wav).all())
