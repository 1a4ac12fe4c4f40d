"""GPU parity of the fp8 compute mode (IRODORI_DTYPE_FP8: the block GEMMs on e4m3 operands,
the batched-throughput workload) against the oracle's fp8 mode (Oracle(gemm_fp8=True), whose quantized
arithmetic test_oracle_fp8.py pins), through the C ABI on the same seeded inputs.

The fp8 pieces are pinned on their own first: the device quantizer bit for bit against the
oracle's, and the fp8 GEMM kernel against the exact product of its (dequantized) operands.
The forward and the sampler then meet the bars below (TOL_BLOCK, TOL_FINAL) and a ratio test.
"""
import dataclasses

import numpy as np
import pytest

import irodori_hip as ih
from conftest import rel_l2
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu

FP8 = ih.InferenceBackendKind.HIP_FP8
# The GPU rounds attention and the GEMM outputs to bf16 where the oracle keeps f32; near an
# e4m3 rounding boundary that bf16 difference flips a code (one e4m3 step, 1/8), so the
# per-block distance grows with depth (about 1e-3 per block at d1024) beyond the bf16 path's.
# Each test therefore also requires the GPU to sit at least twice as close to the fp8 model
# as that model sits to f32, which a wrong scale or layout cannot meet.
TOL_BLOCK, TOL_FINAL = 2e-2, 5e-2


@pytest.fixture(scope="module")
def oracle_fp8():
    return Oracle("f32", gemm_fp8=True)


def check_block_increments(dbg, d8, d32):
    # What the first block adds to the residual stream (its input is the same in_proj
    # output on both sides), GPU against the fp8 model, must be at most half as far as the
    # fp8 model's increment is from the f32 one (the quantization itself, about 6.5 %).
    # Later blocks also see the drift of their inputs; their increments are printed.
    for i in range(1, dbg.shape[0]):
        gpu, fp8, f32 = dbg[i] - dbg[i - 1], d8[i] - d8[i - 1], d32[i] - d32[i - 1]
        e, model = rel_l2(gpu, fp8), rel_l2(fp8, f32)
        print("block %d increment: gpu vs fp8 model %.2e, fp8 model vs f32 %.2e" % (i, e, model))
        if i == 1:
            assert e < 0.5 * model


def make_engine(cfg, w, ctx, rows, seq):
    e = ih.HipInferenceEngine(cfg, FP8, max_rows=rows, max_seq=seq, max_ctx=max(ctx.t_ctx, 1))
    e.load_weights(w)
    e.set_context_kv(ctx)
    return e


@pytest.mark.parametrize("S", [40, 37])
def test_forward_per_block_vs_fp8_oracle(oracle_fp8, oracle32, S):
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 0, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 1, 20, 13, seed=1)
    x = ih.make_noise(2, S, cfg.latent_dim, 2)
    t = np.array([0.9, 0.35], np.float32)
    with make_engine(cfg, w, ctx, 2, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v8, d8 = oracle_fp8.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    v32, d32 = oracle32.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    check_block_increments(dbg, d8, d32)
    errs = [rel_l2(dbg[i], d8[i]) for i in range(dbg.shape[0])]
    print("fp8 GPU vs fp8 oracle per block:", ["%.2e" % a for a in errs],
          "v %.2e; vs f32 oracle v %.2e" % (rel_l2(v, v8), rel_l2(v, v32)))
    assert max(errs) < TOL_BLOCK and rel_l2(v, v8) < TOL_BLOCK
    assert rel_l2(v, v8) < 0.5 * rel_l2(v8, v32)  # the head input after two blocks


def test_forward_cfg4_shape_vs_fp8_oracle(oracle_fp8):
    # The benchmark model (12 x d1024, SwiGLU 2816: K = 2816 takes 22 fp8 slices) on one
    # short utterance pair.
    cfg = ih.cfg_full_rf()
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, 1, 64, 48, seed=1)
    x = ih.make_noise(2, 96, cfg.latent_dim, 2)
    t = np.array([0.999, 0.5], np.float32)
    with make_engine(cfg, w, ctx, 2, 96) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True)
    v8, d8 = oracle_fp8.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    v32, d32 = Oracle("f32").forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(dbg[i], d8[i]) for i in range(dbg.shape[0])]
    print("cfg4-shape fp8 per block:", ["%.2e" % a for a in errs], "v %.2e; fp8 vs f32 oracle v %.2e"
          % (rel_l2(v, v8), rel_l2(v8, v32)))
    assert max(errs) < TOL_BLOCK and rel_l2(v, v8) < TOL_BLOCK
    check_block_increments(dbg, d8, d32)


def test_cfg5_shape_forward_per_block_vs_fp8_oracle(oracle_fp8):
    # Config 5's model and launch widths on two utterances: 2 x Joint CFG = 4 rows of 750
    # frames through all 12 fp8 blocks, latent lengths 750 and 431 (the latent key mask),
    # text lengths 256 and 97 of 256 + 375 speaker keys; per block against the fp8 oracle.
    cfg = ih.cfg_full_rf()
    w = ih.DitWeights.random(cfg, 0)
    U, S = 2, 750
    ctx = ih.make_context_kv(cfg, U, 256, 375, seed=1)
    x = ih.make_noise(2 * U, S, cfg.latent_dim, 2)
    t = np.full(2 * U, 0.6, np.float32)
    lengths = [750, 431]
    lat = np.zeros((2 * U, S), np.uint8)
    for r in range(2 * U):
        lat[r, :lengths[r % U]] = 1
    with make_engine(cfg, w, ctx, 2 * U, S) as e:
        v, dbg = e.forward_with_cond_cached(x, t, debug=True, latent_mask=lat)
    v8, d8 = oracle_fp8.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True, latent_mask=lat)
    v32, d32 = Oracle("f32").forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True, latent_mask=lat)
    valid = lat.astype(bool)
    errs = [rel_l2(dbg[i][valid], d8[i][valid]) for i in range(dbg.shape[0])]
    e8, e32 = rel_l2(v[valid], v8[valid]), rel_l2(v[valid], v32[valid])
    print("cfg5-shape fp8 per block:", ["%.2e" % a for a in errs], "v vs fp8 oracle %.2e, vs f32 oracle %.2e; "
          "fp8 vs f32 oracle %.2e" % (e8, e32, rel_l2(v8[valid], v32[valid])))
    assert max(errs) < TOL_BLOCK and e8 < TOL_BLOCK
    # The per-block drift (bf16 roundings flipping e4m3 codes, ~1e-3 per block) accumulates
    # over the 12 blocks, so the half-distance test is applied to the first block's
    # increment; at the head the GPU must still sit closer to the fp8 model than to f32.
    assert e8 < e32
    check_block_increments(dbg, d8, d32)


def test_sample_joint_vs_fp8_oracle(oracle_fp8):
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 3, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 2, 12, 9, seed=4)
    x0 = ih.make_noise(2, 24, cfg.latent_dim, 5)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=3.0, scale_speaker=3.0,
                          min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=6, guidance=g)
    with make_engine(cfg, w, ctx, 4, 24) as e:
        got = e.sample(x0, p, lengths=[24, 17])
        again = e.sample(x0, p, lengths=[24, 17])
    lat = np.zeros((2, 24), np.uint8)
    lat[0, :24] = 1
    lat[1, :17] = 1
    c, u = ctx.rows([0, 1]), ctx.rows([2, 3])
    ref, _ = oracle_fp8.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 6, 3.0,
                                         0.0, 1.0, latent_mask=lat)
    ref32, _ = Oracle("f32").sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), 6, 3.0,
                                              0.0, 1.0, latent_mask=lat)
    err = max(rel_l2(got[0], ref[0]), rel_l2(got[1, :17], ref[1, :17]))
    model = max(rel_l2(ref[0], ref32[0]), rel_l2(ref[1, :17], ref32[1, :17]))
    print("fp8 sampled latent vs fp8 oracle %.2e (fp8 vs f32 oracle %.2e)" % (err, model))
    assert err < TOL_FINAL and err < 0.5 * model
    assert np.array_equal(got, again)


def test_cfg5_full_size_properties():
    # Batched throughput at full size: 16 utterances x Joint CFG = 32 rows x 750 frames, fp8
    # block GEMMs, latent lengths U[200, 750] padded with the latent key mask, text lengths
    # U[32, 256]; the layer count cut to 2 and the steps to 3 for time.  Properties: every
    # valid frame finite, replays bit-identical, and one padded utterance equal to the same
    # utterance sampled alone, unpadded (rows never interact; the fp8 codes are per row and
    # per 32 values, so they do not depend on the batch).
    import dataclasses
    cfg = dataclasses.replace(ih.cfg_full_rf(), num_layers=2)
    w = ih.DitWeights.random(cfg, 0)
    U, S, Tt, Ts = 16, 750, 256, 375
    lengths = np.random.default_rng(5).integers(200, S + 1, U).astype(np.int32)
    ctx = ih.make_context_kv(cfg, U, Tt, Ts, seed=1)
    x0 = ih.make_noise(U, S, cfg.latent_dim, 2)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=3.0, scale_speaker=3.0,
                          min_t=0.0, max_t=1.0)
    p = ih.SamplerParams(num_steps=3, guidance=g)
    with make_engine(cfg, w, ctx, 2 * U, S) as e:
        got = e.sample(x0, p, lengths=lengths)
        again = e.sample(x0, p, lengths=lengths)
    assert all(np.all(np.isfinite(got[u, :n])) for u, n in enumerate(lengths))
    assert np.array_equal(got, again)
    u = int(np.argmin(lengths))
    n = int(lengths[u])
    alone = ctx.rows([u, U + u])
    with make_engine(cfg, w, alone, 2, n) as e:
        one = e.sample(np.ascontiguousarray(x0[u:u + 1, :n]), p)
    err = rel_l2(got[u:u + 1, :n], one)
    print("cfg5 full size: utterance %d (%d frames) padded vs alone rel L2 %.2e" % (u, n, err))
    assert err < 1e-5


def test_device_quantizer_is_bit_exact():
    # The device's e4m3 codes and block scales equal the oracle's (pinned against torch's
    # float8 conversion) bit for bit: random rows over 2^-20 .. 2^20, exact ties, zero and
    # subnormal-coded blocks.
    import torch
    from oracle.oracle import e4m3_decode, mx_quantize_rows
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((64, 256)) * 2.0 ** rng.uniform(-20, 20, (64, 1))).astype(np.float32)
    codes = e4m3_decode(np.arange(0x7E, dtype=np.uint8))
    x[0, :32] = 448.0 * 2.0 ** -3                                  # the bound itself
    x[1, :32] = (codes[1:33] + codes[0:32]) / 2                    # midpoints: ties to even
    x[2, :32] = 0.0
    x[3, :32] = codes[:32] * 2.0 ** -8                             # small codes incl. subnormals
    x[3, 31] = 448.0 * 2.0 ** -8
    d_x = torch.from_numpy(x).cuda()
    d_q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
    d_s = torch.empty((64, 8), dtype=torch.uint8, device="cuda")
    ih.ops.mx_quantize(d_x.data_ptr(), 64, 256, d_q.data_ptr(), d_s.data_ptr())
    torch.cuda.synchronize()
    q_ref, s_ref = mx_quantize_rows(x)
    assert np.array_equal(d_s.cpu().numpy(), s_ref)
    assert np.array_equal(d_q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("M,N,K", [(300, 256, 384), (8192, 1024, 256), (1500, 1024, 2816)])
def test_gemm_fp8_op_vs_exact_product(M, N, K):
    # The fp8 GEMM kernel on e4m3 codes and scales (64x64 tiles, the 128x128 tiles of large
    # batches, K = 2816 in 22 slices) against the float64 product of the dequantized
    # operands.  The products are exact; the scaled MFMA's own accumulation measures about
    # 5e-5 relative, whatever K (a dropped product or a wrong block scale costs >= 1e-2).
    import torch
    from oracle.oracle import e4m3_decode
    rng = np.random.default_rng(M + K)
    a = rng.integers(0, 0x7F, (M, K)).astype(np.uint8) | (rng.integers(0, 2, (M, K)) * 0x80).astype(np.uint8)
    w = rng.integers(0, 0x7F, (N, K)).astype(np.uint8) | (rng.integers(0, 2, (N, K)) * 0x80).astype(np.uint8)
    a_s = rng.integers(118, 128, (M, K // 32)).astype(np.uint8)
    w_s = (2.0 ** rng.uniform(-12, -4, N)).astype(np.float32)
    lut = e4m3_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    ad = lut[a] * np.repeat(2.0 ** (a_s.astype(np.float64) - 127), 32, axis=1)
    ref = (ad @ lut[w].T) * w_s.astype(np.float64)
    dev = [torch.from_numpy(v).cuda() for v in (a, a_s, w, w_s)]
    c = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ih.ops.gemm_fp8(*[t.data_ptr() for t in dev], M, N, K, c.data_ptr())
    torch.cuda.synchronize()
    assert rel_l2(c.cpu().numpy(), ref) < 2e-4


def test_fp8_needs_model_dim_multiple_of_128():
    # The fp8 GEMM inputs are quantized in 128-value K slices: model_dim 192 is refused (the
    # SwiGLU hidden width is padded to 128 at ingest, so 704 is accepted).
    cfg = dataclasses.replace(ih.cfg_tiny(), model_dim=192, num_heads=3)
    with pytest.raises(ih.IrodoriError) as ei:
        ih.HipInferenceEngine(cfg, FP8, max_rows=2, max_seq=16, max_ctx=8)
    assert ei.value.kind == "Shape"
