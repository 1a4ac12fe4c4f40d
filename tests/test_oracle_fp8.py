"""CPU pins of the oracle's fp8 (e4m3fn) GEMM operands, the arithmetic of the HIP path's
fp8 compute mode (the batched-throughput workload; the reference has no fp8 path):

* e4m3 encoding / decoding against torch's float8_e4m3fn conversion (a library routine:
  round to nearest, ties to even), over every code and a dense sweep of values;
* the power-of-two block scale against its defining inequalities;
* the quantized GEMM against exact cases (operands already representable) and the
  rounding bound, so a dropped or doubled scale fails.
"""
import numpy as np
import pytest
import torch

import irodori_hip as ih
from conftest import rel_l2
from oracle.oracle import (Oracle, e4m3_decode, e4m3_encode, mx_dequantize_rows,
                           mx_quantize_rows, mx_scale_exp, quant_weight_cols)


def torch_encode(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2  # 0x7F, 0xFF
    assert np.array_equal(got[~nan], ref[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_encode_matches_torch_round_to_nearest_even():
    # Every code's value, the midpoints between neighbouring codes (ties go to the even
    # code), values just either side of each midpoint, and a random sweep, all |x| <= 448.
    vals = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    eps = np.abs(mids) * 2.0 ** -20 + 1e-12
    rng = np.random.default_rng(0)
    sweep = np.concatenate([vals, mids, mids - eps, mids + eps,
                            rng.uniform(0, 448, 4000), 2.0 ** rng.uniform(-12, 8.8, 4000)])
    sweep = np.concatenate([sweep, -sweep]).astype(np.float32)
    sweep = sweep[np.abs(sweep) <= 448]
    assert np.array_equal(e4m3_encode(sweep), torch_encode(sweep))
    assert np.array_equal(e4m3_encode(vals.astype(np.float32)), np.arange(0x7F, dtype=np.uint8))


def test_encode_saturates_past_448():
    assert np.array_equal(e4m3_encode(np.array([449, 463.9, 1e6, -500], np.float32)),
                          np.array([0x7E, 0x7E, 0x7E, 0xFE], np.uint8))


def test_block_scale_is_the_smallest_power_of_two_that_fits():
    for k in range(-20, 20):
        assert mx_scale_exp(448.0 * 2.0 ** k) == k                   # exactly at the bound
        assert mx_scale_exp(np.nextafter(np.float32(448.0 * 2.0 ** k), np.float32(np.inf))) == k + 1
    assert mx_scale_exp(1.0) == -8 and mx_scale_exp(0.0) == 0
    rng = np.random.default_rng(1)
    for a in (2.0 ** rng.uniform(-30, 30, 2000)).astype(np.float32):
        e = mx_scale_exp(float(a))
        assert float(a) <= 448.0 * 2.0 ** e and float(a) > 448.0 * 2.0 ** (e - 1)


def test_row_quantization_round_trip():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((6, 96)) * 2.0 ** rng.uniform(-8, 8, (6, 1))).astype(np.float32)
    x[2, 32:64] = 0.0                      # an all-zero block
    x[3, :32] = 0.0
    x[3, 5] = 2.0 ** -3                    # a lone power of two is exact
    q, sc = mx_quantize_rows(x)
    y = mx_dequantize_rows(q, sc)
    assert q.shape == x.shape and sc.shape == (6, 3)
    assert not np.any((q & 0x7F) == 0x7F)  # never NaN, never saturated past 448
    assert np.all(y[2, 32:64] == 0) and y[3, 5] == 2.0 ** -3 and np.all(np.delete(y[3, :32], 5) == 0)
    for i in range(6):
        for b in range(3):
            blk, yb = x[i, 32 * b:32 * b + 32], y[i, 32 * b:32 * b + 32]
            e = int(sc[i, b]) - 127
            if not blk.any():
                continue
            assert np.abs(blk).max() <= 448.0 * 2.0 ** e
            # round to nearest: normals within 2^-4 relative, subnormals within 2^-10 * 2^e
            tol = np.maximum(np.abs(blk) * 2.0 ** -4, 2.0 ** (e - 10))
            assert np.all(np.abs(yb - blk) <= tol)


def test_weight_quantization_per_channel():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 5)) * np.array([1e-3, 0.02, 1.0, 30.0, 0.0])).astype(np.float32)
    q, sc = quant_weight_cols(w)
    assert sc[4] == 1.0 and not (q[:, 4] & 0x7F).any()  # zeros (signed zeros keep their sign)
    for n in range(4):
        assert sc[n] == np.float32(np.abs(w[:, n]).max() / np.float32(448.0))
        k = np.argmax(np.abs(w[:, n]))
        assert q[k, n] & 0x7F == 0x7E      # the channel's largest weight maps to +-448
        wd = e4m3_decode(q[:, n]) * sc[n]
        assert np.all(np.abs(wd - w[:, n]) <= np.maximum(np.abs(w[:, n]) * 2.0 ** -4, sc[n] * 2.0 ** -10))


def test_gemm_fp8_exact_on_representable_operands(oracle32):
    # Activations that are already e4m3 values times a power of two per 32-block, and
    # weights that are e4m3 codes times a per-column scale whose largest code is 448: the
    # quantization is then the identity and the fp8 GEMM equals the f32 one.
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 0x7E, (8, 64)).astype(np.uint8) | (rng.integers(0, 2, (8, 64)) * 0x80).astype(np.uint8)
    codes[:, 0] = 0x7E
    codes[:, 32] = 0x7E
    x = e4m3_decode(codes) * np.repeat(2.0 ** rng.integers(-6, 6, (8, 2)), 32, axis=1).astype(np.float32)
    wc = rng.integers(0, 0x7E, (64, 24)).astype(np.uint8)
    wc[7] = 0x7E
    ws = (2.0 ** rng.uniform(-8, 0, 24)).astype(np.float32)
    w = (e4m3_decode(wc) * ws).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64)
    got = oracle32.gemm_fp8(x, w)
    assert rel_l2(got, ref) < 1e-6
    # General operands: within the two operands' rounding (2^-4 each) of the f64 product.
    a = rng.standard_normal((16, 128)).astype(np.float32)
    b = (rng.standard_normal((128, 40)) * 0.02).astype(np.float32)
    err = rel_l2(oracle32.gemm_fp8(a, b), a.astype(np.float64) @ b)
    assert 1e-3 < err < 0.1


def test_fp8_forward_is_close_to_f32(oracle32):
    cfg = ih.cfg_tiny()
    w = ih.DitWeights.random(cfg, 0, std=0.05, norm_jitter=0.1)
    ctx = ih.make_context_kv(cfg, 1, 12, 9, seed=1)
    x = ih.make_noise(2, 24, cfg.latent_dim, 2)
    t = np.array([0.9, 0.4], np.float32)
    v32, d32 = oracle32.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    o8 = Oracle("f32", gemm_fp8=True)
    v8, d8 = o8.forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask, debug=True)
    errs = [rel_l2(d8[i], d32[i]) for i in range(1, d8.shape[0])]
    print("fp8 vs f32 per block:", ["%.2e" % e for e in errs], "v %.2e" % rel_l2(v8, v32))
    assert all(1e-4 < e < 0.1 for e in errs)
    assert rel_l2(v8, v32) < 0.2
    # f64 accumulation of the same quantized operands agrees far more closely.
    v64 = Oracle("f64", gemm_fp8=True).forward(cfg, w, x, t, ctx.k, ctx.v, ctx.mask)
    assert rel_l2(v8, v64) < 0.1 * rel_l2(v8, v32)
