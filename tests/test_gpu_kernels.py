"""GPU parity of the operator entry points against the CPU oracle (src/kernels analogues).

Mirrors the reference's kernel tests (rms_norm.rs / fused_adaln.rs / fused_sdpa_native.rs
test modules: their shapes, deterministic sin/cos inputs, masks and the 1e-5 / 1e-4
tolerances for f32) and adds the isolated joint-attention workload (bf16).
Tolerances: f32 within 1e-5 abs (the reference's own), bf16 within 1e-2 relative L2.
"""
import numpy as np
import pytest
import torch

from conftest import rel_l2
from irodori_hip import _lib as L
from irodori_hip import ops
from test_oracle import SDPA_CASES, _ref_inputs

pytestmark = pytest.mark.gpu


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype).contiguous()


def bf16_round(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


@pytest.mark.parametrize("rows,dim", [(4, 256), (7, 1000), (1500, 1024)])
def test_rms_norm_op(oracle32, rows, dim):
    x = (np.sin(np.arange(rows * dim, dtype=np.float32) * 0.1) * 2.0).reshape(rows, dim)
    w = (1.0 + 0.1 * np.cos(np.arange(dim, dtype=np.float32))).astype(np.float32)
    dx, dw = dev(x), dev(w)
    dy = torch.empty_like(dx)
    ops.rms_norm(dx.data_ptr(), dw.data_ptr(), rows, dim, 1e-6, dy.data_ptr())
    torch.cuda.synchronize()
    want = oracle32.rms_norm(x, w, 1e-6)
    assert np.abs(dy.cpu().numpy() - want).max() < 1e-4  # rms_norm.rs test tolerance


@pytest.mark.parametrize("B,S,D", [(1, 4, 256), (2, 5, 96), (2, 750, 1024)])
def test_fused_adaln_op(oracle32, B, S, D):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((B * S, D)).astype(np.float32)
    sc = (0.1 * rng.standard_normal((B, D))).astype(np.float32)
    sh = (0.1 * rng.standard_normal((B, D))).astype(np.float32)
    dx, dsc, dsh = dev(x), dev(sc), dev(sh)
    dy = torch.empty_like(dx)
    ops.fused_adaln(dx.data_ptr(), dsc.data_ptr(), dsh.data_ptr(), B, S, D, 1e-6, dy.data_ptr())
    torch.cuda.synchronize()
    want = oracle32.fused_adaln(x, sc, sh, B, S, 1e-6)
    assert np.abs(dy.cpu().numpy() - want).max() < 1e-4


def _mask_for(case_mask, B, Skv):
    if case_mask is None:
        return np.ones((B, Skv), np.float32)
    if case_mask == "random":
        m = (np.random.default_rng(0).random((B, Skv)) > 0.4).astype(np.float32)
        m[:, 0] = 1
        return m
    return np.tile(np.asarray(case_mask, np.float32), (B, 1))


@pytest.mark.parametrize("B,H,Sq,Skv,Dh,mask", SDPA_CASES)
def test_sdpa_op_f32(oracle64, B, H, Sq, Skv, Dh, mask):
    q, k, v = _ref_inputs(B, H, Sq, Skv, Dh)
    m = _mask_for(mask, B, Skv)
    dq, dk, dv, dm = dev(q), dev(k), dev(v), dev(m)
    out = torch.empty_like(dq)
    ops.sdpa(L.DTYPE_F32, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq,
             Skv, Dh, Dh ** -0.5, out.data_ptr())
    torch.cuda.synchronize()
    want = oracle64.sdpa(q, k, v, m, Dh ** -0.5)
    assert np.abs(out.cpu().numpy() - want).max() < 1e-5  # fused_sdpa_native.rs tolerance


@pytest.mark.parametrize("B,H,Sq,Skv,Dh,mask", SDPA_CASES)
def test_sdpa_op_bf16(oracle64, B, H, Sq, Skv, Dh, mask):
    q, k, v = (bf16_round(a) for a in _ref_inputs(B, H, Sq, Skv, Dh))
    m = _mask_for(mask, B, Skv)
    dq, dk, dv = (dev(a, torch.bfloat16) for a in (q, k, v))
    dm = dev(m)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    ops.sdpa(L.DTYPE_BF16, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq,
             Skv, Dh, Dh ** -0.5, out.data_ptr())
    torch.cuda.synchronize()
    want = oracle64.sdpa(q, k, v, m, Dh ** -0.5)
    assert rel_l2(out.cpu().numpy(), want) < 1e-2


# The reference's f16-input FA tests (fused_sdpa_native_f16.rs:455-585): shapes, masks and
# tolerances (1e-3 max abs; 1e-6 for the all-masked case), with the oracle fed the same
# f16-rounded inputs as the reference's own CPU check (:384-388).  head_dim 128 runs on the
# generic flash kernel, head_dim 64 on the model's joint attention kernel after staging.
F16_CASES = [
    (1, 2, 4, 6, 128, None, 1e-3),
    (1, 2, 4, 8, 128, [1, 1, 1, 1, 1, 0, 0, 0], 1e-3),
    (1, 16, 32, 48, 128, None, 1e-3),
    (1, 1, 17, 9, 128, None, 1e-3),
    (1, 2, 4, 8, 128, [0] * 8, 1e-6),
    (2, 4, 16, 24, 128, None, 1e-3),
    (1, 16, 32, 48, 64, None, 1e-3),
    # head_dim 64 beyond the reference's cases: a partial last key tile, a random mask and
    # more than one query block per head.
    (2, 3, 100, 70, 64, "random", 1e-3),
    (1, 2, 4, 8, 64, [0] * 8, 1e-6),
]


@pytest.mark.parametrize("B,H,Sq,Skv,Dh,mask,tol", F16_CASES)
def test_sdpa_op_f16(oracle64, B, H, Sq, Skv, Dh, mask, tol):
    q, k, v = (a.astype(np.float16) for a in _ref_inputs(B, H, Sq, Skv, Dh))
    m = _mask_for(mask, B, Skv)
    dq, dk, dv = (dev(a, torch.float16) for a in (q, k, v))
    dm = dev(m)
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    ops.sdpa(L.DTYPE_F16, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq,
             Skv, Dh, Dh ** -0.5, out.data_ptr())
    torch.cuda.synchronize()
    want = oracle64.sdpa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), m, Dh ** -0.5)
    assert np.abs(out.cpu().numpy() - want).max() < tol


def test_sdpa_op_f16_bf16_share_the_joint_kernel(oracle64):
    # Dh = 64 16-bit operators run the model's joint attention kernel: a context longer than
    # one key tile per parity and a query count that is not a multiple of the query block.
    B, H, Sq, Skv, Dh = 1, 4, 75, 300, 64
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((B, H, n, Dh)).astype(np.float32) for n in (Sq, Skv, Skv))
    m = np.ones((B, Skv), np.float32)
    m[0, 200:] = 0
    m[0, 37] = 0
    for dtype, tdt, npdt in ((L.DTYPE_F16, torch.float16, np.float16), (L.DTYPE_BF16, torch.bfloat16, None)):
        qq, kk, vv = ((a.astype(npdt).astype(np.float32) if npdt else bf16_round(a)) for a in (q, k, v))
        dq, dk, dv = (dev(a, tdt) for a in (qq, kk, vv))
        out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
        ops.sdpa(dtype, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dev(m).data_ptr(), B, H, Sq, Skv, Dh,
                 Dh ** -0.5, out.data_ptr())
        torch.cuda.synchronize()
        want = oracle64.sdpa(qq, kk, vv, m, Dh ** -0.5)
        # f16: 11-bit operands (the probabilities too); bf16: 8-bit.
        assert rel_l2(out.cpu().numpy(), want) < (2e-3 if npdt else 1e-2)


def test_sdpa_all_masked_rows_are_zero():
    # attention.rs:770-787: a query row with no valid key yields exactly 0.
    B, H, Sq, Skv, Dh = 2, 2, 5, 70, 64
    q, k, v = _ref_inputs(B, H, Sq, Skv, Dh)
    m = np.ones((B, Skv), np.float32)
    m[1] = 0
    dq, dk, dv, dm = dev(q), dev(k), dev(v), dev(m)
    out = torch.full(q.shape, 7.0, device="cuda")
    ops.sdpa(L.DTYPE_F32, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq,
             Skv, Dh, 0.125, out.data_ptr())
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.array_equal(o[1], np.zeros_like(o[1]))
    assert np.abs(o[0]).sum() > 0


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_sdpa_config2_joint_shape(oracle64, dtype):
    # Isolated joint attention: B=2, H=16, Dh=64, 750 queries; keys = 750 latent ++ 256 text ++
    # 375 speaker, text valid length uniform in [32, 256], Q/K/V ~ N(0, 1).  (RoPE is part
    # of the model path and is covered by the model tests.)  The oracle takes the same
    # rounded operands; the kernel also rounds q * scale * log2(e) and P to the operand type.
    B, H, Sq, Dh, Tt, Ts = 2, 16, 750, 64, 256, 375
    Skv = Sq + Tt + Ts
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((B, H, n, Dh)).astype(np.float32) for n in (Sq, Skv, Skv))
    if dtype == "bf16":
        code, tdt, tol = L.DTYPE_BF16, torch.bfloat16, 1e-2
        q, k, v = (bf16_round(a) for a in (q, k, v))
    else:
        code, tdt, tol = L.DTYPE_F16, torch.float16, 2e-3
        q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
    m = np.ones((B, Skv), np.float32)
    for b in range(B):
        valid = int(rng.integers(32, 257))
        m[b, Sq + valid:Sq + Tt] = 0
    dq, dk, dv = (dev(a, tdt) for a in (q, k, v))
    dm = dev(m)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    ops.sdpa(code, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq,
             Skv, Dh, Dh ** -0.5, out.data_ptr())
    torch.cuda.synchronize()
    want = oracle64.sdpa(q, k, v, m, Dh ** -0.5)
    err = rel_l2(out.cpu().numpy(), want)
    print("config 2 %s: rel L2 %.2e, max abs %.2e" % (dtype, err, np.abs(out.cpu().numpy() - want).max()))
    assert err < tol


@pytest.mark.parametrize("Skv", [4097, 4796, 16384])
def test_sdpa_key_tiles_beyond_one_list_word(oracle64, Skv):
    # More than 64 key tiles per row: the joint kernel's tile list spans several words per
    # lane.  Row 0 drops whole tiles from the first word (and, when present, the second)
    # so that the entries of later words shift down; row 1 has a partial mask in every tile.
    B, H, Sq, Dh = 2, 2, 70, 64
    rng = np.random.default_rng(Skv)
    q, k, v = (bf16_round(rng.standard_normal((B, H, n, Dh)).astype(np.float32)) for n in (Sq, Skv, Skv))
    m = np.ones((B, Skv), np.float32)
    m[0, 640:1600] = 0
    m[0, 4160:4300] = 0
    m[0, 9000:9999] = 0
    m[1, ::7] = 0
    dq, dk, dv = (dev(a, torch.bfloat16) for a in (q, k, v))
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    ops.sdpa(L.DTYPE_BF16, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dev(m).data_ptr(), B, H, Sq, Skv, Dh,
             Dh ** -0.5, out.data_ptr())
    torch.cuda.synchronize()
    want = oracle64.sdpa(q, k, v, m, Dh ** -0.5)
    err = rel_l2(out.cpu().numpy(), want)
    print("Skv %d: rel L2 %.2e" % (Skv, err))
    assert err < 1e-2
