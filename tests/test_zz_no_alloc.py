"""irodori_op_sdpa_noalloc (no counterpart in the reference; for callers that cannot
allocate): the same kernels as irodori_op_sdpa, the staging in the library's fixed per-GPU
buffer.  Checked against irodori_op_sdpa through the C ABI on two calls in a row (the
second smaller, so the first call's staging is still in the buffer), bit for bit (same
kernels, same inputs), and against the oracle; shapes beyond the buffer are refused."""
import numpy as np
import pytest
import torch

from irodori_hip import _lib as L
from irodori_hip import ops
from irodori_hip.config import IrodoriError

pytestmark = pytest.mark.gpu

TYPES = [(L.DTYPE_BF16, torch.bfloat16), (L.DTYPE_F16, torch.float16)]


def _inputs(B, H, Sq, Skv, seed):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((B, H, n, 64)).astype(np.float32) for n in (Sq, Skv, Skv))
    m = (rng.random((B, Skv)) > 0.3).astype(np.float32)
    m[:, 0] = 1
    return q, k, v, m


def _run(fn, dtype, tdt, q, k, v, m):
    B, H, Sq, _ = q.shape
    Skv = k.shape[2]
    dq, dk, dv = (torch.from_numpy(a).to("cuda").to(tdt).contiguous() for a in (q, k, v))
    dm = torch.from_numpy(m).to("cuda")
    out = torch.full((B, H, Sq, 64), 7.0, dtype=torch.float32, device="cuda")
    fn(dtype, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq, Skv, 64, 0.125,
       out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy(), [a.float().cpu().numpy() for a in (dq, dk, dv)]


@pytest.mark.parametrize("dtype,tdt", TYPES, ids=["bf16", "f16"])
def test_noalloc_matches_allocating_entry_point(oracle64, dtype, tdt):
    # Config 2's shape (2 rows x 16 heads, 750 queries, 1381 keys), then a smaller call.
    for shape, seed in (((2, 16, 750, 1381), 1), ((1, 3, 37, 100), 2)):
        q, k, v, m = _inputs(*shape, seed)
        got, (qq, kk, vv) = _run(ops.sdpa_noalloc, dtype, tdt, q, k, v, m)
        want, _ = _run(ops.sdpa, dtype, tdt, q, k, v, m)
        assert np.array_equal(got, want), shape
        ref = oracle64.sdpa(qq, kk, vv, m, 0.125)
        err = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
        assert err < (2e-3 if dtype == L.DTYPE_F16 else 1e-2), (shape, err)


def test_noalloc_refuses_shapes_beyond_its_buffer():
    # 4 x 32 heads x 2048 queries: Q alone takes 16 MiB of staging.
    B, H, Sq, Skv = 4, 32, 2048, 64
    q = torch.zeros((B, H, Sq, 64), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((B, H, Skv, 64), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((B, H, Sq, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(IrodoriError) as ei:
        ops.sdpa_noalloc(L.DTYPE_BF16, q.data_ptr(), kv.data_ptr(), kv.data_ptr(), 0, B, H, Sq, Skv, 64, 0.125,
                         out.data_ptr())
    assert ei.value.kind == "Shape" and "noalloc" in str(ei.value)
