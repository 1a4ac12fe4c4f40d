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


def _boundary_shape(sq):
    # One head of 64 keys: the staging is Q (sq x 128 bytes, rounded up to 256) + V^T
    # (8192 bytes) + the key bits (one word, rounded up to 256).  sq = 131006 fills the
    # 16 MiB buffer exactly; 131007 is one 256-byte step past it.
    return 1, 1, sq, 64


def test_noalloc_accepts_the_largest_shape_that_fits():
    B, H, Sq, Skv = _boundary_shape(131006)
    assert Sq * 128 + 8192 + 256 == L.SDPA_SCRATCH_BYTES
    q, k, v, m = _inputs(B, H, Sq, Skv, 4)
    got, _ = _run(ops.sdpa_noalloc, L.DTYPE_BF16, torch.bfloat16, q, k, v, m)
    want, _ = _run(ops.sdpa, L.DTYPE_BF16, torch.bfloat16, q, k, v, m)
    assert np.array_equal(got, want)


def test_noalloc_refuses_shapes_beyond_its_buffer():
    B, H, Sq, Skv = _boundary_shape(131007)
    q = torch.zeros((B, H, Sq, 64), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((B, H, Skv, 64), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((B, H, Sq, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(IrodoriError) as ei:
        ops.sdpa_noalloc(L.DTYPE_BF16, q.data_ptr(), kv.data_ptr(), kv.data_ptr(), 0, B, H, Sq, Skv, 64, 0.125,
                         out.data_ptr())
    assert ei.value.kind == "Shape" and "noalloc" in str(ei.value)


def test_noalloc_under_graph_capture_replays_the_eager_result():
    # One eager call (it resolves the buffer's address), then the same call captured in a
    # graph on torch's capture stream and replayed several times, with eager work on the
    # same buffers between the replays; every replay rewrites the output bit for bit.
    B, H, Sq, Skv = 2, 4, 200, 300
    q, k, v, m = _inputs(B, H, Sq, Skv, 5)
    dq, dk, dv = (torch.from_numpy(a).to("cuda").to(torch.bfloat16).contiguous() for a in (q, k, v))
    dm = torch.from_numpy(m).to("cuda")
    out = torch.full((B, H, Sq, 64), 7.0, dtype=torch.float32, device="cuda")

    def call(stream):
        ops.sdpa_noalloc(L.DTYPE_BF16, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dm.data_ptr(), B, H, Sq, Skv,
                         64, 0.125, out.data_ptr(), stream)

    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = out.cpu().numpy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    other_q, other_k, other_v, other_m = _inputs(1, 2, 50, 70, 6)
    for rep in range(4):
        out.fill_(7.0)
        # An eager call of another shape in between leaves other contents in the buffer.
        _run(ops.sdpa_noalloc, L.DTYPE_BF16, torch.bfloat16, other_q, other_k, other_v, other_m)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), rep

