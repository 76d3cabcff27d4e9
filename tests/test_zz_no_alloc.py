"""dnnopt_hip_sgemm_noalloc: the fp32 GEMM without device allocation.

It runs the plan and kernels of dnnopt_hip_sgemm with split-k scratch in a
fixed array of the library, so its result must equal dnnopt_hip_sgemm's bit
for bit.  Each case makes two calls in a row on the shared array, the second
with a smaller input, and checks both; a plan that needs more scratch than
the array holds is refused with DNNOPT_ERR_SCRATCH_LIMIT and C untouched.
"""

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _operands(orc, M, N, K, ta, tb, dev, tid0):
    A = u.normal(orc, M * K, tid0, 0, 0.02)
    B = u.normal(orc, K * N, tid0 + 1, 0, 0.02)
    C0 = u.uniform(orc, M * N, tid0 + 2)
    return (torch.from_numpy(A).to(dev), M if ta else K, torch.from_numpy(B).to(dev), K if tb else N,
            torch.from_numpy(C0).to(dev))


def _both(lib, M, N, K, ta, tb, ops, beta):
    """C from dnnopt_hip_sgemm and from the no-allocation entry point."""
    dA, lda, dB, ldb, dC0 = ops
    ref = dC0.clone()
    lib.sgemm(M, N, K, 1.25, dA, lda, dB, ldb, beta, ref, N, transA=ta, transB=tb, stream=_stream())
    got = dC0.clone()
    st = lib.sgemm_noalloc(M, N, K, 1.25, dA, lda, dB, ldb, beta, got, N, transA=ta, transB=tb, stream=_stream())
    assert st == 0, lib.so.dnnopt_hip_status_string(st)
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


# (first call, second smaller call): split-k skinny (C2, C1), the k-major
# split-k kernel (C3 transpose case, 4 MiB of partials), split-k register
# tiles, and plans without scratch (tall kernel, row-dot).
PAIRS = [
    ((7, 11003, 2048, 0, 0), (7, 1009, 2048, 0, 0)),
    ((1, 4096, 4096, 0, 0), (3, 4099, 2048, 0, 0)),
    ((64, 64, 262144, 1, 0), (40, 36, 40000, 1, 0)),
    ((100, 100, 65536, 0, 0), (33, 17, 8192, 0, 1)),
    ((65536, 64, 256, 0, 0), (5, 1000, 300, 0, 1)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_sgemm(lib, orc, dev, first, second):
    for i, (M, N, K, ta, tb) in enumerate((first, second)):
        ops = _operands(orc, M, N, K, ta, tb, dev, 1 + 3 * i)
        for beta in (1.0, 0.0):
            ref, got = _both(lib, M, N, K, ta, tb, ops, beta)
            assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (M, N, K, ta, tb, beta)
        # and against fp64, so that the pair is not merely equally wrong
        A = ops[0].cpu().numpy().reshape((K, M) if ta else (M, K))
        B = ops[2].cpu().numpy().reshape((N, K) if tb else (K, N))
        want, scale = u.exact(A.T if ta else A, B.T if tb else B, 1.25, 1.0, ops[4].cpu().numpy().reshape(M, N))
        ref, got = _both(lib, M, N, K, ta, tb, ops, 1.0)
        u.assert_fp32_close(got.reshape(M, N), want, scale, K, f"noalloc {M}x{N}x{K} ta={ta} tb={tb}")


def test_noalloc_refuses_large_scratch(lib, orc, dev):
    """A split-k plan needing more partial-sum space than the array holds is
    refused before anything is enqueued; a following small call still works."""
    b = u.binding()
    M, N, K = 600, 600, 300000
    dA = torch.zeros(M * K, dtype=torch.float32, device=dev)
    dB = torch.zeros(K * N, dtype=torch.float32, device=dev)
    dC = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    with lib.tunables(TILE_SPLITS=32):  # a plan whose partial sums exceed the array
        assert lib.plan_sgemm(M, N, K)["workspace_bytes"] > b.NOALLOC_SCRATCH_BYTES - 4 * 16384
        st = lib.sgemm_noalloc(M, N, K, 1.0, dA, K, dB, N, 0.0, dC, N, stream=_stream())
    assert st == b.ERR_SCRATCH_LIMIT
    assert "scratch" in lib.so.dnnopt_hip_status_string(st).decode()
    torch.cuda.synchronize()
    assert bool((dC == 7.0).all())
    del dA, dB
    M, N, K = 7, 1009, 2048
    ops = _operands(orc, M, N, K, 0, 0, dev, 1)
    ref, got = _both(lib, M, N, K, 0, 0, ops, 1.0)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


# Split-k skinny (partials summed by a reduce kernel), split-k register tiles
# (tickets, last workgroup sums), the k-major TransA split-k kernel.
CAPTURED = [(7, 1009, 2048, 0, 0), (100, 100, 65536, 0, 0), (64, 64, 65536, 1, 0)]


def test_noalloc_graph_capture(lib, orc, dev):
    """Calls captured into a CUDA graph replay to the eager result bit for bit,
    three times, with eager calls on the same scratch array and NaN-filled
    outputs between the replays; eager calls leave device free memory
    unchanged."""
    ops = [_operands(orc, M, N, K, ta, tb, dev, 1 + 3 * i) for i, (M, N, K, ta, tb) in enumerate(CAPTURED)]
    refs = [torch.empty((M, N), dtype=torch.float32, device=dev) for (M, N, K, ta, tb) in CAPTURED]
    outs = [torch.empty((M, N), dtype=torch.float32, device=dev) for (M, N, K, ta, tb) in CAPTURED]

    def run(dst):
        for (M, N, K, ta, tb), (dA, lda, dB, ldb, _), c in zip(CAPTURED, ops, dst):
            st = lib.sgemm_noalloc(M, N, K, 1.25, dA, lda, dB, ldb, 0.0, c, N, transA=ta, transB=tb,
                                   stream=_stream())
            assert st == 0, lib.so.dnnopt_hip_status_string(st)

    run(refs)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(dev)[0]
    for _ in range(3):
        run(refs)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0, "an eager noalloc call changed device free memory"
    # each eager result against fp64 as well
    for (M, N, K, ta, tb), (dA, _, dB, _, _), r in zip(CAPTURED, ops, refs):
        A = dA.cpu().numpy().reshape((K, M) if ta else (M, K))
        B = dB.cpu().numpy().reshape((N, K) if tb else (K, N))
        want, scale = u.exact(A.T if ta else A, B.T if tb else B, 1.25)
        u.assert_fp32_close(r.cpu().numpy(), want, scale, K, f"noalloc {M}x{N}x{K} ta={ta}")

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(outs)
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        run([torch.empty_like(r) for r in refs])  # eager work on the shared array between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (M, N, K, ta, tb), o, r in zip(CAPTURED, outs, refs):
            assert torch.equal(o.view(torch.int32), r.view(torch.int32)), (rep, M, N, K, ta, tb)


_FIRST_CALL_CAPTURED = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
import _util as u
lib = u.load_lib()
dev = torch.device("cuda:0")
g0 = torch.Generator(device=dev)
g0.manual_seed(5)
M, N, K = 7, 1009, 2048
A = torch.randn(M, K, device=dev, generator=g0) * 0.02
B = torch.randn(K, N, device=dev, generator=g0) * 0.02
C = torch.empty(M, N, device=dev)
ref = torch.empty(M, N, device=dev)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    st = lib.sgemm_noalloc(M, N, K, 1.0, A, K, B, N, 0.0, C, N, stream=torch.cuda.current_stream().cuda_stream)
assert st == 0, lib.so.dnnopt_hip_status_string(st)
lib.sgemm(M, N, K, 1.0, A, K, B, N, 0.0, ref, N, stream=torch.cuda.current_stream().cuda_stream)
for i in range(3):
    C.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(C.view(torch.int32), ref.view(torch.int32)), i
print("first call captured: ok", flush=True)
"""


def test_noalloc_first_call_under_capture(dev):
    """A process whose first noalloc call is made under graph capture (so the
    scratch address lookup and the ticket clearing are recorded too) replays
    to dnnopt_hip_sgemm's result."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, here], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "first call captured: ok" in r.stdout
