"""Concurrent synchronous calls from several host threads of one process.

The reference's small-M calls are reentrant and share no buffers
(src/gemm/gemm_tiny_fp32.cpp:167-218, src/gemm/gemm_smallm_wide_fp32.cpp:
412-490); callers on several threads get independent, correct results.  Here
each host thread enqueues on its own stream with its own workspace and
staging buffers.  The shapes below all split k across workgroups (a kernel
writes partial sums that a second launch reduces), which is where a shared
workspace would mix two calls' partials.  ctypes releases the GIL for the
duration of each call, so the threads' calls overlap inside the library.
"""

import threading

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CBLAS_ROW, CBLAS_N, CBLAS_T = 101, 111, 112
THREADS = 4
ROUNDS = 3


def _shapes(orc):
    """(name, call(C) -> None, C shape, fp64 want, tolerance scale, K)."""
    out = []
    # C1: 1 x 4096 x 4096, beta 0, through dnnopt::gemm_fp32 on host memory.
    M, N, K = 1, 4096, 4096
    A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N))
    out.append(("C1 gemm_fp32", lambda lib, C, A=A, B=B, M=M, N=N, K=K: lib.cxx["gemm_fp32"](
        M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, C.ctypes.data, N), (M, N), None, want, scale, K))
    # C2 M=7 N=1009: beta 1, through cblas_sgemm row-major.
    M, N, K = 7, 1009, 2048
    A, B = u.normal(orc, M * K, 1, 0, 0.02), u.normal(orc, K * N, 2, 0, 0.02)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), 1.0, 1.0, C0)
    out.append(("C2 cblas_sgemm", lambda lib, C, A=A, B=B, M=M, N=N, K=K: lib.so.cblas_sgemm(
        CBLAS_ROW, CBLAS_N, CBLAS_N, M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 1.0, C.ctypes.data, N),
        (M, N), C0, want, scale, K))
    # C3 transpose case: 64 x 64 x 262144 with A stored K x M.
    M, N, K = 64, 64, 262144
    At, B = u.uniform(orc, K * M, 1), u.uniform(orc, K * N, 2)
    want, scale = u.exact(At.reshape(K, M).T, B.reshape(K, N))
    out.append(("C3 TransA cblas_sgemm", lambda lib, C, At=At, B=B, M=M, N=N, K=K: lib.so.cblas_sgemm(
        CBLAS_ROW, CBLAS_T, CBLAS_N, M, N, K, 1.0, At.ctypes.data, M, B.ctypes.data, N, 0.0, C.ctypes.data, N),
        (M, N), None, want, scale, K))
    return out


def test_threads_host_pointer_calls(lib, orc, dev):
    shapes = _shapes(orc)
    errors = []
    stop = threading.Event()

    def worker(t):
        order = shapes[t % len(shapes):] + shapes[:t % len(shapes)]
        for r in range(ROUNDS):
            for name, call, shape, C0, want, scale, K in order:
                if stop.is_set():
                    return
                C = (np.full(shape, np.nan, np.float32) if C0 is None else C0.copy())
                call(lib, C)
                st = lib.so.dnnopt_hip_last_status()
                try:
                    assert st == 0, f"status {st}"
                    u.assert_fp32_close(C, want, scale, K, f"thread {t} round {r} {name}")
                except AssertionError as e:
                    errors.append(str(e))
                    stop.set()
                    return

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors[0]


def test_threads_device_pointer_calls(lib, orc, dev):
    """Device operands used in place by concurrent dnnopt::gemm_fp32 calls
    (split-k skinny launches at C2 N = 1009 and N = 4099)."""
    cases = []
    for N in (1009, 4099):
        M, K = 7, 2048
        A, B = u.normal(orc, M * K, 1, 0, 0.02), u.normal(orc, K * N, 2, 0, 0.02)
        C0 = u.uniform(orc, M * N, 3).reshape(M, N)
        want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), 1.0, 1.0, C0)
        cases.append((M, N, K, torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), C0, want, scale))
    outs = [[torch.empty((c[0], c[1]), dtype=torch.float32, device=dev) for c in cases] for _ in range(THREADS)]
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        for r in range(ROUNDS * 2):
            for i, (M, N, K, dA, dB, C0, want, scale) in enumerate(cases):
                dC = outs[t][i]
                dC.copy_(torch.from_numpy(C0))  # synchronous host-to-device copy
                torch.cuda.synchronize()
                lib.cxx["gemm_fp32"](M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 1.0, dC.data_ptr(), N)
                got = dC.cpu().numpy()
                try:
                    assert lib.so.dnnopt_hip_last_status() == 0
                    u.assert_fp32_close(got, want, scale, K, f"thread {t} round {r} 7x{N}x{K} device pointers")
                except AssertionError as e:
                    errors.append(str(e))
                    return

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors[0]
