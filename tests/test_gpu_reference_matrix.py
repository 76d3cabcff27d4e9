"""The reference's own test matrices, run on the GPU through the drop-in APIs.

* tests/test_gemm_correctness.cpp:160-183: every shape through the C++ API
  (dnnopt::gemm_fp32, gemm_bf16, gemm_int8) on host arrays, beta = 0, with
  the reference's tolerances (fp32 K*2e-5 :94, bf16 K*2e-3 :128, int8
  K*2e-2 :145) and this build's own bars (fp32 (2K+4)u against fp64, bf16
  1e-2 of |A||B|, int8 bit-exact against the oracle's restatement of the
  reference's gemm_int8 routing).  Its alpha/beta cases (:188-224, tolerance
  K*4e-5) follow.
* tests/integration/test_dispatch_logic.cpp:143-153: the nine oneDNN shapes
  through the hook's argument list (dnnopt_onednn_sgemm, column-major, host
  arrays), tolerance K*2e-5 (:222) and (2K+4)u.

The reference draws std::mt19937 / rand() values, which are not portable
across standard libraries; the inputs here come from the build's SplitMix64
generator with the reference's ranges (U[-1, 1) for the correctness matrix,
U[0, 1) for the dispatch shapes).
"""

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CORRECTNESS_SHAPES = [
    (1, 1, 1), (4, 4, 4), (8, 8, 8), (16, 16, 16), (32, 32, 32), (64, 64, 64), (128, 128, 128), (256, 256, 256),
    (1, 128, 64), (7, 13, 5), (3, 3, 1000), (128, 1, 768), (1, 1000, 2048),
    (128, 768, 768), (128, 3072, 768),
    (5, 7, 11), (13, 17, 19), (127, 127, 127),
]


@pytest.mark.parametrize("M,N,K", CORRECTNESS_SHAPES)
def test_gemm_correctness_matrix(lib, orc, dev, M, N, K):
    A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N))
    # fp32
    C = np.zeros(M * N, np.float32)
    lib.cxx["gemm_fp32"](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, C.ctypes.data, N)
    assert lib.last_status() == 0
    C = C.reshape(M, N)
    assert np.abs(C - want).max() < K * 2e-5, "reference tolerance (test_gemm_correctness.cpp:94)"
    u.assert_fp32_close(C, want, scale, K, f"gemm_fp32 {M}x{N}x{K}")
    # bf16 (fp32 operands rounded to bf16 inside)
    Cb = np.zeros(M * N, np.float32)
    lib.cxx["gemm_bf16"](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, Cb.ctypes.data, N)
    assert lib.last_status() == 0
    Cb = Cb.reshape(M, N)
    assert np.abs(Cb - want).max() < K * 2e-3, "reference tolerance (test_gemm_correctness.cpp:128)"
    assert (np.abs(Cb - want) <= 1e-2 * scale + 1e-30).all(), f"gemm_bf16 {M}x{N}x{K}"
    # int8 through the fp32 API
    Ci = np.zeros(M * N, np.float32)
    lib.cxx["gemm_int8"](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, Ci.ctypes.data, N)
    assert lib.last_status() == 0
    assert np.abs(Ci.reshape(M, N) - want).max() < K * 2e-2, "reference tolerance (test_gemm_correctness.cpp:145)"
    Co = np.zeros(M * N, np.float32)
    orc.orc_gemm_int8(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(Co), N)
    u.assert_bits_equal(Ci, Co, f"gemm_int8 {M}x{N}x{K}")


@pytest.mark.parametrize("alpha,beta", [(2.0, 0.0), (1.0, 0.5)])
def test_gemm_correctness_alpha_beta(lib, orc, dev, alpha, beta):
    M, N, K = 32, 48, 64  # test_gemm_correctness.cpp:188-224
    A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
    C0 = u.uniform(orc, M * N, 3) if beta else np.zeros(M * N, np.float32)
    C = C0.copy()
    lib.cxx["gemm_fp32"](M, N, K, alpha, A.ctypes.data, K, B.ctypes.data, N, beta, C.ctypes.data, N)
    assert lib.last_status() == 0
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), alpha, beta, C0.reshape(M, N))
    assert np.abs(C.reshape(M, N) - want).max() < K * 4e-5
    u.assert_fp32_close(C.reshape(M, N), want, scale, K, f"alpha={alpha} beta={beta}")


DISPATCH_SHAPES = [  # (M, N, K, transa, transb): test_dispatch_logic.cpp:143-153
    (1, 256, 1024, "N", "N"), (256, 1024, 1, "T", "N"), (4, 256, 1024, "N", "N"), (32, 256, 256, "N", "N"),
    (32, 256, 512, "N", "N"), (32, 512, 256, "N", "N"), (8, 512, 512, "N", "N"), (8, 512, 1376, "N", "N"),
    (256, 256, 256, "N", "N"),
]


@pytest.mark.parametrize("M,N,K,ta,tb", DISPATCH_SHAPES)
def test_dispatch_logic_shapes(lib, orc, dev, M, N, K, ta, tb):
    """Column-major, lda = M (K when transposed), ldb = K, ldc = M, alpha 1,
    beta 0, as the reference's test (:195-204)."""
    opA = u.uniform(orc, M * K, 1, 0.0, 1.0).reshape(M, K)
    opB = u.uniform(orc, K * N, 2, 0.0, 1.0).reshape(K, N)
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb)
    C = np.zeros(M * N, np.float32)
    assert lib.onednn_sgemm(ta, tb, M, N, K, 1.0, A, lda, B, ldb, 0.0, C, M) == u.binding().OK
    got = u.cm_load(C, M, N, M)
    want, scale = u.exact(opA, opB)
    assert np.abs(got - want).max() < K * 2e-5, "reference tolerance (test_dispatch_logic.cpp:222)"
    u.assert_fp32_close(got, want, scale, K, f"onednn {ta}{tb} {M}x{N}x{K}")
