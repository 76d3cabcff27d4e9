"""GPU parity of the oneDNN-hook entry points (column-major C, optional bias,
K == 0, ldc < M) and of bf16 GEMMs with transposed operands, through the
C-ABI, against the CPU oracle and the fp64 closed form.

Tolerances are those of _util.py: fp32 accumulation within
(2K+4) * 2^-24 * scale of the fp64 product (the bias adds one more rounding:
|bias| joins the scale); the K == 0 path and small-integer inputs are
compared bit for bit.
"""

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev_copy(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


TRANS = [("N", "N"), ("T", "N"), ("N", "T"), ("T", "T")]


# ---------------------------------------------------------------- bf16 with transposes (row-major)
# Skinny (M <= 8), LDS tiles (M > 8, even strides), register tiles (odd
# strides), ragged M/N/K.
BF16_EX = [(1, 4096, 4096, 0), (4, 1000, 512, 0), (7, 33, 65, 1), (32, 300, 260, 0), (9, 33, 250, 1),
           (256, 1024, 512, 0), (100, 1001, 129, 0), (64, 100, 129, 1), (130, 64, 1000, 0)]


@pytest.mark.parametrize("M,N,K,odd", BF16_EX)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_bf16_ex_transposes(lib, orc, dev, M, N, K, odd, ta, tb):
    opA = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    opB = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02)).reshape(K, N)
    SA = opA.T if ta else opA
    SB = opB.T if tb else opB
    # row-major storage with padded strides (odd when `odd`, else even)
    lda = SA.shape[1] + (1 if odd else 2)
    ldb = SB.shape[1] + (1 if odd else 4)
    A = np.zeros((SA.shape[0], lda), np.uint16)
    A[:, :SA.shape[1]] = SA
    B = np.zeros((SB.shape[0], ldb), np.uint16)
    B[:, :SB.shape[1]] = SB
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dC = dev_copy(C0, dev)
    lib.gemm_bf16_ex(M, N, K, 0.5, dev_copy(A.view(np.int16), dev), lda, dev_copy(B.view(np.int16), dev), ldb, 1.0,
                     dC, N, transA=ta, transB=tb, stream=stream())
    want, scale = u.exact(u.bf16_value(opA), u.bf16_value(opB), 0.5, 1.0, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"bf16_ex {ta}{tb} {M}x{N}x{K}")


def test_bf16_ex_misaligned_b_rows(lib, orc, dev):
    """B stored N x K starting 2 bytes off a 4-byte boundary: the register
    tiles with shifted loads serve it."""
    M, N, K = 64, 200, 256
    A = u.bf16_bits(orc, u.normal(orc, M * K, 1))
    B = u.bf16_bits(orc, u.normal(orc, N * K + 1, 2, 0, 0.02))
    dA, dB = dev_copy(A.view(np.int16), dev), dev_copy(B.view(np.int16), dev)
    dC = torch.zeros((M, N), dtype=torch.float32, device=dev)
    lib.gemm_bf16_ex(M, N, K, 1.0, dA, K, dB.data_ptr() + 2, K, 0.0, dC, N, transB=1, stream=stream())
    want, scale = u.exact(u.bf16_value(A).reshape(M, K), u.bf16_value(B[1:]).reshape(N, K).T)
    u.assert_fp32_close(host(dC), want, scale, K, "bf16_ex misaligned B")


# ---------------------------------------------------------------- row dot: M <= 8, B stored N x K
ROWDOT = [(M, N, K) for M in (1, 2, 3, 4, 5, 6, 7, 8) for (N, K) in ((1, 1), (5, 3), (257, 1000), (1009, 2051))]
ROWDOT += [(1, 4096, 4096), (7, 11003, 2048), (4, 33, 65536)]


@pytest.mark.parametrize("M,N,K", ROWDOT)
def test_rowdot_fp32(lib, orc, dev, M, N, K):
    """fp32 C = A B^T (+ beta C) with B stored N x K (the row-dot kernel; from
    M = 5 at N >= 2048 the 16-row MFMA tiles); the row padding past K holds
    Inf and NaN, which must not reach any product."""
    lda, ldb = K + 3, K + 5
    A = np.full((M, lda), np.inf, np.float32)
    B = np.full((N, ldb), np.nan, np.float32)
    A[:, :K] = u.normal(orc, M * K, 1).reshape(M, K)
    B[:, :K] = u.normal(orc, N * K, 2, 0, 0.02).reshape(N, K)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    p = lib.plan_sgemm(M, N, K, transB=1)
    assert p["name"] in (("dnnopt_tile_f32", "dnnopt_tile_f32_dma") if M >= 5 and N >= 2048 else ("dnnopt_rowdot",)), p
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    for beta in (0.0, 0.5):
        dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
        lib.sgemm(M, N, K, 1.5, dA, lda, dB, ldb, beta, dC, N, transB=1, stream=stream())
        want, scale = u.exact(A[:, :K], B[:, :K].T, 1.5, beta, C0 if beta else None)
        u.assert_fp32_close(host(dC), want, scale, K, f"rowdot f32 {M}x{N}x{K} beta={beta}")


@pytest.mark.parametrize("M,N,K", [(1, 11008, 4096), (4, 1009, 2051), (8, 257, 1000), (3, 5, 3), (2, 64, 65536)])
@pytest.mark.parametrize("odd", [0, 1])
def test_rowdot_bf16(lib, orc, dev, M, N, K, odd):
    """bf16 storage; odd strides put rows off 4-byte boundaries (shifted
    loads).  Row padding holds bf16 Inf (0x7F80)."""
    lda, ldb = K + 2 + odd, K + 4 + odd
    A = np.full((M, lda), 0x7F80, np.uint16)
    B = np.full((N, ldb), 0x7F80, np.uint16)
    A[:, :K] = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    B[:, :K] = u.bf16_bits(orc, u.normal(orc, N * K, 2, 0, 0.02)).reshape(N, K)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dC = dev_copy(C0, dev)
    lib.gemm_bf16_ex(M, N, K, 1.0, dev_copy(A.view(np.int16), dev), lda, dev_copy(B.view(np.int16), dev), ldb, 1.0,
                     dC, N, transB=1, stream=stream())
    want, scale = u.exact(u.bf16_value(A[:, :K]), u.bf16_value(B[:, :K]).T, 1.0, 1.0, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"rowdot bf16 {M}x{N}x{K} odd={odd}")


def test_rowdot_repeatable(lib, orc, dev):
    M, N, K = 7, 1009, 4096
    A, B = u.normal(orc, M * K, 1), u.normal(orc, N * K, 2, 0, 0.02)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    outs = []
    for _ in range(10):
        dC = torch.zeros((M, N), dtype=torch.float32, device=dev)
        lib.sgemm(M, N, K, 1.0, dA, K, dB, K, 0.0, dC, N, transB=1, stream=stream())
        outs.append(dC)
    first = host(outs[0]).view(np.uint32)
    for o in outs[1:]:
        assert np.array_equal(host(o).view(np.uint32), first)


# ---------------------------------------------------------------- column-major hook, device pointers
# Column-major (M, N, K): the row-major problem is N x M x K, so these reach
# the fp32 tiles (with and without k-splits), the skinny kernel (with
# k-splits: (4099, 3, 2048)) and, for transa = 'T', the row-dot kernel.
HOOK = [(7, 1009, 2048), (31, 4096, 1024), (64, 300, 257), (1, 513, 77), (200, 3, 129), (16, 11008, 512),
        (4099, 3, 2048), (16, 20, 65536)]


def _hook_case(orc, M, N, K, ta, tb, pad, bf16):
    opA = u.normal(orc, M * K, 1).reshape(M, K)
    opB = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    if bf16:
        opA = u.bf16_value(u.bf16_bits(orc, opA))
        opB = u.bf16_value(u.bf16_bits(orc, opB))
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=pad)
    if bf16:
        A, B = u.bf16_bits(orc, A).view(np.int16), u.bf16_bits(orc, B).view(np.int16)
    return opA, opB, A, lda, B, ldb


@pytest.mark.parametrize("M,N,K", HOOK)
@pytest.mark.parametrize("ta,tb", TRANS)
@pytest.mark.parametrize("bf16", [False, True])
def test_hook_device(lib, orc, dev, M, N, K, ta, tb, bf16):
    opA, opB, A, lda, B, ldb = _hook_case(orc, M, N, K, ta, tb, 2, bf16)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    bias = None if bf16 else u.uniform(orc, M, 4)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    for beta, ldc in ((0.0, M), (1.0, M + 3)):
        Cbuf = u.cm_store(C0 if beta else np.full_like(C0, np.nan), ldc, fill=-777.0)
        dC = dev_copy(Cbuf, dev)
        if bf16:
            lib.ext_gemm_bf16bf16f32(ta, tb, M, N, K, 1.5, dA, lda, dB, ldb, beta, dC, ldc, stream=stream())
        else:
            lib.ext_sgemm(ta, tb, M, N, K, 1.5, dA, lda, dB, ldb, beta, dC, ldc, bias=dev_copy(bias, dev),
                          stream=stream())
        got = host(dC)
        want, scale = u.exact(opA, opB, 1.5, beta, C0 if beta else None)
        if bias is not None:
            want, scale = want + bias[:, None], scale + np.abs(bias)[:, None]
        u.assert_fp32_close(u.cm_load(got, M, N, ldc), want, scale, K + 1,
                            f"hook {'bf16' if bf16 else 'f32'} {ta}{tb} {M}x{N}x{K} beta={beta}")
        assert (got.reshape(N, ldc)[:, M:] == -777.0).all(), "padding rows of C written"


# (hook M, N, K, transa): the library's row-major problem is N x M, so these
# reach, in order, the skinny kernel, the row-dot kernel, a tile, the tall
# kernel (K % 16 == 0 and not), a tile with k-splits and the skinny kernel
# with k-splits.
BIAS_ROUNDING = [(1009, 3, 70, "N"), (1009, 5, 70, "T"), (300, 100, 64, "N"), (48, 8192, 64, "N"),
                 (40, 5000, 70, "N"), (64, 16, 65536, "N"), (7, 2, 200000, "N")]


@pytest.mark.parametrize("M,N,K,ta", BIAS_ROUNDING)
def test_hook_bias_rounds_separately(lib, orc, dev, M, N, K, ta):
    """beta == 0 with a bias: C = round(round(alpha * acc) + bias), the bias
    added to the finished product as its own rounding (the reference adds it
    after the GEMM).  Integer operands keep acc exact, alpha = 1/3 makes
    alpha * acc inexact, so a fused alpha * acc + bias differs in some
    elements and the comparison is bit for bit."""
    opA = u.small_ints(orc, M * K, 1).reshape(M, K)
    opB = u.small_ints(orc, K * N, 2).reshape(K, N)
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, "N")
    bias = u.uniform(orc, M, 4, -100.0, 100.0)
    alpha = np.float32(1.0 / 3.0)
    acc = (opA.astype(np.int64) @ opB.astype(np.int64)).astype(np.float32)  # |acc| < 2^24: exact
    want = (alpha * acc) + bias[:, None]  # float32 ops, each rounded
    fused = ((np.float64(alpha) * acc.astype(np.float64)) + bias[:, None].astype(np.float64)).astype(np.float32)
    assert (fused != want).any(), "inputs do not separate fused from unfused rounding"
    dC = dev_copy(np.full(M * N, np.nan, np.float32), dev)
    lib.ext_sgemm(ta, "N", M, N, K, float(alpha), dev_copy(A, dev), lda, dev_copy(B, dev), ldb, 0.0, dC, M,
                  bias=dev_copy(bias, dev), stream=stream())
    u.assert_bits_equal(u.cm_load(host(dC), M, N, M), want, f"bias rounding {M}x{N}x{K} {ta}")


@pytest.mark.parametrize("ldc_delta", [2, 0, -3])
@pytest.mark.parametrize("with_bias", [False, True])
def test_hook_k_zero_bitwise(lib, orc, dev, ldc_delta, with_bias):
    """K == 0 (including overlapping columns, ldc < M) against the oracle,
    bit for bit: beta 0 (C not read), 1, -2 and 0.3 (one rounding each)."""
    M, N = 9, 6
    ldc = M + ldc_delta
    total = (N - 1) * ldc + M
    bias = u.uniform(orc, M, 4) if with_bias else None
    dbias = dev_copy(bias, dev) if with_bias else None
    for beta in (0.0, 1.0, -2.0, 0.3):
        C0 = u.uniform(orc, total, 3)
        if beta == 0.0:
            C0[:] = np.nan  # not read
        want = C0.copy()
        nan = np.full(2, np.nan, np.float32)
        assert orc.orc_onednn_sgemm(b"N", b"N", M, N, 0, float("nan"), u.ptr(nan), M, u.ptr(nan), 1, beta,
                                    u.ptr(want), ldc, None if bias is None else u.ptr(bias)) == 0
        dC = dev_copy(C0, dev)
        lib.ext_sgemm("N", "N", M, N, 0, float("nan"), None, M, None, 1, beta, dC, ldc, bias=dbias, stream=stream())
        got = host(dC)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (beta, ldc)


@pytest.mark.parametrize("ta,tb", TRANS)
@pytest.mark.parametrize("beta,with_bias", [(0.0, False), (0.5, True), (1.0, False)])
@pytest.mark.parametrize("bf16", [False, True])
def test_hook_overlapping_columns(lib, orc, dev, ta, tb, beta, with_bias, bf16):
    """ldc < M: small-integer inputs (every rounding exact), so the result at
    every address -- decided by the reference's write-back and bias loop
    order -- must equal the oracle's bit for bit."""
    if bf16 and with_bias:
        with_bias = False
    M, N, K, ldc = 40, 23, 70, 11
    opA = u.small_ints(orc, M * K, 1).reshape(M, K)
    opB = u.small_ints(orc, K * N, 2).reshape(K, N)
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=1)
    if bf16:
        A, B = u.bf16_bits(orc, A), u.bf16_bits(orc, B)
    total = (N - 1) * ldc + M
    C0 = u.small_ints(orc, total, 3)
    bias = u.small_ints(orc, M, 4) if with_bias else None
    want = C0.copy()
    if bf16:
        orc.orc_onednn_gemm_bf16bf16f32(ta.encode(), tb.encode(), M, N, K, 1.0, u.ptr(A), lda, u.ptr(B), ldb, beta,
                                        u.ptr(want), ldc)
    else:
        orc.orc_onednn_sgemm(ta.encode(), tb.encode(), M, N, K, 1.0, u.ptr(A), lda, u.ptr(B), ldb, beta,
                             u.ptr(want), ldc, None if bias is None else u.ptr(bias))
    dC = dev_copy(C0, dev)
    if bf16:
        lib.ext_gemm_bf16bf16f32(ta, tb, M, N, K, 1.0, dev_copy(A.view(np.int16), dev), lda,
                                 dev_copy(B.view(np.int16), dev), ldb, beta, dC, ldc, stream=stream())
    else:
        lib.ext_sgemm(ta, tb, M, N, K, 1.0, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, beta, dC, ldc,
                      bias=None if bias is None else dev_copy(bias, dev), stream=stream())
    u.assert_bits_equal(host(dC), want, f"overlap ldc={ldc} bf16={bf16} beta={beta} bias={with_bias} {ta}{tb}")


# ---------------------------------------------------------------- the hook's own argument list (host memory)
@pytest.mark.parametrize("ta,tb", TRANS)
def test_onednn_host_pointers(lib, orc, dev, ta, tb):
    M, N, K = 24, 1000, 300
    opA, opB, A, lda, B, ldb = _hook_case(orc, M, N, K, ta, tb, 0, False)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    bias = u.uniform(orc, M, 4)
    b = u.binding()
    for beta, ldc in ((0.0, M + 5), (1.0, M)):
        C = u.cm_store(C0, ldc, fill=-777.0)
        assert lib.onednn_sgemm(ta, tb, M, N, K, 1.0, A, lda, B, ldb, beta, C, ldc, bias=bias) == b.OK
        want, scale = u.exact(opA, opB, 1.0, beta, C0 if beta else None)
        u.assert_fp32_close(u.cm_load(C, M, N, ldc), want + bias[:, None], scale + np.abs(bias)[:, None], K + 1,
                            f"onednn host {ta}{tb} beta={beta}")
        assert (C.reshape(N, ldc)[:, M:] == -777.0).all(), "padding rows of C written"
    opA, opB, Ab, lda, Bb, ldb = _hook_case(orc, M, N, K, ta, tb, 3, True)
    C = u.cm_store(C0, M)
    assert lib.onednn_gemm_bf16bf16f32(ta, tb, M, N, K, 1.0, Ab, lda, Bb, ldb, 1.0, C, M) == b.OK
    want, scale = u.exact(opA, opB, 1.0, 1.0, C0)
    u.assert_fp32_close(u.cm_load(C, M, N, M), want, scale, K, f"onednn bf16 host {ta}{tb}")
    # packed operands: unimplemented, C untouched
    Cp = u.cm_store(C0, M)
    assert lib.onednn_sgemm("P", tb, M, N, K, 1.0, A, lda, B, ldb, 0.0, Cp, M) == b.ERR_UNSUPPORTED
    assert np.array_equal(Cp, u.cm_store(C0, M))


def test_cxx_host_padded_c_beta_zero(lib, orc, dev):
    """Host-pointer C++ API, beta == 0, ldc > N: the padding between rows of C
    is the caller's and must come back unchanged."""
    M, N, K, ldc = 5, 300, 64, 307
    A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
    for fn in ("gemm_fp32", "gemm_bf16"):
        C = np.full((M, ldc), -777.0, np.float32)
        lib.cxx[fn](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, C.ctypes.data, ldc)
        assert lib.last_status() == 0
        assert (C[:, N:] == -777.0).all(), fn
        want, scale = u.exact(A.reshape(M, K), B.reshape(K, N))
        tol = u.fp32_tol(K, scale) if fn == "gemm_fp32" else 1e-2 * scale
        assert (np.abs(C[:, :N] - want) <= tol).all(), fn


def test_ticket_reduction_mode(lib, orc, dev):
    """The split-k reduction by the last-arriving workgroup (the library's
    alternative to the reduce kernel, tunable SPLIT_REDUCE=0) gives results
    within the fp32 bound, bias included, for k-split shapes of the skinny and
    tile kernels and of the oneDNN hook."""
    s = torch.cuda.current_stream().cuda_stream

    def dcopy(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def host(t):
        torch.cuda.synchronize()
        return t.cpu().numpy()

    with lib.tunables(SPLIT_REDUCE=0, TILE_SPLITS=4):
        # row-major fp32: skinny with k-splits, tiles with 4 forced k-splits
        # (tiles take the ticket path up to 16 splits, the skinny kernel always)
        for M, N, K in ((1, 4096, 4096), (7, 1009, 2048), (3, 257, 5000), (1024, 256, 1024), (300, 600, 2048)):
            p = lib.plan_sgemm(M, N, K)
            assert p["splits"] > 1 and (M <= 8 or p["splits"] <= 16), (M, N, K, p)
            A, B, C0 = u.normal(orc, M * K, 1), u.normal(orc, K * N, 2, 0, 0.02), u.uniform(orc, M * N, 3)
            dC = dcopy(C0)
            lib.sgemm(M, N, K, 1.0, dcopy(A), K, dcopy(B), N, 1.0, dC, N, stream=s)
            want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), 1.0, 1.0, C0.reshape(M, N))
            u.assert_fp32_close(host(dC).reshape(M, N), want, scale, K, f"ticket sgemm {M}x{N}x{K}")
        # column-major hook with bias: skinny (transa 'N') and tiles with k-splits
        for M, N, K, ta in ((4099, 3, 2048, "N"), (256, 1024, 1024, "N"), (256, 1024, 1024, "T")):
            opA = u.normal(orc, M * K, 1).reshape(M, K)
            opB = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
            A, lda, B, ldb = u.hook_operands(opA, opB, ta, "N")
            C0 = u.uniform(orc, M * N, 3).reshape(M, N)
            bias = u.uniform(orc, M, 4)
            dC = dcopy(u.cm_store(C0, M))
            lib.ext_sgemm(ta, "N", M, N, K, 1.0, dcopy(A), lda, dcopy(B), ldb, 0.5, dC, M, bias=dcopy(bias),
                          stream=s)
            want, scale = u.exact(opA, opB, 1.0, 0.5, C0)
            u.assert_fp32_close(u.cm_load(host(dC), M, N, M), want + bias[:, None],
                                scale + np.abs(bias)[:, None], K + 1, f"ticket hook {ta} {M}x{N}x{K}")
    assert lib.get_tunable("SPLIT_REDUCE") == 1


@pytest.mark.parametrize("M,N,K,dt", [(1, 4096, 4096, "f32"), (2, 4099, 2048, "f32"), (3, 11003, 2048, "f32"),
                                      (7, 1009, 2048, "f32"), (1, 11008, 4096, "bf16"), (3, 1001, 5000, "bf16")])
def test_split_sums_bit_identical_across_modes(lib, dev, M, N, K, dt):
    """The skinny kernel's split-k sums, by the last-arriving workgroup
    (SPLIT_REDUCE=0), the planner's choice (1) or the reduce kernel (2), add
    the splits in the same order: the three give the same bits."""
    g = torch.Generator(device="cpu").manual_seed(M * N + K)
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    A = torch.randn(M, K, generator=g).to(dtype).to(dev)
    B = (torch.randn(K, N, generator=g) * 0.02).to(dtype).to(dev)
    C0 = (torch.rand(M, N, generator=g) * 2 - 1).to(dev)
    outs = []
    for mode in (0, 1, 2):
        C = C0.clone()
        with lib.tunables(SPLIT_REDUCE=mode):
            assert lib.plan_sgemm(M, N, K)["splits"] > 1
            fn = lib.sgemm if dt == "f32" else lib.gemm_bf16
            fn(M, N, K, 1.0, A, K, B, N, 1.0, C, N, stream=torch.cuda.current_stream().cuda_stream)
        outs.append(C)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2]), (M, N, K, dt)


@pytest.mark.parametrize("M,N,K,tb,forced", [(128, 3072, 768, 0, 0), (784, 128, 1152, 1, 0), (196, 256, 2304, 0, 0),
                                             (176, 64, 4608, 1, 0), (49, 512, 4608, 1, 0), (128, 768, 3072, 0, 0),
                                             (300, 600, 2048, 0, 4), (1000, 1000, 3000, 1, 6)])
def test_tile_split_sums_bit_identical_across_modes(lib, dev, M, N, K, tb, forced):
    """fp32 MFMA tiles with k-splits: the tile's last-arriving workgroup
    (SPLIT_REDUCE=0, and the default up to 8 splits) and the reduce kernel
    (2) add the partials in the same split order and apply the same
    epilogue, so C is bit-identical (beta = 1 over a preset C)."""
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N * 3 + K)
    A = torch.randn(M, K, generator=g).to(dev)
    B = (torch.randn(*((N, K) if tb else (K, N)), generator=g) * 0.02).to(dev)
    C0 = (torch.rand(M, N, generator=g) * 2 - 1).to(dev)
    outs = []
    for mode in (0, 1, 2):
        C = C0.clone()
        with lib.tunables(SPLIT_REDUCE=mode, TILE_SPLITS=forced):
            p = lib.plan_sgemm(M, N, K, transB=tb)
            assert p["name"].startswith("dnnopt_tile_f32") and p["splits"] > 1, p
            lib.sgemm(M, N, K, 0.75, A, K, B, K if tb else N, 1.0, C, N, transB=tb,
                      stream=torch.cuda.current_stream().cuda_stream)
        outs.append(C)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[2]), (M, N, K, tb, forced)
