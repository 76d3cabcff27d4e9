"""Pins for the CPU oracle (oracle/oracle.c) -- no GPU needed.

Every oracle function is checked against something that does not share its
code: the reference's own sources built in oracle/_ref (bit-exact), committed
golden fixtures made from them, closed forms, exact small-integer cases, the
fp64 error bound, and planted mistakes that a weaker check would miss.
"""

import os

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

# Shapes of the reference's own tests (tests/test_gemm_correctness.cpp:160-183,
# tests/test_cblas.cpp:341-349) plus ragged edges.
REF_SHAPES = [
    (1, 1, 1), (4, 4, 4), (8, 8, 8), (16, 16, 16), (1, 128, 64), (7, 13, 5), (3, 3, 1000),
    (128, 1, 768), (1, 1000, 2048), (5, 7, 11), (13, 17, 19), (32, 64, 48), (1, 64, 32),
]


def _f(x):
    """A fresh C-contiguous float32 copy."""
    return np.array(x, np.float32, order="C", copy=True)


# ---------------------------------------------------------------- generator
def test_splitmix64_published_vector(orc):
    # SplitMix64 reference output for state 1234567 (Vigna's splitmix64.c).
    out = np.zeros(5, np.uint64)
    orc.orc_splitmix64(1234567, u.ptr(out), 5)
    assert out.tolist() == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821,
    ]


def test_generator_ranges(orc):
    x = u.uniform(orc, 200000, 7)
    assert x.min() >= -1.0 and x.max() < 1.0 and abs(x.mean()) < 0.01
    g = u.normal(orc, 200000, 8, 0.0, 0.02)
    assert abs(g.mean()) < 2e-4 and abs(g.std() - 0.02) < 2e-4
    q = u.ints8(orc, 200000, 9)
    assert q.min() == -127 and q.max() == 127
    # Different tensor ids give unrelated streams; same id is reproducible.
    assert not np.array_equal(u.uniform(orc, 64, 1), u.uniform(orc, 64, 2))
    assert np.array_equal(u.uniform(orc, 64, 1), u.uniform(orc, 64, 1))


# ---------------------------------------------------------------- bf16
def test_bf16_closed_form(orc):
    cases = {
        0x3F800000: 0x3F80, 0x3F808000: 0x3F80,  # tie, even below
        0x3F818000: 0x3F82,  # tie, even above
        0x3F808001: 0x3F81, 0x3F807FFF: 0x3F80,
        0x7F7FFFFF: 0x7F80,  # rounds up to infinity
        0x80000000: 0x8000, 0x00000001: 0x0000,
    }
    for bits, want in cases.items():
        f = np.array([bits], np.uint32).view(np.float32)[0]
        assert orc.orc_bf16_rne(float(f)) == want, hex(bits)


def test_bf16_matches_reference_header(orc, ref):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite values
    vals = bits.view(np.float32)
    for v in vals[:20000]:
        assert orc.orc_bf16_rne(float(v)) == ref.ref_bf16_round(float(v))


def test_bf16_matches_torch_rne(orc):
    torch = pytest.importorskip("torch")
    x = u.normal(orc, 50000, 11, 0.0, 3.0)
    got = u.bf16_bits(orc, x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- scalar fp32 path
@pytest.mark.parametrize("shape", REF_SHAPES)
@pytest.mark.parametrize("ab", [(1.0, 0.0), (2.5, -0.3)])
def test_naive_bitwise_vs_reference(orc, ref, shape, ab):
    M, N, K = shape
    alpha, beta = ab
    A = u.uniform(orc, M * K, 1)
    B = u.uniform(orc, K * N, 2)
    C0 = u.uniform(orc, M * N, 3)
    c1, c2 = C0.copy(), C0.copy()
    ref.ref_gemm_naive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(c1), N)
    orc.orc_gemm_naive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(c2), N)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), alpha, beta, C0.reshape(M, N))
    u.assert_fp32_close(c2.reshape(M, N), want, scale, K, "naive")


def test_int8_bitwise_vs_reference(orc, ref):
    for M, N, K in [(1, 7, 300), (9, 13, 77), (8, 4093, 64), (17, 9, 1)]:
        A = u.ints8(orc, M * K, 1)
        B = u.ints8(orc, N * K, 2)
        c1 = np.empty(M * N, np.int32)
        c2 = np.empty(M * N, np.int32)
        ref.ref_gemm_s8s8s32(M, N, K, u.ptr(A), K, u.ptr(B), K, u.ptr(c1), N)
        orc.orc_gemm_s8s8s32(M, N, K, u.ptr(A), K, u.ptr(B), K, u.ptr(c2), N)
        assert np.array_equal(c1, c2)
        want = A.reshape(M, K).astype(np.int64) @ B.reshape(N, K).astype(np.int64).T
        assert np.array_equal(c2.reshape(M, N), want)


def test_int8_extremes_no_overflow(orc):
    K = 4096
    A = np.full(K, -128, np.int8)
    B = np.full(2 * K, -128, np.int8)
    C = np.empty(2, np.int32)
    orc.orc_gemm_s8s8s32(1, 2, K, u.ptr(A), K, u.ptr(B), K, u.ptr(C), 2)
    assert C.tolist() == [K * 128 * 128] * 2  # 67,108,864 < 2^31


def test_saxpy_bitwise_vs_reference(orc, ref):
    # increments of 0: X[0] broadcast, every update on Y[0] in order
    # (cblas_saxpy.cpp:45-49)
    for n, incx, incy in [(1, 1, 1), (37, 1, 1), (100, 3, 2), (50, 0, 1), (50, 2, 0), (50, 0, 0)]:
        X = u.uniform(orc, max(1, n * incx), 5)
        Y0 = u.uniform(orc, max(1, n * incy), 6)
        y1, y2 = Y0.copy(), Y0.copy()
        ref.ref_saxpy(n, 0.7, u.ptr(X), incx, u.ptr(y1), incy)
        orc.orc_saxpy(n, 0.7, u.ptr(X), incx, u.ptr(y2), incy, 0)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    # alpha == 0 and N <= 0 are no-ops (cblas_saxpy.cpp:15)
    y = Y0.copy()
    orc.orc_saxpy(n, 0.0, u.ptr(X), incx, u.ptr(y), incy, 1)
    assert np.array_equal(y, Y0)


# ---------------------------------------------------------------- small-M kernels (order-faithful)
def _run_smallm(orc, fn, M, N, K, alpha, beta, A, B, C0):
    C = C0.copy()
    if fn == "gemv":
        orc.orc_gemv_1xn_f32(N, K, alpha, u.ptr(A), u.ptr(B), N, beta, u.ptr(C))
    elif fn == "wide":
        orc.orc_smallm_wide_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N)
    elif fn == "adaptive":
        orc.orc_adaptive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N, 6 if M == 7 else 5,
                             65536, 2)
    else:
        assert orc.orc_gemm_f32_smallm(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N, 2) == 0
    return C


SMALLM = [("gemv", 1, 67, 300), ("gemv", 1, 4096, 64), ("wide", 2, 1009, 96), ("wide", 3, 53, 257),
          ("wide", 5, 97, 80), ("wide", 7, 47, 600), ("adaptive", 5, 4099, 700), ("adaptive", 7, 61, 1300),
          ("route", 7, 1009, 64)]


@pytest.mark.parametrize("fn,M,N,K", SMALLM)
def test_smallm_exact_on_integers(orc, fn, M, N, K):
    """Small integers keep every partial sum exact, so any correct order must
    reproduce the integer product bit for bit; a wrong index, stride or a
    dropped term cannot."""
    rng = np.random.default_rng(M * 1000 + N)
    A = _f(rng.integers(-8, 9, M * K))
    B = _f(rng.integers(-8, 9, K * N))
    C0 = _f(rng.integers(-50, 51, M * N))
    C = _run_smallm(orc, fn, M, N, K, 1.0, 2.0, A, B, C0)
    want = A.reshape(M, K).astype(np.int64) @ B.reshape(K, N).astype(np.int64) + 2 * C0.reshape(M, N)
    assert np.array_equal(C.reshape(M, N), want.astype(np.float32))


@pytest.mark.parametrize("fn,M,N,K", SMALLM)
def test_smallm_error_bound(orc, fn, M, N, K):
    A = u.normal(orc, M * K, 1, 0, 0.02)
    B = u.normal(orc, K * N, 2, 0, 0.02)
    C0 = u.uniform(orc, M * N, 3)
    for alpha, beta in [(1.0, 1.0), (1.0, 0.0), (-0.5, 0.25)]:
        C = _run_smallm(orc, fn, M, N, K, alpha, beta, A, B, C0)
        want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), alpha, beta, C0.reshape(M, N))
        u.assert_fp32_close(C.reshape(M, N), want, scale, K, fn)


def test_smallm_beta0_never_reads_c(orc):
    N, K = 70, 33
    B = u.uniform(orc, K * N, 2)
    for fn, m in (("gemv", 1), ("wide", 3), ("adaptive", 5)):
        # every buffer sized for the m rows the routine touches
        A = u.uniform(orc, m * K, 1)
        C = _run_smallm(orc, fn, m, N, K, 1.0, 0.0, A, B, np.full(m * N, np.nan, np.float32))
        assert C.size == m * N and np.isfinite(C).all(), fn


def test_fused_order_is_not_the_naive_order(orc):
    """The GEMV restatement must use the fused k-ordered sums of the NEON
    kernel, not the separately rounded naive loop: on random data the two
    differ in the last bits somewhere, and K = 1 makes them agree."""
    N, K = 512, 512
    A, B = u.uniform(orc, K, 1), u.uniform(orc, K * N, 2)
    C0 = np.zeros(N, np.float32)
    fused = _run_smallm(orc, "gemv", 1, N, K, 1.0, 0.0, A, B, C0)
    naive = C0.copy()
    orc.orc_gemm_naive_f32(1, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(naive), N)
    assert not np.array_equal(fused, naive)
    f1 = _run_smallm(orc, "gemv", 1, N, 1, 1.0, 0.0, A, B, C0)
    n1 = C0.copy()
    orc.orc_gemm_naive_f32(1, N, 1, 1.0, u.ptr(A), 1, u.ptr(B), N, 0.0, u.ptr(n1), N)
    assert np.array_equal(f1, n1)


def test_adaptive_reduces_to_wide(orc):
    """With one Kc block and beta = 0 the adaptive tiles and the wide driver
    perform the same operations; with several blocks and beta != 0 the
    per-block re-rounding of C must show."""
    M, N, K = 5, 160, 200
    A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
    C0 = u.uniform(orc, M * N, 3)
    w = _run_smallm(orc, "wide", M, N, K, 1.0, 0.0, A, B, C0)
    a = C0.copy()
    orc.orc_adaptive_f32(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(a), N, 5, 1 << 28, 1)
    assert np.array_equal(w.view(np.uint32), a.view(np.uint32))
    a2 = C0.copy()
    orc.orc_adaptive_f32(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 1.0, u.ptr(a2), N, 5, 4096, 1)
    w2 = _run_smallm(orc, "wide", M, N, K, 1.0, 1.0, A, B, C0)
    assert not np.array_equal(w2.view(np.uint32), a2.view(np.uint32))


# ---------------------------------------------------------------- bf16 / dynamic int8
def test_bf16_oracle_bound(orc):
    M, N, K = 4, 300, 513
    A = u.bf16_bits(orc, u.normal(orc, M * K, 1))
    B = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02))
    C = np.zeros(M * N, np.float32)
    orc.orc_gemm_bf16(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(C), N)
    want, scale = u.exact(u.bf16_value(A).reshape(M, K), u.bf16_value(B).reshape(K, N))
    u.assert_fp32_close(C.reshape(M, N), want, scale, K, "bf16")


def test_int8_dynq_closed_form(orc):
    # max|A| = 127 and max|B| = 254: scales 1 and 2, quantization exact.
    A = _f([[127, -64, 3]])
    B = _f([[254, 2], [-100, 0], [6, -254]])
    C = np.zeros(2, np.float32)
    orc.orc_gemm_int8_dynq(1, 2, 3, 1.0, u.ptr(A), 3, u.ptr(B), 2, 0.0, u.ptr(C), 2)
    assert C.tolist() == (A.astype(np.float64) @ B.astype(np.float64)).ravel().tolist()
    # An all-zero operand has scale 1 and a zero product; beta keeps C.
    Z = np.zeros(3, np.float32)
    C2 = _f([5, -7])
    orc.orc_gemm_int8_dynq(1, 2, 3, 1.0, u.ptr(Z), 3, u.ptr(B), 2, 0.5, u.ptr(C2), 2)
    assert C2.tolist() == [2.5, -3.5]


def _oracle_dynq(so, fn="orc_gemm_int8_dynq"):
    def run(M, N, K, A, B):
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        C = np.full(M * N, np.nan, np.float32)
        getattr(so, fn)(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(C), N)
        return C

    return run


def test_int8_dynq_rounding_ties(orc):
    # Quantized values that are exact ties or fractions: only nearest-even
    # rounding (lrintf, src/gemm/gemm_pack_int8.cpp:66-71) gives these C.
    u.check_dynq_ties(_oracle_dynq(orc))


@pytest.mark.parametrize("wrong", ["truncf", "roundf", "floorf"])
def test_int8_dynq_ties_reject_other_roundings(tmp_path, wrong):
    """Build copies of the oracle whose quantizer rounds the wrong way and
    show that the tie test rejects each (a planted mistake, on the CPU)."""
    import ctypes
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler on this host")
    so_path = tmp_path / f"liboracle_{wrong}.so"
    subprocess.run([cc, "-O1", "-fPIC", "-ffp-contract=off", "-fopenmp", "-std=c11", "-shared",
                    f"-DORC_QUANT_ROUND={wrong}", "-o", str(so_path), os.path.join(u.ROOT, "oracle", "oracle.c"),
                    "-lm"], check=True)
    bad = ctypes.CDLL(str(so_path))
    res, args = u.ORACLE_ABI["orc_gemm_int8_dynq"]
    bad.orc_gemm_int8_dynq.restype = res
    bad.orc_gemm_int8_dynq.argtypes = args
    with pytest.raises(AssertionError, match="quantization ties"):
        u.check_dynq_ties(_oracle_dynq(bad))


def _oracle_int8(so, fn="orc_gemm_int8"):
    def run(M, N, K, A, B, alpha, beta, C0):
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        C = np.ascontiguousarray(C0, np.float32).copy()
        getattr(so, fn)(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N)
        return C

    return run


def test_int8_route_closed_forms(orc):
    """gemm_int8's two routes (M <= 8 small-M, M > 8 packed) on inputs whose
    results the arithmetic fixes: the small-M division quantizer (87.5 -> 88
    where the reciprocal gives 87), the M = 1 and M >= 2 epilogues and the
    packed path's fused one, and the sign of a zero result."""
    u.check_int8_routes(_oracle_int8(orc))
    # The ties (scales 1 and 2: division and reciprocal agree) hold on both routes.
    u.check_dynq_ties(_oracle_dynq(orc, "orc_gemm_int8"))


@pytest.mark.parametrize("define,case", [("ORC_SMALLM_RECIP", "division"), ("ORC_SMALLM_FUSED", "beta-fma")])
def test_int8_route_rejects_planted(tmp_path, define, case):
    """Copies of the oracle whose small-M route quantizes with the reciprocal,
    or uses one fused epilogue, are built and rejected by the closed forms."""
    import ctypes
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler on this host")
    so_path = tmp_path / f"liboracle_{define}.so"
    subprocess.run([cc, "-O1", "-fPIC", "-ffp-contract=off", "-fopenmp", "-std=c11", "-shared", f"-D{define}",
                    "-o", str(so_path), os.path.join(u.ROOT, "oracle", "oracle.c"), "-lm"], check=True)
    bad = ctypes.CDLL(str(so_path))
    res, args = u.ORACLE_ABI["orc_gemm_int8"]
    bad.orc_gemm_int8.restype = res
    bad.orc_gemm_int8.argtypes = args
    with pytest.raises(AssertionError, match=f"closed form \\({case}"):
        u.check_int8_routes(_oracle_int8(bad))


def test_int8_smallm_stores_rows_0_to_m_minus_1(orc):
    """The reference's M = 3 store skips row 2 and its M = 7 store adds zeros
    to a row 7 past C (src/gemm/gemm_smallm_int8.cpp:391, 445); the
    restatement stores exactly rows 0..M-1."""
    name, N, K, A, B, alpha, beta, C0, want = u.int8_route_cases(3)[0]
    C = _oracle_int8(orc)(3, N, K, A, B, alpha, beta, C0).reshape(3, N)
    assert np.array_equal(C, want)  # row 2 written (the defect leaves 0 there)
    name, N, K, A, B, alpha, beta, C0, want = u.int8_route_cases(7)[0]
    buf = np.full((8, N), -0.0, np.float32)  # the defect would turn row 7's -0 into +0
    buf[:7] = C0
    orc.orc_gemm_int8(7, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(buf), N)
    assert np.array_equal(buf[:7], want)
    assert np.array_equal(buf[7].view(np.uint32), np.full(N, 0x80000000, np.uint32))


def test_int8_smallm_matches_dynq_when_division_is_exact(orc):
    """With power-of-two scales (max|X| = 127 * 2^e) division and reciprocal
    agree, and with beta = 0 and alpha > 0 the epilogues agree too: the two
    routes then give the same bits (special case that reduces to the packed
    restatement)."""
    for M, N, K in [(1, 37, 19), (4, 64, 100), (8, 13, 257)]:
        A = u.small_ints(orc, M * K, 1, 127)
        A[0] = 127.0
        B = (u.small_ints(orc, K * N, 2, 127) * 2.0).astype(np.float32)
        B[0] = 254.0
        C1 = np.full(M * N, np.nan, np.float32)
        C2 = np.full(M * N, np.nan, np.float32)
        orc.orc_gemm_int8_smallm(M, N, K, 0.5, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(C1), N)
        orc.orc_gemm_int8_dynq(M, N, K, 0.5, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(C2), N)
        assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))
        want = 0.5 * 2.0 * (A.reshape(M, K).astype(np.float64) @ (B.reshape(K, N) / 2.0).astype(np.float64))
        assert np.array_equal(C1.reshape(M, N), want.astype(np.float32))


def test_int8_dynq_reference_tolerance(orc):
    # tests/test_gemm_correctness.cpp:145 bounds the int8 path by K * 2e-2.
    for M, N, K in [(1, 128, 64), (7, 13, 5), (3, 3, 1000), (13, 17, 19)]:
        A, B = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2)
        for fn in ("orc_gemm_int8_dynq", "orc_gemm_int8"):
            C = np.zeros(M * N, np.float32)
            getattr(orc, fn)(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.0, u.ptr(C), N)
            want, _ = u.exact(A.reshape(M, K), B.reshape(K, N))
            assert np.abs(C.reshape(M, N) - want).max() < K * 2e-2, (fn, M, N, K)


def test_colscale_is_one_rounding(orc):
    M, N, K = 3, 11, 64
    A, B = u.ints8(orc, M * K, 1), u.ints8(orc, N * K, 2)
    s = u.uniform(orc, N, 4, 0.001, 0.01)
    C = np.zeros(M * N, np.float32)
    orc.orc_gemm_s8_colscale(M, N, K, u.ptr(A), K, u.ptr(B), K, u.ptr(s), u.ptr(C), N)
    acc = (A.reshape(M, K).astype(np.int64) @ B.reshape(N, K).astype(np.int64).T).astype(np.float32)
    assert np.array_equal(C.reshape(M, N), acc * s[None, :])


# ---------------------------------------------------------------- cblas
CBLAS_CASES = [(o, ta, tb) for o in (101, 102) for ta in (111, 112) for tb in (111, 112)]


@pytest.mark.parametrize("order,ta,tb", CBLAS_CASES)
def test_cblas_oracle_semantics(orc, order, ta, tb):
    M, N, K = 7, 13, 11
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    alpha, beta = 2.5, -0.3
    if order == 101:  # row-major storage of op(A), op(B), C
        A = _f(opA.T if ta == 112 else opA)
        B = _f(opB.T if tb == 112 else opB)
        C = _f(C0)
        lda, ldb, ldc = A.shape[1], B.shape[1], N
    else:  # column-major storage: the row-major view of X is X^T
        A = _f((opA.T if ta == 112 else opA).T)
        B = _f((opB.T if tb == 112 else opB).T)
        C = _f(C0.T)
        lda, ldb, ldc = A.shape[1], B.shape[1], M
    orc.orc_cblas_sgemm(order, ta, tb, M, N, K, alpha, u.ptr(A), lda, u.ptr(B), ldb, beta, u.ptr(C), ldc)
    got = C if order == 101 else C.T
    want, scale = u.exact(opA, opB, alpha, beta, C0)
    u.assert_fp32_close(got, want, scale, K, f"cblas {order} {ta} {tb}")


def test_beta_zero_leaves_c_unread(orc):
    """beta == 0: the reference's kernels store alpha*acc without reading C, so
    NaN/Inf in C must not reach the result, and alpha*0 keeps its sign (-0.0),
    which a zero-fill-then-add restatement would turn into +0.0."""
    M, N, K = 5, 6, 9
    opA = u.small_ints(orc, M * K, 1).reshape(M, K)
    opA[2, :] = 0.0  # row 2 of the product is exactly zero
    opB = u.small_ints(orc, K * N, 2).reshape(K, N)
    want = (-1.0 * (opA.astype(np.float64) @ opB)).astype(np.float32)
    assert np.signbit(want[2]).all()
    poison = np.tile(np.array([np.nan, np.inf, -np.inf], np.float32), M * N)[: M * N]
    # row-major cblas
    C = poison.reshape(M, N).copy()
    orc.orc_cblas_sgemm(101, 111, 111, M, N, K, -1.0, u.ptr(_f(opA)), K, u.ptr(_f(opB)), N, 0.0, u.ptr(C), N)
    u.assert_bits_equal(C, want, "cblas beta=0")
    # oneDNN hook, column-major, ldc >= M and ldc < M (the small-ldc temporary)
    A, lda, B, ldb = u.hook_operands(opA, opB, "N", "N")
    C = poison.copy()
    assert _hook(orc, "N", "N", M, N, K, -1.0, A, lda, B, ldb, 0.0, C, M, None) == 0
    u.assert_bits_equal(u.cm_load(C, M, N, M), want, "hook beta=0")
    ldc = 3
    C = np.full((N - 1) * ldc + M, np.nan, np.float32)
    assert _hook(orc, "N", "N", M, N, K, -1.0, A, lda, B, ldb, 0.0, C, ldc, None) == 0
    C0 = np.zeros_like(C)
    u.assert_bits_equal(C, _overlap_closed_form(opA, opB, C0, M, N, ldc, -1.0, 0.0, None), "hook beta=0 ldc<M")


def test_cblas_early_exits(orc):
    C = _f([1, 2, 3, 4])
    A = B = np.full(4, np.nan, np.float32)
    orc.orc_cblas_sgemm(101, 111, 111, 2, 2, 2, 0.0, u.ptr(A), 2, u.ptr(B), 2, 1.0, u.ptr(C), 2)
    orc.orc_cblas_sgemm(101, 111, 111, 2, 2, 0, 1.0, u.ptr(A), 2, u.ptr(B), 2, 0.0, u.ptr(C), 2)
    assert C.tolist() == [1, 2, 3, 4]


# ---------------------------------------------------------------- oneDNN hook (column-major)
HOOK_T = [("N", "N"), ("T", "N"), ("N", "T"), ("t", "t")]


def _hook(orc, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias=None, bf16=False):
    if bf16:
        return orc.orc_onednn_gemm_bf16bf16f32(ta.encode(), tb.encode(), M, N, K, alpha, u.ptr(A), lda, u.ptr(B), ldb,
                                               beta, u.ptr(C), ldc)
    return orc.orc_onednn_sgemm(ta.encode(), tb.encode(), M, N, K, alpha, u.ptr(A), lda, u.ptr(B), ldb, beta,
                                u.ptr(C), ldc, None if bias is None else u.ptr(bias))


@pytest.mark.parametrize("ta,tb", HOOK_T)
@pytest.mark.parametrize("beta,with_bias,bf16", [(0.0, False, False), (1.0, True, False), (-2.0, True, False),
                                                 (0.5, False, False), (0.0, False, True), (-2.0, False, True)])
def test_onednn_hook_exact_on_integers(orc, ta, tb, beta, with_bias, bf16):
    """Column-major C = alpha op(A) op(B) + beta C (+ bias[i]) on small
    integers, where every rounding is exact: the result must equal the integer
    closed form, and the padding rows of C (ldc > M) must be untouched.  The
    shapes are all different, so a swapped or untransposed operand fails."""
    M, N, K, ldc = 5, 7, 6, 9
    opA = u.small_ints(orc, M * K, 1).reshape(M, K)
    opB = u.small_ints(orc, K * N, 2).reshape(K, N)
    C0 = u.small_ints(orc, M * N, 3).reshape(M, N)
    bias = u.small_ints(orc, M, 4) if with_bias else None
    alpha = 0.5
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=2)
    if bf16:  # small integers are exact in bf16
        A, B = u.bf16_bits(orc, A), u.bf16_bits(orc, B)
    C = u.cm_store(C0, ldc, fill=12345.0)
    assert _hook(orc, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, bf16) == 0
    want = alpha * (opA.astype(np.float64) @ opB) + beta * C0
    if with_bias:
        want = want + bias[:, None]
    assert np.array_equal(u.cm_load(C, M, N, ldc), want.astype(np.float32))
    assert (C.reshape(N, ldc)[:, M:] == 12345.0).all()


@pytest.mark.parametrize("with_bias", [False, True])
def test_onednn_hook_k_zero(orc, with_bias):
    """K == 0: C = 0 (beta 0, C not read: NaN in, zeros out), C *= beta, or C
    unchanged (beta 1); alpha is not used (NaN); then the bias."""
    M, N, ldc = 4, 3, 6
    bias = u.small_ints(orc, M, 4) if with_bias else None
    add = bias[:, None] if with_bias else 0.0
    C0 = u.small_ints(orc, M * N, 3).reshape(M, N)
    nan = np.full(4, np.nan, np.float32)
    for beta, want in [(0.0, np.zeros((M, N))), (1.0, C0), (-2.0, -2.0 * C0)]:
        C = u.cm_store(np.full((M, N), np.nan, np.float32) if beta == 0.0 else C0, ldc, fill=7.0)
        assert _hook(orc, "N", "N", M, N, 0, float("nan"), nan, M, nan, 1, beta, C, ldc, bias) == 0
        assert np.array_equal(u.cm_load(C, M, N, ldc), (want + add).astype(np.float32)), beta
        assert (C.reshape(N, ldc)[:, M:] == 7.0).all()


def test_onednn_hook_early_exits(orc):
    C = _f([1, 2, 3, 4])
    nan = np.full(4, np.nan, np.float32)
    assert _hook(orc, "N", "N", 0, 2, 2, 1.0, nan, 1, nan, 2, 0.0, C, 1) == 0
    assert _hook(orc, "N", "N", 2, 0, 2, 1.0, nan, 2, nan, 2, 0.0, C, 2) == 0
    assert _hook(orc, "P", "N", 2, 2, 2, 1.0, nan, 2, nan, 2, 0.0, C, 2) == 1
    assert _hook(orc, "N", "p", 2, 2, 2, 1.0, nan, 2, nan, 2, 0.0, C, 2) == 1
    assert C.tolist() == [1, 2, 3, 4]
    # The bf16 hook has no packed check: 'P' reads as not transposed.
    A = u.bf16_bits(orc, _f([1, 2, 3, 4]))
    B = u.bf16_bits(orc, _f([1, 0, 0, 1]))
    assert _hook(orc, "P", "N", 2, 2, 2, 1.0, A, 2, B, 2, 0.0, C, 2, bf16=True) == 0
    assert C.tolist() == [1, 2, 3, 4]


def _overlap_closed_form(opA, opB, C0flat, M, N, ldc, alpha, beta, bias):
    """ldc < M, restated with numpy slices: the row-major rows C^T[r] (from
    the rows of C as they were on entry) written back at stride ldc in row
    order, then bias added column by column in order."""
    flat = C0flat.astype(np.float64).copy()
    G = np.stack([flat[r * ldc: r * ldc + M] for r in range(N)])
    R = alpha * (opB.T.astype(np.float64) @ opA.T)
    if beta != 0.0:  # beta == 0: C unread, and alpha * 0 keeps its sign
        R = R + beta * G
    for r in range(N):
        flat[r * ldc: r * ldc + M] = R[r]
    if bias is not None:
        for j in range(N):
            flat[j * ldc: j * ldc + M] += bias
    return flat.astype(np.float32)


@pytest.mark.parametrize("beta,with_bias", [(0.0, False), (0.5, True), (1.0, False)])
def test_onednn_hook_overlapping_columns(orc, beta, with_bias):
    M, N, K, ldc = 7, 5, 4, 3
    opA = u.small_ints(orc, M * K, 1).reshape(M, K)
    opB = u.small_ints(orc, K * N, 2).reshape(K, N)
    total = (N - 1) * ldc + M
    C0 = u.small_ints(orc, total, 3)
    bias = u.small_ints(orc, M, 4) if with_bias else None
    A, lda, B, ldb = u.hook_operands(opA, opB, "N", "T")
    C = C0.copy()
    assert _hook(orc, "N", "T", M, N, K, 1.0, A, lda, B, ldb, beta, C, ldc, bias) == 0
    assert np.array_equal(C, _overlap_closed_form(opA, opB, C0, M, N, ldc, 1.0, beta, bias))


def test_onednn_hook_overlap_k_zero(orc):
    """K == 0 with ldc < M: scaling and bias apply once per covering column."""
    M, N, ldc = 5, 4, 2
    total = (N - 1) * ldc + M
    C0 = u.small_ints(orc, total, 3)
    bias = u.small_ints(orc, M, 4)
    C = C0.copy()
    nan = np.full(2, np.nan, np.float32)
    assert _hook(orc, "N", "N", M, N, 0, 1.0, nan, M, nan, 1, -2.0, C, ldc, bias) == 0
    want = C0.astype(np.float64)
    for j in range(N):
        want[j * ldc: j * ldc + M] *= -2.0
    for j in range(N):
        want[j * ldc: j * ldc + M] += bias
    assert np.array_equal(C, want.astype(np.float32))


def test_onednn_hook_random_tolerance(orc):
    """Random inputs: the fp64 error bound, every transpose combination."""
    M, N, K = 9, 13, 37
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    bias = u.uniform(orc, M, 4)
    for ta, tb in HOOK_T:
        A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=1)
        C = u.cm_store(C0, M)
        assert _hook(orc, ta, tb, M, N, K, 1.5, A, lda, B, ldb, 0.25, C, M, bias) == 0
        want, scale = u.exact(opA, opB, 1.5, 0.25, C0)
        u.assert_fp32_close(u.cm_load(C, M, N, M), want + bias[:, None], scale + np.abs(bias)[:, None], K + 1,
                            f"hook {ta}{tb}")


def test_onednn_hook_checks_catch_mistakes(orc):
    """Plausible mistakes in a hook implementation change the exact integer
    result: a 'T' operand read as not transposed (square A, so the call is
    still well formed), the bias added along N instead of M, beta dropped."""
    M, N, ldc = 5, 7, 5
    sq = u.small_ints(orc, M * M, 5).reshape(M, M)
    opB = u.small_ints(orc, M * N, 6).reshape(M, N)
    C0 = u.small_ints(orc, M * N, 3).reshape(M, N)
    bias = u.small_ints(orc, M, 4)
    A, lda, B, ldb = u.hook_operands(sq, opB, "T", "N")
    right, wrong = u.cm_store(C0, ldc), u.cm_store(C0, ldc)
    _hook(orc, "T", "N", M, N, M, 1.0, A, lda, B, ldb, 1.0, right, ldc, bias)
    _hook(orc, "N", "N", M, N, M, 1.0, A, lda, B, ldb, 1.0, wrong, ldc, bias)
    want = sq.astype(np.float64) @ opB + C0 + bias[:, None]
    assert np.array_equal(u.cm_load(right, M, N, ldc), want.astype(np.float32))
    assert not np.array_equal(right, wrong)
    bias_n = np.resize(bias, N)
    assert not np.array_equal(want, sq.astype(np.float64) @ opB + C0 + bias_n[None, :])
    assert not np.array_equal(want, sq.astype(np.float64) @ opB + bias[:, None])


# ---------------------------------------------------------------- the checks catch mistakes
def test_planted_mistakes_are_caught(orc):
    """Plant plausible mistakes in the oracle's output (on the CPU) and show
    the fp32 tolerance used by the GPU tests rejects every one."""
    M, N, K = 7, 64, 64
    A = u.normal(orc, M * K, 1, 0, 0.02).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(A, B, 1.0, 1.0, C0)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    wrong = {
        "dropped beta": A64 @ B64,
        "dropped last k": A64[:, :-1] @ B64[:-1, :] + C0,
        "transposed B": A64 @ B64.T + C0,
        "wrong sign": -(A64 @ B64) + C0,
        "row shift": np.roll(A64 @ B64, 1, axis=0) + C0,
    }
    for name, bad in wrong.items():
        with pytest.raises(AssertionError):
            u.assert_fp32_close(bad.astype(np.float32), want, scale, K, name)


# ---------------------------------------------------------------- committed fixtures
def test_golden_fixtures(orc):
    path = os.path.join(u.GOLDEN, "oracle_golden.npz")
    g = np.load(path, allow_pickle=False)
    for key in sorted(k for k in g.files if k.endswith("_meta")):
        name = key[: -len("_meta")]
        meta = g[key]
        kind = str(g[name + "_kind"])
        M, N, K = (int(x) for x in meta[:3])
        alpha, beta = float(meta[3]), float(meta[4])
        A, B = g[name + "_A"], g[name + "_B"]
        if kind == "s8":
            C = np.empty(M * N, np.int32)
            orc.orc_gemm_s8s8s32(M, N, K, u.ptr(A), K, u.ptr(B), K, u.ptr(C), N)
            assert np.array_equal(C, g[name + "_C"]), name
            continue
        C = g[name + "_C0"].copy()
        if kind == "naive":
            orc.orc_gemm_naive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N)
        elif kind == "adaptive":
            orc.orc_adaptive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N, 5 if M == 5 else 6,
                                 65536, 1)
        else:
            assert orc.orc_gemm_f32_smallm(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N, 2) == 0
        assert np.array_equal(C.view(np.uint32), g[name + "_C"].view(np.uint32)), name
