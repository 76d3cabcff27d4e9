"""Seeded random shapes over every entry point and route (fp32 with both
operand layouts, bf16 storage, int8, fp32-API int8): padded strides, C blocks
inside wider matrices, assorted alpha / beta.  Each case is checked against
fp64 (fp32 / bf16, the (2K+4)u tolerance), exact int64 products (int8) or a
numpy restatement of the per-tensor quantization (fp32-API int8)."""

import numpy as np
import pytest

import _util as u

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _cases(seed=20261208, count=120):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        kind = str(rng.choice(["f32", "bf16", "s8", "i8f"]))
        M = int(rng.choice([rng.integers(1, 9), rng.integers(9, 65), rng.integers(65, 700), rng.integers(700, 20000)]))
        N = int(rng.choice([rng.integers(1, 70), rng.integers(70, 3000), rng.integers(3000, 40000)]))
        K = int(rng.choice([rng.integers(1, 70), rng.integers(70, 2000), rng.integers(2000, 20000)]))
        if M * N * K > 2e8 or M * K > 4e7 or N * K > 4e7:
            continue
        ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        pads = tuple(int(x) for x in rng.integers(0, 5, 3))
        alpha, beta = float(rng.choice([1.0, -0.5])), float(rng.choice([0.0, 1.0, 0.25]))
        out.append((len(out), kind, M, N, K, ta, tb, pads, alpha, beta))
    return out


def _bf16(x):
    b = x.view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}")
def test_random_shape(lib, dev, case):
    i, kind, M, N, K, ta, tb, (pa, pb, pc), alpha, beta = case
    rng = np.random.default_rng(1000 + i)
    s = torch.cuda.current_stream().cuda_stream

    def dc(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    ldc = N + pc
    C0 = rng.standard_normal((M, ldc)).astype(np.float32)
    if kind in ("f32", "bf16"):
        lda, ldb = (M if ta else K) + pa, (K if tb else N) + pb
        As = rng.standard_normal((K if ta else M, lda)).astype(np.float32)
        Bs = (rng.standard_normal((N if tb else K, ldb)) * 0.05).astype(np.float32)
        dC = dc(C0)
        if kind == "bf16":
            Ab, Bb = _bf16(As), _bf16(Bs)
            As, Bs = u.bf16_value(Ab), u.bf16_value(Bb)
            lib.gemm_bf16_ex(M, N, K, alpha, dc(Ab.view(np.int16)), lda, dc(Bb.view(np.int16)), ldb, beta, dC, ldc,
                             transA=ta, transB=tb, stream=s)
        else:
            lib.sgemm(M, N, K, alpha, dc(As), lda, dc(Bs), ldb, beta, dC, ldc, transA=ta, transB=tb, stream=s)
        got = dC.cpu().numpy()
        Amk = np.ascontiguousarray(As[:, :M].T if ta else As[:, :K])
        Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
        want, scale = u.exact(Amk, Bkn, alpha, beta, C0[:, :N])
        u.assert_fp32_close(got[:, :N], want, scale, K, f"{kind} case {i}")
    elif kind == "s8":
        lda, ldb = K + pa, K + pb
        A = rng.integers(-128, 128, (M, lda)).astype(np.int8)
        B = rng.integers(-128, 128, (N, ldb)).astype(np.int8)
        dC = torch.full((M, ldc), 7, dtype=torch.int32, device=dev)
        lib.gemm_s8s8s32(M, N, K, dc(A), lda, dc(B), ldb, dC, ldc, stream=s)
        got = dC.cpu().numpy()
        want = A[:, :K].astype(np.int64) @ B[:, :K].astype(np.int64).T
        assert np.array_equal(got[:, :N].astype(np.int64), want), f"s8 case {i}"
        assert (got[:, N:] == 7).all()
        return
    else:
        lda, ldb = K + pa, N + pb
        A = rng.standard_normal((M, lda)).astype(np.float32)
        B = rng.standard_normal((K, ldb)).astype(np.float32)
        dC = dc(C0)
        lib.gemm_int8_f32(M, N, K, alpha, dc(A), lda, dc(B), ldb, beta, dC, ldc, stream=s)
        got = dC.cpu().numpy()
        # scale_X = max|X| / 127 (1 if zero); M <= 8 (the reference's small-M
        # route): q = clamp(rint(x / s)), else q = clamp(rint(x * (1 / s)))
        sa = np.float32(np.abs(A[:, :K]).max()) / np.float32(127)
        sb = np.float32(np.abs(B[:, :N]).max()) / np.float32(127)
        sa, sb = (sa if sa != 0 else np.float32(1)), (sb if sb != 0 else np.float32(1))
        if M <= 8:
            qa = np.clip(np.rint(A[:, :K] / sa), -128, 127).astype(np.int64)
            qb = np.clip(np.rint(B[:, :N] / sb), -128, 127).astype(np.int64)
        else:
            qa = np.clip(np.rint(A[:, :K] * (np.float32(1) / sa)), -128, 127).astype(np.int64)
            qb = np.clip(np.rint(B[:, :N] * (np.float32(1) / sb)), -128, 127).astype(np.int64)
        acc = (qa @ qb).astype(np.float32)
        dq = np.float32(np.float32(sa * sb) * np.float32(alpha))
        r = dq * acc
        if beta == 0.0:
            want = r + np.float32(0) if 1 < M <= 8 else r  # M 2..8 store 0 + t acc
        elif M == 1:  # fma(beta, C, t acc): one rounding of the exact sum
            want = (np.float64(beta) * C0[:, :N].astype(np.float64) + r.astype(np.float64)).astype(np.float32)
        elif M <= 8:  # beta C, then the rounded sum
            want = (C0[:, :N] * np.float32(beta)) + r
        else:  # fma(dq, acc, beta * C): one rounding of the exact sum
            want = (np.float64(dq) * acc.astype(np.float64) + (np.float32(beta) * C0[:, :N]).astype(np.float64))
            want = want.astype(np.float32)
        assert np.array_equal(got[:, :N].view(np.uint32), want.view(np.uint32)), f"i8f case {i}"
    assert np.array_equal(got[:, N:], C0[:, N:]), f"case {i} wrote outside the C block"


def _cblas_cases(seed=20261209, count=32):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        M = int(rng.choice([rng.integers(1, 9), rng.integers(9, 300), rng.integers(300, 3000)]))
        N = int(rng.choice([rng.integers(1, 70), rng.integers(70, 3000)]))
        K = int(rng.choice([rng.integers(1, 70), rng.integers(70, 3000)]))
        if M * N * K > 1e8:
            continue
        order = int(rng.choice([101, 102]))
        ta, tb = int(rng.choice([111, 112])), int(rng.choice([111, 112]))
        pads = tuple(int(x) for x in rng.integers(0, 4, 3))
        out.append((len(out), order, ta, tb, M, N, K, pads, float(rng.choice([1.0, 0.5])), float(rng.choice([0.0, 1.0, -0.5]))))
    return out


@pytest.mark.parametrize("case", _cblas_cases(), ids=lambda c: f"{c[0]}-{c[1]}{c[2]}{c[3]}-{c[4]}x{c[5]}x{c[6]}")
def test_random_cblas_host_arrays(lib, case):
    """cblas_sgemm on host arrays (staged through the library's device
    buffers): both orders, both transposes, padded leading dimensions."""
    i, order, ta, tb, M, N, K, (pa, pb, pc), alpha, beta = case
    rng = np.random.default_rng(2000 + i)
    # op(A) is M x K, op(B) is K x N; stored row-major (order 101) as given or
    # column-major (102), i.e. the transposed array row-major.
    a_rows, a_cols = (M, K) if ta == 111 else (K, M)
    b_rows, b_cols = (K, N) if tb == 111 else (N, K)
    c_rows, c_cols = M, N
    if order == 102:
        a_rows, a_cols, b_rows, b_cols, c_rows, c_cols = a_cols, a_rows, b_cols, b_rows, c_cols, c_rows
    lda, ldb, ldc = a_cols + pa, b_cols + pb, c_cols + pc
    A = rng.standard_normal((a_rows, lda)).astype(np.float32)
    B = rng.standard_normal((b_rows, ldb)).astype(np.float32)
    C0 = rng.standard_normal((c_rows, ldc)).astype(np.float32)
    C = C0.copy()
    lib.cblas_sgemm(order, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc)
    Am, Bm, Cm, Cg = A[:, :a_cols], B[:, :b_cols], C0[:, :c_cols], C[:, :c_cols]
    if order == 102:  # the stored arrays are the transposes of the column-major matrices
        Am, Bm, Cm, Cg = Am.T, Bm.T, Cm.T, Cg.T
    opA = Am if ta == 111 else Am.T
    opB = Bm if tb == 111 else Bm.T
    want, scale = u.exact(np.ascontiguousarray(opA), np.ascontiguousarray(opB), alpha, beta, np.ascontiguousarray(Cm))
    u.assert_fp32_close(np.ascontiguousarray(Cg), want, scale, K, f"cblas case {i}")
    assert np.array_equal(C[:, c_cols:], C0[:, c_cols:]), f"cblas case {i} wrote outside the C block"


def _hook_cases(seed=20261210, count=32):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        M = int(rng.choice([rng.integers(1, 70), rng.integers(70, 3000), rng.integers(3000, 12000)]))
        N = int(rng.choice([rng.integers(1, 9), rng.integers(9, 300), rng.integers(300, 3000)]))
        K = int(rng.choice([rng.integers(1, 70), rng.integers(70, 2500)]))
        if M * N * K > 1e8:
            continue
        ta, tb = str(rng.choice(["N", "T"])), str(rng.choice(["N", "T"]))
        bf16 = bool(rng.integers(0, 2))
        out.append((len(out), M, N, K, ta, tb, int(rng.integers(0, 4)), bf16, float(rng.choice([0.0, 1.0])),
                    int(rng.integers(0, 4)), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _hook_cases(), ids=lambda c: f"{c[0]}-{c[4]}{c[5]}-{c[1]}x{c[2]}x{c[3]}")
def test_random_onednn_hook(lib, dev, case):
    """The column-major oneDNN hook on device pointers: random shapes, both
    transposes, fp32 (with or without bias) and bf16, padded C."""
    i, M, N, K, ta, tb, pad, bf16, beta, dldc, with_bias = case
    rng = np.random.default_rng(3000 + i)
    opA = rng.standard_normal((M, K)).astype(np.float32)
    opB = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    if bf16:
        opA, opB = u.bf16_value(_bf16(opA)), u.bf16_value(_bf16(opB))
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=pad)
    if bf16:
        A, B = _bf16(np.ascontiguousarray(A, np.float32)).view(np.int16), _bf16(np.ascontiguousarray(B, np.float32)).view(np.int16)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(M).astype(np.float32) if with_bias and not bf16 else None
    ldc = M + dldc
    Cbuf = u.cm_store(C0 if beta else np.full_like(C0, np.nan), ldc, fill=-777.0)
    s = torch.cuda.current_stream().cuda_stream
    dC = torch.from_numpy(Cbuf).to(dev)
    dA, dB = torch.from_numpy(np.ascontiguousarray(A)).to(dev), torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    if bf16:
        lib.ext_gemm_bf16bf16f32(ta, tb, M, N, K, 1.5, dA, lda, dB, ldb, beta, dC, ldc, stream=s)
    else:
        lib.ext_sgemm(ta, tb, M, N, K, 1.5, dA, lda, dB, ldb, beta, dC, ldc,
                      bias=None if bias is None else torch.from_numpy(bias).to(dev), stream=s)
    got = dC.cpu().numpy()
    want, scale = u.exact(opA, opB, 1.5, beta, C0 if beta else None)
    if bias is not None:
        want, scale = want + bias[:, None], scale + np.abs(bias)[:, None]
    u.assert_fp32_close(u.cm_load(got, M, N, ldc), want, scale, K + 1, f"hook case {i}")
    assert (got.reshape(N, ldc)[:, M:] == -777.0).all(), f"hook case {i}: padding rows of C written"
