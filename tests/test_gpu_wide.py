"""The last-resort kernel (dnnopt_wide): shapes whose operand spans exceed
the other kernels' 32-bit buffer offsets.

* Forced (tunable WIDE = 1) on small ragged shapes, for every data type and
  layout the entry points take: fp32 with both transposes, padded strides,
  beta and the oneDNN hook's bias; bf16 storage (also transposed A and B) and
  fp32 rounded to bf16 against fp64 at the usual bound; int8 bit-exact (int32
  C, the per-column scale, the fp32-API dynamic dequantization against the
  oracle).  Repeated calls are bit-identical.
* Genuinely huge operands reach it through the planners by themselves (fp32
  with B stored N x K and 70 M-element rows, bf16 with 20 M-element rows of
  A, int8 with 716 M-byte rows), checked against closed forms: A(i, k) = i + 1
  (int8: 1) and B(k, j) = (j + 1) (-1)^k with K odd give C = (i + 1)(j + 1)
  (int8: j + 1) exactly, whatever the summation order, since every partial
  sum of consecutive k is an exact small integer.
* The scalar reference kernel (GemmAlgo::kNaive) with more rows than one
  launch's grid covers (M > 262140), bit-exact against the oracle.
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


F32_CASES = [(5, 70, 33), (70, 130, 1000), (1, 1, 1), (33, 65, 7), (9, 200, 129)]


@pytest.mark.parametrize("M,N,K", F32_CASES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_wide_fp32(lib, orc, dev, M, N, K, ta, tb):
    opA = u.normal(orc, M * K, 1, 0, 0.5).reshape(M, K)
    opB = u.normal(orc, K * N, 2, 0, 0.5).reshape(K, N)
    A = np.ascontiguousarray(opA.T) if ta else opA
    B = np.ascontiguousarray(opB.T) if tb else opB
    pa, pb = 3, 5
    A = np.pad(A, ((0, 0), (0, pa)), constant_values=np.nan)
    B = np.pad(B, ((0, 0), (0, pb)), constant_values=np.nan)
    lda, ldb, ldc = A.shape[1], B.shape[1], N + 2
    C0 = u.uniform(orc, M * ldc, 3).reshape(M, ldc)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    with lib.tunables(WIDE=1):
        assert lib.plan_sgemm(M, N, K, transA=ta, transB=tb)["name"] == "dnnopt_wide"
        for beta in (0.0, 0.5):
            start = C0 if beta else np.where(np.arange(ldc) < N, np.nan, C0)
            outs = []
            for rep in range(2):
                dC = dev_copy(start, dev)
                lib.sgemm(M, N, K, 1.25, dA, lda, dB, ldb, beta, dC, ldc, transA=ta, transB=tb, stream=stream())
                outs.append(host(dC))
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "not repeatable"
            got = outs[0]
            assert np.array_equal(got[:, N:].view(np.uint32), start[:, N:].view(np.uint32)), "padding written"
            want, scale = u.exact(opA, opB, 1.25, beta, C0[:, :N] if beta else None)
            u.assert_fp32_close(got[:, :N], want, scale, K, f"wide fp32 {M}x{N}x{K} ta={ta} tb={tb} beta={beta}")


@pytest.mark.parametrize("M,N,K", [(7, 130, 65), (70, 9, 300)])
@pytest.mark.parametrize("ta,tb", [("N", "N"), ("T", "N"), ("N", "T"), ("T", "T")])
def test_wide_hook_bias(lib, orc, dev, M, N, K, ta, tb):
    """The oneDNN hook (column-major, bias as its own rounding) on the
    last-resort kernel."""
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    A, lda, B, ldb = u.hook_operands(opA, opB, ta, tb, pad=2)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    bias = u.uniform(orc, M, 4)
    with lib.tunables(WIDE=1):
        for beta, ldc in ((0.0, M), (1.0, M + 3)):
            Cbuf = u.cm_store(C0 if beta else np.full_like(C0, np.nan), ldc, fill=-777.0)
            dC = dev_copy(Cbuf, dev)
            lib.ext_sgemm(ta, tb, M, N, K, 1.5, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, beta, dC, ldc,
                          bias=dev_copy(bias, dev), stream=stream())
            got = host(dC)
            want, scale = u.exact(opA, opB, 1.5, beta, C0 if beta else None)
            want, scale = want + bias[:, None], scale + np.abs(bias)[:, None]
            u.assert_fp32_close(u.cm_load(got, M, N, ldc), want, scale, K + 1, f"wide hook {ta}{tb} beta={beta}")
            assert (got.reshape(N, ldc)[:, M:] == -777.0).all(), "padding rows of C written"


@pytest.mark.parametrize("M,N,K", [(5, 70, 33), (70, 130, 257), (130, 3, 64)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_wide_bf16_storage(lib, orc, dev, M, N, K, ta, tb):
    opA = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    opB = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02)).reshape(K, N)
    A = np.ascontiguousarray(opA.T) if ta else opA
    B = np.ascontiguousarray(opB.T) if tb else opB
    lda, ldb = A.shape[1], B.shape[1]
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(u.bf16_value(opA), u.bf16_value(opB), 0.5, 1.0, C0)
    with lib.tunables(WIDE=1):
        assert lib.plan_bf16_ex(M, N, K, transA=ta, transB=tb)["name"] == "dnnopt_wide"
        dC = dev_copy(C0, dev)
        lib.gemm_bf16_ex(M, N, K, 0.5, dev_copy(A.view(np.int16), dev), lda, dev_copy(B.view(np.int16), dev), ldb,
                         1.0, dC, N, transA=ta, transB=tb, stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"wide bf16 {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("M,N,K", [(3, 70, 33), (70, 130, 257)])
def test_wide_fp32_rounded_to_bf16(lib, orc, dev, M, N, K):
    A = u.normal(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    want, scale = u.exact(u.bf16_value(u.bf16_bits(orc, A)), u.bf16_value(u.bf16_bits(orc, B)), 1.0, 0.0)
    with lib.tunables(WIDE=1):
        assert lib.plan_bf16(M, N, K, fp32_inputs=1)["name"] == "dnnopt_wide"
        dC = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, N, stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"wide fp32->bf16 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 70, 33), (70, 130, 1001), (9, 4, 4096)])
def test_wide_int8(lib, orc, dev, M, N, K):
    A, B = u.ints8(orc, M * K, 1).reshape(M, K), u.ints8(orc, N * K, 2).reshape(N, K)
    acc = A.astype(np.int64) @ B.astype(np.int64).T
    s = u.uniform(orc, N, 4, 0.001, 0.01)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    with lib.tunables(WIDE=1):
        assert lib.plan_s8(M, N, K)["name"] == "dnnopt_wide"
        dC = torch.full((M, N), -7, dtype=torch.int32, device=dev)
        lib.gemm_s8s8s32(M, N, K, dA, K, dB, K, dC, N, stream=stream())
        assert np.array_equal(host(dC).astype(np.int64), acc)
        dF = torch.zeros((M, N), dtype=torch.float32, device=dev)
        lib.gemm_s8s8f32_colscale(M, N, K, dA, K, dB, K, dev_copy(s, dev), dF, N, stream=stream())
        assert np.array_equal(host(dF), acc.astype(np.float32) * s[None, :])


@pytest.mark.parametrize("M,N,K", [(9, 70, 33), (70, 130, 1001)])
def test_wide_int8_dynamic_quantization(lib, orc, dev, M, N, K):
    """The fp32-API gemm_int8 above M = 8 with its quantization pass (Q8B =
    0): the int8 GEMM and its dequantizing epilogue on the last-resort
    kernel, bit-exact against the oracle."""
    A, B, C0 = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2), u.uniform(orc, M * N, 3)
    with lib.tunables(WIDE=1, Q8B=0):
        for beta in (0.0, 0.5):
            Co = C0.copy()
            orc.orc_gemm_int8(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(Co), N)
            dC = dev_copy(C0, dev)
            lib.gemm_int8_f32(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, beta, dC, N,
                              stream=stream())
            assert np.array_equal(host(dC).view(np.uint32), Co.view(np.uint32)), beta


def test_naive_rows_beyond_one_launch(lib, orc, dev):
    """GemmAlgo::kNaive with more rows than one launch covers (65535 x 4)."""
    M, N, K = 262144 + 5, 3, 4
    A = u.normal(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want = C0.copy()
    orc.orc_gemm_naive_f32(M, N, K, 0.75, u.ptr(A), K, u.ptr(B), N, 0.5, u.ptr(want), N)
    dC = dev_copy(C0, dev)
    lib.sgemm_naive(M, N, K, 0.75, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.5, dC, N, stream=stream())
    assert np.array_equal(host(dC).view(np.uint32), want.view(np.uint32))


def _signs(K, dtype):
    s = torch.ones(K, dtype=dtype, device="cuda:0")
    s[1::2] = -1
    return s


def test_wide_huge_fp32_b_rows(lib, dev):
    """B stored N x K with rows of 70 M floats (280 MB): no tile or row-dot
    kernel can address a tile of it, so the planner picks the last-resort
    kernel."""
    M, N, K = 2, 3, 70_000_001
    p = lib.plan_sgemm(M, N, K, transB=1)
    assert p["name"] == "dnnopt_wide", p
    A = torch.arange(1, M + 1, dtype=torch.float32, device=dev)[:, None].expand(M, K).contiguous()
    B = (torch.arange(1, N + 1, dtype=torch.float32, device=dev)[:, None] * _signs(K, torch.float32)[None, :])
    B = B.contiguous()
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    lib.sgemm(M, N, K, 1.0, A, K, B, K, 0.0, C, N, transB=1, stream=stream())
    want = np.outer(np.arange(1, M + 1), np.arange(1, N + 1)).astype(np.float32)
    assert np.array_equal(host(C), want)
    del A, B
    torch.cuda.empty_cache()


def test_wide_huge_bf16_a_rows(lib, dev):
    """bf16 storage with rows of A of 20 M elements (40 MB each, 2.56 GB per
    64-row tile)."""
    M, N, K = 64, 64, 20_000_001
    p = lib.plan_bf16(M, N, K)
    assert p["name"] == "dnnopt_wide", p
    A = torch.arange(1, M + 1, dtype=torch.float32, device=dev)[:, None].expand(M, K).to(torch.bfloat16).contiguous()
    B = (_signs(K, torch.bfloat16)[:, None] * torch.arange(1, N + 1, device=dev).to(torch.bfloat16)[None, :])
    B = B.contiguous()
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    lib.gemm_bf16(M, N, K, 1.0, A.view(torch.int16), K, B.view(torch.int16), N, 0.0, C, N, stream=stream())
    want = np.outer(np.arange(1, M + 1), np.arange(1, N + 1)).astype(np.float32)
    assert np.array_equal(host(C), want)
    del A, B
    torch.cuda.empty_cache()


def test_wide_huge_int8_rows(lib, dev):
    """int8 with rows of 716 M bytes: beyond the row-dot kernel's and the
    int8 tiles' offsets."""
    M, N, K = 2, 2, 716_000_001
    p = lib.plan_s8(M, N, K)
    assert p["name"] == "dnnopt_wide", p
    A = torch.ones((M, K), dtype=torch.int8, device=dev)
    B = (torch.arange(1, N + 1, dtype=torch.int8, device=dev)[:, None] * _signs(K, torch.int8)[None, :]).contiguous()
    C = torch.full((M, N), -7, dtype=torch.int32, device=dev)
    lib.gemm_s8s8s32(M, N, K, A, K, B, K, C, N, stream=stream())
    want = np.tile(np.arange(1, N + 1, dtype=np.int32), (M, 1))
    assert np.array_equal(host(C), want)
    del A, B
    torch.cuda.empty_cache()
