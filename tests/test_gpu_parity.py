"""Parity of the gfx950 kernels with the CPU oracle, through the C-ABI.

Inputs come from the seeded SplitMix64 generator (tests/_util.py); device
memory is plain torch tensors.  Tolerances are those stated in _util.py:
fp32/bf16 element-wise (2K+4) * 2^-24 * (|alpha| |A||B| + |beta C0|) against
the fp64 product (bf16: of the bf16-rounded operands), int8 bit-exact.
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


# ---------------------------------------------------------------- fp32 skinny (M <= 8)
SKINNY = [(M, N, K) for M in (1, 2, 3, 4, 5, 6, 7, 8) for (N, K) in ((1, 1), (3, 7), (257, 64), (1009, 300))]
SKINNY += [(1, 4096, 4096), (2, 255, 2048), (5, 4099, 129), (8, 513, 1000), (7, 256, 8), (3, 11003, 33)]


@pytest.mark.parametrize("M,N,K", SKINNY)
def test_sgemm_skinny(lib, orc, dev, M, N, K):
    A = u.normal(orc, M * K, 1, 0, 0.02).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    for alpha, beta in ((1.0, 1.0), (1.0, 0.0), (-0.75, 0.5)):
        dC = dev_copy(C0 if beta != 0.0 else np.full_like(C0, np.nan), dev)
        lib.sgemm(M, N, K, alpha, dA, K, dB, N, beta, dC, N, stream=stream())
        got = host(dC)
        want, scale = u.exact(A, B, alpha, beta, C0)
        u.assert_fp32_close(got, want, scale, K, f"skinny {M}x{N}x{K} a={alpha} b={beta}")


# Few rows on 16-row MFMA tiles: 16 x 16 with k over 8 waves for B stored
# N x K from M = 5 (N >= 2048) to M = 16, 16 x 128 with two k-groups above
# that and for B stored K x N (9 <= M <= 32); ragged N / K, padded strides,
# k-splits across workgroups at small N.
FEW = [(5, 2048, 1000, 1, 0), (7, 4099, 2048, 1, 4), (8, 2053, 77, 1, 0), (9, 1009, 300, 1, 2), (13, 300, 4096, 1, 0),
       (16, 4096, 129, 1, 1), (17, 2000, 513, 1, 0), (32, 1001, 64, 1, 3), (9, 1000, 517, 0, 0), (13, 4099, 2048, 0, 4),
       (16, 77, 8192, 0, 1), (48, 1500, 700, 0, 2), (64, 4099, 129, 0, 0), (300, 1001, 257, 0, 1), (512, 515, 64, 0, 0)]


# A stored K x M (transA): 16-row tiles up to M = 16 with B stored N x K, up
# to M = 32 with B stored K x N.
FEW_TA = [(7, 11003, 300, 1, 0), (8, 4096, 129, 1, 3), (13, 2053, 517, 1, 1), (16, 1001, 64, 1, 0),
          (11, 2048, 1000, 0, 2), (16, 4099, 129, 0, 0), (24, 300, 2048, 0, 1), (32, 1001, 77, 0, 4)]


@pytest.mark.parametrize("M,N,K,tb,pad,ta", [f + (0,) for f in FEW] + [f + (1,) for f in FEW_TA])
def test_sgemm_few_rows_tiles(lib, orc, dev, M, N, K, tb, pad, ta):
    """The 16-row tiles (forced where the cost model may pick another tile),
    then the planner's own choice on the same inputs."""
    cfg = 35 if tb and M <= 16 else 36
    with lib.tunables(TILE_CFG=cfg):
        p = lib.plan_sgemm(M, N, K, transA=ta, transB=tb)
    assert p["name"] == "dnnopt_tile_f32" and p["rows"] == 16 and p["cols"] == (16 if tb and M <= 16 else 128), p
    lda, ldb = (M + pad if ta else K + pad), (K + pad if tb else N + pad)
    As = u.normal(orc, (K if ta else M) * lda, 1, 0, 0.02).reshape(K if ta else M, lda)
    Amk = np.ascontiguousarray(As[:, :M].T if ta else As[:, :K])
    Bs = u.normal(orc, (N if tb else K) * ldb, 2, 0, 0.02).reshape(N if tb else K, ldb)
    Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dA, dB = dev_copy(As, dev), dev_copy(Bs, dev)
    for forced in (True, False):
        for alpha, beta in ((1.0, 1.0), (-0.75, 0.0)):
            dC = dev_copy(C0 if beta != 0.0 else np.full_like(C0, np.nan), dev)
            with lib.tunables(TILE_CFG=cfg if forced else 0):
                lib.sgemm(M, N, K, alpha, dA, lda, dB, ldb, beta, dC, N, transA=ta, transB=tb, stream=stream())
            want, scale = u.exact(Amk, Bkn, alpha, beta, C0)
            u.assert_fp32_close(host(dC), want, scale, K,
                                f"few rows {M}x{N}x{K} ta={ta} tb={tb} a={alpha} b={beta} forced={forced}")


@pytest.mark.parametrize("cfg,tb", [(c, tb) for c in (41, 42, 43, 44, 45, 46, 47) for tb in (0, 1)] +
                         [(c, 1) for c in (48, 49, 50)])
def test_sgemm_lds_dma_tiles(lib, orc, dev, cfg, tb):
    """fp32 tiles with both operands copied into LDS by the memory unit,
    forced with 1 to 3 k-splits: ragged M and N, a K tail inside a 32-k
    block, padded strides filled with NaN (they must reach no product of a
    stored output), alpha and beta != 0; and a K of 5 with N off the
    64-column groups.  The 32-column wave tiles (48-50) take B stored N x K
    only; with B stored K x N a forced one is refused (the rule's tile)."""
    if cfg >= 48:
        with lib.tunables(TILE_CFG=cfg):
            assert lib.plan_sgemm(300, 1000, 520, transB=0)["name"] == "dnnopt_tile_f32"
    for M, N, K, pa, pb in ((300, 1000, 520, 3, 5), (17, 1001, 5, 0, 1)):
        lda, ldb = K + pa, (K + pb if tb else N + pb)
        As = np.full((M, lda), np.nan, np.float32)
        As[:, :K] = u.normal(orc, M * K, 1).reshape(M, K)
        rows, cols = (N, K) if tb else (K, N)
        Bs = np.full((rows, ldb), np.nan, np.float32)
        Bs[:, :cols] = u.normal(orc, rows * cols, 2, 0, 0.02).reshape(rows, cols)
        Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
        C0 = u.uniform(orc, M * N, 3).reshape(M, N)
        want, scale = u.exact(As[:, :K], Bkn, 0.5, 0.25, C0)
        dA, dB = dev_copy(As, dev), dev_copy(Bs, dev)
        for splits in (1, 2, 3):
            with lib.tunables(TILE_CFG=cfg, TILE_SPLITS=splits):
                p = lib.plan_sgemm(M, N, K, transB=tb)
                assert p["name"] == "dnnopt_tile_f32_dma", p
                dC = dev_copy(C0, dev)
                lib.sgemm(M, N, K, 0.5, dA, lda, dB, ldb, 0.25, dC, N, transB=tb, stream=stream())
            u.assert_fp32_close(host(dC), want, scale, K, f"f32 dma cfg {cfg} tb={tb} {M}x{N}x{K} splits={splits}")


@pytest.mark.parametrize("M,N,K,tb", [(128, 4096, 4096, 0), (128, 4096, 4096, 1), (1024, 1024, 1024, 1),
                                      (384, 3072, 768, 1), (2048, 2048, 2048, 1)])
def test_sgemm_planned_lds_dma_tiles(lib, orc, dev, M, N, K, tb):
    """Shapes where the planner itself takes the fp32 LDS-DMA tiles (with
    and without k-splits), against the fp64 product; beta != 0."""
    p = lib.plan_sgemm(M, N, K, transB=tb)
    assert p["name"] == "dnnopt_tile_f32_dma", p
    A = u.normal(orc, M * K, 71).reshape(M, K)
    Bs = u.normal(orc, N * K, 72, 0, 0.02).reshape((N, K) if tb else (K, N))
    C0 = u.uniform(orc, M * N, 73).reshape(M, N)
    dC = dev_copy(C0, dev)
    lib.sgemm(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(Bs, dev), K if tb else N, -0.5, dC, N, transB=tb,
              stream=stream())
    want, scale = u.exact(A, np.ascontiguousarray(Bs.T) if tb else Bs, 1.0, -0.5, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"planned f32 dma {M}x{N}x{K} tb={tb}")


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096)] + [(M, N, 2048) for M in (2, 3, 5, 7) for N in (1009, 4099, 11003)])
def test_sgemm_configs_c1_c2(lib, orc, dev, M, N, K):
    """Full benchmark shapes: C1 (beta 0, C pre-filled NaN) and C2 (beta 1),
    against fp64 and against the order-faithful oracle of the reference path."""
    if M == 1:
        A, B = u.uniform(orc, K, 1).reshape(1, K), u.uniform(orc, K * N, 2).reshape(K, N)
        C0, beta = np.full((1, N), np.nan, np.float32), 0.0
    else:
        A, B = u.normal(orc, M * K, 1, 0, 0.02).reshape(M, K), u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
        C0, beta = u.uniform(orc, M * N, 3).reshape(M, N), 1.0
    dC = dev_copy(C0, dev)
    lib.sgemm(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, beta, dC, N, stream=stream())
    got = host(dC)
    want, scale = u.exact(A, B, 1.0, beta, C0 if beta else None)
    u.assert_fp32_close(got, want, scale, K, f"C1/C2 {M}x{N}x{K}")
    Co = C0.copy()
    assert orc.orc_gemm_f32_smallm(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(Co), N, 4) == 0
    d = np.abs(got.astype(np.float64) - Co)
    assert (d <= 2 * u.fp32_tol(K, scale)).all(), "far from the reference-path oracle"


# Wide N with G / T == 1 and a remainder: column tiles of one and of two
# k-splits in one launch, summed by the reduce kernel that follows.
@pytest.mark.parametrize("kind,M,N,K", [("f32", 1, 33000, 512), ("f32", 3, 36988, 512), ("f32", 8, 34994, 300),
                                        ("bf16", 1, 66000, 300), ("bf16", 8, 67999, 300)])
def test_skinny_tiles_of_one_and_two_splits(lib, orc, dev, kind, M, N, K):
    p = lib.plan_sgemm(M, N, K) if kind == "f32" else lib.plan_bf16(M, N, K)
    T = -(-N // (256 if kind == "f32" else 512))
    assert p["name"] == "dnnopt_skinny" and p["grid_x"] > T and p["grid_x"] % T and p["grid_x"] // T == 1, p
    A = u.normal(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    if kind == "bf16":
        A, B = u.bf16_bits(orc, A), u.bf16_bits(orc, B)
        dA, dB, Av, Bv = dev_copy(A.view(np.int16), dev), dev_copy(B.view(np.int16), dev), u.bf16_value(A), u.bf16_value(B)
    else:
        dA, dB, Av, Bv = dev_copy(A, dev), dev_copy(B, dev), A, B
    for alpha, beta in ((1.0, 1.0), (-0.5, 0.0)):
        dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
        if kind == "bf16":
            lib.gemm_bf16(M, N, K, alpha, dA, K, dB, N, beta, dC, N, stream=stream())
        else:
            lib.sgemm(M, N, K, alpha, dA, K, dB, N, beta, dC, N, stream=stream())
        want, scale = u.exact(Av, Bv, alpha, beta, C0 if beta else None)
        u.assert_fp32_close(host(dC), want, scale, K, f"{kind} {M}x{N}x{K} a={alpha} b={beta}")


def test_sgemm_deterministic(lib, orc, dev):
    M, N, K = 7, 4099, 2048
    A, B = u.normal(orc, M * K, 1, 0, 0.02), u.normal(orc, K * N, 2, 0, 0.02)
    dA, dB = dev_copy(A, dev), dev_copy(B, dev)
    outs = []
    for _ in range(3):
        dC = torch.zeros(M * N, dtype=torch.float32, device=dev)
        lib.sgemm(M, N, K, 1.0, dA, K, dB, N, 0.0, dC, N, stream=stream())
        outs.append(host(dC))
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])


def test_sgemm_strided_operands(lib, orc, dev):
    """lda/ldb/ldc larger than the row length, row-major sub-matrices."""
    M, N, K = 5, 300, 200
    lda, ldb, ldc = K + 9, N + 13, N + 7
    A = u.uniform(orc, M * lda, 1).reshape(M, lda)
    B = u.uniform(orc, K * ldb, 2).reshape(K, ldb)
    C0 = u.uniform(orc, M * ldc, 3).reshape(M, ldc)
    for (m, n) in ((M, N), (40, N)):
        AA = u.uniform(orc, m * lda, 1).reshape(m, lda) if m != M else A
        CC = u.uniform(orc, m * ldc, 3).reshape(m, ldc) if m != M else C0
        dC = dev_copy(CC, dev)
        lib.sgemm(m, n, K, 1.0, dev_copy(AA, dev), lda, dev_copy(B, dev), ldb, 1.0, dC, ldc, stream=stream())
        got = host(dC)
        want, scale = u.exact(AA[:, :K], B[:, :n], 1.0, 1.0, CC[:, :n])
        u.assert_fp32_close(got[:, :n], want, scale, K, f"strided m={m}")
        assert np.array_equal(got[:, n:], CC[:, n:]), "wrote outside the C block"


# ---------------------------------------------------------------- fp32 tiles and transposes
TILE = [(9, 13, 17), (16, 16, 16), (65, 17, 300), (128, 128, 128), (127, 127, 127), (256, 256, 256),
        (128, 768, 768), (33, 1, 65), (100, 5, 1), (64, 64, 4096), (300, 70, 63)]


@pytest.mark.parametrize("M,N,K", TILE)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_sgemm_tiles_and_transposes(lib, orc, dev, M, N, K, ta, tb):
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    A = np.ascontiguousarray(opA.T) if ta else opA
    B = np.ascontiguousarray(opB.T) if tb else opB
    dC = dev_copy(C0, dev)
    lib.sgemm(M, N, K, 2.5, dev_copy(A, dev), A.shape[1], dev_copy(B, dev), B.shape[1], -0.3, dC, N,
              transA=ta, transB=tb, stream=stream())
    want, scale = u.exact(opA, opB, 2.5, -0.3, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"tile {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("M,N,K,ta", [(65536, 16, 256, 0), (65536, 64, 256, 0), (64, 64, 262144, 0),
                                      (64, 64, 262144, 1)])
def test_sgemm_configs_c3(lib, orc, dev, M, N, K, ta):
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    B = u.uniform(orc, K * N, 2).reshape(K, N)
    A = np.ascontiguousarray(opA.T) if ta else opA
    dC = dev_copy(np.full((M, N), np.nan, np.float32), dev)
    lib.sgemm(M, N, K, 1.0, dev_copy(A, dev), A.shape[1], dev_copy(B, dev), N, 0.0, dC, N, transA=ta,
              stream=stream())
    want, scale = u.exact(opA, B)
    u.assert_fp32_close(host(dC), want, scale, K, f"C3 {M}x{N}x{K} ta={ta}")


def test_sgemm_tall_large_c_stride(lib, orc, dev):
    """65536 x 64 x 256 with ldc = 16384: C spans 4 GiB, beyond the tall
    kernel's 32-bit C offsets, so the planner takes the tiles.  C's padding
    holds NaN and must stay untouched."""
    M, N, K, ldc = 65536, 64, 256, 16384
    assert lib.plan_sgemm_ex(M, N, K, K, N, ldc)["name"] != "dnnopt_tall_f32"
    A, B = u.uniform(orc, M * K, 1).reshape(M, K), u.uniform(orc, K * N, 2).reshape(K, N)
    dC = torch.full((M, ldc), float("nan"), dtype=torch.float32, device=dev)
    lib.sgemm(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, ldc, stream=stream())
    got = host(dC[:, :N].contiguous())
    want, scale = u.exact(A, B)
    u.assert_fp32_close(got, want, scale, K, "65536x64x256 ldc=16384")
    rows = torch.tensor([0, 1, 4095, 32768, M - 1], device=dev)
    pad = host(dC[rows, N:N + 4096].contiguous())
    assert np.isnan(pad).all(), "wrote outside the C block"
    del dC
    torch.cuda.empty_cache()


# B beyond 2 GiB (3.3 GB): every kernel addresses its operands with 32-bit
# offsets from per-workgroup bases, so the planners shorten the k-range per
# workgroup (skinny, MFMA tiles) or keep the row range small (B stored N x K).
# Data comes from the device generator; checked on 96 columns against fp64.
@pytest.mark.parametrize("kind,M,tb", [("f32", 2, 0), ("f32", 12, 0), ("f32", 6, 1), ("f32", 40, 0),
                                       ("bf16", 4, 0), ("bf16", 32, 0)])
def test_operands_beyond_2gib(lib, dev, kind, M, tb):
    N, K = (16384 if kind == "bf16" else 8192), 100000
    g = torch.Generator(device=dev)
    g.manual_seed(1234 + M)
    A = torch.randn(M, K, device=dev, generator=g)
    B = torch.randn(N, K, device=dev, generator=g) if tb else torch.randn(K, N, device=dev, generator=g)
    if kind == "bf16":
        A, B = A.to(torch.bfloat16), B.to(torch.bfloat16)
    assert B.numel() * B.element_size() > 2 ** 31 + 2 ** 30
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    if kind == "bf16":
        lib.gemm_bf16(M, N, K, 1.0, A, K, B, N, 0.0, dC, N, stream=stream())
    else:
        lib.sgemm(M, N, K, 1.0, A, K, B, K if tb else N, 0.0, dC, N, transB=tb, stream=stream())
    cols = torch.randperm(N, generator=torch.Generator().manual_seed(7))[:96].to(dev)
    Bc = (B[cols, :].T if tb else B[:, cols]).double()
    want = (A.double() @ Bc).cpu().numpy()
    scale = (A.double().abs() @ Bc.abs()).cpu().numpy()
    got = host(dC[:, cols].contiguous())
    del A, B, Bc, dC
    torch.cuda.empty_cache()
    u.assert_fp32_close(got, want, scale, K, f"{kind} {M}x{N}x{K} tb={tb}, B beyond 2 GiB")


# k-major outer-product kernel (A stored K x M, B stored K x N, 32 < M, N <= 64,
# K >= 32768, row strides multiples of 4): K not a multiple of 4, ragged M and
# N, padded strides whose padding holds NaN (it may only reach outputs outside
# C), alpha / beta, a padded C whose padding must stay untouched.
# (M, N, K, A row padding, B row padding)
KOUTER = [(64, 64, 262144, 0, 0), (33, 61, 32771, 3, 7), (48, 40, 100003, 0, 4), (64, 33, 40000, 4, 3),
          (61, 64, 65537, 3, 0), (36, 36, 32768, 0, 0)]


@pytest.mark.parametrize("M,N,K,pa,pb", KOUTER)
def test_sgemm_kouter(lib, orc, dev, M, N, K, pa, pb):
    lda, ldb, ldc = M + pa, N + pb, N + 5
    assert lda % 4 == 0 and ldb % 4 == 0
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    A = np.full((K, lda), np.nan, np.float32)
    A[:, :M] = opA.T
    B = np.full((K, ldb), np.nan, np.float32)
    B[:, :N] = opB
    C0 = u.uniform(orc, M * ldc, 3).reshape(M, ldc)
    dC = dev_copy(C0, dev)
    if lda == M and ldb == N:
        p = lib.plan_sgemm(M, N, K, transA=1)
        assert p["name"] == "dnnopt_kouter_f32", p
    lib.sgemm(M, N, K, 1.5, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, -0.5, dC, ldc, transA=1,
              stream=stream())
    got = host(dC)
    want, scale = u.exact(opA, opB, 1.5, -0.5, C0[:, :N])
    u.assert_fp32_close(got[:, :N], want, scale, K, f"kouter {M}x{N}x{K} lda={lda} ldb={ldb}")
    assert np.array_equal(got[:, N:], C0[:, N:]), "wrote outside the C block"


def test_sgemm_kouter_misaligned_falls_back(lib, orc, dev):
    # Operands that do not start on 16-byte boundaries go to the register tiles.
    M = N = 64
    K = 32768
    opA = u.uniform(orc, M * K, 1).reshape(M, K)
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    bufA = dev_copy(np.concatenate([np.zeros(1, np.float32), np.ascontiguousarray(opA.T).ravel()]), dev)
    dB = dev_copy(opB, dev)
    dC = dev_copy(np.zeros((M, N), np.float32), dev)
    lib.sgemm(M, N, K, 1.0, bufA[1:], M, dB, N, 0.0, dC, N, transA=1, stream=stream())
    want, scale = u.exact(opA, opB)
    u.assert_fp32_close(host(dC), want, scale, K, "kouter misaligned A")


# Tall-skinny fp32 with B resident in LDS: every column-tile width, ragged N
# and K (K tails inside a 16-k chunk, N not a multiple of 16), padded strides,
# B stored K x N or N x K, more row tiles than waves and fewer.
# (N <= 16 goes to the register tiles; kept here as ragged tall-skinny cases.)
# (M, N, K, A row padding, B row padding): partial last row tiles, K tails,
# padded rows; the small-M rows and N <= 16 go to the register tiles.
TALL = [(65536, 64, 256, 0, 0), (65536, 16, 256, 1, 0), (65537, 33, 300, 0, 3), (70001, 64, 17, 2, 1),
        (4096, 1, 1024, 0, 0), (100003, 7, 64, 1, 2), (50000, 48, 333, 0, 0), (49999, 17, 5, 3, 0),
        (60000, 60, 250, 1, 1), (70000, 32, 128, 0, 0), (8192, 33, 300, 0, 3), (4097, 17, 5, 3, 0),
        (65536, 13, 130, 1, 2), (50001, 16, 64, 0, 0), (65536, 12, 256, 0, 0), (16384, 64, 256, 0, 0),
        (20001, 40, 300, 1, 0), (16383, 64, 256, 0, 0), (30000, 33, 255, 0, 1),
        # A by LDS-DMA (N <= 16, K = 128 / 192 / 256, rows of A a multiple of 16 bytes)
        (65536, 16, 256, 0, 0), (65537, 13, 128, 4, 1), (70001, 16, 192, 0, 3), (50000, 15, 256, 8, 0),
        (16384, 16, 256, 0, 0), (131072, 14, 128, 0, 0),
        # ... and N <= 12 or K = 64 on the same kernel
        (65536, 1, 256, 0, 0), (65536, 8, 256, 4, 0), (262144, 16, 64, 0, 2), (131075, 5, 128, 0, 0),
        # ... and from 4K rows (one tile per wave or fewer)
        (4096, 16, 256, 0, 0), (8191, 16, 128, 0, 1), (4097, 3, 64, 4, 0),
        # ... and 16 < N <= 64 (K = 128 with N > 32 stays on the register-ring kernel)
        (65536, 64, 192, 0, 2), (65537, 40, 256, 4, 0), (49153, 33, 64, 0, 1), (65536, 48, 128, 0, 0)]


def _routes_tall(M, N, K, lda=None):
    # one 32-row tile for at least 3/4 of the waves of one 8-wave workgroup per CU (256 CUs),
    # or (K >= 256) one 16-row tile for every other wave; N <= 12, and N <= 16 with K < 128,
    # stay on the register tiles; N <= 16 with K a multiple of 64 up to 256 and rows of A a
    # multiple of 16 bytes take the LDS-DMA kernel
    waves = 256 * 8
    rows_ok = -(-M // 32) * 4 >= 3 * waves or (K >= 256 and -(-M // 16) * 2 >= waves)
    lda = K if lda is None else lda
    dma = N <= 64 and K % 64 == 0 and 64 <= K <= 256 and lda % 4 == 0 and not (K == 128 and N > 32)
    if dma and N <= 16:
        return "dnnopt_tall_dma_f32" if M >= 4096 else None
    if not (N > 12 and (N > 16 or K >= 128) and N <= 64 and rows_ok and M >= 4096):
        return None
    return "dnnopt_tall_dma_f32" if dma else "dnnopt_tall_f32"


@pytest.mark.parametrize("M,N,K,pa,pb", TALL)
@pytest.mark.parametrize("tb", [0, 1])
def test_sgemm_tall_skinny(lib, orc, dev, M, N, K, pa, pb, tb):
    p = lib.plan_sgemm_ex(M, N, K, K + pa, (K if tb else N) + pb, N, transB=tb)
    route = _routes_tall(M, N, K, K + pa)
    if route:
        assert p["name"] == route, p
    else:
        assert p["name"] in ("dnnopt_tile_f32", "dnnopt_tile_f32_dma"), p
    lda = K + pa
    opA = np.zeros((M, lda), np.float32)
    opA[:, :K] = u.uniform(orc, M * K, 1).reshape(M, K)
    opA[:, K:] = np.inf  # row padding past K must never reach a product
    opB = u.uniform(orc, K * N, 2).reshape(K, N)
    SB = opB.T if tb else opB
    ldb = SB.shape[1] + pb
    B = np.zeros((SB.shape[0], ldb), np.float32)
    B[:, :SB.shape[1]] = SB
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    for beta in (0.0, 0.75):
        dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
        lib.sgemm(M, N, K, 1.25, dev_copy(opA, dev), lda, dev_copy(B, dev), ldb, beta, dC, N, transB=tb,
                  stream=stream())
        want, scale = u.exact(opA[:, :K], opB, 1.25, beta, C0 if beta else None)
        u.assert_fp32_close(host(dC), want, scale, K, f"tall {M}x{N}x{K} tb={tb} beta={beta}")


@pytest.mark.parametrize("M,N,K", [(65536, 16, 256), (65537, 13, 128), (65536, 16, 192), (16384, 15, 256),
                                   (65536, 64, 256), (65537, 33, 192), (65536, 48, 64), (65536, 32, 128)])
def test_tall_dma_matches_register_ring_kernel(lib, dev, M, N, K):
    """The LDS-DMA tall kernel adds the same products in the same order as
    the register-ring tall kernel (forced by TALL_RT=1): bit-identical C for
    both B layouts, beta 0 and 0.5; A off 16-byte alignment falls back to the
    register-ring kernel (same bits); a column-bias call through the oneDNN
    hook (column-major C^T, the tall product with B^T as A) too."""
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    A = torch.rand(M, K, generator=g).to(dev) * 2 - 1
    B = torch.rand(K, N, generator=g).to(dev) * 2 - 1
    BT = B.t().contiguous()
    C0 = torch.rand(M, N, generator=g).to(dev)
    assert lib.plan_sgemm(M, N, K)["name"] == "dnnopt_tall_dma_f32"
    for tb, Bx, ldb in ((0, B, N), (1, BT, K)):
        for beta in (0.0, 0.5):
            outs = []
            for rt in (0, 1):
                C = C0.clone()
                with lib.tunables(TALL_RT=rt):
                    want_name = "dnnopt_tall_dma_f32" if rt == 0 else "dnnopt_tall_f32"
                    assert lib.plan_sgemm(M, N, K, transB=tb)["name"] == want_name
                    lib.sgemm(M, N, K, 1.25, A, K, Bx, ldb, beta, C, N, transB=tb, stream=stream())
                outs.append(C)
            torch.cuda.synchronize()
            assert torch.equal(outs[0], outs[1]), (M, N, K, tb, beta)
    exact = (A.double() @ B.double()).cpu().numpy() * 1.25
    scale = (A.double().abs() @ B.double().abs()).cpu().numpy() * 1.25
    C = torch.empty(M, N, device=dev)
    lib.sgemm(M, N, K, 1.25, A, K, B, N, 0.0, C, N, stream=stream())
    u.assert_fp32_close(host(C), exact, scale, K, f"tall dma {M}x{N}x{K}")
    # A starting 4 bytes past a 16-byte boundary (rows of K floats stay 16-byte multiples)
    buf = torch.empty(M * K + 4, device=dev)
    Am = buf[1:1 + M * K].view(M, K)
    Am.copy_(A)
    C = torch.empty(M, N, device=dev)
    lib.sgemm(M, N, K, 1.25, Am, K, B, N, 0.0, C, N, stream=stream())
    ref = torch.empty(M, N, device=dev)
    with lib.tunables(TALL_RT=1):
        lib.sgemm(M, N, K, 1.25, A, K, B, N, 0.0, ref, N, stream=stream())
    torch.cuda.synchronize()
    assert torch.equal(C, ref), (M, N, K, "misaligned A")
    # column-major hook: C^T (N x M, ldc = N) = B^T A^T with a bias per column of the row-major C
    bias = torch.rand(N, generator=g).to(dev)
    outs = []
    for rt in (0, 1):
        Ct = C0.clone()
        with lib.tunables(TALL_RT=rt):
            lib.ext_sgemm("N", "N", N, M, K, 1.0, B, N, A, K, 0.5, Ct, N, bias=bias, stream=stream())
        outs.append(Ct)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), (M, N, K, "hook bias")


def test_sgemm_naive_bitwise(lib, orc, dev):
    """The kNaive kernel reproduces the reference's scalar loop bit for bit
    (the oracle's naive loop is itself pinned to the reference build)."""
    for M, N, K, alpha, beta in [(7, 13, 5, 1.0, 0.0), (3, 3, 1000, 2.5, -0.3), (33, 70, 129, 1.0, 0.5)]:
        A, B, C0 = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2), u.uniform(orc, M * N, 3)
        Co = C0.copy()
        orc.orc_gemm_naive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(Co), N)
        dC = dev_copy(C0, dev)
        lib.sgemm_naive(M, N, K, alpha, dev_copy(A, dev), K, dev_copy(B, dev), N, beta, dC, N, stream=stream())
        assert np.array_equal(host(dC).view(np.uint32), Co.view(np.uint32))


# ---------------------------------------------------------------- bf16
BF16 = [(1, 11008, 4096), (4, 11008, 4096), (32, 11008, 4096), (256, 11008, 4096), (3, 1001, 130), (8, 5, 7),
        (9, 33, 250), (64, 100, 129), (1, 1, 1)]


@pytest.mark.parametrize("M,N,K", BF16)
def test_bf16_storage(lib, orc, dev, M, N, K):
    A = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    B = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02)).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dA = dev_copy(A.view(np.int16), dev)
    dB = dev_copy(B.view(np.int16), dev)
    for beta in (0.0, 1.0):
        dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
        lib.gemm_bf16(M, N, K, 1.0, dA, K, dB, N, beta, dC, N, stream=stream())
        want, scale = u.exact(u.bf16_value(A), u.bf16_value(B), 1.0, beta, C0 if beta else None)
        u.assert_fp32_close(host(dC), want, scale, K, f"bf16 {M}x{N}x{K} beta={beta}")


# LDS-staged bf16 tiles: ragged M/N/K (K tails inside a 64-k block), padded
# even strides, k split across workgroups (few tiles), exact tile multiples.
LDS = [(100, 1001, 129, 1, 1), (33, 130, 8192, 0, 0), (17, 4096, 300, 2, 0), (256, 256, 64, 0, 0),
       (129, 127, 1000, 0, 1), (64, 64, 64, 0, 0), (300, 600, 70, 4, 8)]


@pytest.mark.parametrize("M,N,K,pa,pb", LDS)
@pytest.mark.parametrize("mode", ["bf16", "f2b"])
def test_bf16_lds_tiles(lib, orc, dev, M, N, K, pa, pb, mode):
    lda, ldb = K + pa, N + pb
    p = lib.plan_bf16(M, N, K, fp32_inputs=int(mode == "f2b"))
    if (K % 2 == 0 and N % 2 == 0) or mode == "f2b":
        # operands staged through LDS: by the registers (fp32 inputs) or by
        # the memory unit's LDS path (bf16 storage)
        assert p["name"] in ("dnnopt_tile_bf16_lds", "dnnopt_tile_bf16_dma"), p
    A32 = u.normal(orc, M * lda, 1).reshape(M, lda)
    B32 = u.normal(orc, K * ldb, 2, 0, 0.02).reshape(K, ldb)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    A, B = u.bf16_bits(orc, A32), u.bf16_bits(orc, B32)
    want, scale = u.exact(u.bf16_value(A)[:, :K], u.bf16_value(B)[:, :N], 0.5, 1.0, C0)
    dC = dev_copy(C0, dev)
    if mode == "bf16":
        lib.gemm_bf16(M, N, K, 0.5, dev_copy(A.view(np.int16), dev), lda, dev_copy(B.view(np.int16), dev), ldb, 1.0,
                      dC, N, stream=stream())
    else:
        lib.gemm_bf16_f32in(M, N, K, 0.5, dev_copy(A32, dev), lda, dev_copy(B32, dev), ldb, 1.0, dC, N,
                            stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"lds {mode} {M}x{N}x{K}")


# bf16 storage, B stored K x N, 6 <= M <= 8: LDS-staged 32 x 64 tiles when
# both row strides are even, the skinny kernel otherwise; A stored K x M stays
# on the skinny kernel.
@pytest.mark.parametrize("M,N,K,pa,pb,ta", [(6, 1001, 130, 2, 1, 0), (7, 11008, 4096, 0, 0, 0), (8, 4099, 300, 0, 1, 0),
                                            (6, 77, 1000, 4, 3, 0), (7, 300, 129, 0, 0, 0), (8, 515, 64, 0, 1, 1)])
def test_bf16_small_m_kn_tiles(lib, orc, dev, M, N, K, pa, pb, ta):
    lda, ldb = (M if ta else K) + pa, N + pb
    p = lib.plan_bf16_ex(M, N, K, transA=ta)
    tiled = not ta and lda % 2 == 0 and ldb % 2 == 0
    if lda == (M if ta else K) and ldb == N:
        assert p["name"] == ("dnnopt_tile_bf16_lds" if tiled else "dnnopt_skinny"), p
    Amk = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    As = np.zeros((K, lda) if ta else (M, lda), np.uint16)
    if ta:
        As[:, :M] = Amk.T
    else:
        As[:, :K] = Amk
    Bs = u.bf16_bits(orc, u.normal(orc, K * ldb, 2, 0, 0.02)).reshape(K, ldb)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(u.bf16_value(Amk), u.bf16_value(Bs)[:, :N], -0.5, 0.75, C0)
    dC = dev_copy(C0, dev)
    lib.gemm_bf16_ex(M, N, K, -0.5, dev_copy(As.view(np.int16), dev), lda, dev_copy(Bs.view(np.int16), dev), ldb, 0.75,
                     dC, N, transA=ta, stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"bf16 small-M K x N {M}x{N}x{K} ta={ta}")


# bf16 storage, B stored N x K, M <= 32: 16 x 48 / 32 x 48 LDS-staged tiles;
# ragged N (not a multiple of 48), K tails, padded even strides.
@pytest.mark.parametrize("M,N,K,pa,pb", [(5, 1001, 300, 0, 2), (16, 4099, 130, 2, 0), (17, 11008, 4096, 0, 0),
                                         (32, 97, 1000, 4, 4), (24, 48, 64, 0, 0), (9, 50, 520, 2, 2)])
def test_bf16_tb_48_column_tiles(lib, orc, dev, M, N, K, pa, pb):
    """The 48-column tiles (forced where the cost model may pick another),
    then the planner's own choice on the same inputs."""
    lda, ldb = K + pa, K + pb
    cfg = 38 if M <= 16 else 37
    with lib.tunables(TILE_CFG=cfg):
        p = lib.plan_bf16_ex(M, N, K, transB=1)
    assert p["name"] == "dnnopt_tile_bf16_lds" and p["cols"] == 48 and p["rows"] == (16 if M <= 16 else 32), p
    A = u.bf16_bits(orc, u.normal(orc, M * lda, 1)).reshape(M, lda)
    B = u.bf16_bits(orc, u.normal(orc, N * ldb, 2, 0, 0.02)).reshape(N, ldb)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(u.bf16_value(A)[:, :K], np.ascontiguousarray(u.bf16_value(B)[:, :K].T), 0.5, 1.0, C0)
    dA, dB = dev_copy(A.view(np.int16), dev), dev_copy(B.view(np.int16), dev)
    for forced in (True, False):
        dC = dev_copy(C0, dev)
        with lib.tunables(TILE_CFG=cfg if forced else 0):
            lib.gemm_bf16_ex(M, N, K, 0.5, dA, lda, dB, ldb, 1.0, dC, N, transB=1, stream=stream())
        u.assert_fp32_close(host(dC), want, scale, K, f"bf16 TB 48-column tiles {M}x{N}x{K} forced={forced}")


@pytest.mark.parametrize("tb", [0, 1])
def test_bf16_dma_256_row_tiles(lib, orc, dev, tb):
    """bf16 storage with more 128-row tiles than CUs takes 256 x 96 tiles:
    ragged M and N, a K tail inside a 64-k block, padded strides, B stored
    K x N and N x K."""
    M, N, K = 1030, 4100, 200
    lda, ldb = K + 8, (K + 4 if tb else N + 2)
    with lib.tunables(TILE_CFG=33):  # the cost model may pick another tile here
        p = lib.plan_bf16_ex(M, N, K, transB=tb)
    assert p["name"] == "dnnopt_tile_bf16_dma" and p["rows"] == 256, p
    A = u.bf16_bits(orc, u.normal(orc, M * lda, 1)).reshape(M, lda)
    Bs = u.bf16_bits(orc, u.normal(orc, (N if tb else K) * ldb, 2, 0, 0.02)).reshape(N if tb else K, ldb)
    Bkn = Bs[:, :K].T if tb else Bs[:, :N]
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    want, scale = u.exact(u.bf16_value(A)[:, :K], u.bf16_value(np.ascontiguousarray(Bkn)), 0.5, 1.0, C0)
    dA, dB = dev_copy(A.view(np.int16), dev), dev_copy(Bs.view(np.int16), dev)
    for forced in (True, False):
        dC = dev_copy(C0, dev)
        with lib.tunables(TILE_CFG=33 if forced else 0):
            lib.gemm_bf16_ex(M, N, K, 0.5, dA, lda, dB, ldb, 1.0, dC, N, transB=tb, stream=stream())
        u.assert_fp32_close(host(dC), want, scale, K, f"dma 256-row tiles tb={tb} forced={forced}")


def _bf16_storage_sweep_cases():
    """Seeded shapes for bf16 storage above M = 128 (the LDS-DMA tiles, 128-
    and 256-row): ragged M / N / K, even padded strides, both B layouts,
    assorted alpha / beta.  Sizes keep the fp64 reference to about a second."""
    rng = np.random.default_rng(20261202)
    cases = []
    while len(cases) < 12:
        M = int(rng.integers(129, 1101))
        N = int(rng.integers(90, 5001))
        K = int(rng.integers(1, 301))
        if M * N * K > 400_000_000:
            continue
        tb = int(rng.integers(0, 2))
        pa, pb = 2 * int(rng.integers(0, 5)), 2 * int(rng.integers(0, 5))
        alpha = float(rng.choice([1.0, 0.5, -2.0]))
        beta = float(rng.choice([0.0, 1.0, 0.25]))
        cases.append((M, N, K, tb, pa, pb, alpha, beta))
    # two shapes with more 128 x 96 tiles than CUs (the cost model gives them 128 x 128 tiles)
    cases += [(1100, 3000, 96, 0, 2, 0, 1.0, 0.0), (1024, 3100, 130, 1, 0, 4, -2.0, 0.25)]
    return cases


@pytest.mark.parametrize("M,N,K,tb,pa,pb,alpha,beta", _bf16_storage_sweep_cases())
def test_bf16_storage_sweep(lib, orc, dev, M, N, K, tb, pa, pb, alpha, beta):
    lda, ldb = K + pa, (K + pb if tb else N + pb)
    p = lib.plan_bf16_ex(M, N, K, transB=tb)
    # rows of A and B on 4-byte boundaries: the LDS-staged tiles (the cost
    # models pick LDS-DMA or register-ring staging); else the register tiles
    if lda % 2 == 0 and ldb % 2 == 0:
        assert p["name"] in ("dnnopt_tile_bf16_dma", "dnnopt_tile_bf16_lds"), p
    else:
        assert p["name"] == "dnnopt_tile_bf16", p
    A = u.bf16_bits(orc, u.normal(orc, M * lda, 11)).reshape(M, lda)
    rows = N if tb else K
    Bs = u.bf16_bits(orc, u.normal(orc, rows * ldb, 12, 0, 0.02)).reshape(rows, ldb)
    Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
    C0 = u.uniform(orc, M * N, 13).reshape(M, N)
    want, scale = u.exact(u.bf16_value(A)[:, :K], u.bf16_value(Bkn), alpha, beta, C0 if beta else None)
    dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
    lib.gemm_bf16_ex(M, N, K, alpha, dev_copy(A.view(np.int16), dev), lda, dev_copy(Bs.view(np.int16), dev), ldb,
                     beta, dC, N, transB=tb, stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"bf16 sweep {M}x{N}x{K} tb={tb} a={alpha} b={beta}")


@pytest.mark.parametrize("tb", [0, 1])
def test_bf16_dma_128x128_four_wave_tiles(lib, orc, dev, tb):
    """128 x 128 LDS-DMA tiles on 4 waves of 64 x 64: forced with 1 to 4
    k-splits on a ragged shape (M and N off the tile, a K tail inside a 64-k
    block, padded even strides, beta != 0), and as the planner's own choice
    (256 x 4096 x 4096 with 4 k-splits); B stored K x N and N x K."""
    def run(M, N, K, pa, pb, alpha, beta, seed):
        lda, ldb = K + pa, (K + pb if tb else N + pb)
        A = u.bf16_bits(orc, u.normal(orc, M * lda, seed)).reshape(M, lda)
        rows = N if tb else K
        Bs = u.bf16_bits(orc, u.normal(orc, rows * ldb, seed + 1, 0, 0.02)).reshape(rows, ldb)
        Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
        C0 = u.uniform(orc, M * N, seed + 2).reshape(M, N)
        want, scale = u.exact(u.bf16_value(A)[:, :K], u.bf16_value(Bkn), alpha, beta, C0 if beta else None)
        dC = dev_copy(C0 if beta else np.full_like(C0, np.nan), dev)
        lib.gemm_bf16_ex(M, N, K, alpha, dev_copy(A.view(np.int16), dev), lda, dev_copy(Bs.view(np.int16), dev),
                         ldb, beta, dC, N, transB=tb, stream=stream())
        return host(dC), want, scale

    M, N, K = 300, 1000, 520
    for splits in (1, 2, 3, 4):
        with lib.tunables(TILE_CFG=39, TILE_SPLITS=splits):
            p = lib.plan_bf16_ex(M, N, K, transB=tb)
            assert (p["name"], p["rows"], p["cols"], p["splits"]) == ("dnnopt_tile_bf16_dma", 128, 128, splits), p
            got, want, scale = run(M, N, K, 2, 4, 0.5, 0.25, 21)
        u.assert_fp32_close(got, want, scale, K, f"128x128 forced, {splits} splits, tb={tb}")
    for (M, N, K), splits in (((256, 4096, 4096), 4),):
        p = lib.plan_bf16_ex(M, N, K, transB=tb)
        assert (p["name"], p["rows"], p["cols"], p["splits"], p["block"]) == ("dnnopt_tile_bf16_dma", 128, 128, splits,
                                                                             256), p
        got, want, scale = run(M, N, K, 0, 0, 1.0, 0.0, 31)
        u.assert_fp32_close(got, want, scale, K, f"128x128 planned {M}x{N}x{K} tb={tb}")


@pytest.mark.parametrize("mode", ["f2b", "bf16", "bf16_tb"])
def test_lds_256x96_register_ring_tiles(lib, orc, dev, mode):
    """256 x 96 LDS-staged tiles on 8 waves of 64 x 48, operands staged through
    a register ring (fp32 inputs rounded in registers, or bf16 storage with B
    stored K x N or N x K): forced with 1 to 3 k-splits on a ragged shape (M
    and N off the tile, a K tail inside a 64-k block, padded strides, beta !=
    0, alpha != 1)."""
    M, N, K, pa, pb = 300, 1000, 520, 2, 4
    tb = int(mode == "bf16_tb")
    lda, ldb = K + pa, (K + pb if tb else N + pb)
    rows = N if tb else K
    A32 = u.normal(orc, M * lda, 41).reshape(M, lda)
    B32 = u.normal(orc, rows * ldb, 42, 0, 0.02).reshape(rows, ldb)
    C0 = u.uniform(orc, M * N, 43).reshape(M, N)
    A, Bs = u.bf16_bits(orc, A32), u.bf16_bits(orc, B32)
    Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
    want, scale = u.exact(u.bf16_value(A)[:, :K], u.bf16_value(Bkn), 0.5, 0.25, C0)
    for splits in (1, 2, 3):
        with lib.tunables(TILE_CFG=40, TILE_SPLITS=splits):
            if mode == "f2b":
                p = lib.plan_bf16(M, N, K, fp32_inputs=1)
            else:
                p = lib.plan_bf16_ex(M, N, K, transB=tb)
            assert (p["name"], p["rows"], p["cols"], p["splits"]) == ("dnnopt_tile_bf16_lds", 256, 96, splits), p
            dC = dev_copy(C0, dev)
            if mode == "f2b":
                lib.gemm_bf16_f32in(M, N, K, 0.5, dev_copy(A32, dev), lda, dev_copy(B32, dev), ldb, 0.25, dC, N,
                                    stream=stream())
            else:
                lib.gemm_bf16_ex(M, N, K, 0.5, dev_copy(A.view(np.int16), dev), lda, dev_copy(Bs.view(np.int16), dev),
                                 ldb, 0.25, dC, N, transB=tb, stream=stream())
            got = host(dC)
        u.assert_fp32_close(got, want, scale, K, f"256x96 register ring, {mode}, {splits} splits")


@pytest.mark.parametrize("M,N,K,rows,cols,splits", [(96, 4096, 1024, 32, 64, 1), (256, 4096, 4096, 64, 128, 2),
                                                    (384, 11008, 1024, 256, 96, 1), (1024, 4096, 1024, 256, 96, 1),
                                                    (128, 4096, 1024, None, None, None)])
def test_bf16_fp32_inputs_cost_model_picks(lib, orc, dev, M, N, K, rows, cols, splits):
    """fp32 inputs: the tile and split count the cost models pick (32 x 64
    unsplit, 64 x 128 with 2 splits, 256 x 96 tiles in fewer rounds), each
    within the fp32 bound of the exact product of the bf16-rounded
    operands."""
    p = lib.plan_bf16(M, N, K, fp32_inputs=1)
    assert p["name"] == "dnnopt_tile_bf16_lds", p
    if rows is not None:
        assert (p["rows"], p["cols"], p["splits"]) == (rows, cols, splits), p
    A = u.normal(orc, M * K, 51).reshape(M, K)
    B = u.normal(orc, K * N, 52, 0, 0.02).reshape(K, N)
    dC = torch.full((M * N,), float("nan"), dtype=torch.float32, device=dev)
    lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, N, stream=stream())
    want, scale = u.exact(u.bf16_value(u.bf16_bits(orc, A)), u.bf16_value(u.bf16_bits(orc, B)))
    u.assert_fp32_close(host(dC).reshape(M, N), want, scale, K, f"f32 inputs planned {M}x{N}x{K}")


def test_bf16_fp32_inputs_wide_c_stride_keeps_128_row_tiles(lib, orc, dev):
    """A C row stride at which 256 rows span more than 2^31 bytes (ldc =
    2^21 + 2^14 floats): the 256 x 96 register-ring tile, whose unsplit
    epilogue addresses C with 32-bit offsets from the tile's first row, is
    not used (the model would pick it for 384 x 11008 x 1024) and every row
    is written; the padding columns between rows stay untouched."""
    M, N, K = 384, 11008, 1024
    ldc = (1 << 21) + (1 << 14)
    assert lib.plan_bf16(M, N, K, fp32_inputs=1)["rows"] == 256
    A = u.normal(orc, M * K, 61).reshape(M, K)
    B = u.normal(orc, K * N, 62, 0, 0.02).reshape(K, N)
    dC = torch.full(((M - 1) * ldc + N,), float("nan"), dtype=torch.float32, device=dev)
    with lib.tunables(TILE_CFG=40):  # a forced 256-row tile is refused at this stride too
        lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, ldc, stream=stream())
        got_forced = host(torch.as_strided(dC, (M, N), (ldc, 1)))
    dC.fill_(float("nan"))
    lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, ldc, stream=stream())
    got = host(torch.as_strided(dC, (M, N), (ldc, 1)))
    pad = host(torch.as_strided(dC, (M - 1, 64), (ldc, 1), N))
    del dC
    torch.cuda.empty_cache()
    want, scale = u.exact(u.bf16_value(u.bf16_bits(orc, A)), u.bf16_value(u.bf16_bits(orc, B)))
    u.assert_fp32_close(got, want, scale, K, "f32 inputs, ldc 2^21 + 2^14")
    u.assert_fp32_close(got_forced, want, scale, K, "f32 inputs, forced 256-row tile, ldc 2^21 + 2^14")
    assert np.isnan(pad).all(), "a write landed between the rows of C"


def test_bf16_dma_k_split_ticket_matches_reduce_kernel(lib, orc, dev):
    """A 2-way k-split of 256 x 96 LDS-DMA tiles summed by the last workgroup
    to finish (tunable TILE_TICKET=1) gives the same bits as the reduce kernel
    (the default), repeatably, within the fp32 bound of the exact result."""
    M, N, K = 300, 1000, 520
    A = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
    B = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02)).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dA = torch.from_numpy(A.view(np.int16)).to(dev)
    dB = torch.from_numpy(B.view(np.int16)).to(dev)
    res = {}
    for ticket in (0, 1):
        with lib.tunables(TILE_CFG=33, TILE_SPLITS=2, TILE_TICKET=ticket):
            p = lib.plan_bf16(M, N, K)
            assert p["name"] == "dnnopt_tile_bf16_dma" and p["splits"] == 2, p
            outs = []
            for rep in range(3):
                dC = dev_copy(C0, dev)
                lib.gemm_bf16(M, N, K, 0.5, dA, K, dB, N, 1.0, dC, N, stream=stream())
                outs.append(host(dC))
        res[ticket] = outs
    assert (lib.get_tunable("TILE_CFG"), lib.get_tunable("TILE_SPLITS"), lib.get_tunable("TILE_TICKET")) == (0, 0, 0)
    want, scale = u.exact(u.bf16_value(A), u.bf16_value(B), 0.5, 1.0, C0)
    for ticket, outs in res.items():
        for o in outs:
            assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), f"ticket={ticket} not repeatable"
        u.assert_fp32_close(outs[0], want, scale, K, f"dma k-split ticket={ticket}")
    assert np.array_equal(res[0][0].view(np.uint32), res[1][0].view(np.uint32))


def test_bf16_lds_misaligned_falls_back(lib, orc, dev):
    """bf16 operands 2 bytes off a 4-byte boundary take the register-only tiles."""
    M, N, K = 128, 512, 256
    A = u.bf16_bits(orc, u.normal(orc, M * K + 1, 1))
    B = u.bf16_bits(orc, u.normal(orc, K * N + 1, 2, 0, 0.02))
    dA, dB = dev_copy(A.view(np.int16), dev), dev_copy(B.view(np.int16), dev)
    want, scale = u.exact(u.bf16_value(A[1:]).reshape(M, K), u.bf16_value(B[1:]).reshape(K, N))
    for a_off, b_off in ((2, 0), (0, 2), (2, 2)):
        dC = torch.zeros((M, N), dtype=torch.float32, device=dev)
        AA = A[1:] if a_off else A[:-1]
        BB = B[1:] if b_off else B[:-1]
        want, scale = u.exact(u.bf16_value(AA).reshape(M, K), u.bf16_value(BB).reshape(K, N))
        lib.gemm_bf16(M, N, K, 1.0, dA.data_ptr() + a_off, K, dB.data_ptr() + b_off, N, 0.0, dC, N, stream=stream())
        u.assert_fp32_close(host(dC), want, scale, K, f"misaligned a+{a_off} b+{b_off}")


@pytest.mark.parametrize("M,N,K", [(1, 11008, 4096), (4, 11008, 4096), (32, 11008, 4096), (256, 11008, 4096),
                                   (4, 1000, 512), (7, 33, 65), (32, 300, 260), (256, 1024, 512)])
def test_bf16_fp32_inputs(lib, orc, dev, M, N, K):
    """fp32-input gemm_bf16, including every C4 shape at full size."""
    A = u.normal(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    dC = torch.zeros(M * N, dtype=torch.float32, device=dev)
    lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, N, stream=stream())
    got = host(dC).reshape(M, N)
    Ar, Br = u.bf16_value(u.bf16_bits(orc, A)), u.bf16_value(u.bf16_bits(orc, B))
    want, scale = u.exact(Ar, Br)
    u.assert_fp32_close(got, want, scale, K, "bf16 rounded in registers")
    w2, s2 = u.exact(A, B)
    assert (np.abs(got - w2) <= 1e-2 * s2 + 1e-30).all(), "bf16 vs unrounded fp32 beyond 1e-2"


# ---------------------------------------------------------------- int8
S8 = [(M, N, 4096) for M in (1, 8, 128) for N in (4096, 4093)]
S8 += [(1, 1, 1), (3, 5, 15), (17, 33, 17), (16, 16, 255), (9, 100, 300), (40, 7, 1000), (130, 70, 64),
       (2, 3, 257)]


@pytest.mark.parametrize("M,N,K", S8)
def test_int8_bit_exact(lib, orc, dev, M, N, K):
    A = u.ints8(orc, M * K, 1).reshape(M, K)
    B = u.ints8(orc, N * K, 2).reshape(N, K)
    dC = torch.full((M, N), -7, dtype=torch.int32, device=dev)
    lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), K, dev_copy(B, dev), K, dC, N, stream=stream())
    want = (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int64)  # exact below 2^53
    assert np.array_equal(host(dC).astype(np.int64), want)


def test_int8_padded_strides_and_extremes(lib, orc, dev):
    M, N, K = 9, 21, 300
    lda, ldb, ldc = K + 5, K + 3, N + 2
    A = u.ints8(orc, M * lda, 1, -128, 127).reshape(M, lda)
    B = u.ints8(orc, N * ldb, 2, -128, 127).reshape(N, ldb)
    A[0, :K] = -128
    B[0, :K] = -128
    dC = torch.full((M, ldc), 99, dtype=torch.int32, device=dev)
    lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, dC, ldc, stream=stream())
    got = host(dC)
    want = (A[:, :K].astype(np.float64) @ B[:, :K].astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got[:, :N].astype(np.int64), want)
    assert (got[:, N:] == 99).all()
    assert got[0, 0] == K * 128 * 128


# M <= 4: the int8 row-dot kernel (v_dot4 on 16-byte row chunks); M = 5..8:
# the MFMA tiles, same checks.  K values around the 16-byte chunk and the
# 1 KiB step, rows off 4-byte boundaries.
S8_ROWDOT = [(M, N, K) for M in range(1, 9) for (N, K) in ((7, 1), (33, 15), (100, 17), (65, 1024), (129, 4097))]


@pytest.mark.parametrize("M,N,K", S8_ROWDOT)
def test_int8_rowdot_bit_exact(lib, orc, dev, M, N, K):
    b = u.binding()
    assert lib.plan_s8(M, N, K)["kernel"] == (b.K_ROWDOT_S8 if M <= 4 else b.K_MFMA_S8)
    for pad in (0, 1, 3):  # 1, 3: rows start off 4-byte boundaries (funnel-shifted loads)
        lda, ldb, ldc = K + pad, K + 2 * pad, N + 1
        A = u.ints8(orc, M * lda, 1, -128, 127).reshape(M, lda)
        B = u.ints8(orc, N * ldb, 2, -128, 127).reshape(N, ldb)
        A[:, K:] = 127  # row padding must never reach a product
        B[:, K:] = 127
        dC = torch.full((M, ldc), -7, dtype=torch.int32, device=dev)
        lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, dC, ldc, stream=stream())
        got = host(dC)
        want = A[:, :K].astype(np.int64) @ B[:, :K].astype(np.int64).T
        assert np.array_equal(got[:, :N].astype(np.int64), want), (M, N, K, pad)
        assert (got[:, N] == -7).all()
        s = u.uniform(orc, N, 4, 0.001, 0.01)
        dF = torch.zeros((M, ldc), dtype=torch.float32, device=dev)
        lib.gemm_s8s8f32_colscale(M, N, K, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, dev_copy(s, dev), dF, ldc,
                                  stream=stream())
        assert np.array_equal(host(dF)[:, :N], want.astype(np.float32) * s[None, :]), (M, N, K, pad)


def test_int8_rowdot_extremes(lib, orc, dev):
    # -128 * -128 summed over K = 4097 (67,125,248): exact in int32
    for M in (1, 4, 8):
        N, K = 70, 4097
        A = np.full((M, K), -128, np.int8)
        B = np.full((N, K), -128, np.int8)
        dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
        lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), K, dev_copy(B, dev), K, dC, N, stream=stream())
        assert (host(dC) == K * 128 * 128).all()


@pytest.mark.parametrize("M,N", [(1, 4096), (8, 4093), (128, 4093)])
def test_int8_colscale(lib, orc, dev, M, N):
    K = 4096
    A, B = u.ints8(orc, M * K, 1).reshape(M, K), u.ints8(orc, N * K, 2).reshape(N, K)
    s = u.uniform(orc, N, 4, 0.001, 0.01)
    dC = torch.zeros((M, N), dtype=torch.float32, device=dev)
    lib.gemm_s8s8f32_colscale(M, N, K, dev_copy(A, dev), K, dev_copy(B, dev), K, dev_copy(s, dev), dC, N,
                              stream=stream())
    acc = (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(host(dC), acc * s[None, :])


@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (7, 13, 5), (3, 3, 1000), (13, 17, 19), (64, 300, 257),
                                   (8, 4093, 4096), (1, 4096, 4096), (128, 1024, 512), (40, 70, 2000)])
def test_int8_dynamic_quant_matches_oracle(lib, orc, dev, M, N, K):
    A, B, C0 = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2), u.uniform(orc, M * N, 3)
    for beta in (0.0, 0.5):
        Co = C0.copy()
        orc.orc_gemm_int8(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(Co), N)
        dC = dev_copy(C0, dev)
        lib.gemm_int8_f32(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, beta, dC, N, stream=stream())
        assert np.array_equal(host(dC).view(np.uint32), Co.view(np.uint32))


@pytest.mark.parametrize("M,N,K,pa,pb", [(9, 300, 130, 3, 5), (2, 1000, 77, 1, 4), (130, 257, 600, 0, 1),
                                        (16, 515, 256, 4, 9), (24, 1030, 200, 4, 2)])
def test_int8_dynamic_quant_padded_strides(lib, orc, dev, M, N, K, pa, pb):
    # Rows of A and B that do not start on 16-byte boundaries, padding between
    # rows (NaN, never read) and a C block inside a wider matrix.
    lda, ldb, ldc = K + pa, N + pb, N + 2
    A = np.full((M, lda), np.nan, np.float32)
    A[:, :K] = u.uniform(orc, M * K, 1).reshape(M, K)
    B = np.full((K, ldb), np.nan, np.float32)
    B[:, :N] = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    C0 = u.uniform(orc, M * ldc, 3).reshape(M, ldc)
    Co, Ak, Bn = C0.copy(), np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :N])
    orc.orc_gemm_int8(M, N, K, 0.75, u.ptr(Ak), K, u.ptr(Bn), N, 0.5, u.ptr(Co), ldc)
    dC = dev_copy(C0, dev)
    lib.gemm_int8_f32(M, N, K, 0.75, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, 0.5, dC, ldc, stream=stream())
    assert np.array_equal(host(dC).view(np.uint32), Co.view(np.uint32))


def test_int8_dynamic_quant_rounding_ties(lib, dev):
    """Quantized values that are exact ties and fractions (scales 1 and 2):
    the device quantizer must round to nearest even like the reference's
    lrintf (src/gemm/gemm_pack_int8.cpp:66-71), independently of the oracle."""

    def run(M, N, K, A, B):
        dC = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        lib.gemm_int8_f32(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.0, dC, N, stream=stream())
        return host(dC)

    u.check_dynq_ties(run)


def _gpu_int8(lib, dev, a_scale=1.0, b_scale=1.0, alpha_scale=1.0):
    """gemm_int8_f32 through the C-ABI for check_int8_routes; A and B are
    scaled by powers of two and alpha by their inverse, which leaves every
    quantized value and the dequantization factor unchanged."""

    def run(M, N, K, A, B, alpha, beta, C0):
        dA = dev_copy((np.asarray(A, np.float64) * a_scale).astype(np.float32), dev)
        dB = dev_copy((np.asarray(B, np.float64) * b_scale).astype(np.float32), dev)
        dC = dev_copy(C0, dev)
        lib.gemm_int8_f32(M, N, K, float(np.float32(alpha * alpha_scale)), dA, K, dB, N, beta, dC, N,
                          stream=stream())
        return host(dC)

    return run


def test_int8_route_closed_forms(lib, dev):
    """The reference's two gemm_int8 routes on closed-form inputs (division
    quantizer and small-M epilogues at M <= 8, the packed path above),
    independent of the oracle: every bit of C is fixed by the arithmetic."""
    u.check_int8_routes(_gpu_int8(lib, dev))


@pytest.mark.parametrize("b_scale", [2.0 ** -80, 2.0 ** -60, 2.0 ** 60, 2.0 ** 80])
def test_int8_route_closed_forms_extreme_scales(lib, dev, b_scale):
    """Scales outside [2^-64, 2^64] take the exact division (2^-80, 2^80), the
    others the reciprocal with one correction (2^-60, 2^60): same bits."""
    u.check_int8_routes(_gpu_int8(lib, dev, b_scale=b_scale, alpha_scale=1.0 / b_scale), Ms=(1, 3, 8, 9))


def test_int8_smallm_far_apart_rows_of_a(lib, orc, dev):
    """Rows of A 2^28 floats apart ((M - 1) * lda * 4 >= 2^31 bytes): the
    small-M kernel reads A through 64-bit addresses."""
    M, N, K = 3, 777, 300
    lda = (1 << 28) + 64
    A = u.uniform(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.5).reshape(K, N)
    dA = torch.zeros((M - 1) * lda + K, dtype=torch.float32, device=dev)
    for m in range(M):
        dA[m * lda:m * lda + K] = torch.from_numpy(A[m]).to(dev)
    C0 = u.uniform(orc, M * N, 3)
    Co = C0.copy()
    orc.orc_gemm_int8(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.5, u.ptr(Co), N)
    dC = dev_copy(C0, dev)
    lib.gemm_int8_f32(M, N, K, 1.0, dA, lda, dev_copy(B, dev), N, 0.5, dC, N, stream=stream())
    got = host(dC)
    del dA
    assert np.array_equal(got.view(np.uint32), Co.view(np.uint32))


def test_int8_f32_large_c_stride(lib, orc, dev):
    """M > 8 with a C stride past the 64-row q8b tiles' 31-bit offsets
    (64 * ldc * 4 >= 2^31): the call takes the quantization pass and the
    planner-checked int8 kernels instead, bit-exact."""
    M, N, K = 64, 500, 256
    ldc = (1 << 23) + 300000
    assert 64 * ldc * 4 >= 2 ** 31
    A = u.uniform(orc, M * K, 1).reshape(M, K)
    B = u.normal(orc, K * N, 2, 0, 0.5).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    Co = C0.copy()
    orc.orc_gemm_int8(M, N, K, 0.5, u.ptr(A), K, u.ptr(B), N, 0.25, u.ptr(Co), N)
    dC = torch.full(((M - 1) * ldc + N,), 7.0, dtype=torch.float32, device=dev)
    rows = torch.as_strided(dC, (M, N), (ldc, 1))
    rows.copy_(torch.from_numpy(C0).to(dev))
    lib.gemm_int8_f32(M, N, K, 0.5, dev_copy(A, dev), K, dev_copy(B, dev), N, 0.25, dC, ldc, stream=stream())
    got = host(rows.contiguous())
    gap = host(dC[N:N + 1000])
    del dC, rows
    assert np.array_equal(got.view(np.uint32), Co.view(np.uint32))
    assert (gap == 7.0).all()


# ---------------------------------------------------------------- saxpy, C++ and BLAS APIs on host memory
def test_saxpy(lib, orc, dev):
    for n, incx, incy in [(1, 1, 1), (1000, 1, 1), (777, 3, 2), (500, 0, 1), (300, 2, 0), (300, 0, 0)]:
        X, Y0 = u.uniform(orc, max(1, n * incx), 5), u.uniform(orc, max(1, n * incy), 6)
        Yo = Y0.copy()
        orc.orc_saxpy(n, 0.7, u.ptr(X), incx, u.ptr(Yo), incy, 1)
        dY = dev_copy(Y0, dev)
        lib.saxpy(n, 0.7, dev_copy(X, dev), incx, dY, incy, stream=stream())
        assert np.array_equal(host(dY).view(np.uint32), Yo.view(np.uint32))
        Yh = Y0.copy()
        lib.so.cblas_saxpy(n, 0.7, X.ctypes.data, incx, Yh.ctypes.data, incy)
        assert lib.last_status() == 0 and np.array_equal(Yh.view(np.uint32), Yo.view(np.uint32))


CBLAS_SIZES = [(4, 4, 4), (16, 16, 16), (32, 64, 48), (128, 128, 128), (7, 13, 11), (1, 64, 32), (256, 256, 256)]


@pytest.mark.parametrize("M,N,K", CBLAS_SIZES)
def test_cblas_matrix_of_the_reference(lib, orc, M, N, K):
    """Every Order x Trans case of tests/test_cblas.cpp:78-334 plus Fortran
    sgemm_, on host arrays, against the oracle's restatement of
    cblas_sgemm.cpp (explicit transposes + scalar loop)."""
    b = u.binding()
    for order in (101, 102):
        for ta in (111, 112):
            for tb in (111, 112):
                rows_a, cols_a = (M, K) if ta == 111 else (K, M)
                rows_b, cols_b = (K, N) if tb == 111 else (N, K)
                if order == 102:
                    rows_a, cols_a, rows_b, cols_b = cols_a, rows_a, cols_b, rows_b
                A = u.uniform(orc, rows_a * cols_a, 1)
                B = u.uniform(orc, rows_b * cols_b, 2)
                crow, ccol = (M, N) if order == 101 else (N, M)
                C0 = u.uniform(orc, crow * ccol, 3)
                Co, Cg = C0.copy(), C0.copy()
                orc.orc_cblas_sgemm(order, ta, tb, M, N, K, 2.5, u.ptr(A), cols_a, u.ptr(B), cols_b, -0.3,
                                    u.ptr(Co), ccol)
                lib.cblas_sgemm(order, ta, tb, M, N, K, 2.5, A, cols_a, B, cols_b, -0.3, Cg, ccol)
                _, scale = u.exact(np.abs(A).reshape(1, -1)[:, :1], np.abs(B).reshape(1, -1)[:1, :1])
                tol = K * 5e-4  # tests/test_cblas.cpp alpha/beta tolerance
                assert np.abs(Cg - Co).max() < tol, (order, ta, tb)
    # Fortran entry: column-major NN with alpha 1, beta 0
    A = u.uniform(orc, M * K, 1)
    B = u.uniform(orc, K * N, 2)
    C = np.zeros(M * N, np.float32)
    import ctypes

    ci = lambda v: ctypes.byref(ctypes.c_int(v))  # noqa: E731
    cf = lambda v: ctypes.byref(ctypes.c_float(v))  # noqa: E731
    lib.so.sgemm_(ctypes.c_char_p(b"N"), ctypes.c_char_p(b"N"), ci(M), ci(N), ci(K), cf(1.0), A.ctypes.data,
                  ci(M), B.ctypes.data, ci(K), cf(0.0), C.ctypes.data, ci(M))
    want, scale = u.exact(A.reshape(K, M).T, B.reshape(N, K).T)
    u.assert_fp32_close(C.reshape(N, M).T, want, scale, K, "sgemm_")


def test_cxx_api_host_and_device_pointers(lib, orc, dev):
    M, N, K = 5, 1009, 2048
    A, B, C0 = u.normal(orc, M * K, 1, 0, .02), u.normal(orc, K * N, 2, 0, .02), u.uniform(orc, M * N, 3)
    want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), 1.0, 1.0, C0.reshape(M, N))
    Ch = C0.copy()
    lib.gemm_fp32(M, N, K, 1.0, A, K, B, N, 1.0, Ch, N)
    u.assert_fp32_close(Ch.reshape(M, N), want, scale, K, "gemm_fp32 host")
    dC = dev_copy(C0, dev)
    lib.gemm_fp32(M, N, K, 1.0, dev_copy(A, dev), K, dev_copy(B, dev), N, 1.0, dC, N)
    u.assert_fp32_close(host(dC).reshape(M, N), want, scale, K, "gemm_fp32 device")
    Cn, Co = C0.copy(), C0.copy()
    lib.gemm_fp32(M, N, K, 1.0, A, K, B, N, 1.0, Cn, N, algo="kNaive")
    orc.orc_gemm_naive_f32(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 1.0, u.ptr(Co), N)
    assert np.array_equal(Cn.view(np.uint32), Co.view(np.uint32))
    # bf16 on fp32 storage, native bf16, fp32-API int8, native int8
    Cb = np.zeros(M * N, np.float32)
    lib.cxx["gemm_bf16"](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.0, Cb.ctypes.data, N)
    assert lib.last_status() == 0
    w2, s2 = u.exact(A.reshape(M, K), B.reshape(K, N))
    assert (np.abs(Cb.reshape(M, N) - w2) <= 1e-2 * s2).all()
    Ab, Bb = u.bf16_bits(orc, A), u.bf16_bits(orc, B)
    Cbb = np.zeros(M * N, np.float32)
    lib.cxx["gemm_bf16_bf16bf16f32"](M, N, K, 1.0, Ab.ctypes.data, K, Bb.ctypes.data, N, 0.0, Cbb.ctypes.data, N)
    wb, sb = u.exact(u.bf16_value(Ab).reshape(M, K), u.bf16_value(Bb).reshape(K, N))
    u.assert_fp32_close(Cbb.reshape(M, N), wb, sb, K, "gemm_bf16_bf16bf16f32 host")
    Ci, Cio = C0.copy(), C0.copy()
    lib.cxx["gemm_int8"](M, N, K, 1.0, A.ctypes.data, K, B.ctypes.data, N, 0.5, Ci.ctypes.data, N)
    orc.orc_gemm_int8(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 0.5, u.ptr(Cio), N)
    assert np.array_equal(Ci.view(np.uint32), Cio.view(np.uint32))
    A8, B8 = u.ints8(orc, M * K, 1), u.ints8(orc, N * K, 2)
    C8 = np.zeros(M * N, np.int32)
    lib.cxx["gemm_int8_int8int8int32"](M, N, K, A8.ctypes.data, K, B8.ctypes.data, K, C8.ctypes.data, N)
    assert lib.last_status() == 0
    assert np.array_equal(C8.reshape(M, N), (A8.reshape(M, K).astype(np.int64) @ B8.reshape(N, K).T.astype(np.int64)))


def test_empty_problems_do_not_touch_c(lib, dev):
    C = torch.full((4, 4), 3.0, device=dev)
    A = torch.ones(16, device=dev)
    for M, N, K in ((0, 4, 4), (4, 0, 4), (4, 4, 0), (-1, 4, 4)):
        lib.sgemm(M, N, K, 1.0, A, 4, A, 4, 0.0, C, 4, stream=stream())
    assert (host(C) == 3.0).all()


@pytest.mark.parametrize("kind,M,N,K", [("f32", 1, 4096, 4096), ("f32", 7, 1009, 2048), ("f32", 3, 257, 5000),
                                        ("s8", 1, 4096, 4096), ("s8", 128, 4093, 4096), ("bf16", 4, 11008, 4096),
                                        ("f32t", 64, 64, 262144)])
def test_split_k_repeatable(lib, orc, dev, kind, M, N, K):
    """Split-k launches reduce partial sums across workgroups; 25 repetitions
    must agree bit for bit with each other and with the exact result."""
    if kind == "s8":
        A, B = u.ints8(orc, M * K, 1).reshape(M, K), u.ints8(orc, N * K, 2).reshape(N, K)
        dA, dB = dev_copy(A, dev), dev_copy(B, dev)
        want = (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int64)
        outs = []
        for _ in range(25):
            dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
            lib.gemm_s8s8s32(M, N, K, dA, K, dB, K, dC, N, stream=stream())
            outs.append(dC)
        for o in outs:
            assert np.array_equal(host(o).astype(np.int64), want)
        return
    if kind == "bf16":
        A = u.bf16_bits(orc, u.normal(orc, M * K, 1)).reshape(M, K)
        B = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02)).reshape(K, N)
        dA, dB = dev_copy(A.view(np.int16), dev), dev_copy(B.view(np.int16), dev)
        run = lambda dC: lib.gemm_bf16(M, N, K, 1.0, dA, K, dB, N, 0.0, dC, N, stream=stream())  # noqa: E731
        want, scale = u.exact(u.bf16_value(A), u.bf16_value(B))
    else:
        ta = 1 if kind == "f32t" else 0
        opA = u.uniform(orc, M * K, 1).reshape(M, K)
        B = u.uniform(orc, K * N, 2).reshape(K, N)
        A = np.ascontiguousarray(opA.T) if ta else opA
        dA, dB = dev_copy(A, dev), dev_copy(B, dev)
        run = lambda dC: lib.sgemm(M, N, K, 1.0, dA, A.shape[1], dB, N, 0.0, dC, N, transA=ta,  # noqa: E731
                                   stream=stream())
        want, scale = u.exact(opA, B)
    outs = []
    for _ in range(25):
        dC = torch.full((M, N), np.nan, dtype=torch.float32, device=dev)
        run(dC)
        outs.append(dC)
    first = host(outs[0])
    u.assert_fp32_close(first, want, scale, K, f"split-k {kind} {M}x{N}x{K}")
    for o in outs[1:]:
        assert np.array_equal(host(o).view(np.uint32), first.view(np.uint32))


# ---------------------------------------------------------------- shapes outside the benchmark configs
# N == 1, tall-skinny N <= 7, K <= 16, M in 8..31 with moderate N, and mixes:
# every entry point must route each to a kernel that gives the right result.
EDGE = [(65536, 1, 256), (5000, 1, 3), (40000, 7, 300), (20000, 3, 16), (1000, 5, 1), (12, 700, 16), (9, 1000, 5),
        (31, 257, 1000), (17, 64, 8192), (8, 1, 1), (24, 33, 7), (300, 2, 2049)]


@pytest.mark.parametrize("M,N,K", EDGE)
def test_edge_shapes_every_entry_point(lib, orc, dev, M, N, K):
    A32 = u.uniform(orc, M * K, 1).reshape(M, K)
    B32 = u.uniform(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    # fp32, every transpose combination
    for ta in (0, 1):
        for tb in (0, 1):
            A = np.ascontiguousarray(A32.T) if ta else A32
            B = np.ascontiguousarray(B32.T) if tb else B32
            dC = dev_copy(C0, dev)
            lib.sgemm(M, N, K, 0.5, dev_copy(A, dev), A.shape[1], dev_copy(B, dev), B.shape[1], 2.0, dC, N,
                      transA=ta, transB=tb, stream=stream())
            want, scale = u.exact(A32, B32, 0.5, 2.0, C0)
            u.assert_fp32_close(host(dC), want, scale, K, f"f32 edge {M}x{N}x{K} ta={ta} tb={tb}")
    # bf16 storage, every transpose combination
    Ab, Bb = u.bf16_bits(orc, A32), u.bf16_bits(orc, B32)
    want, scale = u.exact(u.bf16_value(Ab), u.bf16_value(Bb), 1.0, 1.0, C0)
    for ta in (0, 1):
        for tb in (0, 1):
            A = np.ascontiguousarray(Ab.T) if ta else Ab
            B = np.ascontiguousarray(Bb.T) if tb else Bb
            dC = dev_copy(C0, dev)
            lib.gemm_bf16_ex(M, N, K, 1.0, dev_copy(A.view(np.int16), dev), A.shape[1],
                             dev_copy(B.view(np.int16), dev), B.shape[1], 1.0, dC, N, transA=ta, transB=tb,
                             stream=stream())
            u.assert_fp32_close(host(dC), want, scale, K, f"bf16 edge {M}x{N}x{K} ta={ta} tb={tb}")
    # fp32 storage rounded to bf16 in registers
    dC = dev_copy(C0, dev)
    lib.gemm_bf16_f32in(M, N, K, 1.0, dev_copy(A32, dev), K, dev_copy(B32, dev), N, 1.0, dC, N, stream=stream())
    u.assert_fp32_close(host(dC), want, scale, K, f"f2b edge {M}x{N}x{K}")
    # int8, exact
    A8, B8 = u.ints8(orc, M * K, 1).reshape(M, K), u.ints8(orc, N * K, 2).reshape(N, K)
    dC = torch.zeros((M, N), dtype=torch.int32, device=dev)
    lib.gemm_s8s8s32(M, N, K, dev_copy(A8, dev), K, dev_copy(B8, dev), K, dC, N, stream=stream())
    assert np.array_equal(host(dC).astype(np.int64), A8.astype(np.int64) @ B8.T.astype(np.int64))


# ---------------------------------------------------------------- seeded sweeps over every route
def _sgemm_sweep_cases():
    """Seeded fp32 shapes spread over the dispatcher's routes (skinny, row-dot,
    16-row tiles, 64-row tiles, tall-skinny, k-outer), both operand layouts,
    padded strides, assorted alpha / beta.  Sizes keep the fp64 reference
    under a second each."""
    rng = np.random.default_rng(20261203)
    cases = []
    while len(cases) < 28:
        kind = len(cases) % 7
        if kind == 0:
            M, N, K = int(rng.integers(1, 9)), int(rng.integers(1, 6000)), int(rng.integers(1, 3000))
        elif kind == 1:
            M, N, K = int(rng.integers(9, 33)), int(rng.integers(16, 5000)), int(rng.integers(1, 2000))
        elif kind == 2:
            M, N, K = int(rng.integers(33, 600)), int(rng.integers(16, 3000)), int(rng.integers(1, 700))
        elif kind == 3:
            M, N, K = int(rng.integers(20000, 70000)), int(rng.integers(17, 65)), 256
            if (len(cases) // 7) % 2:  # K off the 64-grid: the register-ring tall kernel
                M, K = M + 30000, 200
        elif kind == 4:
            M, N, K = int(rng.integers(1, 5)), int(rng.integers(1, 9000)), int(rng.integers(1, 2100))
        elif kind == 5:
            M, N, K = 4 * int(rng.integers(9, 17)), 4 * int(rng.integers(9, 17)), int(rng.integers(32768, 70000))
        else:
            M, N, K = int(rng.integers(1, 400)), int(rng.integers(1, 400)), int(rng.integers(1, 400))
        if M * N * K > 250_000_000:
            continue
        ta = int(rng.integers(0, 2)) if kind not in (3, 5) else int(kind == 5)
        tb = int(rng.integers(0, 2)) if kind not in (3, 5) else 0
        if kind == 4:
            tb = 1
        pa, pb = int(rng.integers(0, 4)) * (kind != 5), int(rng.integers(0, 4)) * (kind != 5)
        alpha = float(rng.choice([1.0, 0.5, -1.25]))
        beta = float(rng.choice([0.0, 1.0, -0.5]))
        cases.append((M, N, K, ta, tb, pa, pb, alpha, beta))
    return cases


_SGEMM_SWEEP = _sgemm_sweep_cases()


@pytest.mark.parametrize("M,N,K,ta,tb,pa,pb,alpha,beta", _SGEMM_SWEEP)
def test_sgemm_route_sweep(lib, orc, dev, M, N, K, ta, tb, pa, pb, alpha, beta):
    lda = (M if ta else K) + pa
    ldb = (K if tb else N) + pb
    As = u.normal(orc, (K if ta else M) * lda, 1, 0, 0.5).reshape(K if ta else M, lda)
    Bs = u.normal(orc, (N if tb else K) * ldb, 2, 0, 0.5).reshape(N if tb else K, ldb)
    Amk = np.ascontiguousarray(As[:, :M].T if ta else As[:, :K])
    Bkn = np.ascontiguousarray(Bs[:, :K].T if tb else Bs[:, :N])
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dC = dev_copy(C0 if beta != 0.0 else np.full_like(C0, np.nan), dev)
    lib.sgemm(M, N, K, alpha, dev_copy(As, dev), lda, dev_copy(Bs, dev), ldb, beta, dC, N, transA=ta, transB=tb,
              stream=stream())
    want, scale = u.exact(Amk, Bkn, alpha, beta, C0 if beta != 0.0 else None)
    u.assert_fp32_close(host(dC), want, scale, K, f"sweep {M}x{N}x{K} ta={ta} tb={tb} a={alpha} b={beta}")


def test_sgemm_route_sweep_covers_every_route(lib):
    names = {lib.plan_sgemm(M, N, K, transA=ta, transB=tb)["name"] for M, N, K, ta, tb, *_ in _SGEMM_SWEEP}
    assert names >= {"dnnopt_skinny", "dnnopt_rowdot", "dnnopt_tile_f32", "dnnopt_tall_f32", "dnnopt_tall_dma_f32",
                     "dnnopt_kouter_f32"}, names


def _s8_sweep_cases():
    rng = np.random.default_rng(20261204)
    cases = []
    while len(cases) < 16:
        band = len(cases) % 4
        M = int(rng.integers(*((1, 5), (5, 17), (17, 300), (1, 300))[band]))
        N, K = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
        if M * N * K > 400_000_000:
            continue
        pa, pb = int(rng.integers(0, 5)), int(rng.integers(0, 5))
        cases.append((M, N, K, pa, pb))
    return cases


@pytest.mark.parametrize("M,N,K,pa,pb", _s8_sweep_cases())
def test_int8_route_sweep(lib, orc, dev, M, N, K, pa, pb):
    lda, ldb, ldc = K + pa, K + pb, N + 1
    A = u.ints8(orc, M * lda, 1, -128, 127).reshape(M, lda)
    B = u.ints8(orc, N * ldb, 2, -128, 127).reshape(N, ldb)
    dC = torch.full((M, ldc), 5, dtype=torch.int32, device=dev)
    lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, dC, ldc, stream=stream())
    got = host(dC)
    want = (A[:, :K].astype(np.float64) @ B[:, :K].astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got[:, :N].astype(np.int64), want), (M, N, K, pa, pb)
    assert (got[:, N:] == 5).all()


def _dynq_sweep_cases():
    rng = np.random.default_rng(20261205)
    cases = []
    while len(cases) < 12:
        band = len(cases) % 3
        M = int(rng.integers(*((1, 9), (9, 17), (17, 300))[band]))
        N, K = int(rng.integers(1, 2500)), int(rng.integers(1, 2500))
        if M * N * K > 30_000_000:
            continue
        pa, pb = int(rng.integers(0, 5)), int(rng.integers(0, 5))
        alpha = float(rng.choice([1.0, 0.5, -2.0]))
        beta = float(rng.choice([0.0, 1.0, 0.25]))
        cases.append((M, N, K, pa, pb, alpha, beta))
    return cases


@pytest.mark.parametrize("M,N,K,pa,pb,alpha,beta", _dynq_sweep_cases())
def test_int8_dynamic_quant_sweep(lib, orc, dev, M, N, K, pa, pb, alpha, beta):
    """fp32-API gemm_int8 over every int8 route, padded strides (rows off
    16-byte boundaries), assorted alpha / beta: bit-exact with the oracle."""
    lda, ldb, ldc = K + pa, N + pb, N + 3
    A = np.full((M, lda), np.nan, np.float32)
    A[:, :K] = u.normal(orc, M * K, 1, 0, 1.5).reshape(M, K)
    B = np.full((K, ldb), np.nan, np.float32)
    B[:, :N] = u.uniform(orc, K * N, 2).reshape(K, N)
    C0 = u.uniform(orc, M * ldc, 3).reshape(M, ldc)
    Co, Ak, Bn = C0.copy(), np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :N])
    orc.orc_gemm_int8(M, N, K, alpha, u.ptr(Ak), K, u.ptr(Bn), N, beta, u.ptr(Co), ldc)
    dC = dev_copy(C0 if beta != 0.0 else np.where(np.arange(ldc)[None, :] < N, np.nan, C0).astype(np.float32), dev)
    lib.gemm_int8_f32(M, N, K, alpha, dev_copy(A, dev), lda, dev_copy(B, dev), ldb, beta, dC, ldc, stream=stream())
    got = host(dC)
    assert np.array_equal(got[:, :N].view(np.uint32), Co[:, :N].view(np.uint32)), (M, N, K)
    assert np.array_equal(got[:, N:], C0[:, N:]), "wrote outside the C block"


def _wide_sweep_cases():
    """Seeded wide-N, short-K shapes for the streaming kernels (skinny, row-dot,
    int8 row-dot): many column tiles, so the k-split counts per tile vary."""
    rng = np.random.default_rng(20261206)
    cases = []
    while len(cases) < 12:
        kind = ("f32", "f32t", "bf16", "s8")[len(cases) % 4]
        M = int(rng.integers(1, 9 if kind != "f32t" and kind != "s8" else 5))
        N = int(rng.integers(12000, 160000))
        K = int(rng.integers(1, 700))
        if M * N * K > 200_000_000:
            continue
        cases.append((kind, M, N, K))
    return cases


@pytest.mark.parametrize("kind,M,N,K", _wide_sweep_cases())
def test_wide_n_sweep(lib, orc, dev, kind, M, N, K):
    if kind == "s8":
        A = u.ints8(orc, M * K, 1, -128, 127).reshape(M, K)
        B = u.ints8(orc, N * K, 2, -128, 127).reshape(N, K)
        dC = torch.full((M, N), 3, dtype=torch.int32, device=dev)
        lib.gemm_s8s8s32(M, N, K, dev_copy(A, dev), K, dev_copy(B, dev), K, dC, N, stream=stream())
        want = (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int64)
        assert np.array_equal(host(dC).astype(np.int64), want)
        return
    A = u.normal(orc, M * K, 1).reshape(M, K)
    Bkn = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dC = dev_copy(C0, dev)
    if kind == "bf16":
        Ab, Bb = u.bf16_bits(orc, A), u.bf16_bits(orc, Bkn)
        lib.gemm_bf16(M, N, K, 0.5, dev_copy(Ab.view(np.int16), dev), K, dev_copy(Bb.view(np.int16), dev), N, 1.0,
                      dC, N, stream=stream())
        A, Bkn = u.bf16_value(Ab), u.bf16_value(Bb)
    elif kind == "f32t":
        lib.sgemm(M, N, K, 0.5, dev_copy(A, dev), K, dev_copy(np.ascontiguousarray(Bkn.T), dev), K, 1.0, dC, N,
                  transB=1, stream=stream())
    else:
        lib.sgemm(M, N, K, 0.5, dev_copy(A, dev), K, dev_copy(Bkn, dev), N, 1.0, dC, N, stream=stream())
    want, scale = u.exact(A, Bkn, 0.5, 1.0, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"wide {kind} {M}x{N}x{K}")


def _bf16_ex_sweep_cases():
    """Seeded bf16-storage shapes over every bf16 route of dnnopt_hip_gemm_bf16_ex:
    skinny (B stored K x N, A either layout), row-dot and 16 / 32 x 48 tiles (B
    stored N x K), 32 x 64 and 64-row LDS tiles, odd strides (register tiles)."""
    rng = np.random.default_rng(20261207)
    cases = []
    while len(cases) < 16:
        M = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 33)), int(rng.integers(33, 200))]))
        N, K = int(rng.integers(1, 3000)), int(rng.integers(1, 1200))
        if M * N * K > 150_000_000:
            continue
        ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        pa, pb = int(rng.integers(0, 4)), int(rng.integers(0, 4))
        cases.append((M, N, K, ta, tb, pa, pb))
    return cases


@pytest.mark.parametrize("M,N,K,ta,tb,pa,pb", _bf16_ex_sweep_cases())
def test_bf16_ex_route_sweep(lib, orc, dev, M, N, K, ta, tb, pa, pb):
    lda, ldb = (M if ta else K) + pa, (K if tb else N) + pb
    As = u.bf16_bits(orc, u.normal(orc, (K if ta else M) * lda, 1)).reshape(K if ta else M, lda)
    Bs = u.bf16_bits(orc, u.normal(orc, (N if tb else K) * ldb, 2, 0, 0.02)).reshape(N if tb else K, ldb)
    Amk = np.ascontiguousarray(u.bf16_value(As)[:, :M].T if ta else u.bf16_value(As)[:, :K])
    Bkn = np.ascontiguousarray(u.bf16_value(Bs)[:, :K].T if tb else u.bf16_value(Bs)[:, :N])
    C0 = u.uniform(orc, M * N, 3).reshape(M, N)
    dC = dev_copy(C0, dev)
    lib.gemm_bf16_ex(M, N, K, -0.5, dev_copy(As.view(np.int16), dev), lda, dev_copy(Bs.view(np.int16), dev), ldb, 0.75,
                     dC, N, transA=ta, transB=tb, stream=stream())
    want, scale = u.exact(Amk, Bkn, -0.5, 0.75, C0)
    u.assert_fp32_close(host(dC), want, scale, K, f"bf16_ex sweep {M}x{N}x{K} ta={ta} tb={tb} pads={pa},{pb}")
