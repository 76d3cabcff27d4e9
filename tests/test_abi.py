"""C-ABI library checks that need no GPU: it loads, it exports every symbol the
headers declare, the dispatcher's plans are sane, and argument/no-device
errors come back as status codes with C untouched."""

import os
import re
import subprocess

import numpy as np
import pytest

import _util as u

INCLUDE = os.path.join(u.ROOT, "include")


def _c_functions(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{)]*(?:\([^)]*\)[^;{)]*)*\)\s*;", text)
    skip = {"if", "for", "while", "return", "sizeof", "switch"}
    return sorted({n for n in names if n not in skip})


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}


def test_library_loads(lib):
    assert lib.so.dnnopt_hip_abi_version() == u.binding().ABI_VERSION
    hdr = open(os.path.join(u.ROOT, "include", "dnnopt_hip.h")).read()
    m = re.search(r"#define DNNOPT_HIP_ABI_VERSION (\d+)", hdr)
    assert m and int(m.group(1)) == lib.so.dnnopt_hip_abi_version()


def test_every_c_declaration_is_exported(lib):
    exported = _exports(lib.path)
    declared = _c_functions(os.path.join(INCLUDE, "dnnopt_hip.h")) + _c_functions(
        os.path.join(INCLUDE, "dnnopt", "blas", "cblas.h"))
    assert declared, "header parse found nothing"
    missing = [n for n in declared if n not in exported]
    assert not missing, missing
    b = u.binding()
    assert set(declared) == set(b.C_ABI) | set(b.BLAS_ABI)


def test_every_cxx_declaration_is_exported(lib):
    exported = _exports(lib.path)
    b = u.binding()
    for key, (sym, _, _) in b.CXX_ABI.items():
        assert sym in exported, key
    # every dnnopt:: function of the C++ headers has a binding entry
    for hdr in ("gemm/gemm.h", "aligned_alloc.h"):
        names = set(re.findall(r"^\s*(?:void\*?|int)\s+(\w+)\s*\(", open(os.path.join(INCLUDE, "dnnopt", hdr)).read(),
                               re.M))
        for n in names - {"operator"}:
            assert any(k == n or k.startswith(n + "_") for k in b.CXX_ABI), n
    # nothing internal leaks out of the library
    leaked = [s for s in exported if "dnnopt_hip" in s and s.startswith("_Z")]
    assert not leaked, leaked


def test_status_strings(lib):
    b = u.binding()
    for st in range(6):
        assert lib.so.dnnopt_hip_status_string(st)
    assert lib.so.dnnopt_hip_status_string(b.ERR_NO_DEVICE) == b"no HIP device visible"


# ---------------------------------------------------------------- dispatcher
def test_plans_for_the_configs(lib):
    b = u.binding()
    p = lib.plan_sgemm(1, 4096, 4096)
    assert p["kernel"] == b.K_SKINNY_F32 and p["rows"] == 1 and p["splits"] >= 1
    # enough waves for a 256-CU part
    assert p["grid_x"] * p["grid_y"] * p["block"] // 64 >= 1024
    for M in (2, 3, 5, 7):
        for N in (1009, 4099, 11003):
            p = lib.plan_sgemm(M, N, 2048)
            assert p["kernel"] == b.K_SKINNY_F32 and p["rows"] == M
            tiles = -(-N // 256)
            # G >= T workgroups, each tile split G/T or G/T + 1 ways
            G = p["grid_x"]
            assert G >= tiles and p["splits"] == -(-G // tiles) and p["splits"] > 1
            # whole splits per column tile: 256 workgroups rounded up when the last
            # tile is at most a quarter wide, else down (at most a fifth of the CUs idle)
            assert G % tiles == 0, p
            if N - (tiles - 1) * 256 <= 64:
                assert G >= 256, p
            elif N > 4096:
                assert 256 - 256 // 5 <= G <= 256, p
    assert lib.plan_sgemm(65536, 16, 256)["kernel"] == b.K_TALL_F32  # C3 N=16: B resident in LDS
    assert lib.plan_sgemm(65536, 64, 256)["kernel"] == b.K_TALL_F32
    p = lib.plan_sgemm(64, 64, 262144, transA=1)  # C3 split-K: k-major outer-product kernel
    assert p["kernel"] == b.K_TILE_F32 and p["name"] == "dnnopt_kouter_f32" and p["splits"] > 16
    assert (p["rows"], p["cols"], p["block"]) == (64, 64, 256)
    # rows of A not a multiple of 4 floats, M or N <= 32, or a short k: register tiles
    for M, N, K in ((63, 64, 262144), (32, 64, 262144), (64, 32, 262144), (64, 64, 16384)):
        assert lib.plan_sgemm(M, N, K, transA=1)["name"] == "dnnopt_tile_f32", (M, N, K)
    assert lib.plan_sgemm(64, 64, 262144)["name"] == "dnnopt_tile_f32"
    for M in (1, 4):
        assert lib.plan_bf16(M, 11008, 4096)["kernel"] == b.K_SKINNY_BF16
        assert lib.plan_bf16(M, 11008, 4096, fp32_inputs=1)["kernel"] == b.K_SKINNY_F2B
    for M in (32, 256):
        assert lib.plan_bf16(M, 11008, 4096)["kernel"] == b.K_TILE_BF16
    for M in (1, 8, 128):
        for N in (4096, 4093):
            p = lib.plan_s8(M, N, 4096)
            if M <= 4:  # B stored N x K: every row streamed once by the row-dot kernel
                assert p["kernel"] == b.K_ROWDOT_S8 and p["rows"] == M and p["name"] == "dnnopt_rowdot"
            else:
                assert p["kernel"] == b.K_MFMA_S8 and p["rows"] >= min(M, 16)
    for M in (1, 4):
        assert lib.plan_s8(M, 4096, 4096)["kernel"] == b.K_ROWDOT_S8
    for M in (5, 9):
        assert lib.plan_s8(M, 4096, 4096)["kernel"] == b.K_MFMA_S8
    # fp32-API int8: M <= 8 quantizes B as it streams it (fp32 skinny grid)
    for M in (1, 8):
        p = lib.plan_int8_f32(M, 4096, 4096)
        assert p["kernel"] == b.K_SKINNY_Q8 and p["name"] == "dnnopt_skinny_q8" and p["rows"] == M, p
        q = lib.plan_sgemm(M, 4096, 4096)
        with lib.tunables(SPLIT_REDUCE=2):  # the fp32 plan with the reduce kernel: partials only
            r = lib.plan_sgemm(M, 4096, 4096)
        assert (p["grid_x"], p["splits"], p["workspace_bytes"]) == (q["grid_x"], q["splits"], r["workspace_bytes"])
    # M > 8: int8 tiles that quantize the fp32 B while staging it
    for M in (9, 128):
        p = lib.plan_int8_f32(M, 4096, 4096)
        assert p["kernel"] == b.K_MFMA_S8 and p["name"] == "dnnopt_s8_lds_q8b" and (p["rows"], p["cols"]) == (64, 32), p


def test_plan_split_never_exceeds_k(lib):
    for K in (1, 7, 64, 65, 1000):
        for M in (1, 7):
            p = lib.plan_sgemm(M, 4096, K)
            assert p["splits"] <= max(1, K)
        p = lib.plan_sgemm(64, 64, K)
        assert p["splits"] <= max(1, -(-K // 64))


def test_plans_for_weights_stored_n_by_k(lib):
    """M <= 8 with B stored N x K (an inner product's weights) streams the rows
    of B with the row-dot kernel (enough workgroups for two per CU) up to
    M = 4 and for narrow N; from M = 5 at N >= 2048, and for 8 < M <= 32,
    16 x 16 MFMA tiles with k over the 8 waves of a workgroup."""
    b = u.binding()
    for M, N, K in ((1, 4096, 4096), (4, 11003, 2048), (3, 1009, 2048), (8, 5, 7), (7, 1009, 2048)):
        p = lib.plan_sgemm(M, N, K, transB=1)
        assert p["kernel"] == b.K_ROWDOT_F32 and p["name"] == "dnnopt_rowdot", p
        assert p["grid_x"] * p["cols"] >= N
    p = lib.plan_sgemm(4, 11003, 2048, transB=1)
    assert p["grid_x"] >= 256
    for M, N, K in ((5, 4096, 4096), (7, 11003, 2048), (16, 4096, 4096)):
        p = lib.plan_sgemm(M, N, K, transB=1)
        assert p["kernel"] == b.K_TILE_F32 and (p["rows"], p["cols"], p["block"]) == (16, 16, 512), (M, N, p)
    # 16 x 128 tiles (two k-groups of two column waves) above M = 16 with B
    # stored N x K and from M = 9 with B stored K x N, up to M = 32
    for M, tb in ((17, 1), (32, 1), (9, 0), (16, 0), (32, 0)):
        p = lib.plan_sgemm(M, 4096, 4096, transB=tb)
        assert p["kernel"] == b.K_TILE_F32 and (p["rows"], p["cols"], p["block"]) == (16, 128, 256), (M, tb, p)
    # From M = 12 (A stored M x K, N >= 64) the fitted cost models pick the
    # tile and k-split: the register tiles' model where it puts them 10% ahead
    # of the rule, then the LDS-DMA tiles' where theirs puts them 10% ahead of
    # that (measured on MI355X, us): B stored N x K 128 x 768 x 768 16.1 ->
    # 8.6 and 200 x 512 x 512 15.7 -> 6.9 (16 x 16 tiles, k over 8 waves, no
    # split, instead of 64 x 128 with 6 / 4 splits), 196 x 256 x 2304 18.7 ->
    # 9.4 (32 x 64 LDS-DMA tiles of 32-column waves, 8 splits); 128 x 4096 x
    # 4096 77.6 -> 52 (B stored N x K, 32 x 64 LDS-DMA) and 57.7 -> 52 (K x
    # N, 64 x 128 LDS-DMA with 4 splits), 512 x 4096 x 4096 178.3 -> 150 (64
    # x 128 LDS-DMA, 8 waves), 1024 x 1024 x 1024 (B stored N x K) 40.7 ->
    # 23.3; beyond 10^10 MACs the LDS-DMA tiles alone (2048 x 2048 x 2048, B
    # stored N x K, 198.6 -> 134.6).
    cases = {(128, 768, 768, 1): ("", 16, 16, 1, 512), (200, 512, 512, 1): ("", 16, 16, 1, 512),
             (196, 256, 2304, 1): ("_dma", 32, 64, 8, 256), (784, 128, 1152, 0): ("", 16, 16, 1, 512),
             (128, 4096, 4096, 1): ("_dma", 32, 64, 1, 256), (128, 4096, 4096, 0): ("_dma", 64, 128, 4, 512),
             (512, 4096, 4096, 0): ("_dma", 64, 128, 1, 512), (1024, 1024, 1024, 1): ("_dma", 64, 64, 1, 256),
             (2048, 2048, 2048, 1): ("_dma", 64, 128, 1, 512)}
    for (M, N, K, tb), (kind, *want) in cases.items():
        p = lib.plan_sgemm(M, N, K, transB=tb)
        assert p["kernel"] == b.K_TILE_F32 and p["name"] == "dnnopt_tile_f32" + kind, (M, N, K, tb, p)
        assert [p["rows"], p["cols"], p["splits"], p["block"]] == want, (M, N, K, tb, p)
    # the 32-column wave tiles only while 64 x 128 tiles would fill the chip
    # fewer than 4 times (3303 x 3922 x 2969: 1612 such tiles; 32 x 64 tiles
    # measured 763 us against 639 us for 64 x 128 with 2 splits)
    p = lib.plan_sgemm(3303, 3922, 2969, transB=1)
    assert (p["name"], p["rows"], p["cols"], p["splits"], p["block"]) == ("dnnopt_tile_f32_dma", 64, 128, 2, 512), p
    # the LDS-DMA tiles need A stored M x K: A stored K x M keeps the rule
    assert lib.plan_sgemm(2048, 2048, 2048, transA=1)["name"] == "dnnopt_tile_f32"
    # a forced configuration or split count turns the model off
    with lib.tunables(TILE_CFG=2):
        assert (lib.plan_sgemm(128, 768, 768, transB=1)["rows"], lib.plan_sgemm(128, 768, 768, transB=1)["cols"]) == (64, 64)
    with lib.tunables(TILE_SPLITS=3):
        p = lib.plan_sgemm(128, 768, 768, transB=1)
        assert (p["rows"], p["cols"], p["splits"]) == (64, 128, 3), p
    # A stored K x M: 16-row tiles up to M = 16 (B stored N x K) / 32 (K x N)
    for M, tb, rows in ((7, 1, 16), (16, 1, 16), (17, 1, 64), (9, 0, 16), (32, 0, 16), (33, 0, 64)):
        assert lib.plan_sgemm(M, 4096, 4096, transA=1, transB=tb)["rows"] == rows, (M, tb)
    assert lib.plan_bf16_ex(1, 11008, 4096, transB=1)["kernel"] == b.K_ROWDOT_BF16
    assert lib.plan_bf16_ex(4, 11008, 4096, transA=1, transB=1)["kernel"] == b.K_ROWDOT_BF16
    # bf16 storage, B stored K x N: the skinny kernel up to M = 5, the
    # LDS-staged tiles from M = 6 when rows are 4-byte aligned; fp32 inputs and
    # A stored K x M keep the skinny kernel
    for M, name in ((5, "dnnopt_skinny"), (6, "dnnopt_tile_bf16_lds"), (8, "dnnopt_tile_bf16_lds")):
        assert lib.plan_bf16(M, 11008, 4096)["name"] == name, M
        assert lib.plan_bf16_ex(M, 11008, 4096)["name"] == name, M
        assert lib.plan_bf16_ex(M, 11008, 4096, transA=1)["name"] == "dnnopt_skinny", M
        assert lib.plan_bf16(M, 11008, 4096, fp32_inputs=1)["name"] == "dnnopt_skinny", M
    # bf16, B stored N x K, M >= 5 (rows 4-byte aligned): the LDS-staged tiles
    for M in (5, 8):
        assert lib.plan_bf16_ex(M, 11008, 4096, transB=1)["name"] == "dnnopt_tile_bf16_lds"
        assert lib.plan_bf16_ex(M, 11008, 4096, transA=1, transB=1)["name"] == "dnnopt_tile_bf16_lds"
    # transposed A (stored K x M) with B stored N x K stays on the MFMA tiles (fp32)
    assert lib.plan_sgemm(4, 300, 64, transA=1, transB=1)["kernel"] == b.K_TILE_F32
    assert lib.plan_bf16_ex(32, 11008, 4096, transB=1)["name"] == "dnnopt_tile_bf16_lds"


def test_plans_for_tall_skinny(lib):
    """Large M with N <= 64 and B small enough for LDS: the B-resident kernel;
    B too large for LDS or transposed A: the MFMA tiles."""
    b = u.binding()
    for M, N, K in ((65536, 17, 256), (65536, 64, 256), (49153, 20, 512), (100000, 33, 300), (262144, 48, 333)):
        p = lib.plan_sgemm(M, N, K)
        assert p["kernel"] == b.K_TALL_F32 and p["cols"] >= N, p
        assert p["grid_x"] * 4 * 32 >= min(M, p["grid_x"] * 4 * 32)
    assert lib.plan_sgemm(65536, 64, 257)["kernel"] == b.K_TILE_F32   # 272 x 64 x 4 bytes > 64 KiB
    assert lib.plan_sgemm(65536, 64, 256, transA=1)["kernel"] == b.K_TILE_F32
    assert lib.plan_sgemm(1000, 64, 256)["kernel"] == b.K_TILE_F32    # too few rows
    assert lib.plan_sgemm(8192, 64, 256)["kernel"] == b.K_TILE_F32    # fewer row tiles than waves
    p = lib.plan_sgemm(32768, 64, 256)
    assert p["kernel"] == b.K_TALL_F32 and p["rows"] == 16            # 16-row tiles at mid M (K >= 256)
    assert lib.plan_sgemm(32768, 64, 128)["kernel"] == b.K_TILE_F32   # ... but not for short K
    assert lib.plan_sgemm(65536, 64, 256)["rows"] == 16
    assert lib.plan_sgemm(65536, 65, 64)["kernel"] == b.K_TILE_F32
    assert lib.plan_sgemm(65536, 16, 256)["kernel"] == b.K_TALL_F32   # N = 16 with K >= 128: B in LDS
    # K = 64..256 (a multiple of 64) and rows of A a multiple of 16 bytes: A
    # copied into LDS by the memory unit, any N down to 1 and up to 64
    # (except K = 128 with N > 32), 8-wave workgroups
    for M, N, K in ((65536, 16, 256), (65536, 16, 64), (65536, 12, 256), (65536, 1, 256), (131072, 8, 128),
                    (65536, 64, 256), (65536, 32, 128), (65536, 40, 192), (65536, 64, 64)):
        p = lib.plan_sgemm(M, N, K)
        assert (p["kernel"], p["name"], p["block"], p["cols"]) == (
            b.K_TALL_F32, "dnnopt_tall_dma_f32", 512, 16 * -(-N // 16)), (M, N, K, p)
    assert lib.plan_sgemm(65536, 48, 128)["name"] == "dnnopt_tall_f32"
    assert lib.plan_sgemm(65536, 64, 256, transA=1)["kernel"] == b.K_TILE_F32
    assert lib.plan_sgemm_ex(65536, 16, 256, 257, 16, 16)["name"] == "dnnopt_tall_f32"  # rows of A off 16 bytes
    assert lib.plan_sgemm(65536, 16, 100)["kernel"] == b.K_TILE_F32   # short K off the 64 grid: register tiles
    assert lib.plan_sgemm(65536, 12, 300)["kernel"] == b.K_TILE_F32   # N <= 12 off the grid: register tiles


def test_plan_respects_c_row_stride(lib):
    """The B-in-LDS tall kernel stores C through 32-bit offsets from C's first
    element: a row stride that puts ((M - 1) * ldc + N) * 4 at or past 2^31
    routes the GEMM to the tiles, which address C with 64-bit pointers."""
    b = u.binding()
    M, N, K = 65536, 64, 256
    assert lib.plan_sgemm_ex(M, N, K, K, N, N)["kernel"] == b.K_TALL_F32
    assert lib.plan_sgemm_ex(M, N, K, K, N, 8192)["kernel"] == b.K_TALL_F32   # (65535 * 8192 + 64) * 4 < 2^31
    assert lib.plan_sgemm_ex(M, N, K, K, N, 8193)["kernel"] == b.K_TILE_F32   # ... and past it
    assert lib.plan_sgemm_ex(M, N, K, K, N, 16384)["kernel"] == b.K_TILE_F32
    # the stride-free plan is the packed case
    assert lib.plan_sgemm(M, N, K) == lib.plan_sgemm_ex(M, N, K, K, N, N)
    with pytest.raises(b.DnnoptError):
        lib.plan_sgemm_ex(M, N, K, K, N, N - 1)


def test_plan_respects_b_row_stride(lib):
    """The tall kernel stages B through one descriptor with 32-bit offsets:
    ((K - 1) * ldb + N) * 4 at or past 2^31 routes the GEMM to the tiles."""
    b = u.binding()
    M, N, K = 65536, 64, 256
    assert lib.plan_sgemm_ex(M, N, K, K, 2105375, N)["kernel"] == b.K_TALL_F32   # (255 * 2105375 + 64) * 4 < 2^31
    assert lib.plan_sgemm_ex(M, N, K, K, 2105376, N)["kernel"] == b.K_TILE_F32   # ... and past it


def test_plan_rejects_bad_args(lib):
    b = u.binding()
    with pytest.raises(b.DnnoptError):
        lib.plan_sgemm(0, 4, 4)
    with pytest.raises(b.DnnoptError):
        lib.plan_sgemm(4, 4, 4, transA=2)


# ---------------------------------------------------------------- no-device behaviour
no_device = pytest.mark.skipif(u.load_lib().device_count() > 0, reason="a device is visible")


@no_device
def test_c_abi_without_device(lib):
    b = u.binding()
    A = np.ones(16, np.float32)
    C = np.full(16, 7.0, np.float32)
    st = lib.so.dnnopt_hip_sgemm(0, 0, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, C.ctypes.data, 4,
                                 None)
    assert st == b.ERR_NO_DEVICE
    assert (C == 7.0).all()
    # empty problems succeed without touching anything
    assert lib.so.dnnopt_hip_sgemm(0, 0, 0, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None) == b.OK
    assert lib.so.dnnopt_hip_gemm_s8s8s32(4, 4, 0, None, 4, None, 4, None, 4, None) == b.OK
    # invalid arguments are reported before the device is needed
    assert lib.so.dnnopt_hip_sgemm(0, 0, 4, 4, 4, 1.0, A.ctypes.data, 3, A.ctypes.data, 4, 0.0, C.ctypes.data, 4,
                                   None) == b.ERR_INVALID_ARG
    assert lib.so.dnnopt_hip_sgemm(3, 0, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, C.ctypes.data, 4,
                                   None) == b.ERR_INVALID_ARG
    assert lib.so.dnnopt_hip_fill(C.ctypes.data, 16, 2, 0, 1, 1, 0.0, 1.0, None) == b.ERR_INVALID_ARG


@no_device
def test_cxx_and_cblas_api_without_device(lib):
    b = u.binding()
    A = np.ones(16, np.float32)
    C = np.full(16, 7.0, np.float32)
    lib.cxx["gemm_fp32"](4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, C.ctypes.data, 4)
    assert lib.last_status() == b.ERR_NO_DEVICE and (C == 7.0).all()
    lib.cxx["gemm_fp32"](0, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, C.ctypes.data, 4)
    assert lib.last_status() == b.OK
    lib.so.cblas_sgemm(102, 112, 111, 4, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0, C.ctypes.data, 4)
    assert lib.last_status() == b.ERR_NO_DEVICE and (C == 7.0).all()
    # alpha == 0 and beta == 1 returns before anything (cblas_sgemm.cpp:115)
    lib.so.cblas_sgemm(101, 111, 111, 4, 4, 4, 0.0, A.ctypes.data, 4, A.ctypes.data, 4, 1.0, C.ctypes.data, 4)
    assert (C == 7.0).all()


def test_hook_argument_checks(lib):
    """The column-major hook entry points decide these before any device work
    (same answers with or without a GPU)."""
    b = u.binding()
    A = np.ones(64, np.float32)
    C = np.full(64, 7.0, np.float32)
    ext = lambda *a, **k: lib.ext_sgemm(*a, check=False, **k)  # noqa: E731
    # packed operands: unimplemented (the oneDNN side falls back), fp32 only
    assert ext("P", "N", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_UNSUPPORTED
    assert ext("N", "p", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_UNSUPPORTED
    assert lib.onednn_sgemm("P", "N", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_UNSUPPORTED
    # M == 0 or N == 0: nothing, even with null pointers
    assert ext("N", "N", 0, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4) == b.OK
    assert lib.onednn_gemm_bf16bf16f32("N", "N", 4, 0, 4, 1.0, None, 4, None, 4, 0.0, None, 4) == b.OK
    # negative sizes, ldc < 1, short leading dimensions (column-major: lda >= M
    # for 'N', >= K for 'T'), null operands with K > 0
    assert ext("N", "N", -1, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_INVALID_ARG
    assert ext("N", "N", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 0) == b.ERR_INVALID_ARG
    assert ext("N", "N", 4, 4, 4, 1.0, A, 3, A, 4, 0.0, C, 4) == b.ERR_INVALID_ARG
    assert ext("T", "N", 4, 4, 5, 1.0, A, 4, A, 5, 0.0, C, 4) == b.ERR_INVALID_ARG
    assert ext("N", "T", 4, 5, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_INVALID_ARG
    assert ext("N", "N", 4, 4, 4, 1.0, None, 4, A, 4, 0.0, C, 4) == b.ERR_INVALID_ARG
    assert lib.onednn_sgemm("N", "N", 4, 4, 4, 1.0, A, 2, A, 4, 0.0, C, 4) == b.ERR_INVALID_ARG
    # sizes beyond 32 bits
    assert ext("N", "N", 1 << 31, 4, 4, 1.0, A, 1 << 31, A, 4, 0.0, C, 1 << 31) == b.ERR_UNSUPPORTED
    # K == 0 with beta == 1 and no bias changes nothing (no device needed)
    assert lib.onednn_sgemm("N", "N", 4, 4, 0, 1.0, None, 4, None, 1, 1.0, C, 4) == b.OK
    assert (C == 7.0).all()


@no_device
def test_hook_without_device(lib):
    b = u.binding()
    A = np.ones(16, np.float32)
    C = np.full(16, 7.0, np.float32)
    assert lib.ext_sgemm("N", "N", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4, check=False) == b.ERR_NO_DEVICE
    assert lib.onednn_sgemm("T", "N", 4, 4, 4, 1.0, A, 4, A, 4, 0.0, C, 4) == b.ERR_NO_DEVICE
    assert lib.onednn_sgemm("N", "N", 4, 4, 0, 1.0, None, 4, None, 1, 0.0, C, 4) == b.ERR_NO_DEVICE
    assert lib.last_status() == b.ERR_NO_DEVICE and (C == 7.0).all()


def test_thread_setters_round_trip(lib):
    lib.so.openblas_set_num_threads(6)
    assert lib.so.openblas_get_num_threads() == 6
    lib.cxx["gemm_set_num_threads"](3)
    assert lib.cxx["gemm_get_num_threads"]() == 3
    lib.so.blas_set_num_threads(0)
    assert lib.so.openblas_get_num_threads() == 0


def test_aligned_alloc(lib):
    p = lib.cxx["aligned_malloc"](1000, 64)
    assert p and p % 64 == 0
    lib.cxx["aligned_free"](p)
    q = lib.cxx["aligned_malloc_huge"](5 << 20, 64)
    assert q and q % 64 == 0
    lib.cxx["aligned_free_huge"](q, 5 << 20)
    # size 0 gives no block (src/utils/aligned_alloc.cpp:16, :29), and freeing
    # the null pointer is a no-op
    assert not lib.cxx["aligned_malloc"](0, 64)
    assert not lib.cxx["aligned_malloc_huge"](0, 64)
    lib.cxx["aligned_free"](None)


def test_aligned_malloc_zero_matches_reference(ref):
    import ctypes
    fn = getattr(ref, "_ZN6dnnopt14aligned_mallocEmm")
    fn.restype, fn.argtypes = ctypes.c_void_p, [ctypes.c_size_t, ctypes.c_size_t]
    assert fn(0, 64) is None


def test_plans_route_lds_dma_kernels(lib):
    """int8 above M = 16 and bf16 storage above M = 128 copy their operands
    into LDS with the memory unit; the int8 tile is the largest of 64 x 64,
    64 x 32 and 32 x 32 that gives every CU a tile; fp32-input bf16 and
    unaligned operands keep the register-staged kernels."""
    b = u.binding()
    cases = {(128, 4096): (64, 32), (128, 4093): (64, 32), (256, 4096): (64, 64), (128, 8192): (64, 64),
             (32, 4096): (32, 32), (17, 4096): (32, 32)}
    for (M, N), (bm, bn) in cases.items():
        p = lib.plan_s8(M, N, 4096)
        assert p["name"] == "dnnopt_s8_dma" and (p["rows"], p["cols"]) == (bm, bn), (M, N, p)
    assert lib.plan_s8(8, 4096, 4096)["name"] == "dnnopt_mfma_s8"   # M <= 16: register tiles, k over 8 waves
    for M in (129, 256):
        assert lib.plan_bf16(M, 11008, 4096)["name"] == "dnnopt_tile_bf16_dma"
        assert lib.plan_bf16_ex(M, 11008, 4096, transB=1)["name"] == "dnnopt_tile_bf16_dma"
        assert lib.plan_bf16(M, 11008, 4096, fp32_inputs=1)["name"] == "dnnopt_tile_bf16_lds"
    assert lib.plan_bf16(128, 11008, 4096)["name"] == "dnnopt_tile_bf16_lds"
    # bf16 storage above M = 128 (planner's figure of 256 CUs when no GPU is
    # visible): 128 x 96 tiles, 256 x 96 once those take more than one round,
    # and 128 x 128 tiles on 4 waves where the first cost model puts them 5%
    # ahead (measured on MI355X: 256 x 4096 35.7 -> 22.2 us).
    cases = {(256, 11008): (128, 96, 1, 512), (384, 11008): (256, 96, 1, 512), (512, 11008): (256, 96, 1, 512),
             (256, 4096): (128, 128, 4, 256)}
    for (M, N), want in cases.items():
        for p in (lib.plan_bf16(M, N, 4096), lib.plan_bf16_ex(M, N, 4096, transB=1)):
            assert p["name"] == "dnnopt_tile_bf16_dma" and (p["rows"], p["cols"], p["splits"], p["block"]) == want, (M, N, p)
    # bf16 storage from M = 12: the second model's tile and split where it
    # puts them 10% ahead (measured on MI355X, us, before -> after, B stored
    # K x N): 384 x 8192 x 4096 49.4 -> 42.5 and 1024 x 4096 x 4096 51.0 ->
    # 44.1 (128 x 128 on 8 waves), 512 x 2048 x 4096 22.8 -> 21.1 (8 waves,
    # 4 splits), 200 x 512 x 512 8.5 -> 5.5 (32 x 64 unsplit instead of 128 x
    # 96 with 4 splits); B stored N x K 200 x 512 x 512 8.3 -> 5.1 and 32 x
    # 768 x 768 7.3 -> 5.7 (16 x 48 unsplit).  C4's shapes keep their tiles.
    cases = {(384, 8192, 4096, 0): ("dma", 128, 128, 1, 512), (1024, 4096, 4096, 0): ("dma", 128, 128, 1, 512),
             (512, 2048, 4096, 0): ("dma", 128, 128, 4, 512), (200, 512, 512, 0): ("lds", 32, 64, 1, 256),
             (200, 512, 512, 1): ("lds", 16, 48, 1, 192), (32, 768, 768, 1): ("lds", 16, 48, 1, 192),
             (32, 11008, 4096, 0): ("lds", 32, 64, 1, 256), (32, 11008, 4096, 1): ("lds", 32, 48, 1, 192)}
    for (M, N, K, tb), (kind, *want) in cases.items():
        p = lib.plan_bf16_ex(M, N, K, transB=tb)
        assert p["name"] == "dnnopt_tile_bf16_" + kind and [p["rows"], p["cols"], p["splits"], p["block"]] == want, (
            M, N, K, tb, p)
    # fp32 inputs: the first model (M > 64) between 128 x 96 and 256 x 96
    # register-ring tiles, then the second (from M = 12) over every
    # LDS-staged tile and split, each where 5% ahead (measured on MI355X, us,
    # before -> after: 512 x 11008 x 4096 145.7 -> 121.5 and 384 x 11008 x
    # 1024 48.6 -> 37.9 on 256 x 96; 512 x 4096 x 4096 78.4 -> 66.3 (64 x 128,
    # unsplit), 256 x 4096 x 4096 47.6 -> 41.5 (64 x 128, 2 splits), 96 x
    # 4096 x 1024 17.4 -> 14.3 (32 x 64, unsplit)); C4f's M = 256 keeps
    # 128 x 96; unaligned strides change nothing.
    cases = {(96, 4096, 1024): (32, 64, 1), (256, 4096, 4096): (64, 128, 2), (512, 4096, 4096): (64, 128, 1),
             (256, 11008, 4096): (128, 96, 1), (384, 11008, 1024): (256, 96, 1), (512, 11008, 4096): (256, 96, 1),
             (1024, 4096, 4096): (256, 96, 1)}
    for (M, N, K), want in cases.items():
        p = lib.plan_bf16(M, N, K, fp32_inputs=1)
        assert p["name"] == "dnnopt_tile_bf16_lds" and (p["rows"], p["cols"], p["splits"]) == want, (M, N, K, p)
    with lib.tunables(TILE_CFG=40, TILE_SPLITS=3):
        p = lib.plan_bf16(300, 1000, 520, fp32_inputs=1)
        assert (p["name"], p["rows"], p["cols"], p["splits"]) == ("dnnopt_tile_bf16_lds", 256, 96, 3), p
    # a forced tile or split count turns the model off
    with lib.tunables(TILE_SPLITS=2):
        assert (lib.plan_bf16(256, 4096, 4096)["rows"], lib.plan_bf16(256, 4096, 4096)["cols"]) == (128, 96)
