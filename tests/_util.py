"""Shared helpers of the test suite: library/oracle loading, synthetic inputs,
tolerances.

Tolerances (stated once, used everywhere):

* fp32 and bf16 kernels accumulate in fp32.  For any summation order the
  forward error of a K-term sum is at most gamma_K * sum|a_k b_k| with
  gamma_K ~= K * 2^-24; the epilogue adds at most two more roundings.  A
  result passes when, element-wise,
      |C - C_exact| <= (2K + 4) * 2^-24 * (|alpha| * S + |beta * C0|)
  with S = |A| @ |B| computed in fp64 and C_exact the fp64 product (on the
  bf16-rounded operands for bf16).  This is tighter than the 1e-5 * K scaled
  bound the path is specified with (2 * 2^-24 = 1.2e-7 < 1e-5).
* bf16 against the unrounded fp32 inputs: |C - C_exact| <= 1e-2 * (|alpha| S
  + |beta C0|)  (bf16 rounding of both operands costs at most 2^-7 relative
  per product).
* int8: bit-exact.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")
U = 2.0 ** -24

_bind = None


def binding():
    global _bind
    if _bind is None:
        path = os.path.join(ROOT, "dnn-opt_amd", "python", "dnnopt_hip.py")
        spec = importlib.util.spec_from_file_location("dnnopt_hip", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _bind = mod
    return _bind


def load_lib():
    return binding().load()


P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float

ORACLE_ABI = {
    "orc_mix64": (ctypes.c_uint64, [ctypes.c_uint64]),
    "orc_splitmix64": (None, [ctypes.c_uint64, P, ctypes.c_size_t]),
    "orc_tensor_key": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint32]),
    "orc_fill_uniform_f32": (None, [P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_double,
                                    ctypes.c_double]),
    "orc_fill_normal_f32": (None, [P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_double,
                                   ctypes.c_double]),
    "orc_fill_int8": (None, [P, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint32, I, I]),
    "orc_bf16_rne": (ctypes.c_uint16, [F]),
    "orc_bf16_to_f32": (F, [ctypes.c_uint16]),
    "orc_round_bf16": (None, [P, P, ctypes.c_size_t]),
    "orc_gemm_naive_f32": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_gemv_1xn_f32": (None, [I, I, F, P, P, I, F, P]),
    "orc_smallm_wide_f32": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_adaptive_f32": (None, [I, I, I, F, P, I, P, I, F, P, I, I, I, I]),
    "orc_gemm_f32_smallm": (I, [I, I, I, F, P, I, P, I, F, P, I, I]),
    "orc_gemm_s8s8s32": (None, [I, I, I, P, I, P, I, P, I]),
    "orc_gemm_s8_colscale": (None, [I, I, I, P, I, P, I, P, P, I]),
    "orc_gemm_bf16": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_gemm_int8_dynq": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_gemm_int8_smallm": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_gemm_int8": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "orc_cblas_sgemm": (None, [I, I, I, I, I, I, F, P, I, P, I, F, P, I]),
    "orc_saxpy": (None, [I, F, P, I, P, I, I]),
    "orc_onednn_sgemm": (I, [ctypes.c_char, ctypes.c_char, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, F, P,
                             ctypes.c_int64, P, ctypes.c_int64, F, P, ctypes.c_int64, P]),
    "orc_onednn_gemm_bf16bf16f32": (I, [ctypes.c_char, ctypes.c_char, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, F, P, ctypes.c_int64, P, ctypes.c_int64, F, P,
                                        ctypes.c_int64]),
    "orc_max_threads": (I, []),
}

REF_ABI = {
    "ref_bf16_round": (ctypes.c_uint16, [F]),
    "ref_bf16_widen": (F, [ctypes.c_uint16]),
    "ref_gemm_naive_f32": (None, [I, I, I, F, P, I, P, I, F, P, I]),
    "ref_gemm_s8s8s32": (None, [I, I, I, P, I, P, I, P, I]),
    "ref_saxpy": (None, [I, F, P, I, P, I]),
}


def _bind_table(so, table):
    for name, (res, args) in table.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    return so


def load_oracle():
    if not os.path.exists(ORACLE_SO):
        raise FileNotFoundError(f"{ORACLE_SO} missing: run __graft_entry__.build()")
    return _bind_table(ctypes.CDLL(ORACLE_SO), ORACLE_ABI)


def load_ref():
    if not os.path.exists(REF_SO):
        return None
    # Lazy binding: the AArch64-only paths of the reference stay unresolved
    # and are never called.
    return _bind_table(ctypes.CDLL(REF_SO, mode=os.RTLD_LAZY), REF_ABI)


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------- inputs
SEED = 42
TID_A, TID_B, TID_C, TID_SCALE = 1, 2, 3, 4


def uniform(orc, n, tid, lo=-1.0, hi=1.0, seed=SEED):
    out = np.empty(n, np.float32)
    orc.orc_fill_uniform_f32(ptr(out), n, seed, tid, lo, hi)
    return out


def normal(orc, n, tid, mu=0.0, sigma=1.0, seed=SEED):
    out = np.empty(n, np.float32)
    orc.orc_fill_normal_f32(ptr(out), n, seed, tid, mu, sigma)
    return out


def ints8(orc, n, tid, lo=-127, hi=127, seed=SEED):
    out = np.empty(n, np.int8)
    orc.orc_fill_int8(ptr(out), n, seed, tid, lo, hi)
    return out


def bf16_bits(orc, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    orc.orc_round_bf16(ptr(x), ptr(out), x.size)
    return out


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- reference maths
def exact(A, B, alpha=1.0, beta=0.0, C0=None):
    """fp64 alpha*A@B + beta*C0 and the error scale |alpha| |A|@|B| + |beta C0|."""
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    prod = A64 @ B64
    scale = abs(alpha) * (np.abs(A64) @ np.abs(B64))
    val = alpha * prod
    if beta != 0.0 and C0 is not None:
        val = val + beta * C0.astype(np.float64)
        scale = scale + abs(beta) * np.abs(C0.astype(np.float64))
    return val, scale


def fp32_tol(K, scale):
    return (2 * K + 4) * U * scale + 1e-30


def assert_bits_equal(got, want, what=""):
    """Exact equality (NaNs compared by bit pattern); on failure name the
    mismatching positions so a wrong address pattern is visible."""
    g, w = np.asarray(got, np.float32).reshape(-1), np.asarray(want, np.float32).reshape(-1)
    bad = np.nonzero(g.view(np.uint32) != w.view(np.uint32))[0]
    if bad.size:
        show = ", ".join(f"[{i}] got {g[i]!r} want {w[i]!r}" for i in bad[:12])
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ: {show}")


def assert_fp32_close(got, want, scale, K, what=""):
    got = np.asarray(got, np.float64)
    tol = fp32_tol(K, scale)
    err = np.abs(got - want)
    bad = ~(err <= tol)
    if bad.any():
        idx = np.unravel_index(np.argmax(np.where(bad, err / np.maximum(tol, 1e-300), 0)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} outside (2K+4)u*scale; worst at {idx}: "
            f"got {got[idx]!r} want {want[idx]!r} tol {tol[idx]!r}"
        )
    return float((err / np.maximum(scale, 1e-300)).max())


# ---------------------------------------------------------------- column-major (oneDNN hook) layouts
def cm_store(X: np.ndarray, ld: int, fill=0.0, dtype=np.float32) -> np.ndarray:
    """Column-major storage of X (rows x cols) with leading dimension ld >= rows:
    a flat buffer of cols * ld elements, X[i, j] at [j * ld + i]; the padding
    rows hold `fill`."""
    rows, cols = X.shape
    buf = np.full((cols, ld), fill, dtype)
    buf[:, :rows] = X.T
    return buf.reshape(-1)


def cm_load(buf: np.ndarray, rows: int, cols: int, ld: int) -> np.ndarray:
    return buf.reshape(cols, ld)[:, :rows].T


def hook_operands(opA: np.ndarray, opB: np.ndarray, ta: str, tb: str, pad=0, dtype=np.float32, fill=0.0):
    """Stored A, B (flat column-major buffers) and lda, ldb for op(A) = opA
    (M x K) and op(B) = opB (K x N) under the BLAS letters ta, tb."""
    SA = opA.T if ta in "Tt" else opA
    SB = opB.T if tb in "Tt" else opB
    lda, ldb = SA.shape[0] + pad, SB.shape[0] + pad
    return cm_store(SA, lda, fill, dtype), lda, cm_store(SB, ldb, fill, dtype), ldb


def small_ints(orc, n, tid, lim=3, seed=SEED):
    """Integers in [-lim, lim] as float32 (every product and short sum exact)."""
    return np.rint(uniform(orc, n, tid, -lim - 0.499, lim + 0.499, seed)).astype(np.float32)


# ---------------------------------------------------------------- int8 quantization ties
# The fp32-API int8 path quantizes with lrintf: nearest, ties to even
# (reference: src/gemm/gemm_pack_int8.cpp:66-71).  These operands have
# per-tensor scales 1 (max|A| = 127) and 2 (max|B| = 254, x * 0.5 exact), so
# every quantized value is the rounding of the listed number itself: exact
# ties (0.5, 1.5, 2.5, -0.5, -2.5, -63.5, 62.5) and fractions (63.7), where
# truncation and rounding half away from zero both give other integers.
DYNQ_TIE_A = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 63.7, -63.5, 62.5]
DYNQ_TIE_B = [254.0, 1.0, 3.0, 5.0, -1.0, -5.0, 127.4, -127.0, 125.0]
DYNQ_TIE_Q = [127, 0, 2, 2, 0, -2, 64, -64, 62]


def dynq_tie_cases():
    """(name, M, N, K, A, B, expected C) with A row-major M x K and B K x N,
    alpha = 1, beta = 0.  Every product and sum is an exact small integer, so
    C must equal the expected values bit for bit."""
    q = np.array(DYNQ_TIE_Q, np.float64)
    k = len(DYNQ_TIE_A)
    out = []
    # A's quantization against B = 127 I (scale 1): C[0][j] = 127 q(A[j]).
    A = np.array([DYNQ_TIE_A], np.float32)
    B = (127.0 * np.eye(k)).astype(np.float32)
    out.append(("A ties, scale 1, M=1", 1, k, k, A, B, (127.0 * q)[None, :].astype(np.float32)))
    # 20 rows (past the 16-row MFMA tiles): row i is the tie row rotated by i.
    A = np.stack([np.roll(DYNQ_TIE_A, i) for i in range(20)]).astype(np.float32)
    want = np.stack([np.roll(q, i) for i in range(20)]) * 127.0
    out.append(("A ties, scale 1, M=20", 20, k, k, A, B, want.astype(np.float32)))
    # B's quantization (scale 2) against A = [127] (scale 1): C[0][j] = 2 * 127 q(B[j]).
    A = np.array([[127.0]], np.float32)
    B = np.array([DYNQ_TIE_B], np.float32)
    out.append(("B ties, scale 2, K=1", 1, k, 1, A, B, (254.0 * q)[None, :].astype(np.float32)))
    return out


def check_dynq_ties(gemm_int8_f32):
    """gemm_int8_f32(M, N, K, A, B) -> C (M x N float32).  Raises
    AssertionError naming the first case whose C is not bit-exact."""
    for name, M, N, K, A, B, want in dynq_tie_cases():
        got = np.asarray(gemm_int8_f32(M, N, K, A, B), np.float32).reshape(M, N)
        if not np.array_equal(got, want):
            bad = np.argwhere(got != want)[0]
            raise AssertionError(f"int8 quantization ties ({name}): C{tuple(bad)} = {got[tuple(bad)]}, "
                                 f"want {want[tuple(bad)]}")


# ---------------------------------------------------------------- int8 small-M route (M <= 8)
# The reference's gemm_int8 takes gemm_smallm_int8 for M <= 8
# (src/gemm/gemm.cpp:431-434) and its packed path above.  The two differ in
# the quantizer (x / s against x * (1 / s)) and in the epilogue, and these
# closed forms tell every variant apart:
#   "division": max|B| = 128, s_B = fl(128 / 127); x = 88.18897247314453 has
#     x / s_B = 87.5 exactly in fp32 (quantized 88, ties to even) but
#     x * fl(1 / s_B) = 87.49999 (87) (src/gemm/gemm_smallm_int8.cpp:159,
#     280-281 against src/gemm/gemm_pack_int8.cpp:66-71).  A = [127] (s_A = 1),
#     so C = fl(s_B * 127 q) with q = 127 for the column holding 128.
#   "beta-fma" (scales 1, acc = 1, alpha = 2^-24, beta = fl(1/3), C = 3):
#     beta * C = 1 + 2^-25 exactly.  M = 1 (`result + beta * C[j]`, the
#     beta * C product fused, :170-175): fl(1 + 2^-25 + 2^-24) = 1 + 2^-23.
#     M >= 2 (beta * C rounded to 1 first, :243-250, then C + t acc,
#     :356-383): fl(1 + 2^-24) = 1 (tie, even).  Packed path
#     fma(t, acc, fl(beta C)): 1.
#   "fused-sum" (scales 1, acc = 3, alpha = fl(1/3), beta = 1, C = 2^24):
#     t acc = 1 + 2^-25 exactly, rounded alone to 1.  M = 1 and M >= 2:
#     fl(2^24 + 1) = 2^24 (tie, even); packed path fma(t, acc, C) =
#     fl(2^24 + 1 + 2^-25) = 2^24 + 2.
#   "zero-sign" (acc = 0, alpha = -1, beta = 0): t acc = -0.  M = 1 stores it
#     (-0); M >= 2 stores 0 + (-0) = +0; the packed path stores -0.
DIV_PIN_X = 88.18897247314453
_S128 = np.float32(128.0) / np.float32(127.0)


def int8_route_cases(M):
    """(name, N, K, A (M x K), B (K x N), alpha, beta, C0 (M x N), want)
    for the fp32-API gemm_int8 at M rows; want is the reference's result for
    M's route (M <= 8 small-M, else packed)."""
    small = M <= 8
    f32 = np.float32
    out = []
    A = np.full((M, 1), 127.0, f32)
    B = np.array([[128.0, DIV_PIN_X]], f32)
    q = 88 if small else 87
    want = np.tile(np.array([_S128 * f32(127 * 127), _S128 * f32(127 * q)], f32), (M, 1))
    out.append(("division", 2, 1, A, B, 1.0, 0.0, np.full((M, 2), np.nan, f32), want))
    A = np.tile(np.array([[127.0, 1.0, 0.0]], f32), (M, 1))
    B = np.array([[0.0], [1.0], [127.0]], f32)
    one_third = float(f32(1.0) / f32(3.0))
    w = f32(1.0 + 2.0 ** -23) if M == 1 else f32(1.0)
    out.append(("beta-fma", 1, 3, A, B, 2.0 ** -24, one_third, np.full((M, 1), 3.0, f32), np.full((M, 1), w, f32)))
    B = np.array([[0.0], [3.0], [127.0]], f32)
    w = f32(2.0 ** 24) if small else f32(2.0 ** 24 + 2)
    out.append(("fused-sum", 1, 3, A, B, one_third, 1.0, np.full((M, 1), 2.0 ** 24, f32),
                np.full((M, 1), w, f32)))
    A = np.tile(np.array([[127.0, 0.0]], f32), (M, 1))
    B = np.array([[0.0], [127.0]], f32)
    w = f32(0.0) if (small and M > 1) else f32(-0.0)
    out.append(("zero-sign", 1, 2, A, B, -1.0, 0.0, np.full((M, 1), np.nan, f32), np.full((M, 1), w, f32)))
    return out


def check_int8_routes(gemm_int8_f32, Ms=(1, 2, 3, 5, 7, 8, 9, 20)):
    """gemm_int8_f32(M, N, K, A, B, alpha, beta, C0) -> C (M x N float32).
    Raises AssertionError naming the first case and M whose C differs in any
    bit from the reference's closed form."""
    for M in Ms:
        for name, N, K, A, B, alpha, beta, C0, want in int8_route_cases(M):
            got = np.asarray(gemm_int8_f32(M, N, K, A, B, alpha, beta, C0), np.float32).reshape(M, N)
            if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
                bad = tuple(np.argwhere(got.view(np.uint32) != want.view(np.uint32))[0])
                raise AssertionError(f"int8 route closed form ({name}, M={M}): C{bad} = {got[bad]!r}, "
                                     f"want {want[bad]!r}")
