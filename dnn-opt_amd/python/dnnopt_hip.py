"""ctypes binding of libdnnopt_blas.so (the gfx950 small/irregular GEMM path).

Host-side mirror of the reference's operator interface for this path:

* ``gemm_fp32 / gemm_bf16 / gemm_bf16_bf16bf16f32 / gemm_int8 /
  gemm_int8_int8int8int32`` keep the reference's names and argument meaning
  (``include/dnnopt/gemm/gemm.h:14-58`` of the reference) and take host numpy
  arrays or device pointers, synchronously.
* ``cblas_sgemm`` / ``sgemm_`` / ``cblas_saxpy`` are the BLAS entry points
  (``include/dnnopt/blas/cblas.h:29-50``).
* ``onednn_sgemm`` / ``onednn_gemm_bf16bf16f32`` are the column-major oneDNN
  hook entry points (``integration/onednn/0001-dnnopt-integration.patch:279-370,
  573-630``), with the hook's argument list (scalars by pointer).
* ``Lib.sgemm``, ``Lib.gemm_bf16`` ... call the stream-ordered C-ABI of
  ``include/dnnopt_hip.h`` on device pointers and raise ``DnnoptError`` on a
  non-zero status.

The library is loaded from this package's ``lib/`` directory; a missing
library raises instead of falling back to anything else.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, c_char, c_double, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint32, c_uint64,
                    c_void_p)

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# DNNOPT_HIP_LIB selects another build of the library (e.g. a variant built
# with different compile-time tunables); the default is this package's lib/.
LIB_PATH = os.environ.get("DNNOPT_HIP_LIB") or os.path.join(PKG_DIR, "lib", "libdnnopt_blas.so")

OK, ERR_INVALID_ARG, ERR_NO_DEVICE, ERR_HIP, ERR_UNSUPPORTED, ERR_OUT_OF_MEMORY, ERR_SCRATCH_LIMIT = range(7)
NOALLOC_SCRATCH_BYTES = 16 << 20  # DNNOPT_NOALLOC_SCRATCH_BYTES

(K_NONE, K_SKINNY_F32, K_SKINNY_BF16, K_SKINNY_F2B, K_MFMA_S8, K_TILE_F32, K_TILE_BF16, K_NAIVE_F32, K_ROWDOT_F32,
 K_ROWDOT_BF16, K_TALL_F32, K_ROWDOT_S8, K_SKINNY_Q8, K_WIDE) = range(14)

# DNNOPT_HIP_ABI_VERSION of include/dnnopt_hip.h that these bindings follow.
ABI_VERSION = 4

CblasRowMajor, CblasColMajor = 101, 102
CblasNoTrans, CblasTrans, CblasConjTrans = 111, 112, 113


class DnnoptError(RuntimeError):
    def __init__(self, status: int, what: str, text: str):
        super().__init__(f"{what}: status {status} ({text})")
        self.status = status


class Plan(ctypes.Structure):
    _fields_ = [
        ("kernel", c_int),
        ("rows", c_int),
        ("cols", c_int),
        ("splits", c_int),
        ("grid_x", c_int),
        ("grid_y", c_int),
        ("grid_z", c_int),
        ("block", c_int),
        ("workspace_bytes", c_size_t),
        ("name", c_char * 64),
    ]

    def as_dict(self):
        return {f: (getattr(self, f).decode() if f == "name" else getattr(self, f)) for f, _ in self._fields_}


_F = c_float
_I = c_int
_P = c_void_p
_L = c_int64
_C = c_char

# name -> (restype, argtypes); every symbol declared in include/dnnopt_hip.h
# and the BLAS header, so a test can check the export list against this.
C_ABI = {
    "dnnopt_hip_sgemm": (_I, [_I, _I, _I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_sgemm_noalloc": (_I, [_I, _I, _I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_sgemm_naive": (_I, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_gemm_bf16": (_I, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_gemm_bf16_ex": (_I, [_I, _I, _I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_gemm_bf16_f32in": (_I, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_gemm_s8s8s32": (_I, [_I, _I, _I, _P, _I, _P, _I, _P, _I, _P]),
    "dnnopt_hip_gemm_s8s8f32_colscale": (_I, [_I, _I, _I, _P, _I, _P, _I, _P, _P, _I, _P]),
    "dnnopt_hip_gemm_int8_f32": (_I, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _P]),
    "dnnopt_hip_saxpy": (_I, [_I, _F, _P, _I, _P, _I, _P]),
    "dnnopt_hip_ext_sgemm": (_I, [_C, _C, _L, _L, _L, _F, _P, _L, _P, _L, _F, _P, _L, _P, _P]),
    "dnnopt_hip_ext_gemm_bf16bf16f32": (_I, [_C, _C, _L, _L, _L, _F, _P, _L, _P, _L, _F, _P, _L, _P]),
    "dnnopt_onednn_sgemm": (_I, [_P] * 14),
    "dnnopt_onednn_gemm_bf16bf16f32": (_I, [_P] * 13),
    "dnnopt_hip_plan_sgemm": (_I, [_I, _I, _I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_plan_sgemm_ex": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_plan_gemm_bf16": (_I, [_I, _I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_plan_gemm_bf16_ex": (_I, [_I, _I, _I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_plan_gemm_s8": (_I, [_I, _I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_plan_gemm_int8_f32": (_I, [_I, _I, _I, POINTER(Plan)]),
    "dnnopt_hip_fill": (_I, [_P, c_size_t, _I, _I, c_uint64, c_uint32, c_double, c_double, _P]),
    "dnnopt_hip_status_string": (ctypes.c_char_p, [_I]),
    "dnnopt_hip_last_status": (_I, []),
    "dnnopt_hip_device_count": (_I, []),
    "dnnopt_hip_abi_version": (_I, []),
    "dnnopt_hip_set_tunable": (_I, [_I, _I, POINTER(ctypes.c_int)]),
    "dnnopt_hip_get_tunable": (_I, [_I, POINTER(ctypes.c_int)]),
}

# Keys of dnnopt_hip_set_tunable (include/dnnopt_hip.h DNNOPT_TUNE_*).
TUNE = {"Q8B": 0, "KOUTER": 1, "KOUTER_WGS_PER_CU": 2, "WAVES_PER_CU": 3, "SKINNY_NW": 4,
        "SKINNY_WGS_PER_CU": 5, "MAX_SPLITS": 6, "SPLIT_REDUCE": 7, "SKINNY_WGS": 8, "TILE_SPLITS": 9,
        "TILE_CFG": 10, "TILE_TICKET": 11, "S8_CFG": 12, "S8_ROWDOT": 13, "S8_SPLITS": 14, "ROWDOT_KW": 15,
        "TALL_RT": 16, "TALL_WGS_PER_CU": 17, "TALL": 18, "WIDE": 19}

BLAS_ABI = {
    "cblas_sgemm": (None, [_I, _I, _I, _I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I]),
    "cblas_saxpy": (None, [_I, _F, _P, _I, _P, _I]),
    "sgemm_": (None, [_P] * 13),
    "SGEMM": (None, [_P] * 13),
    "openblas_set_num_threads": (None, [_I]),
    "openblas_get_num_threads": (_I, []),
    "blas_set_num_threads": (None, [_I]),
    "omp_set_num_threads_blas": (None, [_I]),
}

# Itanium-mangled names of the C++ API (include/dnnopt/gemm/gemm.h,
# include/dnnopt/aligned_alloc.h), all with void or int results.
CXX_ABI = {
    "gemm_fp32": ("_ZN6dnnopt9gemm_fp32EiiifPKfiS1_ifPfi", None, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I]),
    "gemm_fp32_algo": (
        "_ZN6dnnopt9gemm_fp32EiiifPKfiS1_ifPfiNS_8GemmAlgoE",
        None,
        [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I, _I],
    ),
    "gemm_bf16": ("_ZN6dnnopt9gemm_bf16EiiifPKfiS1_ifPfi", None, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I]),
    "gemm_bf16_bf16bf16f32": (
        "_ZN6dnnopt21gemm_bf16_bf16bf16f32EiiifPKNS_10bfloat16_tEiS2_ifPfi",
        None,
        [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I],
    ),
    "gemm_int8": ("_ZN6dnnopt9gemm_int8EiiifPKfiS1_ifPfi", None, [_I, _I, _I, _F, _P, _I, _P, _I, _F, _P, _I]),
    "gemm_int8_int8int8int32": (
        "_ZN6dnnopt23gemm_int8_int8int8int32EiiiPKaiS1_iPii",
        None,
        [_I, _I, _I, _P, _I, _P, _I, _P, _I],
    ),
    "gemm_set_num_threads": ("_ZN6dnnopt20gemm_set_num_threadsEi", None, [_I]),
    "gemm_get_num_threads": ("_ZN6dnnopt20gemm_get_num_threadsEv", _I, []),
    "aligned_malloc": ("_ZN6dnnopt14aligned_mallocEmm", _P, [c_size_t, c_size_t]),
    "aligned_free": ("_ZN6dnnopt12aligned_freeEPv", None, [_P]),
    "aligned_malloc_huge": ("_ZN6dnnopt19aligned_malloc_hugeEmm", _P, [c_size_t, c_size_t]),
    "aligned_free_huge": ("_ZN6dnnopt17aligned_free_hugeEPvm", None, [_P, c_size_t]),
}

GEMM_ALGO = {"kAuto": 0, "kNaive": 1, "kNeonFp32": 2}


def _ptr(x):
    """Device or host address of a torch tensor, numpy array or int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)!r}")


def _share_torch_hip_runtime():
    """When PyTorch-ROCm is installed, initialise its HIP runtime first.

    The torch wheel ships its own libamdhip64 under the same soname as the
    system one this library links.  Whichever copy a process loads first is
    the one every later library binds to; loading the system copy first
    leaves torch with a second, device-less runtime.  Letting torch go first
    gives the process a single HIP runtime shared by torch tensors (device
    memory, streams) and these kernels.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        return
    try:
        torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch without a usable backend
        pass


class Lib:
    """Loaded libdnnopt_blas.so with typed entry points."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build() or make -C dnn-opt_amd")
        self.path = path
        _share_torch_hip_runtime()
        self.so = ctypes.CDLL(path)
        for table in (C_ABI, BLAS_ABI):
            for name, (res, args) in table.items():
                fn = getattr(self.so, name)
                fn.restype = res
                fn.argtypes = args
        self.cxx = {}
        for key, (sym, res, args) in CXX_ABI.items():
            fn = getattr(self.so, sym)
            fn.restype = res
            fn.argtypes = args
            self.cxx[key] = fn

    # ---------------------------------------------------------------- status
    def _check(self, st: int, what: str):
        if st != OK:
            raise DnnoptError(st, what, self.so.dnnopt_hip_status_string(st).decode())

    def device_count(self) -> int:
        return self.so.dnnopt_hip_device_count()

    def last_status(self) -> int:
        return self.so.dnnopt_hip_last_status()

    # ---------------------------------------------------------------- tunables
    def set_tunable(self, name: str, value: int) -> int:
        """Set one dispatcher tunable (TUNE key name); returns the old value."""
        old = ctypes.c_int(0)
        self._check(self.so.dnnopt_hip_set_tunable(TUNE[name], int(value), ctypes.byref(old)), "set_tunable")
        return old.value

    def get_tunable(self, name: str) -> int:
        v = ctypes.c_int(0)
        self._check(self.so.dnnopt_hip_get_tunable(TUNE[name], ctypes.byref(v)), "get_tunable")
        return v.value

    def tunables(self, **values):
        """Context manager: set tunables for the enclosed calls, then restore them."""
        lib = self

        class _Ctx:
            def __enter__(self):
                self.old = {k: lib.set_tunable(k, v) for k, v in values.items()}
                return lib

            def __exit__(self, *exc):
                for k, v in self.old.items():
                    lib.set_tunable(k, v)
                return False

        return _Ctx()

    # ---------------------------------------------------------------- plans
    def plan_sgemm(self, M, N, K, transA=0, transB=0) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_sgemm(transA, transB, M, N, K, ctypes.byref(p)), "plan_sgemm")
        return p.as_dict()

    def plan_sgemm_ex(self, M, N, K, lda, ldb, ldc, transA=0, transB=0) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_sgemm_ex(transA, transB, M, N, K, lda, ldb, ldc, ctypes.byref(p)),
                    "plan_sgemm_ex")
        return p.as_dict()

    def plan_bf16(self, M, N, K, fp32_inputs=0) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_gemm_bf16(fp32_inputs, M, N, K, ctypes.byref(p)), "plan_bf16")
        return p.as_dict()

    def plan_bf16_ex(self, M, N, K, transA=0, transB=0) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_gemm_bf16_ex(transA, transB, M, N, K, ctypes.byref(p)), "plan_bf16_ex")
        return p.as_dict()

    def plan_s8(self, M, N, K, with_scale=0) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_gemm_s8(with_scale, M, N, K, ctypes.byref(p)), "plan_s8")
        return p.as_dict()

    def plan_int8_f32(self, M, N, K) -> dict:
        p = Plan()
        self._check(self.so.dnnopt_hip_plan_gemm_int8_f32(M, N, K, ctypes.byref(p)), "plan_int8_f32")
        return p.as_dict()

    # ---------------------------------------------------------------- C-ABI (device pointers)
    def sgemm(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, transA=0, transB=0, stream=None):
        self._check(
            self.so.dnnopt_hip_sgemm(transA, transB, M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
                                     stream),
            "dnnopt_hip_sgemm",
        )

    def sgemm_noalloc(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, transA=0, transB=0, stream=None) -> int:
        """dnnopt_hip_sgemm_noalloc; returns the status (the caller checks it:
        ERR_SCRATCH_LIMIT is an expected outcome for large split-k plans)."""
        return self.so.dnnopt_hip_sgemm_noalloc(transA, transB, M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta,
                                                _ptr(C), ldc, stream)

    def sgemm_naive(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_sgemm_naive(M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc, stream),
            "dnnopt_hip_sgemm_naive",
        )

    def gemm_bf16(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_bf16(M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc, stream),
            "dnnopt_hip_gemm_bf16",
        )

    def gemm_bf16_ex(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, transA=0, transB=0, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_bf16_ex(transA, transB, M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta,
                                            _ptr(C), ldc, stream),
            "dnnopt_hip_gemm_bf16_ex",
        )

    def ext_sgemm(self, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias=None, stream=None,
                  check=True):
        """Column-major oneDNN hook on device pointers; returns the status."""
        st = self.so.dnnopt_hip_ext_sgemm(_char(transa), _char(transb), M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb,
                                          beta, _ptr(C), ldc, _ptr(bias), stream)
        if check:
            self._check(st, "dnnopt_hip_ext_sgemm")
        return st

    def ext_gemm_bf16bf16f32(self, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None,
                             check=True):
        st = self.so.dnnopt_hip_ext_gemm_bf16bf16f32(_char(transa), _char(transb), M, N, K, alpha, _ptr(A), lda,
                                                     _ptr(B), ldb, beta, _ptr(C), ldc, stream)
        if check:
            self._check(st, "dnnopt_hip_ext_gemm_bf16bf16f32")
        return st

    def onednn_sgemm(self, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias=None):
        """The hook's own argument list (scalars by pointer); host or device
        memory, synchronous.  Returns the status."""
        sc = _HookScalars(transa, transb, M, N, K, alpha, lda, ldb, beta, ldc)
        return self.so.dnnopt_onednn_sgemm(*sc.head(), _ptr(A), sc.ref("lda"), _ptr(B), sc.ref("ldb"),
                                           sc.ref("beta"), _ptr(C), sc.ref("ldc"), _ptr(bias))

    def onednn_gemm_bf16bf16f32(self, transa, transb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc):
        sc = _HookScalars(transa, transb, M, N, K, alpha, lda, ldb, beta, ldc)
        return self.so.dnnopt_onednn_gemm_bf16bf16f32(*sc.head(), _ptr(A), sc.ref("lda"), _ptr(B), sc.ref("ldb"),
                                                      sc.ref("beta"), _ptr(C), sc.ref("ldc"))

    def gemm_bf16_f32in(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_bf16_f32in(M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
                                               stream),
            "dnnopt_hip_gemm_bf16_f32in",
        )

    def gemm_s8s8s32(self, M, N, K, A, lda, B, ldb, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_s8s8s32(M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C), ldc, stream),
            "dnnopt_hip_gemm_s8s8s32",
        )

    def gemm_s8s8f32_colscale(self, M, N, K, A, lda, B, ldb, scale, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_s8s8f32_colscale(M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(scale), _ptr(C),
                                                     ldc, stream),
            "dnnopt_hip_gemm_s8s8f32_colscale",
        )

    def gemm_int8_f32(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream=None):
        self._check(
            self.so.dnnopt_hip_gemm_int8_f32(M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
                                             stream),
            "dnnopt_hip_gemm_int8_f32",
        )

    def saxpy(self, N, alpha, X, incX, Y, incY, stream=None):
        self._check(self.so.dnnopt_hip_saxpy(N, alpha, _ptr(X), incX, _ptr(Y), incY, stream), "dnnopt_hip_saxpy")

    def fill(self, dst, n, dtype, dist, seed, tensor_id, p0, p1, stream=None):
        """dtype: 0 fp32, 1 bf16, 2 int8; dist: 0 uniform, 1 normal, 2 integer."""
        self._check(self.so.dnnopt_hip_fill(_ptr(dst), n, dtype, dist, seed, tensor_id, p0, p1, stream),
                    "dnnopt_hip_fill")

    # ---------------------------------------------------------------- reference API (host or device)
    def gemm_fp32(self, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, algo=None):
        if algo is None:
            self.cxx["gemm_fp32"](M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc)
        else:
            self.cxx["gemm_fp32_algo"](M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
                                       GEMM_ALGO.get(algo, algo))
        self._check(self.last_status(), "dnnopt::gemm_fp32")

    def cblas_sgemm(self, order, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc):
        self.so.cblas_sgemm(order, ta, tb, M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc)
        self._check(self.last_status(), "cblas_sgemm")


def _char(c):
    return c.encode() if isinstance(c, str) else bytes([c]) if isinstance(c, int) else c


class _HookScalars:
    """The scalars of a hook call kept alive as ctypes objects (the hook
    takes every scalar by pointer, as oneDNN's extended_sgemm passes them)."""

    def __init__(self, transa, transb, M, N, K, alpha, lda, ldb, beta, ldc):
        self.v = {
            "transa": c_char(_char(transa)), "transb": c_char(_char(transb)),
            "M": c_int64(M), "N": c_int64(N), "K": c_int64(K), "alpha": c_float(alpha),
            "lda": c_int64(lda), "ldb": c_int64(ldb), "beta": c_float(beta), "ldc": c_int64(ldc),
        }

    def ref(self, k):
        return ctypes.cast(ctypes.byref(self.v[k]), c_void_p)

    def head(self):
        return [self.ref(k) for k in ("transa", "transb", "M", "N", "K", "alpha")]


_LIB = None


def load(path: str = LIB_PATH) -> Lib:
    """The process-wide library instance."""
    global _LIB
    if _LIB is None or _LIB.path != path:
        _LIB = Lib(path)
    return _LIB
