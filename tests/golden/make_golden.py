"""Write tests/golden/oracle_golden.npz.

Run in the development container, where oracle/_ref (the reference's own
gemm.cpp and gemm_int8_native.cpp built for x86) exists:

    python tests/golden/make_golden.py

Expected outputs of the "naive" and "s8" cases come from the reference build
(GemmAlgo::kNaive and the native int8 scalar loop); the "smallm" cases record
the oracle's order-faithful restatement of the NEON small-M kernels (the
reference cannot run those here) as regression fixtures.  Inputs are the
seeded SplitMix64 streams of tests/_util.py, stored alongside.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _util as u  # noqa: E402


def main():
    orc = u.load_oracle()
    ref = u.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libref.so is needed (build oracle/ with the reference present)")
    out = {}

    def put(name, kind, M, N, K, alpha, beta, A, B, C0, C):
        out[name + "_kind"] = np.array(kind)
        out[name + "_meta"] = np.array([M, N, K, alpha, beta], np.float64)
        out[name + "_A"], out[name + "_B"] = A, B
        if C0 is not None:
            out[name + "_C0"] = C0
        out[name + "_C"] = C

    for i, (M, N, K, alpha, beta) in enumerate([(7, 13, 5, 1.0, 0.0), (3, 3, 400, 2.5, -0.3),
                                                 (1, 67, 129, 1.0, 1.0), (13, 17, 19, 1.0, 0.5)]):
        A, B, C0 = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2), u.uniform(orc, M * N, 3)
        C = C0.copy()
        ref.ref_gemm_naive_f32(M, N, K, alpha, u.ptr(A), K, u.ptr(B), N, beta, u.ptr(C), N)
        put(f"naive{i}", "naive", M, N, K, alpha, beta, A, B, C0, C)

    for i, (M, N, K) in enumerate([(1, 13, 300), (9, 4093 % 37, 77), (8, 8, 512)]):
        A, B = u.ints8(orc, M * K, 1), u.ints8(orc, N * K, 2)
        C = np.empty(M * N, np.int32)
        ref.ref_gemm_s8s8s32(M, N, K, u.ptr(A), K, u.ptr(B), K, u.ptr(C), N)
        put(f"s8_{i}", "s8", M, N, K, 0.0, 0.0, A, B, None, C)

    for i, (M, N, K) in enumerate([(1, 101, 257), (2, 67, 130), (3, 53, 96), (5, 4099 % 200, 700),
                                   (7, 19, 1300)]):
        A = u.normal(orc, M * K, 1, 0, 0.02)
        B = u.normal(orc, K * N, 2, 0, 0.02)
        C0 = u.uniform(orc, M * N, 3)
        C = C0.copy()
        # Force the adaptive-tile route for the M = 5, 7 cases the way the
        # reference does above N*K = 4Mi: call the adaptive restatement.
        if M in (5, 7):
            orc.orc_adaptive_f32(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 1.0, u.ptr(C), N, 5 if M == 5 else 6,
                                 65536, 1)
            kind = "adaptive"
        else:
            assert orc.orc_gemm_f32_smallm(M, N, K, 1.0, u.ptr(A), K, u.ptr(B), N, 1.0, u.ptr(C), N, 1) == 0
            kind = "smallm"
        put(f"{kind}{i}", kind, M, N, K, 1.0, 1.0, A, B, C0, C)

    path = os.path.join(HERE, "oracle_golden.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
