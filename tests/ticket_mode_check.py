"""Child process of test_gpu_hook.py::test_ticket_reduction_mode (not a test
module): run k-split shapes of the fp32 skinny and tile kernels and of the
oneDNN hook (with bias) under the environment the parent set
(DNNOPT_SPLIT_REDUCE=0: the last-arriving workgroup reduces the splits) and
compare with the fp64 closed form."""

import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import _util as u  # noqa: E402

import torch  # noqa: E402


def main():
    assert os.environ.get("DNNOPT_SPLIT_REDUCE") == "0"
    lib, orc = u.load_lib(), u.load_oracle()
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream

    def dcopy(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def host(t):
        torch.cuda.synchronize()
        return t.cpu().numpy()

    # row-major fp32: skinny with k-splits, tiles with k-splits
    # (tiles take the ticket path up to 16 splits, the skinny kernel always)
    for M, N, K in ((1, 4096, 4096), (7, 1009, 2048), (3, 257, 5000), (1024, 256, 1024), (300, 600, 2048)):
        p = lib.plan_sgemm(M, N, K)
        assert p["splits"] > 1 and (M <= 8 or p["splits"] <= 16), (M, N, K, p)
        A, B, C0 = u.normal(orc, M * K, 1), u.normal(orc, K * N, 2, 0, 0.02), u.uniform(orc, M * N, 3)
        dC = dcopy(C0)
        lib.sgemm(M, N, K, 1.0, dcopy(A), K, dcopy(B), N, 1.0, dC, N, stream=s)
        want, scale = u.exact(A.reshape(M, K), B.reshape(K, N), 1.0, 1.0, C0.reshape(M, N))
        u.assert_fp32_close(host(dC).reshape(M, N), want, scale, K, f"ticket sgemm {M}x{N}x{K}")
        print(f"sgemm {M}x{N}x{K} splits={p['splits']} ok", flush=True)
    # column-major hook with bias: skinny (transa 'N') and tiles with k-splits
    for M, N, K, ta in ((4099, 3, 2048, "N"), (256, 1024, 1024, "N"), (256, 1024, 1024, "T")):
        opA = u.normal(orc, M * K, 1).reshape(M, K)
        opB = u.normal(orc, K * N, 2, 0, 0.02).reshape(K, N)
        A, lda, B, ldb = u.hook_operands(opA, opB, ta, "N")
        C0 = u.uniform(orc, M * N, 3).reshape(M, N)
        bias = u.uniform(orc, M, 4)
        dC = dcopy(u.cm_store(C0, M))
        lib.ext_sgemm(ta, "N", M, N, K, 1.0, dcopy(A), lda, dcopy(B), ldb, 0.5, dC, M, bias=dcopy(bias), stream=s)
        want, scale = u.exact(opA, opB, 1.0, 0.5, C0)
        u.assert_fp32_close(u.cm_load(host(dC), M, N, M), want + bias[:, None], scale + np.abs(bias)[:, None], K + 1,
                            f"ticket hook {ta} {M}x{N}x{K}")
        print(f"hook {ta} {M}x{N}x{K} ok", flush=True)
    print("ticket mode ok", flush=True)


if __name__ == "__main__":
    main()
