"""Host-side contract of bench.py (no GPU needed): the multi-GPU refusal,
the algorithmic byte and flop counts the roofline is priced on, and the
committed HBM-traffic figures the roofline's `traffic` field reads."""

import glob
import json
import os
import subprocess
import sys

import pytest

import _util as u

sys.path.insert(0, u.ROOT)
import bench  # noqa: E402

# C1..C5 and the oneDNN-hook workload.
WORKLOADS = ["c1", "c2", "c3", "c4", "c4f", "c5", "c5f", "hook"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(u.ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("wl", WORKLOADS)
def test_algorithmic_counts(wl):
    """bytes = sA*M*K + sB*K*N + 4*M*N*(1 + [beta != 0]) (+ 4*N for a column
    scale or bias), flops = 2*M*N*K, with the element sizes of each kind."""
    size = {"f32": (4, 4), "bf16": (2, 2), "f2b": (4, 4), "s8": (1, 1), "s8s": (1, 1), "hf32": (4, 4), "hbf16": (2, 2),
            "i8f": (4, 4)}
    _, cases = bench.workload(wl)
    assert cases
    for c in cases:
        sa, sb = size[c.kind]
        extra = 4 * c.N if c.kind == "s8s" or (c.kind == "hf32" and c.init.get("bias")) else 0
        want = sa * c.M * c.K + sb * c.K * c.N + 4 * c.M * c.N * (2 if c.beta != 0.0 else 1) + extra
        assert c.bytes_alg() == want, c.name
        assert c.flops_alg() == 2.0 * c.M * c.N * c.K


def test_config_shapes_match_the_baseline():
    shapes = {wl: {(c.M, c.N, c.K) for c in bench.workload(wl)[1]} for wl in WORKLOADS}
    assert shapes["c1"] == {(1, 4096, 4096)}
    assert shapes["c2"] == {(m, n, 2048) for m in (2, 3, 5, 7) for n in (1009, 4099, 11003)}
    assert shapes["c3"] == {(65536, 16, 256), (65536, 64, 256), (64, 64, 262144)}
    assert shapes["c4"] == {(m, 11008, 4096) for m in (1, 4, 32, 256)}
    assert shapes["c4f"] == shapes["c4"]
    assert {c.kind for c in bench.workload("c4f")[1]} == {"f2b"}
    assert shapes["c5"] == {(m, n, 4096) for m in (1, 8, 128) for n in (4096, 4093)}


def test_traffic_profiles_are_consistent():
    """Every committed traffic figure belongs to a kernel summary that exists,
    is at least the algorithmic bytes of some case of its workload, and no
    more than twice the largest (a re-read bug would show up here)."""
    files = glob.glob(os.path.join(u.ROOT, "profiles", "*_traffic.json"))
    assert files
    for f in files:
        t = json.load(open(f))
        assert t["traffic_bytes_per_launch"] > 0 and t["fetch_scale"] > 0 and t["write_scale"] > 0
        alg = [c.bytes_alg() for c in bench.workload(t["workload"])[1]]
        assert 0.9 * min(alg) <= t["traffic_bytes_per_launch"] <= 2 * max(alg), f
    for f in glob.glob(os.path.join(u.ROOT, "profiles", "*_kernel_trace.txt")):
        text = open(f).read()
        assert "rocprofv3 --kernel-trace --stats" in text and "avg_us" in text, f


def test_counter_files_name_a_traced_kernel():
    """Every MFMA/LDS counter file names the kernel instance it read, and that
    instance appears in a committed kernel trace of the same workload, so the
    counters describe a kernel the bench launches."""
    files = glob.glob(os.path.join(u.ROOT, "profiles", "*_mfma_counters.txt"))
    assert files
    for f in files:
        wl = os.path.basename(f)[: -len("_mfma_counters.txt")].rsplit("_", 1)[1]
        names = [l.split("kernel:", 1)[1].strip() for l in open(f) if l.startswith("# kernel:")]
        assert names, f
        inst = names[0].replace("void ", "").replace("dnnopt_hip::", "").replace("(anonymous namespace)::", "")
        traces = glob.glob(os.path.join(u.ROOT, "profiles", f"*_{wl}_kernel_trace.txt"))
        assert traces, f
        assert any(inst in open(t).read() for t in traces), (f, inst)
