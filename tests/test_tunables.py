"""The dispatcher's tunables (dnnopt_hip_set_tunable): the shipped library
plans from built-in defaults whatever DNNOPT_* variables a process inherits,
and changes a plan only when a caller sets a tunable explicitly.  Plans need
no GPU (the planner assumes the MI355X's 256 CUs without one)."""

import json
import os
import subprocess
import sys

import _util as u

SHAPES = [  # (entry, M, N, K): every planner family the knobs below steer
    ("sgemm", 1, 4096, 4096), ("sgemm", 7, 1009, 2048), ("sgemm", 7, 11003, 2048), ("sgemm", 300, 600, 2048),
    ("sgemm", 65536, 64, 256), ("bf16", 256, 11008, 4096), ("bf16", 4, 11008, 4096), ("s8", 128, 4096, 4096),
    ("s8", 1, 4096, 4096), ("int8_f32", 128, 4096, 4096),
]

_CHILD = r"""
import json, os, sys
sys.path.insert(0, os.environ["TESTS_DIR"])
import _util as u
from test_tunables import SHAPES, plans
lib = u.load_lib()
print(json.dumps({"plans": plans(lib), "tunables": {k: lib.get_tunable(k) for k in u.binding().TUNE}}))
"""


def plans(lib):
    out = []
    for entry, M, N, K in SHAPES:
        if entry == "sgemm":
            p = lib.plan_sgemm(M, N, K)
        elif entry == "bf16":
            p = lib.plan_bf16(M, N, K)
        elif entry == "s8":
            p = lib.plan_s8(M, N, K)
        else:
            p = lib.plan_int8_f32(M, N, K)
        out.append({k: (v.decode() if isinstance(v, bytes) else v) for k, v in p.items()})
    return out


def _child(env_extra):
    env = {k: v for k, v in os.environ.items() if not k.startswith("DNNOPT_")}
    env.update(env_extra, TESTS_DIR=os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CHILD], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_inherited_environment_changes_no_plan():
    base = _child({})
    knobs = {"DNNOPT_TILE_CFG": "33", "DNNOPT_TILE_SPLITS": "2", "DNNOPT_SPLIT_REDUCE": "0",
             "DNNOPT_SKINNY_WGS": "100", "DNNOPT_TALL": "0", "DNNOPT_S8_CFG": "2", "DNNOPT_Q8B": "0",
             "DNNOPT_SKINNY_NW": "16", "DNNOPT_S8_ROWDOT": "0", "DNNOPT_KOUTER": "0"}
    steered = _child(knobs)
    assert steered["plans"] == base["plans"]
    assert steered["tunables"] == base["tunables"]
    assert base["tunables"]["SPLIT_REDUCE"] == 1 and base["tunables"]["S8_CFG"] == -1


def test_explicit_tunable_changes_plan_and_restores():
    lib = u.load_lib()
    before = plans(lib)
    with lib.tunables(TALL=0, SKINNY_WGS=100):
        p = lib.plan_sgemm(65536, 64, 256)
        assert p["name"] != "dnnopt_tall_f32", p
        assert lib.plan_sgemm(7, 11003, 2048)["grid_x"] == 100
    assert plans(lib) == before
    old = lib.set_tunable("SPLIT_REDUCE", 0)
    try:
        assert old == 1 and lib.plan_sgemm(1, 4096, 4096)["workspace_bytes"] > 0
    finally:
        lib.set_tunable("SPLIT_REDUCE", old)


def test_tunable_keys_are_checked():
    import ctypes

    lib = u.load_lib()
    v = ctypes.c_int(0)
    assert lib.so.dnnopt_hip_get_tunable(20, ctypes.byref(v)) != 0
    assert lib.so.dnnopt_hip_set_tunable(-1, 0, None) != 0
    assert lib.so.dnnopt_hip_get_tunable(7, None) != 0


def test_split_reduce_choice():
    """SPLIT_REDUCE 1 (default) lets the skinny planner sum the splits in the
    last-arriving workgroup (a plan that takes the ticket slots) for at most 3
    rows and 48 KiB of partials per tile, the reduce kernel otherwise; 0 and
    2 force one or the other."""
    lib = u.load_lib()
    ticket_bytes = 4096 * 64 * 4

    def ticket(plan_fn):
        base = plan_fn()
        with lib.tunables(SPLIT_REDUCE=2):
            red = plan_fn()
        assert (base["grid_x"], base["splits"]) == (red["grid_x"], red["splits"])
        return base["workspace_bytes"] - red["workspace_bytes"] == ticket_bytes

    assert lib.get_tunable("SPLIT_REDUCE") == 1
    for M, N, K, want in ((1, 4096, 4096, True), (2, 4099, 2048, True), (3, 4099, 2048, True),
                          (3, 11003, 2048, True), (2, 1009, 2048, False), (3, 1009, 2048, False),
                          (4, 11003, 2048, False), (5, 11003, 2048, False), (7, 4099, 2048, False)):
        assert ticket(lambda: lib.plan_sgemm(M, N, K)) == want, (M, N, K)
    assert ticket(lambda: lib.plan_bf16(1, 11008, 4096))
    assert not ticket(lambda: lib.plan_bf16(4, 11008, 4096))
    with lib.tunables(SPLIT_REDUCE=0):
        assert lib.plan_sgemm(7, 1009, 2048)["workspace_bytes"] > lib.plan_sgemm(1, 1, 1)["workspace_bytes"]


def test_tuning_build_seeds_from_environment(tmp_path):
    """A -DDNNOPT_TUNING=1 build seeds each tunable from DNNOPT_<NAME> once:
    a whole integer at or above the key's lowest value (0 for SPLIT_REDUCE,
    whose 0 selects the last-workgroup sums, and for S8_CFG; 1 elsewhere),
    switches as 0 / 1; anything else leaves the default.  The table's source
    file is built on its own with the host compiler."""
    import ctypes
    import shutil

    import pytest

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    so = str(tmp_path / "libtune.so")
    subprocess.run([gxx, "-std=c++17", "-O1", "-shared", "-fPIC", "-DDNNOPT_TUNING=1", "-D__HIP_PLATFORM_AMD__",
                    "-I" + os.path.join(root, "dnn-opt_amd", "csrc"), "-I" + os.path.join(root, "include"),
                    "-I/opt/rocm/include", os.path.join(root, "dnn-opt_amd", "csrc", "tune.cpp"), "-o", so],
                   check=True, capture_output=True)
    tune = u.binding().TUNE
    keys = ("SPLIT_REDUCE", "S8_CFG", "MAX_SPLITS", "TALL", "TILE_CFG")
    child = ("import ctypes, json, sys\n"
             "L = ctypes.CDLL(sys.argv[1])\n"
             "out = {}\n"
             "for k, i in json.loads(sys.argv[2]).items():\n"
             "    v = ctypes.c_int(-99)\n"
             "    assert L.dnnopt_hip_get_tunable(i, ctypes.byref(v)) == 0\n"
             "    out[k] = v.value\n"
             "print(json.dumps(out))\n")

    def seeded(env):
        e = {k: v for k, v in os.environ.items() if not k.startswith("DNNOPT_")}
        e.update({"DNNOPT_" + k: v for k, v in env.items()})
        r = subprocess.run([sys.executable, "-c", child, so, json.dumps({k: tune[k] for k in keys})], env=e,
                           check=True, capture_output=True, text=True)
        return json.loads(r.stdout)

    defaults = {"SPLIT_REDUCE": 1, "S8_CFG": -1, "MAX_SPLITS": 256, "TALL": 1, "TILE_CFG": 0}
    assert seeded({}) == defaults
    assert seeded({"SPLIT_REDUCE": "0", "S8_CFG": "0", "MAX_SPLITS": "12", "TALL": "0", "TILE_CFG": "43"}) == {
        "SPLIT_REDUCE": 0, "S8_CFG": 0, "MAX_SPLITS": 12, "TALL": 0, "TILE_CFG": 43}
    # Below a key's lowest value, or not a whole integer: the default stays.
    assert seeded({"SPLIT_REDUCE": "-1", "S8_CFG": "-2", "MAX_SPLITS": "0", "TALL": "x", "TILE_CFG": "4x"}) == defaults
