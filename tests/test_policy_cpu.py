"""The operator plugin surface (registry v2, policy v4, binding v4, the
Q4-down registrations and the gfx950 backend's host parts) on the CPU.

* tests/cpp/policy_parity.cpp is compiled against this repository's
  implementation and its decision trace (1.46 M cases: registry add_bundle
  over ~70 bundle mutations, the Q4-down policy over 2 profiles x 2^15 runtime
  masks x 16 reuse values, test-defined mandatory / direct / amortized /
  disabled / malformed registries, apply_decision over every lifecycle, route
  and backend failure combination) is compared with
  - tests/golden/policy_trace.json, the same program built against the
    reference's own sources (src/arcllm_v1_primitive_registry_v2.cpp,
    src/arcllm_v1_generic_policy_engine_v4.cpp,
    src/arcllm_v1_generic_backend_binding_v4.cpp,
    src/registrations/arcllm_v1_q4k_down_reference_registration_v2.cpp);
  - that build itself, line by line, when oracle/_ref/policy_parity_ref is
    there (``make -C oracle ref``);
* the trace is shown to catch a planted mistake (an off-by-one in the
  threshold comparison, planted in a copy of the policy under tmp);
* the host EXEC148 repack of the P0 path against the oracle
  (orc_exec148_tensor) and the reference's golden EXEC148 blocks;
* the MI355X registration: accepted by the registry, each acquisition path
  chosen from exactly its measured threshold on, residency = family bytes.
"""
import json
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import oracle_lib as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
HOST = os.path.join(ROOT, "arcllm_amd", "host")
PKG = os.path.join(ROOT, "arcllm_amd")
REF_TRACE = os.path.join(ROOT, "oracle", "_ref", "policy_parity_ref")
SURFACE = [os.path.join(HOST, s) for s in ("registry_v2.cpp", "policy_v4.cpp", "binding_v4.cpp")]
REGISTRATION = os.path.join(HOST, "registrations", "arcllm_v1_q4k_down_reference_registration_v2.cpp")
CXX = shutil.which("g++") or "g++"


def _build(out, sources, extra=()):
    cmd = [CXX, "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror", f"-I{ROOT}/include",
           f"-I{HOST}/registrations", *sources, "-o", str(out), *extra]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return str(out)


def _sections(stdout):
    out = {}
    for line in stdout.splitlines():
        m = re.fullmatch(r"(\w+) cases=(\d+) fnv=([0-9a-f]{16})", line)
        assert m, line
        out[m.group(1)] = {"cases": int(m.group(2)), "fnv1a64": m.group(3)}
    return out


@pytest.fixture(scope="module")
def trace_exe(tmp_path_factory):
    d = tmp_path_factory.mktemp("policy")
    return _build(d / "policy_parity", [os.path.join(ROOT, "tests", "cpp", "policy_parity.cpp"), *SURFACE,
                                        REGISTRATION])


def test_policy_trace_matches_reference_golden(trace_exe):
    got = _sections(subprocess.run([trace_exe], capture_output=True, text=True, check=True).stdout)
    with open(os.path.join(GOLD, "policy_trace.json")) as f:
        want = json.load(f)["sections"]
    assert got == want
    assert got["q4"]["cases"] == 2 * (1 << 15) * 16
    assert got["total"]["cases"] > 1_400_000


@pytest.mark.skipif(not os.path.exists(REF_TRACE), reason="oracle/_ref/policy_parity_ref not built")
def test_policy_trace_identical_to_reference_build(trace_exe, tmp_path):
    mine, ref = tmp_path / "mine.txt", tmp_path / "ref.txt"
    subprocess.run([trace_exe, str(mine)], check=True, capture_output=True)
    subprocess.run([REF_TRACE, str(ref)], check=True, capture_output=True)
    with open(mine) as a, open(ref) as b:
        for i, (x, y) in enumerate(zip(a, b)):
            assert x == y, f"trace line {i}: mine {x!r} reference {y!r}"
    assert os.path.getsize(mine) == os.path.getsize(ref)


def test_policy_trace_catches_a_planted_threshold_mistake(trace_exe, tmp_path):
    with open(os.path.join(HOST, "policy_v4.cpp")) as f:
        src = f.read()
    needle = "s.req.future_reuse_units < bar->minimum_reuse_units"
    assert src.count(needle) == 1
    src = src.replace(needle, "s.req.future_reuse_units <= bar->minimum_reuse_units")
    src = src.replace('"../../include/', f'"{ROOT}/include/')
    planted = tmp_path / "policy_planted.cpp"
    planted.write_text(src)
    exe = _build(tmp_path / "planted", [os.path.join(ROOT, "tests", "cpp", "policy_parity.cpp"), SURFACE[0],
                                        str(planted), SURFACE[2], REGISTRATION])
    got = _sections(subprocess.run([exe], capture_output=True, text=True, check=True).stdout)
    good = _sections(subprocess.run([trace_exe], capture_output=True, text=True, check=True).stdout)
    assert got["q4"] != good["q4"]
    assert got["registry"] == good["registry"] and got["binding"] == good["binding"]


# ------------------------------------------------------------ gfx950 backend host parts
HIP_LIB = os.path.join(PKG, "libarcllm_hip.so")


@pytest.fixture(scope="module")
def host_check(tmp_path_factory):
    if not os.path.exists(HIP_LIB):
        pytest.skip("libarcllm_hip.so not built (python -m arcllm_amd.build)")
    d = tmp_path_factory.mktemp("q4backend")
    return _build(d / "q4_backend_host_check",
                  [os.path.join(ROOT, "tests", "cpp", "q4_backend_host_check.cpp"),
                   os.path.join(HOST, "q4_down_backend.cpp"), *SURFACE],
                  [f"-L{PKG}", "-l:libarcllm_hip.so", f"-Wl,-rpath,{PKG}"])


def _repack(exe, tmp_path, q4, rows, K, threads):
    src, dst = tmp_path / "in.q4", tmp_path / "out.e148"
    q4.tofile(src)
    subprocess.run([exe, "repack", str(src), str(rows), str(K), str(dst), str(threads)], check=True)
    return np.fromfile(dst, np.uint8)


@pytest.mark.parametrize("rows,K,threads", [(1, 256, 1), (3, 512, 2), (37, 2304, 5), (64, 18944, 16)])
def test_host_repack_matches_oracle(host_check, tmp_path, rows, K, threads):
    rng = np.random.default_rng(rows * 1000 + K)
    q4 = rng.integers(0, 256, rows * (K // 256) * 144, dtype=np.uint8)
    got = _repack(host_check, tmp_path, q4, rows, K, threads)
    assert got.size == rows * (K // 256) * 148
    assert np.array_equal(got, orc.exec148(q4, rows, K))


def test_host_repack_matches_reference_golden_blocks(host_check, tmp_path):
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    blocks, want = g["blocks"], g["exec148"]
    got = _repack(host_check, tmp_path, np.ascontiguousarray(blocks).ravel(), len(blocks), 256, 3)
    assert np.array_equal(got.reshape(want.shape), want)


def test_mi355x_registration_thresholds(host_check):
    family = 14 * 3584 * (18944 // 256) * 148
    out = subprocess.run([host_check, "registration", str(family)], capture_output=True, text=True,
                         check=True).stdout.split("\n")
    assert out[0] == "add 0 -"
    thr = [int(x) for x in out[1].split()[1:]]
    assert len(thr) == 6 and thr[0] < min(thr[1], thr[2]) and thr[3:] == [2 * t for t in thr[:3]]
    for line in out[2:]:
        if not line:
            continue
        p, path, first, nbytes = line.split()
        prof = int(p[1:])
        # acquisition from exactly the threshold on, for the model's family bytes
        assert int(first) == thr[3 * prof + int(path)]
        assert int(nbytes) == family == 549527552
