"""Route B of the decode step and the failure paths of the Q4-down backend
on the GPU.

* arc_session_route_down: a layer's Q4_K ffn_down switched to its EXEC148
  image (built from the resident tensor, arc_model_tensor_device +
  arc_exec148_materialize) decodes the oracle's tokens (near-tie rule of
  test_decode_gpu.py); switching back to route A and to B again re-captures
  the step and keeps the kernel count; bad layers, a layer whose ffn_down is
  Q6_K and a misaligned image are rejected before any launch.
* A P3 sidecar with one flipped byte: arcllm_q4_paths acquires it, the GPU
  validation finds exactly one mismatched block, the acquisition fails with
  VALIDATION_FAILED's message and the image is released (the tool exits 2).
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import gguf_write as gw
import oracle_lib as orc
from decode_common import tiny_dims

pytestmark = pytest.mark.gpu

SEED = 0x2B0_7E5


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def test_session_route_down_switches_and_matches_oracle():
    d = tiny_dims(layers=3)  # layer 1: Q4_K ffn_down
    T = arc.synth_model_tensors(d, SEED)
    model = arc.Model(d, T)
    s = arc.Session(model, 96)
    ctx, steps, kv_seed = 30, 12, 5
    o = orc.DecodeOracle(d, T, 96)

    rows, K = d.hidden, d.ffn
    img = arc.DeviceBuffer(rows * (K // 256) * 148)
    arc.exec148_materialize(model.tensor_device(1, arc.T_FFN_DOWN), rows, K, img)
    arc.synchronize()
    assert arc.exec148_validate(model.tensor_device(1, arc.T_FFN_DOWN), img, rows, K) == 0
    # the model's own EXEC148 reserve: one slot, for layer 1
    base, stride, slots = model.exec148_reserve()
    assert slots == 1 and base % 256 == 0 and stride >= rows * (K // 256) * 148
    arc.exec148_materialize(model.tensor_device(1, arc.T_FFN_DOWN), rows, K, base)
    arc.synchronize()
    assert arc.exec148_validate(model.tensor_device(1, arc.T_FFN_DOWN), base, rows, K) == 0

    results = {}
    for name, route in (("A", None), ("B", img), ("A again", None), ("B again", base)):
        s.route_down(1, route)
        s.fill_kv(ctx, kv_seed)
        toks, nf = s.decode(77, ctx, steps)
        assert nf == 0
        assert s.kernels_per_step == 1 + 4 * d.layers
        results[name] = toks
        _log(f"route {name}: {toks.tolist()}")
        o.fill_kv(ctx, kv_seed, arc.synth_normal)
        _log(f"route {name}: near-tie steps {o.follow(77, ctx, toks)}")
    assert np.array_equal(results["A"], results["A again"])
    assert np.array_equal(results["B"], results["B again"])

    with pytest.raises(arc.ArcError):
        s.route_down(0, img)  # layer 0's ffn_down is Q6_K
    with pytest.raises(arc.ArcError):
        s.route_down(d.layers, None)  # no such layer
    with pytest.raises(arc.ArcError):
        s.route_down(1, img.ptr + 4)  # not 16-byte aligned
    s.route_down(1, None)
    s.close()
    img.close()
    model.close()


def test_corrupted_sidecar_fails_validation(tmp_path):
    d = tiny_dims(layers=2)
    T = arc.synth_model_tensors(d, SEED + 1)
    path = str(tmp_path / "m.gguf")
    gw.write_qwen2_model(path, d, T)
    sidecar = str(tmp_path / "family.e148")
    r = subprocess.run([arc.Q4_PATHS_PATH, "--model", path, "--ctx", "8", "--steps", "2", "--paths", "p1",
                        "--sidecar", sidecar], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    img = np.fromfile(sidecar, np.uint8)
    assert img.size == d.hidden * (d.ffn // 256) * 148
    img[148 * 3 + 30] ^= 0x10  # one code nibble of block 3
    img.tofile(sidecar)
    r = subprocess.run([arc.Q4_PATHS_PATH, "--model", path, "--ctx", "8", "--steps", "2", "--paths", "p3",
                        "--sidecar", sidecar], capture_output=True, text=True, timeout=120)
    _log(r.stderr.strip())
    assert r.returncode == 2 and r.stdout == ""
    assert "p3 validation failed: 1 EXEC148 blocks differ from their Q4_K source" in r.stderr
