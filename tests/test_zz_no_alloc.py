"""arc_lmhead_argmax_noalloc (argmax partials in the library's static device
scratch) against arc_lmhead_argmax (the same kernels with a caller workspace):
token, non-finite count and logits must be identical, on two calls in a row
whose second is smaller, through the C ABI."""
import sys

import numpy as np
import pytest

import arcllm_amd as arc

pytestmark = pytest.mark.gpu

SEED = 0x0A110C


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def run_both(qtype, rows, K, seed, with_logits=True):
    w = arc.synth_packed(qtype, seed, 1, rows, K)
    h = arc.synth_normal(seed, 2, K)
    nw = arc.synth_normal(seed, 3, K, 1.0, 0.05)
    D = arc.DeviceBuffer.from_array
    wd, hd, nwd = D(w), D(h), D(nw)
    ws = arc.DeviceBuffer(arc.lmhead_workspace_bytes(qtype, rows, K))
    out_a, out_b = arc.DeviceBuffer(8), arc.DeviceBuffer(8)
    la = arc.DeviceBuffer(rows * 4) if with_logits else None
    lb = arc.DeviceBuffer(rows * 4) if with_logits else None
    arc.lmhead_argmax(qtype, wd, rows, K, hd, nwd, 1e-6, la, ws, out_a)
    arc.lmhead_argmax_noalloc(qtype, wd, rows, K, hd, nwd, 1e-6, lb, out_b)
    arc.synchronize()
    a, b = out_a.download(np.uint32), out_b.download(np.uint32)
    _log(f"qtype {qtype} rows {rows} K {K}: workspace token {a[0]} nonfinite {a[1]}; no-alloc token {b[0]} "
         f"nonfinite {b[1]}")
    assert a[0] == b[0] and a[1] == b[1]
    if with_logits:
        ya, yb = la.download(np.float32), lb.download(np.float32)
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
        assert int(np.argmax(ya)) == int(a[0])
    return int(b[0])


def test_noalloc_matches_workspace_entry_point_twice_second_smaller():
    run_both(arc.Q6_K, 152064, 3584, SEED)
    run_both(arc.Q6_K, 4097, 3584, SEED + 1)


def test_noalloc_q4k_without_logits_and_without_norm():
    run_both(arc.Q4_K, 30000, 2048, SEED + 2, with_logits=False)
    # no norm weight: the staged x is h itself
    rows, K = 1000, 1024
    w = arc.synth_packed(arc.Q6_K, SEED + 3, 1, rows, K)
    h = arc.synth_normal(SEED + 3, 2, K)
    D = arc.DeviceBuffer.from_array
    wd, hd = D(w), D(h)
    ws = arc.DeviceBuffer(arc.lmhead_workspace_bytes(arc.Q6_K, rows, K))
    oa, ob = arc.DeviceBuffer(8), arc.DeviceBuffer(8)
    arc.lmhead_argmax(arc.Q6_K, wd, rows, K, hd, None, 1e-6, None, ws, oa)
    arc.lmhead_argmax_noalloc(arc.Q6_K, wd, rows, K, hd, None, 1e-6, None, ob)
    arc.synchronize()
    assert np.array_equal(oa.download(np.uint32), ob.download(np.uint32))


def test_noalloc_rejects_bad_arguments():
    L = arc.lib()
    assert L.arc_lmhead_argmax_noalloc(14, 16, 8, 512, 16, None, 1e-6, None, None, None) != 0  # null out
    assert L.arc_lmhead_argmax_noalloc(14, 16, 8, 256 * 81, 16, None, 1e-6, None, 16, None) != 0  # K > panel
    assert L.arc_lmhead_argmax_noalloc(148, 16, 8, 512, 16, None, 1e-6, None, 16, None) != 0  # EXEC148
