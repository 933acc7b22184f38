"""EXEC148 on the GPU: the repack (bit-exact against the oracle's
restatement of the reference materializer, which tests/test_oracle_cpu.py
pins to the blocks the reference's own code wrote into the golden file), its
exact validation, and the route-B GEMVs over EXEC148 blocks against the fp64
oracle of the source Q4_K tensor (the two formats hold the same element
values; tests/test_oracle_cpu.py checks that bit for bit).

Bars: repack bytes exact; mismatch counts exact; GEMV outputs within 1e-3
max relative error (per-element floor tau = 1e-3 * max|r|) of the fp64
oracle.
"""
import os
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3
SEED = 0xE148_0001
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def dev(a):
    return arc.DeviceBuffer.from_array(a)


def q4(rows, K, stream):
    return arc.synth_packed(arc.Q4_K, SEED, stream, rows, K, 0.01, 0.005)


def gpu_exec148(w, rows, K):
    e = arc.DeviceBuffer(rows * (K // 256) * 148)
    arc.exec148_materialize(dev(w), rows, K, e)
    return e


@pytest.mark.parametrize("rows,K", [(3, 512), (300, 2560), (3584, 18944)])
def test_materialize_matches_oracle(rows, K):
    """Tails (6 and 3000 blocks: partial workgroups) and the full FFN-down
    shape (265,216 blocks)."""
    _log(f"exec148 materialize {rows}x{K}")
    w = q4(rows, K, 1)
    got = gpu_exec148(w, rows, K).download(np.uint8)
    assert np.array_equal(got, orc.exec148(w, rows, K))


def test_materialize_reference_golden_blocks():
    """The golden Q4_K blocks (random and edge-scale blocks) against the
    EXEC148 blocks the reference's materializer produced for them."""
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    blocks = np.ascontiguousarray(g["blocks"]).ravel()
    n = len(g["blocks"])
    got = gpu_exec148(blocks, n, 256).download(np.uint8).reshape(n, 148)
    assert np.array_equal(got, g["exec148"])


def test_validate_exact_and_planted_mismatches():
    rows, K = 77, 2560  # 770 blocks: three full workgroups and a partial one
    w = q4(rows, K, 2)
    wd = dev(w)
    e = gpu_exec148(w, rows, K)
    assert arc.exec148_validate(wd, e, rows, K) == 0
    img = e.download(np.uint8).reshape(-1, 148)
    # one changed bit in each of: a d byte, an (sc, mn) byte, the first and
    # the last code byte, two bits of one block (counted once), the last block
    planted = {0: [(1, 0x01)], 5: [(9, 0x40)], 256: [(20, 0x01)], 511: [(147, 0x80)], 600: [(30, 0x10), (100, 0x02)],
               769: [(3, 0x08)]}
    bad = img.copy()
    for b, edits in planted.items():
        for pos, bit in edits:
            bad[b, pos] ^= bit
    assert arc.exec148_validate(wd, dev(bad.ravel()), rows, K) == len(planted)


def test_validate_many_sums_over_tensors():
    """Several tensor pairs in one call: exact images count 0, planted blocks
    in two of them are summed, a swapped pair (image of another tensor)
    mismatches on every block."""
    rows, K = 40, 768
    ws = [q4(rows, K, 20 + i) for i in range(3)]
    wd = [dev(w) for w in ws]
    es = [gpu_exec148(w, rows, K) for w in ws]
    assert arc.exec148_validate_many(wd, es, rows, K) == 0
    nb = rows * (K // 256)
    imgs = [e.download(np.uint8).reshape(-1, 148).copy() for e in es]
    imgs[0][7, 25] ^= 0x10
    imgs[2][0, 2] ^= 0x01
    imgs[2][nb - 1, 147] ^= 0x80
    bad = [dev(im.ravel()) for im in imgs]
    assert arc.exec148_validate_many(wd, bad, rows, K) == 3
    assert arc.exec148_validate_many([wd[1], wd[0]], [es[0], es[1]], rows, K) == 2 * nb


@pytest.mark.parametrize("rows,K", [(64, 512), (1000, 3584), (3584, 18944)])
def test_route_b_gemv(rows, K):
    w = q4(rows, K, 3)
    x = arc.synth_normal(SEED, 4, K)
    e = gpu_exec148(w, rows, K)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv(arc.EXEC148, e, rows, K, dev(x), y)
    err = orc.rel_err(y.download(np.float32), orc.gemv_r64(arc.Q4_K, w, rows, K, x))
    _log(f"route B gemv {rows}x{K}: rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("rows,K,splits", [(3584, 18944, 74), (512, 2560, 5), (33, 2304, 9)])
def test_route_b_splitk_with_residual(rows, K, splits):
    w = q4(rows, K, 5)
    x = arc.synth_normal(SEED, 6, K)
    res = arc.synth_normal(SEED, 7, rows)
    e = gpu_exec148(w, rows, K)
    part = arc.DeviceBuffer(splits * rows * 4)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv_splitk(arc.EXEC148, e, rows, K, splits, dev(x), part, y, residual=dev(res))
    ref = orc.gemv_r64(arc.Q4_K, w, rows, K, x, res)
    err = orc.rel_err(y.download(np.float32), ref)
    # route A on the same tensor, for comparison
    ya = arc.DeviceBuffer(rows * 4)
    arc.gemv_splitk(arc.Q4_K, dev(w), rows, K, splits, dev(x), part, ya, residual=dev(res))
    err_a = orc.rel_err(ya.download(np.float32), ref)
    _log(f"split-K {rows}x{K}/{splits}: route B rel_err={err:.3e}, route A rel_err={err_a:.3e}")
    assert err <= TOL and err_a <= TOL


def test_exec148_argument_errors():
    w = dev(q4(4, 512, 8))
    e = arc.DeviceBuffer(4 * 2 * 148 + 64)
    with pytest.raises(arc.ArcError):
        arc.exec148_materialize(w, 4, 500, e)  # K not a multiple of 256
    with pytest.raises(arc.ArcError):
        arc.exec148_materialize(w, 4, 512, e.ptr + 4)  # destination not 16-byte aligned
    out = arc.DeviceBuffer(4 * 512 * 4)
    with pytest.raises(arc.ArcError):
        arc.dequant(arc.EXEC148, e, 4, 512, out)
