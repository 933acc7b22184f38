"""CPU-side checks of the C-ABI library: it loads, exports every entry
point include/*.h declares, rejects bad arguments before touching a GPU,
and its synthetic generators are deterministic and match the documented
distributions.  No GPU compute is issued here."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

import arcllm_amd as arc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_c_symbols():
    syms = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(arc_[a-z0-9_]+)\s*\(", text):
            syms.add(m.group(1))
    return syms


def test_library_exports_every_declared_symbol():
    lib = arc.lib()
    syms = declared_c_symbols()
    assert len(syms) >= 25
    missing = [s for s in sorted(syms) if not hasattr(lib, s)]
    assert not missing, missing
    assert set(arc.EXPORTED) <= syms | {"arc_tune_force"}


def test_device_memory_is_allocated_in_one_place():
    """hipMalloc is called only by device_alloc (arc_runtime.cpp), which the
    model arena, the session arena and arc_malloc go through; no kernel
    source or host file allocates device memory by itself."""
    calls = {}
    for path in glob.glob(os.path.join(ROOT, "arcllm_amd", "csrc", "*")) + \
            glob.glob(os.path.join(ROOT, "arcllm_amd", "host", "**", "*"), recursive=True):
        if not os.path.isfile(path):
            continue
        text = re.sub(r"//.*", "", open(path).read())
        for name in ("hipMalloc(", "hipMallocAsync(", "hipExtMallocWithFlags(", "hipMallocManaged(", "arc_malloc("):
            if name in text:
                calls.setdefault(os.path.basename(path), []).append(name)
    assert calls == {"arc_runtime.cpp": ["hipMalloc(", "arc_malloc("]}, calls


def test_version_and_device_count_without_gpu_is_not_an_error():
    assert b"gfx950" in arc.lib().arc_version()
    assert arc.device_count() >= 0


@pytest.mark.parametrize(
    "call",
    [
        lambda L: L.arc_gemv(12, 16, 8, 300, 16, None, 16, None),  # K not a multiple of 256
        lambda L: L.arc_gemv(12, None, 8, 256, 16, None, 16, None),  # null weights
        lambda L: L.arc_gemv(12, 24, 8, 256, 16, None, 16, None),  # Q4_K base not 16-aligned
        lambda L: L.arc_gemv(14, 17, 8, 256, 16, None, 16, None),  # Q6_K base odd
        lambda L: L.arc_gemv(12, 16, 8, 256, 20, None, 16, None),  # x not 16-aligned
        lambda L: L.arc_gemv(13, 16, 8, 256, 16, None, 16, None),  # unsupported type
        lambda L: L.arc_gemv(12, 16, 0, 256, 16, None, 16, None),  # zero rows
        lambda L: L.arc_gemv_splitk(14, 16, 8, 512, 3, 16, 16, None, 16, None),  # splits > blocks
        lambda L: L.arc_gemv_splitk(14, 16, 8, 512, 0, 16, 16, None, 16, None),  # zero splits
        lambda L: L.arc_lmhead_argmax(14, 16, 8, 512, 16, None, 1e-6, None, None, 16, None),  # no workspace
        lambda L: L.arc_dequant(12, 16, 8, 100, 16, None),
        lambda L: L.arc_gemv(214, 18, 8, 256, 16, None, 16, None),  # padded Q6_K base not 4-aligned
        lambda L: L.arc_q6_pad(None, 8, 256, 16, None),  # null source
        lambda L: L.arc_q6_pad(17, 8, 256, 4096, None),  # Q6_K source odd
        lambda L: L.arc_q6_pad(16, 8, 256, 4098, None),  # padded image not 4-aligned
        lambda L: L.arc_q6_pad(4096, 8, 256, 4096 + 210, None),  # image overlaps its source
        lambda L: L.arc_q6_pad(16, 8, 300, 4096, None),  # K not a multiple of 256
        lambda L: L.arc_tune_force(3, 1),
    ],
)
def test_bad_arguments_are_rejected(call):
    L = arc.lib()
    rc = call(L)
    assert rc in (1, 2), rc
    assert L.arc_last_error()


def test_error_raises_arcerror():
    with pytest.raises(arc.ArcError) as e:
        arc.gemv(12, 16, 8, 300, 16, 16)
    assert e.value.code == 1 and "multiple of 256" in str(e.value)


def test_lmhead_workspace_bytes():
    assert arc.lmhead_workspace_bytes(14, 152064, 3584) >= 16 * (152064 // 16)
    assert arc.lmhead_workspace_bytes(arc.Q6_K_PADDED, 152064, 3584) == arc.lmhead_workspace_bytes(14, 152064, 3584)
    # the C function answers 0 for what the LM head does not take; the binding raises
    assert arc.lib().arc_lmhead_workspace_bytes(14, 0, 3584) == 0
    assert arc.lib().arc_lmhead_workspace_bytes(14, 10, 300) == 0
    assert arc.lib().arc_lmhead_workspace_bytes(148, 10, 3584) == 0
    for bad in ((14, 0, 3584), (14, 10, 300), (148, 10, 3584)):
        with pytest.raises(arc.ArcError):
            arc.lmhead_workspace_bytes(*bad)


def test_synth_packed_deterministic_and_distributed():
    a = arc.synth_packed(arc.Q4_K, 1, 2, 64, 3584)
    b = arc.synth_packed(arc.Q4_K, 1, 2, 64, 3584)
    c = arc.synth_packed(arc.Q4_K, 1, 3, 64, 3584)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    blk = a.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and np.all(dm >= 0)
    # |N(0, s)| has mean s*sqrt(2/pi)
    assert abs(d.mean() / (0.01 * np.sqrt(2 / np.pi)) - 1) < 0.08
    assert abs(dm.mean() / (0.005 * np.sqrt(2 / np.pi)) - 1) < 0.08
    nib = blk[:, 16:].ravel()
    assert abs((nib & 15).mean() - 7.5) < 0.1 and abs((nib >> 4).mean() - 7.5) < 0.1


def test_synth_q6_scales_in_range():
    w = arc.synth_packed(arc.Q6_K, 5, 1, 128, 3584).reshape(-1, 210)
    sc = w[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d = w[:, 208:210].copy().view(np.float16).astype(np.float64)
    assert np.all(d >= 0) and abs(d.mean() / (0.01 * np.sqrt(2 / np.pi)) - 1) < 0.08


def test_synth_slices_regenerate_alone():
    whole = arc.synth_packed(arc.Q6_K, 9, 4, 10, 512)
    assert whole.size == 10 * 2 * 210
    x = arc.synth_normal(9, 4, 100000)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    assert np.array_equal(arc.synth_normal(9, 4, 10), x[:10])
