"""GPU parity of the hand-written gfx950 kernels against the CPU oracle.

Bars: dequantised weights bit-exact; float outputs within 1e-3 max relative
error vs the fp64-accumulated oracle (per-element |y-r| / max(|r|, tau),
tau = 1e-3 * max|r|); argmax token IDs exact.  Inputs come from the seeded
synthetic generators (configs: Q4_K d ~ |N(0,0.01)|, dmin ~ |N(0,0.005)|,
uniform scale/nibble bytes; Q6_K uniform ql/qh, int8 scales in [-32, 31],
d ~ |N(0,0.01)|; x ~ N(0,1)).
"""
import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3
SEED = 0xA4C1_1A55


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"
    name, archname = arc.device_info()
    print(f"device: {name} {archname}", flush=True)
    yield
    arc.tune_force(0, 0)


def dev(a):
    return arc.DeviceBuffer.from_array(a)


def packed(qtype, rows, K, stream):
    return arc.synth_packed(qtype, SEED, stream, rows, K, 0.01, 0.005)


def special_blocks(qtype, n):
    """Blocks whose fp16 d/dmin hit the binary16 edge cases, plus saturated
    scale and code bytes."""
    rng = np.random.default_rng(7)
    bb = arc.BLOCK_BYTES[qtype]
    specials = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7E01]
    out = rng.integers(0, 256, (n, bb), dtype=np.uint8)
    for i in range(n):
        h = specials[i % len(specials)]
        hb = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
        if qtype == arc.Q4_K:
            out[i, 0:2] = hb
            out[i, 2:4] = np.frombuffer(np.uint16(specials[(i + 3) % len(specials)]).tobytes(), np.uint8)
            if i % 3 == 0:
                out[i, 4:16] = 0xFF if i % 2 else 0x00
        else:
            out[i, 208:210] = hb
            if i % 3 == 0:
                out[i, 192:208] = 0x80 if i % 2 else 0x7F
    return out.ravel()


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return np.all((a.view(np.uint32) == b.view(np.uint32)) | nan)


@pytest.mark.parametrize("qtype", [arc.Q4_K, arc.Q6_K])
def test_dequant_bit_exact(qtype):
    rows, K = 24, 1024
    w = np.concatenate([packed(qtype, rows, K, 1), special_blocks(qtype, 48)])
    rows_total = rows + 48 // (K // 256)
    out = arc.DeviceBuffer(rows_total * K * 4)
    arc.dequant(qtype, dev(w), rows_total, K, out)
    got = out.download(np.float32).reshape(rows_total, K)
    ref = orc.dequant(qtype, w, rows_total, K)
    assert same_bits(got, ref)


@pytest.mark.parametrize(
    "qtype,rows,K,bias",
    [
        (arc.Q4_K, 4, 256, False),
        (arc.Q4_K, 37, 512, True),
        (arc.Q4_K, 512, 3584, True),
        (arc.Q4_K, 3584, 3584, False),
        (arc.Q4_K, 18944, 3584, False),  # config: gate projection
        (arc.Q6_K, 5, 768, True),
        (arc.Q6_K, 512, 3584, True),
        (arc.Q6_K, 3584, 18944, False),
        (arc.Q6_K, 1000, 3584, False),
    ],
)
def test_gemv_vs_fp64(qtype, rows, K, bias):
    w = packed(qtype, rows, K, 2)
    x = arc.synth_normal(SEED, 3, K)
    b = arc.synth_normal(SEED, 4, rows) if bias else None
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv(qtype, dev(w), rows, K, dev(x), y, bias=None if b is None else dev(b))
    got = y.download(np.float32)
    ref = orc.gemv_r64(qtype, w, rows, K, x, b)
    err = orc.rel_err(got, ref)
    print(f"rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("bs,rpl", [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (8, 1),
                                    (8, 2), (16, 1)])
@pytest.mark.parametrize("qtype", [arc.Q4_K, arc.Q6_K])
def test_gemv_every_layout(qtype, bs, rpl):
    if qtype == arc.Q6_K and rpl == 4:
        pytest.skip("Q6_K layouts with 4 rows per lane are not built: (bs=2, rpl=4) took a GPU memory "
                    "fault once with no cause found in its source or code; kept off the GPU")
    rows, K = 301, 3584  # ragged row count, 14 blocks: uneven round-robin for bs=4,8,16
    w = packed(qtype, rows, K, 5)
    x = arc.synth_normal(SEED, 6, K)
    y = arc.DeviceBuffer(rows * 4)
    arc.tune_force(bs, rpl)
    try:
        arc.gemv(qtype, dev(w), rows, K, dev(x), y)
    finally:
        arc.tune_force(0, 0)
    assert orc.rel_err(y.download(np.float32), orc.gemv_r64(qtype, w, rows, K, x)) <= TOL


@pytest.mark.parametrize("qtype,rows", [(arc.Q6_K, 1001), (arc.Q4_K, 301), (arc.Q6_K, 3)])
def test_wide_gemv_cooperative_ragged(qtype, rows):
    """K = 18944 (74 super-blocks: the cooperative workgroup kernel) with row
    counts that leave the last workgroup's tiles partly or wholly past the
    end, with bias."""
    K = 18944
    w = packed(qtype, rows, K, 80)
    x = arc.synth_normal(SEED, 81, K)
    b = arc.synth_normal(SEED, 82, rows)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv(qtype, dev(w), rows, K, dev(x), y, bias=dev(b))
    assert orc.rel_err(y.download(np.float32), orc.gemv_r64(qtype, w, rows, K, x, b)) <= TOL


def test_wide_splitk_cooperative_ragged():
    """One-column split-K on the cooperative kernel with a ragged row count:
    partials against the oracle, y the in-order sum of the partials + res."""
    rows, K, splits = 1001, 18944, 74
    w = packed(arc.Q4_K, rows, K, 83)
    x = arc.synth_normal(SEED, 84, K)
    res = arc.synth_normal(SEED, 85, rows)
    part = arc.DeviceBuffer(splits * rows * 4)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv_splitk(arc.Q4_K, dev(w), rows, K, splits, dev(x), part, y, residual=dev(res))
    gp = part.download(np.float32, splits * rows).reshape(rows, splits).T
    rp = orc.splitk_r64(arc.Q4_K, w, rows, K, splits, x)
    for j in range(splits):
        assert orc.rel_err(gp[j], rp[j]) <= TOL
    acc = np.zeros(rows, np.float32)
    for j in range(splits):
        acc = (acc + gp[j]).astype(np.float32)
    acc = (acc + res).astype(np.float32)
    assert np.array_equal(acc.view(np.uint32), y.download(np.float32).view(np.uint32))


def test_q6_four_rows_per_lane_layout_refused():
    """Q6_K layouts with 4 rows per lane are not built: a forced one is
    refused on the host (nothing is launched); the automatic choice never
    takes it."""
    rows, K = 64, 512
    w = dev(packed(arc.Q6_K, rows, K, 9))
    x = dev(arc.synth_normal(SEED, 10, K))
    y = arc.DeviceBuffer(rows * 4)
    arc.tune_force(2, 4)
    try:
        with pytest.raises(arc.ArcError):
            arc.gemv(arc.Q6_K, w, rows, K, x, y)
    finally:
        arc.tune_force(0, 0)


def test_gemv_q6_unaligned_base():
    """Q6_K tensor starting 2 bytes past a 4-byte boundary, odd blocks per row."""
    rows, K = 7, 768
    w = packed(arc.Q6_K, rows, K, 7)
    buf = arc.DeviceBuffer(w.nbytes + 64)
    host = np.zeros(w.nbytes + 64, np.uint8)
    host[2:2 + w.nbytes] = w
    buf.upload(host)
    x = arc.synth_normal(SEED, 8, K)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv(arc.Q6_K, buf.ptr + 2, rows, K, dev(x), y)
    assert orc.rel_err(y.download(np.float32), orc.gemv_r64(arc.Q6_K, w, rows, K, x)) <= TOL


@pytest.mark.parametrize("qtype", [arc.Q4_K, arc.Q6_K])
def test_gemv_one_hot_columns(qtype):
    """x = e_k gives column k of the dequantised matrix."""
    rows, K = 64, 512
    w = packed(qtype, rows, K, 9)
    deq = orc.dequant(qtype, w, rows, K)
    wd = dev(w)
    y = arc.DeviceBuffer(rows * 4)
    for k in (0, 31, 32, 63, 64, 127, 128, 200, 255, 256, 300, 511):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        arc.gemv(qtype, wd, rows, K, dev(x), y)
        np.testing.assert_allclose(y.download(np.float32), deq[:, k], rtol=2e-7, atol=1e-30)


def test_gemv_zero_codes_give_minus_min_sum():
    """All nibbles zero: y = -sum_j dmin*mn_j*(sum of x over sub-block j)."""
    rows, K = 16, 512
    w = packed(arc.Q4_K, rows, K, 10).reshape(-1, 144).copy()
    w[:, 16:] = 0
    w = w.ravel()
    x = arc.synth_normal(SEED, 11, K)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv(arc.Q4_K, dev(w), rows, K, dev(x), y)
    assert orc.rel_err(y.download(np.float32), orc.gemv_r64(arc.Q4_K, w, rows, K, x)) <= TOL


@pytest.mark.parametrize("rows,K", [(64, 512), (1000, 3584), (18944, 3584)])
def test_gateup_swiglu(rows, K):
    wg = packed(arc.Q4_K, rows, K, 20)
    wu = packed(arc.Q4_K, rows, K, 21)
    x = arc.synth_normal(SEED, 22, K)
    s = arc.DeviceBuffer(rows * 4)
    arc.gateup_swiglu(arc.Q4_K, dev(wg), dev(wu), rows, K, dev(x), s)
    g = orc.gemv_r64(arc.Q4_K, wg, rows, K, x)
    u = orc.gemv_r64(arc.Q4_K, wu, rows, K, x)
    err = orc.rel_err(s.download(np.float32), orc.swiglu_f64(g, u))
    print(f"rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize(
    "rows,K,bias",
    [(4, 256, False), (37, 512, True), (301, 2560, True), (1000, 3584, False), (3584, 3584, True), (18944, 3584, False)],
)
def test_rowstream_gemv_vs_fp64(rows, K, bias):
    """The row-stream Q4_K kernel forced on for every shape it takes (the
    automatic choice gives it plain GEMVs of 8192 rows or more)."""
    w = packed(arc.Q4_K, rows, K, 40)
    x = arc.synth_normal(SEED, 41, K)
    b = arc.synth_normal(SEED, 42, rows) if bias else None
    y = arc.DeviceBuffer(rows * 4)
    arc.tune_rowstream(1)
    try:
        arc.gemv(arc.Q4_K, dev(w), rows, K, dev(x), y, bias=None if b is None else dev(b))
    finally:
        arc.tune_rowstream(-1)
    err = orc.rel_err(y.download(np.float32), orc.gemv_r64(arc.Q4_K, w, rows, K, x, b))
    print(f"rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("rows,K", [(64, 512), (1000, 3584), (18944, 3584)])
def test_rowstream_gateup_swiglu(rows, K):
    wg = packed(arc.Q4_K, rows, K, 43)
    wu = packed(arc.Q4_K, rows, K, 44)
    x = arc.synth_normal(SEED, 45, K)
    s = arc.DeviceBuffer(rows * 4)
    arc.tune_rowstream(1)
    try:
        arc.gateup_swiglu(arc.Q4_K, dev(wg), dev(wu), rows, K, dev(x), s)
    finally:
        arc.tune_rowstream(-1)
    g = orc.gemv_r64(arc.Q4_K, wg, rows, K, x)
    u = orc.gemv_r64(arc.Q4_K, wu, rows, K, x)
    err = orc.rel_err(s.download(np.float32), orc.swiglu_f64(g, u))
    print(f"rel_err={err:.3e}")
    assert err <= TOL


def test_rowstream_mode_rejects_bad_values():
    with pytest.raises(arc.ArcError):
        arc.tune_rowstream(2)


@pytest.mark.parametrize(
    "qtype,rows,K,splits",
    [(arc.Q6_K, 3584, 18944, 74), (arc.Q6_K, 100, 2560, 3), (arc.Q4_K, 512, 2560, 5), (arc.Q4_K, 3584, 18944, 74),
     (arc.Q6_K, 33, 2304, 9), (arc.Q4_K, 70, 38400, 150)],
)
def test_splitk(qtype, rows, K, splits):
    w = packed(qtype, rows, K, 30)
    x = arc.synth_normal(SEED, 31, K)
    res = arc.synth_normal(SEED, 32, rows)
    part = arc.DeviceBuffer(splits * rows * 4)
    y = arc.DeviceBuffer(rows * 4)
    arc.gemv_splitk(qtype, dev(w), rows, K, splits, dev(x), part, y, residual=dev(res))
    nb = K // 256
    bps = -(-nb // splits)
    used = -(-nb // bps)
    gp = part.download(np.float32, used * rows).reshape(rows, used).T
    rp = orc.splitk_r64(qtype, w, rows, K, used, x) if used == splits else None
    if rp is not None:
        for j in range(used):
            assert orc.rel_err(gp[j], rp[j]) <= TOL
    ref = orc.gemv_r64(qtype, w, rows, K, x, res)
    err = orc.rel_err(y.download(np.float32), ref)
    print(f"rel_err={err:.3e}")
    assert err <= TOL
    # pass 2 is a fixed-order sum of the partials: recompute it in the same order
    acc = np.zeros(rows, np.float32)
    for j in range(used):
        acc = (acc + gp[j]).astype(np.float32)
    acc = (acc + res).astype(np.float32)
    assert np.array_equal(acc.view(np.uint32), y.download(np.float32).view(np.uint32))


def test_splitk_deterministic():
    rows, K, splits = 3584, 18944, 74
    w = dev(packed(arc.Q6_K, rows, K, 40))
    x = dev(arc.synth_normal(SEED, 41, K))
    part = arc.DeviceBuffer(splits * rows * 4)
    outs = []
    for _ in range(3):
        y = arc.DeviceBuffer(rows * 4)
        arc.gemv_splitk(arc.Q6_K, w, rows, K, splits, x, part, y)
        outs.append(y.download(np.float32).view(np.uint32))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_rmsnorm():
    n = 3584
    x = arc.synth_normal(SEED, 50, n)
    w = arc.synth_normal(SEED, 51, n, 1.0, 0.05)
    y = arc.DeviceBuffer(n * 4)
    arc.rmsnorm(dev(x), dev(w), n, 1e-6, y)
    assert orc.rel_err(y.download(np.float32), orc.rmsnorm_f64(x, w, 1e-6)) <= 1e-5


def _lmhead(qtype, w, rows, K, h, nw, eps=1e-6, logits=True):
    ws = arc.DeviceBuffer(arc.lmhead_workspace_bytes(qtype, rows, K))
    out = arc.DeviceBuffer(8)
    lg = arc.DeviceBuffer(rows * 4) if logits else None
    arc.lmhead_argmax(qtype, w, rows, K, dev(h), None if nw is None else dev(nw), eps, lg, ws, out)
    o = out.download(np.uint32)
    return int(o[0]), int(o[1]), (lg.download(np.float32) if logits else None)


@pytest.mark.parametrize("rows", [4097, 30000, 152064])
def test_lmhead_argmax(rows):
    """Config 2 (at 152,064 rows the Qwen2.5-7B vocabulary): RMSNorm + Q6_K LM
    head + argmax, every logit against the fp64 oracle, the token exactly."""
    K = 3584
    w = packed(arc.Q6_K, rows, K, 60)
    h = arc.synth_normal(SEED, 61, K)
    nw = arc.synth_normal(SEED, 62, K, 1.0, 0.05)
    tok, nonfinite, logits = _lmhead(arc.Q6_K, dev(w), rows, K, h, nw)
    xr = orc.rmsnorm_f64(h, nw, 1e-6)
    ref = orc.gemv_r64_xd(arc.Q6_K, w, rows, K, xr)
    order = np.argsort(-ref, kind="stable")
    margin = ref[order[0]] - ref[order[1]]
    print(f"token={tok} ref={order[0]} margin={margin:.4e}")
    assert nonfinite == 0
    assert orc.rel_err(logits, ref) <= TOL
    assert tok == int(order[0])
    # the GPU's own argmax over the logits it materialised, lowest index on ties
    t = orc.top2(logits)
    assert tok == t.top1


def test_lmhead_ties_go_to_lowest_index():
    rows, K = 5000, 3584
    w = packed(arc.Q6_K, rows, K, 63).reshape(rows, -1).copy()
    h = arc.synth_normal(SEED, 64, K)
    ref = orc.gemv_r64(arc.Q6_K, w.ravel(), rows, K, h)
    best = int(np.argmax(ref))
    for low in (0, 1, 17, best // 2):
        if low >= best:
            continue
        w2 = w.copy()
        w2[low] = w2[best]  # identical rows -> bitwise identical logits
        tok, nf, logits = _lmhead(arc.Q6_K, dev(w2.ravel()), rows, K, h, None)
        assert logits[low] == logits[best]
        assert tok == low, (tok, low, best)


def test_lmhead_all_equal_rows_pick_zero():
    rows, K = 300, 512
    one = packed(arc.Q6_K, 1, K, 65)
    w = np.tile(one, rows)
    h = arc.synth_normal(SEED, 66, K)
    tok, nf, _ = _lmhead(arc.Q6_K, dev(w), rows, K, h, None)
    assert tok == 0 and nf == 0


def test_lmhead_nonfinite_rows_are_skipped_and_counted():
    rows, K = 3000, 3584
    w = packed(arc.Q6_K, rows, K, 67).reshape(rows, -1).copy()
    h = arc.synth_normal(SEED, 68, K)
    ref = orc.gemv_r64(arc.Q6_K, w.ravel(), rows, K, h)
    top = int(np.argmax(ref))
    nb = K // 256
    # NaN d in one block of the top row, +inf d in another row
    w[top, 208:210] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)
    w[5, 210 * (nb - 1) + 208:210 * (nb - 1) + 210] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    tok, nf, logits = _lmhead(arc.Q6_K, dev(w.ravel()), rows, K, h, None)
    assert nf == 2
    assert not np.isfinite(logits[top]) and not np.isfinite(logits[5])
    t = orc.top2(logits)
    assert t.finite == 0
    assert tok == t.top1
    ref[top] = -np.inf
    ref[5] = -np.inf
    assert tok == int(np.argmax(ref))


LAYOUTS = [(1, 1), (1, 2), (2, 1), (2, 2), (4, 1), (4, 2), (8, 1), (8, 2), (16, 1)]


@pytest.mark.parametrize("bs,rpl", LAYOUTS)
def test_every_layout_fused_splitk_lmhead(bs, rpl):
    """Fused gate/up, one-column-per-split split-K and LM head under each
    forced lane layout (ragged rows, 14 and 74 super-block columns)."""
    rows, K = 301, 3584
    wg = packed(arc.Q4_K, rows, K, 70)
    wu = packed(arc.Q4_K, rows, K, 71)
    x = arc.synth_normal(SEED, 72, K)
    s = arc.DeviceBuffer(rows * 4)
    dr, dk = 77, 2560  # down-like: 10 columns, one per split
    wd = packed(arc.Q6_K, dr, dk, 73)
    xd = arc.synth_normal(SEED, 74, dk)
    part = arc.DeviceBuffer(10 * dr * 4)
    yd = arc.DeviceBuffer(dr * 4)
    wl = packed(arc.Q6_K, rows, K, 75)
    arc.tune_force(bs, rpl)
    try:
        arc.gateup_swiglu(arc.Q4_K, dev(wg), dev(wu), rows, K, dev(x), s)
        arc.gemv_splitk(arc.Q6_K, dev(wd), dr, dk, 10, dev(xd), part, yd)
        tok, nf, logits = _lmhead(arc.Q6_K, dev(wl), rows, K, x, None)
    finally:
        arc.tune_force(0, 0)
    g = orc.gemv_r64(arc.Q4_K, wg, rows, K, x)
    u = orc.gemv_r64(arc.Q4_K, wu, rows, K, x)
    assert orc.rel_err(s.download(np.float32), orc.swiglu_f64(g, u)) <= TOL
    rp = orc.splitk_r64(arc.Q6_K, wd, dr, dk, 10, xd)
    gp = part.download(np.float32).reshape(dr, 10).T
    for j in range(10):
        assert orc.rel_err(gp[j], rp[j]) <= TOL
    assert orc.rel_err(yd.download(np.float32), rp.sum(0)) <= TOL
    ref = orc.gemv_r64(arc.Q6_K, wl, rows, K, x)
    assert orc.rel_err(logits, ref) <= TOL
    assert tok == int(np.argmax(ref)) and nf == 0


def _pad_q6(w, rows, K):
    b = np.asarray(w, np.uint8).reshape(rows * (K // 256), 210)
    out = np.zeros((b.shape[0], 212), np.uint8)
    out[:, :210] = b
    return out.ravel()


@pytest.mark.parametrize("rows,K", [(1, 256), (37, 768), (3584, 18944)])
def test_q6_pad_image(rows, K):
    """arc_q6_pad writes each 210-byte block followed by two zero bytes, from
    a source that starts 2 bytes past a dword boundary too."""
    w = packed(arc.Q6_K, rows, K, 80)
    src = arc.DeviceBuffer(w.size + 2)
    src.upload(np.concatenate([np.zeros(2, np.uint8), w]))
    img = arc.DeviceBuffer(rows * (K // 256) * 212)
    arc.check(arc.lib().arc_q6_pad(src.ptr + 2, rows, K, img.ptr, None))
    arc.synchronize()
    assert np.array_equal(img.download(np.uint8), _pad_q6(w, rows, K))


@pytest.mark.parametrize("rows,K", [(37, 512), (1000, 3584), (3584, 18944)])
def test_padded_q6_gemv_and_dequant_bit_identical(rows, K):
    """The padded layout (the model's Q6_K tensors) gives the same bits as the
    GGUF layout: dequant, plain GEMV with bias, split-K with residual."""
    w = packed(arc.Q6_K, rows, K, 81)
    wp = _pad_q6(w, rows, K)
    x = dev(arc.synth_normal(SEED, 82, K))
    bias = dev(arc.synth_normal(SEED, 83, rows))
    d1, d2 = arc.DeviceBuffer(rows * K * 4), arc.DeviceBuffer(rows * K * 4)
    arc.dequant(arc.Q6_K, dev(w), rows, K, d1)
    arc.dequant(arc.Q6_K_PADDED, dev(wp), rows, K, d2)
    assert same_bits(d1.download(np.float32), d2.download(np.float32))
    y1, y2 = arc.DeviceBuffer(rows * 4), arc.DeviceBuffer(rows * 4)
    arc.gemv(arc.Q6_K, dev(w), rows, K, x, y1, bias=bias)
    arc.gemv(arc.Q6_K_PADDED, dev(wp), rows, K, x, y2, bias=bias)
    assert same_bits(y1.download(np.float32), y2.download(np.float32))
    ref = orc.gemv_r64(arc.Q6_K, w, rows, K, arc.synth_normal(SEED, 82, K))
    assert orc.rel_err(y2.download(np.float32) - bias.download(np.float32), ref) <= TOL
    nb = K // 256
    splits = min(nb, 74)
    part = arc.DeviceBuffer(splits * rows * 4)
    res = dev(arc.synth_normal(SEED, 84, rows))
    arc.gemv_splitk(arc.Q6_K, dev(w), rows, K, splits, x, part, y1, residual=res)
    arc.gemv_splitk(arc.Q6_K_PADDED, dev(wp), rows, K, splits, x, part, y2, residual=res)
    assert same_bits(y1.download(np.float32), y2.download(np.float32))


def test_padded_q6_lmhead_bit_identical():
    rows, K = 30000, 3584
    w = packed(arc.Q6_K, rows, K, 85)
    h = arc.synth_normal(SEED, 86, K)
    nw = arc.synth_normal(SEED, 87, K, 1.0, 0.05)
    t1, n1, l1 = _lmhead(arc.Q6_K, dev(w), rows, K, h, nw)
    t2, n2, l2 = _lmhead(arc.Q6_K_PADDED, dev(_pad_q6(w, rows, K)), rows, K, h, nw)
    assert (t1, n1) == (t2, n2) and same_bits(l1, l2)


def test_stream_probes_fold_the_same_chunks():
    """The streaming-read probes behind the bench's stream ceiling read what
    they are given: the plain and the non-temporal probe fold the same 16-byte
    chunks into the same per-thread words, equal to the fold computed here,
    for a size that is not a multiple of the grid's stride."""
    grid = 8
    n16 = grid * 256 * 3 + 77
    rng = np.random.default_rng(5)
    host = rng.integers(0, 2**32, size=n16 * 4, dtype=np.uint64).astype(np.uint32)
    buf = dev(host)
    want = np.zeros(grid * 256, dtype=np.uint32)
    chunks = np.bitwise_xor.reduce(host.reshape(n16, 4), axis=1)
    for i in range(n16):
        want[i % (grid * 256)] ^= chunks[i]
    o1, o2 = arc.DeviceBuffer(grid * 256 * 4), arc.DeviceBuffer(grid * 256 * 4)
    arc.probe_read(buf, n16 * 16, o1, grid)
    arc.probe_read_nt(buf, n16 * 16, o2, grid)
    assert np.array_equal(o1.download(np.uint32), want)
    assert np.array_equal(o2.download(np.uint32), want)
