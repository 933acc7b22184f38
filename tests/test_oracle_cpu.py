"""Pins the CPU oracle (oracle/arc_oracle.c) before it is trusted as the
GPU checker:

* golden vectors written by the reference's own code (tests/golden/, made by
  tests/golden/make_golden.py through oracle/_ref): binary16 table, Q6_K
  decode and GEMV arms over the reference's five fixture strata, Q4_K
  canonical tuples;
* the reference's own known-answer program (tests/q4_down_exec148_synthetic.cpp)
  when oracle/_ref is built;
* library routines: numpy's binary16 conversion, float64 matrix products,
  scipy's expit, complex rotation;
* inverse encoders (the packers of tests/q4_down_exec148_synthetic.cpp:7-8 and
  tests/test_q6cb1_package.py:113-138 restated), closed forms and invariants.
"""
import json
import os
import subprocess

import numpy as np
import pytest
from scipy.special import expit

import oracle_lib as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
O = orc.oracle()


def _p(a):
    return a.ctypes.data


# ------------------------------------------------------------------ fp16
def test_half_to_float_matches_reference_table():
    ref = np.load(os.path.join(GOLD, "half_table.npz"))["bits"]
    got = np.array([O.orc_half_to_float(h) for h in range(65536)], np.float32).view(np.uint32)
    assert np.array_equal(got, ref)


def test_half_to_float_matches_numpy_except_nan_payload():
    bits = np.arange(65536, dtype=np.uint16)
    np_f = bits.view(np.float16).astype(np.float32)
    got = np.array([O.orc_half_to_float(int(h)) for h in bits], np.float32)
    nan = np.isnan(np_f)
    assert np.array_equal(got[~nan].view(np.uint32), np_f[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    # the reference maps every NaN payload to one quiet NaN
    assert np.all(got[nan].view(np.uint32) == np.float32("nan").view(np.uint32))


def test_float_to_half_rne_matches_numpy():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),
        (rng.standard_normal(20000) * 1e4).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, np.inf, -np.inf, 5.96e-8, 2.98e-8,
                  2.9802322e-08, 8.9406967e-08, 6.1035156e-05, 6.0975552e-05], np.float32),
        # exact ties between adjacent binary16 values
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -24) + np.float32(2.0 ** -25)),
        (np.float32(1.0) + np.arange(0, 1024, dtype=np.float32) * np.float32(2.0 ** -10) + np.float32(2.0 ** -11)),
    ])
    got = np.array([O.orc_float_to_half_rne(float(v)) for v in vals], np.uint16)
    exp = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


# ------------------------------------------------------------------ Q6_K
@pytest.fixture(scope="module")
def q6gold():
    return np.load(os.path.join(GOLD, "q6_fixtures.npz"))


@pytest.mark.parametrize("stratum", range(5))
def test_q6_decode_matches_reference(q6gold, stratum):
    p = f"s{stratum}_"
    packed = q6gold[p + "packed"]
    nblk = packed.size // 210
    q = np.zeros(nblk * 256, np.int32)
    sc = np.zeros_like(q)
    val = np.zeros(nblk * 256, np.float32)
    s = orc.C.c_int()
    for b in range(nblk):
        blk = np.ascontiguousarray(packed[b * 210:(b + 1) * 210])
        for k in range(256):
            q[b * 256 + k] = O.orc_q6k_code(_p(blk), k, orc.C.byref(s))
            sc[b * 256 + k] = s.value
            val[b * 256 + k] = O.orc_q6k_weight(_p(blk), k)
    assert np.array_equal(q, q6gold[p + "q"])
    assert np.array_equal(sc, q6gold[p + "scale"])
    assert np.array_equal(val.view(np.uint32), q6gold[p + "value_bits"])
    # the reference generator's semantic invariant: codes it wrote decode back
    assert np.array_equal(q, q6gold[p + "expected_q"].astype(np.int32))


@pytest.mark.parametrize("stratum", range(5))
def test_q6_gemv_arms_match_reference(q6gold, stratum):
    p = f"s{stratum}_"
    packed, x = q6gold[p + "packed"], q6gold[p + "x"]
    n, rows = int(q6gold["n"]), int(q6gold["rows"])
    r64 = orc.gemv_r64(orc.Q6_K, packed, rows, n, x)
    assert np.array_equal(r64.view(np.uint64), q6gold[p + "r64"].view(np.uint64))  # same order -> bit-exact
    s32 = orc.gemv_r0(orc.Q6_K, packed, rows, n, x)
    assert np.array_equal(s32.view(np.uint32), q6gold[p + "s32_bits"])


def _set_q6_code(block, k, code):
    """Q6_K code setter restated from tests/test_q6cb1_package.py:113-128."""
    half, kk = k >> 7, k & 127
    l, quarter = kk & 31, kk >> 5
    ql, qh = half * 64, 128 + half * 32
    lo, hi = code & 15, (code >> 4) & 3
    if quarter == 0:
        block[ql + l] = (block[ql + l] & 0xF0) | lo
        block[qh + l] = (block[qh + l] & 0xFC) | hi
    elif quarter == 1:
        block[ql + l + 32] = (block[ql + l + 32] & 0xF0) | lo
        block[qh + l] = (block[qh + l] & 0xF3) | (hi << 2)
    elif quarter == 2:
        block[ql + l] = (block[ql + l] & 0x0F) | (lo << 4)
        block[qh + l] = (block[qh + l] & 0xCF) | (hi << 4)
    else:
        block[ql + l + 32] = (block[ql + l + 32] & 0x0F) | (lo << 4)
        block[qh + l] = (block[qh + l] & 0x3F) | (hi << 6)


def test_q6_code_roundtrip_known_answer():
    # tests/test_q6cb1_package.py:129-138: code = (k*37+11) & 63 round-trips
    block = np.zeros(210, np.uint8)
    for k in range(256):
        _set_q6_code(block, k, (k * 37 + 11) & 63)
    s = orc.C.c_int()
    for k in range(256):
        assert O.orc_q6k_code(_p(block), k, orc.C.byref(s)) + 32 == (k * 37 + 11) & 63


def test_q6_scale_index_and_value_closed_form():
    rng = np.random.default_rng(11)
    block = rng.integers(0, 256, 210, dtype=np.uint8)
    block[208:210] = [0x00, 0x3C]  # d = 1.0
    codes = rng.integers(0, 64, 256)
    for k in range(256):
        _set_q6_code(block, k, int(codes[k]))
    s = orc.C.c_int()
    for k in range(256):
        q = O.orc_q6k_code(_p(block), k, orc.C.byref(s))
        half, kk = k >> 7, k & 127
        slot = half * 8 + (kk & 31) // 16 + 2 * (kk >> 5)
        assert s.value == int(block[192 + slot].astype(np.int8))
        assert q == codes[k] - 32
        assert O.orc_q6k_weight(_p(block), k) == np.float32(1.0) * np.float32(s.value) * np.float32(q)


# ------------------------------------------------------------------ Q4_K
def _sm(b, s, m):
    """Q4_K scale/min packer restated from tests/q4_down_exec148_synthetic.cpp:7."""
    for j in range(4):
        b[4 + j] = (b[4 + j] & 0xC0) | (s[j] & 63)
        b[8 + j] = (b[8 + j] & 0xC0) | (m[j] & 63)
    for j in range(4, 8):
        b[j] = (b[j] & 63) | ((s[j] >> 4) << 6)
        b[4 + j] = (b[4 + j] & 63) | ((m[j] >> 4) << 6)
        b[8 + j] = ((m[j] & 15) << 4) | (s[j] & 15)


def _sq(b, k, q):
    """Q4_K nibble packer restated from tests/q4_down_exec148_synthetic.cpp:8."""
    g, w = k // 64, k % 64
    o = 16 + g * 32 + (w % 32)
    b[o] = (b[o] & 0xF0) | (q & 15) if w < 32 else (b[o] & 15) | ((q & 15) << 4)


@pytest.mark.parametrize("case", range(8))
def test_q4_inverse_encoder_roundtrip(case):
    rng = np.random.default_rng(100 + case)
    b = rng.integers(0, 256, 144, dtype=np.uint8)
    edge = case % 2 == 1
    s = [(63 if j & 1 else 0) if edge else int(rng.integers(0, 64)) for j in range(8)]
    m = [(0 if j & 1 else 63) if edge else int(rng.integers(0, 64)) for j in range(8)]
    _sm(b, s, m)
    qs = rng.integers(0, 16, 256) if case < 4 else np.full(256, 15 * (case & 1))
    for k in range(256):
        _sq(b, k, int(qs[k]))
    sc, mn = orc.C.c_uint32(), orc.C.c_uint32()
    for j in range(8):
        O.orc_q4k_scale_min(_p(b), j, orc.C.byref(sc), orc.C.byref(mn))
        assert (sc.value, mn.value) == (s[j], m[j])
    for k in range(256):
        assert O.orc_q4k_code(_p(b), k) == qs[k]


def test_q4_decode_matches_reference_tuples():
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    table = np.load(os.path.join(GOLD, "half_table.npz"))["bits"].view(np.float32)
    sc, mn = orc.C.c_uint32(), orc.C.c_uint32()
    for blk, t in zip(g["blocks"], g["tuples"]):
        blk = np.ascontiguousarray(blk)
        for j in range(8):
            O.orc_q4k_scale_min(_p(blk), j, orc.C.byref(sc), orc.C.byref(mn))
            assert (sc.value, mn.value) == (t[4 + 2 * j], t[5 + 2 * j])
        codes = np.array([O.orc_q4k_code(_p(blk), k) for k in range(256)])
        assert np.array_equal(codes, t[20:276])
        # the fp32 affine step on the reference's decoded fields, IEEE single
        # rounding per operation: (d*sc)*q - dmin*mn
        d = table[int(t[0]) | (int(t[1]) << 8)]
        dm = table[int(t[2]) | (int(t[3]) << 8)]
        with np.errstate(all="ignore"):
            for k in range(256):
                j = k >> 5
                exp = np.float32(np.float32(d * np.float32(t[4 + 2 * j])) * np.float32(codes[k])) - \
                    np.float32(dm * np.float32(t[5 + 2 * j]))
                got = np.float32(O.orc_q4k_weight(_p(blk), k))
                assert (got.view(np.uint32) == exp.view(np.uint32)) or (np.isnan(got) and np.isnan(exp))


def test_exec148_reference_known_answer():
    if not os.path.exists(orc.REF_KAT):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    out = subprocess.run([orc.REF_KAT], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "EXEC148_SYNTHETIC=PASS" in out.stdout


def test_sha256_known_answers():
    kat = json.load(open(os.path.join(GOLD, "sha256_kat.json")))
    import hashlib
    assert kat["abc"] == hashlib.sha256(b"abc").hexdigest()
    assert kat["empty"] == hashlib.sha256(b"").hexdigest()
    ex = np.load(os.path.join(GOLD, "q4_tuples.npz"))["exec148"]
    assert kat["exec148_2rows"] == hashlib.sha256(bytes(ex[:8].ravel())).hexdigest()


def test_exec148_layout_against_oracle_decode():
    """EXEC148 (148-byte) blocks hold unpacked (sc, mn) bytes and sequential
    nibble pairs; they must agree with the oracle's Q4_K decode."""
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    sc, mn = orc.C.c_uint32(), orc.C.c_uint32()
    for blk, e in zip(g["blocks"][:20], g["exec148"][:20]):
        blk = np.ascontiguousarray(blk)
        assert np.array_equal(e[:4], blk[:4])
        for j in range(8):
            O.orc_q4k_scale_min(_p(blk), j, orc.C.byref(sc), orc.C.byref(mn))
            assert (e[4 + 2 * j], e[5 + 2 * j]) == (sc.value, mn.value)
        for k in range(256):
            q = (e[20 + (k >> 1)] >> (4 * (k & 1))) & 15
            assert q == O.orc_q4k_code(_p(blk), k)


def test_exec148_oracle_matches_reference_materializer():
    """orc_exec148_block against the blocks the reference's own materializer
    (src/q4_down_exec148_materializer.h) wrote into the golden file, and both
    canonical tuples against the reference validator's source tuples."""
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    e = np.zeros(148, np.uint8)
    t1, t2 = np.zeros(276, np.uint8), np.zeros(276, np.uint8)
    for blk, ref_e, ref_t in zip(g["blocks"], g["exec148"], g["tuples"]):
        blk = np.ascontiguousarray(blk)
        O.orc_exec148_block(_p(blk), _p(e))
        assert np.array_equal(e, ref_e)
        O.orc_q4k_canon(_p(blk), _p(t1))
        O.orc_exec148_canon(_p(e), _p(t2))
        assert np.array_equal(t1, ref_t) and np.array_equal(t2, ref_t)
        # route-B element values equal the Q4_K element decode bit for bit
        for k in range(0, 256, 7):
            a = np.float32(O.orc_exec148_weight(_p(e), k))
            b = np.float32(O.orc_q4k_weight(_p(blk), k))
            assert a.view(np.uint32) == b.view(np.uint32) or (np.isnan(a) and np.isnan(b))


def test_exec148_tuple_mismatch_is_detected():
    """A flipped nibble or scale byte in an EXEC148 block changes its canonical
    tuple (what validation compares)."""
    g = np.load(os.path.join(GOLD, "q4_tuples.npz"))
    blk = np.ascontiguousarray(g["blocks"][3])
    e = np.zeros(148, np.uint8)
    O.orc_exec148_block(_p(blk), _p(e))
    t0, t1 = np.zeros(276, np.uint8), np.zeros(276, np.uint8)
    O.orc_q4k_canon(_p(blk), _p(t0))
    for pos, mask in ((4, 1), (19, 32), (20, 1), (147, 0x10)):
        bad = e.copy()
        bad[pos] ^= mask
        O.orc_exec148_canon(_p(bad), _p(t1))
        assert not np.array_equal(t0, t1)


def test_sha256_oracle_known_answers_and_hashlib():
    """orc_sha256 against the reference's Sha256 outputs (golden KATs) and
    against hashlib on every length 0..200 (all padding cases)."""
    import hashlib
    kat = json.load(open(os.path.join(GOLD, "sha256_kat.json")))
    assert orc.sha256(np.frombuffer(b"abc", np.uint8)) == kat["abc"]
    assert orc.sha256(np.zeros(0, np.uint8)) == kat["empty"]
    ex = np.load(os.path.join(GOLD, "q4_tuples.npz"))["exec148"]
    assert orc.sha256(ex[:8]) == kat["exec148_2rows"]
    rng = np.random.default_rng(5)
    for n in range(0, 201):
        b = rng.integers(0, 256, n, dtype=np.uint8)
        assert orc.sha256(b) == hashlib.sha256(bytes(b)).hexdigest(), n
    big = rng.integers(0, 256, 1 << 16, dtype=np.uint8)
    assert orc.sha256(big) == hashlib.sha256(bytes(big)).hexdigest()


# ------------------------------------------------------------------ GEMV
def _synthetic(qtype, rows, K, seed):
    rng = np.random.default_rng(seed)
    bb = orc.BLOCK_BYTES[qtype]
    w = rng.integers(0, 256, rows * (K // 256) * bb, dtype=np.uint8).reshape(-1, bb)
    d = np.abs(rng.standard_normal(len(w)) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if qtype == orc.Q4_K:
        w[:, 0:2] = d
        w[:, 2:4] = np.abs(rng.standard_normal(len(w)) * 0.005).astype(np.float16).view(np.uint8).reshape(-1, 2)
    else:
        w[:, 208:210] = d
    return w.ravel(), rng.standard_normal(K).astype(np.float32)


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K])
def test_r64_matches_float64_matmul(qtype):
    rows, K = 40, 1536
    w, x = _synthetic(qtype, rows, K, 5)
    deq = orc.dequant(qtype, w, rows, K).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    got = orc.gemv_r64(qtype, w, rows, K, x)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K])
def test_block_dequant_equals_per_element_decode(qtype):
    """orc_dequant decodes a block at a time; it must equal the per-element
    definition bit for bit, random bytes and special halves included."""
    rows, K = 6, 512
    bb = orc.BLOCK_BYTES[qtype]
    rng = np.random.default_rng(61)
    w = rng.integers(0, 256, rows * (K // 256) * bb, dtype=np.uint8)
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03ff, 0x7bff, 0x7c00, 0xfc00, 0x7e00], np.uint16)
    off = 0 if qtype == orc.Q4_K else 208
    blocks = w.reshape(-1, bb)
    for i in range(len(blocks)):
        j = i % len(specials)
        blocks[i, off:off + 2] = specials[j:j + 1].view(np.uint8)
    deq = orc.dequant(qtype, w, rows, K)
    fn = O.orc_q4k_weight if qtype == orc.Q4_K else O.orc_q6k_weight
    per = np.array([[fn(_p(blocks[r * (K // 256) + k // 256]), k % 256) for k in range(K)] for r in range(rows)],
                   np.float32)
    assert np.array_equal(deq.view(np.uint32), per.view(np.uint32))


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K])
def test_r64_one_hot_is_column(qtype):
    rows, K = 16, 512
    w, _ = _synthetic(qtype, rows, K, 6)
    deq = orc.dequant(qtype, w, rows, K)
    for k in (0, 33, 255, 256, 511):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        assert np.array_equal(orc.gemv_r64(qtype, w, rows, K, x), deq[:, k].astype(np.float64))


def test_r0_bias_and_splitk_consistency():
    rows, K = 12, 2560
    w, x = _synthetic(orc.Q6_K, rows, K, 7)
    b = np.linspace(-1, 1, rows).astype(np.float32)
    r64 = orc.gemv_r64(orc.Q6_K, w, rows, K, x, b)
    r0 = orc.gemv_r0(orc.Q6_K, w, rows, K, x, b)
    assert orc.rel_err(r0, r64) < 1e-4
    for splits in (1, 3, 10):
        part = orc.splitk_r64(orc.Q6_K, w, rows, K, splits, x)
        np.testing.assert_allclose(part.sum(0) + b, r64, rtol=1e-12, atol=1e-12)
    mt = orc.gemv_r0(orc.Q6_K, w, rows, K, x, b, threads=4)
    assert np.array_equal(mt.view(np.uint32), r0.view(np.uint32))


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K])
def test_splitk_partials_are_r64_of_their_column_slices(qtype):
    """Brute force: partial j of orc_gemv_splitk_r64 is, bit for bit, R64 of
    the sub-tensor made of the super-block columns [j*bps, min((j+1)*bps, nb))
    of every row against the matching slice of x; splits past the last
    column are zero."""
    rows, K = 9, 2560
    nb, bb = K // 256, orc.BLOCK_BYTES[qtype]
    w, x = _synthetic(qtype, rows, K, 17)
    w2 = w.reshape(rows, nb * bb)
    for splits in (1, 3, 4, 7, 10):
        bps = -(-nb // splits)
        part = orc.splitk_r64(qtype, w, rows, K, splits, x)
        for j in range(splits):
            b0, b1 = j * bps, min((j + 1) * bps, nb)
            if b0 >= nb:
                assert not part[j].any()
                continue
            sub = np.ascontiguousarray(w2[:, b0 * bb:b1 * bb]).ravel()
            ref = orc.gemv_r64(qtype, sub, rows, (b1 - b0) * 256, np.ascontiguousarray(x[b0 * 256:b1 * 256]))
            assert np.array_equal(part[j].view(np.uint64), ref.view(np.uint64)), (splits, j)


# ----------------------------------------------------- norm / act / rope
def test_rmsnorm_matches_formula():
    rng = np.random.default_rng(8)
    x = rng.standard_normal(3584).astype(np.float32)
    w = (1 + 0.05 * rng.standard_normal(3584)).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    np.testing.assert_allclose(orc.rmsnorm_f64(x, w, 1e-6), ref, rtol=1e-13)
    np.testing.assert_allclose(orc.rmsnorm_f32(x, w, 1e-6), ref, rtol=2e-6)


def test_swiglu_matches_expit():
    g = np.linspace(-30, 30, 4001)
    u = np.cos(g)
    np.testing.assert_allclose(orc.swiglu_f64(g, u), g * expit(g) * u, rtol=1e-14, atol=1e-300)
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    s = np.empty_like(g32)
    O.orc_swiglu_f32(_p(g32), _p(u32), len(g32), _p(s))
    np.testing.assert_allclose(s, g * expit(g) * u, rtol=3e-6, atol=1e-30)


def test_rope_adjacent_pairs_match_complex_rotation():
    heads, dim, pos, theta = 4, 128, 1234, 1e6
    rng = np.random.default_rng(9)
    x = rng.standard_normal(heads * dim)
    y = x.copy()
    O.orc_rope_f64(_p(y), heads, dim, pos, theta)
    z = x.reshape(heads, dim // 2, 2)
    c = z[..., 0] + 1j * z[..., 1]  # adjacent (2p, 2p+1) pairs, not NeoX halves
    ang = pos * theta ** (-2.0 * np.arange(dim // 2) / dim)
    r = c * np.exp(1j * ang)
    np.testing.assert_allclose(y.reshape(heads, dim // 2, 2)[..., 0], r.real, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y.reshape(heads, dim // 2, 2)[..., 1], r.imag, rtol=1e-12, atol=1e-12)
    x32 = x.astype(np.float32)
    O.orc_rope_f32(_p(x32), heads, dim, pos, np.float32(theta))
    np.testing.assert_allclose(x32, y, rtol=0, atol=5e-3)  # float angle at pos 1234


def test_top2_ties_nonfinite_and_signed_zero():
    v = np.array([1.0, 3.0, 3.0, -np.inf, np.nan, 2.0, 3.0], np.float32)
    t = orc.top2(v)
    # ties -> lowest index is top-1; the equal value at index 2 becomes top-2
    assert (t.top1, t.top2, t.finite) == (1, 2, 0)
    w = np.array([-0.0, 0.0, -1.0], np.float32)
    t = orc.top2(w)
    assert (t.top1, t.top2, t.finite) == (0, 1, 1)  # +0.0 == -0.0: the first index stays top-1
    rng = np.random.default_rng(10)
    r = rng.standard_normal(100000).astype(np.float32)
    r[[500, 90000]] = r.max() + 1
    assert orc.top2(r).top1 == int(np.argmax(r)) == 500


def test_attention_decode_matches_softmax():
    qh, kvh, dim, pos = 28, 4, 128, 37
    rng = np.random.default_rng(12)
    q = rng.standard_normal(qh * dim)
    kc = rng.standard_normal((pos + 1) * kvh * dim).astype(np.float16)
    vc = rng.standard_normal((pos + 1) * kvh * dim).astype(np.float16)
    out = np.empty(qh * dim)
    O.orc_attention_decode_f64(_p(q), _p(kc.view(np.uint16)), _p(vc.view(np.uint16)), pos, qh, kvh, dim, _p(out))
    K = kc.astype(np.float64).reshape(pos + 1, kvh, dim)
    V = vc.astype(np.float64).reshape(pos + 1, kvh, dim)
    Q = q.reshape(qh, dim)
    for h in range(qh):
        kh = h // (qh // kvh)
        s = K[:, kh, :] @ Q[h] / np.sqrt(dim)
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[h * dim:(h + 1) * dim], p @ V[:, kh, :], rtol=1e-12, atol=1e-12)
