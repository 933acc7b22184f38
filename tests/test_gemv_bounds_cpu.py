"""The bounds model of the packed GEMV (tests/gemv_bounds.py) over the
launchable layouts and epilogues of Q4_K, Q6_K (GGUF and padded 212-byte
blocks) and EXEC148, over grids from one workgroup to one wave tile per wave,
and over the Q6_K layouts with four rows per lane that the library refuses to
launch (one of them, k_gemv<Q6_K, 2, 4, PLAIN, 4>, took a GPU memory fault
once at 301 x 3584): every weight read, epilogue load, x pre-load and x
staging access, LDS access and store stays inside its buffer.  Also the
row-stream kernel, the F_EMBED embedding-row decode (every token id the
control block can hold) and the F_ARGNEXT argmax tail (best loads,
out_tokens stores, the next token).  A mistake planted in the model (an
unclamped row, block, token or step index) is reported."""
import itertools

import pytest

import gemv_bounds as gb

SHAPES = [(1, 256), (5, 512), (64, 3584), (301, 3584), (33, 18944)]


def grids(c):
    nb = c.K // 256
    tr = (64 // (4 * c.bs)) * c.rpl
    want = max(1, ((c.rows + tr - 1) // tr + c.waves - 1) // c.waves)
    return sorted({1, want})


def run(c, mistake=None):
    out = []
    for gx in grids(c):
        c.gx = gx
        r = gb.simulate(c, mistake)
        out.append((gx, r))
    return out


def cases():
    for fmt in (gb.Q4, gb.Q6, gb.E148, gb.Q6P):
        for (bs, rpl), W, (rows, K) in itertools.product(gb.built_layouts(fmt), (4, 8), SHAPES):
            nb = K // 256
            yield gb.Config(fmt, bs, rpl, gb.PLAIN, W, rows, K, tensor_align=2 if fmt == gb.Q6 else 0)
            if fmt == gb.Q4 and rpl <= 2:
                yield gb.Config(fmt, bs, rpl, gb.SWIGLU, W, rows, K)
            if nb >= 3:
                sb = (nb + 2) // 3
                yield gb.Config(fmt, bs, rpl, gb.PARTIAL, W, rows, K, splits=3, split_bps=sb, nsplit=3,
                                panel=min(sb, 74))
            if fmt != gb.E148:
                yield gb.Config(fmt, bs, rpl, gb.ARGMAX, W, rows, K)
            if bs >= 8 or rpl == 1:
                yield gb.Config(fmt, bs, rpl, gb.COLPART, W, rows, K, splits=nb, split_bps=1, nsplit=nb, panel=1)


def test_every_launchable_configuration_stays_in_bounds():
    n = 0
    for c in cases():
        for gx, r in run(c):
            assert not r.violations, (c, gx, r.violations)
            n += r.checked
    assert n > 10_000


@pytest.mark.parametrize("W", [4, 8])
@pytest.mark.parametrize("bs", [1, 2])
@pytest.mark.parametrize("align", [0, 2])
def test_refused_q6_four_rows_per_lane_layouts_stay_in_bounds(bs, W, align):
    """The refused layouts' index arithmetic is in bounds too, at the shape
    that faulted and around it: the fault's cause is not an index of
    gemv_body (the layout stays refused, its GPU cases skipped)."""
    for rows in (300, 301, 302, 3584):
        c = gb.Config(gb.Q6, bs, 4, gb.PLAIN, W, rows, 3584, tensor_align=align)
        for gx, r in run(c):
            assert not r.violations, (rows, gx, r.violations)


def test_qkrope_and_vstore_epilogues_stay_in_bounds():
    for fmt in (gb.Q4,):
        c = gb.Config(fmt, 4, 2, gb.QKROPE, 4, 3584 + 512, 3584, row_split=3584, kv_dim=512, pos=700, max_ctx=701)
        for gx, r in run(c):
            assert not r.violations, (gx, r.violations)
    for fmt in (gb.Q4, gb.Q6, gb.Q6P):
        c = gb.Config(fmt, 4, 1, gb.VSTORE, 4, 512, 3584, kv_dim=512, pos=0, max_ctx=1,
                      tensor_align=2 if fmt == gb.Q6 else 0)
        for gx, r in run(c):
            assert not r.violations, (gx, r.violations)


def test_attention_o_launch_gemv_part_stays_in_bounds():
    """The o projection's part of the attention + o launch: Q4_K, 8 quads
    per row, one row per lane, 4 waves, a ring of 3 buffers (the loads of
    two items go out before the wait for x), over one workgroup to one wave
    tile per wave, at the 7B shape and small ones."""
    for rows in (256, 1792, 3584):
        c = gb.Config(gb.Q4, 8, 1, gb.PLAIN, 4, rows, rows, ring=3)
        for gx, r in run(c):
            assert not r.violations, (rows, gx, r.violations)


@pytest.mark.parametrize("mistake", ["row", "block"])
def test_planted_index_mistake_is_reported(mistake):
    found = False
    for c in (gb.Config(gb.Q4, 2, 2, gb.PLAIN, 4, 301, 3584), gb.Config(gb.Q6, 4, 1, gb.PLAIN, 4, 5, 512)):
        for gx, r in run(c, mistake):
            found |= bool(r.violations)
    assert found


RS_SHAPES = [(1, 256), (4, 256), (37, 512), (301, 3584), (1000, 3584), (13, 2560)]


def rs_cases():
    for rows, K in RS_SHAPES:
        want = -(-rows // gb.RS_WAVES)
        for gx in sorted({1, min(want, 3), want, min(want, 256)}):
            for ring in (2, 3, 4):
                yield rows, K, gb.PLAIN, False, gx, ring
                yield rows, K, gb.SWIGLU, True, gx, ring
                yield rows, K, gb.SWIGLU, False, gx, ring


def test_row_stream_launches_stay_in_bounds():
    """The row-stream Q4_K kernel (plain and gate/up + SwiGLU, with and
    without the fused norm) for 1 to 14 super-blocks per row, ragged row
    counts, ring depths 2 to 4 and grids from one workgroup to one row per
    wave."""
    bad = []
    n = 0
    for rows, K, epi, norm, gx, ring in rs_cases():
        r = gb.simulate_rs(rows, K, epi, norm, gx, ring)
        n += r.checked
        if r.violations:
            bad.append(((rows, K, epi, norm, gx, ring), r.violations[:3]))
    assert n > 0
    assert not bad, bad


@pytest.mark.parametrize("mistake", ["block", "row"])
def test_row_stream_planted_mistake_is_reported(mistake):
    # 2 super-blocks: owner lanes of blocks 2 .. 13 sit past the row
    r = gb.simulate_rs(37, 512, gb.PLAIN, False, 2, mistake=mistake)
    assert r.violations


def test_embedding_row_decode_stays_in_bounds():
    """F_EMBED: every token id the control block can hold -- in range, the
    last row, one past it and the largest uint32 -- decodes inside the
    token table; the raw row stays inside h_out."""
    for nb, rows in ((14, 152064), (2, 4096), (1, 1)):
        r = gb.simulate_embed(nb, rows, [0, 1, rows - 1, rows, rows + 7, 2**32 - 1])
        assert r.checked > 0
        assert not r.violations, (nb, rows, r.violations)


def test_argmax_tail_stays_in_bounds():
    """F_ARGNEXT: the best-of-workgroup loads, the out_tokens store at every
    step up to past the cap, and the token handed to the next step."""
    for rows, n in ((152064, 1024), (4096, 37), (5, 1)):
        r = gb.simulate_argnext(rows, n, n, 64, range(0, 70), [0, rows - 1, rows, 2**32 - 1])
        assert not r.violations, (rows, n, r.violations)


@pytest.mark.parametrize("mistake", ["token"])
def test_embedding_planted_mistake_is_reported(mistake):
    assert gb.simulate_embed(14, 100, [100], mistake).violations


@pytest.mark.parametrize("mistake", ["step", "idx"])
def test_argmax_tail_planted_mistake_is_reported(mistake):
    assert gb.simulate_argnext(100, 10, 10, 64, range(0, 70), [0, 100], mistake).violations
