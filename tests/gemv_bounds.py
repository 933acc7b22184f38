"""CPU bounds model of the packed GEMV workgroup body (gemv_body in
arcllm_amd/csrc/arc_gemv.hpp) and of its launch (launch_one): for one
configuration it enumerates, for every lane of every workgroup and split,
the byte ranges the kernel reads from the weight tensor (its prefetch ring
included: the PF - 1 loads issued before the first item and, past the last
item, the repeated loads of that item), the epilogue operands it loads
(load_ep), the x elements and LDS words of the x staging (stage_x,
stage_x_rms, put_group), the LDS words the dot products read (compute), the
split-K column LDS (finish_column) and every global store (finish,
finish_column), and reports each access outside its buffer.

The index formulas are those of the kernel source, restated here in numpy
over arrays of lanes; the model is test infrastructure (a checker), not
part of the product.  `mistake` plants a known error in the model (an
unclamped row or block index) so a test can show the checker catches it.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

Q4, Q6, E148, Q6P = 12, 14, 148, 214
BLOCK_BYTES = {Q4: 144, Q6: 210, E148: 148, Q6P: 212}
KQK, XBLK, SLOT, WAVE = 256, 272, 68, 64
PLAIN, SWIGLU, PARTIAL, ARGMAX, COLPART, QKROPE, VSTORE = range(7)
RING = 2  # ARC_PF_Q4 / ARC_PF_Q6 / ARC_PF_E148 (ring_depth)


@dataclass
class Config:
    fmt: int
    bs: int
    rpl: int
    epi: int
    waves: int
    rows: int
    K: int
    splits: int = 1
    split_bps: int | None = None  # default: all of K
    kb_off: int = 0
    panel: int | None = None      # default: min(nb, 74)
    gx: int | None = None         # default: the largest launch_one makes (one wave tile per wave)
    tensor_align: int = 0         # tensor base address mod 4 (Q6_K: 0 or 2)
    nsplit: int = 1               # PARTIAL / COLPART partial columns per row
    row_split: int = 0            # QKROPE: first row of w1
    kv_dim: int = 0               # QKROPE / VSTORE cache row width
    pos: int = 0
    max_ctx: int = 1
    ring: int = RING              # register buffers (a GEMV that waits for its x takes one more)


@dataclass
class Report:
    violations: list = field(default_factory=list)
    checked: int = 0

    def bad(self, what, mask, values, limit):
        if np.any(mask):
            v = np.asarray(values)[mask]
            self.violations.append(f"{what}: {int(mask.sum())} accesses, e.g. {int(v.flat[0])} vs limit {limit}")

    def check(self, what, lo, hi, lo_ok, hi_ok):
        """Every half-open range [lo, hi) inside [lo_ok, hi_ok)."""
        lo = np.asarray(lo, np.int64)
        hi = np.asarray(hi, np.int64)
        self.checked += lo.size
        self.bad(what + " below start", lo < lo_ok, lo, lo_ok)
        self.bad(what + " past end", hi > hi_ok, hi, hi_ok)


def x_group_offset(fmt, v, t):
    """arc_device.hpp x_group_offset (element offset of group t of lane slot v)."""
    if fmt == E148:
        return v * 64 + t * 16
    if fmt == Q4:
        c = v + 4 * (t >> 1)
        return (c >> 1) * 64 + (t & 1) * 32 + (c & 1) * 16
    qa = v >> 1
    q = np.where(t & 1, qa + 2, qa)
    return (t >> 1) * 128 + q * 32 + (v & 1) * 16


def block_reads(fmt, v, blk_off, tensor_align):
    """Byte ranges [lo, hi) of one lane's block loads, relative to the tensor
    base (q4_load, e148_load, q6_load, q6p_load)."""
    if fmt == Q4:
        return [(blk_off, blk_off + 4), (blk_off + 4, blk_off + 16), (blk_off + 16 + v * 16, blk_off + 32 + v * 16),
                (blk_off + 80 + v * 16, blk_off + 96 + v * 16)]
    if fmt == E148:
        return [(blk_off, blk_off + 4), (blk_off + 4 + 4 * v, blk_off + 8 + 4 * v),
                (blk_off + 20 + 32 * v, blk_off + 36 + 32 * v), (blk_off + 36 + 32 * v, blk_off + 52 + 32 * v)]
    if fmt == Q6P:
        # padded Q6_K: the five 16-byte pieces at their own (dword) addresses
        # and the dword at 208 holding d
        return [(blk_off + o, blk_off + o + 16) for o in (v * 16, 64 + v * 16, 128 + (v & 1) * 16, 160 + (v & 1) * 16,
                                                           192 + 0 * v)] + [(blk_off + 208 + 0 * v, blk_off + 212 + 0 * v)]
    # Q6_K: a dwordx4 plus the following dword from the dword boundary at or
    # below each piece (the descriptor base sits at that boundary too)
    sh = (blk_off + tensor_align) & 3
    a = blk_off - sh
    out = []
    for o in (v * 16, 64 + v * 16, 128 + (v & 1) * 16, 160 + (v & 1) * 16, 192 + 0 * v):
        out.append((a + o, a + o + 20))
    return out


def simulate(c: Config, mistake: str | None = None) -> Report:
    rep = Report()
    nb = c.K // KQK
    kBB = BLOCK_BYTES[c.fmt]
    row_bytes = nb * kBB
    nmat = 2 if c.epi == SWIGLU else 1
    RG = WAVE // (4 * c.bs)
    TR = RG * c.rpl
    ntiles = (c.rows + TR - 1) // TR
    split_bps = c.split_bps if c.split_bps is not None else nb
    panel = c.panel if c.panel is not None else min(nb, 74)
    W = c.waves
    want = (ntiles + W - 1) // W
    gx = c.gx if c.gx is not None else max(1, want)
    assert 1 <= gx <= max(1, want)
    lds_words = panel * XBLK + (W * TR * panel if c.epi == COLPART else 0)
    # tensor bytes per matrix (QKROPE: w0 has row_split rows, w1 the rest)
    mat_rows = [c.row_split, c.rows - c.row_split] if c.epi == QKROPE else [c.rows] * nmat
    mat_bytes = [r * row_bytes for r in mat_rows]
    if c.fmt in (Q6, Q6P):
        lo_ok = -c.tensor_align
        hi_ok = [b + 4 for b in mat_bytes]  # the descriptor's range (tensor_rsrc)
    else:
        lo_ok = 0
        hi_ok = mat_bytes

    lane = np.arange(WAVE)
    v = lane & 3
    bs = (lane >> 2) % c.bs
    rg = lane // (4 * c.bs)

    clamp_row = (lambda r: np.minimum(r, c.rows)) if mistake == "row" else (lambda r: np.minimum(r, c.rows - 1))
    clamp_bl = (lambda b, n: b) if mistake == "block" else (lambda b, n: np.minimum(b, n - 1))

    for split in range(c.splits):
        kb = split * split_bps + c.kb_off
        split_end = min((split + 1) * split_bps, nb)
        if kb >= split_end:
            continue
        nbl = min(panel, split_end - kb)
        nj = (nbl + c.bs - 1) // c.bs
        # x staging (stage_x from column kb, or stage_x_rms over all of x):
        # group gi of nbl * 16, its 16 elements of x and its LDS slot
        gi = np.arange(nbl * 16)
        e = (kb + (gi >> 4)) * KQK + x_group_offset(c.fmt, (gi >> 2) & 3, gi & 3)
        rep.check("x staging read", e, e + 16, 0, nb * KQK)
        dst = (gi >> 4) * XBLK + ((gi >> 2) & 3) * SLOT + (gi & 3) * 16
        rep.check("x staging LDS store", dst, dst + 16, 0, panel * XBLK)
        sdst = (gi >> 4) * XBLK + ((gi >> 2) & 3) * SLOT + 64 + (gi & 3)
        rep.check("x group-sum LDS store", sdst, sdst + 1, 0, panel * XBLK)
        # x_pre: each thread's groups loaded ahead of the ring, indices clamped
        # into the panel (8-wave launches: all groups of an 80-block panel;
        # 4-wave: the first), and with the fused norm its first group of the
        # norm weights
        NT = W * WAVE
        G = -(-(80 * 16) // NT) if NT >= 512 else 1
        t = np.arange(NT)
        for i in range(G):
            gp = np.minimum(t + i * NT, nbl * 16 - 1)
            ep = (kb + (gp >> 4)) * KQK + x_group_offset(c.fmt, (gp >> 2) & 3, gp & 3)
            rep.check("x pre-load", ep, ep + 16, 0, nb * KQK)
        if kb == 0 and nbl == nb:
            gp = np.minimum(t, nbl * 16 - 1)
            ep = (gp >> 4) * KQK + x_group_offset(c.fmt, (gp >> 2) & 3, gp & 3)
            rep.check("norm weight pre-load", ep, ep + 16, 0, nb * KQK)

        for bx in range(gx):
            for wave in range(W):
                gw = bx * W + wave
                stride = gx * W
                my_tiles = (ntiles - gw + stride - 1) // stride if gw < ntiles else 0
                S = my_tiles * nj

                def rows_of(ti):
                    tile = min(gw + ti * stride, ntiles - 1)
                    return [clamp_row(tile * TR + rg * c.rpl + r) for r in range(c.rpl)]

                def load(li, lj):
                    bl = clamp_bl(bs + c.bs * lj, nbl)
                    for m in range(nmat):
                        for row in rows_of(li):
                            if c.epi == QKROPE:
                                in0 = row < c.row_split
                                rr = np.where(in0, row, row - c.row_split)
                                for mi, sel in ((0, in0), (1, ~in0)):
                                    if not np.any(sel):
                                        continue
                                    off = rr[sel] * row_bytes + (kb + bl[sel]) * kBB
                                    for lo, hi in block_reads(c.fmt, v[sel], off, c.tensor_align):
                                        rep.check(f"weight read (w{mi})", lo, hi, lo_ok, hi_ok[mi])
                            else:
                                off = row * row_bytes + (kb + bl) * kBB
                                for lo, hi in block_reads(c.fmt, v, off, c.tensor_align):
                                    rep.check(f"weight read (w{m})", lo, hi, lo_ok, hi_ok[m])

                # the ring: PF-1 loads before the first item, one per item;
                # load k reads item min(k, S-1) (item 0 when S = 0)
                for k in range(c.ring - 1 + S):
                    it = min(k, S - 1) if S > 0 else 0
                    load(it // nj, it % nj)

                # epilogue operands: tile 0 before the loop, then each tile's first item
                for ti in range(max(1, my_tiles)):
                    for row in rows_of(ti):
                        if c.epi in (PLAIN, COLPART, VSTORE, QKROPE):
                            rep.check("epilogue row operand", row, row + 1, 0, c.rows)
                        if c.epi == PARTIAL:
                            idx = row * c.nsplit + split
                            rep.check("partial accumulate load", idx, idx + 1, 0, c.rows * c.nsplit)
                    if c.epi == QKROPE:
                        row = rows_of(ti)[0]
                        lr = np.where(row < c.row_split, row, row - c.row_split)
                        ri = c.pos * 64 + ((lr & 127) >> 1)
                        rep.check("rope load", ri, ri + 1, 0, c.max_ctx * 64)

                # dot products and stores of each consumed item
                for it in range(S):
                    ti, j = it // nj, it % nj
                    bl = bs + c.bs * j
                    use = bl < nbl
                    base = bl[use] * XBLK + v[use] * SLOT
                    rep.check("dot LDS read", base, base + SLOT, 0, panel * XBLK)
                    tile = gw + ti * stride
                    rows = [tile * TR + rg * c.rpl + r for r in range(c.rpl)]
                    if c.epi == COLPART:
                        cc = bs + c.bs * j
                        ok = (v == 0) & (cc < nbl)
                        for r in range(c.rpl):
                            w_ = (wave * TR + rg[ok] * c.rpl + r) * panel + cc[ok]
                            rep.check("column LDS store", panel * XBLK + w_, panel * XBLK + w_ + 1, 0, lds_words)
                        if j == nj - 1:
                            for r in range(c.rpl):
                                valid = rows[r] < c.rows
                                for ccol in range(nbl):
                                    idx = rows[r][valid] * c.nsplit + kb + ccol
                                    rep.check("column partial store", idx, idx + 1, 0, c.rows * c.nsplit)
                                rep.check("row sum store", rows[r][valid], rows[r][valid] + 1, 0, c.rows)
                    elif j == nj - 1:
                        head = (v == 0) & (bs == 0)
                        for r in range(c.rpl):
                            row = rows[r][head]
                            row = row[row < c.rows]
                            if c.epi == PARTIAL:
                                rep.check("partial store", row * c.nsplit + split, row * c.nsplit + split + 1, 0,
                                          c.rows * c.nsplit)
                            elif c.epi == VSTORE:
                                rep.check("cache store", c.pos * c.kv_dim + row, c.pos * c.kv_dim + row + 1, 0,
                                          c.max_ctx * c.kv_dim)
                            elif c.epi == QKROPE:
                                if r == 0:
                                    isq = row < c.row_split
                                    lr = np.where(isq, row, row - c.row_split)
                                    rep.check("q store", lr[isq], lr[isq] + 2, 0, c.row_split)
                                    ck = c.pos * c.kv_dim + lr[~isq]
                                    rep.check("k cache store", ck, ck + 2, 0, c.max_ctx * c.kv_dim)
                            else:
                                rep.check("output store", row, row + 1, 0, c.rows)
    return rep


def built_layouts(fmt):
    """The (bs, rpl) layouts launch_cfg instantiates (layout_built)."""
    lay = [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (8, 1), (8, 2), (16, 1)]
    return [(b, r) for b, r in lay if not (fmt in (Q6, Q6P) and r == 4)]


# ------------------------------------------------------------ row stream
RS_MAX_BLOCKS, RS_OWNERS, RS_WAVES = 14, 56, 12
RS_LDS_FLOATS = RS_MAX_BLOCKS * KQK // 64 * 68


def rs_lds_index(e):
    """arc_gemv_rs.hpp rs_lds_index: 4 pad floats after every 64."""
    return e + 4 * (e >> 6)


def simulate_rs(rows: int, K: int, epi: int, norm: bool, gx: int | None = None, ring: int = 3,
                mistake: str | None = None) -> Report:
    """Bounds model of gemv_rs_body (arc_gemv_rs.hpp) and launch_rs: every
    thread's x / norm-weight float4 loads (indices clamped), the LDS stores
    of the staging and each lane's reads of its 64 values, the weight chunk
    and header loads of the ring (clamped tile, row and block, and the loads
    past the last tile), the epilogue operand loads, the bpermute source
    lane, the block-sum slots and the output stores.  `mistake` = "block"
    drops the owner lanes' block clamp, "row" the tile and row clamps."""
    rep = Report()
    nb = K // KQK
    assert 1 <= nb <= RS_MAX_BLOCKS, "launch_rs takes rows of 1 .. 14 super-blocks"
    W = RS_WAVES
    NT = W * WAVE
    XQ = -(-(RS_MAX_BLOCKS * KQK // 4) // NT)
    nq = nb * KQK // 4
    row_bytes = nb * 144
    nmat = 2 if epi == SWIGLU else 1
    ntiles = rows
    want = -(-ntiles // W)
    if gx is None:
        gx = min(want, 256)
    assert 1 <= gx <= want
    t = np.arange(NT)
    lane, wave = t & 63, t >> 6

    for i in range(XQ):
        q = np.minimum(t + i * NT, nq - 1)
        rep.check("x float4 load", 4 * q, 4 * q + 4, 0, K)
        if norm:
            rep.check("norm weight float4 load", 4 * q, 4 * q + 4, 0, K)
        st = t + i * NT
        st = st[st < nq]
        li = rs_lds_index(4 * st)
        rep.check("LDS x store", li, li + 4, 0, RS_LDS_FLOATS)
    rep.check("block-sum slot", wave, wave + 1, 0, W)

    header = lane >= RS_OWNERS
    k = np.where(header, 0, lane >> 2)
    g = lane & 3
    owner = ~header & (k < nb)
    hk = lane - RS_OWNERS
    kc = k if mistake == "block" else np.minimum(k, nb - 1)
    oa = np.where(header, np.minimum(hk, nb - 1) * 144, kc * 144 + 16 + 32 * g)
    ob = np.where(header, np.minimum(hk + 8, nb - 1) * 144, oa + 16)
    src = RS_OWNERS + (k & 7)
    rep.check("bpermute source lane", src, src + 1, 0, WAVE)
    xe = rs_lds_index(np.minimum(k, nb - 1) * KQK + 64 * g)
    rep.check("LDS x read", xe, xe + 64, 0, RS_LDS_FLOATS)

    clamp_tile = (lambda v: v) if mistake == "row" else (lambda v: min(v, ntiles - 1))
    stride = gx * W
    for bx in range(gx):
        for wv in range(W):
            gw = bx * W + wv
            my = (ntiles - gw + stride - 1) // stride if gw < ntiles else 0
            lane_sel = wave == wv

            def load(ti):
                tile = clamp_tile(gw + ti * stride)
                row = tile if mistake == "row" else min(tile, rows - 1)
                for m in range(nmat):
                    for o in (oa, ob):
                        off = row * row_bytes + o[lane_sel]
                        rep.check(f"weight load (w{m})", off, off + 16, 0, rows * row_bytes)
                if epi == PLAIN:
                    rep.check("epilogue operand load", np.array([row]), np.array([row + 1]), 0, rows)

            # the ring: items 0 .. ring-2 first, then item t + ring - 1 before
            # consuming item t, for t < (my // ring) * ring
            for i in range(ring - 1):
                load(i)
            full = (my // ring) * ring
            for tt in range(full):
                load(tt + ring - 1)
            for ti in range(my):
                row = gw + ti * stride
                rep.check("output store", np.array([row]), np.array([row + 1]), 0, rows)
    return rep


# ------------------------------------------------- embedding row and argmax tail
def simulate_embed(nb: int, emb_rows: int, tokens, mistake: str | None = None) -> Report:
    """Bounds model of the F_EMBED staging (arc_gemv.hpp gemv_body /
    stage_x_rms / emb_group): for each token id the device may hold in
    ctl->token, the row the launch decodes (erow = emb + (token < emb_rows ?
    token : 0) * nb * 144), every byte emb_group reads for every group of
    the row (d, dmin, the 12 scale bytes, 16 nibble bytes) and the raw row
    workgroup 0 writes to h_out.  `mistake` = "token" drops the clamp."""
    rep = Report()
    table = emb_rows * nb * 144
    gi = np.arange(nb * 16)
    e = (gi >> 4) * KQK + x_group_offset(Q4, (gi >> 2) & 3, gi & 3)
    for tok in tokens:
        row = tok if mistake == "token" else (tok if tok < emb_rows else 0)
        base = row * nb * 144
        b = base + (e >> 8) * 144
        rep.check("embedding header read", b, b + 16, 0, table)
        k0 = e & 255
        l64 = k0 & 63
        nib = b + 16 + (k0 >> 6) * 32 + (l64 & 31)
        rep.check("embedding nibble read", nib, nib + 16, 0, table)
        rep.check("raw row store (h_out)", e, e + 16, 0, nb * KQK)
    return rep


def simulate_argnext(rows: int, n: int, best_len: int, out_cap: int, steps, idx_values,
                     mistake: str | None = None) -> Report:
    """Bounds model of argmax_finish (F_ARGNEXT): the last workgroup reads the
    n per-workgroup bests (i = thread, thread + NT, ... < n) from a buffer of
    best_len entries, turns the folded index into the token (idx < rows, else
    0), and writes out_tokens[step] only while step < out_cap.  `mistake` =
    "step" drops the out_cap check, "idx" the token clamp."""
    rep = Report()
    for NT in (256, 512):
        t = np.arange(NT)
        for k in range(-(-n // NT)):
            i = t + k * NT
            i = i[i < n]
            rep.check("per-workgroup best load", i, i + 1, 0, best_len)
    for step in steps:
        if mistake == "step" or step < out_cap:
            rep.check("out_tokens store", np.array([step]), np.array([step + 1]), 0, out_cap)
    for idx in idx_values:
        tok = idx if mistake == "idx" else (idx if idx < rows else 0)
        rep.check("next token (embedding row of the next step)", np.array([tok]), np.array([tok + 1]), 0, rows)
    return rep
