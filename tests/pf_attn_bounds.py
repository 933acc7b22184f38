"""Bounds model of the prompt pass's MFMA attention kernel k_pf_attn_mf
(csrc/arc_prefill.hip).

Restates, for every workgroup (query block b of 32 rows, q head hq) and
every lane of its 4 waves, each global index the kernel forms -- the q loads
(8 steps of two float4 per lane), the K fragment loads (two 32-key tiles of
each chunk, 8 steps of 16 bytes), the V row loads (16 x 16 bytes per lane),
the fp16 output stores -- and each LDS index (the wave's V^T rows with the
key permutation, the 16-byte V^T fragment reads, the [4][128][32] output
combine reusing those rows, the per-wave (max, sum)), and checks them
against the buffers: q [M][hidden] fp32, the caches [max_ctx][kv_heads*128]
fp16, x [M][ldx] fp16, LDS 4 x 128 x 72 halves + 2 x 4 x 32 floats.  It
also checks that every (query row, key position <= its own) pair is covered
by exactly one wave's chunk, and that the permuted V^T column of a key is
the column the MFMA fragment reads for it.  A mistake can be planted (an
unclamped key row, an unpermuted V^T column) to show that the model reports
it.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

HD, CHUNK, VT_LD = 128, 64, 64 + 8


@dataclass
class Report:
    checked: int = 0
    violations: list = field(default_factory=list)

    def check(self, what, lo, hi, limit_lo, limit_hi):
        lo = np.asarray(lo)
        hi = np.asarray(hi)
        self.checked += lo.size
        bad = (lo < limit_lo) | (hi > limit_hi)
        if bad.any():
            self.violations.append((what, int(lo[bad].min()), int(hi[bad].max()), limit_lo, limit_hi))


def swap_bits_2_3(k):
    k = np.asarray(k)
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1)


def simulate(kv_heads: int, hpk: int, max_ctx: int, pos0: int, M: int, ldx: int | None = None,
             mistake: str | None = None) -> Report:
    rep = Report()
    hidden = kv_heads * hpk * HD
    ldx = hidden if ldx is None else ldx
    kvd = kv_heads * HD
    assert pos0 + M <= max_ctx and ldx >= hidden
    lane = np.arange(64)
    l32, h2 = lane & 31, lane >> 5
    clamp = (lambda r: r) if mistake == "row" else (lambda r: np.minimum(r, max_ctx - 1))
    perm = (lambda k: k) if mistake == "perm" else swap_bits_2_3
    cover = np.zeros((M, pos0 + M), np.int32)
    for b in range((M + 31) // 32):
        q0 = 32 * b
        qlast = min(q0 + 31, M - 1)
        nkc = (pos0 + qlast + CHUNK) // CHUNK
        for hq in range(kv_heads * hpk):
            g = hq // hpk
            qrow = np.minimum(q0 + l32, M - 1)
            for st in range(8):
                e = qrow * hidden + hq * HD + 8 * h2 + 16 * st
                rep.check("q load", e, e + 8, 0, M * hidden)
            for w in range(4):
                for c in range(w, nkc, 4):
                    kbase = c * CHUNK
                    vrow = clamp(kbase + lane)
                    e = vrow * kvd + g * HD
                    rep.check("V row load", e, e + HD, 0, max_ctx * kvd)
                    for kt in range(2):
                        krow = clamp(kbase + 32 * kt + l32)
                        for st in range(8):
                            e = krow * kvd + g * HD + 8 * h2 + 16 * st
                            rep.check("K fragment load", e, e + 8, 0, max_ctx * kvd)
                    # V^T rows: key `lane` of the chunk at column perm(lane), dims 8e + j
                    col = perm(lane)
                    for e8 in range(16):
                        for j in range(8):
                            a = (w * HD + 8 * e8 + j) * VT_LD + col
                            rep.check("V^T LDS store", a, a + 1, w * HD * VT_LD, (w + 1) * HD * VT_LD)
                    # fragment reads: step st of tile kt, keys 16 st + 8(j/4) + 4 h2 + j%4 at the lane's
                    # 8 contiguous columns; the column each key was stored at must be the one read
                    for kt in range(2):
                        for st in range(2):
                            k0 = 32 * kt + 16 * st + 8 * h2
                            for t in range(4):
                                a = (w * HD + 32 * t + l32) * VT_LD + k0
                                rep.check("V^T LDS fragment read", a, a + 8, w * HD * VT_LD, (w + 1) * HD * VT_LD)
                            for j in range(8):
                                key = 32 * kt + 16 * st + 8 * (j >> 2) + 4 * h2 + (j & 3)
                                stored = 32 * (key >> 5) + perm(key & 31)
                                wrong = stored != k0 + j
                                if np.any(wrong):
                                    rep.violations.append(("V^T column of key", int(key[wrong][0]),
                                                           int(stored[wrong][0]), int((k0 + j)[wrong][0]), 0))
                    # the scores' D layout: value i of tile kt -> key 8(i/4) + 4 h2 + i%4 for query l32
                    if hq == 0:
                        for kt in range(2):
                            for i in range(16):
                                kpos = kbase + 32 * kt + 8 * (i >> 2) + 4 * h2 + (i & 3)
                                qq = q0 + l32
                                ok = (qq < M) & (kpos <= pos0 + qq)
                                np.add.at(cover, (qq[ok], kpos[ok]), 1)
            # the combine over the reused V^T rows as [4][128][32] floats, and (m, l) per wave
            for w in range(4):
                for t in range(4):
                    for i in range(16):
                        d = 32 * t + 8 * (i >> 2) + 4 * h2 + (i & 3)
                        a = (w * HD + d) * 32 + l32
                        rep.check("output combine LDS store", a, a + 1, 0, 4 * HD * VT_LD // 2)
            tid = np.arange(256)
            qq, d0 = tid & 31, (tid >> 5) * 16
            for v in range(4):
                for d in range(16):
                    a = (v * HD + d0 + d) * 32 + qq
                    rep.check("output combine LDS read", a, a + 1, 0, 4 * HD * VT_LD // 2)
            ok = q0 + qq < M
            e = (q0 + qq[ok]) * ldx + hq * HD + d0[ok]
            rep.check("x store", e, e + 16, 0, (M - 1) * ldx + hidden)
    rows = np.arange(M)
    want = (np.arange(pos0 + M)[None, :] <= (pos0 + rows)[:, None]).astype(np.int32)
    if not np.array_equal(cover, want):
        bad = np.argwhere(cover != want)[0]
        rep.violations.append(("coverage of (row, key)", int(bad[0]), int(bad[1]), int(cover[tuple(bad)]), 1))
    return rep
