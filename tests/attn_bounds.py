"""Bounds model of the decode attention kernel k_attn (csrc/arc_decode.hip).

Restates, for every workgroup (split s, kv head g) and every lane of its W
waves (4 or 8), each global index the kernel forms -- the K and V cache
loads of its chunks (the early loads of splits 0..7 / 0..3 included), the q
loads, the output, split-partial and (m, l) stores, the merge's partial
loads, the arrival counter -- and each LDS index, and checks them against
the buffer sizes the session allocates.  The kernel's constants: chunks of
16 W positions, kMaxSplits = 64, head dim 128, merge batches of 16; a split
covers at least min_cps chunks.
A mistake can be planted (an unclamped cache row, an unclamped query head)
to show that the model reports it.  (The merge's split clamps keep the loads
on written partials; the partial buffers hold kMaxSplits per head, so those
loads stay in bounds either way.)
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

MAX_SPLITS, WAVE, HD, MB = 64, 64, 128, 16
EARLY = {4: 8, 8: 4}


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


def plan(T, chunk=64, min_cps=1):
    nch = (T + chunk - 1) // chunk
    cps = max((nch + MAX_SPLITS - 1) // MAX_SPLITS, min_cps)
    return nch, cps, (nch + cps - 1) // cps


def simulate(kv_heads: int, hpk: int, max_ctx: int, T: int, mistake: str | None = None,
             waves: int = 4, min_cps: int = 1) -> Report:
    """One launch at T cached positions (T = position + 1 <= max_ctx)."""
    rep = Report()
    kvd = kv_heads * HD
    cache_elems = max_ctx * kvd                       # one layer's K (or V) cache, fp16 elements
    q_elems = kv_heads * hpk * HD
    po_elems = kv_heads * MAX_SPLITS * hpk * HD
    pml_elems = kv_heads * MAX_SPLITS * hpk * 2
    chunk = 16 * waves
    nch, cps, nsplit = plan(T, chunk, min_cps)
    tid = np.arange(waves * WAVE)
    w, lane = tid >> 6, tid & 63
    r16, grp = lane & 15, lane >> 4
    clamp = (lambda r, m: r) if mistake == "row" else np.minimum

    def load(g, t0, tmax):
        tw = t0 + 16 * w
        krow = clamp(tw + r16, tmax)
        k0 = krow * kvd + g * HD + 32 * grp
        rep.check("K load", k0, k0 + 32, 0, cache_elems)
        for j in range(16):
            vrow = clamp(tw + j, tmax)
            v0 = vrow * kvd + g * HD + 2 * lane
            rep.check("V load", v0, v0 + 2, 0, cache_elems)

    for g in range(kv_heads):
        rep.check("arrival counter", np.array([g]), np.array([g + 1]), 0, kv_heads)
        for s in range(MAX_SPLITS):
            early = s < EARLY[waves]
            if early:
                load(g, s * chunk, max_ctx - 1)
            qh = r16 if mistake == "qhead" else np.minimum(r16, hpk - 1)
            q0 = (g * hpk + qh) * HD + 32 * grp
            rep.check("q load", q0, q0 + 32, 0, q_elems)
            if s >= nsplit:
                continue
            c0, c1 = s * cps, min(s * cps + cps, nch)
            if cps != 1 or not early:
                load(g, c0 * chunk, T - 1)
            for c in range(c0, c1):
                if c + 1 < c1:
                    load(g, (c + 1) * chunk, T - 1)
                # LDS: the wave's weights [16][8], rescale [8]
                pw = (4 * grp[:, None] + np.arange(4)[None, :]) * 8 + r16[:, None]
                sel = np.broadcast_to((r16 < hpk)[:, None], pw.shape)
                rep.check("LDS weights store", pw[sel], pw[sel] + 1, 0, 16 * 8)
                rep.check("LDS rescale store", r16[r16 < hpk], r16[r16 < hpk] + 1, 0, 8)
            # split end: the waves' (m, l), their rescaled o, then one thread per (head, dim quad)
            sel = (grp == 0) & (r16 < hpk)
            mi = w[sel] * 8 + r16[sel]
            rep.check("LDS wave (m, l) store", mi, mi + 1, 0, waves * 8)
            h_all = np.arange(hpk)
            ow = (w[:, None] * hpk + h_all[None, :]) * HD + 2 * lane[:, None]
            rep.check("LDS wave o store", ow, ow + 2, 0, waves * hpk * HD)
            owner = tid < hpk * (HD // 4)
            hh = np.minimum(tid // (HD // 4), hpk - 1)
            dq4 = tid % (HD // 4)
            for v in range(waves):
                rd = (v * hpk + hh) * HD + 4 * dq4
                rep.check("LDS wave o read", rd, rd + 4, 0, waves * hpk * HD)
            base = g * MAX_SPLITS
            if nsplit == 1:
                o = (g * hpk + hh[owner]) * HD + 4 * dq4[owner]
                rep.check("out store", o, o + 4, 0, q_elems)
                continue
            p = ((base + s) * hpk + hh[owner]) * HD + 4 * dq4[owner]
            rep.check("partial o store", p, p + 4, 0, po_elems)
            m = ((base + s) * hpk + hh[owner & (dq4 == 0)]) * 2
            rep.check("partial (m, l) store", m, m + 2, 0, pml_elems)
        if nsplit == 1:
            continue
        # the merge, in the last workgroup to arrive (any split of head g)
        ss = np.minimum(lane, nsplit - 1)
        for k in range(-(-8 // waves)):
            h = np.minimum(w + waves * k, hpk - 1)
            m = ((base + ss) * hpk + h) * 2
            rep.check("merge (m, l) load", m, m + 2, 0, pml_elems)
            hk = w + waves * k
            sel = hk < hpk
            fw = lane[sel] * hpk + hk[sel]
            rep.check("LDS split weight store", fw, fw + 1, 0, MAX_SPLITS * hpk)
        src = (base * hpk + hh) * HD + 4 * dq4
        for s0 in range(0, nsplit, MB):
            for u in range(MB):
                sp = min(s0 + u, nsplit - 1)
                p = src[owner] + sp * hpk * HD
                rep.check("merge o load", p, p + 4, 0, po_elems)
                if s0 + u < nsplit:
                    fw = (s0 + u) * hpk + hh[owner]
                    rep.check("LDS split weight load", fw, fw + 1, 0, MAX_SPLITS * hpk)
        o = (g * hpk + hh[owner]) * HD + 4 * dq4[owner]
        rep.check("out store", o, o + 4, 0, q_elems)
    return rep
