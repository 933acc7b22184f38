"""Writes the golden vectors under tests/golden/ from the reference's own
code, compiled by oracle/Makefile (``make -C oracle ref``) into
oracle/_ref/libref.so from the reference sources where they lie:

  half_table.npz        all 65536 binary16 patterns -> float32 bits,
                        q6cb::half_to_float (src/q6cb_q6_reference.hpp:20-36)
  q6_fixtures.npz       the reference's Q6CB fixture generator
                        (src/q6cb_fixture_generator.hpp:160-192) for each of its
                        five conditioning strata, with decode_q6_element outputs
                        (:49-91) and the R64 / S32 / T32 GEMV arms (:118-175)
  q4_tuples.npz         random and edge Q4_K super-blocks with the reference's
                        canonical source tuples (d, dmin bytes; 8 x (sc, mn);
                        256 codes) and EXEC148 materialisation
                        (src/q4_down_exec148_materializer.h)
  sha256_kat.json       SHA-256 of "abc" and of a 148-block EXEC148 image via
                        the reference's Sha256 class
  policy_trace.json     per-section case counts and FNV-1a-64 hashes of the
                        decision trace of tests/cpp/policy_parity.cpp built
                        against the reference's registry v2 / policy v4 /
                        binding v4 / Q4-down registration sources
                        (oracle/_ref/policy_parity_ref)

Run: python tests/golden/make_golden.py [policy]   (needs `make -C oracle ref`;
"policy" rewrites policy_trace.json only)
"""
from __future__ import annotations

import ctypes as C
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as orc  # noqa: E402


def policy_trace() -> None:
    exe = os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle", "_ref", "policy_parity_ref")
    if not os.path.exists(exe):
        raise SystemExit("oracle/_ref/policy_parity_ref missing: run `make -C oracle ref` first")
    out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    sections = {}
    for line in out.splitlines():
        name, cases, fnv = line.split()
        sections[name] = {"cases": int(cases.split("=")[1]), "fnv1a64": fnv.split("=")[1]}
    with open(os.path.join(HERE, "policy_trace.json"), "w") as f:
        json.dump({"program": "tests/cpp/policy_parity.cpp", "sections": sections}, f, indent=1)


def main() -> None:
    if sys.argv[1:] == ["policy"]:
        policy_trace()
        return
    if not orc.have_ref():
        raise SystemExit("oracle/_ref/libref.so missing: run `make -C oracle ref` first")
    R = orc.ref()

    # 1. binary16 table
    table = np.array([R.ref_half_to_float(h) for h in range(65536)], dtype=np.float32).view(np.uint32)
    np.savez_compressed(os.path.join(HERE, "half_table.npz"), bits=table)

    # 2. Q6 fixtures over the reference's five strata
    out = {}
    n, rows = 512, 3
    for stratum in range(5):
        seed = 0x6F7261636C650000 + stratum
        nb = n // 256
        packed = np.zeros(rows * nb * 210, dtype=np.uint8)
        x = np.zeros(n, dtype=np.float32)
        eq = np.zeros(rows * n, dtype=np.int8)
        es = np.zeros(rows * nb * 16, dtype=np.int8)
        rc = R.ref_q6_fixture(n, rows, seed, stratum, packed.ctypes.data, x.ctypes.data, eq.ctypes.data,
                              es.ctypes.data)
        assert rc == 0, f"reference fixture generator failed: {rc}"
        q = np.zeros(rows * nb * 256, dtype=np.int32)
        sc = np.zeros_like(q)
        val = np.zeros(rows * nb * 256, dtype=np.float32)
        for b in range(rows * nb):
            blk = packed[b * 210:(b + 1) * 210]
            o = slice(b * 256, (b + 1) * 256)
            qq = np.zeros(256, np.int32)
            ss = np.zeros(256, np.int32)
            vv = np.zeros(256, np.float32)
            R.ref_q6_decode_block(blk.ctypes.data, qq.ctypes.data, ss.ctypes.data, vv.ctypes.data)
            q[o], sc[o], val[o] = qq, ss, vv
        r64 = np.zeros(rows, np.float64)
        s32 = np.zeros(rows, np.float32)
        t32 = np.zeros(rows, np.float32)
        assert R.ref_q6_arms(packed.ctypes.data, packed.nbytes, n, rows, x.ctypes.data, r64.ctypes.data,
                             s32.ctypes.data, t32.ctypes.data) == 0
        p = f"s{stratum}_"
        out.update({p + "packed": packed, p + "x": x, p + "expected_q": eq, p + "expected_scale": es,
                    p + "q": q, p + "scale": sc, p + "value_bits": val.view(np.uint32), p + "r64": r64,
                    p + "s32_bits": s32.view(np.uint32), p + "t32_bits": t32.view(np.uint32)})
    out["n"] = np.array(n)
    out["rows"] = np.array(rows)
    np.savez_compressed(os.path.join(HERE, "q6_fixtures.npz"), **out)

    # 3. Q4 tuples: random blocks plus edge blocks (scale bytes 0x00/0xff,
    #    nibbles 0/15, special binary16 d/dmin)
    rng = np.random.default_rng(0x51345F4B)
    blocks = [rng.integers(0, 256, 144, dtype=np.uint8) for _ in range(48)]
    specials = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00]
    for i, h in enumerate(specials):
        b = rng.integers(0, 256, 144, dtype=np.uint8)
        b[0:2] = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
        b[2:4] = np.frombuffer(np.uint16(specials[-1 - i]).tobytes(), np.uint8)
        blocks.append(b)
    for fill in (0x00, 0xFF, 0x0F, 0xF0, 0x3F, 0xC0):
        b = np.full(144, fill, dtype=np.uint8)
        b[0:4] = [0x00, 0x3C, 0x00, 0x38]  # d = 1.0, dmin = 0.5
        blocks.append(b)
    blk = np.stack(blocks)
    tuples = np.zeros((len(blk), 276), np.uint8)
    ex148 = np.zeros((len(blk), 148), np.uint8)
    for i, b in enumerate(blk):
        b = np.ascontiguousarray(b)
        t = np.zeros(276, np.uint8)
        e = np.zeros(148, np.uint8)
        R.ref_q4_source_tuple(b.ctypes.data, t.ctypes.data)
        R.ref_exec148_materialize_block(b.ctypes.data, e.ctypes.data)
        tuples[i], ex148[i] = t, e
    np.savez_compressed(os.path.join(HERE, "q4_tuples.npz"), blocks=blk, tuples=tuples, exec148=ex148)

    # 4. SHA-256 known answers through the reference's implementation
    def sha(data: bytes) -> str:
        buf = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
        o = np.zeros(32, np.uint8)
        R.ref_sha256(buf.ctypes.data, len(data), o.ctypes.data)
        return bytes(o).hex()

    with open(os.path.join(HERE, "sha256_kat.json"), "w") as f:
        json.dump({"abc": sha(b"abc"), "empty": sha(b""), "exec148_2rows": sha(bytes(ex148[:8].ravel()))},
                  f, indent=1)

    # 5. plugin surface decision trace
    policy_trace()
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
