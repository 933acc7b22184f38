"""Pins the oracle's decode-step composition (orc_decode_step) against an
independent numpy fp64 implementation on a tiny model: dequantised weight
matrices (oracle decode, pinned elsewhere) multiplied with numpy, RoPE as a
complex rotation of adjacent pairs, softmax attention over the fp16 cache
with kv head = q head // (q_heads / kv_heads), SwiGLU via scipy expit.  The
fp16-operand mode (the batched prompt pass's arithmetic) is pinned the same
way, with numpy's own binary16 rounding of the layer-GEMM operands."""
import numpy as np
import pytest
from scipy.special import expit

import arcllm_amd as arc
import oracle_lib as orc
from decode_common import tiny_dims


def numpy_step(d, T, kc, vc, max_ctx, pos, token, f16=False):
    H, KVD, F = d.hidden, d.kv_heads * 128, d.ffn
    deq_exact = lambda qt, a, rows, K: orc.dequant(qt, a, rows, K).astype(np.float64)
    if f16:  # layer GEMMs: both operands rounded to binary16 (weights from fp32, inputs via fp32)
        deq = lambda qt, a, rows, K: orc.dequant(qt, a, rows, K).astype(np.float16).astype(np.float64)
        op = lambda x: x.astype(np.float32).astype(np.float16).astype(np.float64)
    else:
        deq, op = deq_exact, (lambda x: x)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + float(d.rms_eps)) * w.astype(np.float64)

    def rope(x, heads):
        z = x.reshape(heads, 64, 2)
        c = z[..., 0] + 1j * z[..., 1]
        c = c * np.exp(1j * pos * float(d.rope_theta) ** (-2.0 * np.arange(64) / 128))
        return np.stack([c.real, c.imag], -1).reshape(-1)

    h = deq_exact(arc.Q4_K, T[0], d.vocab, H)[token].copy()
    for layer in range(d.layers):
        t = lambda w: T[3 + 12 * layer + w]
        xn = op(rms(h, t(0)))
        q = deq(arc.Q4_K, t(1), H, H) @ xn + t(4)
        k = deq(arc.Q4_K, t(2), KVD, H) @ xn + t(5)
        v = deq(d.v_type[layer], t(3), KVD, H) @ xn + t(6)
        q, k = rope(q, d.q_heads), rope(k, d.kv_heads)
        base = layer * max_ctx * KVD
        kc[base + pos * KVD: base + (pos + 1) * KVD] = k.astype(np.float32).astype(np.float16).view(np.uint16)
        vc[base + pos * KVD: base + (pos + 1) * KVD] = v.astype(np.float32).astype(np.float16).view(np.uint16)
        K = kc[base: base + (pos + 1) * KVD].view(np.float16).astype(np.float64).reshape(pos + 1, d.kv_heads, 128)
        V = vc[base: base + (pos + 1) * KVD].view(np.float16).astype(np.float64).reshape(pos + 1, d.kv_heads, 128)
        att = np.zeros(H)
        for hh in range(d.q_heads):
            g = hh // (d.q_heads // d.kv_heads)
            s = K[:, g, :] @ q[hh * 128:(hh + 1) * 128] / np.sqrt(128.0)
            p = np.exp(s - s.max())
            att[hh * 128:(hh + 1) * 128] = (p / p.sum()) @ V[:, g, :]
        h = h + deq(arc.Q4_K, t(7), H, H) @ op(att)
        xn = op(rms(h, t(8)))
        gg = deq(arc.Q4_K, t(9), F, H) @ xn
        uu = deq(arc.Q4_K, t(10), F, H) @ xn
        h = h + deq(d.down_type[layer], t(11), H, F) @ op(gg * expit(gg) * uu)
    return deq_exact(arc.Q6_K, T[1], d.vocab, H) @ rms(h, T[2])


@pytest.mark.parametrize("f16", [False, True])
def test_oracle_decode_step_matches_numpy_composition(f16):
    d = tiny_dims(layers=3, vocab=1024)
    T = arc.synth_model_tensors(d, 0xD0C0DE)
    max_ctx = 64
    o = orc.DecodeOracle(d, T, max_ctx, f16_operands=f16)
    o.fill_kv(20, 77, arc.synth_normal)
    kc, vc = o.kc.copy(), o.vc.copy()
    token = 5
    for pos in (20, 21, 22):
        lo = o.step(token, pos)
        ln = numpy_step(d, T, kc, vc, max_ctx, pos, token, f16)
        np.testing.assert_allclose(lo, ln, rtol=1e-9, atol=1e-9 * np.abs(ln).max())
        assert np.array_equal(o.kc, kc) and np.array_equal(o.vc, vc)
        token = int(np.argmax(lo))


def test_fill_kv_matches_session_contract():
    """arc_session_fill_kv draws fp16(N(0,1)) from stream 1000000 + 2*layer + kv;
    the oracle's fill reproduces it from the same generator."""
    d = tiny_dims(layers=2, vocab=256)
    o = orc.DecodeOracle(d, arc.synth_model_tensors(d, 1), 8)
    o.fill_kv(5, 3, arc.synth_normal)
    kvd = 256
    k0 = o.kc[:5 * kvd].view(np.float16).astype(np.float32)
    assert np.array_equal(k0, arc.synth_normal(3, 1000000, 5 * kvd).astype(np.float16).astype(np.float32))
    assert np.all(o.kc[5 * kvd: 8 * kvd] == 0)


def test_f16_gemv_is_exact_products_of_rounded_operands():
    rng = np.random.default_rng(4)
    for qt in (arc.Q4_K, arc.Q6_K):
        rows, K = 24, 768
        w = arc.synth_packed(qt, 9, 3, rows, K)
        x = rng.standard_normal(K) * 3.0
        got = orc.gemv_r64_f16(qt, w, rows, K, x)
        ref = orc.dequant(qt, w, rows, K).astype(np.float16).astype(np.float64) @ \
            x.astype(np.float32).astype(np.float16).astype(np.float64)
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
        # and it differs from the exact-operand product (the rounding is real)
        assert not np.array_equal(got, orc.gemv_r64_xd(qt, w, rows, K, x))


@pytest.mark.parametrize("qtype", [arc.Q4_K, arc.Q6_K])
def test_element_products_are_exact_in_fp32(qtype):
    """The batched prompt pass decodes weights as fmaf(d*sc, q, -dmin*mn)
    (Q4_K) and fmaf(d*sc, q+32, -32*d*sc) (Q6_K); both equal the element
    decode's separate multiply and subtract bit for bit because the product
    d*sc*q is exact in binary32: d has 11 significant bits, sc at most 6
    (Q4_K) or 7 (Q6_K) and q at most 4 (Q4_K) or 6 (Q6_K), so only the final
    subtraction rounds.  Checked here on every element of random blocks,
    including the extreme scales and codes: the float64 product rounds to
    binary32 without change."""
    rng = np.random.default_rng(qtype)
    nb = 64
    blk = arc.synth_packed(qtype, 7, 1, 1, nb * 256).reshape(nb, -1).copy()
    dpos = 0 if qtype == arc.Q4_K else 208
    # random finite fp16 d (all exponents), including the largest ones
    for b in range(nb):
        bits = int(rng.integers(0x0001, 0x7BFF)) if b % 4 else 0x7BFF
        blk[b, dpos:dpos + 2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
    O = orc.oracle()
    for b in range(nb):
        p = blk[b].ctypes.data
        d = np.float64(np.frombuffer(blk[b, dpos:dpos + 2].tobytes(), np.float16)[0])
        for k in range(256):
            if qtype == arc.Q4_K:
                sc, mn = orc.C.c_uint32(), orc.C.c_uint32()
                O.orc_q4k_scale_min(p, k >> 5, orc.C.byref(sc), orc.C.byref(mn))
                prod = d * sc.value * O.orc_q4k_code(p, k)
            else:
                s = orc.C.c_int()
                q = O.orc_q6k_code(p, k, orc.C.byref(s))
                prod = d * s.value * q
            assert np.float64(np.float32(prod)) == prod


@pytest.mark.parametrize("f16", [0, 1])
def test_prompt_pass_oracle_equals_stepwise_oracle(f16):
    """orc_prompt_pass (layer by layer over all positions) against
    orc_decode_step_ex called per position with teacher forcing: last logits
    and every cache row bit-identical; a planted change in one prompt token
    changes the logits."""
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, 0x5EED)
    max_ctx, pos0 = 64, 5
    prompt = (np.arange(23, dtype=np.uint32) * 131 + 7) % d.vocab
    a = orc.DecodeOracle(d, T, max_ctx, f16_operands=bool(f16))
    a.fill_kv(pos0, 3, arc.synth_normal)
    b = orc.DecodeOracle(d, T, max_ctx, f16_operands=bool(f16))
    b.fill_kv(pos0, 3, arc.synth_normal)
    la = a.prompt(prompt, pos0)
    for i, t in enumerate(prompt):
        lb = b.step(int(t), pos0 + i)
    assert np.array_equal(la.view(np.uint64), lb.view(np.uint64))
    assert np.array_equal(a.kc, b.kc) and np.array_equal(a.vc, b.vc)
    c = orc.DecodeOracle(d, T, max_ctx, f16_operands=bool(f16))
    c.fill_kv(pos0, 3, arc.synth_normal)
    planted = prompt.copy()
    planted[10] = (planted[10] + 1) % d.vocab
    assert not np.array_equal(c.prompt(planted, pos0), la)
