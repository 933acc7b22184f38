"""The batched MFMA prompt pass (arc_session_prefill, n >= 2) against the
oracle fed the same prompt token by token, and against the GPU's own
step-by-step prompt pass.

The MFMA pass rounds its layer-GEMM operands to fp16 (activations and
dequantised weights; fp32 accumulation).  Its pin is the oracle's fp16-operand
mode (orc_decode_step_ex with f16_operands, pinned against numpy's binary16
rounding in test_decode_oracle_cpu.py).  The metric is normwise,
max|gpu - ref| / max|ref|, per layer cache (K and V over all prompt rows) and
for the last position's logits: with fp16 operands an output that cancels to
near zero moves by an fp16 ulp of its largest terms when one operand rounds
the other way, which an element-relative metric reports as O(1) although the
product is as accurate as its operands.  Bounds: F16_NORM against the
fp16-operand oracle (the residue is fp32-vs-fp64 accumulation and the operand
roundings it flips), EXACT_NORM against the exact fp64 oracle (fp16 operand
rounding itself), and the next token equal to the exact oracle's unless its
top-2 margin is below PF_TIE * max|logit|.
"""
import os
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc
from decode_common import tiny_dims

pytestmark = pytest.mark.gpu

SEED = 0x9F11_0000
# measured (one MI355X): 3-layer model <= 7e-4 / 4e-3, 28-layer 7B shape
# 5.2e-3 / 2.3e-2 (fp16-operand / exact oracle)
F16_NORM = 1e-2
EXACT_NORM = 5e-2
PF_TIE = 2e-2


def norm_err(g, w):
    w = np.asarray(w, np.float64)
    return float(np.max(np.abs(np.asarray(g, np.float64) - w)) / max(np.max(np.abs(w)), 1e-30))


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def _cache(sess, d, layer, n, max_ctx):
    kvd = d.kv_heads * 128
    k, v = sess.kv(layer)
    out = []
    for ptr in (k, v):
        h = np.empty(n * kvd, np.uint16)
        arc.check(arc.lib().arc_memcpy_dtoh(h.ctypes.data, ptr, h.nbytes, None))
        out.append(h.view(np.float16).astype(np.float64))
    return out


def _oracle_cache(o, d, layer, n, max_ctx):
    kvd = d.kv_heads * 128
    base = layer * max_ctx * kvd
    return [c[base:base + n * kvd].view(np.float16).astype(np.float64) for c in (o.kc, o.vc)]


def _errors(s, lg, o, ref, d, n, max_ctx):
    worst = 0.0
    for layer in range(d.layers):
        got = _cache(s, d, layer, n, max_ctx)
        want = _oracle_cache(o, d, layer, n, max_ctx)
        for g, w in zip(got, want):
            worst = max(worst, norm_err(g, w))
    return norm_err(lg, ref), worst


def check_prompt(d, T, prompt, max_ctx):
    model = arc.Model(d, T)
    s = arc.Session(model, max_ctx)
    nxt, nf = s.prefill(prompt, logits=True)
    lg = s.logits()
    o16 = orc.DecodeOracle(d, T, max_ctx, f16_operands=True)
    o64 = orc.DecodeOracle(d, T, max_ctx)
    for i, t in enumerate(prompt):
        ref16 = o16.step(int(t), i)
        ref64 = o64.step(int(t), i)
    assert nf == 0
    e16 = _errors(s, lg, o16, ref16, d, len(prompt), max_ctx)
    e64 = _errors(s, lg, o64, ref64, d, len(prompt), max_ctx)
    order = np.argsort(-ref64, kind="stable")
    margin = float(ref64[order[0]] - ref64[order[1]])
    _log(f"prompt {len(prompt)}: vs fp16-operand oracle logits {e16[0]:.3g} K/V {e16[1]:.3g}; vs exact oracle "
         f"logits {e64[0]:.3g} K/V {e64[1]:.3g}; next gpu={nxt} oracle={int(order[0])} margin={margin:.4g} "
         f"kernels={s.prefill_kernels}")
    assert max(e16) <= F16_NORM
    assert max(e64) <= EXACT_NORM
    if nxt != int(order[0]):
        assert margin < PF_TIE * float(np.max(np.abs(ref64))) and nxt == int(order[1])
    return s, model, nxt, lg


@pytest.mark.parametrize("n", [2, 37, 100])
def test_mfma_prefill_matches_oracle(n):
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED + n)
    rng = np.random.default_rng(n)
    prompt = rng.integers(0, d.vocab, n).astype(np.uint32)
    s, *_ = check_prompt(d, T, prompt, 512)
    assert s.prefill_kernels == 8 * d.layers + 3


@pytest.mark.parametrize("n", [37, 300])
def test_prefill_attention_mfma_matches_valu_kernel(n):
    """The prompt pass's attention on MFMA (32-row query blocks per q head,
    key chunks over 4 waves merged in LDS) against the VALU kernel (one
    query row per workgroup), on the 7-q-heads-per-kv-head grouping, one
    pass (37 tokens) and two passes (300: the second starts at position
    256): last-position logits and every layer's cache rows within 2e-3
    normwise, the same next token."""
    d = arc.ModelDims()
    d.hidden, d.q_heads, d.kv_heads, d.head_dim = 1792, 14, 2, 128
    d.ffn, d.vocab, d.layers = 512, 2048, 3
    d.rms_eps, d.rope_theta = 1e-6, 1e6
    for layer in range(d.layers):
        d.v_type[layer], d.down_type[layer] = arc.Q6_K, arc.Q4_K
    T = arc.synth_model_tensors(d, SEED + 11)
    model = arc.Model(d, T)
    prompt = np.random.default_rng(11).integers(0, d.vocab, n).astype(np.uint32)
    res = {}
    for mfma in (True, False):
        arc.tune_prefill_attention(mfma)
        try:
            sess = arc.Session(model, 320)
            nxt, _ = sess.prefill(prompt, logits=True)
            lg = sess.logits()
            caches = [_cache(sess, d, layer, n, 320) for layer in range(d.layers)]
        finally:
            arc.tune_prefill_attention(True)
        res[mfma] = (int(nxt), lg, caches)
    (n1, l1, c1), (n0, l0, c0) = res[True], res[False]
    e = norm_err(l1, l0)
    ec = max(norm_err(a, b) for la, lb in zip(c1, c0) for a, b in zip(la, lb))
    _log(f"n {n}: mfma vs valu attention: logits {e:.3g}, caches {ec:.3g}, next {n1} / {n0}")
    assert e <= 2e-3 and ec <= 2e-3
    assert n1 == n0


def test_mfma_prefill_two_passes_and_offset():
    d = tiny_dims(layers=2)
    T = arc.synth_model_tensors(d, SEED + 7)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, d.vocab, 300).astype(np.uint32)
    check_prompt(d, T, prompt, 320)
    # a prompt split over two calls continues the positions
    model = arc.Model(d, T)
    a = arc.Session(model, 320)
    a.prefill(prompt[:120])
    n2, _ = a.prefill(prompt[120:], pos0=120)
    b = arc.Session(model, 320)
    n1, _ = b.prefill(prompt)
    assert n1 == n2


def test_mfma_prefill_agrees_with_stepwise_pass():
    """The MFMA prompt pass and the stepwise prompt pass (decode step per
    token) against the exact oracle's logits, and both continuations against
    the oracle's greedy tokens: the stepwise pass (fp32 GEMVs) within the
    decode near-tie rule, the MFMA pass (fp16 operands) within PF_TIE."""
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED + 11)
    model = arc.Model(d, T)
    prompt = (np.arange(64, dtype=np.uint32) * 61 + 5) % d.vocab
    a = arc.Session(model, 128)
    na, _ = a.prefill(prompt, logits=True)
    la = a.logits()
    b = arc.Session(model, 128)
    nb, _ = b.prefill(prompt, logits=True, stepwise=True)
    lb = b.logits()
    o = orc.DecodeOracle(d, T, 128)
    ref = o.prompt(prompt, 0)
    e_a, e_b = norm_err(la, ref), norm_err(lb, ref)
    order = np.argsort(-ref, kind="stable")
    scale = float(np.max(np.abs(ref)))
    margin = float(ref[order[0]] - ref[order[1]])
    _log(f"mfma vs oracle logits normwise {e_a:.3g}, stepwise vs oracle normwise {e_b:.3g}, next {na} / {nb} / "
         f"oracle {int(order[0])} (margin {margin:.4g})")
    assert e_a <= EXACT_NORM and e_b <= 2e-4  # e_b: the decode tests' end-to-end bound
    assert nb == int(order[0]) or (margin < 2e-3 * scale and nb == int(order[1]))
    assert na == int(order[0]) or (margin < PF_TIE * scale and na == int(order[1]))
    if na != int(order[0]) or nb != int(order[0]):
        return  # a near tie: the continuations start from different tokens
    ref_t, second, margins, scales = o.greedy(int(order[0]), 64, 8)
    ta, _ = a.decode(na, 64, 8)
    tb, _ = b.decode(nb, 64, 8)
    _log(f"continuations mfma {ta.tolist()} stepwise {tb.tolist()} oracle {ref_t.tolist()}")
    for toks, bound in ((tb, 2e-3), (ta, PF_TIE)):
        diff = np.nonzero(toks != ref_t)[0]
        if diff.size:
            i = int(diff[0])
            assert margins[i] < bound * scales[i] and toks[i] == second[i]


def test_qwen7b_shape_prefill_matches_f16_oracle():
    d = arc.qwen25_7b_dims()
    _log("generating the 7B-shaped model")
    T = arc.synth_model_tensors(d, SEED)
    prompt = (np.arange(16, dtype=np.uint32) * 7919 + 13) % d.vocab
    check_prompt(d, T, prompt, 64)


PF_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "prefill7b_256.npz")


def test_qwen7b_prefill_256_matches_oracle_fixture():
    """Config 4 at full size: the 256-token MFMA prompt pass on the 28-layer
    7B-shaped model against the oracle's prompt pass written in the build
    container (tests/golden/make_decode_fixtures.py): last-position logits
    against the fp16-operand oracle (all 152,064) and the exact oracle (its
    256 largest), sampled cache rows of every layer, the next token, and 16
    greedy decode steps continuing from the written cache."""
    fx = np.load(PF_FIXTURE)
    d = arc.qwen25_7b_dims()
    model = arc.Model(d, seed=int(fx["seed"]))
    prompt = fx["prompt"]
    max_ctx = int(fx["max_ctx"])
    s = arc.Session(model, max_ctx)
    nxt, nf = s.prefill(prompt, logits=True)
    lg = s.logits()
    e16 = norm_err(lg, fx["f16_logits"].astype(np.float64))
    idx, val = fx["exact_top_idx"], fx["exact_top_val"]
    e64 = float(np.max(np.abs(lg[idx].astype(np.float64) - val)) / float(fx["exact_scale"]))
    kvd = d.kv_heads * d.head_dim
    worst = 0.0
    for layer in range(d.layers):
        k, v = s.kv(layer)
        for ptr, want in ((k, fx["cache_k"][layer]), (v, fx["cache_v"][layer])):
            for j, p in enumerate(fx["cache_pos"]):
                h = np.empty(kvd, np.uint16)
                arc.check(arc.lib().arc_memcpy_dtoh(h.ctypes.data, ptr + int(p) * kvd * 2, h.nbytes, None))
                worst = max(worst, norm_err(h.view(np.float16).astype(np.float64),
                                            want[j].view(np.float16).astype(np.float64)))
    _log(f"7B prefill 256: logits vs fp16-operand oracle {e16:.3g}, vs exact oracle (top 256) {e64:.3g}, "
         f"cache rows {worst:.3g}; next gpu {nxt} oracle {int(fx['f16_next'])} (margin {float(fx['f16_margin']):.4g}), "
         f"kernels {s.prefill_kernels}")
    assert nf == 0
    assert e16 <= F16_NORM and worst <= F16_NORM and e64 <= EXACT_NORM
    assert s.prefill_kernels == 8 * d.layers + 3
    if nxt != int(fx["f16_next"]):
        assert float(fx["f16_margin"]) < PF_TIE * float(fx["f16_scale"]) and nxt == int(fx["f16_second"])
        return
    cont, nf2 = s.decode(nxt, len(prompt), len(fx["cont_tokens"]))
    ref = fx["cont_tokens"]
    _log(f"continuation gpu {cont.tolist()}\n             oracle {ref.tolist()}")
    assert nf2 == 0
    diff = np.nonzero(cont != ref)[0]
    if diff.size:
        i = int(diff[0])
        assert fx["cont_margin"][i] < PF_TIE * fx["cont_scale"][i] and cont[i] == fx["cont_second"][i]
