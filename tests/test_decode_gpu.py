"""Greedy decode on the GPU vs the fp64 oracle: token IDs must be identical.

The GPU runs the captured decode step (embedding, layers x [QK+RoPE+K store,
V store, GQA chunks, GQA merge, O+residual, gate/up+SwiGLU, down+residual],
LM head + argmax)
and feeds its own argmax back; the oracle does the same in fp64 from the
same random-init weights and the same fp16 KV pre-fill.

The 28-layer 7B-shaped runs compare with oracle fixtures written in the
build container (tests/golden/make_decode_fixtures.py: 64 fp64 greedy steps
per context, margins and first-step logits); the small models run the oracle
here.

Near-tie rule: the GPU computes logits in fp32 with a relative error bound of
1e-3 (of max|logit|, the GEMV bar), so a step whose fp64 top1-top2 margin is
below 2e-3 * max|logit| may legitimately pick the runner-up.  At the first
differing step the test requires exactly that (margin below the bound and the
GPU token equal to the oracle's runner-up) and stops comparing, since the two
sequences then continue from different tokens.  Every other step must match.
"""
import os
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc
from decode_common import tiny_dims

pytestmark = pytest.mark.gpu

SEED = 0x7B0DEC0DE
TIE_BOUND = 2e-3
# End-to-end logits (a whole decode step in fp32 against the fp64 oracle):
# normwise max|gpu - ref| / max|ref| <= E2E_NORM, plus the reference's own
# component gates max_abs <= 0.02 and RMSE <= 0.005
# (src/sa1_component_benchmark.cpp:312-314).  The per-element metric with
# its 1e-3 * max|ref| floor is the bar of single kernels; through a full
# step, fp32 rounding of the hidden state alone (~1e-7 relative) moves a
# near-zero logit by ~1e-3 of that floor, so it is reported, not asserted.
# Measured (one MI355X): 2-layer models 7e-7 .. 7e-6, the 28-layer 7B shape
# 6.5e-5.
E2E_NORM = 2e-4


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_pair(d, T, model, max_ctx, ctx, token, steps, kv_seed):
    sess = arc.Session(model, max_ctx)
    sess.fill_kv(ctx, kv_seed)
    gpu, nf = sess.decode(token, ctx, steps)
    _log(f"gpu ctx={ctx} steps={steps} tokens={gpu.tolist()}")
    o = orc.DecodeOracle(d, T, max_ctx)
    o.fill_kv(ctx, kv_seed, arc.synth_normal)
    ref, second, margins, scale = o.greedy(token, ctx, steps, log=_log)
    _log(f"ctx={ctx} ref={ref.tolist()}\n      min margin={margins.min():.4g} "
         f"median margin={np.median(margins):.4g} kernels/step={sess.kernels_per_step}")
    return sess, gpu, nf, ref, second, margins, scale


def assert_tokens_match(gpu, ref, second, margins, scale):
    diff = np.nonzero(gpu != ref)[0]
    if diff.size == 0:
        return len(gpu)
    i = int(diff[0])
    bound = TIE_BOUND * scale[i]
    _log(f"first differing step {i}: gpu={int(gpu[i])} oracle={int(ref[i])} runner-up={int(second[i])} "
         f"margin={margins[i]:.4g} bound={bound:.4g}")
    assert margins[i] < bound and gpu[i] == second[i], "token differs at a step that is not a near tie"
    return i


def test_tiny_model_64_steps_mixed_quant_types():
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED)
    model = arc.Model(d, T)
    sess, gpu, nf, ref, second, margins, scale = run_pair(d, T, model, 256, 100, 17, 64, 11)
    assert nf == 0
    assert assert_tokens_match(gpu, ref, second, margins, scale) >= 48


def test_tiny_model_first_step_logits_and_eager_replay():
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED)
    model = arc.Model(d, T)
    s1 = arc.Session(model, 128)
    s1.fill_kv(40, 5)
    tok, _ = s1.decode(9, 40, 1, logits=True)
    lg = s1.logits()
    o = orc.DecodeOracle(d, T, 128)
    o.fill_kv(40, 5, arc.synth_normal)
    ref = o.step(9, 40)
    e2e_check(lg, ref, "tiny model, ctx 40")
    assert int(tok[0]) == int(np.argmax(ref))
    # the graph replay and kernel-by-kernel launches give the same tokens
    a = arc.Session(model, 128)
    a.fill_kv(40, 5)
    b = arc.Session(model, 128)
    b.fill_kv(40, 5)
    ta, _ = a.decode(9, 40, 32, graph=True)
    tb, _ = b.decode(9, 40, 32, graph=False)
    assert np.array_equal(ta, tb)
    # decoding in two calls continues from the cache exactly like one call
    c = arc.Session(model, 128)
    c.fill_kv(40, 5)
    t1, _ = c.decode(9, 40, 10)
    t2, _ = c.decode(int(t1[-1]), 50, 22)
    assert np.array_equal(np.concatenate([t1, t2]), ta)


def test_tiny_model_row_stream_gemvs_forced():
    """The decode step with the row-stream kernel forced on: the o projection
    and Q4_K down (residual epilogue), the fused gate/up with the ffn norm.
    First-step logits against the fp64 oracle, then 64 greedy steps."""
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED)
    model = arc.Model(d, T)
    arc.tune_rowstream(1)
    try:
        s1 = arc.Session(model, 128)
        s1.fill_kv(40, 5)
        tok, _ = s1.decode(9, 40, 1, logits=True)
        lg = s1.logits()
        sess, gpu, nf, ref, second, margins, scale = run_pair(d, T, model, 256, 100, 17, 64, 11)
    finally:
        arc.tune_rowstream(-1)
    o = orc.DecodeOracle(d, T, 128)
    o.fill_kv(40, 5, arc.synth_normal)
    ref1 = o.step(9, 40)
    e2e_check(lg, ref1, "tiny model, row-stream forced, ctx 40")
    assert int(tok[0]) == int(np.argmax(ref1))
    assert nf == 0
    assert assert_tokens_match(gpu, ref, second, margins, scale) >= 48


def test_seven_query_heads_per_kv_head_long_context():
    """The 7B model's GQA grouping (7 query heads per kv head) on a small
    model, at a context long enough for several attention splits per kv head
    (and more than one chunk per split past 4096 positions): first-step
    logits (end-to-end gates) and 16 greedy tokens against the oracle."""
    d = arc.ModelDims()
    d.hidden, d.q_heads, d.kv_heads, d.head_dim = 1792, 14, 2, 128
    d.ffn, d.vocab, d.layers = 512, 2048, 2
    d.rms_eps, d.rope_theta = 1e-6, 1e6
    for layer in range(d.layers):
        d.v_type[layer], d.down_type[layer] = arc.Q6_K, arc.Q4_K
    T = arc.synth_model_tensors(d, SEED + 7)
    model = arc.Model(d, T)
    for ctx, max_ctx in ((700, 720), (4200, 4220)):
        s = arc.Session(model, max_ctx)
        s.fill_kv(ctx, 21)
        tok, nf = s.decode(33, ctx, 1, logits=True)
        lg = s.logits()
        o = orc.DecodeOracle(d, T, max_ctx)
        o.fill_kv(ctx, 21, arc.synth_normal)
        ref = o.step(33, ctx)
        e2e_check(lg, ref, f"hpk 7, ctx {ctx}")
        assert nf == 0
        gpu, _ = s.decode(int(tok[0]), ctx + 1, 15)
        ref_t, second, margins, scale = o.greedy(int(np.argmax(ref)), ctx + 1, 15)
        assert int(tok[0]) == int(np.argmax(ref)) or float(np.sort(ref)[-1] - np.sort(ref)[-2]) < TIE_BOUND * float(
            np.max(np.abs(ref)))
        if int(tok[0]) == int(np.argmax(ref)):
            assert_tokens_match(gpu, ref_t, second, margins, scale)


def test_attention_o_one_launch_matches_two_launches():
    """Attention and the o projection as one launch (the o workgroups load
    their first weights, then wait for every kv head's output) against the
    two-launch step, on the 7-heads-per-kv-head grouping at a one-split and
    a many-split context, captured graph and eager: first-step logits within
    1e-5 of the logit scale (the two o launches may sum in another lane
    layout), the same 24 greedy tokens, 4 against 5 launches per layer, and
    the same tokens again (the done and pass counters are back at zero)."""
    d = arc.ModelDims()
    d.hidden, d.q_heads, d.kv_heads, d.head_dim = 1792, 14, 2, 128
    d.ffn, d.vocab, d.layers = 512, 2048, 2
    d.rms_eps, d.rope_theta = 1e-6, 1e6
    for layer in range(d.layers):
        d.v_type[layer], d.down_type[layer] = arc.Q6_K, arc.Q4_K
    T = arc.synth_model_tensors(d, SEED + 9)
    model = arc.Model(d, T)
    for ctx in (40, 700):
        for graph in (True, False):
            res = {}
            for fuse in (True, False, True):
                arc.tune_fuse_attn_o(fuse)
                try:
                    s = arc.Session(model, 760)
                    s.fill_kv(ctx, 21)
                    tok, nf0 = s.decode(5, ctx, 1, logits=True, graph=graph)
                    lg = s.logits()
                    toks, nf1 = s.decode(int(tok[0]), ctx + 1, 24, graph=graph)
                    kps = s.kernels_per_step
                finally:
                    arc.tune_fuse_attn_o(True)
                assert nf0 == 0 and nf1 == 0
                assert kps == 1 + (4 if fuse else 5) * d.layers
                if fuse in res:
                    assert np.array_equal(lg, res[fuse][0]) and np.array_equal(toks, res[fuse][1])
                res[fuse] = (lg, toks)
            (lf, tf), (lu, tu) = res[True], res[False]
            err = float(np.max(np.abs(lf.astype(np.float64) - lu))) / float(np.max(np.abs(lu)))
            _log(f"ctx {ctx} graph {graph}: fused vs two launches, logits {err:.3g}, tokens {tf.tolist()}")
            assert err <= 1e-5
            assert np.array_equal(tf, tu)


def test_attention_o_wait_gives_up_and_reports_an_error():
    """The bounded wait of the attention + o launch: with the attention made
    to withhold its signal (a host setting; every kernel still runs to its
    end), each o workgroup's wait gives up after its poll limit and the
    decode call returns an error naming the expired waits; the session then
    decodes normally again, with the tokens of a fresh session."""
    d = tiny_dims(layers=2)
    T = arc.synth_model_tensors(d, SEED + 13)
    model = arc.Model(d, T)
    ref = arc.Session(model, 128)
    ref.fill_kv(40, 3)
    want, _ = ref.decode(7, 40, 4)
    s = arc.Session(model, 128)
    s.fill_kv(40, 3)
    arc.tune_fuse_attn_o(2)
    try:
        with pytest.raises(arc.ArcError, match="gave up"):
            s.decode(7, 40, 1)
    finally:
        arc.tune_fuse_attn_o(True)
    s2 = arc.Session(model, 128)
    s2.fill_kv(40, 3)
    got, nf = s2.decode(7, 40, 4)
    assert nf == 0 and np.array_equal(got, want)
    s.fill_kv(40, 3)
    again, nf = s.decode(7, 40, 4, graph=False)
    assert nf == 0 and np.array_equal(again, want)


def test_decode_rejects_bad_requests():
    d = tiny_dims(layers=1)
    model = arc.Model(d, seed=3)
    s = arc.Session(model, 16)
    with pytest.raises(arc.ArcError):
        s.decode(d.vocab, 0, 1)  # token out of vocabulary
    with pytest.raises(arc.ArcError):
        s.decode(1, 10, 7)  # runs past the context


FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "decode7b_greedy.npz")


@pytest.fixture(scope="module")
def qwen7b_fixture():
    """The 7B-shaped model of tests/golden/make_decode_fixtures.py and the
    oracle's 64-step greedy runs at T = 512, 2048, 4096."""
    fx = np.load(FIXTURE)
    d = arc.qwen25_7b_dims()
    _log("building the 7B-shaped random-init model")
    model = arc.Model(d, seed=int(fx["seed"]))
    _log(f"model resident: {model.weight_bytes / 1e9:.3f} GB")
    return d, model, fx


def e2e_check(lg, ref, what):
    """Asserts the end-to-end logit gates; returns the normwise error."""
    lg = np.asarray(lg, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(lg - ref)
    scale = float(np.max(np.abs(ref)))
    norm = float(err.max()) / scale
    rmse = float(np.sqrt(np.mean(err * err)))
    _log(f"{what}: logits normwise {norm:.3g}, max_abs {err.max():.3g}, rmse {rmse:.3g}, per-element (1e-3 floor) "
         f"{orc.rel_err(lg, ref):.3g}")
    assert norm <= E2E_NORM and float(err.max()) <= 0.02 and rmse <= 0.005
    return norm


def top_err(gpu_logits, idx, val, scale):
    """max |gpu - oracle| / max(|oracle|, 1e-3 * max|logit|) over the oracle's
    largest logits (the metric of orc.rel_err, with the whole vector's scale)."""
    g = np.asarray(gpu_logits, np.float64)[idx]
    den = np.maximum(np.abs(val), 1e-3 * scale)
    return float(np.max(np.abs(g - val) / den))


@pytest.mark.parametrize("ctx", [512, 2048, 4096])
def test_qwen7b_shape_64_greedy_steps_match_oracle(qwen7b_fixture, ctx):
    """North-star case: 64 greedy steps of the 28-layer 7B-shaped model from
    a KV cache pre-filled to T positions; all 64 tokens equal to the fp64
    oracle's (the near-tie rule above does not apply here); the first step's 256 largest logits
    within 1e-3 per element, and at T = 4096 all 152,064 within the
    end-to-end gates."""
    d, model, fx = qwen7b_fixture
    steps = int(fx["steps"])
    sess = arc.Session(model, int(fx["max_ctx"]))
    sess.fill_kv(ctx, 99 + ctx)
    first, nf0 = sess.decode(int(fx["start_token"]), ctx, 1, logits=True)
    lg = sess.logits()
    scale = float(fx[f"t{ctx}_scale"][0])
    e_top = top_err(lg, fx[f"t{ctx}_top_idx"], fx[f"t{ctx}_top_val"], scale)
    msg = f"ctx {ctx}: first-step logits vs oracle (256 largest) {e_top:.3g}"
    _log(msg)
    assert e_top <= 1e-3
    if ctx == 4096:
        e2e_check(lg, fx["t4096_logits"].astype(np.float64), f"ctx {ctx}, all {lg.size} first-step logits")
    rest, nf1 = sess.decode(int(first[0]), ctx + 1, steps - 1)
    gpu = np.concatenate([first, rest])
    ref, second = fx[f"t{ctx}_tokens"], fx[f"t{ctx}_second"]
    margins, scales = fx[f"t{ctx}_margin"], fx[f"t{ctx}_scale"]
    _log(f"ctx {ctx}: gpu {gpu.tolist()}\n         oracle {ref.tolist()}\n         min margin {margins.min():.4g} "
         f"(bound {TIE_BOUND} * max|logit|), kernels/step {sess.kernels_per_step}")
    assert nf0 == 0 and nf1 == 0
    assert sess.kernels_per_step == 1 + 4 * d.layers  # 4 per layer (attention + o fused), LM head + argmax
    matched = assert_tokens_match(gpu, ref, second, margins, scales)
    _log(f"ctx {ctx}: {matched} of {steps} steps compared and identical")
    # the kernels are deterministic and the fixture fixed: every one of the
    # 64 tokens must equal the oracle's, near ties included
    assert matched == steps, f"ctx {ctx}: only {matched} of {steps} greedy tokens equal the oracle's"
