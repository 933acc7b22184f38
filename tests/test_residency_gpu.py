"""The residency plan on the GPU: a model is one device allocation and a
session one more, with the KV cache, working memory and EXEC148 reserve the
plan reports (arc_session_residency, the reference's weight / KV / working
accounting, src/arcllm_v1_runtime.cpp:227-266), and nothing after session
creation allocates device memory: the batched prompt pass over two passes,
the stepwise prompt pass, decoding with and without the captured graph, the
logits read-back, building and validating an EXEC148 image in the model's
reserve, and decoding through it (route B)."""
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc
from decode_common import tiny_dims

pytestmark = pytest.mark.gpu

SEED = 0x5E55_1011


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def test_one_allocation_each_and_none_after_session_creation():
    d = tiny_dims(layers=3)  # layer 1's ffn_down is Q4_K
    T = arc.synth_model_tensors(d, SEED)
    max_ctx = 300
    n0 = arc.device_allocations()
    model = arc.Model(d, T)
    assert arc.device_allocations() == n0 + 1
    s = arc.Session(model, max_ctx)
    assert arc.device_allocations() == n0 + 2

    r = s.residency()
    _log(f"residency {r}")
    kvd = d.kv_heads * 128
    assert r["kv_bytes"] == 2 * d.layers * max_ctx * kvd * 2
    assert r["weight_bytes"] == model.weight_bytes
    base, stride, slots = model.exec148_reserve()
    rows, K = d.hidden, d.ffn
    q4_layers = [layer for layer in range(d.layers) if d.down_type[layer] == arc.Q4_K]
    assert slots == len(q4_layers) == 1
    assert stride >= rows * (K // 256) * 148 and stride % 256 == 0 and base % 256 == 0
    assert r["exec148_reserve_bytes"] == stride * slots
    assert r["model_arena_bytes"] >= r["weight_bytes"] + r["exec148_reserve_bytes"]
    assert r["working_bytes"] > 0
    assert r["total_bytes"] == r["model_arena_bytes"] + r["kv_bytes"] + r["working_bytes"]

    rng = np.random.default_rng(3)
    prompt = rng.integers(0, d.vocab, 280).astype(np.uint32)  # two passes of the batched prompt pass
    nxt, nf = s.prefill(prompt, logits=True)
    assert nf == 0
    s.logits()
    toks, nf = s.decode(nxt, len(prompt), 8)
    assert nf == 0
    toks_eager, _ = s.decode(nxt, len(prompt), 8, logits=True, graph=False)
    assert np.array_equal(toks, toks_eager)
    b = arc.Session(model, 64)  # a second session is a creation, not a call
    n1 = arc.device_allocations()
    b.prefill(prompt[:20], stepwise=True)

    # route B from the model's reserve
    src = model.tensor_device(q4_layers[0], arc.T_FFN_DOWN)
    arc.exec148_materialize(src, rows, K, base)
    arc.synchronize()
    assert arc.exec148_validate(src, base, rows, K) == 0
    s.route_down(q4_layers[0], base)
    toks_b, nf = s.decode(nxt, len(prompt), 8)
    assert nf == 0
    o = orc.DecodeOracle(d, T, max_ctx)
    o.prompt(prompt, 0)
    _log(f"route A {toks.tolist()} route B {toks_b.tolist()}")
    o.follow(nxt, len(prompt), toks_b)
    s.route_down(q4_layers[0], None)
    assert arc.device_allocations() == n1
    b.close()
    s.close()
    model.close()
