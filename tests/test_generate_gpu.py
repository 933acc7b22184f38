"""arcllm::v1::runtime::generate end to end on the GPU, through the CLI
(tests/gguf_write.py model file -> GGUF reader -> upload -> prompt pass ->
greedy decode), against the fp64 oracle fed the same prompt; and the prompt
entry point arc_session_prefill on its own.

Token comparison uses the near-tie rule of test_decode_gpu.py (a differing
step must be a top-2 tie within 2e-3 * max|logit| and ends the comparison).
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import arcllm_amd as arc
import gguf_write as gw
import oracle_lib as orc
from decode_common import tiny_dims

pytestmark = pytest.mark.gpu

SEED = 0x6E7E_CA7E


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def oracle_follow(d, T, prompt, gpu_tokens):
    """Every generated token checked against the oracle, teacher-forced: the
    prompt through the oracle (fp16-operand mode when it has two or more
    tokens, like the batched prompt pass), the first token against its argmax
    (runner-up allowed below the prompt pass's near-tie bound, 2e-2 of
    max|logit|), then each later token against the exact oracle fed the GPU's
    previous token (DecodeOracle.follow).  Returns the near-tie steps."""
    gpu_tokens = np.asarray(gpu_tokens)
    o = orc.DecodeOracle(d, T, len(prompt) + len(gpu_tokens), f16_operands=len(prompt) > 1)
    for i, t in enumerate(prompt):
        lg = o.step(int(t), i)
    o.f16 = 0
    order = np.argsort(-lg, kind="stable")
    ties = 0
    if int(gpu_tokens[0]) != int(order[0]):
        margin, scale = float(lg[order[0]] - lg[order[1]]), float(np.max(np.abs(lg)))
        assert int(gpu_tokens[0]) == int(order[1]) and margin < 2e-2 * scale, "first token is not a near tie"
        ties = 1
    return ties + o.follow(int(gpu_tokens[0]), len(prompt), gpu_tokens[1:])


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def thresholds():
    """The gfx950 registration's reuse thresholds (future decode tokens)."""
    r = subprocess.run([arc.Q4_PATHS_PATH, "--thresholds"], capture_output=True, text=True, timeout=30, check=True)
    return json.loads(r.stdout)


def test_generate_cli_matches_oracle(tmp_path):
    d = tiny_dims(layers=3)
    T = arc.synth_model_tensors(d, SEED)
    path = str(tmp_path / "model.gguf")
    gw.write_qwen2_model(path, d, T)
    prompt = [17, 5, 900, 33, 2048, 7, 4095]
    max_new = thresholds()["profile0"]["p1"] + 3
    r = subprocess.run([arc.CLI_PATH, "--model", path, "--shader-dir", "builtin", "--tokens",
                        ",".join(map(str, prompt)), "--max-new", str(max_new), "--profile", "0",
                        "--within-validated-domain", "1"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout)
    assert res["schema"] == "arcllm.v1.runtime.result.v0.1"
    gpu = res["generated_token_ids"]
    _log(f"gpu={gpu}")
    assert len(gpu) == max_new
    _log(f"near-tie steps: {oracle_follow(d, T, prompt, gpu)}")
    st = res["stats"]
    per_step = 1 + 4 * d.layers  # q/k/v, attention + o, gate/up, down; LM head + next token
    # batched prompt pass: embed + first norm, 8 launches per layer, LM head + next token
    assert st["prefill_dispatches"] == 8 * d.layers + 3 and st["prefill_submits"] == 1
    assert st["decode_dispatches_per_step"] == per_step and st["decode_submits_per_step"] == 1
    # layer 1's ffn_down is Q4_K: within the evidence scope and with
    # max_new - 1 future tokens (>= the P1 threshold) the policy acquires the EXEC148 image by P1
    # before the first decode step, every step runs route B, and the close
    # decision evicts it
    assert st["decode_steps"] == max_new - 1 and st["route_b_steps"] == max_new - 1
    assert st["route_a_steps"] == 0 and st["finite"] is True
    assert st["acquire_events"] == 1 and st["evict_events"] == 1
    assert (st["b_allocations"], st["b_materializations"], st["b_validations"], st["b_releases"]) == (1, 1, 1, 1)
    assert (st["p1_calls"], st["p3_calls"], st["p0_calls"]) == (1, 0, 0)


def _q4_model(tmp_path, layers, seed):
    d = tiny_dims(layers=layers)
    T = arc.synth_model_tensors(d, seed)
    path = str(tmp_path / "q4.gguf")
    gw.write_qwen2_model(path, d, T)
    return d, T, path


def _cli(path, prompt, max_new, profile, scope, sidecar=None):
    cmd = [arc.CLI_PATH, "--model", path, "--shader-dir", "builtin", "--tokens", ",".join(map(str, prompt)),
           "--max-new", str(max_new), "--profile", str(profile), "--within-validated-domain", str(scope)]
    if sidecar:
        cmd += ["--sidecar", sidecar]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def test_generate_routes_by_scope_and_reuse(tmp_path):
    """Route A outside the evidence scope or below the P1 threshold of the
    profile; route B from the threshold on (max_new - 1 future tokens at the
    first decode step), with the same tokens as the oracle either way."""
    d, T, path = _q4_model(tmp_path, 2, SEED + 7)
    prompt = [5, 77, 1024]
    th = thresholds()
    t0, t1 = th["profile0"]["p1"], th["profile1"]["p1"]
    longest = t1 + 2
    cases = [  # (max_new, profile, scope, route B expected)
        (longest, 0, 0, False), (t0, 0, 1, False), (t0 + 1, 0, 1, True), (t1, 1, 1, False), (t1 + 1, 1, 1, True)]
    for max_new, prof, scope, route_b in cases:
        _log(f"case max_new={max_new} profile={prof} scope={scope}")
        res = _cli(path, prompt, max_new, prof, scope)
        st = res["stats"]
        steps = max_new - 1
        assert st["decode_steps"] == steps
        if route_b:
            assert (st["route_a_steps"], st["route_b_steps"]) == (0, steps)
            assert (st["acquire_events"], st["evict_events"], st["p1_calls"], st["b_releases"]) == (1, 1, 1, 1)
        else:
            assert (st["route_a_steps"], st["route_b_steps"]) == (steps, 0)
            assert (st["acquire_events"], st["evict_events"], st["b_allocations"]) == (0, 0, 0)
        assert len(res["generated_token_ids"]) == max_new
        _log(f"near-tie steps: {oracle_follow(d, T, prompt, res['generated_token_ids'])}")


def test_q4_paths_tool_all_acquisition_paths(tmp_path):
    """P1 (GPU repack), P3 (sidecar written from the P1 image) and P0 (host
    repack) give the same EXEC148 image, equal to the oracle's repack of the
    layers' Q4_K tensors, validated with zero mismatched blocks; route A and
    route B decode the same tokens as the oracle from a prefilled KV cache."""
    d, T, path = _q4_model(tmp_path, 3, SEED + 8)
    ctx, steps, kv_seed = 40, 12, 77
    sidecar = str(tmp_path / "family.e148")
    r = subprocess.run([arc.Q4_PATHS_PATH, "--model", path, "--ctx", str(ctx), "--steps", str(steps),
                        "--paths", "p1,p3,p0", "--sidecar", sidecar, "--seed", str(kv_seed - 1)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout)
    _log(json.dumps({k: v for k, v in res.items() if k != "route_a"}))
    q4_layers = [layer for layer in range(d.layers) if d.down_type[layer] == arc.Q4_K]
    assert res["q4_layers"] == q4_layers
    image = np.concatenate([orc.exec148(T[3 + 12 * layer + 11], d.hidden, d.ffn) for layer in q4_layers])
    assert res["family_bytes"] == image.size
    h = 1469598103934665603
    for b in image.tobytes():
        h = ((h ^ b) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    want = f"{h:016x}"
    for p in ("p1", "p3", "p0"):
        assert res["paths"][p]["mismatched_blocks"] == 0
        assert res["paths"][p]["image_fnv"] == want, p
    assert res["images_equal"] is True
    assert os.path.getsize(sidecar) == image.size
    o = orc.DecodeOracle(d, T, ctx + steps + 2)
    for route in ("route_a", "route_b"):
        assert len(res[route]["tokens"]) == steps
        o.fill_kv(ctx, kv_seed, arc.synth_normal)
        _log(f"{route}: near-tie steps {o.follow(1234, ctx, res[route]['tokens'])}")


def test_generate_single_token_request(tmp_path):
    d = tiny_dims(layers=1)
    T = arc.synth_model_tensors(d, SEED + 1)
    path = str(tmp_path / "one.gguf")
    gw.write_qwen2_model(path, d, T)
    r = subprocess.run([arc.CLI_PATH, "--model", path, "--shader-dir", "builtin", "--tokens", "3", "--max-new", "1",
                        "--profile", "1", "--within-validated-domain", "0"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout)
    assert len(res["generated_token_ids"]) == 1
    oracle_follow(d, T, [3], res["generated_token_ids"])
    assert res["stats"]["decode_steps"] == 0 and res["stats"]["decode_dispatches_per_step"] == 0


def test_session_prefill_logits_and_continuation():
    d = tiny_dims(layers=2)
    T = arc.synth_model_tensors(d, SEED + 2)
    model = arc.Model(d, T)
    prompt = np.array([11, 400, 3000, 12, 1], np.uint32)
    s = arc.Session(model, 64)
    nxt, nf = s.prefill(prompt, logits=True)
    lg = s.logits()
    o = orc.DecodeOracle(d, T, 64, f16_operands=True)
    for i, t in enumerate(prompt):
        ref = o.step(int(t), i)
    assert nf == 0
    assert np.max(np.abs(lg - ref)) <= 5e-3 * np.max(np.abs(ref))  # normwise, as tests/test_prefill_gpu.py
    assert nxt == int(np.argmax(lg))
    # prefill in two calls (positions continue) gives the same next token, and
    # eager launches agree with the captured graph
    s2 = arc.Session(model, 64)
    s2.prefill(prompt[:2])
    n2, _ = s2.prefill(prompt[2:], pos0=2, graph=False)
    assert n2 == nxt
    with pytest.raises(arc.ArcError):
        s2.prefill(np.array([d.vocab], np.uint32), pos0=5)
    with pytest.raises(arc.ArcError):
        s2.prefill(np.arange(70, dtype=np.uint32) % 100, pos0=0)
