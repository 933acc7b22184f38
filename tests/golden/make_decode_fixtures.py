"""Writes the oracle fixtures of the full-length decode and prompt-pass
parity tests (test infrastructure; runs the CPU oracle, never the GPU).

  python tests/golden/make_decode_fixtures.py [decode|prefill|all]

decode7b_greedy.npz -- the Qwen2.5-7B-shaped random-init model (seed
  DECODE_SEED), fp16 KV cache pre-filled with N(0, 1) to T = 512, 2048 and
  4096 positions (kv seed 99 + T), 64 greedy steps from token 1234 at
  position T, each step computed by the fp64 oracle (orc_decode_step):
    t{T}_tokens, t{T}_second  argmax / runner-up id of every step
    t{T}_margin, t{T}_scale   top1 - top2 logit gap and max|logit| per step
    t{T}_top_idx, t{T}_top_val  the first step's 256 largest logits
    t4096_logits              the first step's full logits at T = 4096 (fp32)

prefill7b_256.npz -- the same model shape (seed PREFILL_SEED), the 256-token
  prompt (7919 i + 13) mod vocab at positions 0..255, run through the oracle's
  prompt pass (orc_prompt_pass: bit-identical to stepping the tokens one by
  one) once with fp16 GEMM operands (the rounding of the MFMA prompt pass) and
  once exactly in fp64:
    f16_logits                last position's logits, fp16-operand oracle (fp32)
    f16_next, f16_second, f16_margin, f16_scale
    exact_next, exact_second, exact_margin, exact_scale, exact_top_idx/val
    cache_pos                 sampled positions; cache_k / cache_v: the
                              fp16-operand oracle's cache rows there, every
                              layer, [layer][pos][kv_dim] as fp16 bits
    cont_tokens, cont_second, cont_margin, cont_scale
                              16 greedy fp64 decode steps continuing from the
                              fp16-operand oracle's cache and f16_next
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import arcllm_amd as arc  # noqa: E402  (host-side model synthesis only)
import oracle_lib as orc  # noqa: E402

DECODE_SEED = 0x7B0DEC0DE
PREFILL_SEED = 0x9F11_0000
CONTEXTS = (512, 2048, 4096)
STEPS = 64
START_TOKEN = 1234
MAX_CTX = 4096 + STEPS
TOPK = 256
PROMPT = 256
PF_MAX_CTX = 320
CACHE_POS = (0, 1, 17, 128, 200, 255)
CONT_STEPS = 16


def prompt_ids(vocab: int, n: int = PROMPT) -> np.ndarray:
    return ((np.arange(n, dtype=np.uint64) * 7919 + 13) % vocab).astype(np.uint32)


def _log(msg: str) -> None:
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def _top(lg: np.ndarray, k: int = TOPK):
    order = np.argsort(-lg, kind="stable")[:k]
    return order.astype(np.uint32), lg[order].astype(np.float64)


def make_decode(path: str) -> None:
    d = arc.qwen25_7b_dims()
    _log("decode: synthesising the 7B-shaped model")
    T = arc.synth_model_tensors(d, DECODE_SEED)
    out = {"seed": np.uint64(DECODE_SEED), "steps": np.uint32(STEPS), "start_token": np.uint32(START_TOKEN),
           "max_ctx": np.uint32(MAX_CTX), "contexts": np.array(CONTEXTS, np.uint32)}
    for ctx in CONTEXTS:
        o = orc.DecodeOracle(d, T, MAX_CTX)
        o.fill_kv(ctx, 99 + ctx, arc.synth_normal)
        first = o.step(START_TOKEN, ctx)
        # the greedy run repeats step 0 from a fresh cache row: same result
        o2 = orc.DecodeOracle(d, T, MAX_CTX)
        o2.fill_kv(ctx, 99 + ctx, arc.synth_normal)
        toks, second, margins, scale = o2.greedy(START_TOKEN, ctx, STEPS, log=_log)
        assert int(np.argmax(first)) == int(toks[0])
        out[f"t{ctx}_tokens"] = toks
        out[f"t{ctx}_second"] = second
        out[f"t{ctx}_margin"] = margins
        out[f"t{ctx}_scale"] = scale
        out[f"t{ctx}_top_idx"], out[f"t{ctx}_top_val"] = _top(first)
        if ctx == 4096:
            out["t4096_logits"] = first.astype(np.float32)
        _log(f"ctx {ctx}: tokens {toks.tolist()} min margin {margins.min():.4g}")
    np.savez_compressed(path, **out)
    _log(f"wrote {path}")


def make_prefill(path: str) -> None:
    d = arc.qwen25_7b_dims()
    _log("prefill: synthesising the 7B-shaped model")
    T = arc.synth_model_tensors(d, PREFILL_SEED)
    prompt = prompt_ids(d.vocab)
    o16 = orc.DecodeOracle(d, T, PF_MAX_CTX, f16_operands=True)
    o64 = orc.DecodeOracle(d, T, PF_MAX_CTX)
    # layer by layer over all positions: bit-identical to stepping each token
    l16 = o16.prompt(prompt, 0)
    _log("prefill: fp16-operand oracle done")
    l64 = o64.prompt(prompt, 0)
    _log("prefill: exact oracle done")
    out = {"seed": np.uint64(PREFILL_SEED), "prompt": prompt, "max_ctx": np.uint32(PF_MAX_CTX)}
    for name, lg in (("f16", l16), ("exact", l64)):
        order = np.argsort(-lg, kind="stable")
        out[f"{name}_next"] = np.uint32(order[0])
        out[f"{name}_second"] = np.uint32(order[1])
        out[f"{name}_margin"] = np.float64(lg[order[0]] - lg[order[1]])
        out[f"{name}_scale"] = np.float64(np.max(np.abs(lg)))
    out["f16_logits"] = l16.astype(np.float32)
    out["exact_top_idx"], out["exact_top_val"] = _top(l64)
    kvd = d.kv_heads * d.head_dim
    pos = np.array(CACHE_POS, np.uint32)
    ck = np.empty((d.layers, len(pos), kvd), np.uint16)
    cv = np.empty_like(ck)
    for layer in range(d.layers):
        base = layer * PF_MAX_CTX * kvd
        for j, p in enumerate(pos):
            ck[layer, j] = o16.kc[base + p * kvd: base + (p + 1) * kvd]
            cv[layer, j] = o16.vc[base + p * kvd: base + (p + 1) * kvd]
    out["cache_pos"], out["cache_k"], out["cache_v"] = pos, ck, cv
    # exact decode steps continuing from the fp16-operand oracle's cache
    oc = orc.DecodeOracle(d, T, PF_MAX_CTX)
    oc.kc[:] = o16.kc
    oc.vc[:] = o16.vc
    toks, second, margins, scale = oc.greedy(int(out["f16_next"]), PROMPT, CONT_STEPS, log=_log)
    out["cont_tokens"], out["cont_second"], out["cont_margin"], out["cont_scale"] = toks, second, margins, scale
    np.savez_compressed(path, **out)
    _log(f"wrote {path}: f16 next {int(out['f16_next'])} (margin {float(out['f16_margin']):.4g}), exact next "
         f"{int(out['exact_next'])} (margin {float(out['exact_margin']):.4g}), continuation {toks.tolist()}")


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what in ("decode", "all"):
        make_decode(os.path.join(HERE, "decode7b_greedy.npz"))
    if what in ("prefill", "all"):
        make_prefill(os.path.join(HERE, "prefill7b_256.npz"))
