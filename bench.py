"""Benchmark of the packed Q4_K/Q6_K decode hot path on one MI355X.

Workload (one "step"): the fused FFN block of a Qwen2.5-7B-shaped decode
layer -- Q4_K gate+up [18944 x 3584] with the SwiGLU epilogue, then the Q6_K
down projection [3584 x 18944] split-K over 74 super-block columns with its
fixed-order second pass -- over seeded synthetic weights and x ~ N(0, 1).
Inputs are resident in HBM before timing; the step rotates over `--banks`
copies of the weights (default 8, 1.06 GB) so the 256 MB Infinity Cache
cannot serve them.

value = algorithmic bytes per step (weights + x/s/y reads and writes,
132,257,792 B) / time, in GB/s.  The roofline object is for the dominant
kernel (the fused gate/up + SwiGLU launch), timed with HIP events on its
own stream: K back-to-back launches over the same weight banks, median of
three such loops after a warm-up.  cpu_baseline times the oracle's serial-fp32 restatement of the
reference CPU kernels on the same workload (bounded sample, 1 thread).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import arcllm_amd as arc  # noqa: E402

H, FFN, VOC = 3584, 18944, 152064
SPLITS = 74
SEED = 0x0B5E_7C4_2026
PEAK_HBM_GBS = 8000.0
PEAK_FP16_FLOPS = 2.5e15  # dense fp16 MFMA, MI355X

Q4_ROW = (H // 256) * 144
Q6_ROW_DOWN = (FFN // 256) * 210
W_GATE = FFN * Q4_ROW                      # 38,191,104
W_DOWN = H * Q6_ROW_DOWN                   # 55,695,360
BYTES_GATEUP = 2 * W_GATE + H * 4 + FFN * 4                  # weights + x read + s write
BYTES_DOWN = W_DOWN + FFN * 4 + H * 4                         # weights + s read + y write
BYTES_STEP = 2 * W_GATE + W_DOWN + H * 4 + FFN * 4 * 2 + H * 4  # 132,257,792
BYTES_GATE = W_GATE + H * 4 + FFN * 4                        # config: single gate GEMV
W_LM = VOC * (H // 256) * 210
BYTES_LM = W_LM + H * 4 * 2 + 4                              # + h, norm weight, token id


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_loop(fn, iters: int, stream: arc.Stream) -> float:
    """Average ms per call of fn(i) over iters launches on `stream`."""
    e0, e1 = arc.Event(), arc.Event()
    e0.record(stream)
    for i in range(iters):
        fn(i)
    e1.record(stream)
    stream.synchronize()
    return e0.elapsed_ms(e1) / iters


def cpu_baseline(sample_reps: int) -> dict:
    """The oracle's serial-fp32 restatement of the reference CPU kernels
    (per-element decode, one row at a time) on the same FFN block."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc  # the checker; used here only as the CPU baseline

    wg = arc.synth_packed(arc.Q4_K, SEED, 1, FFN, H)
    wu = arc.synth_packed(arc.Q4_K, SEED, 2, FFN, H)
    wd = arc.synth_packed(arc.Q6_K, SEED, 3, H, FFN)
    x = arc.synth_normal(SEED, 4, H)

    def step(threads: int) -> float:
        t0 = time.perf_counter()
        g = orc.gemv_r0(arc.Q4_K, wg, FFN, H, x, threads=threads)
        u = orc.gemv_r0(arc.Q4_K, wu, FFN, H, x, threads=threads)
        s = np.empty_like(g)
        orc.oracle().orc_swiglu_f32(g.ctypes.data, u.ctypes.data, FFN, s.ctypes.data)
        orc.gemv_r0(arc.Q6_K, wd, H, FFN, s, threads=threads)
        return time.perf_counter() - t0

    step(1)  # warmup
    t1 = sorted(step(1) for _ in range(sample_reps))[sample_reps // 2]
    ncores = min(os.cpu_count() or 1, 16)
    step(ncores)
    tn = sorted(step(ncores) for _ in range(sample_reps))[sample_reps // 2]
    return {
        "value": round(BYTES_STEP / t1 / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full FFN block (gate+up+SwiGLU+down), median of {sample_reps} after 1 warmup; "
                  f"oracle serial-fp32 per-element decode, gcc -O2 -ffp-contract=off",
        "ms_per_step": round(t1 * 1e3, 2),
        "all_cores": {"cores": ncores, "value": round(BYTES_STEP / tn / 1e9, 4), "ms_per_step": round(tn * 1e3, 2)},
    }


def decode_leg(steps: int, warmup: int, graph: bool = True) -> dict:
    """Greedy decode of the 28-layer Qwen2.5-7B-shaped random-init model
    (Q4_K attn q/k/o, gate, up; Q6_K attn v, ffn down, output), fp16 KV cache
    pre-filled with N(0, 1) to each context, `steps` tokens per context timed
    wall-clock around one captured-graph decode call (one graph replay per
    token, token IDs downloaded at the end).  Bytes per token = all weights
    + the K and V rows read by attention (2 * layers * (ctx+i) * kv_dim * 2 B)."""
    d = arc.qwen25_7b_dims()
    log("decode: generating the 7B-shaped model")
    model = arc.Model(d, seed=SEED)
    wbytes = model.weight_bytes
    kvd = d.kv_heads * d.head_dim
    ctxs = (512, 2048, 4096)
    sess = arc.Session(model, max(ctxs) + max(steps, warmup, 1))
    out = {"model": "Qwen2.5-7B shape, 28 layers, Q4_K_M layout, random init",
           "launch": "captured graph, one replay per token" if graph else "kernel-by-kernel launches",
           "weight_bytes": wbytes, "steps": steps, "kernels_per_step": None, "contexts": {}}
    for ctx in ctxs:
        sess.fill_kv(ctx, SEED + ctx)
        sess.decode(1234, ctx, max(warmup, 1), graph=graph)  # captures the step graph on first use
        arc.synchronize()
        t0 = time.perf_counter()
        toks, nf = sess.decode(1234, ctx, steps, graph=graph)
        dt = time.perf_counter() - t0
        kv_bytes = sum(2 * d.layers * (ctx + i + 1) * kvd * 2 for i in range(steps))
        gbs = (wbytes * steps + kv_bytes) / dt / 1e9
        out["contexts"][str(ctx)] = {"tokens_per_s": round(steps / dt, 2), "ms_per_token": round(dt / steps * 1e3, 4),
                                     "GB/s": round(gbs, 1), "frac_of_peak_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                     "nonfinite": int(nf), "first_tokens": toks[:4].tolist()}
        log(f"decode ctx {ctx}: {steps / dt:.1f} tok/s, {dt / steps * 1e3:.3f} ms/token, {gbs:.0f} GB/s")
    out["kernels_per_step"] = sess.kernels_per_step
    sess.close()
    out["prefill"] = prefill_leg(model, d)
    model.close()
    return out


def prefill_leg(model, d, reps: int = 5) -> dict:
    """The 256-token prompt pass (config 4): TTFT = wall-clock of one
    arc_session_prefill call on a fresh session (token upload, 28 layers of
    MFMA GEMMs + causal GQA, LM head + argmax on the last row, control-block
    download), median of `reps` after a warmup.  MFMA work = the projections,
    2 * 256 * sum(N*K) over the layers."""
    S = 256
    prompt = (np.arange(S, dtype=np.uint64) * 7919 + 13) % d.vocab
    prompt = prompt.astype(np.uint32)
    kvd = d.kv_heads * d.head_dim
    nk = 0
    for layer in range(d.layers):
        nk += (d.hidden + 2 * kvd) * d.hidden + d.hidden * d.hidden + 2 * d.ffn * d.hidden + d.hidden * d.ffn
    flops = 2.0 * S * nk
    sess = arc.Session(model, S + 64)
    sess.prefill(prompt)  # warmup: buffers, code objects
    times = []
    for _ in range(reps):
        arc.synchronize()
        t0 = time.perf_counter()
        tok, nf = sess.prefill(prompt)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[reps // 2]
    log(f"prefill 256: TTFT {t * 1e3:.2f} ms, {flops / t / 1e12:.1f} TFLOP/s on the MFMA projections")
    out = {"tokens": S, "ttft_ms": round(t * 1e3, 3), "mfma_flops": flops,
           "mfma_tflops": round(flops / t / 1e12, 2), "mfma_frac_of_dense_fp16_peak": round(flops / t / PEAK_FP16_FLOPS, 4),
           "kernels": sess.prefill_kernels, "next_token": int(tok), "nonfinite": int(nf),
           "note": "fp16 GEMM operands (activations, dequantised weights), fp32 accumulation"}
    sess.close()
    return out


def load_traffic() -> dict | None:
    p = os.path.join(ROOT, "profiles", "gateup_swiglu_ffn7b_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--banks", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--components", action="store_true", help="also time the gate GEMV and LM head")
    ap.add_argument("--no-decode", action="store_true", help="skip the 28-layer decode leg")
    ap.add_argument("--decode-steps", type=int, default=64)
    ap.add_argument("--decode-eager", action="store_true",
                    help="launch the decode step kernel by kernel instead of replaying its captured graph")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: every box has one MI355X and the "
                                   "hot path is a single-GPU decode kernel; --gpus must be 1"}))
        return 2

    if arc.device_count() < 1:
        raise SystemExit("no HIP device visible")
    name, gfx = arc.device_info()
    log(f"device {name} {gfx}")

    B = max(1, args.banks)
    stream = arc.Stream()
    log("generating weights")
    wg_h = arc.synth_packed(arc.Q4_K, SEED, 1, FFN, H)
    wu_h = arc.synth_packed(arc.Q4_K, SEED, 2, FFN, H)
    wd_h = arc.synth_packed(arc.Q6_K, SEED, 3, H, FFN)
    x_h = arc.synth_normal(SEED, 4, H)
    banks = []
    for b in range(B):
        if b == 0:
            g, u, d = (arc.DeviceBuffer.from_array(a) for a in (wg_h, wu_h, wd_h))
        else:
            g, u, d = arc.DeviceBuffer(W_GATE), arc.DeviceBuffer(W_GATE), arc.DeviceBuffer(W_DOWN)
            for dst, src in ((g, banks[0][0]), (u, banks[0][1]), (d, banks[0][2])):
                arc.check(arc.lib().arc_memcpy_dtod(dst.ptr, src.ptr, src.nbytes, stream.handle))
        banks.append((g, u, d))
    stream.synchronize()
    x = arc.DeviceBuffer.from_array(x_h)
    s = arc.DeviceBuffer(FFN * 4)
    part = arc.DeviceBuffer(SPLITS * H * 4)
    y = arc.DeviceBuffer(H * 4)

    def ffn_step(i: int) -> None:
        g, u, d = banks[i % B]
        arc.gateup_swiglu(arc.Q4_K, g, u, FFN, H, x, s, stream)
        arc.gemv_splitk(arc.Q6_K, d, H, FFN, SPLITS, s, part, y, stream=stream)

    def gateup(i: int) -> None:
        g, u, _ = banks[i % B]
        arc.gateup_swiglu(arc.Q4_K, g, u, FFN, H, x, s, stream)

    def down(i: int) -> None:
        _, _, d = banks[i % B]
        arc.gemv_splitk(arc.Q6_K, d, H, FFN, SPLITS, s, part, y, stream=stream)

    log(f"warmup {args.warmup}")
    time_loop(ffn_step, max(args.warmup, 1), stream)
    arc.synchronize()
    log(f"timing {args.steps} steps")
    ms = time_loop(ffn_step, args.steps, stream)
    arc.synchronize()
    gbs = BYTES_STEP / (ms / 1e3) / 1e9

    # the roofline kernel back to back on its stream (launch latency hidden
    # behind the previous launch, as in the step): warmed up until the clocks
    # settle, then the median of three timed loops of K launches
    time_loop(gateup, max(args.warmup, 50), stream)
    ms_gu = sorted(time_loop(gateup, args.steps, stream) for _ in range(3))[1]
    ms_dn = time_loop(down, args.steps, stream)
    ach = BYTES_GATEUP / (ms_gu / 1e3) / 1e9
    log(f"step {ms * 1e3:.2f} us ({gbs:.1f} GB/s); gate/up {ms_gu * 1e3:.2f} us ({ach:.1f} GB/s); "
        f"down {ms_dn * 1e3:.2f} us ({BYTES_DOWN / (ms_dn / 1e3) / 1e9:.1f} GB/s)")

    # practical read ceiling of this box at the same byte counts, same rotation
    probe_out = arc.DeviceBuffer(2048 * 256 * 4)
    probe = [arc.DeviceBuffer(BYTES_STEP // 4096 * 4096) for _ in range(B)]
    ms_c_step = time_loop(lambda i: arc.probe_read(probe[i % B], probe[i % B].nbytes, probe_out, 2048, stream),
                          args.steps, stream)
    ms_c_gu = time_loop(lambda i: arc.probe_read(probe[i % B], BYTES_GATEUP // 4096 * 4096, probe_out, 2048, stream),
                        args.steps, stream)
    del probe
    ceil_step = (BYTES_STEP // 4096 * 4096) / (ms_c_step / 1e3) / 1e9
    ceil_gu = (BYTES_GATEUP // 4096 * 4096) / (ms_c_gu / 1e3) / 1e9
    log(f"stream-read ceiling: {ceil_step:.0f} GB/s at {BYTES_STEP} B, {ceil_gu:.0f} GB/s at {BYTES_GATEUP} B")

    traffic = load_traffic()
    result = {
        "metric": "Q4_K/Q6_K GEMV HBM GB/s (% of peak); 7B-shape decode tokens/s, 1 MI355X",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k packed weights, fp32 activations and accumulation",
        "data": "synthetic (seeded random-init packed weights, x ~ N(0,1)); weights rotated over "
                f"{B} HBM-resident banks ({B * (2 * W_GATE + W_DOWN) / 1e9:.2f} GB)",
        "config": {
            "workload": "fused FFN block, Qwen2.5-7B shape: Q4_K gate+up [18944x3584] + SwiGLU, "
                        "Q6_K down [3584x18944] split-K 74 + fixed-order reduce",
            "hidden": H, "ffn": FFN, "splits": SPLITS, "algorithmic_bytes_per_step": BYTES_STEP,
            "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        },
        "roofline": {
            "kernel": "k_gemv<Q4_K, swiglu> (fused gate/up + SwiGLU)",
            "bound": "hbm",
            "achieved": round(ach, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4),
            "traffic": traffic.get("bytes_per_launch") if traffic else None,
            "avg_launch_us": round(ms_gu * 1e3, 3),
            "algorithmic_bytes_per_launch": BYTES_GATEUP,
        },
        "stream_ceiling": {
            "kernel": "arc_probe_read (coalesced 16 B/lane streaming read, same bank rotation)",
            "GB/s_at_step_bytes": round(ceil_step, 1),
            "GB/s_at_gateup_bytes": round(ceil_gu, 1),
            "value_frac_of_ceiling": round(gbs / ceil_step, 4),
            "roofline_frac_of_ceiling": round(ach / ceil_gu, 4),
        },
        "device": f"{name} {gfx}",
    }

    if args.components:
        comp = {}
        gate_ms = time_loop(lambda i: arc.gemv(arc.Q4_K, banks[i % B][0], FFN, H, x, s, stream=stream),
                            args.steps, stream)
        comp["q4k_gate_gemv"] = {"us": round(gate_ms * 1e3, 3), "GB/s": round(BYTES_GATE / (gate_ms / 1e3) / 1e9, 1)}
        banks.clear()
        arc.synchronize()
        lm_h = arc.synth_packed(arc.Q6_K, SEED, 5, VOC, H)
        lm = [arc.DeviceBuffer.from_array(lm_h)]
        for _ in range(1):
            c = arc.DeviceBuffer(W_LM)
            arc.check(arc.lib().arc_memcpy_dtod(c.ptr, lm[0].ptr, W_LM, stream.handle))
            lm.append(c)
        h = arc.DeviceBuffer.from_array(arc.synth_normal(SEED, 6, H))
        nw = arc.DeviceBuffer.from_array(arc.synth_normal(SEED, 7, H, 1.0, 0.05))
        ws = arc.DeviceBuffer(arc.lmhead_workspace_bytes(arc.Q6_K, VOC, H))
        out = arc.DeviceBuffer(8)
        lm_ms = time_loop(lambda i: arc.lmhead_argmax(arc.Q6_K, lm[i % 2], VOC, H, h, nw, 1e-6, None, ws, out,
                                                      stream), max(args.steps // 4, 10), stream)
        comp["q6k_lmhead_argmax"] = {"us": round(lm_ms * 1e3, 3),
                                     "GB/s": round(BYTES_LM / (lm_ms / 1e3) / 1e9, 1),
                                     "token": int(out.download(np.uint32)[0])}
        result["components"] = comp

    if not args.no_decode:
        banks.clear()
        for buf in (probe_out, x, s, part, y):
            buf.close()
        arc.synchronize()
        result["decode"] = decode_leg(args.decode_steps, 8, graph=not args.decode_eager)

    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(args.cpu_reps)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
