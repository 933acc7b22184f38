"""Standalone parity of the decode attention kernel and of the prompt pass's
MFMA projection GEMMs against the fp64 oracle, per element at the GEMV bar
(|gpu - ref| <= 1e-3 * max(|ref|, 1e-3 * max|ref|)).

Attention (arc_attention_decode: the decode step's kernel and split plan):
oracle orc_attention_decode_f64, the restatement of
src/arcllm_v1_i001r_p8c_profile_runtime.cpp:1177-1212
(shaders/p7_attention_kv_online.comp), over the same fp16 caches, at
context lengths on both sides of every chunk and split boundary, 7 query
heads per kv head (the 7B shape).

Prompt-pass attention (arc_prefill_attention: the MFMA kernel the pass runs
and the VALU one), row by row against the same fp64 attention over positions
0 .. pos0 + m.

Prompt pass (arc_prefill_gemm / arc_prefill_gateup / arc_prefill_qkv: the
run_prefill kernels, split plans and fixed-order split reductions):
oracle orc_gemv_r64_f16 (each decoded weight and each input element rounded
to binary16, exact products, fp64 sum: the contract of the MFMA prompt pass,
whose reference is the fp32 build_prefill, src/arcllm_v1_runtime.cpp:340-369),
on every projection shape of the 7B model with M = 2, 37 and 256 prompt
rows (for M = 256 a spread of rows covering the 32-row block boundaries).
"""
import numpy as np
import pytest

import arcllm_amd as arc
import oracle_lib as orc

pytestmark = pytest.mark.gpu

SEED = 0xA77E_2026
TOL = 1e-3
H, KVH, HPK, FFN = 3584, 4, 7, 18944
KVD = KVH * 128


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert arc.device_count() >= 1, "no HIP device visible"


def dev(a):
    return arc.DeviceBuffer.from_array(np.ascontiguousarray(a))


# ------------------------------------------------------------- attention
@pytest.fixture(scope="module")
def kv_cache():
    max_ctx = 4160
    kc = arc.synth_normal(SEED, 1, max_ctx * KVD).astype(np.float16)
    vc = arc.synth_normal(SEED, 2, max_ctx * KVD).astype(np.float16)
    return max_ctx, kc, vc, dev(kc), dev(vc)


@pytest.mark.parametrize("qscale", [1.0, 4.0])
@pytest.mark.parametrize("T", [1, 63, 64, 65, 448, 449, 512, 1023, 1024, 1025, 2048, 4095, 4096, 4097])
def test_attention_decode_vs_fp64(kv_cache, T, qscale):
    """Every output element of the 28 query heads within 1e-3 of the fp64
    softmax attention (qscale 4 makes the softmax peaked, so the running
    maximum and the split merge's rescaling carry the result)."""
    max_ctx, kc, vc, dkc, dvc = kv_cache
    q = (arc.synth_normal(SEED, 10 + T, KVH * HPK * 128) * qscale).astype(np.float32)
    out = arc.DeviceBuffer(q.nbytes)
    ws = arc.DeviceBuffer(arc.attention_workspace_bytes(KVH, HPK))
    arc.attention_decode(dev(q), dkc, dvc, KVH, HPK, max_ctx, T, out, ws)
    got = out.download(np.float32)
    ref = orc.attention_decode_f64(q, kc, vc, T, KVH * HPK, KVH)
    err = orc.rel_err(got, ref)
    print(f"T={T} qscale={qscale}: per-element error {err:.3g}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("waves,min_cps", [(8, 1), (4, 2), (8, 3)])
@pytest.mark.parametrize("T", [1, 127, 128, 129, 511, 512, 513, 2048, 4096, 4097])
def test_attention_decode_launch_shapes_vs_fp64(kv_cache, T, waves, min_cps):
    """The tuning launch shapes: 8 waves (128-position chunks) and several
    chunks per split, against the fp64 attention (qscale 4)."""
    max_ctx, kc, vc, dkc, dvc = kv_cache
    q = (arc.synth_normal(SEED, 20 + T, KVH * HPK * 128) * 4.0).astype(np.float32)
    out = arc.DeviceBuffer(q.nbytes)
    ws = arc.DeviceBuffer(arc.attention_workspace_bytes(KVH, HPK))
    arc.tune_attention(waves, min_cps)
    try:
        arc.attention_decode(dev(q), dkc, dvc, KVH, HPK, max_ctx, T, out, ws)
    finally:
        arc.tune_attention(0, 0)
    err = orc.rel_err(out.download(np.float32), orc.attention_decode_f64(q, kc, vc, T, KVH * HPK, KVH))
    print(f"T={T} waves={waves} min_cps={min_cps}: per-element error {err:.3g}", flush=True)
    assert err <= TOL


def test_attention_tuning_rejects_bad_shapes():
    for waves, cps in ((16, 0), (3, 0), (0, -1)):
        with pytest.raises(arc.ArcError):
            arc.tune_attention(waves, cps)


def test_attention_decode_repeatable_and_rejects_bad_context(kv_cache):
    """Two calls give identical outputs (fixed reduction order, counters
    reset by the call); T = 0 and T > max_ctx are refused."""
    max_ctx, kc, vc, dkc, dvc = kv_cache
    q = arc.synth_normal(SEED, 99, KVH * HPK * 128)
    out1, out2 = arc.DeviceBuffer(q.nbytes), arc.DeviceBuffer(q.nbytes)
    ws = arc.DeviceBuffer(arc.attention_workspace_bytes(KVH, HPK))
    arc.attention_decode(dev(q), dkc, dvc, KVH, HPK, max_ctx, 3000, out1, ws)
    arc.attention_decode(dev(q), dkc, dvc, KVH, HPK, max_ctx, 3000, out2, ws)
    assert np.array_equal(out1.download(np.float32), out2.download(np.float32))
    for T in (0, max_ctx + 1):
        with pytest.raises(arc.ArcError):
            arc.attention_decode(dev(q), dkc, dvc, KVH, HPK, max_ctx, T, out1, ws)


# ---------------------------------------------------- prompt-pass GEMMs
def check_rows(M):
    """Rows compared against the oracle: all of a short prompt, and for the
    full 256 rows both sides of each 32-row block boundary and the ends."""
    if M <= 40:
        return list(range(M))
    return [0, 1, 31, 32, 63, 64, 127, 128, 200, 254, 255]


def packed_pair(qtype, rows, K, stream):
    """(bytes the oracle reads, device tensor the GPU reads): Q6_K is held
    padded on the device, as the model arena holds it."""
    w = arc.synth_packed(arc.Q6_K if qtype == arc.Q6_K_PADDED else qtype, SEED, stream, rows, K)
    d = dev(w)
    if qtype != arc.Q6_K_PADDED:
        return w, d, qtype
    p = arc.DeviceBuffer(rows * (K // 256) * 212)
    arc.q6_pad(d, rows, K, p)
    return w, p, arc.Q6_K


def x16(M, K, stream, scale=1.0):
    return (arc.synth_normal(SEED, stream, M * K) * scale).astype(np.float16).reshape(M, K)


SHAPES = [  # name, qtype, N, K
    ("attn_q", arc.Q4_K, H, H),
    ("attn_o", arc.Q4_K, H, H),
    ("attn_k", arc.Q4_K, KVD, H),
    ("attn_v Q6_K", arc.Q6_K_PADDED, KVD, H),
    ("ffn_down Q6_K", arc.Q6_K_PADDED, H, FFN),
    ("ffn_down Q4_K", arc.Q4_K, H, FFN),
]


@pytest.mark.parametrize("M", [2, 37, 256])
@pytest.mark.parametrize("name,qtype,N,K", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_gemm_vs_fp16_operand_oracle(name, qtype, N, K, M):
    w, dw, oq = packed_pair(qtype, N, K, 20 + N % 97 + K % 89)
    x = x16(M, K, 30 + M)
    y = arc.DeviceBuffer(M * N * 4)
    ws = arc.DeviceBuffer(arc.prefill_gemm_workspace_bytes(N, K))
    arc.prefill_gemm(qtype, dw, N, K, dev(x.view(np.uint16)), M, y, ws)
    got = y.download(np.float32).reshape(M, N)
    worst = 0.0
    for m in check_rows(M):
        ref = orc.gemv_r64_f16(oq, w, N, K, x[m].astype(np.float64))
        worst = max(worst, orc.rel_err(got[m], ref))
    print(f"{name} M={M}: per-element error {worst:.3g}", flush=True)
    assert worst <= TOL


@pytest.mark.parametrize("M", [2, 37, 256])
def test_prefill_gateup_swiglu_vs_fp16_operand_oracle(M):
    wg, dg, _ = packed_pair(arc.Q4_K, FFN, H, 41)
    wu, du, _ = packed_pair(arc.Q4_K, FFN, H, 42)
    # inputs scaled so silu(g) * u stays inside fp16's range with these
    # O(1)-magnitude test weights (the output is fp16)
    x = x16(M, H, 50 + M, 0.05)
    s = arc.DeviceBuffer(M * FFN * 2)
    ws = arc.DeviceBuffer(arc.prefill_gemm_workspace_bytes(FFN, H))
    arc.prefill_gateup(dg, du, FFN, H, dev(x.view(np.uint16)), M, s, ws)
    got = s.download(np.uint16).view(np.float16).reshape(M, FFN).astype(np.float64)
    worst = 0.0
    for m in check_rows(M):
        xm = x[m].astype(np.float64)
        ref = orc.swiglu_f64(orc.gemv_r64_f16(arc.Q4_K, wg, FFN, H, xm), orc.gemv_r64_f16(arc.Q4_K, wu, FFN, H, xm))
        worst = max(worst, orc.rel_err(got[m], ref))
    # the output is fp16: its rounding (<= 2^-11 relative) is inside the bar
    print(f"gate/up+SwiGLU M={M}: per-element error {worst:.3g}", flush=True)
    assert worst <= TOL


@pytest.mark.parametrize("vtype", [arc.Q6_K_PADDED, arc.Q4_K])
@pytest.mark.parametrize("M", [2, 37, 256])
def test_prefill_qkv_vs_fp16_operand_oracle(vtype, M):
    wq, dq, _ = packed_pair(arc.Q4_K, H, H, 61)
    wk, dk, _ = packed_pair(arc.Q4_K, KVD, H, 62)
    wv, dv, ov = packed_pair(vtype, KVD, H, 63)
    x = x16(M, H, 70 + M)
    N = H + 2 * KVD
    y = arc.DeviceBuffer(M * N * 4)
    ws = arc.DeviceBuffer(arc.prefill_gemm_workspace_bytes(N, H))
    arc.prefill_qkv(dq, dk, dv, vtype, H, KVD, H, dev(x.view(np.uint16)), M, y, ws)
    got = y.download(np.float32).reshape(M, N)
    worst = 0.0
    for m in check_rows(M):
        xm = x[m].astype(np.float64)
        for lo, (qt, w, rows) in ((0, (arc.Q4_K, wq, H)), (H, (arc.Q4_K, wk, KVD)), (H + KVD, (ov, wv, KVD))):
            ref = orc.gemv_r64_f16(qt, w, rows, H, xm)
            worst = max(worst, orc.rel_err(got[m, lo:lo + rows], ref))
    print(f"q|k|v (v qtype {vtype}) M={M}: per-element error {worst:.3g}", flush=True)
    assert worst <= TOL


def test_prefill_gemm_rejects_bad_arguments():
    w = arc.DeviceBuffer(512 * 14 * 144)
    x = arc.DeviceBuffer(300 * H * 2)
    y = arc.DeviceBuffer(300 * 512 * 4)
    ws = arc.DeviceBuffer(arc.prefill_gemm_workspace_bytes(512, H))
    with pytest.raises(arc.ArcError):
        arc.prefill_gemm(arc.Q4_K, w, 512, H, x, 257, y, ws)  # more than 256 rows
    with pytest.raises(arc.ArcError):
        arc.prefill_gemm(arc.Q6_K, w, 512, H, x, 4, y, ws)  # GGUF Q6_K: the prompt pass reads it padded
    with pytest.raises(arc.ArcError):
        arc.prefill_gemm(arc.Q4_K, w, 512, 1000, x, 4, y, ws)  # K not a multiple of 256


# ------------------------------------------------ prompt-pass attention
@pytest.mark.parametrize("mfma", [True, False])
@pytest.mark.parametrize("pos0,M,qscale", [(0, 37, 1.0), (0, 256, 1.0), (0, 256, 4.0), (256, 44, 1.0),
                                            (1000, 64, 4.0), (3900, 256, 1.0)])
def test_prefill_attention_vs_fp64(kv_cache, mfma, pos0, M, qscale):
    """The prompt pass's causal GQA (7 q heads per kv head), MFMA and VALU
    kernels: prompt row m at position pos0 + m against the fp64 attention
    over positions 0 .. pos0 + m (the decode oracle), per element within
    1e-3, on rows covering the 32-row query blocks' edges and, with pos0 >
    0, the offset passes of long prompts.  The output is fp16: its rounding
    (<= 2^-11 relative) is inside the bar."""
    max_ctx, kc, vc, dkc, dvc = kv_cache
    hidden = KVH * HPK * 128
    q = (arc.synth_normal(SEED, 300 + pos0 + M, M * hidden) * qscale).astype(np.float32)
    x = arc.DeviceBuffer(M * hidden * 2)
    arc.prefill_attention(dev(q), dkc, dvc, KVH, HPK, max_ctx, pos0, M, x, hidden, mfma=mfma)
    got = x.download(np.uint16, M * hidden).view(np.float16).astype(np.float64).reshape(M, hidden)
    worst = 0.0
    for m in [r for r in check_rows(M) if r < M] + [M - 1]:
        ref = orc.attention_decode_f64(q[m * hidden:(m + 1) * hidden], kc, vc, pos0 + m + 1, KVH * HPK, KVH)
        worst = max(worst, orc.rel_err(got[m], ref))
    print(f"prefill attention mfma={mfma} pos0={pos0} M={M} qscale={qscale}: per-element error {worst:.3g}",
          flush=True)
    assert worst <= TOL


def test_prefill_attention_rejects_bad_arguments(kv_cache):
    max_ctx, kc, vc, dkc, dvc = kv_cache
    hidden = KVH * HPK * 128
    q = arc.DeviceBuffer(4 * hidden * 4)
    x = arc.DeviceBuffer(4 * hidden * 2)
    with pytest.raises(arc.ArcError):
        arc.prefill_attention(q, dkc, dvc, KVH, HPK, max_ctx, max_ctx - 2, 4, x, hidden)  # rows past the cache
    with pytest.raises(arc.ArcError):
        arc.prefill_attention(q, dkc, dvc, KVH, 9, max_ctx, 0, 4, x, hidden)  # 9 q heads per kv head
    with pytest.raises(arc.ArcError):
        arc.prefill_attention(q, dkc, dvc, KVH, HPK, max_ctx, 0, 4, x, hidden - 8)  # ldx below the row
