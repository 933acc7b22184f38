"""ctypes bindings of the CPU oracle (oracle/liboracle.so) and, where it was
built, of the reference's own code (oracle/_ref/libref.so).  Test
infrastructure only: the checker, never the thing measured or shipped."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libref.so")
REF_KAT = os.path.join(ORACLE_DIR, "_ref", "q4_down_exec148_synthetic")

Q4_K, Q6_K = 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}

_P = C.c_void_p
_U32 = C.c_uint32
_o = None
_r = None


class Top2(C.Structure):
    _fields_ = [("top1", C.c_uint32), ("top2", C.c_uint32), ("logit1", C.c_float), ("logit2", C.c_float),
                ("finite", C.c_int)]


ORC_MAX_LAYERS = 64
_PA = _P * ORC_MAX_LAYERS


class OrcModel(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("ffn", C.c_uint32), ("vocab", C.c_uint32), ("layers", C.c_uint32), ("eps", C.c_double),
                ("theta", C.c_double), ("emb", _P), ("out", _P), ("out_norm", _P),
                ("attn_norm", _PA), ("ffn_norm", _PA), ("q", _PA), ("k", _PA), ("v", _PA), ("o", _PA),
                ("qb", _PA), ("kb", _PA), ("vb", _PA), ("gate", _PA), ("up", _PA), ("down", _PA),
                ("v_type", C.c_int * ORC_MAX_LAYERS), ("down_type", C.c_int * ORC_MAX_LAYERS)]


def oracle() -> C.CDLL:
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"], check=True)
        L = C.CDLL(ORACLE_SO)
        sig = {
            "orc_half_to_float": ([C.c_uint16], C.c_float),
            "orc_float_to_half_rne": ([C.c_float], C.c_uint16),
            "orc_q4k_weight": ([_P, _U32], C.c_float),
            "orc_q6k_weight": ([_P, _U32], C.c_float),
            "orc_q4k_code": ([_P, _U32], C.c_uint32),
            "orc_q6k_code": ([_P, _U32, C.POINTER(C.c_int)], C.c_int),
            "orc_q4k_scale_min": ([_P, _U32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)], None),
            "orc_dequant": ([C.c_int, _P, _U32, _U32, _P], C.c_int),
            "orc_exec148_block": ([_P, _P], None),
            "orc_exec148_tensor": ([_P, _U32, _U32, _P], C.c_int),
            "orc_q4k_canon": ([_P, _P], None),
            "orc_exec148_canon": ([_P, _P], None),
            "orc_exec148_weight": ([_P, _U32], C.c_float),
            "orc_sha256": ([_P, C.c_size_t, _P], None),
            "orc_gemv_r0": ([C.c_int, _P, _U32, _U32, _P, _P, _P], C.c_int),
            "orc_gemv_r0_mt": ([C.c_int, _P, _U32, _U32, _P, _P, _P, C.c_int], C.c_int),
            "orc_gemv_r64": ([C.c_int, _P, _U32, _U32, _P, _P, _P], C.c_int),
            "orc_gemv_splitk_r64": ([C.c_int, _P, _U32, _U32, _U32, _P, _P], C.c_int),
            "orc_gemv_r64_xd": ([C.c_int, _P, _U32, _U32, _P, _P], C.c_int),
            "orc_gemv_r64_f16": ([C.c_int, _P, _U32, _U32, _P, _P], C.c_int),
            "orc_rmsnorm_f32": ([_P, _P, _U32, C.c_float, _P], None),
            "orc_rmsnorm_f64": ([_P, _P, _U32, C.c_double, _P], None),
            "orc_swiglu_f32": ([_P, _P, _U32, _P], None),
            "orc_swiglu_f64": ([_P, _P, _U32, _P], None),
            "orc_rope_f32": ([_P, _U32, _U32, _U32, C.c_float], None),
            "orc_rope_f64": ([_P, _U32, _U32, _U32, C.c_double], None),
            "orc_top2": ([_P, _U32, C.POINTER(Top2)], None),
            "orc_attention_decode_f64": ([_P, _P, _P, _U32, _U32, _U32, _U32, _P], None),
            "orc_decode_step": ([C.POINTER(OrcModel), _P, _P, _U32, _U32, _U32, _P], C.c_int),
            "orc_decode_step_ex": ([C.POINTER(OrcModel), _P, _P, _U32, _U32, _U32, C.c_int, _P], C.c_int),
            "orc_prompt_pass": ([C.POINTER(OrcModel), _P, _P, _U32, _U32, _U32, _P, C.c_int, _P], C.c_int),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _o = L
    return _o


def have_ref() -> bool:
    return os.path.exists(REF_SO)


def ref() -> C.CDLL:
    global _r
    if _r is None:
        L = C.CDLL(REF_SO)
        sig = {
            "ref_half_to_float": ([C.c_uint16], C.c_float),
            "ref_q6_decode_block": ([_P, _P, _P, _P], None),
            "ref_q6_fixture": ([_U32, _U32, C.c_uint64, C.c_int, _P, _P, _P, _P], C.c_int),
            "ref_q6_arms": ([_P, C.c_size_t, _U32, _U32, _P, _P, _P, _P], C.c_int),
            "ref_q4_source_tuple": ([_P, _P], None),
            "ref_exec148_materialize_block": ([_P, _P], None),
            "ref_sha256": ([_P, C.c_size_t, _P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _r = L
    return _r


def _p(a: np.ndarray):
    return a.ctypes.data


# ----------------------------------------------------------- conveniences
def dequant(qtype: int, w: np.ndarray, rows: int, K: int) -> np.ndarray:
    out = np.empty(rows * K, dtype=np.float32)
    assert oracle().orc_dequant(qtype, _p(w), rows, K, _p(out)) == 0
    return out.reshape(rows, K)


def exec148(w: np.ndarray, rows: int, K: int) -> np.ndarray:
    """EXEC148 image (148-byte blocks) of a packed Q4_K tensor."""
    out = np.empty(rows * (K // 256) * 148, dtype=np.uint8)
    assert oracle().orc_exec148_tensor(_p(w), rows, K, _p(out)) == 0
    return out


def sha256(data: np.ndarray) -> str:
    buf = np.ascontiguousarray(data, dtype=np.uint8).ravel()
    if buf.size == 0:
        buf = np.zeros(1, np.uint8)
        n = 0
    else:
        n = buf.size
    o = np.zeros(32, np.uint8)
    oracle().orc_sha256(_p(buf), n, _p(o))
    return bytes(o).hex()


def gemv_r64(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray, bias=None) -> np.ndarray:
    y = np.empty(rows, dtype=np.float64)
    assert oracle().orc_gemv_r64(qtype, _p(w), rows, K, _p(x), None if bias is None else _p(bias), _p(y)) == 0
    return y


def gemv_r64_xd(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(rows, dtype=np.float64)
    assert oracle().orc_gemv_r64_xd(qtype, _p(w), rows, K, _p(x), _p(y)) == 0
    return y


def gemv_r64_f16(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(rows, dtype=np.float64)
    assert oracle().orc_gemv_r64_f16(qtype, _p(w), rows, K, _p(x), _p(y)) == 0
    return y


def gemv_r0(qtype: int, w: np.ndarray, rows: int, K: int, x: np.ndarray, bias=None, threads: int = 0) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    b = None if bias is None else _p(bias)
    if threads > 0:
        assert oracle().orc_gemv_r0_mt(qtype, _p(w), rows, K, _p(x), b, _p(y), threads) == 0
    else:
        assert oracle().orc_gemv_r0(qtype, _p(w), rows, K, _p(x), b, _p(y)) == 0
    return y


def splitk_r64(qtype: int, w: np.ndarray, rows: int, K: int, splits: int, x: np.ndarray) -> np.ndarray:
    part = np.empty(splits * rows, dtype=np.float64)
    assert oracle().orc_gemv_splitk_r64(qtype, _p(w), rows, K, splits, _p(x), _p(part)) == 0
    return part.reshape(splits, rows)


def attention_decode_f64(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, T: int, q_heads: int, kv_heads: int,
                         dim: int = 128) -> np.ndarray:
    """fp64 cached GQA over positions 0..T-1; kc/vc fp16 [ctx][kv_heads*dim]."""
    q64 = np.ascontiguousarray(q, dtype=np.float64)
    kb = np.ascontiguousarray(kc).view(np.uint16)
    vb = np.ascontiguousarray(vc).view(np.uint16)
    out = np.empty(q_heads * dim, dtype=np.float64)
    oracle().orc_attention_decode_f64(_p(q64), _p(kb), _p(vb), T - 1, q_heads, kv_heads, dim, _p(out))
    return out


def rmsnorm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty_like(x64)
    oracle().orc_rmsnorm_f64(_p(x64), _p(w), len(x64), eps, _p(y))
    return y


def rmsnorm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    y = np.empty_like(x)
    oracle().orc_rmsnorm_f32(_p(x), _p(w), len(x), eps, _p(y))
    return y


def swiglu_f64(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float64)
    u = np.ascontiguousarray(u, dtype=np.float64)
    s = np.empty_like(g)
    oracle().orc_swiglu_f64(_p(g), _p(u), len(g), _p(s))
    return s


def top2(logits: np.ndarray) -> Top2:
    t = Top2()
    oracle().orc_top2(_p(logits), len(logits), C.byref(t))
    return t


def rel_err(y: np.ndarray, r: np.ndarray) -> float:
    """max_i |y_i - r_i| / max(|r_i|, tau), tau = 1e-3 * max|r| (documented floor)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    tau = 1e-3 * float(np.max(np.abs(r))) if r.size else 0.0
    den = np.maximum(np.abs(r), tau)
    den[den == 0] = 1.0
    return float(np.max(np.abs(y - r) / den)) if r.size else 0.0


class DecodeOracle:
    """The fp64 decode-step restatement over host copies of the model tensors
    (same slot order as arcllm_amd.model_slots) and its own fp16 KV cache."""

    # slot index within a layer -> OrcModel field
    _LAYER_FIELDS = {0: "attn_norm", 1: "q", 2: "k", 3: "v", 4: "qb", 5: "kb", 6: "vb", 7: "o", 8: "ffn_norm",
                     9: "gate", 10: "up", 11: "down"}

    def __init__(self, dims, tensors, max_ctx, f16_operands=False):
        m = OrcModel()
        for f in ("hidden", "q_heads", "kv_heads", "head_dim", "ffn", "vocab", "layers"):
            setattr(m, f, getattr(dims, f))
        m.eps, m.theta = float(dims.rms_eps), float(dims.rope_theta)
        m.emb, m.out, m.out_norm = tensors[0].ctypes.data, tensors[1].ctypes.data, tensors[2].ctypes.data
        for layer in range(dims.layers):
            for w, field in self._LAYER_FIELDS.items():
                getattr(m, field)[layer] = tensors[3 + 12 * layer + w].ctypes.data
            m.v_type[layer] = dims.v_type[layer]
            m.down_type[layer] = dims.down_type[layer]
        self.m, self.dims, self.tensors, self.max_ctx = m, dims, tensors, max_ctx
        self.f16 = 1 if f16_operands else 0
        kvd = dims.kv_heads * dims.head_dim
        self.kc = np.zeros(dims.layers * max_ctx * kvd, np.uint16)
        self.vc = np.zeros_like(self.kc)

    def fill_kv(self, ctx, seed, synth_normal):
        """Same contents as arc_session_fill_kv: fp16(N(0,1)) per layer and K/V stream."""
        kvd = self.dims.kv_heads * self.dims.head_dim
        for layer in range(self.dims.layers):
            for kv, cache in ((0, self.kc), (1, self.vc)):
                vals = synth_normal(seed, 1000000 + 2 * layer + kv, ctx * kvd).astype(np.float16).view(np.uint16)
                base = layer * self.max_ctx * kvd
                cache[base:base + ctx * kvd] = vals

    def step(self, token, pos):
        logits = np.empty(self.dims.vocab, np.float64)
        rc = oracle().orc_decode_step_ex(C.byref(self.m), _p(self.kc), _p(self.vc), self.max_ctx, pos, token,
                                         self.f16, _p(logits))
        assert rc == 0
        return logits

    def prompt(self, tokens, pos0=0):
        """tokens[i] at position pos0 + i (teacher forcing), all positions
        layer by layer (bit-identical to stepping); logits of the last one."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.dims.vocab, np.float64)
        rc = oracle().orc_prompt_pass(C.byref(self.m), _p(self.kc), _p(self.vc), self.max_ctx, pos0, len(toks),
                                      _p(toks), self.f16, _p(logits))
        assert rc == 0
        return logits

    def follow(self, token, pos, gpu_tokens, tie=2e-3):
        """Teacher-forced check of a GPU greedy run, every step compared: step
        i feeds `token` (i = 0) or the GPU's token i - 1 at position pos + i,
        and the GPU's token i must be the oracle's argmax, or its runner-up
        when the top-2 margin is below tie * max|logit| (a near tie, where
        fp32 and fp64 may order the two differently).  Returns the number of
        near-tie steps the GPU took the runner-up at."""
        ties = 0
        for i, g in enumerate(np.asarray(gpu_tokens).tolist()):
            lg = self.step(int(token), pos + i)
            order = np.argsort(-lg, kind="stable")
            if g != int(order[0]):
                margin, scale = float(lg[order[0]] - lg[order[1]]), float(np.max(np.abs(lg)))
                assert g == int(order[1]) and margin < tie * scale, (
                    f"step {i}: gpu token {g}, oracle {int(order[0])} / {int(order[1])}, margin {margin:.4g} "
                    f"(near-tie bound {tie * scale:.4g})")
                ties += 1
            token = g
        return ties

    def greedy(self, token, pos, n, log=None):
        """n greedy steps from `token` at `pos`.  Returns (tokens, runner-up
        tokens, top1-top2 margins, max|logit| per step); `log` gets one line
        per step."""
        toks, second, margins, scale = [], [], [], []
        for i in range(n):
            lg = self.step(token, pos + i)
            order = np.argsort(-lg, kind="stable")
            token = int(order[0])
            toks.append(token)
            second.append(int(order[1]))
            margins.append(float(lg[order[0]] - lg[order[1]]))
            scale.append(float(np.max(np.abs(lg))))
            if log is not None:
                log(f"oracle step {i + 1}/{n} pos={pos + i} token={token} margin={margins[-1]:.4g}")
        return np.array(toks, np.uint32), np.array(second, np.uint32), np.array(margins), np.array(scale)
