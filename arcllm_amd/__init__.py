"""arcllm_amd -- MI355X-native (gfx950) backend for ArcLLM's packed Q4_K/Q6_K
decode hot path.

The product is the C-ABI shared library ``libarcllm_hip.so`` (declared in
``include/arcllm_hip.h``; hand-written HIP kernels in ``csrc/``).  This module
is the Python host mirror over that ABI, via ctypes: device buffers, streams,
events, the kernel entry points, and the greedy ``generate`` runtime.  It
never falls back to a CPU path: every call goes to the library, and loading
fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libarcllm_hip.so")

Q4_K = 12
Q6_K = 14
EXEC148 = 148  # Q4_K repacked as EXEC148 blocks (arc_gemv / arc_gemv_splitk only)
Q6_K_PADDED = 214  # Q6_K blocks padded to 212 bytes (arc_q6_pad)
QK = 256
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q6_K_PADDED: 212}

ARC_OK = 0
_STATUS = {
    1: "INVALID_ARGUMENT",
    2: "UNSUPPORTED",
    3: "DEVICE",
    4: "OUT_OF_MEMORY",
    5: "NO_DEVICE",
}


class ArcError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero arc_status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"arc_status {code} ({_STATUS.get(code, '?')}): {msg}")
        self.code = code


_lib: Optional[C.CDLL] = None

_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float
_FP = C.POINTER(C.c_float)

# name -> argtypes (restype int unless listed in _RESTYPE)
_SIGS = {
    "arc_last_error": [],
    "arc_version": [],
    "arc_device_count": [C.POINTER(C.c_int)],
    "arc_set_device": [C.c_int],
    "arc_device_info": [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t],
    "arc_malloc": [C.POINTER(_P), C.c_size_t],
    "arc_free": [_P],
    "arc_device_allocations": [C.POINTER(_U64)],
    "arc_memcpy_htod": [_P, _P, C.c_size_t, _P],
    "arc_memcpy_dtoh": [_P, _P, C.c_size_t, _P],
    "arc_memcpy_dtod": [_P, _P, C.c_size_t, _P],
    "arc_memset": [_P, C.c_int, C.c_size_t, _P],
    "arc_synchronize": [],
    "arc_stream_create": [C.POINTER(_P)],
    "arc_stream_destroy": [_P],
    "arc_stream_synchronize": [_P],
    "arc_event_create": [C.POINTER(_P)],
    "arc_event_destroy": [_P],
    "arc_event_record": [_P, _P],
    "arc_event_elapsed_ms": [_P, _P, _FP],
    "arc_dequant": [C.c_int, _P, _U32, _U32, _P, _P],
    "arc_q6_pad": [_P, _U32, _U32, _P, _P],
    "arc_gemv": [C.c_int, _P, _U32, _U32, _P, _P, _P, _P],
    "arc_gateup_swiglu": [C.c_int, _P, _P, _U32, _U32, _P, _P, _P],
    "arc_gemv_splitk": [C.c_int, _P, _U32, _U32, _U32, _P, _P, _P, _P, _P],
    "arc_rmsnorm": [_P, _P, _U32, _F, _P, _P],
    "arc_lmhead_workspace_bytes": [C.c_int, _U32, _U32],
    "arc_lmhead_argmax": [C.c_int, _P, _U32, _U32, _P, _P, _F, _P, _P, _P, _P],
    "arc_lmhead_argmax_noalloc": [C.c_int, _P, _U32, _U32, _P, _P, _F, _P, _P, _P],
    "arc_synth_packed": [C.c_int, _U64, _U64, _U32, _U32, _F, _F, _P],
    "arc_synth_normal": [_U64, _U64, C.c_size_t, _F, _F, _P],
    "arc_tune_force": [C.c_int, C.c_int],
    "arc_tune_waves": [C.c_int],
    "arc_tune_rowstream": [C.c_int],
    "arc_tune_attention": [C.c_int, C.c_int],
    "arc_tune_decode": [C.c_int, C.c_int, C.c_int, C.c_int],
    "arc_tune_fuse_attn_o": [C.c_int],
    "arc_tune_prefill_attention": [C.c_int],
    "arc_probe_read": [_P, C.c_size_t, _P, _U32, _P],
    "arc_probe_read_unrolled": [_P, C.c_size_t, _P, _U32, C.c_int, _P],
    "arc_probe_read_nt": [_P, C.c_size_t, _P, _U32, _P],
    "arc_exec148_materialize": [_P, _U32, _U32, _P, _P],
    "arc_exec148_validate": [_P, _P, _U32, _U32, C.POINTER(_U64), _P],
    "arc_exec148_validate_many": [C.POINTER(_P), C.POINTER(_P), _U32, _U32, _U32, C.POINTER(_U64), _P],
    "arc_attention_workspace_bytes": [_U32, _U32],
    "arc_attention_decode": [_P, _P, _P, _U32, _U32, _U32, _U32, _P, _P, _P],
    "arc_prefill_gemm_workspace_bytes": [_U32, _U32],
    "arc_prefill_gemm": [C.c_int, _P, _U32, _U32, _P, _U32, _P, _P, _P],
    "arc_prefill_gateup": [_P, _P, _U32, _U32, _P, _U32, _P, _P, _P],
    "arc_prefill_qkv": [_P, _P, _P, C.c_int, _U32, _U32, _U32, _P, _U32, _P, _P, _P],
    "arc_prefill_attention": [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _U32, C.c_int, _P],
}
_RESTYPE = {
    "arc_last_error": C.c_char_p,
    "arc_version": C.c_char_p,
    "arc_lmhead_workspace_bytes": C.c_size_t,
    "arc_attention_workspace_bytes": C.c_size_t,
    "arc_prefill_gemm_workspace_bytes": C.c_size_t,
}
MAX_LAYERS = 64
T_TOKEN_EMBD, T_OUTPUT, T_OUTPUT_NORM, T_GLOBAL_COUNT = 0, 1, 2, 3
(T_ATTN_NORM, T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_Q_BIAS, T_ATTN_K_BIAS, T_ATTN_V_BIAS, T_ATTN_O,
 T_FFN_NORM, T_FFN_GATE, T_FFN_UP, T_FFN_DOWN, T_LAYER_COUNT) = range(13)
DECODE_LOGITS, DECODE_NO_GRAPH, PREFILL_STEPWISE = 1, 2, 4


class ModelDims(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("q_heads", C.c_uint32), ("kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32), ("layers", C.c_uint32),
                ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("v_type", C.c_int32 * MAX_LAYERS), ("down_type", C.c_int32 * MAX_LAYERS)]


class Residency(C.Structure):
    _fields_ = [("weight_bytes", _U64), ("model_arena_bytes", _U64), ("exec148_reserve_bytes", _U64),
                ("kv_bytes", _U64), ("working_bytes", _U64), ("total_bytes", _U64)]


_SIGS.update({
    "arc_model_dims_qwen25_7b": [C.POINTER(ModelDims)],
    "arc_model_tensor_info": [C.POINTER(ModelDims), C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(_U32),
                              C.POINTER(_U32), C.POINTER(_U64)],
    "arc_model_synth_tensor": [C.POINTER(ModelDims), _U64, C.c_int, C.c_int, _P],
    "arc_model_create": [C.POINTER(ModelDims), C.POINTER(_P), C.POINTER(_P)],
    "arc_model_create_synthetic": [C.POINTER(ModelDims), _U64, C.POINTER(_P)],
    "arc_model_destroy": [_P],
    "arc_model_weight_bytes": [_P],
    "arc_model_exec148_reserve": [_P, C.POINTER(_P), C.POINTER(_U64), C.POINTER(_U32)],
    "arc_session_create": [_P, _U32, C.POINTER(_P)],
    "arc_session_residency": [_P, C.POINTER(Residency)],
    "arc_session_destroy": [_P],
    "arc_session_kv": [_P, _U32, C.POINTER(_P), C.POINTER(_P)],
    "arc_session_fill_kv": [_P, _U32, _U64],
    "arc_session_decode": [_P, _U32, _U32, _U32, C.c_int, _P, C.POINTER(_U32)],
    "arc_session_prefill": [_P, _P, _U32, _U32, C.c_int, C.POINTER(_U32), C.POINTER(_U32)],
    "arc_session_logits": [_P, _P],
    "arc_session_kernels_per_step": [_P],
    "arc_session_prefill_kernels": [_P],
    "arc_model_tensor_device": [_P, C.c_int, C.c_int, C.POINTER(_P)],
    "arc_session_route_down": [_P, _U32, _P],
})
_RESTYPE.update({"arc_model_weight_bytes": _U64, "arc_session_kernels_per_step": _U32,
                 "arc_session_prefill_kernels": _U32})

# Entry points declared in include/*.h that the tests check for.
EXPORTED = sorted(_SIGS)


def lib() -> C.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ArcError(2, f"{LIB_PATH} not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, C.c_int)
        _lib = L
    return _lib


RUNTIME_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libarcllm_runtime.so")
CLI_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "arcllm_runtime")
Q4_PATHS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "arcllm_q4_paths")
_rt = None


def runtime_lib() -> C.CDLL:
    """The host runtime library (GGUF reader, generate); raises if not built."""
    global _rt
    if _rt is None:
        if not os.path.exists(RUNTIME_LIB_PATH):
            raise ArcError(2, f"{RUNTIME_LIB_PATH} not built (run __graft_entry__.build())")
        L = C.CDLL(RUNTIME_LIB_PATH)
        L.arcllm_gguf_describe.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        L.arcllm_gguf_describe.restype = C.c_int
        _rt = L
    return _rt


def gguf_describe(path: str) -> dict:
    """JSON description of a GGUF file after the runtime's container checks;
    raises ArcError with the reader's message when the file is rejected."""
    import json

    cap = 1 << 20
    while True:
        buf = C.create_string_buffer(cap)
        rc = runtime_lib().arcllm_gguf_describe(path.encode(), buf, cap)
        if rc == 2:
            cap *= 4
            continue
        text = buf.value.decode(errors="replace")
        if rc != 0:
            raise ArcError(1, text)
        return json.loads(text)


def check(rc: int) -> None:
    if rc != ARC_OK:
        raise ArcError(rc, lib().arc_last_error().decode(errors="replace"))


def device_count() -> int:
    n = C.c_int(0)
    check(lib().arc_device_count(C.byref(n)))
    return n.value


def device_info() -> tuple[str, str]:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(256)
    check(lib().arc_device_info(name, 256, arch, 256))
    return name.value.decode(), arch.value.decode()


def synchronize() -> None:
    check(lib().arc_synchronize())


class DeviceBuffer:
    """Device memory from arc_malloc, freed on close()/garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _P()
        check(lib().arc_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray, stream: Optional["Stream"] = None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a, stream)
        return b

    def upload(self, a: np.ndarray, stream: Optional["Stream"] = None) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than device buffer")
        check(lib().arc_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes, _sp(stream)))
        if stream is None:
            synchronize()

    def download(self, dtype, count: Optional[int] = None, stream: Optional["Stream"] = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        check(lib().arc_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes, _sp(stream)))
        return out

    def zero(self, stream: Optional["Stream"] = None) -> None:
        check(lib().arc_memset(self.ptr, 0, self.nbytes, _sp(stream)))

    def close(self) -> None:
        if getattr(self, "ptr", None):
            if _lib is not None:
                _lib.arc_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _P()
        check(lib().arc_stream_create(C.byref(p)))
        self.handle = p.value

    def synchronize(self) -> None:
        check(lib().arc_stream_synchronize(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            if _lib is not None:
                _lib.arc_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _P()
        check(lib().arc_event_create(C.byref(p)))
        self.handle = p.value

    def record(self, stream: Optional[Stream] = None) -> None:
        check(lib().arc_event_record(self.handle, _sp(stream)))

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float(0.0)
        check(lib().arc_event_elapsed_ms(self.handle, later.handle, C.byref(ms)))
        return ms.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            if _lib is not None:
                _lib.arc_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _sp(stream: Optional[Stream]):
    return None if stream is None else stream.handle


def _ptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


# ------------------------------------------------------------ kernel calls
def dequant(qtype: int, w, rows: int, K: int, out, stream: Optional[Stream] = None) -> None:
    check(lib().arc_dequant(qtype, _ptr(w), rows, K, _ptr(out), _sp(stream)))


def q6_pad(w, rows: int, K: int, padded, stream: Optional[Stream] = None) -> None:
    """Write the padded (212-byte block, Q6_K_PADDED) image of a Q6_K tensor."""
    check(lib().arc_q6_pad(_ptr(w), rows, K, _ptr(padded), _sp(stream)))


def gemv(qtype: int, w, rows: int, K: int, x, y, bias=None, stream: Optional[Stream] = None) -> None:
    check(lib().arc_gemv(qtype, _ptr(w), rows, K, _ptr(x), _ptr(bias), _ptr(y), _sp(stream)))


def gateup_swiglu(qtype: int, w_gate, w_up, rows: int, K: int, x, s, stream: Optional[Stream] = None) -> None:
    check(lib().arc_gateup_swiglu(qtype, _ptr(w_gate), _ptr(w_up), rows, K, _ptr(x), _ptr(s), _sp(stream)))


def gemv_splitk(qtype: int, w, rows: int, K: int, splits: int, x, partials, y, residual=None,
                stream: Optional[Stream] = None) -> None:
    check(lib().arc_gemv_splitk(qtype, _ptr(w), rows, K, splits, _ptr(x), _ptr(partials), _ptr(residual),
                                _ptr(y), _sp(stream)))


def exec148_materialize(q4, rows: int, K: int, exec148, stream: Optional[Stream] = None) -> None:
    """EXEC148 image of a device Q4_K tensor into `exec148` (rows*(K/256)*148 bytes)."""
    check(lib().arc_exec148_materialize(_ptr(q4), rows, K, _ptr(exec148), _sp(stream)))


def exec148_validate(q4, exec148, rows: int, K: int, stream: Optional[Stream] = None) -> int:
    """Number of EXEC148 blocks that differ from the repack of their source (0 = exact)."""
    n = C.c_uint64(0)
    check(lib().arc_exec148_validate(_ptr(q4), _ptr(exec148), rows, K, C.byref(n), _sp(stream)))
    return int(n.value)


def exec148_validate_many(q4s, execs, rows: int, K: int, stream: Optional[Stream] = None) -> int:
    """Mismatched EXEC148 blocks summed over the pairs (q4s[i], execs[i]) of one shape."""
    if len(q4s) != len(execs):
        raise ValueError("q4s and execs differ in length")
    a = (C.c_void_p * len(q4s))(*[_ptr(x) for x in q4s])
    b = (C.c_void_p * len(execs))(*[_ptr(x) for x in execs])
    n = C.c_uint64(0)
    check(lib().arc_exec148_validate_many(a, b, len(q4s), rows, K, C.byref(n), _sp(stream)))
    return int(n.value)


def rmsnorm(x, w, n: int, eps: float, y, stream: Optional[Stream] = None) -> None:
    check(lib().arc_rmsnorm(_ptr(x), _ptr(w), n, eps, _ptr(y), _sp(stream)))


def lmhead_workspace_bytes(qtype: int, rows: int, K: int) -> int:
    n = int(lib().arc_lmhead_workspace_bytes(qtype, rows, K))
    if n == 0:
        raise ArcError(2, f"no LM-head workspace size for qtype {qtype}, {rows} x {K}")
    return n


def lmhead_argmax(qtype: int, w, rows: int, K: int, h, normw, eps: float, logits, workspace, out,
                  stream: Optional[Stream] = None) -> None:
    check(lib().arc_lmhead_argmax(qtype, _ptr(w), rows, K, _ptr(h), _ptr(normw), eps, _ptr(logits),
                                  _ptr(workspace), _ptr(out), _sp(stream)))


def lmhead_argmax_noalloc(qtype: int, w, rows: int, K: int, h, normw, eps: float, logits, out,
                          stream: Optional[Stream] = None) -> None:
    """arc_lmhead_argmax with its argmax partials in the library's static
    device scratch (no workspace, no allocation)."""
    check(lib().arc_lmhead_argmax_noalloc(qtype, _ptr(w), rows, K, _ptr(h), _ptr(normw), eps, _ptr(logits),
                                          _ptr(out), _sp(stream)))


def probe_read(buf, nbytes: int, out, grid: int = 2048, stream: Optional[Stream] = None) -> None:
    """Streaming-read probe (practical HBM read ceiling); `out` holds grid*256 uint32."""
    check(lib().arc_probe_read(_ptr(buf), nbytes, _ptr(out), grid, _sp(stream)))


def probe_read_unrolled(buf, nbytes: int, out, grid: int = 2048, loads: int = 4,
                        stream: Optional[Stream] = None) -> None:
    """The streaming-read probe with `loads` independent 16-byte loads per lane in flight."""
    check(lib().arc_probe_read_unrolled(_ptr(buf), nbytes, _ptr(out), grid, loads, _sp(stream)))


def probe_read_nt(buf, nbytes: int, out, grid: int = 2048, stream: Optional[Stream] = None) -> None:
    """The one-load streaming-read probe with non-temporal loads."""
    check(lib().arc_probe_read_nt(_ptr(buf), nbytes, _ptr(out), grid, _sp(stream)))


def attention_workspace_bytes(kv_heads: int, hpk: int) -> int:
    n = int(lib().arc_attention_workspace_bytes(kv_heads, hpk))
    if n == 0:
        raise ArcError(2, f"no attention workspace size for {kv_heads} kv heads, {hpk} query heads each")
    return n


def attention_decode(q, kc, vc, kv_heads: int, hpk: int, max_ctx: int, T: int, out, workspace,
                     stream: Optional[Stream] = None) -> None:
    """The decode step's cached GQA over positions 0..T-1 (fp32 q/out, fp16 caches)."""
    check(lib().arc_attention_decode(_ptr(q), _ptr(kc), _ptr(vc), kv_heads, hpk, max_ctx, T, _ptr(out),
                                     _ptr(workspace), _sp(stream)))


def prefill_gemm_workspace_bytes(N: int, K: int) -> int:
    n = int(lib().arc_prefill_gemm_workspace_bytes(N, K))
    if n == 0:
        raise ArcError(1, f"no prompt-pass GEMM workspace size for {N} x {K}")
    return n


def prefill_gemm(qtype: int, w, N: int, K: int, x, M: int, y, workspace, stream: Optional[Stream] = None) -> None:
    """The prompt pass's projection GEMM: y[M][N] (fp32) = x[M][K] (fp16) . w^T."""
    check(lib().arc_prefill_gemm(qtype, _ptr(w), N, K, _ptr(x), M, _ptr(y), _ptr(workspace), _sp(stream)))


def prefill_gateup(w_gate, w_up, N: int, K: int, x, M: int, s, workspace, stream: Optional[Stream] = None) -> None:
    """The prompt pass's fused gate/up + SwiGLU: s[M][N] (fp16)."""
    check(lib().arc_prefill_gateup(_ptr(w_gate), _ptr(w_up), N, K, _ptr(x), M, _ptr(s), _ptr(workspace),
                                   _sp(stream)))


def prefill_attention(q, kc, vc, kv_heads: int, hpk: int, max_ctx: int, pos0: int, M: int, x, ldx: int,
                      mfma: bool = True, stream: Optional[Stream] = None) -> None:
    """The prompt pass's causal GQA: x[m] (fp16, row stride ldx) for prompt rows m < M at positions
    pos0 + m over the fp16 caches; MFMA kernel (default) or the VALU one."""
    check(lib().arc_prefill_attention(_ptr(q), _ptr(kc), _ptr(vc), kv_heads, hpk, max_ctx, pos0, M, _ptr(x), ldx,
                                      1 if mfma else 0, _sp(stream)))


def prefill_qkv(wq, wk, wv, v_qtype: int, H: int, kvd: int, K: int, x, M: int, y, workspace,
                stream: Optional[Stream] = None) -> None:
    """The prompt pass's q|k|v launch before bias and RoPE: y[M][H + 2 kvd] (fp32)."""
    check(lib().arc_prefill_qkv(_ptr(wq), _ptr(wk), _ptr(wv), v_qtype, H, kvd, K, _ptr(x), M, _ptr(y),
                                _ptr(workspace), _sp(stream)))


def tune_force(bs: int, rpl: int) -> None:
    """Force the GEMV lane layout (bs quads per row, rpl rows per lane); 0 = automatic."""
    check(lib().arc_tune_force(bs, rpl))


def tune_waves(waves: int) -> None:
    """Force the waves per GEMV workgroup (4 or 8); 0 = automatic."""
    check(lib().arc_tune_waves(waves))


def tune_attention(waves: int = 0, min_chunks_per_split: int = 0) -> None:
    """Decode attention launch shape: waves per workgroup (4 or 8) and the
    least chunks of 16 * waves positions per split; 0 = automatic."""
    check(lib().arc_tune_attention(int(waves), int(min_chunks_per_split)))


def tune_prefill_attention(mfma: bool = True) -> None:
    """The prompt pass's attention kernel: MFMA (default) or VALU."""
    check(lib().arc_tune_prefill_attention(1 if mfma else 0))


def tune_fuse_attn_o(on=True) -> None:
    """Attention and o projection of decode steps captured later as one
    launch (default) or two; 2 = one launch whose attention withholds its
    signal (a test of the bounded wait: the decode call then fails)."""
    check(lib().arc_tune_fuse_attn_o(int(on) if not isinstance(on, bool) else (1 if on else 0)))


DEC_O, DEC_GATEUP, DEC_DOWN, DEC_LMHEAD = 0, 1, 2, 3


def tune_decode(kind: int, bs: int = 0, rpl: int = 1, waves: int = 0) -> None:
    """Layout / waves of one GEMV of decode steps captured later (kind DEC_*);
    bs = 0 and waves = 0 keep the step's own."""
    check(lib().arc_tune_decode(int(kind), int(bs), int(rpl), int(waves)))


def tune_rowstream(mode: int) -> None:
    """Whole-row Q4_K GEMVs (K <= 3584): -1 automatic (default), 0 quad layout
    only, 1 row-stream kernel."""
    check(lib().arc_tune_rowstream(int(mode)))


# ------------------------------------------------------- synthetic inputs
def synth_packed(qtype: int, seed: int, stream: int, rows: int, K: int, d_sigma: float = 0.01,
                 dmin_sigma: float = 0.005) -> np.ndarray:
    out = np.empty(rows * (K // QK) * BLOCK_BYTES[qtype], dtype=np.uint8)
    check(lib().arc_synth_packed(qtype, seed, stream, rows, K, d_sigma, dmin_sigma, out.ctypes.data))
    return out


def synth_normal(seed: int, stream: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(lib().arc_synth_normal(seed, stream, n, mean, sigma, out.ctypes.data))
    return out


# ------------------------------------------------------------ decode runtime
def qwen25_7b_dims() -> ModelDims:
    d = ModelDims()
    check(lib().arc_model_dims_qwen25_7b(C.byref(d)))
    return d


def tensor_info(dims: ModelDims, layer: int, which: int) -> tuple[int, int, int, int]:
    """(qtype or 0 for fp32, rows, K, bytes) of a tensor slot (layer -1 for globals)."""
    qt, rows, K, nb = C.c_int(), C.c_uint32(), C.c_uint32(), C.c_uint64()
    check(lib().arc_model_tensor_info(C.byref(dims), layer, which, C.byref(qt), C.byref(rows), C.byref(K),
                                      C.byref(nb)))
    return qt.value, rows.value, K.value, nb.value


def model_slots(dims: ModelDims):
    """(layer, which) of every tensor slot, in arc_model_create order."""
    out = [(-1, w) for w in range(T_GLOBAL_COUNT)]
    for layer in range(dims.layers):
        out += [(layer, w) for w in range(T_LAYER_COUNT)]
    return out


def synth_model_tensors(dims: ModelDims, seed: int) -> list:
    """Host arrays of every tensor slot of the random-init model."""
    arrs = []
    for layer, which in model_slots(dims):
        qt, rows, K, nb = tensor_info(dims, layer, which)
        a = np.empty(nb // 4, np.float32) if qt == 0 else np.empty(nb, np.uint8)
        check(lib().arc_model_synth_tensor(C.byref(dims), seed, layer, which, a.ctypes.data))
        arrs.append(a)
    return arrs


class Model:
    """A model resident in HBM (packed super-blocks copied verbatim)."""

    def __init__(self, dims: ModelDims, tensors=None, seed: int = 0):
        self.dims = dims
        h = _P()
        if tensors is None:
            check(lib().arc_model_create_synthetic(C.byref(dims), seed, C.byref(h)))
        else:
            ptrs = (_P * len(tensors))(*[t.ctypes.data for t in tensors])
            check(lib().arc_model_create(C.byref(dims), ptrs, C.byref(h)))
        self.handle = h.value

    @property
    def weight_bytes(self) -> int:
        return int(lib().arc_model_weight_bytes(self.handle))

    def tensor_device(self, layer: int, which: int) -> int:
        """Device address of a resident tensor (layer -1: the global slots)."""
        ptr = _P()
        check(lib().arc_model_tensor_device(self.handle, layer, which, C.byref(ptr)))
        return int(ptr.value)

    def exec148_reserve(self) -> tuple[int, int, int]:
        """(device base, slot stride, slots) of the model's EXEC148 reserve."""
        base, stride, slots = _P(), _U64(0), _U32(0)
        check(lib().arc_model_exec148_reserve(self.handle, C.byref(base), C.byref(stride), C.byref(slots)))
        return int(base.value or 0), int(stride.value), int(slots.value)

    def close(self) -> None:
        if getattr(self, "handle", None):
            if _lib is not None:
                _lib.arc_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def device_allocations() -> int:
    """Device allocations the library has made in this process."""
    n = _U64(0)
    check(lib().arc_device_allocations(C.byref(n)))
    return int(n.value)


class Session:
    """fp16 KV cache + working buffers + the captured decode step."""

    def __init__(self, model: Model, max_ctx: int):
        self.model = model
        self.max_ctx = max_ctx
        h = _P()
        check(lib().arc_session_create(model.handle, max_ctx, C.byref(h)))
        self.handle = h.value

    def fill_kv(self, ctx: int, seed: int) -> None:
        check(lib().arc_session_fill_kv(self.handle, ctx, seed))

    def route_down(self, layer: int, exec148=None) -> None:
        """Route layer's Q4_K ffn_down to an EXEC148 image (route B; kept alive by
        the caller) or, with None, back to the packed tensor (route A)."""
        check(lib().arc_session_route_down(self.handle, layer, _ptr(exec148)))

    def kv(self, layer: int) -> tuple[int, int]:
        k, v = _P(), _P()
        check(lib().arc_session_kv(self.handle, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def decode(self, token: int, pos: int, n_steps: int, logits: bool = False, graph: bool = True):
        out = np.zeros(n_steps, np.uint32)
        nf = C.c_uint32(0)
        flags = (DECODE_LOGITS if logits else 0) | (0 if graph else DECODE_NO_GRAPH)
        check(lib().arc_session_decode(self.handle, token, pos, n_steps, flags, out.ctypes.data, C.byref(nf)))
        return out, nf.value

    def prefill(self, tokens, pos0: int = 0, logits: bool = False, graph: bool = True, stepwise: bool = False):
        """Feed `tokens` at positions pos0..; returns (argmax after the last, nonfinite).  Batched
        MFMA pass for two or more tokens unless `stepwise` (decode step per token)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt, nf = C.c_uint32(0), C.c_uint32(0)
        flags = (DECODE_LOGITS if logits else 0) | (0 if graph else DECODE_NO_GRAPH) | \
            (PREFILL_STEPWISE if stepwise else 0)
        check(lib().arc_session_prefill(self.handle, t.ctypes.data, len(t), pos0, flags, C.byref(nxt), C.byref(nf)))
        return nxt.value, nf.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.dims.vocab, np.float32)
        check(lib().arc_session_logits(self.handle, out.ctypes.data))
        return out

    @property
    def prefill_kernels(self) -> int:
        return int(lib().arc_session_prefill_kernels(self.handle))

    @property
    def kernels_per_step(self) -> int:
        return int(lib().arc_session_kernels_per_step(self.handle))

    def residency(self) -> dict:
        """The planned bytes of the session and its model (arc_session_residency)."""
        r = Residency()
        check(lib().arc_session_residency(self.handle, C.byref(r)))
        return {name: int(getattr(r, name)) for name, _ in Residency._fields_}

    def close(self) -> None:
        if getattr(self, "handle", None):
            if _lib is not None:
                _lib.arc_session_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
