"""Minimal GGUF v3 writer for tests: a Qwen2-architecture model file from the
synthetic slot tensors (arcllm_amd.synth_model_tensors), with the tensor
names and metadata keys of llama.cpp's qwen2 layout that the runtime binds
(the names the reference's runtime binds, src/arcllm_v1_runtime.cpp:196-205).
"""
from __future__ import annotations

import struct

import numpy as np

U32, I32, F32, STRING, U64 = 4, 5, 6, 8, 10
T_F32, T_Q4K, T_Q6K = 0, 12, 14

GLOBAL_NAMES = ["token_embd.weight", "output.weight", "output_norm.weight"]
LAYER_NAMES = ["attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q.bias", "attn_k.bias",
               "attn_v.bias", "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
               "ffn_down.weight"]


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == U32:
        return struct.pack("<I", v)
    if vtype == I32:
        return struct.pack("<i", v)
    if vtype == F32:
        return struct.pack("<f", v)
    if vtype == U64:
        return struct.pack("<Q", v)
    if vtype == STRING:
        return _str(v)
    raise ValueError(vtype)


def write_gguf(path: str, metadata, tensors, alignment: int = 32, version: int = 3, offsets=None) -> None:
    """metadata: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, bytes)].
    `offsets` overrides the computed data offsets (for malformed-file tests)."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, v in metadata:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offs, cur = [], 0
    for _, _, _, data in tensors:
        cur = (cur + alignment - 1) // alignment * alignment
        offs.append(cur)
        cur += len(data)
    if offsets is not None:
        offs = offsets
    for (name, dims, gtype, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, off)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        pos = 0
        for (_, _, _, data), off in sorted(zip(tensors, offs), key=lambda t: t[1]):
            if off > pos:
                f.write(b"\0" * (off - pos))
                pos = off
            f.write(bytes(data))
            pos += len(data)


def qwen2_tensors(dims, slot_tensors):
    """(name, gguf dims, type, bytes) for every slot of a model, in file order."""
    import arcllm_amd as arc

    out = []

    def add(name, layer, which, data):
        qtype, rows, K, _ = arc.tensor_info(dims, layer, which)
        if qtype == 0:
            out.append((name, [K], T_F32, np.ascontiguousarray(data).view(np.uint8)))
        else:
            out.append((name, [K, rows], qtype, np.ascontiguousarray(data).view(np.uint8)))

    for w, name in enumerate(GLOBAL_NAMES):
        add(name, -1, w, slot_tensors[w])
    for layer in range(dims.layers):
        for w, name in enumerate(LAYER_NAMES):
            add(f"blk.{layer}.{name}", layer, w, slot_tensors[3 + 12 * layer + w])
    return out


def qwen2_metadata(dims):
    return [
        ("general.architecture", STRING, "qwen2"),
        ("general.alignment", U32, 32),
        ("qwen2.block_count", U32, dims.layers),
        ("qwen2.embedding_length", U32, dims.hidden),
        ("qwen2.feed_forward_length", U32, dims.ffn),
        ("qwen2.attention.head_count", U32, dims.q_heads),
        ("qwen2.attention.head_count_kv", U32, dims.kv_heads),
        ("qwen2.rope.freq_base", F32, float(dims.rope_theta)),
        ("qwen2.attention.layer_norm_rms_epsilon", F32, float(dims.rms_eps)),
    ]


def write_qwen2_model(path: str, dims, slot_tensors) -> None:
    write_gguf(path, qwen2_metadata(dims), qwen2_tensors(dims, slot_tensors))
