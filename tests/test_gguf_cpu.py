"""The host runtime's GGUF container and request checks, on the CPU.

* A Qwen2 model file written by tests/gguf_write.py reads back with every
  tensor's name, type, dims, offset and size, and the metadata values.
* Malformed files are rejected with the reader's message (bad magic,
  unsupported version, truncation, misaligned / overlapping / out-of-file
  tensor data, unsupported tensor types, Q4_K rows that are not whole
  super-blocks) -- the checks of the reference's GgufReader::read and
  TensorStore::inspect (src/gguf.cpp:108-152, src/tensor_store.cpp:130-239).
* The CLI's argument errors and generate()'s request / model-contract errors
  that precede any device use exit with status 2 and the reference's
  messages (src/arcllm_v1_runtime_cli.cpp, src/arcllm_v1_runtime.cpp:153-252).
"""
import os
import subprocess

import numpy as np
import pytest

import arcllm_amd as arc
import gguf_write as gw
from decode_common import tiny_dims


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tiny_dims(layers=2)
    T = arc.synth_model_tensors(d, 5)
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    gw.write_qwen2_model(path, d, T)
    return d, T, path


def test_model_file_reads_back(tiny):
    d, T, path = tiny
    info = arc.gguf_describe(path)
    assert info["version"] == 3 and info["alignment"] == 32 and info["data_offset"] % 32 == 0
    expect = gw.qwen2_tensors(d, T)
    assert [t["name"] for t in info["tensors"]] == [e[0] for e in expect]
    for got, (name, dims, gtype, data) in zip(info["tensors"], expect):
        assert got["type"] == gtype and got["dims"] == list(dims) and got["nbytes"] == len(data), name
        assert got["offset"] % 32 == 0
    md = info["metadata"]
    assert md["general.architecture"] == "qwen2" and md["qwen2.block_count"] == d.layers
    assert md["qwen2.attention.head_count_kv"] == d.kv_heads
    assert md["qwen2.rope.freq_base"] == 1e6
    # tensor bytes are where the table says
    raw = np.fromfile(path, np.uint8)
    for got, (_, _, _, data) in zip(info["tensors"], expect):
        s = info["data_offset"] + got["offset"]
        assert np.array_equal(raw[s:s + got["nbytes"]], np.asarray(data).view(np.uint8))


def _one_tensor(dims=(256, 2), gtype=gw.T_Q4K, nbytes=None):
    n = nbytes if nbytes is not None else 2 * 144
    return [("w", list(dims), gtype, np.zeros(n, np.uint8))]


@pytest.mark.parametrize(
    "case,needle",
    [
        ("magic", "bad magic"),
        ("version", "unsupported version"),
        ("truncated", "past the end"),
        ("misaligned", "not aligned"),
        ("overlap", "overlap"),
        ("type", "unsupported tensor type"),
        ("q4row", "multiple of 256"),
        ("header", "unexpected end"),
    ],
)
def test_malformed_files_are_rejected(tmp_path, case, needle):
    path = str(tmp_path / f"{case}.gguf")
    md = [("general.architecture", gw.STRING, "qwen2")]
    if case == "version":
        gw.write_gguf(path, md, _one_tensor(), version=4)
    elif case == "truncated":
        gw.write_gguf(path, md, _one_tensor())
        size = os.path.getsize(path)
        with open(path, "r+b") as f:
            f.truncate(size - 10)
    elif case == "misaligned":
        gw.write_gguf(path, md, _one_tensor(), offsets=[8])
    elif case == "overlap":
        t = _one_tensor() + [("w2", [256, 2], gw.T_Q4K, np.zeros(288, np.uint8))]
        gw.write_gguf(path, md, t, offsets=[0, 256])
    elif case == "type":
        gw.write_gguf(path, md, _one_tensor(gtype=1, nbytes=1024))  # F16 is not a runtime type
    elif case == "q4row":
        gw.write_gguf(path, md, _one_tensor(dims=(300, 2), nbytes=288))
    elif case == "header":
        gw.write_gguf(path, md, _one_tensor())
        with open(path, "r+b") as f:
            f.truncate(40)
    else:
        gw.write_gguf(path, md, _one_tensor())
        with open(path, "r+b") as f:
            f.write(b"GGUX")
    with pytest.raises(arc.ArcError, match=needle):
        arc.gguf_describe(path)


def _cli(*args):
    return subprocess.run([arc.CLI_PATH, *args], capture_output=True, text=True, timeout=60)


def _req(model, tokens="1,2,3", max_new="4", extra=()):
    return ["--model", model, "--shader-dir", "unused", "--tokens", tokens, "--max-new", max_new, "--profile", "0",
            "--within-validated-domain", "1", *extra]


@pytest.mark.parametrize(
    "args,needle",
    [
        ([], "required: --model"),
        (["--model"], "missing value for --model"),
        (["--bogus", "1"], "unknown argument"),
        (_req("m.gguf", extra=["--profile", "2"]), "--profile must be 0 or 1"),
        (_req("m.gguf", tokens="1,,2"), "bad token"),
        (_req("m.gguf", tokens="99999999999"), "token exceeds uint32"),
        (_req("m.gguf", max_new="0"), "max_new_tokens >= 1"),
        (_req("/nonexistent/m.gguf"), "cannot open"),
    ],
)
def test_cli_rejects_bad_requests(args, needle):
    r = _cli(*args)
    assert r.returncode == 2, r.stdout
    assert "ArcLLM runtime error:" in r.stderr and needle in r.stderr, r.stderr


def test_request_and_model_contract_errors(tiny, tmp_path):
    d, T, path = tiny
    r = _cli(*_req(path, tokens=str(d.vocab)))
    assert r.returncode == 2 and "input token out of vocabulary" in r.stderr, r.stderr
    r = _cli(*_req(path, tokens=",".join(["1"] * 257)))
    assert r.returncode == 2 and "prefill token count exceeds" in r.stderr, r.stderr
    r = _cli(*_req(path, tokens="1", max_new="4097"))
    assert r.returncode == 2 and "exceeds KV context limit" in r.stderr, r.stderr
    # a file missing one layer tensor fails the census
    bad = str(tmp_path / "census.gguf")
    gw.write_gguf(bad, gw.qwen2_metadata(d), gw.qwen2_tensors(d, T)[:-1])
    r = _cli(*_req(bad))
    assert r.returncode == 2 and "tensor census mismatch" in r.stderr, r.stderr
    # a q projection stored as Q6_K is not the layout the runtime binds
    t = gw.qwen2_tensors(d, T)
    i = [n for n, *_ in t].index("blk.0.attn_q.weight")
    name, dims, _, _ = t[i]
    t[i] = (name, dims, gw.T_Q6K, np.zeros(dims[1] * dims[0] // 256 * 210, np.uint8))
    bad2 = str(tmp_path / "qtype.gguf")
    gw.write_gguf(bad2, gw.qwen2_metadata(d), t)
    r = _cli(*_req(bad2))
    assert r.returncode == 2 and "unexpected type or shape" in r.stderr, r.stderr


def test_no_device_is_an_error_not_a_fallback(tiny):
    if arc.device_count() > 0:
        pytest.skip("a HIP device is present")
    r = _cli(*_req(tiny[2]))
    assert r.returncode == 2 and "no HIP device" in r.stderr, r.stderr


def test_runtime_library_exports_generate():
    out = subprocess.run(["nm", "-D", "--defined-only", arc.RUNTIME_LIB_PATH], capture_output=True, text=True).stdout
    assert "arcllm_gguf_describe" in out
    assert "_ZN6arcllm2v17runtime8generateERKNS1_10RunRequestE" in out
