"""The library's safetensors container parser (q35_safetensors_scan; the same parser feeds
q35_load_safetensors), no GPU needed. Pinned against files written by the `safetensors`
package (the writer of the reference's checkpoints; its reader is what
speccheck/specimpl.py:76-86 uses) and against malformed containers, which must be refused."""
import json
import struct

import numpy as np
import pytest


def _container(entries, data: bytes, pad: int = 0, raw_header: bytes | None = None) -> bytes:
    h = raw_header if raw_header is not None else json.dumps(entries).encode()
    h += b" " * pad
    return struct.pack("<Q", len(h)) + h + data


def test_scan_files_written_by_safetensors(tmp_path):
    from safetensors.numpy import save_file
    from qwen35 import safetensors_scan
    tensors = {
        "model.language_model.norm.weight": np.ones(1024, np.float32),
        "model.language_model.layers.0.linear_attn.A_log": np.linspace(0, 2.7, 16).astype(np.float32),
        "model.language_model.layers.0.linear_attn.conv1d.weight": np.zeros((6144, 1, 4), np.float16),
        "model.visual.blocks.0.attn.qkv.weight": np.arange(12, dtype=np.int64).reshape(3, 4),
        "model.visual.merger.ln_q.weight": np.zeros(0, np.float32),       # empty tensor
        "model.visual.patch_embed.proj.bias": np.ones(3, np.uint8),
    }
    p = tmp_path / "model.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt", "note": "quote \" and \\u00e9 escapes"})
    data = p.read_bytes()
    assert safetensors_scan(data) == (6, 3)
    assert safetensors_scan(np.fromfile(p, dtype=np.uint8)) == (6, 3)


def test_scan_escaped_names_and_padding():
    from qwen35 import safetensors_scan
    entries = {"__metadata__": {"a": "b"},
               "model.visual.xé\"y": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]},
               "t": {"dtype": "F32", "shape": [], "data_offsets": [4, 8]}}
    assert safetensors_scan(_container(entries, b"\0" * 8, pad=5)) == (2, 1)


@pytest.mark.parametrize("case", ["short", "hlen", "json", "offsets", "bytes", "dtype", "dup", "trailing",
                                  "negative", "missing"])
def test_scan_refuses_malformed(case):
    from qwen35 import EngineError, safetensors_scan
    ok = {"a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]}}
    data = b"\0" * 8
    if case == "short":
        blob = b"\x05\0\0"
    elif case == "hlen":
        blob = struct.pack("<Q", 10_000) + b"{}"
    elif case == "json":
        blob = _container(None, data, raw_header=b'{"a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]')
    elif case == "offsets":
        blob = _container({"a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [4, 12]}}, data)
    elif case == "bytes":
        blob = _container({"a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 8]}}, data)
    elif case == "dtype":
        blob = _container({"a": {"dtype": "Q4", "shape": [2, 2], "data_offsets": [0, 8]}}, data)
    elif case == "dup":
        blob = _container(None, data, raw_header=json.dumps(ok)[:-1].encode() + b', "a": '
                          + json.dumps(ok["a"]).encode() + b"}")
    elif case == "trailing":
        blob = _container(None, data, raw_header=json.dumps(ok).encode() + b" x")
    elif case == "negative":
        blob = _container({"a": {"dtype": "BF16", "shape": [-2, 2], "data_offsets": [0, 8]}}, data)
    else:
        blob = _container({"a": {"dtype": "BF16", "shape": [2, 2]}}, data)
    with pytest.raises(EngineError):
        safetensors_scan(blob)
