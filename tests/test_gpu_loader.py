"""Checkpoint loading through the C ABI (q35_load_safetensors; specimpl.Weights,
speccheck/specimpl.py:60-127): a 488-tensor .safetensors file in the checkpoint's layout and
names, written from a seeded random-init engine (with 153 stand-in vision tensors, which are
skipped), loads into a second engine with every tensor bit-identical and the same decode
logits. The file mixes the dtypes a checkpoint can carry: BF16 matrices, F32 A_log values that
bf16 cannot represent (expected: torch's round-to-nearest-even .to(torch.bfloat16)) and an F16
norm weight. Refused files (a wrong shape, a missing tensor) leave the weights untouched."""
import json
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _write(path, tensors):
    """tensors: name -> (dtype tag, shape, raw bytes); writes a .safetensors file."""
    header, off = {}, 0
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, _, raw in tensors.values():
            f.write(raw)


def test_load_checkpoint_roundtrip(tmp_path):
    import torch
    from oracle.weights import registry
    from qwen35 import Engine, EngineError, State
    print("loader: writing a 488-tensor checkpoint", flush=True)
    src = Engine(max_rows=16, max_ctx=256, seed=0)
    dst = Engine(max_rows=16, max_ctx=256, seed=None)
    try:
        rng = np.random.default_rng(3)
        tensors, want = {}, {}
        alog_name = "model.language_model.layers.0.linear_attn.A_log"
        f16_name = "model.language_model.layers.5.input_layernorm.weight"
        for name, shape, _ in registry():
            n = int(np.prod(shape))
            bits = src.read_tensor(name, n)
            if name == alog_name:
                f32 = rng.uniform(0.0, 2.77, n).astype(np.float32)
                tensors[name] = ("F32", shape, f32.tobytes())
                want[name] = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            elif name == f16_name:
                f16 = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
                tensors[name] = ("F16", shape, f16.tobytes())
                want[name] = torch.from_numpy(f16).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            else:
                tensors[name] = ("BF16", shape, bits.tobytes())
                want[name] = bits
        for i in range(153):
            tensors[f"model.visual.blocks.{i}.norm.weight"] = ("F32", (4,), np.ones(4, np.float32).tobytes())
        d = tmp_path / "ckpt"
        d.mkdir()
        _write(d / "model.safetensors", tensors)
        print("loader: loading", flush=True)
        assert dst.load_checkpoint(d) == (335, 153)
        for name, shape, _ in registry():
            got = dst.read_tensor(name, int(np.prod(shape)))
            assert np.array_equal(got, want[name]), name

        # same weights as the source (its own A_log row restored): same decode logits
        dst.load_tensor(alog_name, src.read_tensor(alog_name, 16))
        outs = []
        for e in (src, dst):
            st = State(e, 1, 128)
            y, lg = st.prefill(0, [11, 22, 33, 44], logits=True)
            t, lg2 = st.decode_step([y], logits=True)
            outs.append((y, lg, int(t[0]), lg2))
            st.close()
        assert outs[0][0] == outs[1][0] and outs[0][2] == outs[1][2]
        assert np.array_equal(outs[0][1], outs[1][1]) and np.array_equal(outs[0][3], outs[1][3])

        # refused files leave the weights as they were
        before = dst.read_tensor("model.language_model.norm.weight", 1024)
        bad = tmp_path / "bad"
        bad.mkdir()
        _write(bad / "x.safetensors", {"model.language_model.norm.weight": ("BF16", (1023,), b"\0" * 2046)})
        with pytest.raises(EngineError, match="shape"):
            dst.load_checkpoint(bad)
        _write(bad / "x.safetensors", {"model.language_model.norm.weight": ("BF16", (1024,), b"\0" * 2048)})
        with pytest.raises(EngineError, match="488"):
            dst.load_checkpoint(bad)
        assert np.array_equal(dst.read_tensor("model.language_model.norm.weight", 1024), before)
    finally:
        src.close()
        dst.close()
