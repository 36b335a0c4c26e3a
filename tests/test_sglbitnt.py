"""SGLBITNT reader/writer (CPU).  The reader is pinned by a file assembled byte by byte from the
reference writer's layout (packages/inference/scripts/convert_to_sglkernel.py:135-160, 288-310:
magic, '<I' version, '<I' + config JSON, '<I' count, per tensor '<I' name length + name, '<I' dtype,
'<I' ndims + '<I' dims, '<I' scale flag [+ '<f' scale], '<Q' size + data) and by the loader's checks
(sglkernel_loader.h:75-161)."""

import json
import struct

import numpy as np
import pytest
import torch


def _golden_bytes():
    cfg = json.dumps({"vocab_size": 7, "hidden_size": 128, "num_hidden_layers": 1}).encode()
    b = b"SGLBITNT" + struct.pack("<I", 1) + struct.pack("<I", len(cfg)) + cfg + struct.pack("<I", 2)
    w = np.arange(2 * 32, dtype=np.uint8).reshape(2, 32)            # packed [2, 128/4]
    name = b"model.layers.0.self_attn.q_proj.weight"
    b += struct.pack("<I", len(name)) + name + struct.pack("<I", 0) + struct.pack("<I", 2) + struct.pack("<II", 2, 32)
    b += struct.pack("<I", 1) + struct.pack("<f", 0.375) + struct.pack("<Q", w.nbytes) + w.tobytes()
    e = np.linspace(-1, 1, 7 * 4, dtype=np.float32).reshape(7, 4)
    name = b"model.embed_tokens.weight"
    b += struct.pack("<I", len(name)) + name + struct.pack("<I", 1) + struct.pack("<I", 2) + struct.pack("<II", 7, 4)
    b += struct.pack("<I", 0) + struct.pack("<Q", e.nbytes) + e.tobytes()
    return b, w, e


def test_reader_parses_reference_layout(pkg, tmp_path):
    raw, w, e = _golden_bytes()
    p = tmp_path / "m.bin"
    p.write_bytes(raw)
    f = pkg.SGLBitNetFile(p)
    assert f.config["vocab_size"] == 7 and f.config["hidden_size"] == 128
    q = f.tensors["model.layers.0.self_attn.q_proj.weight"]
    assert q.dtype_id == 0 and q.shape == (2, 32) and q.scale == 0.375
    assert np.array_equal(f.numpy(q.name), w)
    t = f.tensors["model.embed_tokens.weight"]
    assert t.scale is None and t.shape == (7, 4)
    assert torch.equal(f.tensor(t.name), torch.from_numpy(e))


def test_writer_reproduces_reference_layout(pkg, tmp_path):
    raw, w, e = _golden_bytes()
    p = tmp_path / "w.bin"
    pkg.write_sglbitnt(p, {"vocab_size": 7, "hidden_size": 128, "num_hidden_layers": 1},
                       {"model.layers.0.self_attn.q_proj.weight": (torch.from_numpy(w), 0.375),
                        "model.embed_tokens.weight": (torch.from_numpy(e), None)})
    assert p.read_bytes() == raw


@pytest.mark.parametrize("dt", [torch.uint8, torch.float32, torch.float16, torch.bfloat16])
def test_round_trip_dtypes(pkg, tmp_path, dt):
    g = torch.Generator().manual_seed(1)
    t = (torch.randn((5, 3, 4), generator=g) * 10).to(dt) if dt != torch.uint8 else \
        torch.randint(0, 256, (5, 12), generator=g, dtype=torch.uint8)
    p = tmp_path / "r.bin"
    pkg.write_sglbitnt(p, {"vocab_size": 1, "hidden_size": 1}, {"x": (t, 1.5 if dt == torch.uint8 else None)})
    r = pkg.SGLBitNetFile(p).tensor("x")
    assert r.dtype == dt and torch.equal(r, t)


def test_reader_errors(pkg, tmp_path):
    raw, _, _ = _golden_bytes()
    p = tmp_path / "e.bin"
    p.write_bytes(b"SGLBITNX" + raw[8:])
    with pytest.raises(ValueError, match="Invalid magic number"):
        pkg.SGLBitNetFile(p)
    p.write_bytes(raw[:8] + struct.pack("<I", 2) + raw[12:])
    with pytest.raises(ValueError, match="Unsupported version: 2"):
        pkg.SGLBitNetFile(p)
    cfg = json.dumps({"vocab_size": 0, "hidden_size": 128}).encode()
    p.write_bytes(b"SGLBITNT" + struct.pack("<II", 1, len(cfg)) + cfg + struct.pack("<I", 0))
    with pytest.raises(ValueError, match="vocab_size or hidden_size is 0"):
        pkg.SGLBitNetFile(p)
    p.write_bytes(raw[:-10])
    with pytest.raises(ValueError, match="past the end|truncated"):
        pkg.SGLBitNetFile(p)
