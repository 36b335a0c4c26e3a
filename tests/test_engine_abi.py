"""CPU checks of the native engine ABI (include/wfbitnet_engine.h): every declared symbol is exported, model
files and configurations are rejected on the host with the loader's messages (before any GPU use), NULL
handles follow the reference's contract (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:738-929), the
top-p sampler reproduces the reference's algorithm (bitnet_engine.cpp:208-253: float32 softmax, descending
sort, running-sum cutoff, std::uniform_real_distribution<float> on std::mt19937) on the raw MT19937
stream, and the rotary tables equal the closed form."""

import ctypes
import math
import re
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wfbitnet_engine.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+((?:bitnet|wfb)_\w+)\s*\(", text, flags=re.M)))


def test_engine_library_exports_every_declared_symbol(pkg):
    E = pkg.engine
    lib = E.lib()
    names = declared()
    for s in ("bitnet_engine_create", "bitnet_engine_destroy", "bitnet_get_error", "bitnet_generate",
              "bitnet_prefill", "bitnet_decode_step", "bitnet_reset_cache", "bitnet_vocab_size", "bitnet_hidden_size",
              "bitnet_num_layers", "bitnet_max_seq_len", "bitnet_free_result"):
        assert s in names  # the reference header's entry points (bitnet_engine.h:56-157)
    for s in names:
        assert hasattr(lib, s), f"{s} declared in {HEADER.name} but not exported"
    assert set(E.SIGNATURES) == set(names)


def test_struct_layouts_match_the_reference_header(pkg):
    # bitnet_engine.h:22-43: three int32; float, float, int32, float, int32; pointer, int32, pointer, int32
    eng = pkg.engine
    assert ctypes.sizeof(eng.BitNetConfig) == 12
    assert ctypes.sizeof(eng.SamplingParams) == 20
    assert [f[0] for f in eng.GenerationResult._fields_] == ["output_ids", "num_tokens", "logits", "logits_size"]
    assert eng.GenerationResult.logits.offset == 16 and ctypes.sizeof(eng.GenerationResult) == 32


def _cfg(**kw):
    c = {"vocab_size": 64, "hidden_size": 128, "intermediate_size": 256, "num_hidden_layers": 1,
         "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 64, "rms_norm_eps": 1e-5,
         "max_position_embeddings": 32}
    c.update(kw)
    return c


def _tensors(cfg, drop=(), bad=None):
    h, f, v = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    qd = cfg["num_attention_heads"] * cfg["head_dim"]
    kvd = cfg["num_key_value_heads"] * cfg["head_dim"]
    kp = lambda k: (k + 127) // 128 * 128  # noqa: E731
    packed = lambda o, i: (torch.full((o, kp(i) // 4), 0x55, dtype=torch.uint8), 0.5)  # noqa: E731
    t = {"model.embed_tokens.weight": (torch.zeros(v, h), None)}
    pre = "model.layers.0."
    t[pre + "self_attn.q_proj.weight"] = packed(qd, h)
    t[pre + "self_attn.k_proj.weight"] = packed(kvd, h)
    t[pre + "self_attn.v_proj.weight"] = packed(kvd, h)
    t[pre + "self_attn.o_proj.weight"] = packed(h, qd)
    t[pre + "mlp.gate_proj.weight"] = packed(f, h)
    t[pre + "mlp.up_proj.weight"] = packed(f, h)
    t[pre + "mlp.down_proj.weight"] = packed(h, f)
    t[pre + "input_layernorm.weight"] = (torch.ones(h), None)
    t[pre + "post_attention_layernorm.weight"] = (torch.ones(h), None)
    t["model.norm.weight"] = (torch.ones(h), None)
    for d in drop:
        t.pop(d)
    if bad:
        t.update(bad)
    return t


def _create_error(pkg, path):
    E = pkg.engine
    with pytest.raises(RuntimeError) as ei:
        E.NativeEngine(str(path))
    return str(ei.value)


def test_create_rejects_bad_files(pkg, tmp_path):
    assert "Failed to open file" in _create_error(pkg, tmp_path / "missing.bin")
    p = tmp_path / "magic.bin"
    p.write_bytes(b"NOTMAGIC" + b"\0" * 32)
    assert "Invalid magic number" in _create_error(pkg, p)
    p = tmp_path / "version.bin"
    p.write_bytes(b"SGLBITNT" + struct.pack("<I", 2) + b"\0" * 32)
    assert "Unsupported version: 2" in _create_error(pkg, p)
    good = tmp_path / "good.bin"
    pkg.write_sglbitnt(good, _cfg(), _tensors(_cfg()))
    data = good.read_bytes()
    p = tmp_path / "trunc.bin"
    p.write_bytes(data[:-100])
    assert "Truncated tensor data" in _create_error(pkg, p)
    p = tmp_path / "zero.bin"
    pkg.write_sglbitnt(p, _cfg(vocab_size=0), _tensors(_cfg()))
    assert "vocab_size or hidden_size is 0" in _create_error(pkg, p)


@pytest.mark.parametrize("case,needle", [
    ("missing_down", "Tensor not found: model.layers.0.mlp.down_proj.weight"),
    ("missing_norm", "Tensor not found: model.norm.weight"),
    ("q_shape", "self_attn.q_proj.weight: packed shape"),
    ("norm_size", "input_layernorm.weight: 64 elements, expected 128"),
    ("float_as_packed", "expected a packed uint8"),
    ("head_dim", "head_dim must be 64 or 128"),
    ("gqa", "1..8 times num_key_value_heads"),
    ("act", "hidden_act \"gelu\" not supported"),
])
def test_create_rejects_bad_models_on_the_host(pkg, tmp_path, case, needle):
    cfg = _cfg()
    t = None
    if case == "missing_down":
        t = _tensors(cfg, drop=["model.layers.0.mlp.down_proj.weight"])
    elif case == "missing_norm":
        t = _tensors(cfg, drop=["model.norm.weight"])
    elif case == "q_shape":
        t = _tensors(cfg, bad={"model.layers.0.self_attn.q_proj.weight": (torch.zeros(64, 32, dtype=torch.uint8), 1.0)})
    elif case == "norm_size":
        t = _tensors(cfg, bad={"model.layers.0.input_layernorm.weight": (torch.ones(64), None)})
    elif case == "float_as_packed":
        t = _tensors(cfg, bad={"model.layers.0.mlp.up_proj.weight": (torch.ones(256, 32), None)})
    elif case == "head_dim":
        cfg = _cfg(head_dim=96)
    elif case == "gqa":
        cfg = _cfg(num_attention_heads=18, num_key_value_heads=1, hidden_size=1152)
    elif case == "act":
        cfg = _cfg(hidden_act="gelu")
    p = tmp_path / "m.bin"
    pkg.write_sglbitnt(p, cfg, t if t is not None else _tensors(_cfg()))
    assert needle in _create_error(pkg, p)


def test_null_engine_contract(pkg):
    E = pkg.engine
    lib = E.lib()
    p = E.sampling(max_tokens=4)
    res = E.GenerationResult()
    ids = (ctypes.c_int32 * 2)(1, 2)
    assert lib.bitnet_generate(None, ids, 2, ctypes.byref(p), ctypes.byref(res)) == -1
    assert E.last_error() == "Engine not initialized"
    assert lib.bitnet_prefill(None, ids, 2) == -1
    out = ctypes.c_int32(0)
    assert lib.bitnet_decode_step(None, 0, ctypes.byref(p), ctypes.byref(out)) == -1
    for fn in ("bitnet_vocab_size", "bitnet_hidden_size", "bitnet_num_layers", "bitnet_max_seq_len",
               "bitnet_get_num_kv_heads"):
        assert getattr(lib, fn)(None) == 0
    lib.bitnet_reset_cache(None)
    lib.bitnet_engine_destroy(None)
    lib.bitnet_free_result(None)
    lib.bitnet_free_result(ctypes.byref(res))  # NULL members


# ---- sampler -------------------------------------------------------------------------------------


def _mt_raw(seed, n):
    """Raw 32-bit outputs of std::mt19937(seed) (numpy's legacy seeding is the same init_genrand)."""
    return np.random.RandomState(seed)._bit_generator.random_raw(n).astype(np.uint64)


def _canonical(u):
    """std::generate_canonical<float, 24> of one 32-bit draw: float(u) / 2^32, kept below 1."""
    r = np.float32(u) / np.float32(2.0 ** 32)
    return np.float32(np.nextafter(np.float32(1), np.float32(0))) if r >= 1 else r


@pytest.mark.parametrize("top_p,keep", [(1.0, 16), (0.5, 8), (0.0, 16), (0.3, 5)])
def test_sampler_draws_follow_the_mt19937_stream(pkg, top_p, keep):
    """16 equal logits: probabilities are exactly 1/16 (exp(0) = 1, sum 16), std::sort leaves equal keys in
    index order at this size, so draw j is the first i < keep with u_j < (i + 1) / 16, u_j a uniform float
    in [0, keep / 16) from the j-th raw MT19937 output -- the whole chain fixed by the stream."""
    draws = 200
    got = pkg.engine.sample_top_p([0.0] * 16, 1.0, top_p, 42, draws)
    raw = _mt_raw(42, draws)
    want = []
    for u in raw:
        b = np.float32(keep / 16)
        r = np.float32(b * _canonical(u)) + np.float32(0)
        i = 0
        while not (r < np.float32((i + 1) / 16)) and i < keep - 1:
            i += 1
        want.append(i)
    assert got == want


def test_sampler_frequencies_temperature_and_nucleus(pkg):
    logits = [2.0, 1.0, 0.0, -1.0, -3.0]
    n = 40000
    for temp in (1.0, 0.5, 2.0):
        p = np.exp(np.array(logits) / temp)
        p /= p.sum()
        got = np.bincount(pkg.engine.sample_top_p(logits, temp, 1.0, 7, n), minlength=5) / n
        assert np.all(np.abs(got - p) <= 4 * np.sqrt(p * (1 - p) / n) + 1e-9), (temp, got, p)
    # nucleus: probabilities sorted 0.636, 0.234, 0.086, ...; top_p 0.8 keeps the first two, renormalised
    p = np.exp(np.array(logits))
    p /= p.sum()
    got = np.bincount(pkg.engine.sample_top_p(logits, 1.0, 0.8, 11, n), minlength=5) / n
    assert got[2:].sum() == 0
    want = p[0] / (p[0] + p[1])
    assert abs(got[0] - want) <= 4 * math.sqrt(want * (1 - want) / n)
    # a nucleus below the largest probability keeps one token
    assert set(pkg.engine.sample_top_p(logits, 1.0, 1e-6, 3, 100)) == {0}
    # temperature 0.5 above is a case whose float32 running sum of all probabilities ends below 1: top_p 1
    # still samples the whole distribution there (the reference's cutoff would keep only token 0)
    assert len(set(pkg.engine.sample_top_p(logits, 0.5, 1.0, 5, 2000))) >= 3


def test_sampler_rejects_bad_arguments(pkg):
    E = pkg.engine
    for args in (([], 1.0, 1.0), ([1.0], 0.0, 1.0), ([1.0], -1.0, 1.0)):
        with pytest.raises(RuntimeError):
            E.sample_top_p(args[0], args[1], args[2], 0, 1)


# ---- rotary tables -------------------------------------------------------------------------------


@pytest.mark.parametrize("theta,d,n", [(10000.0, 64, 300), (500000.0, 128, 257), (100000.0, 64, 5000)])
def test_rope_tables_closed_form(pkg, theta, d, n):
    cos, sin = pkg.rope_tables(theta, d, n)
    assert cos.shape == (n, d // 2) and cos.dtype == torch.float32
    rows = sorted({0, 1, 2, n // 2, n - 1})
    for p in rows:
        for i in range(d // 2):
            a = p * (1.0 / theta ** (2 * i / d))
            assert cos[p, i].item() == np.float32(math.cos(a)) and sin[p, i].item() == np.float32(math.sin(a))
    assert torch.equal(cos[0], torch.ones(d // 2)) and torch.equal(sin[0], torch.zeros(d // 2))
    assert torch.allclose(cos.double() ** 2 + sin.double() ** 2, torch.ones(n, d // 2, dtype=torch.float64), atol=1e-6)
    with pytest.raises(ValueError):
        pkg.rope_tables(theta, 63, n)
