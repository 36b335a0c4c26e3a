"""The end-to-end CPU baseline (oracle/c/cpu_decode.c: the reference engine's per-token loop over this model,
BitLinears on the AVX2 port of the reference I2_S GEMV) against the same model's torch CPU glue with the numpy
oracle's quantised groups (oracle/model_backend.py), on small random models built without a GPU: an
SGLBITNT file of oracle-packed weights loaded on the host.  Both compute the same quantised groups (integer
accumulators, the same int8 codes up to rounding-boundary flips) with fp32 glue in different orders, so the
prompt logits agree to float rounding and the greedy tokens are equal."""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc
from oracle import refbind
from oracle.model_backend import OracleBackend, cpu_decoder


def _host_model(pkg, tmp_path, cfg, seed):
    M = pkg.model
    rng = np.random.default_rng(seed)
    h, f = cfg.hidden_size, cfg.intermediate_size
    qd, kvd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    shapes = {"q": (qd, h), "k": (kvd, h), "v": (kvd, h), "o": (h, qd), "gate": (f, h), "up": (f, h), "down": (h, f)}
    t = {"model.embed_tokens.weight": (torch.from_numpy((rng.standard_normal((cfg.vocab_size, h)) * 0.02)
                                                        .astype(np.float32)), None)}
    for i in range(cfg.num_layers):
        pre = f"model.layers.{i}."
        for attr, name in M.BitNetDecoder._LINEARS:
            o, k = shapes[attr]
            kp = -(-k // 128) * 128
            w = np.zeros((o, kp), np.float32)
            w[:, :k] = rng.standard_normal((o, k)) * 0.02
            packed, scale = orc.pack_ternary(w, scale=orc.absmean_scale(w[:, :k]))
            t[pre + name + ".weight"] = (torch.from_numpy(packed), float(scale))
        for attr, name in M.BitNetDecoder._NORMS:
            n = {"input_norm": h, "post_attn_norm": h, "attn_sub_norm": qd, "ffn_sub_norm": f}[attr]
            t[pre + name + ".weight"] = (torch.from_numpy((1 + 0.1 * rng.standard_normal(n)).astype(np.float32)), None)
    t["model.norm.weight"] = (torch.ones(h), None)
    config = {"vocab_size": cfg.vocab_size, "hidden_size": h, "intermediate_size": f,
              "num_hidden_layers": cfg.num_layers, "num_attention_heads": cfg.num_heads,
              "num_key_value_heads": cfg.num_kv_heads, "head_dim": cfg.head_dim, "rope_theta": cfg.rope_theta,
              "rms_norm_eps": cfg.rms_eps, "subln_eps": cfg.subln_eps, "hidden_act": cfg.hidden_act,
              "tie_word_embeddings": True}
    path = tmp_path / "m.bin"
    pkg.write_sglbitnt(path, config, t)
    m = M.BitNetDecoder.from_sglbitnt(path, device="cpu", decode_attention="torch", prefill_attention="torch")
    m.backend = OracleBackend(M.quantised_linears(m).values(), "cpu")
    return m


@pytest.mark.parametrize("act", ["silu", "relu2"])
def test_cpu_decoder_matches_host_model(pkg, tmp_path, act):
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=512, hidden_size=192, intermediate_size=320, num_layers=3, num_heads=6,
                         num_kv_heads=2, head_dim=32, rope_theta=10000.0, hidden_act=act)
    model = _host_model(pkg, tmp_path, cfg, seed=3 if act == "silu" else 4)
    prompt = torch.randint(0, cfg.vocab_size, (1, 9), generator=torch.Generator().manual_seed(1))
    new = 12
    with torch.no_grad():
        model.reset(1, 9 + new)
        want_logits = model.forward(prompt, 0)[0].numpy()
        want = model.generate(prompt, new)[0].numpy()
    dec = cpu_decoder(model, 9 + new)
    toks, logits = dec.greedy(prompt[0].numpy(), new)
    assert np.abs(logits - want_logits).max() <= 1e-4 * np.abs(want_logits).max() + 1e-6
    assert np.array_equal(toks, want)


def test_cpu_decoder_rejects_bad_sizes(pkg, tmp_path):
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_layers=1, num_heads=4,
                         num_kv_heads=2, head_dim=32, rope_theta=10000.0)
    model = _host_model(pkg, tmp_path, cfg, seed=5)
    dec = cpu_decoder(model, 8)
    with pytest.raises(ValueError):
        dec.greedy(np.arange(6), 4)  # prompt + new tokens past max_len
    with pytest.raises(ValueError):
        dec.greedy(np.zeros(0, np.int64), 2)
    assert isinstance(dec, refbind.CpuDecoder)
