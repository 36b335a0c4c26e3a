"""Load-time conversion on the device (HF offline ternary layout -> I2_S) against the oracle, and the
SGLBITNT model round trip through the end-to-end model."""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu


def _hf_pack(w):
    """HF offline packing of int8 ternary [N, K] (rows past N padded with zero weights, as the reference's
    quantize_dlm_to_offline.py does)."""
    n, k = w.shape
    nb = (n + 3) // 4
    codes = np.ones((4 * nb, k), dtype=np.uint8)
    codes[:n] = (w + 1).astype(np.uint8)
    packed = np.zeros((nb, k), dtype=np.uint8)
    for i in range(4):
        packed |= codes[i * nb:(i + 1) * nb] << (2 * i)
    return packed


@pytest.mark.parametrize("n,k", [(2560, 2560), (6912, 2560), (13, 640), (7, 130), (576, 576), (1, 128)])
@pytest.mark.parametrize("mode", ["reference", "checkpoint"])
def test_convert_hf_offline_matches_oracle(pkg, dev, n, k, mode):
    rng = np.random.default_rng(n + k)
    w = orc.random_ternary(rng, n, k)
    packed = _hf_pack(w)
    ws = torch.tensor([0.0421], dtype=torch.bfloat16)
    q, s = pkg.convert_hf_offline_i2s(torch.from_numpy(packed).to(dev), ws.to(dev), out_features=n, scale_mode=mode)
    q_ref, s_ref = orc.convert_hf_offline(packed, ws.float().item(), n=n, mode=mode)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert s.item() == float(s_ref)
    assert np.array_equal(orc.unpack_i2s(q.cpu().numpy())[:, :k], w)


def test_convert_hf_offline_transformers_packing_and_host_scale(pkg, dev):
    """A checkpoint packed by transformers' own pack_weights (padding rows are code 0 = -1 there: they
    count in the reference's mean but are not part of the output)."""
    tb = pytest.importorskip("transformers.integrations.bitnet")
    rng = np.random.default_rng(7)
    w = orc.random_ternary(rng, 30, 256)
    packed = tb.pack_weights(torch.from_numpy(w.astype(np.int8))).numpy()
    q, s = pkg.convert_hf_offline_i2s(torch.from_numpy(packed).to(dev), 0.5, out_features=30)
    q_ref, s_ref = orc.convert_hf_offline(packed, 0.5, n=30)
    assert np.array_equal(q.cpu().numpy(), q_ref) and s.item() == float(s_ref)


def test_convert_then_linear_equals_pack_then_linear(pkg, dev):
    """The converted weight drives the BitLinear exactly like the same ternary matrix packed directly."""
    rng = np.random.default_rng(9)
    n, k = 640, 1024
    w = orc.random_ternary(rng, n, k)
    q, s = pkg.convert_hf_offline_i2s(torch.from_numpy(_hf_pack(w)).to(dev), 1.0, out_features=n,
                                      scale_mode="checkpoint")
    a = torch.from_numpy(orc.random_int8(rng, 3, k)).to(dev)
    _, acc = pkg.bitnet_linear(q, a, s, return_acc=True, out_dtype=None)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64),
                          a.cpu().numpy().astype(np.int64) @ w.astype(np.int64).T)


def test_convert_errors(pkg, dev):
    p = torch.zeros((4, 128), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="4\\*\\(NB-1\\)"):
        pkg.convert_hf_offline_i2s(p, 1.0, out_features=12)
    with pytest.raises(RuntimeError, match="k_pad"):
        pkg.convert_hf_offline_i2s(p, 1.0, k_pad=192)
    with pytest.raises(ValueError, match="scale_mode"):
        pkg.convert_hf_offline_i2s(p, 1.0, scale_mode="x")


@pytest.mark.parametrize("ternary_head", [False, True])
def test_sglbitnt_model_round_trip(pkg, dev, tmp_path, ternary_head):
    """save_sglbitnt -> from_sglbitnt: the same packed bytes, scales and norms, so the same greedy tokens."""
    M = pkg.model
    cfg = M.BitNetConfig(vocab_size=1500, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                         num_kv_heads=2, head_dim=64, rope_theta=10000.0, tie_embeddings=not ternary_head,
                         ternary_lm_head=ternary_head)
    model = M.BitNetDecoder(cfg, seed=11, device=dev)
    path = tmp_path / "model.bin"
    model.save_sglbitnt(path)
    f = pkg.SGLBitNetFile(path)
    assert f.tensors["model.layers.1.mlp.down_proj.weight"].shape == (256, 128)
    assert ("lm_head.weight" in f) == ternary_head
    loaded = M.BitNetDecoder.from_sglbitnt(path, device=dev)
    assert loaded.cfg == model.cfg
    for a, b in zip(M.quantised_linears(model).values(), M.quantised_linears(loaded).values()):
        assert torch.equal(a.qweight, b.qweight) and torch.equal(a.scale, b.scale)
    prompt = torch.randint(0, cfg.vocab_size, (2, 7), generator=torch.Generator().manual_seed(12))
    assert torch.equal(model.generate(prompt, 10), loaded.generate(prompt, 10))
