"""The reference's own float BitLinear module against the oracle (CPU) and the HIP module (GPU).

Fixture: tests/golden/ref_bitlinear.npz, written by tests/golden/make_bitlinear_golden.py from
packages/training/src/wrinklefree/models/bitlinear.py (weight_quant :46-64, activation_quant :66-84,
forward :86-113, lambda = 1).  The reference computes in the input dtype: for fp32 inputs its
dequantised forward equals the quantised path up to fp32 rounding; for bf16 inputs its own bf16
roundings (scale, x * scale, q / scale, the bf16 matmul) differ from the fp32 kernel arithmetic by a
few bf16 ulps, inside the 1e-2 relative bar.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

GOLD = Path(__file__).resolve().parent / "golden" / "ref_bitlinear.npz"
CASES = ["f32", "f32_bias", "bf16", "ties"]


def _case(name):
    if not GOLD.exists():
        pytest.skip("golden fixture missing")
    d = np.load(GOLD)
    bias = d[f"{name}_bias"]
    return dict(x=d[f"{name}_x"], w=d[f"{name}_w"], bias=bias if bias.size else None, wq=d[f"{name}_wq"],
                xq=d[f"{name}_xq"], y=d[f"{name}_y"], bf16=bool(d[f"{name}_bf16"]))


def _normwise(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b.astype(np.float64)) / np.linalg.norm(b.astype(np.float64)))


def test_fixture_lists_every_case():
    if not GOLD.exists():
        pytest.skip("golden fixture missing")
    d = np.load(GOLD)
    assert list(d["cases"]) == CASES


@pytest.mark.parametrize("name", CASES)
def test_weight_codes_match_reference_weight_quant(name):
    c = _case(name)
    wq = c["wq"]
    mags = np.unique(np.abs(wq[wq != 0]))
    assert mags.size == 1, "the reference's dequantised weights take one magnitude"
    codes_ref = np.sign(wq).astype(np.int8)
    s = orc.absmean_scale(c["w"])
    q = orc.ternarize(c["w"], s)
    if c["bf16"]:
        # the reference rounds 1/mean|w| and w * scale to bf16: a code flips only where |w|/s sits
        # within a bf16 ulp of 1/2
        assert np.mean(q != codes_ref) <= 5e-3
        assert abs(float(mags[0]) - float(s)) <= float(s) * 2.0 ** -7
    else:
        assert np.array_equal(q, codes_ref)
        assert abs(float(mags[0]) - float(s)) <= 2 * float(np.spacing(np.float32(s)))
    if name == "ties":
        # |w| in {0.5, 1.5} with mean 1: 0.5 -> 0 (half to even), 1.5 -> 2 -> clamp 1
        assert s == np.float32(1.0)
        assert np.array_equal(codes_ref, np.where(np.abs(c["w"]) == 1.5, np.sign(c["w"]), 0).astype(np.int8))


@pytest.mark.parametrize("name", CASES)
def test_activation_codes_match_reference_activation_quant(name):
    c = _case(name)
    q, a_scale = orc.quantize_per_token(c["x"])
    deq = q.astype(np.float32) * a_scale[:, None]
    if name == "ties":
        # absmax 127 -> scale 1: the dequantised values are the codes, .5 ties to even
        assert np.array_equal(c["xq"], q.astype(np.float32))
        assert np.array_equal(q[:, 1:], np.rint(c["x"][:, 1:]).astype(np.int8))
    elif c["bf16"]:
        assert _normwise(deq, c["xq"]) <= 1e-2
        assert np.all(np.abs(deq - c["xq"]) <= 1.5 * a_scale[:, None])
    else:
        # same codes; q / (127 / max) versus q * (max / 127) differ by fp32 rounding only
        np.testing.assert_allclose(deq, c["xq"], rtol=4e-7, atol=0)
    zero = ~np.any(c["x"] != 0, axis=1)
    assert np.all(c["xq"][zero] == 0) and np.all(q[zero] == 0)


@pytest.mark.parametrize("name", CASES)
def test_oracle_forward_matches_reference_forward(name):
    c = _case(name)
    packed, s = orc.pack_ternary(c["w"])
    y = orc.bitlinear_forward(c["x"], packed, s, c["bias"])[0]
    if name == "ties":
        assert np.array_equal(y, c["y"])  # integers below 2^24 on both sides
    elif c["bf16"]:
        assert _normwise(orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(y)), c["y"]) <= 1e-2
    else:
        assert _normwise(y, c["y"]) <= 1e-5
        np.testing.assert_allclose(y, c["y"], rtol=1e-4, atol=1e-5 * float(np.abs(c["y"]).max()))


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_bitlinear_matches_reference_forward(pkg, dev, name):
    c = _case(name)
    dt = torch.bfloat16 if c["bf16"] else torch.float32
    n, k = c["w"].shape
    print(f"[golden bitlinear] case={name} N={n} K={k} dtype={dt}", flush=True)
    mod = pkg.BitLinear(k, n, bias=c["bias"] is not None).to(device=dev, dtype=dt)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(c["w"]).to(dt))
        if c["bias"] is not None:
            mod.bias.copy_(torch.from_numpy(c["bias"]).to(dt))
        y = mod(torch.from_numpy(c["x"]).to(device=dev, dtype=dt)).float().cpu().numpy()
    assert y.dtype == np.float32 and y.shape == c["y"].shape
    if name == "ties":
        assert np.array_equal(y, c["y"])
    elif c["bf16"]:
        assert _normwise(y, c["y"]) <= 1e-2
    else:
        assert _normwise(y, c["y"]) <= 1e-5
