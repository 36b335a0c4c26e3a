"""configs[0] against the reference's OWN model at the level of int8 codes and int32 accumulators.

tests/golden/ref_codes_smollm2.npz (written in the build container by tests/golden/make_codes_golden.py)
holds, for layers 0, 15 and 29 of the reference's stage-1 SmolLM2-135M model on the 32-token prompt (last
16 positions), each BitLinear group's norm input rows, its BitLinear input rows, the int8 codes the
reference's BitLinear.activation_quant gives them (packages/training/src/wrinklefree/models/bitlinear.py:
66-84), one output per group (F.linear of the dequantised operands, bitlinear.py:86-113) and that
BitLinear's weight absmean.

The reference computes its scale as 127.0 / max|x| with a Python-scalar numerator, which torch evaluates as
127 * (1 / max|x|): two roundings, up to one ulp from the correctly rounded quotient that the serving
kernel (SGB/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp:909-944) and these kernels use.  A code can therefore
differ, by one, where the reference's product x * scale lies within an ulp or two of a .5 boundary; the
fused norm + quantiser also normalises in its own fixed order (a few ulps from the reference's RMSNorm /
SubLN), which widens that window a little.  The tests require every other code to be equal and print the
count.  The int32 accumulators of the HIP linear on the reference's own codes must equal the ones the
reference's float output implies (y * s_x * s_w, within 0.25 of an integer), i.e. be exact.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu

F32 = np.float32
GROUPS = ("qkv", "o", "gu", "down")
EPS = {"qkv": "rms_eps", "o": "subln_eps", "gu": "rms_eps", "down": "subln_eps"}
KEPT = {"qkv": "self_attn.q_proj", "o": "self_attn.o_proj", "gu": "mlp.gate_proj", "down": "mlp.down_proj"}


@pytest.fixture(scope="module")
def golden():
    return np.load(Path(__file__).resolve().parent / "golden" / "ref_codes_smollm2.npz", allow_pickle=False)


def _reference_products(lin):
    """x * scale as the reference evaluates it: scale = fl(127 * fl(1 / max|x|)) per row, then the fp32 product."""
    mx = np.abs(lin).max(axis=1, keepdims=True).astype(F32)
    s_ref = (F32(127.0) * (F32(1.0) / mx).astype(F32)).astype(F32)
    return (lin * s_ref).astype(F32)


def _tie_distance_ulps(v):
    """Distance of each product from the nearest .5 boundary, in ulps of the product."""
    half = (np.floor(v) + F32(0.5)).astype(F32)
    return np.abs(v.astype(np.float64) - half) / np.spacing(np.abs(v).astype(F32)).astype(np.float64)


def _check_codes(got, want, lin, bound_ulps, what):
    diff = got.astype(np.int64) - want.astype(np.int64)
    bad = diff != 0
    dist = _tie_distance_ulps(_reference_products(lin))
    assert np.all(np.abs(diff) <= 1), f"{what}: a code differs by more than one"
    assert np.all(dist[bad] <= bound_ulps), f"{what}: a code differs away from a rounding boundary ({dist[bad].max():.1f} ulps)"
    return int(bad.sum()), float(dist[bad].max()) if bad.any() else 0.0


def test_quantiser_on_reference_rows_gives_reference_codes(pkg, dev, golden):
    """The per-token quantiser on the reference BitLinears' own input rows: the reference's codes, except at
    products within 2 ulps of a .5 boundary (the reference's two-rounding scale, see the module docstring)."""
    total, flips, worst = 0, 0, 0.0
    for li in golden["layers"].tolist():
        for g in GROUPS:
            lin, codes = golden[f"lin_{g}_{li}"], golden[f"codes_{g}_{li}"]
            q, s = pkg.quantize_activations_i8_per_token(torch.from_numpy(lin).to(dev))
            n, d = _check_codes(q.cpu().numpy(), codes, lin, 2.0, f"layer {li} {g}")
            total += codes.size
            flips += n
            worst = max(worst, d)
            # the scale is the reference's max / 127 (its dequantisation divides by 127 / max)
            mx = np.abs(lin).max(axis=1).astype(F32)
            assert np.array_equal(s.cpu().numpy(), (mx / F32(127.0)).astype(F32))
    print(f"quantiser on the reference's rows: {flips} of {total} codes differ (at most {worst:.1f} ulps from a tie)",
          flush=True)
    assert flips <= total // 10000


def test_fused_norm_quant_from_reference_norm_inputs(pkg, dev, golden):
    """RMSNorm / SubLN + quantiser in one kernel, fed the reference norms' own input rows (gamma = ones, the
    model's eps): the reference's codes, except at products within 8 ulps of a .5 boundary (own summation
    order of the norm plus the reference's two-rounding scale)."""
    M = pkg.model
    cfg = M.SMOLLM2_135M
    total, flips, worst = 0, 0, 0.0
    for li in golden["layers"].tolist():
        for g in GROUPS:
            pre, lin, codes = golden[f"pre_{g}_{li}"], golden[f"lin_{g}_{li}"], golden[f"codes_{g}_{li}"]
            q, _ = pkg.rmsnorm_quantize_i8(torch.from_numpy(pre).to(dev), None, eps=getattr(cfg, EPS[g]))
            n, d = _check_codes(q.cpu().numpy(), codes, lin, 8.0, f"layer {li} {g}")
            total += codes.size
            flips += n
            worst = max(worst, d)
    print(f"fused norm + quantiser from the reference's norm inputs: {flips} of {total} codes differ (at most "
          f"{worst:.1f} ulps from a tie)", flush=True)
    assert flips <= total // 10000


def test_accumulators_on_reference_codes_are_exact(pkg, dev, golden):
    """The HIP linear on the reference's own int8 codes and its own ternary weights (rne(W * (1 / absmean))
    clamped to [-1, 1], bitlinear.py:46-64, from the recorded absmean): every int32 accumulator equals the one
    the reference's fp32 output implies, y * (127 / max|x|) * (1 / absmean), within 0.25."""
    M = pkg.model
    cfg = M.SMOLLM2_135M
    st = M.random_float_state(cfg, int(golden["seed"][0]))
    worst = 0.0
    for li in golden["layers"].tolist():
        for g in GROUPS:
            lin, codes, y = golden[f"lin_{g}_{li}"], golden[f"codes_{g}_{li}"], golden[f"y_{g}_{li}"]
            w = st[f"model.layers.{li}.{KEPT[g]}.weight"].numpy()
            s_w = (F32(1.0) / golden[f"wmean_{g}_{li}"].astype(F32)).astype(F32)
            wcodes = np.clip(np.rint((w * s_w).astype(F32)), -1, 1).astype(np.int8)
            k = w.shape[1]
            kp = -(-k // 128) * 128
            wpad = np.zeros((w.shape[0], kp), np.int8)
            wpad[:, :k] = wcodes
            apad = np.zeros((codes.shape[0], kp), np.int8)
            apad[:, :k] = codes
            packed = torch.from_numpy(orc.pack_i2s(wpad)).to(dev)
            _, acc = pkg.bitnet_linear(packed, torch.from_numpy(apad).to(dev), 1.0, out_dtype=torch.float32,
                                       return_acc=True)
            acc = acc.cpu().numpy().astype(np.float64)
            mx = np.abs(lin).max(axis=1, keepdims=True).astype(F32)
            s_x = (F32(127.0) * (F32(1.0) / mx).astype(F32)).astype(np.float64)
            implied = y.astype(np.float64) * s_x * float(s_w)
            err = float(np.abs(acc - implied).max())
            worst = max(worst, err)
            assert err <= 0.25, f"layer {li} {g}: accumulators {err:.3f} from the reference's implied integers"
    print(f"accumulators on the reference's codes: at most {worst:.4f} from the implied integers", flush=True)
