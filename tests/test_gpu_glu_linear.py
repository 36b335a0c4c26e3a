"""wfb_linear_i2s_glu (act(gate) * up in the gate|up linear's epilogue): the fp32 output equals the
oracle's gated product of the segmented linear's stored outputs, and re-quantising it gives the same
codes as the unfused path (wfb_glu_rmsnorm_quant_i8 on the stored gate and up), bit for bit."""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # m, half, k, mid dtype
    (8, 14336, 4096, torch.bfloat16),   # Llama-3-8B gate|up (LDS-staged, 4 row tiles x 4 waves)
    (1, 6912, 2560, torch.bfloat16),    # BitNet-2B
    (3, 1536, 640, torch.float32),      # SmolLM2 (fp32 model), K padded
    (16, 14336, 4096, torch.bfloat16),  # LDS-staged at 16 tokens on long rows
    (17, 2048, 1024, torch.bfloat16),   # two token tiles
    (32, 6912, 2560, torch.bfloat16),   # BitNet-2B gate|up at 32 tokens (LDS-staged, two token tiles)
    (24, 2048, 4096, torch.float32),    # 4096-long rows, one round of workgroups
    # K-split tile kernel with the gated epilogue (32 tokens x 64 outputs per tile):
    (24, 14336, 4096, torch.bfloat16),  # 17..32 tokens on long rows of a wide gate|up
    (17, 4096, 4096, torch.float32),    # (its smallest N and K)
    (64, 4096, 512, torch.float32),     # two full token tiles
    (40, 6912, 2560, torch.bfloat16),   # BitNet-2B gate|up at 40 tokens (32 + 8)
    (37, 14336, 4096, torch.bfloat16),  # Llama-3-8B gate|up at 37 tokens
    (33, 14336, 4096, torch.bfloat16),  # a 1-token second tile row
    (49, 14336, 4096, torch.bfloat16),
    (45, 1056, 1152, torch.float32),    # half not a multiple of 64 (a half-full last tile), 9 K blocks
    (64, 96, 128, torch.bfloat16),      # one K block, two tiles per row
]


@pytest.mark.parametrize("act", ["silu", "relu2"])
@pytest.mark.parametrize("case", CASES, ids=[f"m{c[0]}_h{c[1]}_k{c[2]}_{str(c[3])[6:]}" for c in CASES])
def test_glu_linear_matches_oracle_and_unfused(pkg, dev, case, act):
    m, half, k, mid = case
    rng = np.random.default_rng(m * 7 + half + k)
    packed = torch.from_numpy(orc.pack_i2s(orc.random_ternary(rng, 2 * half, k))).to(dev)
    a = torch.from_numpy(orc.random_int8(rng, m, k)).to(dev)
    a_scale = torch.from_numpy(orc.log_uniform(rng, m).astype(np.float32)).to(dev)
    scales = torch.from_numpy(orc.log_uniform(rng, 2).astype(np.float32) * 4).to(dev)
    x = pkg.bitnet_linear_glu(packed, scales, a, act, a_scale=a_scale, mid_dtype=mid)
    # unfused: the stored gate|up, then the gated norm-quant
    y = pkg.bitnet_linear_segmented(packed, [half, half], scales, a, a_scale=a_scale, out_dtype=mid)
    code = orc.ACT_SILU if act == "silu" else orc.ACT_RELU2
    yf = y.float().cpu().numpy()
    assert np.array_equal(x.cpu().numpy(), orc.glu(yf[:, :half], yf[:, half:], code))
    g = (1 + 0.1 * torch.randn(half, generator=torch.Generator().manual_seed(half))).to(torch.bfloat16).to(dev)
    q1, s1 = pkg.glu_rmsnorm_quantize_i8(y[:, :half], y[:, half:], act, g, eps=1e-6)
    q2, s2 = pkg.rmsnorm_quantize_i8(x, g, eps=1e-6)
    assert torch.equal(q1, q2) and torch.equal(s1, s2)


@pytest.mark.parametrize("m,half,k", [(40, 1056, 1152), (20, 4096, 4096), (64, 96, 128), (8, 2048, 1024)])
def test_glu_linear_strided_out_no_token_scales(pkg, dev, m, half, k):
    """Without token scales and into a strided fp32 view (odd row stride, base 4 bytes past a 16-byte
    boundary: the per-element stores), equal to the unfused path, every kernel form."""
    rng = np.random.default_rng(m * 3 + half)
    packed = torch.from_numpy(orc.pack_i2s(orc.random_ternary(rng, 2 * half, k))).to(dev)
    a = torch.from_numpy(orc.random_int8(rng, m, k)).to(dev)
    scales = torch.from_numpy(orc.log_uniform(rng, 2).astype(np.float32) * 4e-3).to(dev)
    big = torch.full((m, half + 5), float("nan"), dtype=torch.float32, device=dev)
    out = big[:, 1:half + 1]
    x = pkg.bitnet_linear_glu(packed, scales, a, "silu", mid_dtype=torch.bfloat16, out=out)
    assert x.data_ptr() == out.data_ptr()
    y = pkg.bitnet_linear_segmented(packed, [half, half], scales, a, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(out.cpu().numpy(), orc.glu(y[:, :half], y[:, half:], orc.ACT_SILU))
    assert torch.isnan(big[:, 0]).all() and torch.isnan(big[:, half + 1:]).all()  # nothing outside the view


def test_glu_linear_errors(pkg, dev):
    packed = torch.zeros((96, 32), dtype=torch.uint8, device=dev)
    a = torch.zeros((2, 128), dtype=torch.int8, device=dev)
    sc = torch.ones(2, device=dev)
    with pytest.raises(ValueError, match="multiple of 32"):
        pkg.bitnet_linear_glu(packed, sc, a)
    with pytest.raises(RuntimeError, match="64 tokens"):
        pkg.bitnet_linear_glu(torch.zeros((128, 32), dtype=torch.uint8, device=dev), sc,
                              torch.zeros((65, 128), dtype=torch.int8, device=dev))
