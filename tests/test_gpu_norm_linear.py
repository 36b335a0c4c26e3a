"""wfb_rmsnorm_linear_i2s and wfb_rmsnorm_linear_i2s_glu (RMSNorm + per-token quant in the prologue of the
decode BitLinear, plain / residual / gated gate|up): outputs bit-identical to the two-call path
(wfb_rmsnorm_quant_i8, then the segmented / residual / gated linear), which the parity tests pin against
the oracle; one shape of each also checked against the oracle directly."""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu


def _inputs(rng, m, h, rows, k, xdt, gdt):
    n = sum(rows)
    packed = torch.from_numpy(orc.pack_i2s(orc.random_ternary(rng, n, k)))
    x = torch.from_numpy(orc.outlier_hidden(rng, m, h).astype(np.float32)).to(xdt)
    g = None if gdt is None else torch.from_numpy((1 + 0.1 * rng.standard_normal(h)).astype(np.float32)).to(gdt)
    scales = torch.from_numpy(orc.log_uniform(rng, len(rows)).astype(np.float32))
    return packed, x, g, scales


CASES = [
    # m, h, segment rows, k, x dtype, gamma dtype
    (8, 4096, [4096, 1024, 1024], 4096, torch.bfloat16, torch.bfloat16),   # Llama-3-8B q|k|v
    (8, 4096, [14336, 14336], 4096, torch.bfloat16, torch.bfloat16),       # Llama-3-8B gate|up
    (1, 576, [576, 192, 192], 640, torch.float32, torch.float32),          # SmolLM2 q|k|v, K padded
    (1, 2560, [2560], 2560, torch.bfloat16, torch.float32),                # BitNet-2B o
    (2, 2560, [6912, 6912], 2560, torch.float32, torch.bfloat16),          # BitNet-2B gate|up
    (3, 1536, [1000, 24], 1536, torch.bfloat16, None),                     # ragged tile, no gamma
    (16, 2560, [3200], 2560, torch.bfloat16, torch.bfloat16),              # M = 16
    (7, 4000, [136], 4096, torch.float32, torch.float32),                  # H < K, odd M
    (16, 4096, [4096], 4096, torch.bfloat16, torch.float32),               # M = 16 at K = 4096
    (16, 576, [576, 192, 192], 640, torch.bfloat16, torch.bfloat16),       # 8 rows per wave (2 waves)
    (5, 1024, [2048], 1024, torch.float32, None),                          # K = 1024
    (12, 3072, [128256], 3072, torch.bfloat16, torch.bfloat16),            # tall output, 12 rows
]


@pytest.mark.parametrize("case", CASES, ids=[f"m{c[0]}_h{c[1]}_n{sum(c[2])}_{str(c[4])[6:]}" for c in CASES])
def test_fused_equals_two_calls(pkg, dev, case):
    m, h, rows, k, xdt, gdt = case
    rng = np.random.default_rng(m * 131 + h + sum(rows))
    packed, x, g, scales = (t.to(dev) if t is not None else None for t in _inputs(rng, m, h, rows, k, xdt, gdt))
    y = pkg.rmsnorm_linear(x, g, packed, scales, rows, eps=1e-6)
    q, a_scale = pkg.rmsnorm_quantize_i8(x, g, eps=1e-6, k_pad=k)
    y_ref = pkg.bitnet_linear_segmented(packed, rows, scales, q, a_scale=a_scale)
    assert torch.equal(y, y_ref)


@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_place", [False, True])
def test_fused_residual_equals_two_calls(pkg, dev, rdt, in_place):
    rng = np.random.default_rng(7)
    m, h, n = 8, 4096, 4096
    packed, x, g, scales = (t.to(dev) for t in _inputs(rng, m, h, [n], h, torch.bfloat16, torch.bfloat16))
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(rdt).to(dev)
    q, a_scale = pkg.rmsnorm_quantize_i8(x, g, eps=1e-5)
    y_ref = pkg.bitnet_linear_residual(packed, q, scales, res.clone(), a_scale=a_scale)
    r = res.clone()
    y = pkg.rmsnorm_linear(x, g, packed, scales, eps=1e-5, residual=r, out=r if in_place else None)
    assert torch.equal(y, y_ref)
    if in_place:
        assert y.data_ptr() == r.data_ptr()


def test_fused_matches_oracle(pkg, dev):
    rng = np.random.default_rng(99)
    m, h, rows = 4, 2560, [2560, 640]
    packed, x, g, scales = _inputs(rng, m, h, rows, h, torch.float32, torch.float32)
    y = pkg.rmsnorm_linear(x.to(dev), g.to(dev), packed.to(dev), scales.to(dev), rows, eps=1e-6, out_dtype=torch.float32)
    q_ref, s_ref = orc.rmsnorm_quant(x.numpy(), g.numpy(), 1e-6)
    acc = (q_ref.astype(np.float32) @ orc.unpack_i2s(packed.numpy()).astype(np.float32).T).astype(np.int64)
    y_ref = orc.rescale_segmented(acc, rows, scales.numpy(), s_ref)
    assert np.array_equal(y.cpu().numpy(), y_ref)


ONE_TOKEN_CASES = [
    # h, rows, k, x dtype, gamma dtype, residual dtype: one token (the GEMV prologue; the quantiser's
    # one-wave order up to 4096 elements, its 256-thread order beyond)
    (4096, [4096, 1024, 1024], 4096, torch.bfloat16, torch.bfloat16, None),   # Llama-3-8B q|k|v (8 waves)
    (4096, [4096], 4096, torch.bfloat16, torch.bfloat16, torch.bfloat16),     # Llama-3-8B o + residual
    (2560, [2560, 640, 640], 2560, torch.bfloat16, torch.bfloat16, None),     # BitNet-2B q|k|v (5 waves)
    (576, [576], 640, torch.float32, None, torch.float32),                    # SmolLM2 o, K padded (2 waves)
    (1536, [576], 1536, torch.bfloat16, torch.float32, torch.bfloat16),       # SmolLM2 down (3 waves)
    (256, [104, 24], 256, torch.bfloat16, torch.bfloat16, None),              # one wave, two segments
    (4000, [136], 4224, torch.float32, torch.bfloat16, None),                 # H <= 4096 < K: one-wave order, 16 lanes
    (14336, [4096], 14336, torch.float32, torch.bfloat16, torch.bfloat16),    # Llama-3-8B down (fp32 gated row)
    (6912, [2560], 6912, torch.float32, torch.bfloat16, torch.bfloat16),      # BitNet-2B down
    (5000, [296, 40], 5120, torch.bfloat16, torch.float32, None),             # H < K, two segments, ragged rows
    (16384, [256], 16384, torch.bfloat16, None, torch.float32),               # longest rows, no gamma
    (4104, [1000], 4224, torch.float32, torch.float32, None),                 # shortest long rows
]


@pytest.mark.parametrize("case", ONE_TOKEN_CASES,
                         ids=[f"h{c[0]}_n{sum(c[1])}_k{c[2]}_{str(c[3])[6:]}" for c in ONE_TOKEN_CASES])
def test_fused_one_token_equals_two_calls_and_oracle(pkg, dev, case):
    """One token: codes formed in the decode GEMV's prologue in the quantiser's order for the row length,
    so outputs equal wfb_rmsnorm_quant_i8 + the linear bit for bit, and the oracle."""
    h, rows, k, xdt, gdt, rdt = case
    rng = np.random.default_rng(h + k + sum(rows))
    packed, x, g, scales = (t.to(dev) if t is not None else None for t in _inputs(rng, 1, h, rows, k, xdt, gdt))
    assert pkg.rmsnorm_linear_supported(1, h, k) and pkg.rmsnorm_linear_supported(2, h, k) == (k <= 4096)
    q, a_scale = pkg.rmsnorm_quantize_i8(x, g, eps=1e-6, k_pad=k)
    if rdt is None:
        y = pkg.rmsnorm_linear(x, g, packed, scales, rows, eps=1e-6, out_dtype=torch.float32)
        y_ref = pkg.bitnet_linear_segmented(packed, rows, scales, q, a_scale=a_scale, out_dtype=torch.float32)
    else:
        res = torch.from_numpy(rng.standard_normal((1, sum(rows))).astype(np.float32)).to(rdt).to(dev)
        y = pkg.rmsnorm_linear(x, g, packed, scales, eps=1e-6, residual=res.clone())
        y_ref = pkg.bitnet_linear_residual(packed, q, scales, res.clone(), a_scale=a_scale)
    assert torch.equal(y, y_ref)
    q_ref, s_ref = orc.rmsnorm_quant(x.float().cpu().numpy(), None if g is None else g.float().cpu().numpy(), 1e-6,
                                     k_pad=k)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(a_scale.cpu().numpy(), s_ref)
    if rdt is None:
        acc = (q_ref.astype(np.float32) @ orc.unpack_i2s(packed.cpu().numpy()).astype(np.float32).T).astype(np.int64)
        assert np.array_equal(y.cpu().numpy(), orc.rescale_segmented(acc, rows, scales.cpu().numpy(), s_ref))


def test_fused_rejects_unsupported_sizes(pkg, dev):
    packed = torch.zeros((64, 1024), dtype=torch.uint8, device=dev)
    sc = torch.ones(1, device=dev)
    with pytest.raises(RuntimeError, match="fused path"):
        pkg.rmsnorm_linear(torch.zeros((17, 4096), device=dev), None, packed, sc)
    with pytest.raises(RuntimeError, match="fused path"):
        pkg.rmsnorm_linear(torch.zeros((2, 4100), device=dev), None, torch.zeros((64, 1280), dtype=torch.uint8, device=dev), sc)
    assert not pkg.rmsnorm_linear_supported(17, 4096, 4096) and pkg.rmsnorm_linear_supported(16, 4096, 4096)


GLU_CASES = [
    # m, h, half, k, x dtype, gamma dtype, act, mid dtype
    (8, 4096, 14336, 4096, torch.bfloat16, torch.bfloat16, "silu", torch.bfloat16),   # Llama-3-8B gate|up
    (4, 4096, 14336, 4096, torch.bfloat16, torch.float32, "silu", torch.bfloat16),
    (16, 4096, 14336, 4096, torch.float32, torch.float32, "silu", torch.float32),
    (1, 2560, 6912, 2560, torch.bfloat16, torch.bfloat16, "relu2", torch.bfloat16),   # BitNet-2B gate|up
    (3, 2560, 6912, 2560, torch.float32, torch.bfloat16, "relu2", torch.float32),
    (16, 2560, 6912, 2560, torch.bfloat16, None, "relu2", torch.bfloat16),
    (1, 576, 1536, 640, torch.float32, torch.float32, "silu", torch.float32),         # SmolLM2, K padded
    (9, 1000, 96, 1024, torch.bfloat16, torch.bfloat16, "silu", torch.bfloat16),      # H < K, ragged tiles
    # one token: the GEMV's gated form (gate rows and their up rows in one workgroup)
    (1, 4096, 14336, 4096, torch.bfloat16, torch.bfloat16, "silu", torch.bfloat16),   # Llama-3-8B, 16 + 16 rows
    (1, 1000, 96, 1024, torch.float32, None, "relu2", torch.float32),                 # H < K, 6 workgroups
    (1, 256, 32, 256, torch.bfloat16, torch.bfloat16, "silu", torch.bfloat16),        # one wave, one workgroup
]


@pytest.mark.parametrize("case", GLU_CASES, ids=[f"m{c[0]}_h{c[1]}_half{c[2]}_{c[6]}_{str(c[4])[6:]}" for c in GLU_CASES])
def test_fused_glu_equals_two_calls(pkg, dev, case):
    m, h, half, k, xdt, gdt, act, mid = case
    rng = np.random.default_rng(m * 17 + h + half)
    packed, x, g, scales = (t.to(dev) if t is not None else None
                            for t in _inputs(rng, m, h, [half, half], k, xdt, gdt))
    y = pkg.rmsnorm_linear_glu(x, g, packed, scales, act, eps=1e-6, mid_dtype=mid)
    q, a_scale = pkg.rmsnorm_quantize_i8(x, g, eps=1e-6, k_pad=k)
    y_ref = pkg.bitnet_linear_glu(packed, scales, q, act, a_scale=a_scale, mid_dtype=mid)
    assert torch.equal(y, y_ref)


@pytest.mark.parametrize("m", [5, 1])
def test_fused_glu_matches_oracle(pkg, dev, m):
    rng = np.random.default_rng(5 + m)
    h, half = 2560, 640
    packed, x, g, scales = _inputs(rng, m, h, [half, half], h, torch.float32, torch.float32)
    y = pkg.rmsnorm_linear_glu(x.to(dev), g.to(dev), packed.to(dev), scales.to(dev), "relu2", eps=1e-6,
                               mid_dtype=torch.float32)
    q_ref, s_ref = orc.rmsnorm_quant(x.numpy(), g.numpy(), 1e-6)
    acc = orc.accumulate(packed.numpy(), q_ref)
    yy = orc.rescale_segmented(acc, [half, half], scales.numpy(), s_ref)
    y_ref = orc.glu(yy[:, :half], yy[:, half:], orc.ACT_RELU2)
    assert np.array_equal(y.cpu().numpy(), y_ref)
