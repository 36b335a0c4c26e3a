"""GPU parity of the fused decode-layer pieces against the CPU oracle, through the C ABI.

* wfb_linear_i2s_segmented: accumulators and outputs equal to separate wfb_linear_i2s calls on the
  segments (bit-exact, every kernel path: GEMV M <= 2, skinny MFMA, tiled MFMA).
* wfb_glu_rmsnorm_quant_i8: int8 codes and scales bit-exact against the oracle's step-by-step fp32
  restatement (the SiLU is evaluated with the same fixed sequence of correctly rounded operations).
"""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


SEGMENTS = {
    "qkv_2b": ([2560, 320, 320], 2560),
    "gate_up_smollm2": ([1536, 1536], 640),
    "qkv_smollm2": ([576, 192, 192], 640),
    "three_odd": ([8, 24, 104], 256),
}


@pytest.mark.parametrize("case", sorted(SEGMENTS))
@pytest.mark.parametrize("m", [1, 2, 5, 64, 130])
def test_segmented_linear_equals_separate_calls(pkg, dev, case, m):
    rows, k = SEGMENTS[case]
    rng = np.random.default_rng(7000 + m + sum(rows))
    packs = [orc.pack_i2s(orc.random_ternary(rng, r, k)) for r in rows]
    scales = orc.log_uniform(rng, len(rows))
    a = orc.random_int8(rng, m, k)
    a_scale = orc.log_uniform(rng, m)
    packed = np.concatenate(packs, axis=0)
    pw, pa, ps = _t(packed, dev), _t(a, dev), _t(a_scale, dev)
    y, acc = pkg.bitnet_linear_segmented(pw, rows, _t(scales, dev), pa, a_scale=ps, out_dtype=torch.float32,
                                         return_acc=True)
    acc_ref = orc.accumulate(packed, a)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), acc_ref)
    y_ref = orc.rescale_segmented(acc_ref, rows, scales, a_scale)
    assert np.array_equal(y.cpu().numpy(), y_ref)
    # the separate-call form, segment by segment
    r0 = 0
    for p, r, s in zip(packs, rows, scales):
        ys = pkg.bitnet_linear(_t(p, dev), pa, float(s), a_scale=ps, out_dtype=torch.float32)
        assert np.array_equal(ys.cpu().numpy(), y.cpu().numpy()[:, r0:r0 + r])
        r0 += r
    yb = pkg.bitnet_linear_segmented(pw, rows, _t(scales, dev), pa, a_scale=ps)
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y_ref))


def test_segmented_rejects_bad_segments(pkg, dev):
    from wrinklefree_monorepo_amd import _lib
    rng = np.random.default_rng(1)
    packed = _t(orc.pack_i2s(orc.random_ternary(rng, 64, 128)), dev)
    a = _t(orc.random_int8(rng, 1, 128), dev)
    sc = torch.ones(2, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError):
        pkg.bitnet_linear_segmented(packed, [32, 16], sc, a)       # rows do not sum to N
    with pytest.raises(RuntimeError, match="multiple of 8"):
        pkg.bitnet_linear_segmented(packed, [36, 28], sc, a)       # not multiples of 8
    assert "multiple of 8" in _lib.last_error()


GLU_CASES = [(1, 1536), (4, 1536), (1, 6912), (16, 6912), (3, 14336), (64, 2560), (5, 4104)]


@pytest.mark.parametrize("act", ["silu", "relu2"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,h", GLU_CASES)
def test_glu_rmsnorm_quant_matches_oracle(pkg, dev, act, dtype, m, h):
    rng = np.random.default_rng(8000 + m + h)
    gu = (rng.standard_normal((m, 2 * h)) * 2.0).astype(np.float32)
    gu[:, ::97] *= 12.0  # a few large gates (silu tails, relu^2 growth)
    gamma = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    x = _t(gu, dev).to(dtype)
    gate, up = x[:, :h], x[:, h:]  # halves of one gate|up output: common row stride 2H
    g = _t(gamma, dev).to(torch.bfloat16)
    kp = (h + 127) // 128 * 128
    q, s = pkg.glu_rmsnorm_quantize_i8(gate, up, act, g, eps=1e-6, k_pad=kp)
    xin = x.to(torch.float32).cpu().numpy()
    gref = g.to(torch.float32).cpu().numpy()
    code = orc.ACT_SILU if act == "silu" else orc.ACT_RELU2
    q_ref, s_ref = orc.glu_rmsnorm_quant(xin[:, :h], xin[:, h:], code, gref, 1e-6, kp)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_glu_separate_gate_and_up_buffers(pkg, dev):
    rng = np.random.default_rng(9)
    m, h = 3, 2560
    gate = (rng.standard_normal((m, h)) * 3).astype(np.float32)
    up = rng.standard_normal((m, h)).astype(np.float32)
    q, s = pkg.glu_rmsnorm_quantize_i8(_t(gate, dev), _t(up, dev), "silu", None, eps=1e-5)
    q_ref, s_ref = orc.glu_rmsnorm_quant(gate, up, orc.ACT_SILU, None, 1e-5)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_glu_rejects_mismatched_inputs(pkg, dev):
    g = torch.zeros((2, 64), device=dev)
    with pytest.raises(RuntimeError):
        pkg.glu_rmsnorm_quantize_i8(g, torch.zeros((2, 72), device=dev))
    with pytest.raises(ValueError):
        pkg.glu_rmsnorm_quantize_i8(g, g, "gelu")


def test_bitnet_linear_native_module(pkg, dev):
    """BitNetLinearNative (reference bitnet_patch.py:28-78): per-tensor activation scale, fp32 out."""
    rng = np.random.default_rng(11)
    n, k = 256, 640
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, ws = orc.pack_ternary(w)
    bias = rng.standard_normal(n).astype(np.float32)
    mod = pkg.BitNetLinearNative(k, n, _t(packed, dev), torch.tensor([ws], device=dev), _t(bias, dev))
    for m in (1, 5):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = mod(_t(x, dev)).cpu().numpy()
        q, a_s = orc.quantize_per_tensor(x)
        acc = orc.accumulate(packed, q.reshape(m, k))
        y_ref = orc.rescale(acc, ws, np.full(m, a_s, np.float32), bias)
        assert np.array_equal(y, y_ref)


@pytest.mark.parametrize("m,n,k", [(1, 2560, 2560), (8, 4096, 14336), (3, 640, 1024), (200, 2560, 6912), (64, 520, 512),
                                   (300, 1016, 640), (1024, 6144, 512), (2048, 6144, 256), (64, 4096, 4096),
                                   (37, 1024, 4096), (57, 2560, 6912)])
@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16])
def test_linear_residual_matches_oracle(pkg, dev, m, n, k, rdt):
    """out = residual + acc * w_scale * a_scale in one launch (GEMV, skinny and tile kernels): the fp32
    sum of the oracle's rescaled output and the residual, rounded to the residual's dtype; in place too."""
    rng = np.random.default_rng(m + n + k)
    packed = orc.pack_i2s(orc.random_ternary(rng, n, k))
    a = orc.random_int8(rng, m, k)
    ws, a_s = orc.log_uniform(rng), orc.log_uniform(rng, m)
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(rdt)
    acc = (a.astype(np.float32) @ orc.unpack_i2s(packed).astype(np.float32).T).astype(np.int64)
    want = torch.from_numpy(orc.rescale(acc, np.float32(ws), a_s) + res.float().numpy()).to(rdt)
    pw, at, st = (torch.from_numpy(x).to(dev) for x in (packed, a, a_s))
    got = pkg.bitnet_linear_residual(pw, at, float(ws), res.to(dev), a_scale=st)
    assert torch.equal(got.cpu(), want)
    buf = res.to(dev)
    pkg.bitnet_linear_residual(pw, at, float(ws), buf, a_scale=st, out=buf)
    assert torch.equal(buf.cpu(), want)


_TILE_EPI_SHAPES = [(100, 2560, 384), (1024, 6144, 512), (2048, 6144, 256)]


# (300, 1004, 640) has N % 8 != 0, which bf16 rows cannot take (16-byte aligned rows); it runs in fp32.
@pytest.mark.parametrize("m,n,k,odt", [(300, 1004, 640, torch.float32)]
                         + [s + (t,) for s in _TILE_EPI_SHAPES for t in (torch.float32, torch.bfloat16)])
def test_tile_epilogue_out_types_match_oracle(pkg, dev, m, n, k, odt):
    """Prefill tile kernel outputs without an accumulator copy (the staged epilogues: fp32 or bf16, whole
    and partial column groups, 32/64/128-row tiles) equal the oracle's rescale bit for bit."""
    rng = np.random.default_rng(3 * m + n + k)
    packed = orc.pack_i2s(orc.random_ternary(rng, n, k))
    a = orc.random_int8(rng, m, k)
    ws, a_s = orc.log_uniform(rng), orc.log_uniform(rng, m)
    acc = (a.astype(np.float32) @ orc.unpack_i2s(packed).astype(np.float32).T).astype(np.int64)
    want = torch.from_numpy(orc.rescale(acc, np.float32(ws), a_s)).to(odt)
    pw, at, st = (torch.from_numpy(x).to(dev) for x in (packed, a, a_s))
    got = pkg.bitnet_linear(pw, at, float(ws), a_scale=st, out_dtype=odt)
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("h,f,qn,kvn", [(2560, 6912, 2560, 640), (1024, 2816, 1024, 256), (512, 1024, 512, 100)])
def test_reference_fused_mlp_and_qkv_ops(pkg, dev, h, f, qn, kvn):
    """bitnet_mlp_forward / bitnet_qkv_forward (the reference's batch-1 fused ops,
    SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-375, schemas torch_extension_cpu.cpp:921-926) equal the
    oracle chain bit for bit: per-token quantisation, exact accumulators, rescale by each projection's own
    weight scale, relu(gate)^2 * up -> SubLN -> re-quantisation -> down.  Also through torch.ops.wfbitnet."""
    rng = np.random.default_rng(h + f)
    x = orc.outlier_hidden(rng, 1, h)[0]
    xt = torch.from_numpy(x).to(dev)
    # qkv
    ws = [orc.pack_i2s(orc.random_ternary(rng, n, h)) for n in (qn, kvn, kvn)]
    sc = [float(orc.log_uniform(rng)) for _ in range(3)]
    q_ref, s_ref = orc.quantize_per_token(x[None, :])
    outs = pkg.bitnet_qkv_forward(xt, *[torch.from_numpy(w).to(dev) for w in ws], *sc)
    for o, w, s_w in zip(outs, ws, sc):
        want = orc.rescale(orc.accumulate(w, q_ref), s_w, s_ref)[0]
        assert o.dtype == torch.float32 and np.array_equal(o.cpu().numpy(), want)
    outs2 = torch.ops.wfbitnet.bitnet_qkv_forward(xt[None, :], *[torch.from_numpy(w).to(dev) for w in ws], *sc)
    assert all(torch.equal(a, b) for a, b in zip(outs, outs2))
    # the q|k|v concatenation is rebuilt after an in-place update of a weight (same tensor, new version)
    wt = [torch.from_numpy(w).to(dev) for w in ws]
    pkg.bitnet_qkv_forward(xt, *wt, *sc)
    w_new = orc.pack_i2s(orc.random_ternary(rng, kvn, h))
    wt[1].copy_(torch.from_numpy(w_new))
    o_new = pkg.bitnet_qkv_forward(xt, *wt, *sc)[1]
    assert np.array_equal(o_new.cpu().numpy(), orc.rescale(orc.accumulate(w_new, q_ref), sc[1], s_ref)[0])
    # mlp
    gw, uw = (orc.pack_i2s(orc.random_ternary(rng, f, h)) for _ in range(2))
    dw = orc.pack_i2s(orc.random_ternary(rng, h, f))
    gs, us, ds = (float(orc.log_uniform(rng)) for _ in range(3))
    gamma = (1.0 + 0.1 * rng.standard_normal(f)).astype(np.float32)
    gate = orc.rescale(orc.accumulate(gw, q_ref), gs, s_ref)
    up = orc.rescale(orc.accumulate(uw, q_ref), us, s_ref)
    h8, hs = orc.glu_rmsnorm_quant(gate, up, orc.ACT_RELU2, gamma, 1e-5)
    want = orc.rescale(orc.accumulate(dw, h8), ds, hs)[0]
    args = [torch.from_numpy(w).to(dev) for w in (gw, uw, dw)]
    y = pkg.bitnet_mlp_forward(xt, *args, gs, us, ds, torch.from_numpy(gamma).to(dev), 1e-5)
    assert y.shape == (h,) and np.array_equal(y.cpu().numpy(), want)
    y2 = torch.ops.wfbitnet.bitnet_mlp_forward(xt, *args, gs, us, ds, torch.from_numpy(gamma).to(dev), 1e-5)
    assert torch.equal(y, y2)
    with pytest.raises(RuntimeError, match="1D or"):
        pkg.bitnet_mlp_forward(xt.reshape(2, -1), *args, gs, us, ds, torch.from_numpy(gamma).to(dev), 1e-5)
