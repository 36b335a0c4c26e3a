"""BitLinear as a training drop-in: the packed weight follows the float weight, and under autograd the
forward is the reference's straight-through estimator at lambda = 1
(packages/training/src/wrinklefree/models/bitlinear.py:86-113).

Pinned by closed forms: the forward value equals the inference forward bit for bit (same kernels), and
the gradients are those of F.linear at the dequantised operands -- grad_x = g @ (codes_w * s_w),
grad_w = g^T @ (codes_x * s_x), grad_b = sum_m g -- computed here in float64 from the CPU oracle's
codes and scales, and, independently, by torch autograd through the reference's detach formula on the
CPU (x + (q(x) - x).detach(), w + (q(w) - w).detach()).  fp32 GEMM tolerance 1e-5 relative (normwise).
"""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _module(pkg, dev, k, n, bias, seed, dtype=torch.float32):
    torch.manual_seed(seed)
    mod = pkg.BitLinear(k, n, bias=bias).to(dev)
    with torch.no_grad():
        mod.weight.normal_(0, 0.02)
        if bias:
            mod.bias.normal_(0, 0.1)
    return mod.to(dtype)


def test_packed_weight_follows_in_place_updates(pkg, dev):
    """Optimizer steps, copy_ and load_state_dict all change what the next forward computes."""
    k, n, m = 640, 384, 5
    mod = _module(pkg, dev, k, n, False, 1)
    rng = np.random.default_rng(1)
    x = torch.from_numpy(orc.outlier_hidden(rng, m, k)).to(dev)

    def expect(w):  # the absmean of the unpadded weight, then codes of the K-padded one
        s = orc.absmean_scale_device_order(w)
        packed = orc.pack_i2s(orc.ternarize(np.pad(w, ((0, 0), (0, mod.k_pad - k))), s))
        q, a_s = orc.quantize_per_token(x.cpu().numpy(), k_pad=mod.k_pad)
        return orc.rescale(orc.accumulate(packed, q), s, a_s)

    with torch.no_grad():
        y0 = mod(x)
    assert np.array_equal(y0.cpu().numpy(), expect(mod.weight.detach().cpu().numpy()))
    opt = torch.optim.SGD(mod.parameters(), lr=5.0)
    mod(x).square().sum().backward()
    opt.step()
    with torch.no_grad():
        y1 = mod(x)
    assert not torch.equal(y1, y0)
    assert np.array_equal(y1.cpu().numpy(), expect(mod.weight.detach().cpu().numpy()))
    with torch.no_grad():
        mod.weight.copy_(-mod.weight)
        y2 = mod(x)
    assert np.array_equal(y2.cpu().numpy(), expect(mod.weight.detach().cpu().numpy()))
    other = _module(pkg, dev, k, n, False, 7)
    mod.load_state_dict(other.state_dict())
    with torch.no_grad():
        y3 = mod(x)
    assert np.array_equal(y3.cpu().numpy(), expect(other.weight.detach().cpu().numpy()))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("k,n,m", [(640, 384, 5), (576, 200, 17), (1024, 256, 96)])
def test_ste_forward_and_gradients(pkg, dev, k, n, m, bias):
    mod = _module(pkg, dev, k, n, bias, k + n + m)
    rng = np.random.default_rng(k * n + m)
    xn = orc.outlier_hidden(rng, m, k)
    g = rng.standard_normal((m, n)).astype(np.float32)
    x = torch.from_numpy(xn).to(dev).requires_grad_(True)
    y = mod(x)
    assert y.requires_grad and y.dtype == torch.float32
    with torch.no_grad():
        y_inf = mod(x)
    assert torch.equal(y.detach(), y_inf)  # same kernels, same value
    y.backward(torch.from_numpy(g).to(dev))

    w = mod.weight.detach().cpu().numpy()
    s_w = orc.absmean_scale_device_order(w)
    assert s_w == np.float32(mod.weight_scale.item())
    packed = orc.pack_i2s(orc.ternarize(np.pad(w, ((0, 0), (0, mod.k_pad - k))), s_w))
    w_deq = orc.unpack_i2s(packed)[:, :k].astype(np.float64) * np.float64(s_w)
    q, s_x = orc.quantize_per_token(xn, k_pad=mod.k_pad)
    x_deq = q[:, :k].astype(np.float64) * s_x.astype(np.float64)[:, None]
    g64 = g.astype(np.float64)
    assert _rel(x.grad.cpu().numpy(), g64 @ w_deq) <= 1e-5
    assert _rel(mod.weight.grad.cpu().numpy(), g64.T @ x_deq) <= 1e-5
    if bias:
        assert _rel(mod.bias.grad.cpu().numpy(), g64.sum(0)) <= 1e-6

    # the reference's own formula, differentiated by torch on the CPU with the oracle's quantisers
    xt = torch.from_numpy(xn).double().requires_grad_(True)
    wt = torch.from_numpy(w).double().requires_grad_(True)
    xq = xt + (torch.from_numpy(x_deq) - xt).detach()
    wq = wt + (torch.from_numpy(w_deq) - wt).detach()
    torch.nn.functional.linear(xq, wq).backward(torch.from_numpy(g64))
    assert _rel(x.grad.cpu().numpy(), xt.grad.numpy()) <= 1e-5
    assert _rel(mod.weight.grad.cpu().numpy(), wt.grad.numpy()) <= 1e-5


def test_ste_bf16_inputs_and_weights(pkg, dev):
    """bf16 module: bf16 output and gradients in each input's dtype."""
    mod = _module(pkg, dev, 512, 256, True, 3, dtype=torch.bfloat16)
    x = torch.randn(4, 3, 512, device=dev, dtype=torch.bfloat16, requires_grad=True)
    y = mod(x)
    assert y.dtype == torch.bfloat16 and y.shape == (4, 3, 256)
    y.float().square().mean().backward()
    assert x.grad.dtype == torch.bfloat16 and mod.weight.grad.dtype == torch.bfloat16
    assert torch.isfinite(x.grad.float()).all() and torch.isfinite(mod.weight.grad.float()).all()


def test_training_steps_reduce_a_regression_loss(pkg, dev):
    """A few SGD steps through the STE fit a target produced by another ternary layer (loss falls)."""
    torch.manual_seed(11)
    student = _module(pkg, dev, 256, 128, False, 11)
    teacher = _module(pkg, dev, 256, 128, False, 12)
    x = torch.randn(64, 256, device=dev)
    with torch.no_grad():
        target = teacher(x)
    opt = torch.optim.Adam(student.parameters(), lr=2e-3)
    losses = []
    for _ in range(30):
        opt.zero_grad()
        loss = (student(x) - target).square().mean()
        loss.backward()
        opt.step()
        losses.append(float(loss.detach()))
    assert losses[-1] < 0.5 * losses[0]


def test_lambda_warmup_below_one_raises(pkg, dev):
    mod = _module(pkg, dev, 256, 128, False, 5)
    x = torch.randn(2, 256, device=dev)
    pkg.set_lambda_source(lambda: 0.25)
    try:
        with pytest.raises(RuntimeError, match="lambda"):
            mod(x)
    finally:
        pkg.set_lambda_source(None)
    pkg.set_lambda_source(lambda: 1.0)
    try:
        mod(x)
    finally:
        pkg.set_lambda_source(None)


@pytest.mark.parametrize("m,k,n", [(6, 640, 256), (3, 576, 200)])
def test_subln_bitlinear_ste_gradients(pkg, dev, m, k, n):
    """SubLN + BitLinear under autograd: forward equals the no-grad fused forward; gradients equal torch
    autograd of the reference composition (SubLN formula of WF/models/subln.py:42-59 in float64, then
    the STE linear with the oracle's codes of the kernel's normalised rows)."""
    torch.manual_seed(m + k)
    mod = pkg.SubLNBitLinear(k, n).to(dev)
    with torch.no_grad():
        mod.norm_weight.copy_(1 + 0.1 * torch.randn(k))
        mod.linear.weight.normal_(0, 0.02)
    rng = np.random.default_rng(k + n)
    xn = orc.outlier_hidden(rng, m, k)
    g = rng.standard_normal((m, n)).astype(np.float32)
    x = torch.from_numpy(xn).to(dev).requires_grad_(True)
    y = mod(x)
    with torch.no_grad():
        assert torch.equal(y, mod(x))
    y.backward(torch.from_numpy(g).to(dev))

    gam = mod.norm_weight.detach().cpu().numpy()
    w = mod.linear.weight.detach().cpu().numpy()
    s_w = np.float32(mod.linear.weight_scale.item())
    w_deq = orc.unpack_i2s(orc.pack_i2s(orc.ternarize(np.pad(w, ((0, 0), (0, mod.linear.k_pad - k))), s_w)))[:, :k]
    w_deq = w_deq.astype(np.float64) * np.float64(s_w)
    q, s_x = orc.rmsnorm_quant(xn, gam, 1e-6, k_pad=mod.linear.k_pad)
    x_deq = q[:, :k].astype(np.float64) * s_x.astype(np.float64)[:, None]
    xt = torch.from_numpy(xn).double().requires_grad_(True)
    gt = torch.from_numpy(gam).double().requires_grad_(True)
    wt = torch.from_numpy(w).double().requires_grad_(True)
    yn = xt * torch.rsqrt(xt.pow(2).mean(dim=-1, keepdim=True) + 1e-6) * gt
    xq = yn + (torch.from_numpy(x_deq) - yn).detach()
    wq = wt + (torch.from_numpy(w_deq) - wt).detach()
    torch.nn.functional.linear(xq, wq).backward(torch.from_numpy(g.astype(np.float64)))
    assert _rel(x.grad.cpu().numpy(), xt.grad.numpy()) <= 1e-5
    assert _rel(mod.norm_weight.grad.cpu().numpy(), gt.grad.numpy()) <= 1e-5
    assert _rel(mod.linear.weight.grad.cpu().numpy(), wt.grad.numpy()) <= 1e-5
