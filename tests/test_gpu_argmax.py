"""Greedy decoding on the device: ternary LM head + argmax (exact, against the oracle's logits) and the
dense LM head with the final RMSNorm fused (floating point, against a float64 torch reference)."""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu


def _packed(rng, n, k):
    return orc.pack_i2s(orc.random_ternary(rng, n, k))


def _first_argmax(x):
    return np.argmax(x, axis=-1)  # numpy returns the first maximum, as std::max_element


# (1, 70000, 4096), (2, 40000, 2560): the GEMV with activation fragments from global memory (grids above
# 2048 workgroups); (8, 128256, 4096), (3, 40000, 2560), (5, 33000, 1024), (12, 65543, 2560), (16, 49152, 4096),
# (6, 34000, 2048), (9, 33100, 1536): the persistent head kernel (8, 5, 2, 4 and 4 waves per workgroup)
# (>= 32768 rows, up to 16 tokens), one-shot elsewhere; (17, 3000, 512), (32, 20000, 2560), (24, 4096, 4096):
# two token tiles per weight fragment; (40, 40000, 2560), (64, 33000, 1024), (17, 32768, 512): more than 16
# tokens on 32768+ rows, in chunks of 16 tokens through the persistent kernel
@pytest.mark.parametrize("m,n,k", [(1, 1000, 256), (2, 5000, 640), (1, 70000, 4096), (2, 40000, 2560),
                                   (3, 4099, 2560), (8, 128256, 4096),
                                   (3, 40000, 2560), (5, 33000, 1024), (12, 65543, 2560), (16, 49152, 4096),
                                   (6, 34000, 2048), (9, 33100, 1536), (17, 3000, 512), (32, 20000, 2560), (24, 4096, 4096), (64, 2048, 384),
                                   (40, 40000, 2560), (64, 33000, 1024), (17, 32768, 512)])
@pytest.mark.parametrize("ldt", [torch.float32, torch.bfloat16])
def test_ternary_head_argmax_matches_oracle(pkg, dev, m, n, k, ldt):
    rng = np.random.default_rng(m * 1000 + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    ws, a_scale = orc.log_uniform(rng), orc.log_uniform(rng, m)
    pw, at, st = torch.from_numpy(packed).to(dev), torch.from_numpy(a).to(dev), torch.from_numpy(a_scale).to(dev)
    tok, logits = pkg.bitnet_linear_argmax(pw, at, float(ws), a_scale=st, logits_dtype=ldt, return_logits=True)
    y_ref = pkg.bitnet_linear(pw, at, float(ws), a_scale=st, out_dtype=ldt)
    assert torch.equal(logits, y_ref)  # the stored logits are the plain linear's, bit for bit
    # exact accumulators through an fp32 GEMM of the unpacked weights (partial sums < 2^24)
    acc = (a.astype(np.float32) @ orc.unpack_i2s(packed).astype(np.float32).T).astype(np.int64)
    y = orc.rescale(acc, np.float32(ws), a_scale)
    yt = torch.from_numpy(y)
    if ldt == torch.bfloat16:
        yt = yt.to(torch.bfloat16).float()
    assert torch.equal(logits.float().cpu(), yt)
    assert np.array_equal(tok.cpu().numpy(), _first_argmax(yt.numpy()))
    # without stored logits, same tokens
    assert torch.equal(pkg.bitnet_linear_argmax(pw, at, float(ws), a_scale=st, logits_dtype=ldt), tok)


@pytest.mark.parametrize("m,n,k", [(4, 36000, 4096), (8, 33011, 2560), (16, 40000, 1024), (7, 33000, 2048)])
def test_persistent_head_accumulators(pkg, dev, m, n, k):
    """The persistent form of the batched-decode kernel with an accumulator copy (>= 32768 rows): every
    int32 accumulator and fp32 output equal the oracle's."""
    rng = np.random.default_rng(m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    ws, a_scale = orc.log_uniform(rng), orc.log_uniform(rng, m)
    y, acc = pkg.bitnet_linear(torch.from_numpy(packed).to(dev), torch.from_numpy(a).to(dev), float(ws),
                               a_scale=torch.from_numpy(a_scale).to(dev), out_dtype=torch.float32, return_acc=True)
    acc_ref = (a.astype(np.float32) @ orc.unpack_i2s(packed).astype(np.float32).T).astype(np.int64)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), acc_ref)
    assert np.array_equal(y.cpu().numpy(), orc.rescale(acc_ref, np.float32(ws), a_scale))


def test_ternary_head_argmax_ties_pick_first(pkg, dev):
    rng = np.random.default_rng(3)
    n, k = 777, 512
    w = orc.random_ternary(rng, n, k)
    w[[40, 41, 500]] = 1     # three identical rows of all +1 ...
    a = np.abs(orc.random_int8(rng, 2, k)).astype(np.int8)  # ... with non-negative activations win
    a[1] = 0                 # all logits 0 -> row 0
    tok = pkg.bitnet_linear_argmax(torch.from_numpy(orc.pack_i2s(w)).to(dev), torch.from_numpy(a).to(dev), 0.5)
    assert tok.cpu().tolist() == [40, 0]


def _dense_ref(x, w, g, eps):
    """float64 reference of the fused dense head (norm rounded to x.dtype like the torch glue)."""
    x32 = x.float()
    y = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    if g is not None:
        y = y * g.float()
    y = y.to(x.dtype).double()
    return y @ w.double().T


@pytest.mark.parametrize("m,n,h,xdt,wdt", [
    (1, 49152, 576, torch.float32, torch.float32),     # SmolLM2-135M tied head, fp32 model
    (1, 49152, 576, torch.bfloat16, torch.bfloat16),   # bf16 model
    (8, 49152, 576, torch.bfloat16, torch.bfloat16),   # batch 8
    (4, 1000, 4096, torch.float32, torch.bfloat16),
    (16, 3001, 1024, torch.bfloat16, torch.float32),
    (3, 17, 64, torch.float32, torch.float32),
])
def test_dense_head_argmax_matches_torch(pkg, dev, m, n, h, xdt, wdt):
    gen = torch.Generator().manual_seed(m + n + h)
    x = (torch.randn((m, h), generator=gen) * 3).to(xdt)
    w = (torch.randn((n, h), generator=gen) * 0.02).to(wdt)
    g = (1 + 0.1 * torch.randn(h, generator=gen)).to(xdt)
    ref = _dense_ref(x, w, g, 1e-5)
    tok, logits = pkg.lm_head_argmax(x.to(dev), w.to(dev), g.to(dev), eps=1e-5, return_logits=True)
    lg = logits.cpu().double()
    # fp32 accumulation over h terms; the norm output may differ from torch's by one rounding of x.dtype
    tol = (1e-5 if xdt == torch.float32 else 1e-2) * float(ref.abs().max()) + 1e-6
    assert float((lg - ref).abs().max()) <= tol
    # the token is the first maximum of the kernel's own logits, and the reference's wherever the
    # reference's top two are further apart than the tolerance
    assert np.array_equal(tok.cpu().numpy(), _first_argmax(logits.cpu().numpy()))
    top2 = torch.topk(ref, 2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * tol
    assert torch.equal(tok.cpu()[clear], ref.argmax(-1)[clear])
    assert torch.equal(pkg.lm_head_argmax(x.to(dev), w.to(dev), g.to(dev), eps=1e-5), tok)


def test_dense_head_argmax_ties_pick_first(pkg, dev):
    gen = torch.Generator().manual_seed(1)
    w = torch.randn((300, 128), generator=gen) * 0.01
    w[77] = w[211] = w[299] = 1.0  # identical best rows for a positive x
    x = torch.rand((2, 128), generator=gen) + 0.5
    tok = pkg.lm_head_argmax(x.to(dev), w.to(dev), None, eps=1e-5)
    assert tok.cpu().tolist() == [77, 77]


def test_argmax_errors(pkg, dev):
    w = torch.zeros((100, 64), device=dev)
    with pytest.raises(RuntimeError, match="M"):
        pkg.lm_head_argmax(torch.zeros((17, 64), device=dev), w)
    with pytest.raises(RuntimeError, match="weight"):
        pkg.lm_head_argmax(torch.zeros((1, 64), device=dev), torch.zeros((100, 32), device=dev))
    pw = torch.zeros((64, 32), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="M"):
        pkg.bitnet_linear_argmax(pw, torch.zeros((65, 128), dtype=torch.int8, device=dev), 1.0)
    with pytest.raises(RuntimeError, match="workspace"):
        pkg.bitnet_linear_argmax(pw, torch.zeros((2, 128), dtype=torch.int8, device=dev), 1.0,
                                 workspace=torch.zeros(3, dtype=torch.int64, device=dev))
