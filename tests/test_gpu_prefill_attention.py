"""Causal GQA prefill attention kernel (wfb_gqa_prefill_attention) against a float64 CPU reference.

The cache writes are exact: the rotary embedding uses the same fp32 operations as the torch formula,
rounded to bf16, so the appended keys must equal torch's bit for bit and every other cache row must be
left untouched.  The attention output is floating point (bf16 operands on the matrix cores, fp32
scores and softmax, probabilities as two bf16 parts, output rounded to bf16) and is held to the 1e-2
relative bar of the BitLinear path per element and a 2e-3 mean.  Cache rows before ``start`` hold an
earlier context that must be attended; rows after the chunk hold random values that must not leak.
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _tables(max_len, d, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.arange(max_len, dtype=torch.float32)[:, None] * inv[None, :]
    return freqs.cos(), freqs.sin()


def _rope_torch(x32, cos_rows, sin_rows):
    """HF rotate-half form in fp32: x32 [T, H, D], cos/sin rows [T, D/2]."""
    c = torch.cat([cos_rows, cos_rows], dim=-1)[:, None, :]
    s = torch.cat([sin_rows, sin_rows], dim=-1)[:, None, :]
    half = x32.shape[-1] // 2
    rot = torch.cat([-x32[..., half:], x32[..., :half]], dim=-1)
    return x32 * c + rot * s


def _reference(q, k_new, v_new, kc, vc, start, t, cos, sin, hq, scale):
    """(out float64 [B*T, hq*D], expected k cache, expected v cache) on the CPU."""
    b, hkv, _, d = kc.shape
    g = hq // hkv
    kc_ref, vc_ref = kc.clone(), vc.clone()
    out = torch.zeros((b * t, hq * d), dtype=torch.float64)
    for i in range(b):
        qb = q[i * t:(i + 1) * t].reshape(t, hq, d).float()
        kb = k_new[i * t:(i + 1) * t].reshape(t, hkv, d).float()
        if cos is not None:
            qb = _rope_torch(qb, cos[start:start + t], sin[start:start + t])
            kb = _rope_torch(kb, cos[start:start + t], sin[start:start + t])
        qb = qb.to(torch.bfloat16).double()
        kc_ref[i, :, start:start + t] = kb.to(torch.bfloat16).transpose(0, 1)
        vc_ref[i, :, start:start + t] = v_new[i * t:(i + 1) * t].reshape(t, hkv, d).transpose(0, 1)
        n = start + t
        allowed = torch.arange(n)[None, :] <= (start + torch.arange(t))[:, None]  # [T, n]
        for kv in range(hkv):
            keys, vals = kc_ref[i, kv, :n].double(), vc_ref[i, kv, :n].double()
            for r in range(g):
                h = kv * g + r
                s = (qb[:, h] @ keys.T) * scale
                s = s.masked_fill(~allowed, float("-inf"))
                out[i * t:(i + 1) * t, h * d:(h + 1) * d] = torch.softmax(s, dim=1) @ vals
    return out, kc_ref, vc_ref


CASES = [
    # b, hq, hkv, d, max_len, start, t, rope
    (2, 32, 8, 128, 300, 0, 256, True),     # Llama-3-8B heads, whole 64-key blocks
    (2, 8, 2, 128, 100, 0, 37, True),       # partial query block
    (3, 9, 3, 64, 160, 11, 20, True),       # SmolLM2-135M heads (G = 3), earlier context
    (1, 4, 4, 128, 200, 70, 65, False),     # G = 1, no rotary, chunk across key blocks
    (2, 16, 2, 64, 90, 5, 1, True),         # G = 8, one token
    (1, 10, 2, 128, 200, 0, 130, True),     # G = 5
    (2, 14, 2, 64, 140, 63, 70, True),      # G = 7, start on a block edge - 1
    (1, 4, 2, 128, 80, 0, 33, True),        # G = 2
    (1, 12, 2, 64, 100, 9, 40, True),       # G = 6
]


@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}_h{c[1]}x{c[2]}_d{c[3]}_s{c[5]}_t{c[6]}" for c in CASES])
@pytest.mark.parametrize("strided", [False, True], ids=["contig", "slices"])
def test_prefill_attention_matches_reference(pkg, dev, case, strided):
    b, hq, hkv, d, max_len, start, t, rope = case
    print(f"[prefill attention] case={case} strided={strided}", flush=True)
    gen = torch.Generator().manual_seed(hash(case) % 1000)
    qkv = torch.randn((b * t, (hq + 2 * hkv) * d), generator=gen).to(torch.bfloat16)
    q, k_new, v_new = qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
    kc = torch.randn((b, hkv, max_len, d), generator=gen).to(torch.bfloat16)
    vc = torch.randn((b, hkv, max_len, d), generator=gen).to(torch.bfloat16)
    cos, sin = _tables(max_len, d) if rope else (None, None)
    scale = 1.0 / math.sqrt(d)
    ref, kc_ref, vc_ref = _reference(q, k_new, v_new, kc, vc, start, t, cos, sin, hq, scale)

    kc_d, vc_d = kc.to(dev), vc.to(dev)
    tabs = (cos.to(dev), sin.to(dev)) if rope else (None, None)
    if strided:
        qkv_d = qkv.to(dev)
        qd, kd, vd = qkv_d[:, :hq * d], qkv_d[:, hq * d:(hq + hkv) * d], qkv_d[:, (hq + hkv) * d:]
    else:
        qd, kd, vd = q.contiguous().to(dev), k_new.contiguous().to(dev), v_new.contiguous().to(dev)
    out = pkg.gqa_prefill_attention(qd, kd, vd, kc_d, vc_d, start, t, *tabs, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(kc_d.cpu(), kc_ref), "key cache differs (appended rows or untouched rows)"
    assert torch.equal(vc_d.cpu(), vc_ref), "value cache differs"
    got = out.cpu().double()
    assert got.shape == ref.shape
    err = (got - ref).abs() / ref.abs().clamp_min(1e-2)
    assert float(err.max()) <= 1e-2, float(err.max())
    assert float(err.mean()) <= 2e-3, float(err.mean())


def test_prefill_attention_unaligned_key_value_rows(pkg, dev):
    """Key / value rows that are not 16-byte aligned take the element-wise append path: same caches
    and output as the aligned call."""
    b, hq, hkv, d, max_len, t = 2, 8, 2, 64, 48, 21
    gen = torch.Generator().manual_seed(11)
    q = torch.randn((b * t, hq * d), generator=gen).to(torch.bfloat16).to(dev)
    kv = torch.randn((b * t, 1 + 2 * hkv * d), generator=gen).to(torch.bfloat16).to(dev)
    k_odd, v_odd = kv[:, 1:1 + hkv * d], kv[:, 1 + hkv * d:]  # 2 bytes past a 16-byte boundary
    cos, sin = (x.to(dev) for x in _tables(max_len, d))
    caches = [torch.zeros((b, hkv, max_len, d), dtype=torch.bfloat16, device=dev) for _ in range(4)]
    out_odd = pkg.gqa_prefill_attention(q, k_odd, v_odd, caches[0], caches[1], 3, t, cos, sin)
    out_al = pkg.gqa_prefill_attention(q, k_odd.contiguous(), v_odd.contiguous(), caches[2], caches[3], 3, t, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    assert torch.equal(out_odd, out_al)


def test_prefill_then_decode_continues_the_cache(pkg, dev):
    """A prefill chunk followed by decode steps over the same cache equals one longer prefill."""
    b, hq, hkv, d, max_len = 2, 8, 2, 128, 64
    gen = torch.Generator().manual_seed(3)
    qkv = torch.randn((b, 24, (hq + 2 * hkv) * d), generator=gen).to(torch.bfloat16).to(dev)
    cos, sin = (x.to(dev) for x in _tables(max_len, d))
    kc1 = torch.zeros((b, hkv, max_len, d), dtype=torch.bfloat16, device=dev)
    vc1 = torch.zeros_like(kc1)
    rows = qkv.reshape(b * 24, -1)
    whole = pkg.gqa_prefill_attention(rows[:, :hq * d], rows[:, hq * d:(hq + hkv) * d], rows[:, (hq + hkv) * d:],
                                      kc1, vc1, 0, 24, cos, sin).reshape(b, 24, -1)
    kc2 = torch.zeros_like(kc1)
    vc2 = torch.zeros_like(kc1)
    first = qkv[:, :20].reshape(b * 20, -1)
    part = pkg.gqa_prefill_attention(first[:, :hq * d], first[:, hq * d:(hq + hkv) * d], first[:, (hq + hkv) * d:],
                                     kc2, vc2, 0, 20, cos, sin).reshape(b, 20, -1)
    second = qkv[:, 20:].reshape(b * 4, -1)
    rest = pkg.gqa_prefill_attention(second[:, :hq * d], second[:, hq * d:(hq + hkv) * d],
                                     second[:, (hq + hkv) * d:], kc2, vc2, 20, 4, cos, sin).reshape(b, 4, -1)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(whole[:, :20], part)  # the same queries over the same keys: the same launch shape
    diff = (whole[:, 20:].float() - rest.float()).abs()
    assert float(diff.max()) <= 1e-2 * float(whole[:, 20:].float().abs().max())


def test_prefill_attention_python_errors(pkg, dev):
    kc = torch.zeros((1, 2, 32, 64), dtype=torch.bfloat16, device=dev)
    q = torch.zeros((4, 8 * 64), dtype=torch.bfloat16, device=dev)
    kv = torch.zeros((4, 2 * 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="bfloat16"):
        pkg.gqa_prefill_attention(q.float(), kv.float(), kv.float(), kc.float(), kc.float(), 0, 4)
    with pytest.raises(RuntimeError, match="within max_len"):
        pkg.gqa_prefill_attention(q, kv, kv, kc, kc.clone(), 30, 4)
    with pytest.raises(RuntimeError, match="rope"):
        pkg.gqa_prefill_attention(q, kv, kv, kc, kc.clone(), 0, 4, torch.zeros((32, 32), device=dev), None)
