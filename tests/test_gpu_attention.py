"""GQA decode attention kernel (wfb_gqa_decode_attention) against a plain PyTorch float64 reference.

The kernel is floating point (softmax), so outputs are compared with a tolerance: fp32 outputs within
2e-5 of max|V| (absolute), bf16 outputs within the 1e-2 relative bar of the BitLinear path.  The
cache writes are exact: the rotary embedding uses the same fp32 operations as the torch formula
(x * cos + rotate_half(x) * sin, each op rounded to fp32, then rounded to the storage dtype), so the
appended key must equal torch's bit for bit, and every other cache entry must be left untouched.
Keys beyond each sequence's position hold random values that must not leak into the result.
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _tables(max_len, d, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.arange(max_len, dtype=torch.float32)[:, None] * inv[None, :]
    return freqs.cos(), freqs.sin()


def _rope_torch(x32, cos_row, sin_row):
    """HF rotate-half form in fp32 on rows x32 [..., D] with cos/sin [D/2]."""
    c = torch.cat([cos_row, cos_row])
    s = torch.cat([sin_row, sin_row])
    half = x32.shape[-1] // 2
    rot = torch.cat([-x32[..., half:], x32[..., :half]], dim=-1)
    return x32 * c + rot * s


def _reference(q, k_new, v_new, kc, vc, pos, cos, sin, hq, scale):
    """(out fp64 [B, hq*D], expected k cache, expected v cache), all on the CPU."""
    b, hkv, _, d = kc.shape
    g = hq // hkv
    dt = kc.dtype
    kc_ref, vc_ref = kc.clone(), vc.clone()
    out = torch.zeros((b, hq * d), dtype=torch.float64)
    for i in range(b):
        p = int(pos[i])
        qb = q[i].reshape(hq, d).float()
        kb = k_new[i].reshape(hkv, d).float()
        if cos is not None:
            qb = _rope_torch(qb, cos[p], sin[p]).to(dt).float()
            kb = _rope_torch(kb, cos[p], sin[p]).to(dt).float()
        kc_ref[i, :, p] = kb.to(dt)
        vc_ref[i, :, p] = v_new[i].reshape(hkv, d)
        keys = kc_ref[i, :, :p + 1].double()
        vals = vc_ref[i, :, :p + 1].double()
        for h in range(hq):
            s = keys[h // g] @ qb[h].double() * scale
            out[i, h * d:(h + 1) * d] = torch.softmax(s, dim=0) @ vals[h // g]
    return out, kc_ref, vc_ref


def _run_case(pkg, dev, b, hq, hkv, d, max_len, pos, dtype, rope, strided=False, seed=0, split=True):
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn((b, (hq + 2 * hkv) * d), generator=gen).to(dtype)
    q, k_new, v_new = qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
    kc = torch.randn((b, hkv, max_len, d), generator=gen).to(dtype)
    vc = torch.randn((b, hkv, max_len, d), generator=gen).to(dtype)
    cos, sin = _tables(max_len, d) if rope else (None, None)
    scale = 1.0 / math.sqrt(d)
    ref, kc_ref, vc_ref = _reference(q, k_new, v_new, kc, vc, pos, cos, sin, hq, scale)

    kc_d, vc_d = kc.to(dev), vc.to(dev)
    pos_d = torch.tensor(pos, dtype=torch.int64, device=dev)
    tabs = (cos.to(dev), sin.to(dev)) if rope else (None, None)
    if strided:  # column slices of one q|k|v buffer
        qkv_d = qkv.to(dev)
        qd, kd, vd = qkv_d[:, :hq * d], qkv_d[:, hq * d:(hq + hkv) * d], qkv_d[:, (hq + hkv) * d:]
    else:
        qd, kd, vd = q.contiguous().to(dev), k_new.contiguous().to(dev), v_new.contiguous().to(dev)
    out = pkg.gqa_decode_attention(qd, kd, vd, kc_d, vc_d, pos_d, *tabs, scale=scale, split=split)
    torch.cuda.synchronize()
    assert torch.equal(kc_d.cpu(), kc_ref), "key cache differs (appended row or untouched rows)"
    assert torch.equal(vc_d.cpu(), vc_ref), "value cache differs"
    got = out.cpu().double()
    if dtype == torch.float32:
        tol = 2e-5 * float(vc.abs().max())
        assert float((got - ref).abs().max()) <= tol
    else:
        err = (got - ref).abs() / ref.abs().clamp_min(1e-2)
        assert float(err.max()) <= 1e-2
    return out


CASES = [
    # b, hq, hkv, d, max_len, pos, dtype, rope
    (1, 9, 3, 64, 160, [159], torch.float32, True),                                    # SmolLM2-135M shape
    (8, 32, 8, 128, 512, [0, 1, 255, 256, 257, 300, 511, 17], torch.bfloat16, True),   # Llama-3-8B shape
    (2, 4, 4, 128, 300, [128, 299], torch.float32, False),                             # G = 1, no rope
    (3, 16, 2, 64, 1100, [1099, 0, 640], torch.float32, True),                         # G = 8, 9 chunks
    (2, 10, 2, 128, 700, [699, 383], torch.bfloat16, True),                            # G = 5
    (2, 12, 2, 64, 520, [511, 512], torch.bfloat16, False),                            # G = 6, chunk edges
    (1, 7, 1, 128, 129, [127], torch.float32, True),                                   # G = 7
    (4, 2, 1, 64, 40, [3, 39, 0, 20], torch.bfloat16, True),                           # G = 2
    (8, 16, 8, 128, 1100, [1099, 0, 63, 64, 255, 256, 700, 1023], torch.bfloat16, True),  # split edges, G = 2
    (8, 8, 8, 64, 1100, [1099, 511, 512, 0, 128, 129, 1000, 7], torch.float32, True),    # fp32, G = 1
    # 513 64-key splits x G = 8 heads pass the combine's 4096 split-heads, so splits double to 128 keys
    # while a bf16 chunk stays 256 keys: a chunk of a split that does not own pos reaches key pos
    (4, 8, 1, 64, 32832, [200, 127, 128, 32831], torch.bfloat16, True),
    (2, 8, 1, 128, 32832, [383, 32700], torch.float32, True),                           # fp32, 128-key splits
    # 64 sequence-heads: split length from each sequence's position (64 .. 512 keys, 1 .. 8 prefetched
    # chunks, partial last splits)
    (8, 32, 8, 128, 4100, [4099, 3000, 2047, 2048, 1023, 767, 768, 5], torch.bfloat16, True),
    # 776 sequence-heads (more than the 768 live-split target): one split per sequence, all its keys
    (97, 16, 8, 64, 200, [(37 * i + 11) % 200 for i in range(97)], torch.bfloat16, True),
    # position-scaled splits with G = 8 (the matrix-core scores' heads 4..7 in the second lane group) and
    # with G = 3 at head_dim 64 (two 32-dimension steps per score tile)
    (16, 64, 8, 128, 2100, [2099, 1500, 640, 64, 63, 0, 1000, 2047, 1, 700, 1999, 128, 129, 300, 1700, 900],
     torch.bfloat16, True),
    (64, 9, 3, 64, 600, [(53 * i + 7) % 600 for i in range(64)], torch.bfloat16, True),
]


@pytest.mark.parametrize("split", [True, False], ids=["split", "single"])
@pytest.mark.parametrize("case", CASES, ids=[f"b{c[0]}_h{c[1]}x{c[2]}_d{c[3]}_L{c[4]}_{str(c[6])[6:]}" for c in CASES])
def test_decode_attention_matches_torch(pkg, dev, case, split):
    """Both forms: key splits on separate workgroups merged by the combine kernel (split; 64-key splits,
    doubled while splits x query heads would pass the combine's 4096, and with the position once the
    batch's sequence-heads would hold more than 768 splits), and one workgroup per (kv head, sequence)
    over all keys (single)."""
    b, hq, hkv, d, max_len, pos, dtype, rope = case
    _run_case(pkg, dev, b, hq, hkv, d, max_len, pos, dtype, rope, seed=hq * 7 + max_len, split=split)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_attention_strided_projection_slices(pkg, dev, dtype):
    _run_case(pkg, dev, 3, 8, 2, 128, 96, [95, 10, 50], dtype, True, strided=True, seed=3)


def test_decode_attention_successive_steps(pkg, dev):
    """Eight decode steps appending to one cache: after each, the output matches attention over the
    reference cache built by the same appends."""
    b, hq, hkv, d, max_len = 2, 6, 2, 64, 48
    gen = torch.Generator().manual_seed(11)
    kc = torch.randn((b, hkv, max_len, d), generator=gen)
    vc = torch.randn((b, hkv, max_len, d), generator=gen)
    cos, sin = _tables(max_len, d)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    tabs = (cos.to(dev), sin.to(dev))
    pos = [20, 30]
    for step in range(8):
        q = torch.randn((b, hq * d), generator=gen)
        kn = torch.randn((b, hkv * d), generator=gen)
        vn = torch.randn((b, hkv * d), generator=gen)
        ref, kc, vc = _reference(q, kn, vn, kc, vc, pos, cos, sin, hq, 1 / 8)
        out = pkg.gqa_decode_attention(q.to(dev), kn.to(dev), vn.to(dev), kc_d, vc_d,
                                       torch.tensor(pos, device=dev), *tabs, scale=1 / 8)
        assert torch.equal(kc_d.cpu(), kc) and torch.equal(vc_d.cpu(), vc), f"step {step}"
        assert float((out.cpu().double() - ref).abs().max()) <= 2e-5 * float(vc.abs().max()), f"step {step}"
        pos = [p + 1 for p in pos]


def test_decode_attention_position_out_of_range(pkg, dev):
    """A device position outside [0, max_len) is caught by the kernel: NaN output rows for that
    sequence, its cache untouched; the other sequences are computed normally."""
    b, hq, hkv, d, max_len = 3, 4, 2, 64, 32
    gen = torch.Generator().manual_seed(5)
    q = torch.randn((b, hq * d), generator=gen)
    kn = torch.randn((b, hkv * d), generator=gen)
    vn = torch.randn((b, hkv * d), generator=gen)
    kc = torch.randn((b, hkv, max_len, d), generator=gen)
    vc = torch.randn((b, hkv, max_len, d), generator=gen)
    for split in (True, False):
        kc_d, vc_d = kc.to(dev), vc.to(dev)
        out = pkg.gqa_decode_attention(q.to(dev), kn.to(dev), vn.to(dev), kc_d, vc_d,
                                       torch.tensor([max_len, 5, -1], device=dev), split=split)
        o = out.cpu()
        assert torch.isnan(o[0]).all() and torch.isnan(o[2]).all() and not torch.isnan(o[1]).any()
        assert torch.equal(kc_d.cpu()[0], kc[0]) and torch.equal(kc_d.cpu()[2], kc[2])
        assert torch.equal(vc_d.cpu()[0], vc[0]) and torch.equal(vc_d.cpu()[2], vc[2])


def test_decode_attention_python_errors(pkg, dev):
    kc = torch.zeros((1, 2, 16, 64), device=dev)
    q = torch.zeros((1, 256), device=dev)
    kv = torch.zeros((1, 128), device=dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError, match="dtype"):
        pkg.gqa_decode_attention(q.bfloat16(), kv, kv, kc, kc.clone(), pos)
    with pytest.raises(RuntimeError, match="pos"):
        pkg.gqa_decode_attention(q, kv, kv, kc, kc.clone(), pos.int())
    with pytest.raises(RuntimeError, match="rope"):
        pkg.gqa_decode_attention(q, kv, kv, kc, kc.clone(), pos, torch.zeros((16, 32), device=dev), None)
    with pytest.raises(RuntimeError, match="head_dim"):
        pkg.gqa_decode_attention(torch.zeros((1, 192), device=dev), torch.zeros((1, 96), device=dev),
                                 torch.zeros((1, 96), device=dev), torch.zeros((1, 2, 16, 48), device=dev),
                                 torch.zeros((1, 2, 16, 48), device=dev), pos)
