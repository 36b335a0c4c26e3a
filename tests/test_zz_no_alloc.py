"""wfb_gqa_decode_attention_noalloc (split partials in the library's own per-GPU scratch, no workspace
argument) against wfb_gqa_decode_attention with a caller workspace, both through the C ABI.

The two run the same kernels on the same split plan, so outputs and caches must be bit-identical.
Two calls in a row, the second on smaller sizes (fewer sequences, a shorter cache), each against a
fresh workspace call; plus the host-side rejection of sizes whose partials would not fit.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

_DT = {torch.float32: 0, torch.bfloat16: 1}


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _tables(max_len, d, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    f = torch.arange(max_len, dtype=torch.float32)[:, None] * inv[None, :]
    return f.cos(), f.sin()


def _inputs(b, hq, hkv, d, max_len, dtype, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn((b, (hq + 2 * hkv) * d), generator=gen).to(dtype).to(dev)
    kc = torch.randn((b, hkv, max_len, d), generator=gen).to(dtype).to(dev)
    vc = torch.randn((b, hkv, max_len, d), generator=gen).to(dtype).to(dev)
    pos = torch.randint(0, max_len, (b,), generator=gen, dtype=torch.int64)
    pos[0] = max_len - 1
    cos, sin = _tables(max_len, d)
    return qkv, kc, vc, pos.to(dev), cos.to(dev), sin.to(dev)


def _call(pkg, noalloc, qkv, kc, vc, pos, cos, sin, hq, hkv, d, stream):
    b, max_len = kc.shape[0], kc.shape[2]
    out = torch.full((b, hq * d), float("nan"), dtype=qkv.dtype, device=qkv.device)
    q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
    ld = qkv.stride(0)
    args = [_p(q), ld, _p(k), ld, _p(v), ld, _DT[qkv.dtype], _p(cos), _p(sin), _p(kc), _p(vc), max_len, _p(pos), b,
            hq, hkv, d, 1.0 / d ** 0.5, _p(out), hq * d]
    if noalloc:
        pkg._lib.call("wfb_gqa_decode_attention_noalloc", *args, stream)
    else:
        work = torch.empty(b * hq * (d + 2) * ((max_len + 63) // 64), dtype=torch.float32, device=qkv.device)
        pkg._lib.call("wfb_gqa_decode_attention", *args, _p(work), stream)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(pkg, dev, dtype):
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # (b, hq, hkv, d, max_len): Llama-3-8B batch 8 at a 4096-slot cache, then a smaller call
    for i, (b, hq, hkv, d, max_len) in enumerate([(8, 32, 8, 128, 4096), (3, 9, 3, 64, 700)]):
        print(f"noalloc case {i}: b={b} hq={hq} hkv={hkv} d={d} max_len={max_len} {dtype}", flush=True)
        qkv, kc, vc, pos, cos, sin = _inputs(b, hq, hkv, d, max_len, dtype, 40 + i, dev)
        kc2, vc2 = kc.clone(), vc.clone()
        want = _call(pkg, False, qkv, kc, vc, pos, cos, sin, hq, hkv, d, stream)
        got = _call(pkg, True, qkv, kc2, vc2, pos, cos, sin, hq, hkv, d, stream)
        torch.cuda.synchronize()
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"case {i}: outputs differ"
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), f"case {i}: caches differ"


def test_noalloc_rejects_sizes_past_its_scratch(pkg, dev):
    """Split partials past the 8 Mi-float scratch are refused on the host, before any GPU work."""
    b, hq, hkv, d, max_len = 64, 32, 8, 128, 8192  # 64 * 32 * 130 * 128 floats > 8 Mi
    vp = ctypes.c_void_p
    st = pkg._lib.status("wfb_gqa_decode_attention_noalloc", vp(16), hq * d, vp(16), hkv * d, vp(16), hkv * d, 1,
                         None, None, vp(16), vp(16), max_len, vp(16), b, hq, hkv, d, 0.1, vp(16), hq * d, None)
    assert st == -1 and "scratch" in pkg._lib.last_error()
