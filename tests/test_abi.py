"""CPU checks of the C-ABI library: it loads, exports every declared symbol, and rejects bad
arguments on the host (before any GPU work) with the reference's error conditions."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wfbitnet.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+(wfb_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("wfb_linear_i2s", "wfb_gemv_i2s", "wfb_gemm_i2s", "wfb_pack_i2s", "wfb_rmsnorm_quant_i8",
              "wfb_quantize_act_i8", "wfb_quantize_act_i8_tensor", "wfb_weight_absmean", "wfb_unpack_i2s",
              "wfb_last_error", "wfb_version"):
        assert s in syms


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    for s in declared_symbols():
        assert hasattr(lib, s), f"{s} declared in include/wfbitnet.h but not exported"
    assert set(pkg._lib.SIGNATURES) | {"wfb_last_error", "wfb_version"} == set(declared_symbols())
    assert lib.wfb_version() == 1


def _linear_status(pkg, fn="wfb_linear_i2s", n=256, k=256, m=1, lda=None, w=16, a=16, out=16, acc=0,
                   out_dtype=1, ldo=None):
    vp = ctypes.c_void_p
    return pkg._lib.status(fn, vp(w) if w else None, n, k, vp(a) if a else None, m, k if lda is None else lda,
                           None, None, 1.0, None, 0, vp(out) if out else None, out_dtype,
                           n if ldo is None else ldo, vp(acc) if acc else None, None)


def test_k_not_multiple_of_128_rejected(pkg):
    assert _linear_status(pkg, k=200) == -1
    assert "must be multiple of 128" in pkg._lib.last_error()


def test_argument_errors(pkg):
    assert _linear_status(pkg, w=0) == -1 and "null" in pkg._lib.last_error()
    assert _linear_status(pkg, w=8) == -1 and "aligned" in pkg._lib.last_error()
    assert _linear_status(pkg, lda=100) == -1 and "stride" in pkg._lib.last_error()
    assert _linear_status(pkg, out=0, acc=0) == -1
    assert _linear_status(pkg, out_dtype=2) == -1 and "dtype" in pkg._lib.last_error()
    assert _linear_status(pkg, ldo=10) == -1
    assert _linear_status(pkg, fn="wfb_gemv_i2s", m=4) == -1 and "GEMV" in pkg._lib.last_error()


def test_prefill_gemm_rejects_row_stride_past_its_offsets(pkg):
    """M > 64 runs the tile GEMM, which addresses up to 128 activation rows of a tile through 32-bit
    offsets from the tile's first row: 127 * lda + K must stay below 2^31 (any M and N are fine)."""
    assert _linear_status(pkg, m=256, lda=2**25) == -1
    assert "too large for the prefill GEMM" in pkg._lib.last_error()
    assert _linear_status(pkg, m=64, lda=2**25, w=8) == -1  # M <= 64 does not take that check
    assert "aligned" in pkg._lib.last_error()


def test_bitlinear_lambda_below_one_raises_before_any_gpu_work(pkg):
    mod = pkg.BitLinear(128, 64)
    pkg.set_lambda_source(lambda: 0.5)
    try:
        with pytest.raises(RuntimeError, match="lambda"):
            mod(torch.zeros(1, 128))
    finally:
        pkg.set_lambda_source(None)


def test_empty_batch_is_a_noop(pkg):
    # M == 0 returns before touching any pointer or the GPU
    assert _linear_status(pkg, m=0, w=0, a=0) == 0
    assert pkg._lib.last_error() == ""


def test_other_entry_points_validate(pkg):
    vp = ctypes.c_void_p
    st = pkg._lib.status
    assert st("wfb_pack_i2s", vp(16), 0, 4, 100, 100, vp(16), vp(16), None) == -1
    assert st("wfb_pack_i2s", vp(16), 9, 4, 128, 128, vp(16), vp(16), None) == -1  # bad dtype
    assert st("wfb_rmsnorm_quant_i8", vp(16), 1, 100, None, 0, 1e-6, 1, 100, vp(16), 100, 104, vp(16), None) == -1
    assert "multiple of 8" in pkg._lib.last_error()
    assert st("wfb_quantize_act_i8", vp(16), 0, 1, 20000, 20000, vp(16), 20000, 20000, vp(16), None) == -1
    assert st("wfb_quantize_act_i8", vp(16), 0, 0, 64, 64, None, 64, 64, None, None) == 0
    assert st("wfb_weight_absmean", vp(16), 0, 10, None, None, None) == -1
    assert st("wfb_unpack_i2s", vp(16), 4, 130, vp(16), None) == -1


def test_python_wrappers_keep_reference_errors(pkg):
    # ValueError for the K % 128 / shape checks of the reference wrappers (bitnet.py:93-104, 131-135)
    with pytest.raises(ValueError):
        pkg.bitnet_gemv(torch.zeros((4, 25), dtype=torch.uint8), torch.zeros(100, dtype=torch.int8), 1.0)
    with pytest.raises(ValueError):
        pkg.bitnet_gemv(torch.zeros((4, 32), dtype=torch.uint8), torch.zeros(100, dtype=torch.int8), 1.0)
    with pytest.raises(ValueError):
        pkg.bitnet_gemm(torch.zeros((4, 25), dtype=torch.uint8), torch.zeros((2, 100), dtype=torch.int8), 1.0)


def test_no_cpu_fallback(pkg):
    # CPU tensors are refused loudly: the product path has no eager / CPU implementation
    with pytest.raises(RuntimeError, match="HIP device"):
        pkg.bitnet_gemv(torch.zeros((4, 32), dtype=torch.uint8), torch.zeros(128, dtype=torch.int8), 1.0)
    with pytest.raises(RuntimeError, match="HIP device"):
        pkg.quantize_activations_i8_per_token(torch.zeros((2, 128)))
    with pytest.raises(RuntimeError, match="HIP device"):
        pkg.BitLinear(128, 64)(torch.zeros(2, 128))


def test_product_does_not_import_oracle():
    pkg_dir = ROOT / "wrinklefree-monorepo_amd"
    for f in list(pkg_dir.rglob("*.py")) + list(pkg_dir.rglob("*.hip")) + list(pkg_dir.rglob("*.h")):
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text and "oracle/" not in text, f


def test_segmented_and_glu_argument_errors(pkg):
    vp = ctypes.c_void_p
    rows = (ctypes.c_int64 * 2)(32, 32)
    st = pkg._lib.status("wfb_linear_i2s_segmented", vp(16), 64, 128, 0, ctypes.cast(rows, vp), vp(16), vp(16), 1, 128,
                         None, None, 0, vp(16), 1, 64, None, None)
    assert st == -1 and "n_seg" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_linear_i2s_segmented", vp(16), 96, 128, 2, ctypes.cast(rows, vp), vp(16), vp(16), 1, 128,
                         None, None, 0, vp(16), 1, 96, None, None)
    assert st == -1 and "sum to 64" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_glu_rmsnorm_quant_i8", vp(16), vp(16), 0, 256, 5, None, 0, 1e-6, 1, 256, vp(16), 256,
                         256, vp(16), None)
    assert st == -1 and "activation" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_glu_rmsnorm_quant_i8", vp(16), vp(16), 0, 250, 1, None, 0, 1e-6, 1, 250, vp(16), 256,
                         256, vp(16), None)
    assert st == -1 and "multiple of 8" in pkg._lib.last_error()


def test_attention_argument_errors(pkg):
    vp = ctypes.c_void_p

    def st(**kw):
        a = dict(q=vp(16), ldq=512, k=vp(16), ldk=128, v=vp(16), ldv=128, dtype=1, rc=None, rs=None, kc=vp(16),
                 vc=vp(16), max_len=64, pos=vp(16), b=1, hq=8, hkv=2, d=64, scale=0.125, out=vp(16), ldo=512,
                 work=None)
        a.update(kw)
        return pkg._lib.status("wfb_gqa_decode_attention", *a.values(), None)

    assert st(d=96) == -1 and "head_dim" in pkg._lib.last_error()
    assert st(hq=18, ldq=18 * 64, ldo=18 * 64) == -1 and "num_heads" in pkg._lib.last_error()
    assert st(hq=6, hkv=4, ldk=256, ldv=256) == -1 and "num_heads" in pkg._lib.last_error()
    assert st(dtype=2) == -1 and "dtype" in pkg._lib.last_error()
    assert st(ldq=256) == -1 and "strides" in pkg._lib.last_error()
    assert st(rc=vp(16)) == -1 and "rope" in pkg._lib.last_error()
    assert st(max_len=1 << 30) == -1 and "max_len" in pkg._lib.last_error()
    assert st(kc=vp(8)) == -1 and "aligned" in pkg._lib.last_error()
    assert st(pos=None) == -1 and "null" in pkg._lib.last_error()
    assert st(scale=float("inf")) == -1 and "finite" in pkg._lib.last_error()
    assert st(b=0) == 0


def test_prefill_attention_argument_errors(pkg):
    vp = ctypes.c_void_p

    def st(**kw):
        a = dict(q=vp(16), ldq=512, k=vp(16), ldk=128, v=vp(16), ldv=128, dtype=1, rc=None, rs=None, kc=vp(16),
                 vc=vp(16), max_len=64, start=0, b=1, t=8, hq=8, hkv=2, d=64, scale=0.125, out=vp(16), ldo=512)
        a.update(kw)
        return pkg._lib.status("wfb_gqa_prefill_attention", *a.values(), None)

    assert st(dtype=0) == -1 and "WFB_BF16" in pkg._lib.last_error()
    assert st(d=96) == -1 and "head_dim" in pkg._lib.last_error()
    assert st(hq=18, ldq=18 * 64, ldo=18 * 64) == -1 and "num_heads" in pkg._lib.last_error()
    assert st(start=60) == -1 and "within max_len" in pkg._lib.last_error()
    assert st(start=-1) == -1 and "within max_len" in pkg._lib.last_error()
    assert st(ldq=256) == -1 and "strides" in pkg._lib.last_error()
    assert st(ldq=516, ldo=516) == -1 and "multiples of 8" in pkg._lib.last_error()
    assert st(rc=vp(16)) == -1 and "rope" in pkg._lib.last_error()
    assert st(max_len=1 << 30) == -1 and "max_len" in pkg._lib.last_error()
    assert st(kc=vp(8)) == -1 and "aligned" in pkg._lib.last_error()
    assert st(out=None) == -1 and "null" in pkg._lib.last_error()
    assert st(scale=float("nan")) == -1 and "finite" in pkg._lib.last_error()
    assert st(b=0) == 0 and st(t=0) == 0


def test_argmax_argument_errors(pkg):
    vp = ctypes.c_void_p
    st = pkg._lib.status("wfb_linear_i2s_argmax", vp(16), 64, 128, vp(16), 65, 128, None, None, 1.0, None, 0, 64,
                         vp(16), vp(16), None)
    assert st == -1 and "M (65)" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_linear_i2s_argmax", vp(16), 64, 128, vp(16), 2, 128, None, None, 1.0, None, 2, 64,
                         vp(16), vp(16), None)
    assert st == -1 and "logits dtype" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_linear_i2s_argmax", vp(16), 64, 128, vp(16), 2, 128, None, None, 1.0, None, 0, 64,
                         None, vp(16), None)
    assert st == -1 and "workspace" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_lm_head_argmax", vp(16), 0, 64, None, 0, 1e-5, vp(16), 0, 64, 17, 100, 64, None, 100,
                         vp(16), vp(16), None)
    assert st == -1 and "M (17)" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_lm_head_argmax", vp(16), 0, 4096, None, 0, 1e-5, vp(16), 0, 4096, 8, 100, 4096, None,
                         100, vp(16), vp(16), None)
    assert st == -1 and "M*H" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_lm_head_argmax", vp(16), 0, 60, None, 0, 1e-5, vp(16), 0, 60, 1, 100, 60, None, 100,
                         vp(16), vp(16), None)
    assert st == -1 and "multiple of 8" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_lm_head_argmax", vp(16), 0, 64, None, 0, 1e-5, vp(8), 0, 64, 1, 100, 64, None, 100,
                         vp(16), vp(16), None)
    assert st == -1 and "aligned" in pkg._lib.last_error()


def test_residual_argument_errors(pkg):
    vp = ctypes.c_void_p
    st = pkg._lib.status("wfb_linear_i2s_residual", vp(16), 64, 128, vp(16), 2, 128, None, None, 1.0, vp(16), 2, 64,
                         vp(16), 1, 64, None)
    assert st == -1 and "residual dtype" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_linear_i2s_residual", vp(16), 64, 128, vp(16), 2, 128, None, None, 1.0, None, 1, 64,
                         vp(16), 1, 64, None)
    assert st == -1 and "null residual" in pkg._lib.last_error()
    st = pkg._lib.status("wfb_linear_i2s_residual", vp(16), 64, 128, vp(16), 2, 128, None, None, 1.0, vp(16), 1, 32,
                         vp(16), 1, 64, None)
    assert st == -1 and "residual row stride" in pkg._lib.last_error()


def test_rmsnorm_linear_argument_errors(pkg):
    vp = ctypes.c_void_p
    seg = (ctypes.c_int64 * 2)(64, 64)

    def st(x_dt=1, g_dt=1, m=8, h=4096, n=128, k=4096, n_seg=1, segp=None, res=None, res_dt=1, out_dt=1, x=16):
        return pkg._lib.status("wfb_rmsnorm_linear_i2s", vp(x) if x else None, x_dt, h, vp(16), g_dt, 1e-5, m, h,
                               vp(16), n, k, n_seg, segp, vp(16), res, res_dt, n, vp(16), out_dt, n, None)

    assert st(x_dt=2) == -1 and "x dtype" in pkg._lib.last_error()
    assert st(g_dt=2) == -1 and "gamma dtype" in pkg._lib.last_error()
    assert st(m=17) == -1 and "M (17)" in pkg._lib.last_error()
    assert st(h=4104, k=4224) == -1 and "needs M == 1" in pkg._lib.last_error()  # long rows: one token only
    assert st(m=2, h=4096, k=4224) == -1 and "needs M == 1" in pkg._lib.last_error()  # ... whatever H
    assert st(m=1, h=16392, k=16512) == -1 and "needs M == 1" in pkg._lib.last_error()  # ... up to 16384
    assert st(h=4100, k=4224) == -1 and "H % 8 == 0" in pkg._lib.last_error()
    assert st(n_seg=2) == -1 and "seg_rows" in pkg._lib.last_error()
    assert st(n_seg=2, segp=ctypes.cast(seg, vp), n=136) == -1 and "sum to 128" in pkg._lib.last_error()
    assert st(res=vp(16), res_dt=2) == -1 and "residual dtype" in pkg._lib.last_error()
    assert st(out_dt=2) == -1 and "out must be" in pkg._lib.last_error()
    assert st(x=8) == -1 and "16-byte aligned" in pkg._lib.last_error()


def test_fusion_predicates_match_the_entry_points(pkg):
    """rmsnorm_linear_supported / rmsnorm_linear_glu_supported accept exactly the sizes the C entry points'
    argument checks accept.  Every call also carries one bad argument checked after the size rules (an
    output dtype / a null output), so an accepted size stops there and nothing is launched."""
    vp = ctypes.c_void_p
    size_rules = ("must be in 0..16", "needs M == 1", "H % 8 == 0")

    def refused(fn, m, h, k, n=128):
        if fn == "wfb_rmsnorm_linear_i2s":
            st = pkg._lib.status(fn, vp(16), 1, h, vp(16), 1, 1e-5, m, h, vp(16), n, k, 1, None, vp(16), None, 1, n,
                                 vp(16), 2, n, None)
            later = "out must be"
        else:
            st = pkg._lib.status(fn, vp(16), 1, h, vp(16), 1, 1e-5, m, h, vp(16), n, k, vp(16), 1, 1, None, n, None)
            later = "null pointer"
        err = pkg._lib.last_error()
        assert st == -1 and (later in err or any(r in err for r in size_rules)), err
        return any(r in err for r in size_rules)

    sizes = [(576, 640), (640, 576), (2560, 2560), (4096, 4096), (4000, 4096), (4096, 4224), (4104, 4224),
             (4100, 4224), (6912, 6912), (14336, 14336), (16384, 16384), (16392, 16512)]
    for m in (1, 2, 8, 16, 17):
        for h, k in sizes:
            assert pkg.rmsnorm_linear_supported(m, h, k) == (not refused("wfb_rmsnorm_linear_i2s", m, h, k)), (m, h, k)
            assert pkg.rmsnorm_linear_glu_supported(m, h, k) == (not refused("wfb_rmsnorm_linear_i2s_glu", m, h, k)), (
                m, h, k)


def test_rmsnorm_linear_glu_argument_errors(pkg):
    vp = ctypes.c_void_p

    def st(x_dt=1, g_dt=1, m=8, h=4096, n=128, k=4096, act=1, mid=1, ldo=64, x=16, out=16):
        return pkg._lib.status("wfb_rmsnorm_linear_i2s_glu", vp(x) if x else None, x_dt, h, vp(16), g_dt, 1e-5, m, h,
                               vp(16), n, k, vp(16), act, mid, vp(out) if out else None, ldo, None)

    assert st(x_dt=2) == -1 and "x dtype" in pkg._lib.last_error()
    assert st(g_dt=2) == -1 and "gamma dtype" in pkg._lib.last_error()
    assert st(act=0) == -1 and "bad activation" in pkg._lib.last_error()
    assert st(mid=2) == -1 and "mid dtype" in pkg._lib.last_error()
    assert st(m=17) == -1 and "M (17)" in pkg._lib.last_error()
    assert st(h=4100, k=4224) == -1 and "H <= K <= 4096" in pkg._lib.last_error()
    assert st(n=96) == -1 and "multiple of 32" in pkg._lib.last_error()
    assert st(ldo=63) == -1 and "row strides" in pkg._lib.last_error()
    assert st(out=0) == -1 and "null pointer" in pkg._lib.last_error()
    assert st(x=8) == -1 and "16-byte aligned" in pkg._lib.last_error()
    assert st(m=0) == 0


def test_linear_glu_argument_errors(pkg):
    vp = ctypes.c_void_p

    def st(n=128, k=256, m=4, act=1, mid=1, lda=256, ldo=64):
        return pkg._lib.status("wfb_linear_i2s_glu", vp(16), n, k, vp(16), m, lda, None, vp(16), act, mid, vp(16), ldo,
                               None)

    assert st(act=3) == -1 and "activation" in pkg._lib.last_error()
    assert st(mid=2) == -1 and "mid dtype" in pkg._lib.last_error()
    assert st(m=65) == -1 and "0..64" in pkg._lib.last_error()
    assert st(n=96) == -1 and "multiple of 32" in pkg._lib.last_error()
    assert st(lda=200) == -1 and "row stride" in pkg._lib.last_error()
    assert st(ldo=32) == -1 and "N/2" in pkg._lib.last_error()
    assert st(m=0) == 0


def test_fused_op_weight_cache(pkg):
    """The fused reference ops' weight concatenations (host logic, CPU tensors): a single weight is used as it
    is (no copy), a set is concatenated once and reused until a weight changes in place, and the cache holds
    the q|k|v and gate|up sets of a 128-layer model."""
    ops = pkg.ops
    w = torch.arange(64, dtype=torch.uint8).reshape(8, 8)
    same, sc = ops._concat_weights((w,), (0.5,))
    assert same is w and sc.tolist() == [0.5]
    a, b = torch.zeros(8, 8, dtype=torch.uint8), torch.ones(16, 8, dtype=torch.uint8)
    cat1, s1 = ops._concat_weights((a, b), (0.25, 2.0))
    cat2, _ = ops._concat_weights((a, b), (0.25, 2.0))
    assert cat2 is cat1 and cat1.shape == (24, 8) and s1.tolist() == [0.25, 2.0]
    b.fill_(3)  # in place: new version counter
    cat3, _ = ops._concat_weights((a, b), (0.25, 2.0))
    assert cat3 is not cat1 and int(cat3[8:].min()) == 3
    assert ops._CONCAT_CACHE_MAX >= 2 * 128
