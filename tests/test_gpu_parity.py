"""GPU parity of every hot-path kernel against the CPU oracle, through the C ABI.

Bars: int8 codes, packed bytes and int32 accumulators bit-exact; fp32 outputs bit-exact (same
operation order as the oracle); bf16 outputs within 1e-2 relative (and here also bit-exact).
Full BASELINE shapes are checked exactly for the GEMV/batched sweep; the large prefill GEMMs are
checked exactly on sampled token rows plus a whole-output checksum identity.
"""

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc

pytestmark = pytest.mark.gpu

SHAPES_2B = [(2560, 2560), (3200, 2560), (13824, 2560), (2560, 6912)]  # (N, K)
BF16_RTOL = 1e-2


def _packed(rng, n, k):
    q = orc.random_ternary(rng, n, k)
    return orc.pack_i2s(q)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _ref_acc(packed, a):
    """Exact accumulators via an fp32 GEMM of the unpacked weights (partial sums < 2^24)."""
    w = orc.unpack_i2s(packed).astype(np.float32)
    return (np.atleast_2d(a).astype(np.float32) @ w.T).astype(np.int64)


def _check_linear(pkg, dev, packed, a, w_scale, a_scale, kernel="auto", bias=None, check_fp32=True):
    n, k = packed.shape[0], packed.shape[1] * 4
    pw, pa, ps = _t(packed, dev), _t(a, dev), _t(a_scale, dev)
    pb = None if bias is None else _t(bias, dev)
    y, acc = pkg.bitnet_linear(pw, pa, float(w_scale), a_scale=ps, bias=pb, return_acc=True, kernel=kernel)
    acc_ref = _ref_acc(packed, a)
    acc_g = acc.cpu().numpy().astype(np.int64)
    assert acc_g.shape == acc_ref.shape
    bad = np.argwhere(acc_g != acc_ref)
    assert bad.size == 0, f"{len(bad)} accumulator mismatches, first at {bad[:3].tolist()}"
    y_ref = orc.rescale(acc_ref, w_scale, a_scale, bias)
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(yb, orc.f32_to_bf16_bits(y_ref)), "bf16 output bits differ"
    yg = orc.bf16_bits_to_f32(yb)
    rel = np.abs(yg - y_ref) / np.maximum(np.abs(y_ref), 1e-30)
    assert float(rel[np.abs(y_ref) > 0].max(initial=0)) <= BF16_RTOL
    if check_fp32:
        y32 = pkg.bitnet_linear(pw, pa, float(w_scale), a_scale=ps, bias=pb, out_dtype=torch.float32, kernel=kernel)
        assert np.array_equal(y32.cpu().numpy(), y_ref)
    if bias is None:
        # the production forms: bf16 out alone (whole-line bf16 epilogue), and with a bf16 residual added
        y1 = pkg.bitnet_linear(pw, pa, float(w_scale), a_scale=ps, kernel=kernel)
        assert np.array_equal(y1.view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y_ref)), \
            "bf16-only output bits differ"
        m = a.shape[0]
        res = torch.linspace(-2.0, 2.0, m * n, dtype=torch.float32).reshape(m, n).to(torch.bfloat16)
        want = torch.from_numpy(y_ref.astype(np.float32) + res.float().numpy()).to(torch.bfloat16)
        got = pkg.bitnet_linear_residual(pw, pa, float(w_scale), res.to(dev), a_scale=ps)
        assert torch.equal(got.cpu(), want), "residual output differs"


# ---- a1: pack -------------------------------------------------------------------------------------


@pytest.mark.parametrize("n,k", SHAPES_2B + [(576, 576), (1536, 576)])
def test_pack_matches_oracle(pkg, dev, n, k):
    rng = np.random.default_rng(n * 7 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    kp = (k + 127) // 128 * 128
    qw, scale = pkg.pack_ternary_i2s(_t(w, dev), k_pad=kp)
    s = np.float32(scale.item())
    assert s == orc.absmean_scale_device_order(w)
    t = np.float32(torch.from_numpy(w).abs().mean().item())  # the reference's own fp32 mean
    assert abs(float(s) - float(t)) <= float(np.spacing(t))
    wpad = np.zeros((n, kp), np.float32)
    wpad[:, :k] = w
    packed_ref = orc.pack_i2s(orc.ternarize(wpad, s))
    assert np.array_equal(qw.cpu().numpy(), packed_ref)
    assert np.array_equal(pkg.unpack_i2s(qw).cpu().numpy(), orc.unpack_i2s(packed_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_half_inputs(pkg, dev, dtype):
    rng = np.random.default_rng(3)
    w = torch.from_numpy((rng.standard_normal((300, 512)) * 0.05).astype(np.float32)).to(dtype)
    qw, scale = pkg.pack_ternary_i2s(w.to(dev))
    wf = w.float().numpy()
    s = np.float32(scale.item())
    assert s == orc.absmean_scale_device_order(wf)
    assert np.array_equal(qw.cpu().numpy(), orc.pack_i2s(orc.ternarize(wf, s)))


def test_pack_given_scale_and_ties(pkg, dev):
    # exact .5 ties under a given scale round half to even, like torch.round
    w = np.tile(np.array([0.5, -0.5, 1.5, -1.5, 0.25, 2.0, -0.75, 0.0], np.float32), (4, 16))
    qw, _ = pkg.pack_ternary_i2s(_t(w, dev), scale=torch.ones(1, device=dev))
    assert np.array_equal(qw.cpu().numpy(), orc.pack_i2s(orc.ternarize(w, 1.0)))


def test_absmean_tiny_weights(pkg, dev):
    w = torch.full((8, 128), 1e-9, device=dev)
    assert pkg.absmean_scale(w).item() == 1.0


# ---- a2 / a3: activation quantisers ------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,h,kp", [(1, 2560, 2560), (7, 576, 640), (64, 6912, 6912), (3, 14336, 14336), (2, 100, 128)])
def test_quant_per_token(pkg, dev, dtype, m, h, kp):
    rng = np.random.default_rng(m * 1000 + h)
    x = torch.from_numpy(orc.outlier_hidden(rng, m, h)).to(dtype)
    q, s = pkg.quantize_activations_i8_per_token(x.to(dev), k_pad=kp)
    q_ref, s_ref = orc.quantize_per_token(x.float().numpy(), k_pad=kp)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


def test_quant_special_rows(pkg, dev):
    x = np.zeros((4, 256), np.float32)
    x[1, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]  # exact ties
    x[2, 100] = -3.25  # single spike
    x[3, :] = 5e-7  # below the 1e-6 floor
    q, s = pkg.quantize_activations_i8_per_token(_t(x, dev))
    q_ref, s_ref = orc.quantize_per_token(x)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)
    assert q[1, :8].tolist() == [127, 0, 2, 2, 0, -2, -2, 126]


@pytest.mark.parametrize("numel", [1, 1000, 2560 * 16, 3 * 1000003])
def test_quant_per_tensor(pkg, dev, numel):
    rng = np.random.default_rng(numel)
    x = (rng.standard_normal(numel) * 3).astype(np.float32)
    q, s = pkg.quantize_activations_i8(_t(x, dev))
    q_ref, s_ref = orc.quantize_per_tensor(x)
    assert np.array_equal(q.cpu().numpy(), q_ref) and s.item() == s_ref[0]


@pytest.mark.parametrize("gdtype", [None, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,h,kp", [(1, 576, 640), (16, 2560, 2560), (5, 6912, 6912), (64, 4096, 4096), (2, 1536, 1536)])
def test_rmsnorm_quant(pkg, dev, gdtype, m, h, kp):
    rng = np.random.default_rng(h + m)
    x = torch.from_numpy(orc.outlier_hidden(rng, m, h)).to(torch.bfloat16)
    g = None if gdtype is None else torch.from_numpy((1 + 0.1 * rng.standard_normal(h)).astype(np.float32)).to(gdtype)
    q, s = pkg.rmsnorm_quantize_i8(x.to(dev), None if g is None else g.to(dev), eps=1e-6, k_pad=kp)
    q_ref, s_ref = orc.rmsnorm_quant(x.float().numpy(), None if g is None else g.float().numpy(), 1e-6, k_pad=kp)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


def test_rmsnorm_quant_fp32_input_eps(pkg, dev):
    rng = np.random.default_rng(77)
    x = rng.standard_normal((9, 2560)).astype(np.float32)
    x[3] = 0.0  # zero row: y = 0, codes 0
    q, s = pkg.rmsnorm_quantize_i8(_t(x, dev), None, eps=1e-5)
    q_ref, s_ref = orc.rmsnorm_quant(x, None, 1e-5)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m,h", [(8, 14336), (3, 6912), (8, 10000), (2, 16384)])
def test_rmsnorm_quant_long_fp32_rows_gamma(pkg, dev, gdtype, m, h):
    """fp32 rows longer than 4096 (the decode layer's gated row: 256 threads per row, gamma's words
    requested with the row's, rows past the last full iteration included) and, gated, the 1024-thread
    form (rows up to 15360): codes and scales equal the oracle's for bf16 and fp32 gamma."""
    rng = np.random.default_rng(h * 3 + m)
    x = orc.outlier_hidden(rng, m, h).astype(np.float32)
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(h)).astype(np.float32)).to(gdtype)
    q, s = pkg.rmsnorm_quantize_i8(_t(x, dev), g.to(dev), eps=1e-6)
    q_ref, s_ref = orc.rmsnorm_quant(x, g.float().numpy(), 1e-6)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)
    up = orc.outlier_hidden(rng, m, h).astype(np.float32)
    for act in ("silu", "relu2"):
        qg, sg = pkg.glu_rmsnorm_quantize_i8(_t(x, dev), _t(up, dev), act, g.to(dev), eps=1e-6)
        qg_ref, sg_ref = orc.glu_rmsnorm_quant(x, up, 1 if act == "silu" else 2, g.float().numpy(), 1e-6)
        assert np.array_equal(qg.cpu().numpy(), qg_ref) and np.array_equal(sg.cpu().numpy(), sg_ref)


# ---- a4 / a5 / a6: GEMV, batched sweep, prefill GEMM ---------------------------------------------


@pytest.mark.parametrize("n,k", SHAPES_2B)
@pytest.mark.parametrize("m", [1, 2])
def test_decode_gemv_2b_shapes(pkg, dev, n, k, m):
    rng = np.random.default_rng(1000 + n + k + m)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _check_linear(pkg, dev, packed, a, orc.log_uniform(rng), orc.log_uniform(rng, m), kernel="gemv")


# (n, k): grids of 2048 workgroups or fewer stage each wave's activation slice in LDS; above that (70000 x
# 4096: 2188 workgroups of 32 rows, 40000 x 2560: 2500, 36000 x 640: 2250 with masked chunks, 33000 x 1024:
# 2063) the fragments come straight from global memory
@pytest.mark.parametrize("n,k", [(2560, 2560), (4099, 640), (70000, 4096), (40000, 2560), (36000, 640), (33000, 1024)])
@pytest.mark.parametrize("m", [1, 2])
def test_decode_gemv_epilogue_operands_and_grid_sizes(pkg, dev, n, k, m):
    """The M <= 2 GEMV on both activation paths: accumulators and bf16 outputs exact, a bias in each float
    dtype and a residual in either dtype (operands loaded as raw bits at kernel entry, converted at the
    epilogue) equal to the oracle's rescale."""
    rng = np.random.default_rng(9000 + m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    ws, a_s = orc.log_uniform(rng), orc.log_uniform(rng, m)
    _check_linear(pkg, dev, packed, a, ws, a_s, kernel="gemv", check_fp32=False)
    acc = _ref_acc(packed, a)
    pw, pa, ps = _t(packed, dev), _t(a, dev), _t(a_s, dev)
    for bdt in (torch.float32, torch.bfloat16, torch.float16):
        bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(bdt)
        y32 = pkg.bitnet_linear(pw, pa, float(ws), a_scale=ps, bias=bias.to(dev), out_dtype=torch.float32,
                                kernel="gemv")
        assert np.array_equal(y32.cpu().numpy(), orc.rescale(acc, ws, a_s, bias.float().numpy())), bdt
    for rdt in (torch.float32, torch.bfloat16):
        res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(rdt)
        want = torch.from_numpy(orc.rescale(acc, np.float32(ws), a_s) + res.float().numpy()).to(rdt)
        got = pkg.bitnet_linear_residual(pw, pa, float(ws), res.to(dev), a_scale=ps)
        assert torch.equal(got.cpu(), want), rdt


@pytest.mark.parametrize("n,k", [(2560, 2560), (2560, 6912), (13824, 2560)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32, 64])
def test_batched_sweep_mfma(pkg, dev, n, k, m):
    rng = np.random.default_rng(2000 + n + k + m)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _check_linear(pkg, dev, packed, a, orc.log_uniform(rng), orc.log_uniform(rng, m), kernel="gemm")
    if m <= 2:
        _check_linear(pkg, dev, packed, a, 1.0, np.ones(m, np.float32), kernel="auto", check_fp32=False)


@pytest.mark.parametrize("m", [3, 4, 5, 8, 9, 12, 16, 17, 31, 32, 40, 64])
@pytest.mark.parametrize("n,k", SHAPES_2B)
def test_batched_decode_outputs_without_accumulator_copy(pkg, dev, m, n, k):
    """M <= 16 without an accumulator copy takes the LDS-staged kernel's whole-line epilogue (17..32 tokens
    too, as two token tiles, on the K = 2560 shapes, and 33..64 as four on the narrow ones): bf16 and fp32
    outputs, a bias, and a residual in either dtype, all equal to the oracle's rescale bit for bit."""
    rng = np.random.default_rng(7000 + m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    ws, a_s = orc.log_uniform(rng), orc.log_uniform(rng, m)
    acc = _ref_acc(packed, a)
    pw, pa, ps = _t(packed, dev), _t(a, dev), _t(a_s, dev)
    y = pkg.bitnet_linear(pw, pa, float(ws), a_scale=ps)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(orc.rescale(acc, ws, a_s)))
    bias = rng.standard_normal(n).astype(np.float32)
    y32 = pkg.bitnet_linear(pw, pa, float(ws), a_scale=ps, bias=_t(bias, dev), out_dtype=torch.float32)
    assert np.array_equal(y32.cpu().numpy(), orc.rescale(acc, ws, a_s, bias))
    for rdt in (torch.float32, torch.bfloat16):
        res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(rdt)
        want = torch.from_numpy(orc.rescale(acc, np.float32(ws), a_s) + res.float().numpy()).to(rdt)
        got = pkg.bitnet_linear_residual(pw, pa, float(ws), res.to(dev), a_scale=ps)
        assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("m,n,k", [(5, 4096, 14336), (8, 4096, 14336), (16, 4096, 14336), (9, 1000, 14208),
                                   (12, 100, 8448), (7, 2600, 10240), (16, 33, 12800)])
def test_batched_long_rows_register_activations(pkg, dev, m, n, k):
    """5 <= M <= 16 with 8192 < K <= 14336 (the Llama-3-8B down projection): the activations do not fit the
    LDS beside the weights, so the staged kernel holds them in registers.  Accumulators (per-lane
    epilogue), bf16 / fp32 outputs and a residual in either dtype (whole-line epilogue) equal the oracle's."""
    rng = np.random.default_rng(8100 + m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    ws, a_s = orc.log_uniform(rng), orc.log_uniform(rng, m)
    _check_linear(pkg, dev, packed, a, ws, a_s, kernel="gemm")
    acc = _ref_acc(packed, a)
    pw, pa, ps = _t(packed, dev), _t(a, dev), _t(a_s, dev)
    y = pkg.bitnet_linear(pw, pa, float(ws), a_scale=ps)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(orc.rescale(acc, ws, a_s)))
    for rdt in (torch.float32, torch.bfloat16):
        res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(rdt)
        want = torch.from_numpy(orc.rescale(acc, np.float32(ws), a_s) + res.float().numpy()).to(rdt)
        got = pkg.bitnet_linear_residual(pw, pa, float(ws), res.to(dev), a_scale=ps)
        assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("m,n,k", [(12, 32800, 128), (24, 16400, 256), (64, 8200, 384), (9, 40, 8192),
                                   (24, 9216, 2560), (24, 9200, 2560), (40, 6144, 8192), (40, 6144, 8320),
                                   (40, 12000, 8320), (17, 18432, 256), (24, 9216, 4096), (24, 9200, 4096),
                                   (32, 4096, 4096), (32, 4112, 4096), (32, 32768, 2560), (32, 32784, 2560),
                                   (33, 4096, 4096), (64, 4096, 4096), (64, 4112, 4096), (48, 2560, 4224),
                                   (40, 1000, 2560), (32, 4096, 7168), (17, 4112, 6912), (24, 2560, 7296),
                                   (33, 2560, 6912), (64, 4096, 7168), (64, 4112, 6912), (48, 2560, 6912),
                                   (49, 2560, 6912), (37, 4096, 4096), (49, 4000, 4096), (64, 2560, 4096),
                                   (33, 4096, 14336), (64, 4104, 14336), (48, 4096, 16384), (64, 4088, 4096)])
def test_batched_kernel_choice_boundaries(pkg, dev, m, n, k):
    # 3 <= M <= 64: the LDS-staged kernel up to 16 tokens, and with two token tiles for 17..32 tokens on
    # rows up to 2560 (outputs up to 32768 rows) or 7168 (outputs up to 4096 rows), with four for 33..64
    # tokens on rows up to 4096 and outputs up to 4096 rows (two token blocks of two-tile workgroups for rows
    # of 4096, and for rows up to 7168 from 49 tokens; two launches of two tiles below that); 33..64 tokens
    # on rows and outputs of 4096 or more: the 32-row tile kernel with its K split (four groups on rows of
    # 8192 or more, two below); else the 32-row tile
    # kernel for M > 16 when N * ceil(M/16) >= 18432 and K <= 8192, else the split-K skinny kernel while
    # N * ceil(M/16) <= 32768 (always for M <= 8), else the whole-K wave-per-rows kernel; these shapes
    # sit on either side of those boundaries
    rng = np.random.default_rng(2500 + m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _check_linear(pkg, dev, packed, a, orc.log_uniform(rng), orc.log_uniform(rng, m), kernel="gemm")


@pytest.mark.parametrize("m,n,k", [(96, 2560, 6912), (256, 2560, 6912), (100, 2560, 7040), (384, 2560, 6912),
                                   (256, 4096, 14336), (512, 4096, 14336), (320, 4096, 8192), (512, 2560, 2560),
                                   (512, 2600, 6912), (480, 4096, 8320)])
def test_gemm_k_groups(pkg, dev, m, n, k):
    # M > 64 on few 32-row tiles: three groups of four waves splitting K on 32 x 256 tiles (160..256 of
    # them), four groups on 32 x 128 tiles for rows of 6912 or more below that; ragged N and K included
    rng = np.random.default_rng(3500 + m + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _check_linear(pkg, dev, packed, a, orc.log_uniform(rng), orc.log_uniform(rng, m), check_fp32=False)


@pytest.mark.parametrize("n,k", [(13824, 2560), (2560, 6912)])
@pytest.mark.parametrize("m", [512, 2048])
def test_prefill_gemm_exact(pkg, dev, n, k, m):
    rng = np.random.default_rng(3000 + n + m)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _check_linear(pkg, dev, packed, a, orc.log_uniform(rng), orc.log_uniform(rng, m), check_fp32=False)


@pytest.mark.parametrize("n,k", [(13824, 2560), (2560, 6912)])
def test_prefill_gemm_8192_sampled(pkg, dev, n, k):
    m = 8192
    rng = np.random.default_rng(4000 + n)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    _, acc = pkg.bitnet_linear(_t(packed, dev), _t(a, dev), 1.0, return_acc=True)
    acc_g = acc.cpu().numpy().astype(np.int64)
    rows = np.sort(rng.choice(m, 96, replace=False))
    rows = np.concatenate([[0, m - 1], rows])
    assert np.array_equal(acc_g[rows], _ref_acc(packed, a[rows]))
    # checksum of the whole output: sum_{m,n} acc = sum_k (sum_m a[m,k]) * (sum_n w[n,k])
    w_col = orc.unpack_i2s(packed).astype(np.int64).sum(axis=0)
    a_col = a.astype(np.int64).sum(axis=0)
    assert acc_g.sum() == int(a_col @ w_col)
    # and per-row sums: sum_n acc[m, n] = a[m] . w_col
    assert np.array_equal(acc_g.sum(axis=1), a.astype(np.int64) @ w_col)


def test_prefill_gemm_activation_offsets_past_4gib(pkg, dev):
    """A strided activation view whose last row starts past 2^32 bytes: (M - 1) * lda + K > 2^32 while
    127 * lda + K < 2^31 (the host's limit for the prefill GEMM), so every row must be read from its
    own place -- a 32-bit offset from the start of A would wrap.  All 300 x 256 accumulators exact."""
    m, n, k = 300, 256, 2560
    lda = 16_777_088  # multiple of 16; 127 * lda + K < 2^31; (m - 1) * lda > 2^32
    assert (m - 1) * lda + k > 2**32 and 127 * lda + k < 2**31
    rng = np.random.default_rng(77)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    big = torch.empty((m, lda), dtype=torch.int8, device=dev)
    big[:, :k].copy_(_t(a, dev))
    y, acc = pkg.bitnet_linear(_t(packed, dev), big[:, :k], 1.0, return_acc=True)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), _ref_acc(packed, a))
    y2 = pkg.bitnet_linear(_t(packed, dev), big[:, :k], 1.0)  # the staged bf16 epilogue
    assert torch.equal(y2, y)
    del big


def test_prefill_gemm_weight_offsets_past_4gib(pkg, dev):
    """N * K / 4 > 2^32: weight rows past the first 4 GiB of the packed matrix (1,049,576 rows of
    K = 16384, 4.3 GB) are read from their own place.  The matrix repeats 4096 random rows, so every
    accumulator is checked against the oracle's product with the row it repeats."""
    m, k, base_rows = 65, 16384, 4096
    n = 2**32 // (k // 4) + 1000
    rng = np.random.default_rng(78)
    base = _packed(rng, base_rows, k)
    a = orc.random_int8(rng, m, k)
    reps = (n + base_rows - 1) // base_rows
    w = _t(base, dev).repeat(reps, 1)[:n]
    assert w.is_contiguous() and w.numel() > 2**32
    _, acc = pkg.bitnet_linear(w, _t(a, dev), 1.0, return_acc=True)
    ref = _ref_acc(base, a).astype(np.int32)  # [m, base_rows]
    del w
    got = acc.cpu().numpy()
    del acc
    full = (n // base_rows) * base_rows
    assert np.array_equal(got[:, :full].reshape(m, -1, base_rows), np.broadcast_to(ref[:, None, :], (m, full // base_rows, base_rows)))
    assert np.array_equal(got[:, full:], ref[:, :n - full])


@pytest.mark.parametrize("m", [1, 2, 3, 17, 33, 300])
@pytest.mark.parametrize("n,k", [(100, 128), (17, 640), (1, 256), (77, 14336), (130, 16384)])
def test_ragged_shapes(pkg, dev, m, n, k):
    rng = np.random.default_rng(m * 31 + n + k)
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, m, k)
    a[:, :3] = -128
    _check_linear(pkg, dev, packed, a, 0.5, orc.log_uniform(rng, m))


def test_strided_activations_bias_and_device_scale(pkg, dev):
    rng = np.random.default_rng(5)
    n, k, m = 257, 512, 6
    packed = _packed(rng, n, k)
    big = orc.random_int8(rng, m, k + 64)
    a_view = _t(big, dev)[:, :k]  # row stride k + 64
    bias = rng.standard_normal(n).astype(np.float32)
    a_scale = orc.log_uniform(rng, m)
    ws = torch.tensor([0.0123], dtype=torch.float32, device=dev)
    for b in (torch.from_numpy(bias).to(dev), torch.from_numpy(bias).to(dev).to(torch.bfloat16)):
        y, acc = pkg.bitnet_linear(_t(packed, dev), a_view, ws, a_scale=_t(a_scale, dev), bias=b,
                                   out_dtype=torch.float32, return_acc=True)
        acc_ref = _ref_acc(packed, big[:, :k])
        assert np.array_equal(acc.cpu().numpy().astype(np.int64), acc_ref)
        y_ref = orc.rescale(acc_ref, np.float32(0.0123), a_scale, b.float().cpu().numpy())
        assert np.array_equal(y.cpu().numpy(), y_ref)


def test_empty_batch(pkg, dev):
    packed = torch.zeros((64, 32), dtype=torch.uint8, device=dev)
    y = pkg.bitnet_linear(packed, torch.zeros((0, 128), dtype=torch.int8, device=dev), 1.0)
    assert y.shape == (0, 64)


def test_gemv_and_gemm_kernels_agree(pkg, dev):
    rng = np.random.default_rng(8)
    packed = _t(_packed(rng, 3200, 2560), dev)
    for m in (1, 2):
        a = _t(orc.random_int8(rng, m, 2560), dev)
        _, acc1 = pkg.bitnet_linear(packed, a, 1.0, return_acc=True, out_dtype=None, kernel="gemv")
        _, acc2 = pkg.bitnet_linear(packed, a, 1.0, return_acc=True, out_dtype=None, kernel="gemm")
        assert torch.equal(acc1, acc2)


# ---- reference op surface -----------------------------------------------------------------------


def test_reference_op_surface(pkg, dev):
    rng = np.random.default_rng(12)
    n, k = 640, 2560
    packed = _packed(rng, n, k)
    a = orc.random_int8(rng, 3, k)
    pw = _t(packed, dev)
    acc = _ref_acc(packed, a)
    y1 = pkg.bitnet_gemv(pw, _t(a[0], dev), 0.25)
    assert np.array_equal(y1.cpu().numpy(), orc.rescale(acc[:1], 0.25)[0])
    y2 = pkg.bitnet_gemm(pw, _t(a, dev), 0.25)
    assert np.array_equal(y2.cpu().numpy(), orc.rescale(acc, 0.25))
    y3 = torch.ops.wfbitnet.bitnet_gemm(pw, _t(a, dev), 0.25)
    assert torch.equal(y2, y3)
    x = rng.standard_normal((3, k)).astype(np.float32)
    q, s = torch.ops.wfbitnet.bitnet_quantize_activations(_t(x, dev))
    q_ref, s_ref = orc.quantize_per_tensor(x)
    assert np.array_equal(q.cpu().numpy(), q_ref) and s.item() == s_ref[0]


def test_bitlinear_module(pkg, dev):
    rng = np.random.default_rng(21)
    for in_f, out_f in ((576, 1536), (2560, 3200)):
        lin = pkg.BitLinear(in_f, out_f).to(dev)
        with torch.no_grad():
            lin.weight.normal_(0, 0.02, generator=torch.Generator(device=dev).manual_seed(in_f))
        x = torch.from_numpy(orc.outlier_hidden(rng, 6, in_f)).to(torch.bfloat16).to(dev)
        y = lin(x.view(2, 3, in_f))
        assert y.shape == (2, 3, out_f) and y.dtype == torch.bfloat16
        w = lin.weight.detach().cpu().numpy()
        packed, s = orc.pack_ternary(np.pad(w, ((0, 0), (0, lin.k_pad - in_f))), scale=orc.absmean_scale_device_order(w))
        assert np.array_equal(lin.qweight.cpu().numpy(), packed)
        y_ref, acc, _, _ = orc.bitlinear_forward(x.float().cpu().numpy(), packed, s)
        assert np.array_equal(y.view(6, out_f).view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y_ref))


def test_subln_bitlinear_fused(pkg, dev):
    rng = np.random.default_rng(22)
    mod = pkg.SubLNBitLinear(1536, 576).to(dev)
    with torch.no_grad():
        mod.norm_weight.copy_(torch.from_numpy((1 + 0.1 * rng.standard_normal(1536)).astype(np.float32)))
        mod.linear.weight.normal_(0, 0.02)
    x = torch.from_numpy(orc.outlier_hidden(rng, 4, 1536)).to(torch.bfloat16).to(dev)
    y, acc = mod(x, return_acc=True)
    w = mod.linear.weight.detach().cpu().numpy()
    packed, s = orc.pack_ternary(w, scale=orc.absmean_scale_device_order(w))
    q_ref, s_ref = orc.rmsnorm_quant(x.float().cpu().numpy(), mod.norm_weight.detach().cpu().numpy(), 1e-6)
    acc_ref = orc.accumulate(packed, q_ref)
    assert np.array_equal(acc.cpu().numpy().astype(np.int64), acc_ref)
    y_ref = orc.rescale(acc_ref, s, s_ref)
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y_ref))


def test_serving_method_per_tensor_matches_reference_contract(pkg, dev):
    rng = np.random.default_rng(23)
    layer = torch.nn.Module()
    meth = pkg.BitNetLinearMethod(per_token=False)
    meth.create_weights(layer, 640, [320, 64], 640, 384, torch.bfloat16, device=dev)
    packed = _packed(rng, 384, 640)
    layer.qweight.data.copy_(_t(packed, dev))
    layer.scale.data.fill_(0.031)
    x = (rng.standard_normal((5, 640)) * 2).astype(np.float32)
    y = meth.apply(layer, _t(x, dev))
    # reference: quantize_activations_i8 (one scale) -> bitnet_gemm(scale) -> * act_scale
    q_ref, s_ref = orc.quantize_per_tensor(x)
    y_ref = orc.rescale(orc.accumulate(packed, q_ref), np.float32(0.031), np.repeat(s_ref, 5))
    assert np.array_equal(y.cpu().numpy(), y_ref)
    with pytest.raises(ValueError):
        meth.create_weights(torch.nn.Module(), 600, [64], 600, 64, torch.bfloat16, device=dev)


@pytest.mark.parametrize("h", [576, 2560, 4096, 4104, 6912, 14336, 16384])
def test_norm_quant_batch_invariant(pkg, dev, h):
    """A row quantises to the same codes and scale whether it comes in a batch of 8 (one 1024-thread
    workgroup per row) or of 100 (one wave per row, or 256 threads per row above H = 4096): every kernel
    keeps the one summation order the row length defines.  Also checked against the oracle."""
    rng = np.random.default_rng(h)
    x = orc.outlier_hidden(rng, 100, h).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    xt, gt = torch.from_numpy(x).to(dev).to(torch.bfloat16), torch.from_numpy(g).to(dev)
    q_big, s_big = pkg.rmsnorm_quantize_i8(xt, gt, eps=1e-6)
    q_small, s_small = pkg.rmsnorm_quantize_i8(xt[:8].contiguous(), gt, eps=1e-6)
    assert torch.equal(q_big[:8], q_small) and torch.equal(s_big[:8], s_small)
    q_ref, s_ref = orc.rmsnorm_quant(xt[:8].float().cpu().numpy(), g, 1e-6)
    assert np.array_equal(q_small.cpu().numpy(), q_ref) and np.array_equal(s_small.cpu().numpy(), s_ref)
    xf = xt.float()  # fp32 rows (the gated product's dtype in the decode layer): same values, same codes
    qf_big, sf_big = pkg.rmsnorm_quantize_i8(xf, gt, eps=1e-6)
    qf_small, sf_small = pkg.rmsnorm_quantize_i8(xf[:8].contiguous(), gt, eps=1e-6)
    assert torch.equal(qf_big[:8], qf_small) and torch.equal(sf_big[:8], sf_small)
    assert np.array_equal(qf_small.cpu().numpy(), q_ref) and np.array_equal(sf_small.cpu().numpy(), s_ref)
    for act in ("silu", "relu2"):
        up = torch.from_numpy(orc.outlier_hidden(rng, 100, h).astype(np.float32)).to(dev)
        gate = xt.float()
        qb, sb = pkg.glu_rmsnorm_quantize_i8(gate, up, act, gt, eps=1e-6)
        qs, ss = pkg.glu_rmsnorm_quantize_i8(gate[:3].contiguous(), up[:3].contiguous(), act, gt, eps=1e-6)
        assert torch.equal(qb[:3], qs) and torch.equal(sb[:3], ss)
    qp, sp = pkg.quantize_activations_i8_per_token(xt)
    qp8, sp8 = pkg.quantize_activations_i8_per_token(xt[:8].contiguous())
    assert torch.equal(qp[:8], qp8) and torch.equal(sp[:8], sp8)
