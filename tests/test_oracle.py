"""CPU checks that pin the oracle: known-answer tests, the reference's compiled kernels (golden
fixtures and oracle/_ref), closed forms and brute force."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bitnet_oracle as orc
from oracle import refbind

GOLDEN = Path(__file__).resolve().parent / "golden" / "ref_kernels.npz"


# ---- a1: scale, ternarisation, layout ---------------------------------------------------------


def test_absmean_kat():
    # packages/training/tests/test_quantization.py:65-71
    assert orc.absmean_scale(np.array([1.0, -2.0, 3.0, -4.0], np.float32)) == np.float32(2.5)
    assert orc.absmean_scale_device_order(np.array([1.0, -2.0, 3.0, -4.0], np.float32)) == np.float32(2.5)


def test_absmean_tiny_becomes_one():
    # convert_to_sglkernel.py:83-85
    w = np.full((4, 128), 1e-9, np.float32)
    assert orc.absmean_scale(w) == np.float32(1.0)
    assert orc.absmean_scale_device_order(w) == np.float32(1.0)


@pytest.mark.parametrize("shape", [(64, 128), (2560, 640), (1000, 384)])
def test_absmean_matches_torch_mean(shape):
    # the reference computes w.abs().mean() with torch in fp32 (convert_to_sglkernel.py:82)
    rng = np.random.default_rng(7)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    t = np.float32(torch.from_numpy(w).abs().mean().item())
    for s in (orc.absmean_scale(w), orc.absmean_scale_device_order(w)):
        assert abs(float(s) - float(t)) <= float(np.spacing(t)), (s, t)
    assert orc.absmean_scale(w) == orc.absmean_scale_device_order(w)


def test_ternarize_half_even():
    w = np.array([[0.5, 1.5, -0.5, -1.5, 0.49, 2.0, -7.0, 0.0]], np.float32)
    assert orc.ternarize(w, 1.0).tolist() == [[0, 1, 0, -1, 0, 1, -1, 0]]
    assert orc.ternarize(w, 1.0).tolist() == torch.from_numpy(w).round().clamp(-1, 1).to(torch.int8).tolist()


def test_byte_kats():
    # packages/inference/tests/test_bitnet_core.py:186-201: 0x00 -> -1, 0x55 -> 0, 0xAA -> +1
    for byte, val in ((0x00, -1), (0x55, 0), (0xAA, 1)):
        w = orc.unpack_i2s(np.full((2, 32), byte, np.uint8))
        assert (w == val).all()


@pytest.mark.parametrize("field,byte", [(0, 0x95), (1, 0x65), (2, 0x59), (3, 0x56)])
def test_single_weight_kat(field, byte):
    # hand-derived from the I2_S rule: only w[128b + 32*field + j] = +1 -> byte j = that pattern, rest 0x55
    for b, j in ((0, 0), (1, 17), (2, 31)):
        q = np.zeros((1, 384), np.int8)
        q[0, 128 * b + 32 * field + j] = 1
        p = orc.pack_i2s(q)
        expect = np.full(96, 0x55, np.uint8)
        expect[32 * b + j] = byte
        assert p[0].tolist() == expect.tolist()


@pytest.mark.parametrize("shape", [(128, 128), (256, 512), (512, 256), (2560, 2560)])
def test_pack_unpack_roundtrip(shape):
    rng = np.random.default_rng(shape[0])
    q = orc.random_ternary(rng, *shape)
    assert np.array_equal(orc.unpack_i2s(orc.pack_i2s(q)), q)


def test_pack_rejects_bad_k():
    with pytest.raises(ValueError):
        orc.pack_i2s(np.zeros((2, 100), np.int8))


def test_random_ternary_distribution():
    q = orc.random_ternary(np.random.default_rng(3), 1000, 1000)
    frac0 = (q == 0).mean()
    assert abs(frac0 - 0.33) < 0.005 and abs((q == 1).mean() - (q == -1).mean()) < 0.005


# ---- a2: activation quantiser ------------------------------------------------------------------


def test_quantize_closed_forms():
    # max = 127 -> inv = 1 exactly: round half to even on the ties
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]], np.float32)
    q, s = orc.quantize_per_token(x)
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -2, 126]]
    assert s[0] == np.float32(1.0)
    # all-zero row -> max treated as 1, scale 1/127, q 0 (bitnet_gemv.cpp:909-915)
    q, s = orc.quantize_per_token(np.zeros((2, 64), np.float32))
    assert (q == 0).all() and (s == np.float32(1.0) / np.float32(127.0)).all()
    # a single spike maps to +-127
    x = np.zeros((1, 256), np.float32)
    x[0, 17] = -3.25
    q, _ = orc.quantize_per_token(x)
    assert q[0, 17] == -127 and (np.delete(q[0], 17) == 0).all()
    # k_pad columns are zero
    q, _ = orc.quantize_per_token(np.ones((3, 576), np.float32), k_pad=640)
    assert q.shape == (3, 640) and (q[:, 576:] == 0).all() and (q[:, :576] == 127).all()


def test_per_tensor_vs_per_token():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    x[2] *= 10
    qt, st = orc.quantize_per_tensor(x)
    qr, sr = orc.quantize_per_token(x)
    assert st[0] == sr.max()
    assert np.array_equal(qt[2], qr[2])


# ---- a3: RMSNorm -------------------------------------------------------------------------------


def test_rmsnorm_order_matches_float64_except_near_ties():
    rng = np.random.default_rng(5)
    for h in (576, 2560, 6912):
        x = orc.outlier_hidden(rng, 16, h)
        xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        g = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
        q1, s1 = orc.rmsnorm_quant(xb, g, 1e-6, exact_order=True)
        q2, s2 = orc.rmsnorm_quant(xb, g, 1e-6, exact_order=False)
        assert np.allclose(s1, s2, rtol=1e-6)
        diff = q1.astype(int) - q2.astype(int)
        assert np.abs(diff).max() <= 1
        assert (diff != 0).mean() < 1e-3


def _bruteforce_block_order(x):
    h = x.shape[1]
    acc = [np.float32(0.0)] * 256
    for it in range((h + 2047) // 2048):
        for t in range(256):
            for e in range(8):
                i = (it * 256 + t) * 8 + e
                if i < h:
                    acc[t] = np.float32(acc[t] + np.float32(x[0, i] * x[0, i]))
    waves = [acc[64 * w:64 * w + 64] for w in range(4)]
    for o in (32, 16, 8, 4, 2, 1):
        waves = [[np.float32(wv[i] + wv[i ^ o]) for i in range(64)] for wv in waves]
    tot = waves[0][0]
    for w in range(1, 4):
        tot = np.float32(tot + waves[w][0])
    return tot


def _bruteforce_wave_order(x):
    h = x.shape[1]
    acc = [np.float32(0.0)] * 64
    for j in range((h + 511) // 512):
        for lane in range(64):
            for e in range(8):
                i = (lane + 64 * j) * 8 + e
                if i < h:
                    acc[lane] = np.float32(acc[lane] + np.float32(x[0, i] * x[0, i]))
    for o in (32, 16, 8, 4, 2, 1):
        acc = [np.float32(acc[i] + acc[i ^ o]) for i in range(64)]
    return acc[0]


@pytest.mark.parametrize("h", [576, 2560, 4096, 4352, 6912])
def test_rmsnorm_sum_order_bruteforce(h):
    # pure-python loops of the stated orders (one wave per row up to 4096, else 256 threads per row)
    rng = np.random.default_rng(h)
    x = rng.standard_normal((1, h)).astype(np.float32)
    tot = _bruteforce_wave_order(x) if h <= orc.WAVE_MAX_H else _bruteforce_block_order(x)
    assert orc._sum_squares_device_order(x)[0] == tot
    assert abs(float(tot) - float((x.astype(np.float64) ** 2).sum())) < 1e-4 * float(tot)


def test_rmsnorm_closed_form():
    # constant row c: mean(x^2) = c^2, y = c / sqrt(c^2 + eps) * gamma
    x = np.full((1, 512), 2.0, np.float32)
    y = orc.rmsnorm(x, None, 0.0)
    assert np.all(y == np.float32(1.0))


# ---- a4/a5: accumulators ------------------------------------------------------------------------


def test_accumulate_identities_small():
    rng = np.random.default_rng(13)
    packed = orc.pack_i2s(orc.random_ternary(rng, 9, 256))
    a = orc.random_int8(rng, 3, 256)
    a[0, :5] = -128
    acc = orc.accumulate(packed, a)
    assert np.array_equal(acc, orc.accumulate_bruteforce(packed, a))
    assert np.array_equal(acc, orc.accumulate_code_identity(packed, a))
    # transposed-operand / wrong-field mistakes would fail this: compare with a direct int matmul
    w = orc.unpack_i2s(packed).astype(np.int64)
    assert np.array_equal(acc, a.astype(np.int64) @ w.T)


def test_accumulate_fp32_exact_at_full_size():
    # fp32 GEMM of the unpacked weights is exact here (all partial sums < 2^24); used by GPU tests
    rng = np.random.default_rng(17)
    packed = orc.pack_i2s(orc.random_ternary(rng, 512, 6912))
    a = orc.random_int8(rng, 4, 6912)
    w = orc.unpack_i2s(packed).astype(np.float32)
    assert np.array_equal((a.astype(np.float32) @ w.T).astype(np.int64), orc.accumulate(packed, a))


def test_rescale_and_bf16():
    acc = np.array([[100, -3, 0]], np.int64)
    y = orc.rescale(acc, 0.5, np.array([2.0], np.float32), bias=np.array([1.0, 0.0, -1.0], np.float32))
    assert y.tolist() == [[101.0, -3.0, -1.0]]
    b = orc.f32_to_bf16_bits(np.array([1.0, 1.00390625, 1.01171875, -2.5], np.float32))
    assert orc.bf16_bits_to_f32(b).tolist() == [1.0, 1.0, 1.015625, -2.5]
    t = torch.tensor([0.1, -1234.567, 3.3e-5], dtype=torch.float32)
    assert np.array_equal(orc.f32_to_bf16_bits(t.numpy()), t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


# ---- C restatement -------------------------------------------------------------------------------


def test_c_oracle_matches_numpy():
    c = refbind.OracleC()
    rng = np.random.default_rng(19)
    packed = orc.pack_i2s(orc.random_ternary(rng, 33, 640))
    a = orc.random_int8(rng, 3, 640)
    assert np.array_equal(c.acc(packed, a).astype(np.int64), orc.accumulate(packed, a))
    x = rng.standard_normal(640).astype(np.float32)
    q, s = c.quantize(x)
    q2, s2 = orc.quantize_per_tensor(x)
    assert np.array_equal(q, q2) and s == s2[0]


@pytest.mark.parametrize("k", [128, 384, 640, 2560, 6912, 14336])
def test_avx2_port_matches_oracle(k):
    """The AVX2 port of the reference GEMV op (bench.py's CPU baseline): exact integer dots, odd block
    counts (the one-block tail), extreme activations (-128 and 127 in every field) and batches."""
    c = refbind.OracleC()
    rng = np.random.default_rng(100 + k)
    packed = orc.pack_i2s(orc.random_ternary(rng, 37, k))
    a = orc.random_int8(rng, 5, k)
    a[1] = 127
    a[2] = -128
    want = orc.accumulate(packed, a)  # [batch, out]
    for b in range(a.shape[0]):
        assert np.array_equal(c.gemv_avx2(packed, a[b], 1.0).astype(np.int64), want[b])
    got = c.gemm_avx2(packed, a, 1.0)  # [out, batch]
    assert np.array_equal(got.T.astype(np.int64), want)
    ws = np.float32(0.0371)
    assert np.array_equal(c.gemv_avx2(packed, a[0], ws), (want[0].astype(np.float32) * ws).astype(np.float32))


def test_avx2_port_rejects_bad_k():
    c = refbind.OracleC()
    with pytest.raises(ValueError):
        c.gemv_avx2(np.zeros((4, 25), np.uint8), np.zeros(100, np.int8), 1.0)


# ---- the reference's own kernels: golden fixtures and oracle/_ref ----------------------------------


def _golden():
    if not GOLDEN.exists():
        pytest.skip("golden fixture missing")
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("k", [128, 256, 640, 2560, 6912])
def test_golden_vec_dot(k):
    g = _golden()
    acc = orc.accumulate(g[f"dot_k{k}_packed"], g[f"dot_k{k}_act"])[0]
    assert np.array_equal(acc.astype(np.float32), g[f"dot_k{k}_out"])


def test_golden_gemm_layout():
    g = _golden()
    acc = orc.accumulate(g["gemm_packed"], g["gemm_act"])  # [batch, out]
    y = orc.rescale(acc, g["gemm_scale"][0])
    assert np.array_equal(y.T, g["gemm_out"])  # reference writes [out, batch]


@pytest.mark.parametrize("case", ["rand", "ties", "zero", "tiny", "outl"])
def test_golden_quantize(case):
    g = _golden()
    q, s = orc.quantize_per_tensor(g[f"quant_{case}_in"])
    assert np.array_equal(q, g[f"quant_{case}_q"])
    assert s[0] == g[f"quant_{case}_scale"][0]


def _ref(path=refbind.REF_AVX2):
    if not refbind.RefLib.exists(path):
        pytest.skip("reference build (oracle/_ref) not present")
    return refbind.RefLib(path)


@pytest.mark.parametrize("k", [128, 640, 2560, 6912, 14336])
def test_reference_build_matches_oracle(k):
    ref = _ref()
    rng = np.random.default_rng(k)
    packed = orc.pack_i2s(orc.random_ternary(rng, 16, k))
    a = orc.random_int8(rng, 1, k)[0]
    got = ref.gemv(packed, a, 1.0)
    assert np.array_equal(got.astype(np.int64), orc.accumulate(packed, a)[0])


@pytest.mark.parametrize("n,k", [(2560, 2560), (3200, 2560), (13824, 2560), (2560, 6912)])
def test_avx2_port_equals_reference_build(n, k):
    """bench.py's CPU baseline is our AVX2 port; on the four BitNet-2B decode shapes its fp32 outputs
    equal the reference's own compiled bitnet_gemv op bit for bit (scale applied as float(acc) * s)."""
    ref = _ref()
    c = refbind.OracleC()
    rng = np.random.default_rng(n + k)
    packed = orc.pack_i2s(orc.random_ternary(rng, n, k))
    a = orc.random_int8(rng, 1, k)[0]
    s = float(orc.log_uniform(rng))
    assert np.array_equal(c.gemv_avx2(packed, a, s), ref.gemv(packed, a, s))


def test_reference_build_rejects_bad_k():
    ref = _ref()
    with pytest.raises(ValueError):
        ref.vec_dot(np.zeros(25, np.uint8), np.zeros(100, np.int8))


def test_reference_avx512_anomaly_documented():
    """With the reference CMake's AVX-512 flags, K >= 8192 takes a 64-byte interleave that is not
    I2_S (bitnet_gemv.cpp:404-460): its result differs from the I2_S contract while K < 8192 agrees."""
    if "avx512bw" not in Path("/proc/cpuinfo").read_text():
        pytest.skip("host CPU lacks AVX-512BW")
    ref = _ref(refbind.REF_AVX512)
    rng = np.random.default_rng(23)
    for k, agree in ((6912, True), (8192, False)):
        packed = orc.pack_i2s(orc.random_ternary(rng, 8, k))
        a = orc.random_int8(rng, 1, k)[0]
        got = ref.gemv(packed, a, 1.0).astype(np.int64)
        assert np.array_equal(got, orc.accumulate(packed, a)[0]) == agree


# ---- gated activation (fixed-sequence SiLU, relu^2) and segmented rescale ------------------------


def test_exp2_fixed_exact_powers_and_accuracy():
    n = np.arange(-125, 126).astype(np.float32)
    assert np.array_equal(orc.exp2_fixed(n), np.exp2(n.astype(np.float64)).astype(np.float32))
    t = np.linspace(-125, 125, 200001).astype(np.float32)
    ref = np.exp2(t.astype(np.float64))
    assert float((np.abs(orc.exp2_fixed(t) - ref) / ref).max()) < 1e-7
    # clamping keeps 2^n a normal number
    assert orc.exp2_fixed(np.float32(200.0)) == np.float32(2.0 ** 125)
    assert orc.exp2_fixed(np.float32(-200.0)) == np.float32(2.0 ** -125)


def test_silu_fixed_against_float64():
    x = np.linspace(-16, 16, 400001).astype(np.float32)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    got = orc.silu_fixed(x).astype(np.float64)
    nz = np.abs(ref) > 0
    assert float((np.abs(got - ref)[nz] / np.abs(ref)[nz]).max()) < 1e-6
    wide = np.linspace(-1e4, 1e4, 200001).astype(np.float32)
    refw = wide.astype(np.float64) * 0.5 * (1.0 + np.tanh(wide.astype(np.float64) / 2.0))
    assert float(np.abs(orc.silu_fixed(wide) - refw).max()) < 2e-6
    assert orc.silu_fixed(np.float32(0.0)) == 0.0
    assert orc.silu_fixed(np.float32(100.0)) == np.float32(100.0)


def test_relu2_gate_closed_form():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(10000) * 4).astype(np.float32)
    u = rng.standard_normal(10000).astype(np.float32)
    v = orc.glu(g, u, orc.ACT_RELU2)
    assert np.all(v[g <= 0] == 0)
    pos = g > 0
    ref = (np.float64(1) * g[pos] * g[pos] * u[pos])
    assert float((np.abs(v[pos] - ref) / np.maximum(np.abs(ref), 1e-30)).max()) < 2.5e-7  # two fp32 roundings
    with pytest.raises(ValueError):
        orc.glu(g, u, 7)


def test_glu_silu_gate_product_and_norm_quant_composition():
    rng = np.random.default_rng(6)
    g = rng.standard_normal((3, 1536)).astype(np.float32)
    u = rng.standard_normal((3, 1536)).astype(np.float32)
    v = orc.glu(g, u, orc.ACT_SILU)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert float(np.abs(v - ref).max()) < 1e-5
    q, s = orc.glu_rmsnorm_quant(g, u, orc.ACT_SILU, None, 1e-6, 1536)
    q2, s2 = orc.rmsnorm_quant(v, None, 1e-6, 1536)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_rescale_segmented_equals_per_segment_rescale():
    rng = np.random.default_rng(8)
    rows = [16, 8, 40]
    acc = rng.integers(-10000, 10000, size=(3, sum(rows)))
    ws = orc.log_uniform(rng, 3)
    a_s = orc.log_uniform(rng, 3)
    y = orc.rescale_segmented(acc, rows, ws, a_s)
    parts, r0 = [], 0
    for r, w in zip(rows, ws):
        parts.append(orc.rescale(acc[:, r0:r0 + r], w, a_s))
        r0 += r
    assert np.array_equal(y, np.concatenate(parts, axis=1))


# ---- HF offline ternary layout (load-time conversion) ----------------------------------------


def test_hf_offline_unpack_docstring_example():
    """The 8-row example of transformers' BitNet unpack_weights docstring (an independent statement of
    the layout: byte j holds rows j, j+NB, j+2NB, j+3NB from the low bits up)."""
    packed = np.array([[0b10100001, 0b00011000], [0b10010000, 0b00001010]], dtype=np.uint8)
    expect = [[0, -1], [-1, 1], [-1, 1], [-1, 1], [1, 0], [0, -1], [1, -1], [1, -1]]
    assert orc.unpack_hf_offline(packed).tolist() == expect


@pytest.mark.parametrize("n,k", [(8, 3), (12, 256), (13, 130), (4, 1)])
def test_hf_offline_unpack_matches_transformers_pack(n, k):
    """Round trip through transformers' own pack_weights (its rows past n are code 0, i.e. -1)."""
    tb = pytest.importorskip("transformers.integrations.bitnet")
    rng = np.random.default_rng(n * 100 + k)
    w = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    packed = tb.pack_weights(torch.from_numpy(w.copy())).numpy()
    assert packed.shape == ((n + 3) // 4, k)
    assert np.array_equal(orc.unpack_hf_offline(packed, n), w)


def test_hf_offline_layout_comment_of_the_reference_packer():
    """quantize_dlm_to_offline.py:31-33: for 8 rows byte 0 has rows [0,2,4,6], byte 1 has [1,3,5,7]."""
    w = np.zeros((8, 1), dtype=np.int8)
    w[[0, 2, 4, 6], 0] = 1   # code 2 in every field of byte 0
    packed = np.zeros((2, 1), dtype=np.uint8)
    packed[0, 0] = 0b10101010
    packed[1, 0] = 0b01010101
    assert np.array_equal(orc.unpack_hf_offline(packed), w)


def test_hf_offline_convert_scale_closed_form():
    rng = np.random.default_rng(4)
    w = rng.integers(-1, 2, size=(40, 256)).astype(np.int8)
    w[:, :7] = 0
    packed = np.zeros((10, 256), dtype=np.uint8)
    for i in range(4):
        packed |= ((w[10 * i:10 * (i + 1)] + 1).astype(np.uint8) << (2 * i))
    ws = np.float32(0.0371)
    q, s = orc.convert_hf_offline(packed, ws)
    assert np.array_equal(orc.unpack_i2s(q), w)
    # the reference repack: mean(|w * ws|) -- here in float64, rounded once
    assert s == np.float32(np.abs(w.astype(np.float64) * np.float64(ws)).mean())
    assert orc.convert_hf_offline(packed, ws, mode="checkpoint")[1] == ws
    z = np.full((2, 128), 0x55, dtype=np.uint8)  # all zero weights -> scale 1
    assert orc.convert_hf_offline(z, ws)[1] == np.float32(1.0)
