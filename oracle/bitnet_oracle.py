"""CPU oracle for the ternary BitLinear hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference algorithm.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may use this module, and only as the checker; no product code imports it.

Reference files (paths under the reference repository):
  PACK = packages/inference/scripts/convert_to_sglkernel.py
  GEMV = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp
  ENG  = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/inference/bitnet_engine.cpp
  OPS  = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp
  METH = packages/inference/extern/sglang-bitnet/python/sglang/srt/layers/quantization/bitnet.py
  SUBLN = packages/training/src/wrinklefree/models/subln.py
  FUSED = packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp
  MSK  = packages/inference/extern/BitNet/gpu/bitnet_kernels/bitnet_kernels.h

How each function is pinned (see tests/test_oracle.py):
  absmean_scale        KAT [1,-2,3,-4] -> 2.5; torch's own fp32 mean (the reference's library call).
  ternarize / pack     byte KATs 0x00/0x55/0xAA and the single-weight KAT 0x95; the reference's
                       compiled kernels (oracle/_ref) and its golden fixtures; round trips.
  quantize_*           closed-form special cases (zero row, spike -> +-127, exact .5 ties) and the
                       reference's compiled quantize_activations_i8 (golden fixtures).
  rmsnorm_quant        float64 recomputation (codes may differ only at near-ties) and a brute
                       force of the stated summation order on small rows.
  accumulate           the reference's compiled bitnet_vec_dot_i2_i8 / bitnet_gemm_i2_i8 (golden
                       fixtures and oracle/_ref), int64 brute force, and the identity
                       sum(code*a) - sum(a) = sum(w*a).
  exp2_fixed / silu_fixed / glu
                       float64 exp2 / silu (relative error bound), exact powers of two, the
                       relu^2 closed form; the composition glu_rmsnorm_quant = rmsnorm_quant(glu).
  rescale_segmented    equals rescale of each segment with its own scale (the separate-call form).
  unpack_hf_offline    transformers' own BitNet pack_weights (an independent implementation of the
                       layout) round trips through it; the 8-row example of its unpack_weights
                       docstring and the byte/row mapping comment of quantize_dlm_to_offline.py:31-33.
  convert_hf_offline   codes = unpack_hf_offline then pack_i2s; the scale's closed form checked against
                       an fp64 mean of |w * weight_scale|.
"""

from __future__ import annotations

import numpy as np

QK_I2_S = 128  # GEMV bitnet_gemv.h:29
F32 = np.float32


# ---- a1: weight scale, ternarisation, I2_S layout ----------------------------------------------


def absmean_scale(w: np.ndarray) -> np.float32:
    """mean(|W|) rounded to fp32 from an exact-enough float64 sum; < 1e-8 -> 1.0 (PACK:81-85)."""
    s = F32(np.abs(w.astype(np.float64)).sum() / w.size) if w.size else F32(0.0)
    return F32(1.0) if float(s) < 1e-8 else s


def absmean_scale_device_order(w: np.ndarray, blocks: int = 1024) -> np.float32:
    """The device kernel's deterministic fp64 summation order (stated in include/wfbitnet.h)."""
    x = np.abs(w.astype(np.float32).ravel()).astype(np.float64)
    n = x.size
    stride = blocks * 256
    pad = (-n) % stride
    xp = np.concatenate([x, np.zeros(pad)]).reshape(-1, blocks, 256)
    acc = np.zeros((blocks, 256))
    for row in xp:  # thread-sequential over grid-stride iterations
        acc = acc + row
    part = acc
    o = 128
    while o >= 1:  # tree in shared memory
        part = part[:, :o] + part[:, o:2 * o]
        o //= 2
    partial = part[:, 0]
    fin = np.zeros(256)
    for i in range(0, blocks, 256):
        fin = fin + partial[i:i + 256]
    o = 128
    while o >= 1:
        fin = fin[:o] + fin[o:2 * o]
        o //= 2
    s = F32(fin[0] / n) if n else F32(0.0)
    return F32(1.0) if float(s) < 1e-8 else s


def ternarize(w: np.ndarray, scale) -> np.ndarray:
    """int8 q = clamp(round_half_even(W / s), -1, 1) in fp32 (PACK:87-88)."""
    q = np.rint(w.astype(F32) / F32(scale))
    return np.clip(q, -1, 1).astype(np.int8)


def pack_i2s(q: np.ndarray) -> np.ndarray:
    """I2_S layout of ternary q [N, K] -> uint8 [N, K/4] (PACK:96-111).

    Byte j of 128-weight block b: code[128b+j]<<6 | code[128b+32+j]<<4 | code[128b+64+j]<<2 | code[128b+96+j],
    code = q + 1.
    """
    n, k = q.shape
    if k % QK_I2_S:
        raise ValueError(f"K ({k}) must be multiple of {QK_I2_S}")
    c = (q.astype(np.int16) + 1).astype(np.uint8).reshape(n, k // QK_I2_S, 4, 32)
    b = (c[:, :, 0] << 6) | (c[:, :, 1] << 4) | (c[:, :, 2] << 2) | c[:, :, 3]
    return b.reshape(n, k // 4).astype(np.uint8)


def unpack_i2s(packed: np.ndarray) -> np.ndarray:
    """int8 weights [N, K] from I2_S (the scalar reference decode, ENG:51-81)."""
    n, kb = packed.shape
    p = packed.reshape(n, kb // 32, 1, 32)
    shifts = np.array([6, 4, 2, 0], dtype=np.uint8).reshape(1, 1, 4, 1)
    codes = (p >> shifts) & 3
    return (codes.astype(np.int8) - 1).reshape(n, kb * 4)


def pack_ternary(w: np.ndarray, scale=None):
    """(packed, scale): the whole of pack_ternary_sglkernel (PACK:51-123)."""
    s = absmean_scale(w) if scale is None else F32(scale)
    return pack_i2s(ternarize(w, s)), s


# ---- a2: activation quantisation ---------------------------------------------------------------


def unpack_hf_offline(packed: np.ndarray, n: int | None = None) -> np.ndarray:
    """HF offline ternary layout uint8 [NB, K] -> int8 [n, K] (default n = 4*NB): row r is
    ((packed[r % NB] >> 2*(r // NB)) & 3) - 1 (PACK:221-236 unpack loop; layout stated in
    packages/inference/scripts/quantize_dlm_to_offline.py:72-96).  Code 3 is never written; the
    reference's repack clamps its +2 to +1, so it maps to +1 here."""
    packed = np.asarray(packed, dtype=np.uint8)
    nb = packed.shape[0]
    n = 4 * nb if n is None else n
    rows = np.arange(n)
    codes = (packed[rows % nb] >> (2 * (rows // nb))[:, None].astype(np.uint8)) & 3
    return (np.minimum(codes, 2).astype(np.int8) - 1)


def convert_hf_offline(packed: np.ndarray, weight_scale, n: int | None = None, k_pad: int | None = None,
                       mode: str = "reference"):
    """(I2_S qweight [n, k_pad/4], fp32 scale) of an HF offline tensor.  mode "reference": the scale the
    reference converter writes, mean(|w * weight_scale|) over all 4*NB rows and K columns (PACK:240-242
    repacking through pack_ternary_sglkernel), i.e. weight_scale * nnz / (4*NB*K) rounded once to fp32
    (< 1e-8 -> 1); mode "checkpoint": weight_scale.  The codes are the unpacked ternary values."""
    packed = np.asarray(packed, dtype=np.uint8)
    nb, k = packed.shape
    w_all = unpack_hf_offline(packed)
    n = 4 * nb if n is None else n
    kp = -(-k // QK_I2_S) * QK_I2_S if k_pad is None else k_pad
    w = np.zeros((n, kp), dtype=np.int8)
    w[:, :k] = w_all[:n]
    ws = float(np.float32(weight_scale))
    if mode == "reference":
        s = np.float32(ws * (np.count_nonzero(w_all) / float(4 * nb * k)))
        if float(s) < 1e-8:
            s = np.float32(1.0)
    else:
        s = np.float32(ws)
    return pack_i2s(w), s


def quantize_row_params(mx: np.ndarray):
    """(scale, inv) from the absmax, fp32: max < 1e-6 -> 1 (GEMV:909-915)."""
    mx = np.where(mx < F32(1e-6), F32(1.0), mx).astype(F32)
    return (mx / F32(127.0)).astype(F32), (F32(127.0) / mx).astype(F32)


def quantize_with_inv(x: np.ndarray, inv) -> np.ndarray:
    """sat_i8(round_half_even(x * inv)) in fp32 (GEMV:917-944, vector path)."""
    return np.clip(np.rint(x.astype(F32) * inv), -128, 127).astype(np.int8)


def quantize_per_token(x: np.ndarray, k_pad: int | None = None):
    """Row-wise quantize_activations_i8: (q int8 [M, k_pad], scale fp32 [M])."""
    x = np.asarray(x, dtype=F32).reshape(-1, x.shape[-1])
    mx = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], F32)
    scale, inv = quantize_row_params(mx.astype(F32))
    q = quantize_with_inv(x, inv[:, None])
    if k_pad is not None and k_pad > x.shape[1]:
        q = np.concatenate([q, np.zeros((q.shape[0], k_pad - x.shape[1]), np.int8)], axis=1)
    return q, scale


def quantize_per_tensor(x: np.ndarray):
    """bitnet_quantize_activations_cpu: ONE scale for the flattened buffer (OPS:409-426)."""
    x = np.asarray(x, dtype=F32)
    mx = F32(np.abs(x).max()) if x.size else F32(0.0)
    scale, inv = quantize_row_params(np.array([mx], F32))
    return quantize_with_inv(x, inv[0]), scale


# ---- a3: RMSNorm / SubLN fused with the quantiser ----------------------------------------------


WAVE_MAX_H = 4096  # rows up to this length use the one-wave-per-row order


def _butterfly64(acc: np.ndarray) -> np.ndarray:
    """Fixed xor butterfly over the last axis (64 lanes, offsets 32..1); returns lane 0."""
    lanes = np.arange(64)
    o = 32
    while o >= 1:
        acc = (acc + acc[..., lanes ^ o]).astype(F32)
        o //= 2
    return acc[..., 0]


def _sum_squares_wave_order(x: np.ndarray, vec: int = 8) -> np.ndarray:
    """One wave per row: lane l adds the squares of elements (l + 64*j)*8 + e sequentially over
    (j, e), then the xor butterfly."""
    m, h = x.shape
    per = 64 * vec
    vpl = (h + per - 1) // per
    xp = np.zeros((m, vpl * per), F32)
    xp[:, :h] = x
    xp = xp.reshape(m, vpl, 64, vec)
    acc = np.zeros((m, 64), F32)
    for j in range(vpl):
        for e in range(vec):
            v = xp[:, j, :, e]
            acc = (acc + (v * v).astype(F32)).astype(F32)
    return _butterfly64(acc)


def _sum_squares_device_order(x: np.ndarray, tpb: int = 256, vec: int = 8) -> np.ndarray:
    """fp32 sum of squares per row in the kernel's stated order: the one-wave order for rows up to
    WAVE_MAX_H, else 256 threads per row (thread-sequential over (iteration, element), xor
    butterfly per wave, waves added in order)."""
    m, h = x.shape
    if h <= WAVE_MAX_H:
        return _sum_squares_wave_order(x, vec)
    per_it = tpb * vec
    its = (h + per_it - 1) // per_it
    xp = np.zeros((m, its * per_it), F32)
    xp[:, :h] = x
    xp = xp.reshape(m, its, tpb, vec)
    acc = np.zeros((m, tpb), F32)
    for it in range(its):
        for e in range(vec):
            v = xp[:, it, :, e]
            acc = (acc + (v * v).astype(F32)).astype(F32)
    waves = acc.reshape(m, tpb // 64, 64)
    lanes = np.arange(64)
    o = 32
    while o >= 1:
        waves = (waves + waves[:, :, lanes ^ o]).astype(F32)
        o //= 2
    tot = waves[:, 0, 0]
    for w in range(1, tpb // 64):
        tot = (tot + waves[:, w, 0]).astype(F32)
    return tot


def rmsnorm(x: np.ndarray, gamma=None, eps: float = 1e-6, exact_order: bool = True) -> np.ndarray:
    """y = x * (1 / sqrt(sum(x^2)/H + eps)) * gamma in fp32 (SUBLN:42-59; ENG:172-183 for fp32 form)."""
    x = np.asarray(x, dtype=F32)
    h = x.shape[1]
    if exact_order:
        ss = _sum_squares_device_order(x)
    else:
        ss = (x.astype(np.float64) ** 2).sum(axis=1).astype(F32)
    r = (F32(1.0) / np.sqrt((ss / F32(h)).astype(F32) + F32(eps))).astype(F32)
    y = (x * r[:, None]).astype(F32)
    if gamma is not None:
        y = (y * np.asarray(gamma, dtype=F32)[None, :]).astype(F32)
    return y


def rmsnorm_quant(x: np.ndarray, gamma=None, eps: float = 1e-6, k_pad: int | None = None, exact_order: bool = True):
    """Fused SubLN + per-token int8 quantisation: (q int8 [M, k_pad], scale fp32 [M])."""
    return quantize_per_token(rmsnorm(x, gamma, eps, exact_order), k_pad)


# ---- gated activation before the MLP SubLN (FUSED:200-216, SiLU form of the stage-1 MLP) ------

ACT_SILU, ACT_RELU2 = 1, 2  # codes of include/wfbitnet.h

# ln(2)^k / k!, k = 7 .. 1, as fp32 (Horner coefficients of 2^f on |f| <= 1/2)
_EXP2_C = [F32(1.525273380405984e-05), F32(1.5403530393381606e-04), F32(1.3333558146428443e-03),
           F32(9.618129107628477e-03), F32(5.550410866482158e-02), F32(2.402265069591007e-01),
           F32(6.931471805599453e-01), F32(1.0)]
_LOG2E = F32(1.4426950408889634)


def exp2_fixed(t: np.ndarray) -> np.ndarray:
    """2^t as the kernels evaluate it: t clamped to [-125, 125], n = rint(t), f = t - n,
    p = Horner(_EXP2_C, f) with one rounding per multiply and per add, result p * 2^n (exact)."""
    t = np.minimum(np.maximum(np.asarray(t, F32), F32(-125.0)), F32(125.0))
    n = np.rint(t).astype(F32)
    f = (t - n).astype(F32)
    p = np.full_like(f, _EXP2_C[0])
    for c in _EXP2_C[1:]:
        p = (p * f).astype(F32)
        p = (p + c).astype(F32)
    return np.ldexp(p, n.astype(np.int32)).astype(F32)


def silu_fixed(g: np.ndarray) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)), exp(-g) = exp2_fixed(-g * log2(e)), fp32 step by step."""
    g = np.asarray(g, F32)
    e = exp2_fixed(((-g).astype(F32) * _LOG2E).astype(F32))
    return (g / (F32(1.0) + e).astype(F32)).astype(F32)


def glu(gate: np.ndarray, up: np.ndarray, act: int) -> np.ndarray:
    """act(gate) * up in fp32: silu (ACT_SILU) or relu^2 (ACT_RELU2, max(g,0)*max(g,0) then * up)."""
    gate, up = np.asarray(gate, F32), np.asarray(up, F32)
    if act == ACT_SILU:
        return (silu_fixed(gate) * up).astype(F32)
    if act == ACT_RELU2:
        r = np.maximum(gate, F32(0.0))
        return ((r * r).astype(F32) * up).astype(F32)
    raise ValueError(f"unknown activation {act}")


def glu_rmsnorm_quant(gate, up, act: int, gamma=None, eps: float = 1e-6, k_pad: int | None = None):
    """wfb_glu_rmsnorm_quant_i8: rmsnorm_quant of glu(gate, up) (same reduction order)."""
    return rmsnorm_quant(glu(gate, up, act), gamma, eps, k_pad)


# ---- a4 / a5 / a6: accumulators and rescale ---------------------------------------------------


def accumulate(packed: np.ndarray, a: np.ndarray) -> np.ndarray:
    """acc[m, n] = sum_k w[n, k] * a[m, k] as int64 (exact: float64 products/sums stay < 2^53)."""
    w = unpack_i2s(packed).astype(np.float64)
    a2 = np.atleast_2d(a).astype(np.float64)
    return np.rint(a2 @ w.T).astype(np.int64)


def accumulate_bruteforce(packed: np.ndarray, a: np.ndarray) -> np.ndarray:
    """Integer-only brute force (small shapes): per row, per 128-block, the scalar loop of ENG:51-81."""
    n, kb = packed.shape
    a2 = np.atleast_2d(a).astype(np.int64)
    out = np.zeros((a2.shape[0], n), np.int64)
    for r in range(n):
        for blk in range(kb // 32):
            for j in range(32):
                byte = int(packed[r, 32 * blk + j])
                for f, shift in enumerate((6, 4, 2, 0)):
                    w = ((byte >> shift) & 3) - 1
                    out[:, r] += w * a2[:, 128 * blk + 32 * f + j]
    return out


def accumulate_code_identity(packed: np.ndarray, a: np.ndarray) -> np.ndarray:
    """sum_k code * a - sum_k a, the form the SIMD kernel evaluates (GEMV:346-402, 685)."""
    codes = (unpack_i2s(packed).astype(np.int64) + 1).astype(np.float64)
    a2 = np.atleast_2d(a).astype(np.float64)
    return np.rint(a2 @ codes.T).astype(np.int64) - a2.sum(axis=1, keepdims=True).astype(np.int64)


def rescale(acc: np.ndarray, w_scale, a_scale=None, bias=None) -> np.ndarray:
    """y = (float(acc) * w_scale) * a_scale[m] (+ bias) in fp32 (GEMV:846; METH:241, 253)."""
    y = (acc.astype(F32) * F32(w_scale)).astype(F32)
    if a_scale is not None:
        y = (y * np.asarray(a_scale, F32).reshape(-1, 1)).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32).reshape(1, -1)).astype(F32)
    return y


def rescale_segmented(acc: np.ndarray, seg_rows, w_scales, a_scale=None, bias=None) -> np.ndarray:
    """wfb_linear_i2s_segmented: output column n takes the scale of its weight segment (MSK:80-82
    with explicit segment sizes); equal to rescale() of each segment with its own scale."""
    ends = np.cumsum(np.asarray(seg_rows, np.int64))
    seg = np.searchsorted(ends, np.arange(acc.shape[-1]), side="right")
    ws = np.asarray(w_scales, F32)[seg]
    y = (acc.astype(F32) * ws.reshape(1, -1)).astype(F32)
    if a_scale is not None:
        y = (y * np.asarray(a_scale, F32).reshape(-1, 1)).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32).reshape(1, -1)).astype(F32)
    return y


def f32_to_bf16_bits(y: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.asarray(y, F32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(F32)


def bitlinear_forward(x: np.ndarray, packed: np.ndarray, w_scale, bias=None):
    """Quantised BitLinear forward (per-token activations): (y fp32 [M, N], acc int64, q, a_scale)."""
    q, a_scale = quantize_per_token(x, k_pad=packed.shape[1] * 4)
    acc = accumulate(packed, q)
    return rescale(acc, w_scale, a_scale, bias), acc, q, a_scale


# ---- synthetic inputs of the benchmark configurations -------------------------------------------


def random_ternary(rng: np.random.Generator, n: int, k: int, p_zero: float = 0.33) -> np.ndarray:
    """i.i.d. ternary with P(0) = p_zero and P(+1) = P(-1)."""
    u = rng.random((n, k))
    half = (1.0 - p_zero) / 2.0
    return np.where(u < half, -1, np.where(u < half + p_zero, 0, 1)).astype(np.int8)


def random_int8(rng: np.random.Generator, m: int, k: int) -> np.ndarray:
    """int8 uniform on [-127, 127]."""
    return rng.integers(-127, 128, size=(m, k), dtype=np.int16).astype(np.int8)


def log_uniform(rng: np.random.Generator, size=None, lo: float = 1e-3, hi: float = 1.0):
    return np.exp(rng.uniform(np.log(lo), np.log(hi), size=size)).astype(F32)


def outlier_hidden(rng: np.random.Generator, m: int, h: int, frac: float = 0.01, mag: float = 20.0) -> np.ndarray:
    """N(0,1) hidden states with a fraction replaced by +-mag (random sign)."""
    x = rng.standard_normal((m, h)).astype(F32)
    mask = rng.random((m, h)) < frac
    x[mask] = np.where(rng.random(mask.sum()) < 0.5, -mag, mag).astype(F32)
    return x
