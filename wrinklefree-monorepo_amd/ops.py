"""Torch-facing ops over the C ABI: the MI355X counterparts of the reference BitNet op wrappers.

Names, argument meaning and error behaviour follow the reference wrappers
(SGB/sgl-kernel/python/sgl_kernel/quantization/bitnet.py:73-179) and the torch ops they call
(SGB/sgl-kernel/csrc/cpu/torch_extension_cpu.cpp:331-426); SGB = packages/inference/extern/sglang-bitnet.
Differences, all deliberate:
  * tensors live on the GPU and work is enqueued on the current HIP stream (no host sync);
  * ``scale`` may be a Python float or a 1-element fp32 device tensor (no ``.item()`` sync);
  * ``bitnet_gemm`` returns [batch, out] directly (the reference op fills [out, batch] and its
    wrapper transposes, bitnet.py:139-145);
  * non-contiguous inputs are rejected instead of being read through ``data_ptr`` as if contiguous.
The ops are also registered as ``torch.ops.wfbitnet.*`` with the reference schemas.
"""

from __future__ import annotations

import collections
import ctypes
import weakref
from typing import Optional, Sequence, Tuple, Union

import torch

from . import _lib
from ._lib import (WFB_ABSMEAN_WS_DOUBLES, WFB_ACT_RELU2, WFB_ACT_SILU, WFB_BF16, WFB_F16, WFB_F32,
                   WFB_MAX_SEGMENTS, WFB_QK_I2S, WFB_SCALE_CHECKPOINT, WFB_SCALE_REFERENCE)

QK_I2_S = WFB_QK_I2S

_DT = {torch.float32: WFB_F32, torch.bfloat16: WFB_BF16, torch.float16: WFB_F16}

Scale = Union[float, torch.Tensor]


def check_kernel_available() -> bool:
    """True when libwfbitnet loads and a HIP device is visible (reference: bitnet.py:38-44)."""
    return _lib.available() and torch.cuda.is_available()


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _require_gpu(name: str, *ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{name}: tensors must be on a HIP device (got {t.device})")
        if not t.is_contiguous():
            raise RuntimeError(f"{name}: tensors must be contiguous")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name}: tensors are on different devices ({dev}, {t.device})")
    assert dev is not None
    return dev


def _float_dtype(name: str, t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise RuntimeError(f"{name}: expected float32, bfloat16 or float16, got {t.dtype}")
    return _DT[t.dtype]


def _scale_args(name: str, scale: Scale, dev: torch.device):
    """(device pointer or None, host float) for the C ABI's w_scale_dev / w_scale pair."""
    if isinstance(scale, torch.Tensor):
        if scale.dtype != torch.float32 or scale.numel() != 1 or scale.device != dev:
            raise RuntimeError(f"{name}: scale tensor must be one fp32 element on {dev}")
        return _p(scale.contiguous()), 0.0
    return None, float(scale)


# ---- a1: offline pack -------------------------------------------------------------------------


def absmean_scale(weights: torch.Tensor) -> torch.Tensor:
    """fp32[1] device tensor holding mean(|W|) (< 1e-8 -> 1.0), as convert_to_sglkernel.py:81-85."""
    name = "absmean_scale"
    dev = _require_gpu(name, weights)
    dt = _float_dtype(name, weights)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    ws = torch.empty(WFB_ABSMEAN_WS_DOUBLES, dtype=torch.float64, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_weight_absmean", _p(weights), dt, weights.numel(), _p(scale), _p(ws), _stream(dev))
    return scale


def pack_ternary_i2s(
    weights: torch.Tensor, scale: Optional[torch.Tensor] = None, k_pad: Optional[int] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Ternarise and pack W [out, in] to I2_S: (qweight uint8 [out, k_pad/4], scale fp32[1]).

    Device counterpart of pack_ternary_sglkernel (packages/inference/scripts/convert_to_sglkernel.py:51-123).
    ``scale`` defaults to absmean(W) over the real columns.  ``k_pad`` (a multiple of 128, >= in)
    zero-pads K: padded weights are 0 (code 01), so accumulators are unchanged.
    """
    name = "pack_ternary_i2s"
    if weights.dim() != 2:
        raise RuntimeError(f"{name}: weights must be 2D [out_features, in_features]")
    dev = _require_gpu(name, weights)
    _float_dtype(name, weights)
    n, k = weights.shape
    kp = k if k_pad is None else int(k_pad)
    if kp % QK_I2_S != 0 or kp < k:
        raise ValueError(f"K ({kp}) must be multiple of {QK_I2_S}")
    if scale is None:
        scale = absmean_scale(weights)
    elif scale.dtype != torch.float32 or scale.numel() != 1 or scale.device != dev:
        raise RuntimeError(f"{name}: scale must be one fp32 element on {dev}")
    w = weights
    if kp != k:
        w = torch.zeros((n, kp), dtype=weights.dtype, device=dev)
        w[:, :k] = weights
    packed = torch.empty((n, kp // 4), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_pack_i2s", _p(w), _DT[w.dtype], n, kp, kp, _p(scale.contiguous()), _p(packed), _stream(dev))
    return packed, scale


def unpack_i2s(packed_weights: torch.Tensor) -> torch.Tensor:
    """int8 [out, in] in {-1, 0, +1} from an I2_S tensor (decode of bitnet_engine.cpp:51-81)."""
    name = "unpack_i2s"
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be 2D uint8")
    dev = _require_gpu(name, packed_weights)
    n, kb = packed_weights.shape
    out = torch.empty((n, kb * 4), dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_unpack_i2s", _p(packed_weights), n, kb * 4, _p(out), _stream(dev))
    return out


_SCALE_MODES = {"reference": WFB_SCALE_REFERENCE, "checkpoint": WFB_SCALE_CHECKPOINT}


def convert_hf_offline_i2s(
    packed_hf: torch.Tensor, weight_scale: Scale = 1.0, out_features: Optional[int] = None,
    k_pad: Optional[int] = None, scale_mode: str = "reference",
) -> Tuple[torch.Tensor, torch.Tensor]:
    """HF offline ternary layout uint8 [ceil(N/4), K] -> (I2_S qweight uint8 [N, k_pad/4], scale fp32 [1]).

    Byte (j, k) of the source holds column k of rows j, j + NB, j + 2NB, j + 3NB (bits 1:0 .. 7:6, code =
    w + 1; packages/inference/scripts/quantize_dlm_to_offline.py:27-98).  ``out_features`` drops the
    padding rows (default 4 * NB).  ``scale_mode="reference"`` gives the scale the reference converter
    writes (its repack takes mean|w * weight_scale|, convert_to_sglkernel.py:221-246);
    ``"checkpoint"`` keeps ``weight_scale``.  ``weight_scale``: float, or a 1-element fp32/bf16 tensor on
    the device (the checkpoint's ``weight_scale``)."""
    name = "convert_hf_offline_i2s"
    if packed_hf.dtype != torch.uint8 or packed_hf.dim() != 2:
        raise RuntimeError(f"{name}: packed_hf must be uint8 [ceil(out/4), in]")
    if scale_mode not in _SCALE_MODES:
        raise ValueError(f"{name}: scale_mode must be one of {sorted(_SCALE_MODES)}")
    dev = _require_gpu(name, packed_hf)
    nb, k = packed_hf.shape
    n = 4 * nb if out_features is None else int(out_features)
    kp = (k + QK_I2_S - 1) // QK_I2_S * QK_I2_S if k_pad is None else int(k_pad)
    ws_ptr, ws_dt, ws_host = None, WFB_F32, 1.0
    if isinstance(weight_scale, torch.Tensor):
        if weight_scale.numel() != 1 or weight_scale.dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError(f"{name}: weight_scale tensor must be one fp32 or bf16 element")
        wst = weight_scale.to(dev).contiguous()
        ws_ptr, ws_dt = _p(wst), _DT[wst.dtype]
    else:
        ws_host = float(weight_scale)
    qweight = torch.empty((n, kp // 4), dtype=torch.uint8, device=dev)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    work = torch.empty((n * (kp // 16) + 255) // 256 + 1, dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_convert_hf_offline_i2s", _p(packed_hf), nb, n, k, kp, ws_ptr, ws_dt, ws_host,
                  _SCALE_MODES[scale_mode], _p(qweight), _p(scale), _p(work), _stream(dev))
    return qweight, scale


# ---- a2 / a3: activation quantisation ----------------------------------------------------------


def quantize_activations_i8(activations: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-TENSOR absmax int8 quantisation: (int8 same shape, fp32[1] scale).

    Same contract as the reference wrapper / op (bitnet.py:155-179, torch_extension_cpu.cpp:409-426):
    one scale for the whole buffer.  The BitLinear path uses the per-token variant below.
    """
    name = "quantize_activations_i8"
    dev = _require_gpu(name, activations)
    dt = _float_dtype(name, activations)
    q = torch.empty(activations.shape, dtype=torch.int8, device=dev)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_quantize_act_i8_tensor", _p(activations), dt, activations.numel(), _p(q), _p(scale), _stream(dev))
    return q, scale


def _rows(name: str, x: torch.Tensor, k_pad: Optional[int]):
    if x.dim() < 1:
        raise RuntimeError(f"{name}: input must have a feature dimension")
    h = x.shape[-1]
    kp = h if k_pad is None else int(k_pad)
    if kp < h:
        raise ValueError(f"{name}: k_pad ({kp}) < features ({h})")
    kp_alloc = (kp + 15) // 16 * 16  # rows of q are 16-byte aligned for the 128-bit loads
    m = x.numel() // h if h else 0
    return h, kp, kp_alloc, m


def quantize_activations_i8_per_token(
    x: torch.Tensor, k_pad: Optional[int] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token absmax int8: (q int8 [..., k_pad], a_scale fp32 [...]).

    The quantiser of bitnet_gemv.cpp:880-1135 applied row by row (the per-token form of
    WF/models/bitlinear.py:66-84 used by the decode engine, bitnet_engine.cpp:268).
    """
    name = "quantize_activations_i8_per_token"
    dev = _require_gpu(name, x)
    dt = _float_dtype(name, x)
    h, kp, kpa, m = _rows(name, x, k_pad)
    q = torch.empty((*x.shape[:-1], kpa), dtype=torch.int8, device=dev)
    a_scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("wfb_quantize_act_i8", _p(x), dt, m, h, h, _p(q), kpa, kpa, _p(a_scale), _stream(dev))
    return (q if kpa == kp else q[..., :kp]), a_scale


def rmsnorm_quantize_i8(
    x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6, k_pad: Optional[int] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused RMSNorm/SubLN + per-token int8 quantisation: (q int8 [..., k_pad], a_scale fp32 [...]).

    y = x / sqrt(mean(x^2) + eps) * weight (WF/models/subln.py:42-59) in fp32, then the quantiser.
    """
    name = "rmsnorm_quantize_i8"
    dev = _require_gpu(name, x, weight)
    dt = _float_dtype(name, x)
    gdt = _float_dtype(name, weight) if weight is not None else WFB_F32
    h, kp, kpa, m = _rows(name, x, k_pad)
    if weight is not None and weight.numel() != h:
        raise RuntimeError(f"{name}: weight has {weight.numel()} elements, expected {h}")
    q = torch.empty((*x.shape[:-1], kpa), dtype=torch.int8, device=dev)
    a_scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call(
            "wfb_rmsnorm_quant_i8", _p(x), dt, h, _p(weight), gdt, float(eps), m, h, _p(q), kpa, kpa, _p(a_scale), _stream(dev)
        )
    return (q if kpa == kp else q[..., :kp]), a_scale


# ---- a4 / a5 / a6: ternary linear ----------------------------------------------------------------

_KERNELS = {"auto": "wfb_linear_i2s", "gemv": "wfb_gemv_i2s", "gemm": "wfb_gemm_i2s"}


def bitnet_linear(
    packed_weights: torch.Tensor,
    activations: torch.Tensor,
    scale: Scale,
    a_scale: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = torch.bfloat16,
    return_acc: bool = False,
    kernel: str = "auto",
):
    """y[m, n] = acc[m, n] * scale * a_scale[m] (+ bias[n]) for int8 activations [M, K] (or [K]).

    Returns y ([M, N] or [N], ``out_dtype`` bf16/fp32), or (y, acc int32) with ``return_acc``;
    ``out_dtype=None`` computes only acc.  ``kernel`` forces "gemv" (M <= 2) or "gemm" (MFMA).
    """
    name = "bitnet_linear"
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [out_features, in_features/4]")
    if activations.dtype != torch.int8 or activations.dim() not in (1, 2):
        raise RuntimeError(f"{name}: activations must be int8 [in_features] or [batch, in_features]")
    n, kb = packed_weights.shape
    k = kb * 4
    if k % QK_I2_S != 0:
        raise ValueError(f"{name}: in_features ({k}) must be multiple of {QK_I2_S}")
    a2 = activations.view(1, -1) if activations.dim() == 1 else activations
    if a2.shape[1] != k:
        raise ValueError(f"{name}: activations have {a2.shape[1]} features, packed weights {k}")
    m = a2.shape[0]
    dev = _require_gpu(name, packed_weights, a_scale, bias)
    if a2.device != dev:
        raise RuntimeError(f"{name}: activations are on {a2.device}, weights on {dev}")
    if a2.stride(1) != 1 or (m > 1 and a2.stride(0) % 16 != 0) or a2.data_ptr() % 16 != 0:
        a2 = a2.contiguous()
    if a_scale is not None and (a_scale.dtype != torch.float32 or a_scale.numel() != m):
        raise RuntimeError(f"{name}: a_scale must be fp32 with one element per token ({m})")
    ws_dev, ws = _scale_args(name, scale, dev)
    if out_dtype is None and not return_acc:
        raise RuntimeError(f"{name}: nothing to compute (out_dtype=None and return_acc=False)")
    out = None
    odt = 0
    if out_dtype is not None:
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError(f"{name}: out_dtype must be float32 or bfloat16")
        out = torch.empty((m, n), dtype=out_dtype, device=dev)
        odt = _DT[out_dtype]
    acc = torch.empty((m, n), dtype=torch.int32, device=dev) if return_acc else None
    bdt = _float_dtype(name, bias) if bias is not None else 0
    if bias is not None and bias.numel() != n:
        raise RuntimeError(f"{name}: bias has {bias.numel()} elements, expected {n}")
    lda = a2.stride(0) if m > 1 else k
    if kernel not in _KERNELS:
        raise ValueError(f"{name}: kernel must be one of {sorted(_KERNELS)}")
    with torch.cuda.device(dev):
        _lib.call(
            _KERNELS[kernel], _p(packed_weights), n, k, _p(a2), m, lda, _p(a_scale), ws_dev, ws,
            _p(bias), bdt, _p(out), odt, n, _p(acc), _stream(dev),
        )
    if activations.dim() == 1:
        out = None if out is None else out.view(n)
        acc = None if acc is None else acc.view(n)
    return (out, acc) if return_acc else out


def bitnet_linear_segmented(
    packed_weights: torch.Tensor,
    seg_rows,
    scales: torch.Tensor,
    activations: torch.Tensor,
    a_scale: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = torch.bfloat16,
    return_acc: bool = False,
):
    """One launch for several projections that read the same activations (fused QKV, gate|up).

    ``packed_weights`` is the row concatenation of the projections' I2_S weights, ``seg_rows`` their
    row counts (multiples of 8), ``scales`` fp32 [n_seg] on the device: output column n is scaled by
    the scale of its segment.  Equal to separate ``bitnet_linear`` calls on the segments.
    """
    name = "bitnet_linear_segmented"
    rows = [int(r) for r in seg_rows]
    if not 1 <= len(rows) <= WFB_MAX_SEGMENTS:
        raise ValueError(f"{name}: 1..{WFB_MAX_SEGMENTS} segments, got {len(rows)}")
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [out_features, in_features/4]")
    if sum(rows) != packed_weights.shape[0]:
        raise ValueError(f"{name}: segment rows sum to {sum(rows)}, packed_weights has {packed_weights.shape[0]}")
    if scales.dtype != torch.float32 or scales.numel() != len(rows):
        raise RuntimeError(f"{name}: scales must be fp32 with one element per segment")
    if activations.dtype != torch.int8 or activations.dim() not in (1, 2):
        raise RuntimeError(f"{name}: activations must be int8 [in_features] or [batch, in_features]")
    n, kb = packed_weights.shape
    k = kb * 4
    a2 = activations.view(1, -1) if activations.dim() == 1 else activations
    if a2.shape[1] != k:
        raise ValueError(f"{name}: activations have {a2.shape[1]} features, packed weights {k}")
    m = a2.shape[0]
    dev = _require_gpu(name, packed_weights, scales, a_scale, bias)
    if a2.device != dev:
        raise RuntimeError(f"{name}: activations are on {a2.device}, weights on {dev}")
    if a2.stride(1) != 1 or (m > 1 and a2.stride(0) % 16 != 0) or a2.data_ptr() % 16 != 0:
        a2 = a2.contiguous()
    if a_scale is not None and (a_scale.dtype != torch.float32 or a_scale.numel() != m):
        raise RuntimeError(f"{name}: a_scale must be fp32 with one element per token ({m})")
    if out_dtype is None and not return_acc:
        raise RuntimeError(f"{name}: nothing to compute (out_dtype=None and return_acc=False)")
    out, odt = None, 0
    if out_dtype is not None:
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError(f"{name}: out_dtype must be float32 or bfloat16")
        out = torch.empty((m, n), dtype=out_dtype, device=dev)
        odt = _DT[out_dtype]
    acc = torch.empty((m, n), dtype=torch.int32, device=dev) if return_acc else None
    bdt = _float_dtype(name, bias) if bias is not None else 0
    if bias is not None and bias.numel() != n:
        raise RuntimeError(f"{name}: bias has {bias.numel()} elements, expected {n}")
    seg = (ctypes.c_int64 * len(rows))(*rows)
    lda = a2.stride(0) if m > 1 else k
    with torch.cuda.device(dev):
        _lib.call(
            "wfb_linear_i2s_segmented", _p(packed_weights), n, k, len(rows), ctypes.cast(seg, ctypes.c_void_p),
            _p(scales), _p(a2), m, lda, _p(a_scale), _p(bias), bdt, _p(out), odt, n, _p(acc), _stream(dev),
        )
    if activations.dim() == 1:
        out = None if out is None else out.view(n)
        acc = None if acc is None else acc.view(n)
    return (out, acc) if return_acc else out


_ACTS = {"silu": WFB_ACT_SILU, "relu2": WFB_ACT_RELU2}


def glu_rmsnorm_quantize_i8(
    gate: torch.Tensor, up: torch.Tensor, act: str = "silu", weight: Optional[torch.Tensor] = None,
    eps: float = 1e-6, k_pad: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """act(gate) * up -> SubLN (weight) -> per-token int8: (q int8 [..., k_pad], a_scale fp32 [...]).

    ``act`` is "silu" (SwiGLU) or "relu2" (relu(gate)^2, the reference fused MLP,
    bitnet_fused_layer.cpp:200-216).  gate and up must have the same shape and row stride with
    contiguous rows (e.g. the two halves of one gate|up output).
    """
    name = "glu_rmsnorm_quantize_i8"
    if act not in _ACTS:
        raise ValueError(f"{name}: act must be one of {sorted(_ACTS)}")
    if weight is not None:
        _require_gpu(name, weight)
    if gate.device.type != "cuda" or up.device != gate.device or (weight is not None and weight.device != gate.device):
        raise RuntimeError(f"{name}: gate, up and weight must be on one HIP device")
    dev = gate.device
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise RuntimeError(f"{name}: gate and up must have the same shape and dtype")
    dt = _float_dtype(name, gate)
    h = gate.shape[-1]
    g2, u2 = gate.reshape(-1, h), up.reshape(-1, h)
    if g2.stride(-1) != 1 or u2.stride(-1) != 1 or g2.stride(0) != u2.stride(0):
        raise RuntimeError(f"{name}: gate and up need contiguous rows with one common row stride")
    m = g2.shape[0]
    ldx = g2.stride(0) if m > 1 else h
    gdt = _float_dtype(name, weight) if weight is not None else WFB_F32
    if weight is not None and weight.numel() != h:
        raise RuntimeError(f"{name}: weight has {weight.numel()} elements, expected {h}")
    _, kp, kpa, _ = _rows(name, gate, k_pad)
    q = torch.empty((*gate.shape[:-1], kpa), dtype=torch.int8, device=dev)
    a_scale = torch.empty(gate.shape[:-1], dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call(
            "wfb_glu_rmsnorm_quant_i8", _p(g2), _p(u2), dt, ldx, _ACTS[act], _p(weight), gdt, float(eps), m, h,
            _p(q), kpa, kpa, _p(a_scale), _stream(dev),
        )
    return (q if kpa == kp else q[..., :kp]), a_scale


def bitnet_linear_residual(
    packed_weights: torch.Tensor, activations: torch.Tensor, scale: Scale, residual: torch.Tensor,
    a_scale: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """residual + BitLinear in one launch: out[m, n] = acc * scale * a_scale[m] + residual[m, n] (fp32 add,
    stored in residual's dtype, float32 or bfloat16).  ``out`` may be ``residual`` itself (in place)."""
    name = "bitnet_linear_residual"
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [out_features, in_features/4]")
    if activations.dtype != torch.int8 or activations.dim() != 2:
        raise RuntimeError(f"{name}: activations must be int8 [batch, in_features]")
    n, kb = packed_weights.shape
    k = kb * 4
    if k % QK_I2_S != 0 or activations.shape[1] != k:
        raise ValueError(f"{name}: in_features must be a multiple of {QK_I2_S} and match the weights")
    m = activations.shape[0]
    dev = _require_gpu(name, packed_weights, a_scale)
    a2 = activations
    if a2.device != dev or residual.device != dev:
        raise RuntimeError(f"{name}: tensors must be on {dev}")
    if a2.stride(1) != 1 or (m > 1 and a2.stride(0) % 16 != 0) or a2.data_ptr() % 16 != 0:
        a2 = a2.contiguous()
    if a_scale is not None and (a_scale.dtype != torch.float32 or a_scale.numel() != m):
        raise RuntimeError(f"{name}: a_scale must be fp32 with one element per token ({m})")
    if residual.dtype not in (torch.float32, torch.bfloat16) or residual.shape != (m, n) or residual.stride(-1) != 1:
        raise RuntimeError(f"{name}: residual must be float32/bfloat16 [{m}, {n}] with contiguous rows")
    if out is None:
        out = torch.empty((m, n), dtype=residual.dtype, device=dev)
    elif out.dtype != residual.dtype or out.shape != (m, n) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must match the residual's dtype and shape")
    ws_dev, ws = _scale_args(name, scale, dev)
    lda = a2.stride(0) if m > 1 else k
    ldr = residual.stride(0) if m > 1 else n
    ldo = out.stride(0) if m > 1 else n
    with torch.cuda.device(dev):
        _lib.call("wfb_linear_i2s_residual", _p(packed_weights), n, k, _p(a2), m, lda, _p(a_scale), ws_dev, ws,
                  _p(residual), _DT[residual.dtype], ldr, _p(out), _DT[out.dtype], ldo, _stream(dev))
    return out


def rmsnorm_linear_supported(m: int, h: int, k: int, gamma_bytes: int = 2) -> bool:
    """Whether rmsnorm_linear takes these sizes: one row of up to 16384 elements (the decode GEMV's
    prologue), or decode batches of 2 .. 16 rows of up to 4096 elements (the LDS-staged kernel's prologue;
    the gated rmsnorm_linear_glu takes only this form, also for one row).  ``gamma_bytes`` is kept for
    callers and no longer limits the size."""
    if h % 8 != 0 or not 0 < h <= k or k % QK_I2_S != 0:
        return False
    return (1 <= m <= 16 and k <= 4096) or (m == 1 and k <= 16384)


def rmsnorm_linear_glu_supported(m: int, h: int, k: int) -> bool:
    """Whether rmsnorm_linear_glu takes these sizes (decode batches of up to 16 rows of up to 4096 elements)."""
    return 1 <= m <= 16 and h % 8 == 0 and 0 < h <= k <= 4096 and k % QK_I2_S == 0


def rmsnorm_linear_preferred(m: int, h: int, n: int, k: int, gamma_bytes: int = 2) -> bool:
    """Whether the fused launch is the faster choice: every supported size (measured on MI355X, the prologue
    costs less than the separate quantiser launch it replaces at the Llama-3-8B, BitNet-2B and SmolLM2
    decode shapes)."""
    return rmsnorm_linear_supported(m, h, k, gamma_bytes)


def rmsnorm_linear(
    x: torch.Tensor, weight: Optional[torch.Tensor], packed_weights: torch.Tensor, scales: torch.Tensor,
    seg_rows=None, eps: float = 1e-6, residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """RMSNorm/SubLN + per-token int8 quantisation + (multi-segment) BitLinear (+ residual) in one launch
    for decode batches (``rmsnorm_linear_supported``): equal, bit for bit, to ``rmsnorm_quantize_i8``
    followed by ``bitnet_linear_segmented`` (``bitnet_linear_residual`` when ``residual`` is given, the
    output then taking the residual's dtype; ``out`` may be ``residual`` itself).

    x: float32/bfloat16 [M, H]; weight: [H] or None; packed_weights: uint8 [N, K/4] with K >= H (codes
    past H are zero); scales: fp32 [n_seg] on the device; seg_rows: row counts (None = one segment).
    """
    name = "rmsnorm_linear"
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: x must be float32/bfloat16 [batch, hidden]")
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [out_features, in_features/4]")
    m, h = x.shape
    n, kb = packed_weights.shape
    k = kb * 4
    rows = [n] if seg_rows is None else [int(r) for r in seg_rows]
    if sum(rows) != n:
        raise ValueError(f"{name}: segment rows sum to {sum(rows)}, packed_weights has {n}")
    if scales.dtype != torch.float32 or scales.numel() != len(rows):
        raise RuntimeError(f"{name}: scales must be fp32 with one element per segment")
    gbytes = 0 if weight is None else weight.element_size()
    if not rmsnorm_linear_supported(m, h, k, gbytes):
        raise RuntimeError(f"{name}: M={m}, H={h}, K={k} outside the fused path (H % 8 == 0, H <= K and either "
                           f"M == 1 with K <= 16384, or M <= 16 with K <= 4096)")
    dev = _require_gpu(name, x, weight, packed_weights, scales, residual)
    if weight is not None and (weight.numel() != h or weight.dtype not in (torch.float32, torch.bfloat16)):
        raise RuntimeError(f"{name}: weight must be float32/bfloat16 with {h} elements")
    if x.stride(1) != 1 or (x.stride(0) * x.element_size()) % 16 != 0 or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    if weight is not None:
        weight = weight.contiguous()
    if residual is not None:
        if residual.dtype not in (torch.float32, torch.bfloat16) or residual.shape != (m, n) or residual.stride(-1) != 1:
            raise RuntimeError(f"{name}: residual must be float32/bfloat16 [{m}, {n}] with contiguous rows")
        out_dtype = residual.dtype
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=dev)
    elif out.dtype != out_dtype or out.shape != (m, n) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must be {out_dtype} [{m}, {n}] with contiguous rows")
    seg = (ctypes.c_int64 * len(rows))(*rows)
    with torch.cuda.device(dev):
        _lib.call("wfb_rmsnorm_linear_i2s", _p(x), _DT[x.dtype], x.stride(0), _p(weight),
                  _DT[weight.dtype] if weight is not None else WFB_F32, float(eps), m, h, _p(packed_weights), n, k,
                  len(rows), ctypes.cast(seg, ctypes.c_void_p), _p(scales), _p(residual),
                  _DT[residual.dtype] if residual is not None else WFB_F32,
                  residual.stride(0) if residual is not None else n, _p(out), _DT[out.dtype], out.stride(0),
                  _stream(dev))
    return out


def rmsnorm_linear_glu(
    x: torch.Tensor, weight: Optional[torch.Tensor], packed_weights: torch.Tensor, scales: torch.Tensor,
    act: str = "silu", eps: float = 1e-6, mid_dtype: torch.dtype = torch.bfloat16, out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """RMSNorm + per-token int8 quantisation + gate|up BitLinear + act(gate) * up in one launch (decode
    batches, ``rmsnorm_linear_glu_supported``): fp32 [M, half], equal, bit for bit, to ``rmsnorm_quantize_i8``
    followed by ``bitnet_linear_glu``.

    x: float32/bfloat16 [M, H]; weight: [H] or None; packed_weights: uint8 gate|up [2 * half, K/4] (half %
    32 == 0, K >= H); scales: fp32 [2] on the device."""
    name = "rmsnorm_linear_glu"
    if act not in _ACTS:
        raise ValueError(f"{name}: act must be one of {sorted(_ACTS)}")
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: x must be float32/bfloat16 [batch, hidden]")
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [2 * half, in_features/4]")
    if mid_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: mid_dtype must be float32 or bfloat16")
    m, h = x.shape
    n, kb = packed_weights.shape
    k = kb * 4
    if n % 64 != 0:
        raise ValueError(f"{name}: gate|up rows ({n}) must be 2 x a multiple of 32")
    if scales.dtype != torch.float32 or scales.numel() != 2:
        raise RuntimeError(f"{name}: scales must be fp32 [2] (gate, up)")
    if not rmsnorm_linear_glu_supported(m, h, k):
        raise RuntimeError(f"{name}: M={m}, H={h}, K={k} outside the fused path (M <= 16, H % 8 == 0, H <= K <= 4096)")
    dev = _require_gpu(name, x, weight, packed_weights, scales)
    if weight is not None and (weight.numel() != h or weight.dtype not in (torch.float32, torch.bfloat16)):
        raise RuntimeError(f"{name}: weight must be float32/bfloat16 with {h} elements")
    if x.stride(1) != 1 or (x.stride(0) * x.element_size()) % 16 != 0 or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    if weight is not None:
        weight = weight.contiguous()
    half = n // 2
    if out is None:
        out = torch.empty((m, half), dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or out.shape != (m, half) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must be float32 [{m}, {half}] with contiguous rows")
    with torch.cuda.device(dev):
        _lib.call("wfb_rmsnorm_linear_i2s_glu", _p(x), _DT[x.dtype], x.stride(0), _p(weight),
                  _DT[weight.dtype] if weight is not None else WFB_F32, float(eps), m, h, _p(packed_weights), n, k,
                  _p(scales), _ACTS[act], _DT[mid_dtype], _p(out), out.stride(0), _stream(dev))
    return out


def bitnet_linear_glu(
    packed_weights: torch.Tensor, scales: torch.Tensor, activations: torch.Tensor, act: str = "silu",
    a_scale: Optional[torch.Tensor] = None, mid_dtype: torch.dtype = torch.bfloat16,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """act(gate) * up from the gate|up projection in one launch (decode batches, M <= 64): fp32 [M, half].

    ``packed_weights`` is gate|up (2 * half rows, half % 32 == 0), ``scales`` fp32 [2] on the device.
    Equal, bit for bit, to ``bitnet_linear_segmented`` with ``out_dtype=mid_dtype`` followed by the gated
    product of ``glu_rmsnorm_quantize_i8`` (so ``rmsnorm_quantize_i8`` of the result equals
    ``glu_rmsnorm_quantize_i8`` of the stored gate and up)."""
    name = "bitnet_linear_glu"
    if act not in _ACTS:
        raise ValueError(f"{name}: act must be one of {sorted(_ACTS)}")
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [2 * half, in_features/4]")
    n, kb = packed_weights.shape
    k = kb * 4
    if n % 64 != 0:
        raise ValueError(f"{name}: gate|up rows ({n}) must be 2 x a multiple of 32")
    if activations.dtype != torch.int8 or activations.dim() != 2 or activations.shape[1] != k:
        raise RuntimeError(f"{name}: activations must be int8 [batch, {k}]")
    m = activations.shape[0]
    if m > 64:
        raise RuntimeError(f"{name}: at most 64 tokens (got {m})")
    if scales.dtype != torch.float32 or scales.numel() != 2:
        raise RuntimeError(f"{name}: scales must be fp32 [2] (gate, up)")
    if mid_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: mid_dtype must be float32 or bfloat16")
    dev = _require_gpu(name, packed_weights, scales, activations, a_scale)
    a2 = activations
    if a2.stride(1) != 1 or (m > 1 and a2.stride(0) % 16 != 0) or a2.data_ptr() % 16 != 0:
        a2 = a2.contiguous()
    if a_scale is not None and (a_scale.dtype != torch.float32 or a_scale.numel() != m):
        raise RuntimeError(f"{name}: a_scale must be fp32 with one element per token ({m})")
    half = n // 2
    if out is None:
        out = torch.empty((m, half), dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or out.shape != (m, half) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must be float32 [{m}, {half}] with contiguous rows")
    lda = a2.stride(0) if m > 1 else k
    with torch.cuda.device(dev):
        _lib.call("wfb_linear_i2s_glu", _p(packed_weights), n, k, _p(a2), m, lda, _p(a_scale), _p(scales),
                  _ACTS[act], _DT[mid_dtype], _p(out), out.stride(0) if m > 1 else half, _stream(dev))
    return out


# ---- greedy decoding: LM head + argmax ----------------------------------------------------------


def _argmax_ws(name: str, workspace: Optional[torch.Tensor], m: int, n: int, dev: torch.device) -> torch.Tensor:
    need = (n + 15) // 16 * m
    if workspace is None:
        return torch.empty(need, dtype=torch.int64, device=dev)
    if workspace.dtype not in (torch.int64, torch.uint64) or workspace.numel() < need or workspace.device != dev \
            or not workspace.is_contiguous():
        raise RuntimeError(f"{name}: workspace must be {need} contiguous 64-bit elements on {dev}")
    return workspace


def bitnet_linear_argmax(
    packed_weights: torch.Tensor, activations: torch.Tensor, scale: Scale, a_scale: Optional[torch.Tensor] = None,
    logits_dtype: torch.dtype = torch.float32, return_logits: bool = False,
    workspace: Optional[torch.Tensor] = None,
):
    """Greedy next tokens of a ternary LM head: int64 [M] = first argmax over n of the BitLinear logits
    acc * scale * a_scale[m] rounded to ``logits_dtype`` (M <= 64).  With ``return_logits`` also the
    logits [M, N].  ``workspace``: optional 64-bit device buffer of ceil(N/16) * M elements."""
    name = "bitnet_linear_argmax"
    if packed_weights.dtype != torch.uint8 or packed_weights.dim() != 2:
        raise RuntimeError(f"{name}: packed_weights must be uint8 2D [out_features, in_features/4]")
    if activations.dtype != torch.int8 or activations.dim() != 2:
        raise RuntimeError(f"{name}: activations must be int8 [batch, in_features]")
    n, kb = packed_weights.shape
    k = kb * 4
    if k % QK_I2_S != 0 or activations.shape[1] != k:
        raise ValueError(f"{name}: in_features must be a multiple of {QK_I2_S} and match the weights")
    m = activations.shape[0]
    dev = _require_gpu(name, packed_weights, a_scale)
    a2 = activations
    if a2.device != dev:
        raise RuntimeError(f"{name}: activations are on {a2.device}, weights on {dev}")
    if a2.stride(1) != 1 or (m > 1 and a2.stride(0) % 16 != 0) or a2.data_ptr() % 16 != 0:
        a2 = a2.contiguous()
    if a_scale is not None and (a_scale.dtype != torch.float32 or a_scale.numel() != m):
        raise RuntimeError(f"{name}: a_scale must be fp32 with one element per token ({m})")
    if logits_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: logits_dtype must be float32 or bfloat16")
    ws_dev, ws = _scale_args(name, scale, dev)
    logits = torch.empty((m, n), dtype=logits_dtype, device=dev) if return_logits else None
    tokens = torch.empty(m, dtype=torch.int64, device=dev)
    wsp = _argmax_ws(name, workspace, m, n, dev)
    lda = a2.stride(0) if m > 1 else k
    with torch.cuda.device(dev):
        _lib.call("wfb_linear_i2s_argmax", _p(packed_weights), n, k, _p(a2), m, lda, _p(a_scale), ws_dev, ws,
                  _p(logits), _DT[logits_dtype], n, _p(wsp), _p(tokens), _stream(dev))
    return (tokens, logits) if return_logits else tokens


def lm_head_argmax(
    x: torch.Tensor, weight: torch.Tensor, norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-5,
    return_logits: bool = False, workspace: Optional[torch.Tensor] = None,
):
    """Greedy next tokens int64 [M] of a dense LM head with the final RMSNorm fused:
    y = x * rsqrt(mean(x^2) + eps) * norm_weight (rounded to x.dtype), logits = y @ weight.T (fp32),
    token = first argmax.  x [M, H] (M <= 16) float32/bfloat16, weight [vocab, H] float32/bfloat16 (e.g. a
    tied embedding).  With ``return_logits`` also the fp32 logits [M, vocab]."""
    name = "lm_head_argmax"
    dev = _require_gpu(name, weight, norm_weight)
    if x.device != dev or x.dim() != 2 or x.stride(-1) != 1:
        raise RuntimeError(f"{name}: x must be [M, H] with contiguous rows on {dev}")
    if x.dtype not in (torch.float32, torch.bfloat16) or weight.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: x and weight must be float32 or bfloat16")
    m, h = x.shape
    if weight.dim() != 2 or weight.shape[1] != h:
        raise RuntimeError(f"{name}: weight must be [vocab, {h}]")
    n = weight.shape[0]
    if norm_weight is not None and norm_weight.numel() != h:
        raise RuntimeError(f"{name}: norm_weight must have {h} elements")
    gdt = _float_dtype(name, norm_weight) if norm_weight is not None else WFB_F32
    logits = torch.empty((m, n), dtype=torch.float32, device=dev) if return_logits else None
    tokens = torch.empty(m, dtype=torch.int64, device=dev)
    wsp = _argmax_ws(name, workspace, m, n, dev)
    ldx = x.stride(0) if m > 1 else h
    with torch.cuda.device(dev):
        _lib.call("wfb_lm_head_argmax", _p(x), _DT[x.dtype], ldx, _p(norm_weight), gdt, float(eps), _p(weight),
                  _DT[weight.dtype], h, m, n, h, _p(logits), n, _p(wsp), _p(tokens), _stream(dev))
    return (tokens, logits) if return_logits else tokens


# ---- GQA decode attention over a KV cache -------------------------------------------------------


def _rows2d(name: str, t: torch.Tensor, b: int, width: int) -> Tuple[torch.Tensor, int]:
    """View t as [b, width] rows with unit inner stride; returns (view, row stride)."""
    t2 = t.reshape(b, width) if t.dim() != 2 or t.shape != (b, width) else t
    if t2.stride(-1) != 1:
        raise RuntimeError(f"{name}: rows must be contiguous")
    return t2, (t2.stride(0) if b > 1 else width)


def rope_tables(theta: float, head_dim: int, max_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin fp32 CPU tensors [max_len, head_dim/2] of the HF rotate-half rotary embedding at positions
    0..max_len-1 (angle p * theta^(-2i/head_dim) in double precision, rounded once to float): the tables
    the decode / prefill attention kernels take, the same values the native engine computes."""
    name = "rope_tables"
    if head_dim < 2 or head_dim % 2 != 0 or max_len < 1 or not theta > 0:
        raise ValueError(f"{name}: bad theta / head_dim / max_len")
    cos = torch.empty((max_len, head_dim // 2), dtype=torch.float32)
    sin = torch.empty_like(cos)
    _lib.call("wfb_rope_tables", float(theta), head_dim, max_len, _p(cos), _p(sin))
    return cos, sin


def gqa_decode_attention(
    q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    pos: torch.Tensor, rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None,
    scale: Optional[float] = None, out: Optional[torch.Tensor] = None, split: bool = True,
) -> torch.Tensor:
    """One decode token per sequence: rotary embedding of q / k_new, append k/v at pos[b] to the caches,
    attention over positions 0..pos[b].  Returns out [batch, num_heads * head_dim].

    q [batch, num_heads*head_dim] (or [batch, 1, num_heads, head_dim]); k_new / v_new
    [batch, num_kv_heads*head_dim]; caches [batch, num_kv_heads, max_len, head_dim] (contiguous, same
    dtype as q: float32 or bfloat16); pos int64 [batch] on the device; rope tables fp32
    [max_len, head_dim/2] (cos and sin of pos * inv_freq) or None.  2-D inputs may be column slices of
    one q|k|v projection output (row strides are passed through).  ``split``: cut long caches into
    key splits on separate workgroups (a workspace is allocated), else one workgroup per (kv head,
    sequence).  Counterpart of the C engine's attention_forward
    (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:381-441).
    """
    name = "gqa_decode_attention"
    _require_gpu(name, k_cache, v_cache, pos, rope_cos, rope_sin)
    dev = k_cache.device
    for t in (q, k_new, v_new) + ((out,) if out is not None else ()):
        if t.device != dev:
            raise RuntimeError(f"{name}: tensors must be on {dev}")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise RuntimeError(f"{name}: caches must be [batch, kv_heads, max_len, head_dim] of one shape")
    b, hkv, max_len, d = k_cache.shape
    if q.dtype != k_cache.dtype or k_new.dtype != q.dtype or v_new.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise RuntimeError(f"{name}: q, k_new, v_new and the caches must share one dtype")
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: dtype must be float32 or bfloat16, got {q.dtype}")
    if pos.dtype != torch.int64 or pos.numel() != b:
        raise RuntimeError(f"{name}: pos must be int64 [{b}]")
    if q.numel() % (b * d) != 0:
        raise RuntimeError(f"{name}: q has {q.numel()} elements, not a multiple of batch*head_dim")
    hq = q.numel() // (b * d)
    q2, ldq = _rows2d(name, q, b, hq * d)
    k2, ldk = _rows2d(name, k_new, b, hkv * d)
    v2, ldv = _rows2d(name, v_new, b, hkv * d)
    if (rope_cos is None) != (rope_sin is None):
        raise RuntimeError(f"{name}: give both rope tables or neither")
    if rope_cos is not None:
        for t in (rope_cos, rope_sin):
            if t.dtype != torch.float32 or t.shape != (max_len, d // 2):
                raise RuntimeError(f"{name}: rope tables must be fp32 [{max_len}, {d // 2}]")
    if out is None:
        out = torch.empty((b, hq * d), dtype=q.dtype, device=dev)
    elif out.dtype != q.dtype or out.shape != (b, hq * d) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must be [{b}, {hq * d}] {q.dtype} with contiguous rows")
    ldo = out.stride(0) if b > 1 else hq * d
    sc = 1.0 / float(d) ** 0.5 if scale is None else float(scale)
    work = torch.empty(b * hq * (d + 2) * ((max_len + 63) // 64), dtype=torch.float32, device=dev) if split else None
    with torch.cuda.device(dev):
        _lib.call(
            "wfb_gqa_decode_attention", _p(q2), ldq, _p(k2), ldk, _p(v2), ldv, _DT[q.dtype], _p(rope_cos),
            _p(rope_sin), _p(k_cache), _p(v_cache), max_len, _p(pos), b, hq, hkv, d, sc, _p(out), ldo, _p(work),
            _stream(dev),
        )
    return out


def gqa_prefill_attention(
    q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    start: int, t: int, rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None,
    scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """A prefill chunk of t tokens per sequence at positions start..start+t-1: rotary embedding of q / k_new,
    append k/v to the caches, causal GQA attention (token i over positions 0..start+i).  Returns out
    [batch*t, num_heads*head_dim] (row b*t + i).

    q [batch*t, num_heads*head_dim] (or any shape with those elements, token-major); k_new / v_new
    [batch*t, num_kv_heads*head_dim]; the three may be column slices of one q|k|v output.  bfloat16 only;
    caches [batch, num_kv_heads, max_len, head_dim] (contiguous); rope tables fp32 [max_len, head_dim/2]
    or None.  The same contract as ``gqa_decode_attention`` for each token of the chunk.
    """
    name = "gqa_prefill_attention"
    _require_gpu(name, k_cache, v_cache, rope_cos, rope_sin)
    dev = k_cache.device
    for x in (q, k_new, v_new) + ((out,) if out is not None else ()):
        if x.device != dev:
            raise RuntimeError(f"{name}: tensors must be on {dev}")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise RuntimeError(f"{name}: caches must be [batch, kv_heads, max_len, head_dim] of one shape")
    b, hkv, max_len, d = k_cache.shape
    for x in (q, k_new, v_new, k_cache, v_cache):
        if x.dtype != torch.bfloat16:
            raise RuntimeError(f"{name}: q, k_new, v_new and the caches must be bfloat16, got {x.dtype}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError(f"{name}: caches must be contiguous")
    rows = b * t
    if rows == 0:
        return torch.empty((0, q.numel() // max(1, d)), dtype=q.dtype, device=dev) if out is None else out
    if q.numel() % (rows * d) != 0:
        raise RuntimeError(f"{name}: q has {q.numel()} elements, not a multiple of batch*t*head_dim")
    hq = q.numel() // (rows * d)
    q2, ldq = _rows2d(name, q, rows, hq * d)
    k2, ldk = _rows2d(name, k_new, rows, hkv * d)
    v2, ldv = _rows2d(name, v_new, rows, hkv * d)
    if (rope_cos is None) != (rope_sin is None):
        raise RuntimeError(f"{name}: give both rope tables or neither")
    if rope_cos is not None:
        for x in (rope_cos, rope_sin):
            if x.dtype != torch.float32 or x.shape != (max_len, d // 2) or not x.is_contiguous():
                raise RuntimeError(f"{name}: rope tables must be contiguous fp32 [{max_len}, {d // 2}]")
    if out is None:
        out = torch.empty((rows, hq * d), dtype=q.dtype, device=dev)
    elif out.dtype != q.dtype or out.shape != (rows, hq * d) or out.stride(-1) != 1:
        raise RuntimeError(f"{name}: out must be [{rows}, {hq * d}] {q.dtype} with contiguous rows")
    ldo = out.stride(0) if rows > 1 else hq * d
    sc = 1.0 / float(d) ** 0.5 if scale is None else float(scale)
    with torch.cuda.device(dev):
        _lib.call(
            "wfb_gqa_prefill_attention", _p(q2), ldq, _p(k2), ldk, _p(v2), ldv, _DT[q.dtype], _p(rope_cos),
            _p(rope_sin), _p(k_cache), _p(v_cache), max_len, int(start), b, int(t), hq, hkv, d, sc, _p(out), ldo,
            _stream(dev),
        )
    return out


def bitnet_gemv(packed_weights: torch.Tensor, activations: torch.Tensor, scale: Scale) -> torch.Tensor:
    """fp32 [out] = acc * scale for one int8 token [in] (reference: bitnet.py:73-111)."""
    if activations.dim() != 1:
        raise RuntimeError("bitnet_gemv: activations must be 1D [in_features]")
    if packed_weights.shape[1] * 4 % QK_I2_S != 0:
        raise ValueError(f"bitnet_gemv: in_features ({packed_weights.shape[1] * 4}) must be multiple of {QK_I2_S}")
    if activations.shape[0] != packed_weights.shape[1] * 4:
        raise ValueError(
            f"bitnet_gemv: activations.shape[0] ({activations.shape[0]}) != in_features ({packed_weights.shape[1] * 4})"
        )
    return bitnet_linear(packed_weights, activations, scale, out_dtype=torch.float32)


def bitnet_gemm(packed_weights: torch.Tensor, activations: torch.Tensor, scale: Scale) -> torch.Tensor:
    """fp32 [batch, out] = acc * scale for int8 tokens [batch, in] (reference: bitnet.py:114-152)."""
    if activations.dim() != 2:
        raise RuntimeError("bitnet_gemm: activations must be 2D [batch, in_features]")
    if packed_weights.shape[1] * 4 % QK_I2_S != 0:
        raise ValueError(f"bitnet_gemm: in_features ({packed_weights.shape[1] * 4}) must be multiple of {QK_I2_S}")
    return bitnet_linear(packed_weights, activations, scale, out_dtype=torch.float32)


def _fused_input(name: str, x: torch.Tensor, packed: torch.Tensor) -> torch.Tensor:
    """One token: a 1-D or [1, hidden] float input as a contiguous [1, hidden] row matching the weights."""
    if not (x.dim() == 1 or (x.dim() == 2 and x.shape[0] == 1)):
        raise RuntimeError(f"{name}: Input must be 1D or [1, hidden_size]")
    h = x.numel()
    if h % QK_I2_S != 0 or packed.dim() != 2 or packed.shape[1] * 4 != h:
        raise ValueError(f"{name}: hidden size ({h}) must be a multiple of {QK_I2_S} and match the weights")
    x = x.reshape(1, h)
    return x if x.dtype in (torch.float32, torch.bfloat16, torch.float16) else x.float()


# Row concatenations of the packed weights the fused ops launch over, with their scales on the device: built
# once per set of weight tensors and reused while those tensors are alive and unmodified (identity, storage
# and version counter all match); room for the q|k|v and gate|up sets of a 128-layer model.  A single weight
# is used as it is (only its scale is cached).  A model that keeps its projections concatenated (model.py)
# never needs it.
_CONCAT_CACHE: "collections.OrderedDict" = collections.OrderedDict()
_CONCAT_CACHE_MAX = 256
_SCALE_CACHE: "collections.OrderedDict" = collections.OrderedDict()


def _scale_tensor(scales: Sequence[float], device: torch.device) -> torch.Tensor:
    key = (tuple(float(x) for x in scales), str(device))
    sc = _SCALE_CACHE.get(key)
    if sc is None:
        sc = torch.tensor(list(key[0]), dtype=torch.float32, device=device)
        _SCALE_CACHE[key] = sc
        while len(_SCALE_CACHE) > _CONCAT_CACHE_MAX:
            _SCALE_CACHE.popitem(last=False)
    else:
        _SCALE_CACHE.move_to_end(key)
    return sc


def _concat_weights(ws: Sequence[torch.Tensor], scales: Sequence[float]) -> Tuple[torch.Tensor, torch.Tensor]:
    if len(ws) == 1:
        return ws[0].contiguous(), _scale_tensor(scales, ws[0].device)
    key = tuple((id(w), w.data_ptr(), w._version, tuple(w.shape)) for w in ws) + (tuple(float(x) for x in scales),)
    hit = _CONCAT_CACHE.get(key)
    if hit is not None and all(r() is w for r, w in zip(hit[0], ws)):
        _CONCAT_CACHE.move_to_end(key)
        return hit[1], hit[2]
    cat = torch.cat([w.contiguous() for w in ws], dim=0)
    sc = torch.tensor([float(x) for x in scales], dtype=torch.float32, device=ws[0].device)
    _CONCAT_CACHE[key] = ([weakref.ref(w) for w in ws], cat, sc)
    while len(_CONCAT_CACHE) > _CONCAT_CACHE_MAX:
        _CONCAT_CACHE.popitem(last=False)
    return cat, sc


def bitnet_qkv_forward(input: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, v_weight: torch.Tensor,
                       q_scale: float, k_scale: float, v_scale: float
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused QKV of one token: the input quantised once (per-token absmax int8), then q / k / v = acc * a_scale *
    w_scale, fp32 1-D outputs.  The op of SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:289-375 (schema
    torch_extension_cpu.cpp:924-926) without its double sum(a) subtraction (anomaly ii): q = acc(q_weight) *
    a_scale * q_scale exactly as bitnet_linear gives it.  Two launches: the quantiser and one segmented linear
    over q|k|v (rows concatenated once per weight set); separate linears where a projection's rows are not a
    multiple of 8."""
    name = "bitnet_qkv_forward"
    x = _fused_input(name, input, q_weight)
    ws = (q_weight, k_weight, v_weight)
    q8, a_s = quantize_activations_i8_per_token(x)
    if all(w.dtype == torch.uint8 and w.dim() == 2 and w.shape[1] == q_weight.shape[1] and w.shape[0] % 8 == 0
           for w in ws) and q_weight.is_cuda:
        cat, sc = _concat_weights(ws, (q_scale, k_scale, v_scale))
        rows = [w.shape[0] for w in ws]
        y = bitnet_linear_segmented(cat, rows, sc, q8, a_scale=a_s, out_dtype=torch.float32).reshape(-1)
        return tuple(torch.split(y, rows))
    return tuple(bitnet_linear(w, q8, float(sc), a_scale=a_s, out_dtype=torch.float32).reshape(-1)
                 for w, sc in ((q_weight, q_scale), (k_weight, k_scale), (v_weight, v_scale)))


def bitnet_mlp_forward(input: torch.Tensor, gate_weight: torch.Tensor, up_weight: torch.Tensor,
                       down_weight: torch.Tensor, gate_scale: float, up_scale: float, down_scale: float,
                       ffn_sub_norm: torch.Tensor, eps: float) -> torch.Tensor:
    """Fused BitNet MLP of one token: quantise the input once, gate / up = acc * a_scale * w_scale (fp32),
    relu(gate)^2 * up, SubLN (ffn_sub_norm, eps), re-quantise, down = acc * h_scale * down_scale; fp32 [hidden].
    The op of SGB/sgl-kernel/csrc/cpu/bitnet_fused_layer.cpp:150-287 (schema torch_extension_cpu.cpp:921-923)
    with every projection scaled by its weight scale and sum(a) removed once (anomaly ii not copied).
    Three launches: the quantiser, gate|up with relu(gate)^2 * up in its epilogue (rows concatenated once per
    weight set), SubLN + quantisation in the down projection's prologue -- bit-identical to the five separate
    calls, which are kept for sizes those kernels do not take."""
    name = "bitnet_mlp_forward"
    x = _fused_input(name, input, gate_weight)
    f = gate_weight.shape[0]
    if up_weight.shape != gate_weight.shape or down_weight.dim() != 2 or down_weight.shape[1] * 4 != f:
        raise ValueError(f"{name}: gate/up must be [intermediate, hidden/4] and down [hidden, intermediate/4]")
    if ffn_sub_norm.numel() != f:
        raise ValueError(f"{name}: ffn_sub_norm must have {f} elements")
    q8, a_s = quantize_activations_i8_per_token(x)
    norm_w = ffn_sub_norm.to(torch.float32).contiguous()
    fused = (gate_weight.dtype == torch.uint8 and up_weight.dtype == torch.uint8 and gate_weight.is_cuda
             and f % 32 == 0 and rmsnorm_linear_supported(1, f, f))
    if fused:
        cat, sc = _concat_weights((gate_weight, up_weight), (gate_scale, up_scale))
        hid = bitnet_linear_glu(cat, sc, q8, "relu2", a_scale=a_s, mid_dtype=torch.float32)
        dw, dsc = _concat_weights((down_weight,), (down_scale,))
        return rmsnorm_linear(hid, norm_w, dw, dsc, eps=float(eps), out_dtype=torch.float32).reshape(-1)
    gate = bitnet_linear(gate_weight, q8, float(gate_scale), a_scale=a_s, out_dtype=torch.float32)
    up = bitnet_linear(up_weight, q8, float(up_scale), a_scale=a_s, out_dtype=torch.float32)
    h8, h_s = glu_rmsnorm_quantize_i8(gate, up, "relu2", norm_w, eps=float(eps))
    return bitnet_linear(down_weight, h8, float(down_scale), a_scale=h_s, out_dtype=torch.float32).reshape(-1)


# ---- torch.ops.wfbitnet registrations (reference schemas, torch_extension_cpu.cpp:913-926) ------

_LIB_DEF = torch.library.Library("wfbitnet", "DEF")
_LIB_DEF.define("bitnet_gemv(Tensor packed_weights, Tensor activations, float scale) -> Tensor")
_LIB_DEF.define("bitnet_gemm(Tensor packed_weights, Tensor activations, float scale) -> Tensor")
_LIB_DEF.define("bitnet_quantize_activations(Tensor input) -> (Tensor, Tensor)")
_LIB_DEF.define("bitnet_mlp_forward(Tensor input, Tensor gate_weight, Tensor up_weight, Tensor down_weight, "
                "float gate_scale, float up_scale, float down_scale, Tensor ffn_sub_norm, float eps) -> Tensor")
_LIB_DEF.define("bitnet_qkv_forward(Tensor input, Tensor q_weight, Tensor k_weight, Tensor v_weight, "
                "float q_scale, float k_scale, float v_scale) -> (Tensor, Tensor, Tensor)")
_LIB_DEF.impl("bitnet_gemv", bitnet_gemv, "CUDA")
_LIB_DEF.impl("bitnet_gemm", bitnet_gemm, "CUDA")
_LIB_DEF.impl("bitnet_quantize_activations", quantize_activations_i8, "CUDA")
_LIB_DEF.impl("bitnet_mlp_forward", bitnet_mlp_forward, "CUDA")
_LIB_DEF.impl("bitnet_qkv_forward", bitnet_qkv_forward, "CUDA")


def _gemv_meta(packed_weights, activations, scale):
    return packed_weights.new_empty((packed_weights.shape[0],), dtype=torch.float32)


def _gemm_meta(packed_weights, activations, scale):
    return packed_weights.new_empty((activations.shape[0], packed_weights.shape[0]), dtype=torch.float32)


def _quant_meta(x):
    return x.new_empty(x.shape, dtype=torch.int8), x.new_empty((1,), dtype=torch.float32)


def _mlp_meta(input, gate_weight, up_weight, down_weight, gate_scale, up_scale, down_scale, ffn_sub_norm, eps):
    return input.new_empty((input.numel(),), dtype=torch.float32)


def _qkv_meta(input, q_weight, k_weight, v_weight, q_scale, k_scale, v_scale):
    return tuple(input.new_empty((w.shape[0],), dtype=torch.float32) for w in (q_weight, k_weight, v_weight))


_LIB_DEF.impl("bitnet_mlp_forward", _mlp_meta, "Meta")
_LIB_DEF.impl("bitnet_qkv_forward", _qkv_meta, "Meta")
_LIB_DEF.impl("bitnet_gemv", _gemv_meta, "Meta")
_LIB_DEF.impl("bitnet_gemm", _gemm_meta, "Meta")
_LIB_DEF.impl("bitnet_quantize_activations", _quant_meta, "Meta")
