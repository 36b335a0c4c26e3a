"""Drop-in BitLinear modules whose forward runs the MI355X kernels.

Surfaces kept from the reference:
  * ``BitLinear(in_features, out_features, bias=False, eps=1e-5)`` with ``forward(x[..., in]) -> [..., out]``
    (packages/training/src/wrinklefree/models/bitlinear.py:36-113);
  * ``convert_linear_to_bitlinear(module, exclude_names)`` (same file :154-192);
  * ``BitNetLinearMethod.create_weights / apply`` with ``qweight`` uint8 [out, in/4] + ``scale`` fp32[1]
    (packages/inference/extern/sglang-bitnet/python/sglang/srt/layers/quantization/bitnet.py:137-255);
  * ``patch_model_with_native_kernels`` (packages/inference/src/wrinklefree_inference/kernels/bitnet_patch.py:165-210).

The forward is the quantised serving forward of the reference CPU path (per-token absmax int8
activations, I2_S ternary weights with a per-tensor absmean scale, exact int32 accumulation, then
acc * w_scale * a_scale).  Under autograd (grad mode on and the weight or the input requiring grad)
``BitLinear`` is the reference training module's straight-through estimator at lambda = 1
(packages/training/src/wrinklefree/models/bitlinear.py:86-113: F.linear(x + (q(x) - x).detach(),
w + (q(w) - w).detach())): the same forward value, computed by the kernels, and the gradients of
F.linear at the quantised operands -- grad_x = grad_y @ q(w), grad_w = grad_y^T @ q(x).  A lambda
warmup blend (lambda < 1) is a float product the ternary kernels do not compute; with a lambda source
registered (:func:`set_lambda_source`) such a step raises.  The packed weight follows the float
weight: any in-place change (optimizer step, ``copy_``, ``load_state_dict``) repacks on the next
forward.  No CPU or eager-torch fallback for the forward.
"""

from __future__ import annotations

from typing import Callable, Iterable, List, Optional

import torch
import torch.nn as nn

from .ops import (
    QK_I2_S,
    bitnet_linear,
    pack_ternary_i2s,
    quantize_activations_i8,
    quantize_activations_i8_per_token,
    rmsnorm_quantize_i8,
    unpack_i2s,
)

_lambda_source: Optional[Callable[[], float]] = None


def set_lambda_source(fn: Optional[Callable[[], float]]) -> None:
    """Register the training loop's lambda-warmup value (the reference reads
    ``wrinklefree.quantization.lambda_warmup.get_current_lambda``, lambda_warmup.py:131-135).  BitLinear
    computes the fully quantised product only, so a forward while the source returns lambda != 1 raises
    instead of silently training a different function."""
    global _lambda_source
    _lambda_source = fn


def _check_lambda(name: str) -> None:
    if _lambda_source is not None:
        lam = float(_lambda_source())
        if lam != 1.0:
            raise RuntimeError(f"{name}: lambda warmup at {lam} (< 1) blends float and quantised operands; the "
                               "ternary kernels compute lambda = 1 only")


def _pad_k(k: int) -> int:
    return (k + QK_I2_S - 1) // QK_I2_S * QK_I2_S


def _out_dtype(x: torch.Tensor) -> torch.dtype:
    return torch.float32 if x.dtype == torch.float32 else torch.bfloat16


class _BitLinearSTE(torch.autograd.Function):
    """Straight-through estimator of the reference training forward at lambda = 1
    (WF/models/bitlinear.py:86-113).  Forward: the kernels' quantised product (per-token int8 codes of x,
    the ternary pack of w, exact accumulators, rescale).  Backward: the gradients of F.linear at the
    dequantised operands, identity through both quantisers -- grad_x = g @ (codes_w * s_w),
    grad_w = g^T @ (codes_x * s_x), grad_b = sum g -- in fp32, cast to each input's dtype."""

    @staticmethod
    def forward(ctx, x2, weight, bias, mod):
        q, a_scale = quantize_activations_i8_per_token(x2, k_pad=mod.k_pad)
        y = bitnet_linear(mod.qweight, q, mod.weight_scale, a_scale=a_scale, bias=bias, out_dtype=_out_dtype(x2))
        ctx.save_for_backward(q, a_scale, mod.qweight, mod.weight_scale)
        ctx.meta = (x2.dtype, weight.dtype, None if bias is None else bias.dtype, mod.in_features)
        return y if y.dtype == x2.dtype else y.to(x2.dtype)

    @staticmethod
    def backward(ctx, gy):
        q, a_scale, qweight, wscale = ctx.saved_tensors
        xdt, wdt, bdt, kin = ctx.meta
        g = gy.to(torch.float32).contiguous()
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            w_deq = unpack_i2s(qweight)[:, :kin].to(torch.float32) * wscale  # [N, K]
            gx = (g @ w_deq).to(xdt)
        if ctx.needs_input_grad[1]:
            x_deq = q[:, :kin].to(torch.float32) * a_scale[:, None]  # [M, K]
            gw = (g.t().contiguous() @ x_deq).to(wdt)
        if bdt is not None and ctx.needs_input_grad[2]:
            gb = g.sum(0).to(bdt)
        return gx, gw, gb, None


class _SubLNBitLinearSTE(torch.autograd.Function):
    """SubLN + BitLinear under autograd: the fused kernel's forward value (RMSNorm + per-token int8 codes
    + the ternary product), the straight-through gradient of the linear as in :class:`_BitLinearSTE`,
    and the RMSNorm's own gradient, from the float norm recomputed in fp32 in the backward (the
    formula of WF/models/subln.py:42-59, x * rsqrt(mean(x^2) + eps) * weight)."""

    @staticmethod
    def forward(ctx, x2, gamma, weight, bias, mod, eps):
        lin = mod.linear
        q, a_scale = rmsnorm_quantize_i8(x2, gamma, eps=eps, k_pad=lin.k_pad)
        y = bitnet_linear(lin.qweight, q, lin.weight_scale, a_scale=a_scale, bias=bias, out_dtype=_out_dtype(x2))
        ctx.save_for_backward(x2, gamma, q, a_scale, lin.qweight, lin.weight_scale)
        ctx.meta = (weight.dtype, None if bias is None else bias.dtype, lin.in_features, eps)
        return y if y.dtype == x2.dtype else y.to(x2.dtype)

    @staticmethod
    def backward(ctx, gy):
        x2, gamma, q, a_scale, qweight, wscale = ctx.saved_tensors
        wdt, bdt, kin, eps = ctx.meta
        g = gy.to(torch.float32).contiguous()
        gx = gg = gw = gb = None
        if ctx.needs_input_grad[2]:
            x_deq = q[:, :kin].to(torch.float32) * a_scale[:, None]
            gw = (g.t().contiguous() @ x_deq).to(wdt)
        if bdt is not None and ctx.needs_input_grad[3]:
            gb = g.sum(0).to(bdt)
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            w_deq = unpack_i2s(qweight)[:, :kin].to(torch.float32) * wscale
            g_norm = g @ w_deq  # gradient at the norm's output (identity through the quantiser)
            with torch.enable_grad():
                xr = x2.detach().to(torch.float32).requires_grad_(ctx.needs_input_grad[0])
                gr = gamma.detach().to(torch.float32).requires_grad_(ctx.needs_input_grad[1])
                yn = xr * torch.rsqrt(xr.pow(2).mean(dim=-1, keepdim=True) + eps) * gr
                wrt = [t for t in (xr, gr) if t.requires_grad]
                grads = list(torch.autograd.grad(yn, wrt, g_norm))
            if ctx.needs_input_grad[0]:
                gx = grads.pop(0).to(x2.dtype)
            if ctx.needs_input_grad[1]:
                gg = grads.pop(0).to(gamma.dtype)
        return gx, gg, gw, gb, None, None


class BitLinear(nn.Linear):
    """Ternary-weight, int8-activation linear layer executed by libwfbitnet.

    ``in_features`` need not be a multiple of 128: K is zero-padded to ``k_pad`` inside the packed
    weight and the quantised activations (padded weights are 0, padded activations are 0, so the
    accumulators are those of the unpadded product).  The packed weight is rebuilt whenever ``weight``
    has changed since the last pack (its version counter or storage), so it never goes stale; under
    autograd the forward is the reference's straight-through estimator (:class:`_BitLinearSTE`).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False, eps: float = 1e-5,
                 device=None, dtype=None):
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        self.eps = eps  # kept for signature parity; the int8 quantiser uses the kernel rule max < 1e-6 -> 1
        self.k_pad = _pad_k(in_features)
        # derived from weight and rebuilt when it changes, so not part of the state dict: checkpoints hold
        # weight (and bias) only, like the reference module's (modules from packed weights keep them)
        self.register_buffer("qweight", None, persistent=False)
        self.register_buffer("weight_scale", None, persistent=False)

    @torch.no_grad()
    def pack(self) -> "BitLinear":
        self.qweight, self.weight_scale = pack_ternary_i2s(self.weight.detach().contiguous(), k_pad=self.k_pad)
        self._packed_from = self._weight_stamp()
        return self

    def _weight_stamp(self):
        w = self.weight
        return None if w is None else (w._version, w.data_ptr(), w.device)

    def ensure_packed(self) -> "BitLinear":
        """Pack if there is no packed weight yet or ``weight`` changed since the last pack."""
        if self.weight is not None and (self.qweight is None or getattr(self, "_packed_from", None) != self._weight_stamp()):
            self.pack()
        return self

    @classmethod
    def from_packed(cls, qweight: torch.Tensor, weight_scale: torch.Tensor, in_features: int,
                    bias: Optional[torch.Tensor] = None) -> "BitLinear":
        """Module around an existing I2_S tensor (e.g. loaded from a converted checkpoint)."""
        out_features = qweight.shape[0]
        mod = cls.__new__(cls)
        nn.Module.__init__(mod)
        mod.in_features, mod.out_features = in_features, out_features
        mod.eps = 1e-5
        mod.k_pad = qweight.shape[1] * 4
        if mod.k_pad < in_features or mod.k_pad % QK_I2_S:
            raise ValueError(f"qweight K ({mod.k_pad}) does not cover in_features ({in_features})")
        mod.register_parameter("weight", None)
        mod.register_parameter("bias", None if bias is None else nn.Parameter(bias, requires_grad=False))
        mod.register_buffer("qweight", qweight)
        mod.register_buffer("weight_scale", weight_scale.reshape(1).to(torch.float32))
        return mod

    def forward_quantized(self, q: torch.Tensor, a_scale: torch.Tensor, out_dtype=torch.bfloat16,
                          return_acc: bool = False):
        """Linear on already-quantised activations q [M, k_pad] with per-token scales a_scale [M]
        (inference only: no gradient flows to the weight)."""
        self.ensure_packed()
        return bitnet_linear(self.qweight, q, self.weight_scale, a_scale=a_scale, bias=self.bias,
                             out_dtype=out_dtype, return_acc=return_acc)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _check_lambda("BitLinear")
        self.ensure_packed()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        w, b = self.weight, self.bias
        if torch.is_grad_enabled() and (x2.requires_grad or (w is not None and w.requires_grad)
                                        or (b is not None and b.requires_grad)):
            if w is None:
                raise RuntimeError("BitLinear: a module built from packed weights has no float weight to train")
            return _BitLinearSTE.apply(x2, w, b, self).view(*lead, self.out_features)
        q, a_scale = quantize_activations_i8_per_token(x2, k_pad=self.k_pad)
        y = bitnet_linear(self.qweight, q, self.weight_scale, a_scale=a_scale, bias=self.bias,
                          out_dtype=_out_dtype(x))
        y = y.view(*lead, self.out_features)
        return y if y.dtype == x.dtype else y.to(x.dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, k_pad={self.k_pad}, " \
               f"bias={self.bias is not None}, packed={self.qweight is not None}"


class BitNetLinearNative(nn.Module):
    """The reference's native-kernel linear (WFI/kernels/bitnet_patch.py:28-78), same constructor and
    forward: per-tensor int8 activation quantisation, y = acc * weight_scale * act_scale (+ bias) in
    fp32.  The scales stay on the device (the reference calls ``weight_scale.item()``); M == 1 runs the
    decode GEMV, larger batches the MFMA GEMM, as there.
    """

    def __init__(self, in_features: int, out_features: int, packed_weight: torch.Tensor,
                 weight_scale: torch.Tensor, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        if packed_weight.shape[0] != out_features or packed_weight.shape[1] * 4 != in_features:
            raise ValueError(f"packed_weight {tuple(packed_weight.shape)} does not match "
                             f"[{out_features}, {in_features}/4]")
        self.register_buffer("packed_weight", packed_weight)
        self.register_buffer("weight_scale", weight_scale.reshape(1).to(torch.float32))
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch_shape = x.shape[:-1]
        x_flat = x.reshape(-1, self.in_features).contiguous()
        m = x_flat.shape[0]
        x_int8, act_scale = quantize_activations_i8(x_flat)
        out = bitnet_linear(self.packed_weight, x_int8, self.weight_scale, a_scale=act_scale.expand(m).contiguous(),
                            bias=self.bias, out_dtype=torch.float32)
        return out.view(*batch_shape, self.out_features)


class SubLNBitLinear(nn.Module):
    """SubLN followed by BitLinear, run as ONE fused RMSNorm + per-token quant kernel and the linear.

    Same math as ``nn.Sequential(SubLN(in_features, eps=1e-6), BitLinear(...))``, the layout stage 1
    gives o_proj and down_proj (packages/training/src/wrinklefree/training/stage1.py:93-113, 146-166).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False, norm_eps: float = 1e-6,
                 device=None, dtype=None):
        super().__init__()
        self.norm_weight = nn.Parameter(torch.ones(in_features, device=device, dtype=dtype))
        self.norm_eps = norm_eps
        self.linear = BitLinear(in_features, out_features, bias=bias, device=device, dtype=dtype)

    def forward(self, x: torch.Tensor, return_acc: bool = False):
        """``return_acc`` (the int32 accumulators, a parity aid) gives a result without autograd."""
        lin = self.linear
        _check_lambda("SubLNBitLinear")
        lin.ensure_packed()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, lin.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if not return_acc and torch.is_grad_enabled() and any(
                t is not None and t.requires_grad for t in (x2, self.norm_weight, lin.weight, lin.bias)):
            if lin.weight is None:
                raise RuntimeError("SubLNBitLinear: a module built from packed weights has no float weight to train")
            y = _SubLNBitLinearSTE.apply(x2, self.norm_weight, lin.weight, lin.bias, self, self.norm_eps)
            return y.view(*lead, lin.out_features)
        q, a_scale = rmsnorm_quantize_i8(x2, self.norm_weight, eps=self.norm_eps, k_pad=lin.k_pad)
        res = bitnet_linear(lin.qweight, q, lin.weight_scale, a_scale=a_scale, bias=lin.bias,
                            out_dtype=_out_dtype(x), return_acc=return_acc)
        y = res[0] if return_acc else res
        y = y.view(*lead, lin.out_features)
        y = y if y.dtype == x.dtype else y.to(x.dtype)
        return (y, res[1]) if return_acc else y


@torch.no_grad()
def convert_linear_to_bitlinear(module: nn.Module, exclude_names: Optional[List[str]] = None) -> nn.Module:
    """Replace every nn.Linear under ``module`` by a packed :class:`BitLinear` (weights copied)."""
    exclude_names = exclude_names or []
    for name, child in module.named_children():
        if name in exclude_names:
            continue
        if isinstance(child, nn.Linear) and not isinstance(child, BitLinear):
            new = BitLinear(child.in_features, child.out_features, bias=child.bias is not None,
                            device=child.weight.device, dtype=child.weight.dtype)
            new.weight.copy_(child.weight)
            if child.bias is not None:
                new.bias.copy_(child.bias)
            new.pack()
            setattr(module, name, new)
        else:
            convert_linear_to_bitlinear(child, exclude_names)
    return module


def patch_model_with_native_kernels(model: nn.Module, targets: Iterable[str] = (
        "q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")) -> nn.Module:
    """Swap the named projection Linears for packed BitLinear modules (in place); returns the model."""
    targets = set(targets)
    for parent in list(model.modules()):
        for name, child in list(parent.named_children()):
            if name in targets and isinstance(child, nn.Linear) and not isinstance(child, BitLinear):
                with torch.no_grad():
                    new = BitLinear(child.in_features, child.out_features, bias=child.bias is not None,
                                    device=child.weight.device, dtype=child.weight.dtype)
                    new.weight.copy_(child.weight)
                    if child.bias is not None:
                        new.bias.copy_(child.bias)
                    new.pack()
                setattr(parent, name, new)
    return model


class BitNetLinearMethod:
    """Serving quant method with the reference's weight schema and ``apply`` signature.

    ``per_token=True`` (default) quantises activations per token, as the BitLinear spec does;
    ``per_token=False`` reproduces the reference op's single per-tensor scale
    (torch_extension_cpu.cpp:409-426).  No fallback: failures raise RuntimeError.
    """

    block_size = QK_I2_S

    def __init__(self, per_token: bool = True):
        self.per_token = per_token

    def create_weights(self, layer: nn.Module, input_size_per_partition: int, output_partition_sizes: List[int],
                       input_size: int, output_size: int, params_dtype: torch.dtype, device=None, **_):
        if input_size_per_partition % self.block_size != 0:
            raise ValueError(
                f"BitNet: input_size_per_partition ({input_size_per_partition}) "
                f"must be divisible by block_size ({self.block_size})")
        out = sum(output_partition_sizes)
        layer.register_parameter("qweight", nn.Parameter(
            torch.empty((out, input_size_per_partition // 4), dtype=torch.uint8, device=device), requires_grad=False))
        layer.register_parameter("scale", nn.Parameter(
            torch.ones(1, dtype=torch.float32, device=device), requires_grad=False))

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        if layer.qweight.dtype != torch.uint8:
            raise ValueError(f"BitNet: Expected qweight dtype uint8, got {layer.qweight.dtype}.")

    def apply(self, layer: nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        try:
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            if self.per_token:
                q, a_scale = quantize_activations_i8_per_token(x2)
            else:
                q, s = quantize_activations_i8(x2)
                a_scale = s.expand(x2.shape[0]).contiguous()
            y = bitnet_linear(layer.qweight, q, layer.scale.data, a_scale=a_scale, bias=bias,
                              out_dtype=_out_dtype(x))
        except (ValueError, RuntimeError) as e:
            raise RuntimeError(f"BitNet apply FAILED: {e}. Native BitNet kernels are required; NO FALLBACK.") from e
        y = y.view(*x.shape[:-1], y.shape[-1])
        return y if y.dtype == x.dtype else y.to(x.dtype)
