"""Minimal BitNet b1.58 decoder (stage-1 layout) running its BitLinears on the MI355X kernels.

Layout follows the stage-1 conversion (packages/training/src/wrinklefree/training/stage1.py:63-214):
HF Llama attention/MLP with q/k/v/gate/up as BitLinear and o_proj/down_proj as SubLN + BitLinear,
gated MLP (SiLU SwiGLU, or relu^2 for the BitNet b1.58 2B form), RMSNorm before attention and MLP, HF rotary embeddings (rotate-half form), GQA.
Random init is normal(0, 0.02) for every weight and ones for every norm (BitNetLlama._init_weights,
packages/training/src/wrinklefree/models/llama.py:58-65).

Every quantised op goes through a *BitLinear backend*: one call per (norm -> quantise -> linear)
group, so the norm before q/k/v (and before gate/up) is fused with the activation quantiser and
shared by the projections that read it, and one call for the MLP middle (act(gate) * up -> SubLN ->
quantise -> down).  ``HipBackend`` runs libwfbitnet -- with ``fused=True`` the projections of a group
run as one segmented launch (q|k|v, gate|up), the gated activation, SubLN and quantiser as one
kernel, and, for decode batches where it is faster (q|k|v and o), the norm + quantiser inside the
linear's own launch (``rmsnorm_linear``); a ternary LM head runs its argmax fused in
(``norm_linear_argmax``).  A test can substitute
another backend with the same three methods to compare the quantised path while the float code stays
identical: embedding, residuals, the prefill rotary embedding + cache append + causal GQA attention
(libwfbitnet's matrix-core kernel for bf16 models, or torch ops with ``prefill_attention="torch"`` and
for fp32 models), the decode-step rotary embedding + cache append + GQA attention (one libwfbitnet
kernel, or torch ops with ``decode_attention="torch"``) and the tied LM head with its final norm and
greedy argmax (one libwfbitnet kernel).
"""

from __future__ import annotations

import copy
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import torch

from .sglbitnt import SGLBitNetFile, write_sglbitnt
from .ops import (QK_I2_S, bitnet_linear, bitnet_linear_argmax, bitnet_linear_glu,
                  bitnet_linear_residual, bitnet_linear_segmented, glu_rmsnorm_quantize_i8, gqa_decode_attention,
                  gqa_prefill_attention,
                  lm_head_argmax, pack_ternary_i2s, rmsnorm_linear, rmsnorm_linear_glu, rmsnorm_linear_glu_supported,
                  rmsnorm_linear_preferred, rmsnorm_quantize_i8, rope_tables)


@dataclass(frozen=True)
class BitNetConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float
    rms_eps: float = 1e-5   # input / post-attention / final RMSNorm
    subln_eps: float = 1e-6  # SubLN before o_proj and down_proj (stage1.py:98, 151)
    tie_embeddings: bool = True
    ternary_lm_head: bool = False
    hidden_act: str = "silu"  # gated MLP activation: "silu" (SwiGLU) or "relu2" (BitNet b1.58 2B)


# SmolLM2-135M architecture (packages/training/configs/model/smollm2_135m.yaml)
SMOLLM2_135M = BitNetConfig(vocab_size=49152, hidden_size=576, intermediate_size=1536, num_layers=30, num_heads=9,
                            num_kv_heads=3, head_dim=64, rope_theta=100000.0)
# BitNet b1.58 2B4T architecture (the BitNet-2B shapes of configs[1]; the model of the MS BitNet GPU
# end-to-end latency table, packages/inference/extern/BitNet/gpu/README.md:91-105): relu^2 MLP, GQA 20/5,
# tied bf16 embedding head
BITNET_2B = BitNetConfig(vocab_size=128256, hidden_size=2560, intermediate_size=6912, num_layers=30, num_heads=20,
                         num_kv_heads=5, head_dim=128, rope_theta=500000.0, hidden_act="relu2")
# Llama-3-8B architecture, every linear ternary (incl. the LM head)
LLAMA3_8B = BitNetConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_layers=32, num_heads=32,
                         num_kv_heads=8, head_dim=128, rope_theta=500000.0, tie_embeddings=False,
                         ternary_lm_head=True)


def _pad_k(k: int) -> int:
    return (k + QK_I2_S - 1) // QK_I2_S * QK_I2_S


class PackedLinear:
    """I2_S weight of one projection: qweight uint8 [out, k_pad/4], scale fp32 [1] (device)."""

    def __init__(self, weight: torch.Tensor):
        self.out_features, self.in_features = weight.shape
        self.k_pad = _pad_k(self.in_features)
        self.qweight, self.scale = pack_ternary_i2s(weight.contiguous(), k_pad=self.k_pad)

    @classmethod
    def from_packed(cls, qweight: torch.Tensor, scale: torch.Tensor, in_features: int) -> "PackedLinear":
        """Wrap an already packed I2_S weight (uint8 [out, k_pad/4]) and its fp32 scale [1]."""
        lin = cls.__new__(cls)
        lin.out_features, lin.k_pad = qweight.shape[0], qweight.shape[1] * 4
        if lin.k_pad % QK_I2_S != 0 or not in_features <= lin.k_pad < in_features + QK_I2_S:
            raise ValueError(f"packed weight of {lin.k_pad} columns does not fit in_features={in_features}")
        lin.in_features = in_features
        lin.qweight, lin.scale = qweight.contiguous(), scale.reshape(1).to(torch.float32).contiguous()
        return lin


class HipBackend:
    """Quantised BitLinear groups on libwfbitnet: fused RMSNorm/SubLN + per-token int8 quantisation,
    then the projections with the rescale fused in their epilogue.

    ``fused=True``: the projections of a group (q|k|v, gate|up) run as one segmented launch on their
    concatenated weights, residual adds ride in the o/down epilogues, and for decode batches the
    norm + quantiser before q|k|v and o runs in the linear's prologue where that is measured faster
    (``rmsnorm_linear_preferred``): a Llama-3-8B decode layer takes 8 kernel launches (norm+q|k|v,
    attention and its split combine, SubLN+o+residual, norm+quant, gate|up, act+SubLN+quant,
    down+residual) instead of 12."""

    def __init__(self, out_dtype: torch.dtype = torch.float32, keep_acc: bool = False, fused: bool = False):
        self.out_dtype = out_dtype
        self.keep_acc = keep_acc
        self.fused = fused
        self.acc_log: List[torch.Tensor] = []
        self._groups: Dict[tuple, tuple] = {}

    def _group(self, linears: Sequence[PackedLinear]):
        key = tuple(id(l) for l in linears)
        g = self._groups.get(key)
        if g is None:
            qw = torch.cat([l.qweight for l in linears], dim=0).contiguous()
            sc = torch.cat([l.scale.reshape(1) for l in linears]).contiguous()
            g = (qw, sc, [l.out_features for l in linears])
            self._groups[key] = g
        return g

    def _linears(self, q: torch.Tensor, a_scale: torch.Tensor, linears: Sequence[PackedLinear]) -> List[torch.Tensor]:
        if self.fused and len(linears) > 1:
            qw, sc, rows = self._group(linears)
            if self.keep_acc:
                y, acc = bitnet_linear_segmented(qw, rows, sc, q, a_scale=a_scale, out_dtype=self.out_dtype,
                                                 return_acc=True)
                self.acc_log.extend(torch.split(acc, rows, dim=1))
            else:
                y = bitnet_linear_segmented(qw, rows, sc, q, a_scale=a_scale, out_dtype=self.out_dtype)
            return list(torch.split(y, rows, dim=1))
        outs = []
        for lin in linears:
            if self.keep_acc:
                y, acc = bitnet_linear(lin.qweight, q, lin.scale, a_scale=a_scale, out_dtype=self.out_dtype,
                                       return_acc=True)
                self.acc_log.append(acc)
            else:
                y = bitnet_linear(lin.qweight, q, lin.scale, a_scale=a_scale, out_dtype=self.out_dtype)
            outs.append(y)
        return outs

    def _fused_norm(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor], n: int, k: int,
                    glu: bool = False) -> bool:
        """Norm + quant in the linear's prologue (one launch) where that is the faster choice (``glu``: the
        gated gate|up form, rmsnorm_linear_glu)."""
        if not self.fused or self.keep_acc or x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16):
            return False
        if norm_weight is not None and norm_weight.dtype not in (torch.float32, torch.bfloat16):
            return False
        if glu:
            return rmsnorm_linear_glu_supported(x.shape[0], x.shape[1], k)
        gb = 0 if norm_weight is None else norm_weight.element_size()
        return rmsnorm_linear_preferred(x.shape[0], x.shape[1], n, k, gb)

    def norm_linears(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor], eps: float,
                     linears: Sequence[PackedLinear]) -> List[torch.Tensor]:
        n = sum(l.out_features for l in linears)
        if self._fused_norm(x, norm_weight, n, linears[0].k_pad):
            if len(linears) > 1:
                qw, sc, rows = self._group(linears)
            else:
                qw, sc, rows = linears[0].qweight, linears[0].scale.reshape(1), [n]
            y = rmsnorm_linear(x, norm_weight, qw, sc, rows, eps=eps, out_dtype=self.out_dtype)
            return list(torch.split(y, rows, dim=1))
        q, a_scale = rmsnorm_quantize_i8(x, norm_weight, eps=eps, k_pad=linears[0].k_pad)
        return self._linears(q, a_scale, linears)

    def norm_linear_argmax(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor], eps: float,
                           linear: PackedLinear) -> torch.Tensor:
        """Greedy next tokens int64 [M] of a ternary LM head: norm + quantise, then the linear with the argmax
        fused in (fp32 logits compared, as the reference engine's std::max_element, never stored)."""
        q, a_scale = rmsnorm_quantize_i8(x, norm_weight, eps=eps, k_pad=linear.k_pad)
        if self.keep_acc:
            self._linears(q, a_scale, [linear])
        return bitnet_linear_argmax(linear.qweight, q, linear.scale, a_scale=a_scale, logits_dtype=torch.float32)

    def _linear_residual(self, q: torch.Tensor, a_scale: torch.Tensor, linear: PackedLinear,
                         residual: torch.Tensor) -> torch.Tensor:
        if self.keep_acc:
            self._linears(q, a_scale, [linear])[0]
        return bitnet_linear_residual(linear.qweight, q, linear.scale, residual.contiguous(), a_scale=a_scale)

    def norm_linear_residual(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor], eps: float,
                             linear: PackedLinear, residual: torch.Tensor) -> torch.Tensor:
        """residual + linear(quantise(norm(x))), the add fused into the linear's epilogue (fp32 add, then
        the residual's dtype)."""
        if self._fused_norm(x, norm_weight, linear.out_features, linear.k_pad) and residual.dtype in (
                torch.float32, torch.bfloat16):
            return rmsnorm_linear(x, norm_weight, linear.qweight, linear.scale.reshape(1), eps=eps,
                                  residual=residual.contiguous())
        q, a_scale = rmsnorm_quantize_i8(x, norm_weight, eps=eps, k_pad=linear.k_pad)
        return self._linear_residual(q, a_scale, linear, residual)

    def mlp_residual(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor], eps: float, gate: PackedLinear,
                     up: PackedLinear, act: str, sub_norm: Optional[torch.Tensor], sub_eps: float, down: PackedLinear,
                     residual: torch.Tensor) -> torch.Tensor:
        """residual + down(quantise(SubLN(act(gate(h)) * up(h)))), h = quantise(norm(x)).  For decode batches
        the gated product rides in the gate|up launch's epilogue (``bitnet_linear_glu``, fp32), and SubLN +
        quantise runs on it as a plain row quantiser -- the same codes as the separate gated kernel."""
        half = gate.out_features
        if (self.fused and not self.keep_acc and x.dim() == 2 and x.shape[0] <= 64 and up.out_features == half
                and half % 32 == 0 and act in ("silu", "relu2")):
            qw, sc, _ = self._group([gate, up])
            if self._fused_norm(x, norm_weight, 2 * half, gate.k_pad, glu=True):
                mid = rmsnorm_linear_glu(x, norm_weight, qw, sc, act, eps=eps, mid_dtype=self.out_dtype)
            else:
                q, a_scale = rmsnorm_quantize_i8(x, norm_weight, eps=eps, k_pad=gate.k_pad)
                mid = bitnet_linear_glu(qw, sc, q, act, a_scale=a_scale, mid_dtype=self.out_dtype)
            return self.norm_linear_residual(mid, sub_norm, sub_eps, down, residual)
        g, u = self.norm_linears(x, norm_weight, eps, [gate, up])
        return self.glu_norm_linear_residual(g, u, act, sub_norm, sub_eps, down, residual)

    def glu_norm_linear_residual(self, gate: torch.Tensor, up: torch.Tensor, act: str,
                                 norm_weight: Optional[torch.Tensor], eps: float, linear: PackedLinear,
                                 residual: torch.Tensor) -> torch.Tensor:
        """residual + linear(quantise(SubLN(act(gate) * up)))."""
        if gate.stride(-1) != 1 or up.stride(-1) != 1 or gate.stride(0) != up.stride(0):
            gate, up = gate.contiguous(), up.contiguous()
        q, a_scale = glu_rmsnorm_quantize_i8(gate, up, act, norm_weight, eps=eps, k_pad=linear.k_pad)
        return self._linear_residual(q, a_scale, linear, residual)

    def glu_norm_linears(self, gate: torch.Tensor, up: torch.Tensor, act: str, norm_weight: Optional[torch.Tensor],
                         eps: float, linears: Sequence[PackedLinear]) -> List[torch.Tensor]:
        """act(gate) * up -> SubLN -> per-token int8 -> linears (one kernel before the projections)."""
        if gate.stride(-1) != 1 or up.stride(-1) != 1 or gate.stride(0) != up.stride(0):
            gate, up = gate.contiguous(), up.contiguous()
        q, a_scale = glu_rmsnorm_quantize_i8(gate, up, act, norm_weight, eps=eps, k_pad=linears[0].k_pad)
        return self._linears(q, a_scale, linears)


class _Layer:
    def __init__(self, cfg: BitNetConfig, gen: torch.Generator, device: torch.device, dtype: torch.dtype):
        h, f = cfg.hidden_size, cfg.intermediate_size
        qd, kvd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim

        def w(o, i):
            return (torch.randn((o, i), generator=gen, dtype=torch.float32, device=gen.device) * 0.02).to(device)

        self.q, self.k, self.v = PackedLinear(w(qd, h)), PackedLinear(w(kvd, h)), PackedLinear(w(kvd, h))
        self.o = PackedLinear(w(h, qd))
        self.gate, self.up = PackedLinear(w(f, h)), PackedLinear(w(f, h))
        self.down = PackedLinear(w(h, f))
        ones = lambda n: torch.ones(n, device=device, dtype=dtype)  # noqa: E731
        self.input_norm, self.attn_sub_norm = ones(h), ones(qd)
        self.post_attn_norm, self.ffn_sub_norm = ones(h), ones(f)


class BitNetDecoder:
    """Decoder-only BitNet model with a per-layer KV cache; float glue in ``dtype``."""

    def __init__(self, cfg: BitNetConfig, seed: int = 0, device: str = "cuda", dtype: torch.dtype = torch.float32,
                 backend=None, init_on_device: bool = False, decode_attention: str = "hip",
                 prefill_attention: str = "hip"):
        """``init_on_device``: draw the random weights with a generator on ``device`` (fast for 8B-scale
        models) instead of the host generator (the default, reproducible across devices).
        ``decode_attention``: "hip" runs each decode step's rotary embedding, cache append and GQA attention
        as one libwfbitnet kernel; "torch" runs them as torch ops.  ``prefill_attention``: "hip" runs a
        prompt's rotary embedding, cache append and causal attention on libwfbitnet's matrix-core kernel
        (bf16 models with head_dim 64/128 and at most 8 query heads per kv head; other models use torch);
        "steps" runs it as one decode-attention launch per prompt position (any model dtype; the native
        engine's fp32 prompt path); "torch" always uses torch ops."""
        self._setup(cfg, device, dtype, backend, decode_attention, prefill_attention)
        gen = torch.Generator(device=self.device if init_on_device else "cpu").manual_seed(seed)
        self.embed = (torch.randn((cfg.vocab_size, cfg.hidden_size), generator=gen, device=gen.device) * 0.02).to(
            self.device, dtype)
        self.layers = [_Layer(cfg, gen, self.device, dtype) for _ in range(cfg.num_layers)]
        self.final_norm = torch.ones(cfg.hidden_size, device=self.device, dtype=dtype)
        if cfg.ternary_lm_head:
            self.lm_head = PackedLinear((torch.randn((cfg.vocab_size, cfg.hidden_size), generator=gen,
                                                     device=gen.device) * 0.02)
                                        .to(self.device))
        else:
            self.lm_head = None  # tied to the embedding
        self.head_weight = self.embed

    def _setup(self, cfg: BitNetConfig, device, dtype: torch.dtype, backend, decode_attention: str,
               prefill_attention: str = "hip") -> None:
        if decode_attention not in ("hip", "torch") or prefill_attention not in ("hip", "torch", "steps"):
            raise ValueError("decode_attention must be 'hip' or 'torch', prefill_attention 'hip', 'steps' or 'torch'")
        self.decode_attention = decode_attention
        self.prefill_attention = prefill_attention
        self.fuse_residual = True  # residual adds in the o / down epilogues when the backend offers it
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        self.backend = backend if backend is not None else HipBackend(out_dtype=dtype if dtype == torch.float32
                                                                       else torch.bfloat16)
        self.kv: List[Optional[List[torch.Tensor]]] = []
        self._lm_t = None

    # ---- SGLBITNT files (the reference engine's packed-model format) ----------------------------

    _LINEARS = (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                ("down", "mlp.down_proj"))
    _NORMS = (("input_norm", "input_layernorm"), ("post_attn_norm", "post_attention_layernorm"),
              ("attn_sub_norm", "self_attn.attn_sub_norm"), ("ffn_sub_norm", "mlp.ffn_sub_norm"))

    def save_sglbitnt(self, path, config_overrides: Optional[Dict] = None) -> None:
        """Write the model as an SGLBITNT file with the tensor names the reference engine loads
        (SGB/sgl-kernel/csrc/inference/bitnet_engine.cpp:622-668): packed linears uint8 [out, k_pad/4] with
        their scale, embedding and norms as float32, a ternary LM head (uint8) or an untied dense head
        (float32) as lm_head.weight, none for a head tied to the embedding.  The config's ``torch_dtype`` is the
        model's glue dtype ("float32" or "bfloat16"), which the native engine computes in.
        ``config_overrides``: extra or replaced keys of the config JSON (e.g. ``eos_token_id``)."""
        cfg = self.cfg
        config = {"vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size,
                  "intermediate_size": cfg.intermediate_size, "num_hidden_layers": cfg.num_layers,
                  "num_attention_heads": cfg.num_heads, "num_key_value_heads": cfg.num_kv_heads,
                  "head_dim": cfg.head_dim, "rope_theta": cfg.rope_theta, "rms_norm_eps": cfg.rms_eps,
                  "subln_eps": cfg.subln_eps, "tie_word_embeddings": self.lm_head is None,
                  "hidden_act": cfg.hidden_act, "max_position_embeddings": 4096,
                  "torch_dtype": "float32" if self.dtype == torch.float32 else "bfloat16"}
        t = {"model.embed_tokens.weight": (self.embed.float(), None)}
        for i, L in enumerate(self.layers):
            pre = f"model.layers.{i}."
            for attr, name in self._LINEARS:
                lin = getattr(L, attr)
                t[pre + name + ".weight"] = (lin.qweight, float(lin.scale.item()))
            for attr, name in self._NORMS:
                t[pre + name + ".weight"] = (getattr(L, attr).float(), None)
        t["model.norm.weight"] = (self.final_norm.float(), None)
        if self.lm_head is not None:
            t["lm_head.weight"] = (self.lm_head.qweight, float(self.lm_head.scale.item()))
        elif self.head_weight is not self.embed:
            t["lm_head.weight"] = (self.head_weight.float(), None)
        config["tie_word_embeddings"] = self.lm_head is None and self.head_weight is self.embed
        config.update(config_overrides or {})
        write_sglbitnt(path, config, t)

    @classmethod
    def from_float_state(cls, state: Dict[str, torch.Tensor], cfg: BitNetConfig, device="cuda",
                         dtype: torch.dtype = torch.float32, backend=None, decode_attention: str = "hip",
                         prefill_attention: str = "hip") -> "BitNetDecoder":
        """Build the model from float weights under HuggingFace Llama names (``model.embed_tokens.weight``,
        ``model.layers.{i}.self_attn.q_proj.weight`` ... ``model.norm.weight``, optional ``lm_head.weight``),
        the names of the stage-1 source model (stage1.py:169-214).  Every projection is absmean-ternarised
        and packed on the device.  SubLN weights are read from the converted model's names
        (``self_attn.o_proj.0.weight``, ``mlp.down_proj.0.weight``) when present, else ones, as stage 1
        creates them.  A ternary LM head (``cfg.ternary_lm_head``) is packed from ``lm_head.weight``; a
        dense untied head keeps it as floats; a tied head uses the embedding."""
        m = cls.__new__(cls)
        m._setup(cfg, device, dtype, backend, decode_attention, prefill_attention)
        dev = m.device

        def get(name, shape=None, ones=False):
            t = state.get(name)
            if t is None:
                if not ones:
                    raise KeyError(f"from_float_state: missing {name}")
                return torch.ones(shape, device=dev, dtype=dtype)
            if shape is not None and tuple(t.shape) != tuple(shape):
                raise ValueError(f"from_float_state: {name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
            return t

        h, f = cfg.hidden_size, cfg.intermediate_size
        qd, kvd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
        shapes = {"q": (qd, h), "k": (kvd, h), "v": (kvd, h), "o": (h, qd), "gate": (f, h), "up": (f, h),
                  "down": (h, f)}
        m.embed = get("model.embed_tokens.weight", (cfg.vocab_size, h)).to(dev, dtype)
        m.layers = []
        for i in range(cfg.num_layers):
            L = _Layer.__new__(_Layer)
            pre = f"model.layers.{i}."
            for attr, name in cls._LINEARS:
                w = get(pre + name + ".weight", shapes[attr]).to(dev, torch.float32)
                setattr(L, attr, PackedLinear(w))
            L.input_norm = get(pre + "input_layernorm.weight", (h,)).to(dev, dtype)
            L.post_attn_norm = get(pre + "post_attention_layernorm.weight", (h,)).to(dev, dtype)
            L.attn_sub_norm = get(pre + "self_attn.o_proj.0.weight", (qd,), ones=True).to(dev, dtype)
            L.ffn_sub_norm = get(pre + "mlp.down_proj.0.weight", (f,), ones=True).to(dev, dtype)
            m.layers.append(L)
        m.final_norm = get("model.norm.weight", (h,)).to(dev, dtype)
        head = None if cfg.tie_embeddings else get("lm_head.weight", (cfg.vocab_size, h))
        m.lm_head = PackedLinear(head.to(dev, torch.float32)) if cfg.ternary_lm_head else None
        m.head_weight = m.embed if head is None or cfg.ternary_lm_head else head.to(dev, dtype)
        return m

    @classmethod
    def from_sglbitnt(cls, path, device="cuda", dtype: torch.dtype = torch.float32, backend=None,
                      decode_attention: str = "hip", prefill_attention: str = "hip") -> "BitNetDecoder":
        """Build the model from an SGLBITNT file (memory-mapped; tensors go to ``device`` one at a time).
        Packed linears keep their I2_S bytes and scale; a uint8 lm_head.weight is a ternary LM head, a float
        one a dense head, none a head tied to the embedding.  Missing SubLN weights are ones (the engine
        skips them, bitnet_engine.cpp:664-668)."""
        f = SGLBitNetFile(path)
        c = f.config
        heads = int(c["num_attention_heads"])
        head_t = f.tensors.get("lm_head.weight")
        cfg = BitNetConfig(vocab_size=int(c["vocab_size"]), hidden_size=int(c["hidden_size"]),
                           intermediate_size=int(c["intermediate_size"]), num_layers=int(c["num_hidden_layers"]),
                           num_heads=heads, num_kv_heads=int(c.get("num_key_value_heads", heads)),
                           head_dim=int(c.get("head_dim", int(c["hidden_size"]) // heads)),
                           rope_theta=float(c.get("rope_theta", 10000.0)),
                           rms_eps=float(c.get("rms_norm_eps", 1e-5)), subln_eps=float(c.get("subln_eps", 1e-6)),
                           tie_embeddings=head_t is None,
                           ternary_lm_head=head_t is not None and head_t.dtype_id == 0,
                           hidden_act=str(c.get("hidden_act", "silu")))
        m = cls.__new__(cls)
        m._setup(cfg, device, dtype, backend, decode_attention, prefill_attention)
        dev = m.device

        def packed(name, in_features):
            info = f.tensors[name]
            if info.dtype_id != 0 or len(info.shape) != 2:
                raise ValueError(f"{name}: expected a packed uint8 [out, in/4] weight")
            scale = torch.tensor([1.0 if info.scale is None else info.scale], dtype=torch.float32, device=dev)
            return PackedLinear.from_packed(f.tensor(name, dev), scale, in_features)

        def floats(name, n):
            if name not in f:
                return torch.ones(n, device=dev, dtype=dtype)
            return f.tensor(name, dev).to(dtype).reshape(n)

        h, inter = cfg.hidden_size, cfg.intermediate_size
        qd = cfg.num_heads * cfg.head_dim
        ins = {"q": h, "k": h, "v": h, "o": qd, "gate": h, "up": h, "down": inter}
        sizes = {"input_norm": h, "post_attn_norm": h, "attn_sub_norm": qd, "ffn_sub_norm": inter}
        m.embed = f.tensor("model.embed_tokens.weight", dev).to(dtype)
        m.layers = []
        for i in range(cfg.num_layers):
            L = _Layer.__new__(_Layer)
            pre = f"model.layers.{i}."
            for attr, name in cls._LINEARS:
                setattr(L, attr, packed(pre + name + ".weight", ins[attr]))
            for attr, name in cls._NORMS:
                setattr(L, attr, floats(pre + name + ".weight", sizes[attr]))
            m.layers.append(L)
        m.final_norm = floats("model.norm.weight", h)
        m.lm_head = packed("lm_head.weight", h) if cfg.ternary_lm_head else None
        m.head_weight = m.embed if head_t is None else (m.embed if cfg.ternary_lm_head else
                                                        f.tensor("lm_head.weight", dev).to(dtype))
        return m

    # ---- float glue --------------------------------------------------------------------------

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """HF rotate-half rotary embedding; x [B, T, H, D], pos [T] (rows of the tables set by reset, the values
        the attention kernels use)."""
        c = self._rope_cos.index_select(0, pos.to(self._rope_cos.device))
        s = self._rope_sin.index_select(0, pos.to(self._rope_sin.device))
        cos, sin = torch.cat([c, c], dim=-1)[None, :, None, :], torch.cat([s, s], dim=-1)[None, :, None, :]
        x32 = x.to(torch.float32)
        half = x32.shape[-1] // 2
        rot = torch.cat([-x32[..., half:], x32[..., :half]], dim=-1)
        return (x32 * cos + rot * sin).to(x.dtype)

    def _rmsnorm(self, x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
        x32 = x.to(torch.float32)
        return (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps) * w.to(torch.float32)).to(x.dtype)

    def _cache(self, li: int, b: int):
        """Layer li's KV cache in the model dtype: K and V [B, kv, L_max, D] (one key = D contiguous
        elements, the layout of the decode attention kernel)."""
        cache = self.kv[li]
        if cache is None:
            cfg = self.cfg
            shape = (b, cfg.num_kv_heads, self._max_len, cfg.head_dim)
            cache = [torch.zeros(shape, device=self.device, dtype=self.dtype),
                     torch.zeros(shape, device=self.device, dtype=self.dtype)]
            self.kv[li] = cache
        return cache

    def _attention(self, li: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, start: int) -> torch.Tensor:
        """Causal GQA attention of T new tokens at positions start.. over the KV cache.  The rep =
        heads / kv_heads query heads that share a kv head are stacked as rows of one matrix
        ([B, kv, rep*T, D]), so no kv repeat is materialised."""
        cfg = self.cfg
        b, t = q.shape[0], q.shape[1]
        kvh, rep, hd = cfg.num_kv_heads, cfg.num_heads // cfg.num_kv_heads, cfg.head_dim
        kc, vc = self._cache(li, b)
        kc[:, :, start:start + t] = k.transpose(1, 2)
        vc[:, :, start:start + t] = v.transpose(1, 2)
        # head h = g*rep + r reads kv head g (repeat_interleave order)
        qq = q.to(torch.float32).reshape(b, t, kvh, rep, hd).permute(0, 2, 3, 1, 4).reshape(b, kvh, rep * t, hd)
        kt = kc[:, :, :start + t].to(torch.float32).transpose(2, 3).contiguous()
        scores = torch.matmul(qq.contiguous(), kt) / math.sqrt(hd)
        if t > 1:
            mask = torch.ones((t, start + t), device=self.device, dtype=torch.bool).tril(diagonal=start)
            scores = scores.masked_fill(~mask.repeat(rep, 1), float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        out = torch.matmul(probs, vc[:, :, :start + t].to(torch.float32))      # [B, kv, rep*T, D]
        out = out.reshape(b, kvh, rep, t, hd).permute(0, 3, 1, 2, 4)           # [B, T, kv, rep, D]
        return out.reshape(b, t, cfg.num_heads * hd).to(self.dtype)

    def _attention_step_torch(self, li: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              pos: torch.Tensor) -> torch.Tensor:
        """One decode token per sequence as torch ops, at the device position pos[0] shared by the batch
        (fixed shapes, so it can be captured in a HIP graph): rotary embedding, the cache write indexed
        by pos, scores over the whole cache with keys past pos masked.  q/k/v are [B, heads*D] rows."""
        cfg = self.cfg
        b = q.shape[0]
        kvh, rep, hd = cfg.num_kv_heads, cfg.num_heads // cfg.num_kv_heads, cfg.head_dim
        p1 = pos[:1]
        q = self._rope(q.reshape(b, 1, cfg.num_heads, hd), p1)
        k = self._rope(k.reshape(b, 1, kvh, hd), p1)
        kc, vc = self._cache(li, b)
        kc.index_copy_(2, p1, k.transpose(1, 2))
        vc.index_copy_(2, p1, v.reshape(b, 1, kvh, hd).transpose(1, 2))
        qq = q.to(torch.float32).reshape(b, kvh, rep, hd)
        scores = torch.matmul(qq, kc.to(torch.float32).transpose(2, 3).contiguous()) / math.sqrt(hd)
        scores = scores.masked_fill(self._key_pos > p1, float("-inf"))          # [B, kv, rep, L_max]
        probs = torch.softmax(scores, dim=-1)
        out = torch.matmul(probs, vc.to(torch.float32))                         # [B, kv, rep, D]
        return out.reshape(b, cfg.num_heads * hd).to(self.dtype)

    def _attention_step_hip(self, li: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            pos: torch.Tensor) -> torch.Tensor:
        """One decode token per sequence in one kernel: rotary embedding of q and k, cache append at pos[b],
        GQA attention over positions 0..pos[b].  q/k/v are [B, heads*D] rows (possibly column slices of
        one q|k|v output)."""
        kc, vc = self._cache(li, q.shape[0])
        return gqa_decode_attention(q, k, v, kc, vc, pos, self._rope_cos, self._rope_sin,
                                    scale=1.0 / math.sqrt(self.cfg.head_dim))

    # ---- forward -------------------------------------------------------------------------------

    def reset(self, batch: int, max_len: int) -> None:
        self._max_len = max_len
        self.kv = [None] * self.cfg.num_layers
        self._key_pos = torch.arange(max_len, device=self.device)
        # cos / sin of every cache position from libwfbitnet's tables (the native engine's values)
        cos, sin = _rope_tables_cpu(self.cfg.rope_theta, self.cfg.head_dim, max_len)
        self._rope_cos, self._rope_sin = cos.to(self.device), sin.to(self.device)

    def _layers(self, x: torch.Tensor, attend, first: int = 0, last: Optional[int] = None) -> torch.Tensor:
        cfg, be = self.cfg, self.backend
        b, t = x.shape[0], x.shape[1]
        for li in range(first, len(self.layers) if last is None else last):
            L = self.layers[li]
            h2 = x.reshape(b * t, cfg.hidden_size)
            q, k, v = be.norm_linears(h2, L.input_norm, cfg.rms_eps, [L.q, L.k, L.v])
            attn = attend(li, q.to(self.dtype), k.to(self.dtype), v.to(self.dtype)).reshape(b * t, -1)
            fused_res = self.fuse_residual and hasattr(be, "norm_linear_residual")
            if fused_res:
                x = be.norm_linear_residual(attn, L.attn_sub_norm, cfg.subln_eps, L.o, h2).reshape(b, t, -1)
            else:
                (o,) = be.norm_linears(attn, L.attn_sub_norm, cfg.subln_eps, [L.o])
                x = x + o.reshape(b, t, -1).to(self.dtype)
            h2 = x.reshape(b * t, cfg.hidden_size)
            if fused_res and hasattr(be, "mlp_residual"):
                x = be.mlp_residual(h2, L.post_attn_norm, cfg.rms_eps, L.gate, L.up, cfg.hidden_act, L.ffn_sub_norm,
                                    cfg.subln_eps, L.down, h2).reshape(b, t, -1)
                continue
            gate, up = be.norm_linears(h2, L.post_attn_norm, cfg.rms_eps, [L.gate, L.up])
            if fused_res:
                x = be.glu_norm_linear_residual(gate, up, cfg.hidden_act, L.ffn_sub_norm, cfg.subln_eps, L.down,
                                                h2).reshape(b, t, -1)
            else:
                (down,) = be.glu_norm_linears(gate, up, cfg.hidden_act, L.ffn_sub_norm, cfg.subln_eps, [L.down])
                x = x + down.reshape(b, t, -1).to(self.dtype)
        return x

    def _logits(self, last: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        if self.lm_head is not None:
            (logits,) = self.backend.norm_linears(last.contiguous(), self.final_norm, cfg.rms_eps, [self.lm_head])
            return logits.to(torch.float32)
        if getattr(self, "_lm_t", None) is None:
            self._lm_t = self.head_weight.to(torch.float32).t().contiguous()  # dense LM head, [H, vocab]
        hn = self._rmsnorm(last, self.final_norm, cfg.rms_eps).to(torch.float32)
        return torch.matmul(hn, self._lm_t)

    def _next_tokens(self, last: torch.Tensor) -> torch.Tensor:
        """Greedy next token ids int64 [B] from the last hidden states [B, H]: the final norm, LM head and
        argmax on the device (ternary head through the backend, tied head through lm_head_argmax)."""
        cfg = self.cfg
        if self.lm_head is not None:
            return self.backend.norm_linear_argmax(last.contiguous(), self.final_norm, cfg.rms_eps, self.lm_head)
        if self.device.type != "cuda":  # host copy of the model (see on_host)
            return torch.argmax(self._logits(last), dim=-1)
        return lm_head_argmax(last.contiguous(), self.head_weight, self.final_norm, cfg.rms_eps)

    def on_host(self, backend) -> "BitNetDecoder":
        """A copy whose float glue runs on the CPU (torch ops, decode attention included) and whose
        quantised groups go to ``backend`` (a host backend holding its own copy of the packed weights);
        the packed weights themselves are shared, not copied."""
        cpu = torch.device("cpu")
        m = copy.copy(self)
        m.device, m.backend, m.decode_attention, m.prefill_attention = cpu, backend, "torch", "torch"
        m.embed, m.final_norm = self.embed.to(cpu), self.final_norm.to(cpu)
        m.head_weight = m.embed if self.head_weight is self.embed else self.head_weight.to(cpu)
        m.layers = []
        for L in self.layers:
            c = copy.copy(L)
            for n in ("input_norm", "attn_sub_norm", "post_attn_norm", "ffn_sub_norm"):
                setattr(c, n, getattr(L, n).to(cpu))
            m.layers.append(c)
        m.kv, m._lm_t = [], None
        return m

    def _prefill_attend(self, b: int, t: int, start: int):
        cfg = self.cfg
        pos = torch.arange(start, start + t, device=self.device)

        def attend(li, q, k, v):
            if self._hip_prefill():
                kc, vc = self._cache(li, b)
                return gqa_prefill_attention(q, k, v, kc, vc, start, t, self._rope_cos, self._rope_sin,
                                             scale=1.0 / math.sqrt(cfg.head_dim))
            if self.prefill_attention == "steps" and self.device.type == "cuda":
                return self._prefill_by_steps(li, q, k, v, b, t, start)
            q = self._rope(q.reshape(b, t, cfg.num_heads, cfg.head_dim), pos)
            k = self._rope(k.reshape(b, t, cfg.num_kv_heads, cfg.head_dim), pos)
            return self._attention(li, q, k, v.reshape(b, t, cfg.num_kv_heads, cfg.head_dim), start)

        return attend

    def _prefill_by_steps(self, li: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, b: int, t: int,
                          start: int) -> torch.Tensor:
        """The prompt's attention as one decode-attention launch per position (the native engine's fp32 prompt
        path, and the reference engine's token-by-token loop, bitnet_engine.cpp:381-441): token i of every
        sequence ropes and appends its key and value at start + i and attends over keys 0..start + i.
        q/k/v are [B*T, width] rows (possibly column slices of one q|k|v output)."""
        cfg = self.cfg
        kc, vc = self._cache(li, b)
        qd = cfg.num_heads * cfg.head_dim
        q3, k3, v3 = q.unflatten(0, (b, t)), k.unflatten(0, (b, t)), v.unflatten(0, (b, t))
        pos = (torch.arange(start, start + t, device=self.device)[:, None]).expand(t, b).contiguous()
        out = torch.empty((b, t, qd), dtype=q.dtype, device=self.device)
        for i in range(t):
            gqa_decode_attention(q3[:, i], k3[:, i], v3[:, i], kc, vc, pos[i], self._rope_cos, self._rope_sin,
                                 scale=1.0 / math.sqrt(cfg.head_dim), out=out[:, i])
        return out.reshape(b * t, qd)

    def forward(self, ids: torch.Tensor, start: int, tokens: bool = False) -> torch.Tensor:
        """ids [B, T] at positions start..start+T-1; returns fp32 logits of the last position [B, vocab], or
        with ``tokens`` the greedy next ids [B]."""
        b, t = ids.shape
        x = self._layers(self.embed[ids], self._prefill_attend(b, t, start))
        return self._next_tokens(x[:, -1, :]) if tokens else self._logits(x[:, -1, :])

    def forward_layers(self, hidden: torch.Tensor, start: int, first: int = 0, last: Optional[int] = None
                       ) -> torch.Tensor:
        """Hidden states [B, T, H] at positions start..start+T-1 through layers first..last-1 (the residual
        stream a HuggingFace decoder layer takes and returns), appending to those layers' KV caches."""
        b, t = hidden.shape[0], hidden.shape[1]
        return self._layers(hidden.to(self.device, self.dtype), self._prefill_attend(b, t, start), first, last)

    def _hip_prefill(self) -> bool:
        cfg = self.cfg
        return (self.prefill_attention == "hip" and self.device.type == "cuda" and self.dtype == torch.bfloat16
                and cfg.head_dim in (64, 128) and cfg.num_heads % cfg.num_kv_heads == 0
                and cfg.num_heads // cfg.num_kv_heads <= 8)

    def decode_step(self, ids: torch.Tensor, pos: torch.Tensor, tokens: bool = False) -> torch.Tensor:
        """One token per sequence, ids [B, 1] at the device positions pos int64 [B]; fixed shapes and no
        host values, so the step can be captured once and replayed.  Returns fp32 logits [B, vocab], or
        with ``tokens`` the greedy next ids [B]."""
        attend = self._attention_step_hip if self.decode_attention == "hip" else self._attention_step_torch
        x = self._layers(self.embed[ids], lambda li, q, k, v: attend(li, q, k, v, pos))
        return self._next_tokens(x[:, -1, :]) if tokens else self._logits(x[:, -1, :])

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, new_tokens: int, graph: bool = False,
                 max_len: Optional[int] = None) -> torch.Tensor:
        """Greedy decoding: prompt [B, T0] -> generated ids [B, new_tokens].  The prompt is one
        forward; every further token is decode_step, run directly or (graph=True) replayed from one
        HIP graph capture, the next ids, position and output column updated on the device.  ``max_len``:
        KV cache positions (default T0 + new_tokens; the split decode attention's key splits follow it)."""
        b, t0 = prompt.shape
        max_len = t0 + new_tokens if max_len is None else int(max_len)
        if max_len < t0 + new_tokens:
            raise ValueError(f"generate: max_len {max_len} < prompt + new tokens ({t0 + new_tokens})")
        self.reset(b, max_len)
        nxt = self.forward(prompt.to(self.device), 0, tokens=True)
        out = torch.empty((b, new_tokens), dtype=torch.long, device=self.device)
        out[:, 0] = nxt
        ids = nxt[:, None].clone()
        pos = torch.full((b,), t0, dtype=torch.long, device=self.device)
        col = torch.ones(1, dtype=torch.long, device=self.device)

        def step():
            n = self.decode_step(ids, pos, tokens=True)
            out.index_copy_(1, col, n[:, None])
            ids.copy_(n[:, None])
            pos.add_(1)
            col.add_(1)

        steps = new_tokens - 1
        if not graph or steps < 2:
            for _ in range(steps):
                step()
            return out
        step()  # also the warm-up before capture
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                step()
        torch.cuda.current_stream().wait_stream(s)
        for _ in range(steps - 1):
            g.replay()
        return out


_ROPE_CACHE: Dict[tuple, tuple] = {}


def _rope_tables_cpu(theta: float, head_dim: int, max_len: int):
    """rope_tables rows 0..max_len-1 (a row depends on its position only, so a longer table computed once
    per (theta, head_dim) is sliced)."""
    key = (float(theta), int(head_dim))
    hit = _ROPE_CACHE.get(key)
    if hit is None or hit[0].shape[0] < max_len:
        hit = rope_tables(theta, head_dim, max(max_len, 4096))
        _ROPE_CACHE[key] = hit
    return hit[0][:max_len], hit[1][:max_len]


def random_float_state(cfg: BitNetConfig, seed: int) -> Dict[str, torch.Tensor]:
    """Float32 CPU weights of a random-init model under HuggingFace Llama names: normal(0, 0.02) for the
    embedding and every projection (and an untied LM head), ones for the RMSNorms (BitNetLlama._init_weights,
    packages/training/src/wrinklefree/models/llama.py:58-65), drawn from torch.Generator(seed) in a fixed
    order -- the same tensors on any host, for :meth:`BitNetDecoder.from_float_state` and for a
    HuggingFace model built from the same state."""
    gen = torch.Generator().manual_seed(seed)
    h, f = cfg.hidden_size, cfg.intermediate_size
    qd, kvd = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim

    def normal(*shape):
        return torch.randn(shape, generator=gen, dtype=torch.float32) * 0.02

    st = {"model.embed_tokens.weight": normal(cfg.vocab_size, h)}
    shapes = {"q": (qd, h), "k": (kvd, h), "v": (kvd, h), "o": (h, qd), "gate": (f, h), "up": (f, h), "down": (h, f)}
    for i in range(cfg.num_layers):
        pre = f"model.layers.{i}."
        for attr, name in BitNetDecoder._LINEARS:
            st[pre + name + ".weight"] = normal(*shapes[attr])
        st[pre + "input_layernorm.weight"] = torch.ones(h)
        st[pre + "post_attention_layernorm.weight"] = torch.ones(h)
    st["model.norm.weight"] = torch.ones(h)
    if not cfg.tie_embeddings:
        st["lm_head.weight"] = normal(cfg.vocab_size, h)
    return st


def quantised_linears(model: BitNetDecoder) -> Dict[str, PackedLinear]:
    """name -> PackedLinear for every ternary projection of the model."""
    out = {}
    for i, L in enumerate(model.layers):
        for n in ("q", "k", "v", "o", "gate", "up", "down"):
            out[f"layers.{i}.{n}"] = getattr(L, n)
    if model.lm_head is not None:
        out["lm_head"] = model.lm_head
    return out
