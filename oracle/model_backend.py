"""BitLinear backend of the end-to-end model on the numpy oracle -- TEST INFRASTRUCTURE ONLY.

Used by tests/ (token and accumulator parity of the HIP backend) and by bench.py's CPU baseline leg
(the same model decoded on the host).  Each call restates one quantised group of the model on the
CPU: RMSNorm/SubLN + per-token int8 (bitnet_oracle.rmsnorm_quant / glu_rmsnorm_quant), exact int32
accumulators of the ternary linear (an fp32 GEMM of the unpacked weights, exact while partial sums
stay below 2^24), and the rescale (bitnet_oracle.rescale).  Greedy picks use the first maximum
(ENG = bitnet_engine.cpp:774-779, std::max_element).
"""

from __future__ import annotations

import numpy as np
import torch

from . import bitnet_oracle as orc


class OracleBackend:
    """Quantised BitLinear groups computed by the numpy oracle on the host; outputs go to ``dev``."""

    def __init__(self, linears, dev):
        self.dev = torch.device(dev)
        self.acc_log = []
        self.w = {}
        for lin in linears:
            packed = lin.qweight.cpu().numpy()
            self.w[id(lin)] = (orc.unpack_i2s(packed).astype(np.float32), np.float32(lin.scale.item()))

    def _apply(self, q, s, linears):
        outs = []
        for lin in linears:
            w, ws = self.w[id(lin)]
            acc = (q.astype(np.float32) @ w.T).astype(np.int64)  # exact: |partial sums| < 2^24
            self.acc_log.append(acc)
            outs.append(torch.from_numpy(orc.rescale(acc, ws, s)).to(self.dev))
        return outs

    def norm_linears(self, x, norm_weight, eps, linears):
        g = None if norm_weight is None else norm_weight.float().cpu().numpy()
        q, s = orc.rmsnorm_quant(x.float().cpu().numpy(), g, eps, k_pad=linears[0].k_pad)
        return self._apply(q, s, linears)

    def norm_linear_argmax(self, x, norm_weight, eps, linear):
        (logits,) = self.norm_linears(x, norm_weight, eps, [linear])
        return torch.argmax(logits, dim=-1)  # first maximum

    def _residual(self, y, residual):
        # the fused epilogue: fp32 add of the rescaled output and the residual, then the residual's dtype
        r = residual.float().cpu().numpy()
        return torch.from_numpy((y.float().cpu().numpy() + r).astype(np.float32)).to(self.dev).to(residual.dtype)

    def norm_linear_residual(self, x, norm_weight, eps, linear, residual):
        (y,) = self.norm_linears(x, norm_weight, eps, [linear])
        return self._residual(y, residual)

    def glu_norm_linear_residual(self, gate, up, act, norm_weight, eps, linear, residual):
        (y,) = self.glu_norm_linears(gate, up, act, norm_weight, eps, [linear])
        return self._residual(y, residual)

    def glu_norm_linears(self, gate, up, act, norm_weight, eps, linears):
        g = None if norm_weight is None else norm_weight.float().cpu().numpy()
        code = orc.ACT_SILU if act == "silu" else orc.ACT_RELU2
        q, s = orc.glu_rmsnorm_quant(gate.float().cpu().numpy(), up.float().cpu().numpy(), code, g, eps,
                                     k_pad=linears[0].k_pad)
        return self._apply(q, s, linears)


def cpu_decoder(model, max_len: int):
    """The model's weights as oracle/c/cpu_decode.c's host decoder (refbind.CpuDecoder): the end-to-end
    CPU baseline.  Packed linears keep their I2_S bytes and scales; the embedding, norms and the fp32
    LM head (dense or tied; a ternary head is not supported here) are copied to host fp32."""
    from . import refbind

    cfg = model.cfg
    if model.lm_head is not None:
        raise ValueError("cpu_decoder: ternary LM heads are not supported")

    def host(t):
        return t.detach().float().cpu().numpy()

    def stack(attr):
        return np.stack([getattr(L, attr).qweight.cpu().numpy() for L in model.layers])

    L0 = model.layers[0]
    dims = dict(layers=cfg.num_layers, hidden=cfg.hidden_size, inter=cfg.intermediate_size, heads=cfg.num_heads,
                kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, vocab=cfg.vocab_size, max_len=max_len,
                kpad_h=L0.q.k_pad, kpad_qd=L0.o.k_pad, kpad_f=L0.down.k_pad,
                act=2 if cfg.hidden_act == "relu2" else 1, rms_eps=cfg.rms_eps, subln_eps=cfg.subln_eps)
    import sys

    cos, sin = sys.modules[type(model).__module__]._rope_tables_cpu(cfg.rope_theta, cfg.head_dim, max_len)
    arrays = dict(
        embed=host(model.embed), head=host(model.head_weight), final_norm=host(model.final_norm),
        in_norm=np.stack([host(L.input_norm) for L in model.layers]),
        post_norm=np.stack([host(L.post_attn_norm) for L in model.layers]),
        attn_sub=np.stack([host(L.attn_sub_norm) for L in model.layers]),
        ffn_sub=np.stack([host(L.ffn_sub_norm) for L in model.layers]),
        scales=np.stack([[float(getattr(L, n).scale.item()) for n in ("q", "k", "v", "o", "gate", "up", "down")]
                         for L in model.layers]).astype(np.float32),
        wq=stack("q"), wk=stack("k"), wv=stack("v"), wo=stack("o"), wg=stack("gate"), wu=stack("up"),
        wd=stack("down"), rope_cos=cos.numpy(), rope_sin=sin.numpy())
    return refbind.CpuDecoder(dims, arrays)
