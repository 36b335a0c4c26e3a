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
