"""Write tests/golden/ref_codes_smollm2.npz: the reference model's own int8 activation codes, layer by layer.

The model is the one of make_e2e_golden.py (the reference's stage-1 conversion of transformers'
LlamaForCausalLM at the SmolLM2-135M shape, float weights random_float_state(SEED), fp32, eager attention),
run once over the same 32-token prompt.  For layers 0, 15 and 29, forward hooks record, for the last 16
prompt positions, what each BitLinear group of the layer sees (packages/training/src/wrinklefree/training/
stage1.py:63-214):

  group  norm before it (eps)                          BitLinears          output kept
  qkv    input_layernorm, transformers RMSNorm (1e-5)   q_proj k_proj v_proj   q_proj
  o      SubLN (1e-6; models/subln.py:42-59)            o_proj                 o_proj
  gu     post_attention_layernorm (1e-5)                gate_proj up_proj      gate_proj
  down   SubLN (1e-6)                                   down_proj              down_proj

  pre_<g>    fp32 [16, K]  the norm's input rows
  lin_<g>    fp32 [16, K]  the BitLinear's input rows (the norm's output)
  codes_<g>  int8 [16, K]  the reference's int8 codes of lin_<g>: BitLinear.activation_quant
             (models/bitlinear.py:66-84) returns codes / s with s = 127 / max|x| per token; the script calls it
             and recovers the integer codes as round(returned * s) (exact: |code| <= 127)
  y_<g>      fp32 [16, N]  the output of the kept BitLinear, F.linear(x_quant, w_quant) (bitlinear.py:86-113)
  wmean_<g>  fp32 []       that BitLinear's weight absmean clamp(mean|W|, eps), from which its weight_quant
             takes scale = 1 / wmean (bitlinear.py:46-64)

Only inputs and outputs are stored (no reference code).  The GPU test rebuilds the float weights from
random_float_state(SEED) and checks the quantiser, the fused norm + quantiser and the int32 accumulators
against these rows.  Run from the repository root (this container only):  python tests/golden/make_codes_golden.py
"""

from __future__ import annotations

import platform
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
import make_e2e_golden as e2e  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_codes_smollm2.npz"
LAYERS = (0, 15, 29)
KEEP = slice(16, 32)  # prompt positions recorded


def main() -> None:
    import transformers

    model, cfg, M = e2e.build_reference_model()
    prompt = torch.randint(0, cfg.vocab_size, (1, e2e.PROMPT_LEN),
                           generator=torch.Generator().manual_seed(e2e.PROMPT_SEED))
    rec = {}
    hooks = []

    def pre_hook(key):
        def f(mod, args):
            rec.setdefault(key, args[0][0, KEEP].detach().clone())
        return f

    def lin_hook(key):
        def f(mod, args):
            x = args[0][0, KEEP].detach()
            if key not in rec:
                rec[key] = x.clone()
                xq = mod.activation_quant(x)  # the reference's own quantiser: codes / s
                s = 127.0 / x.abs().max(dim=-1, keepdim=True).values.clamp(min=mod.eps)
                codes = torch.round(xq * s)
                assert float((codes - xq * s).abs().max()) < 1e-3 and float(codes.abs().max()) <= 128
                rec["codes" + key[3:]] = codes.to(torch.int8)
                rec["wmean" + key[3:]] = mod.weight.abs().mean().clamp(min=mod.eps).detach().clone()
        return f

    def out_hook(key):
        def f(mod, args, out):
            rec.setdefault(key, out[0, KEEP].detach().clone())
        return f

    for li in LAYERS:
        L = model.model.layers[li]
        att, mlp = L.self_attn, L.mlp
        groups = {
            "qkv": (L.input_layernorm, att.q_proj),
            "o": (att.o_proj[0], att.o_proj[1]),
            "gu": (L.post_attention_layernorm, mlp.gate_proj),
            "down": (mlp.down_proj[0], mlp.down_proj[1]),
        }
        for g, (norm, lin) in groups.items():
            assert type(lin).__name__ == "BitLinear", (g, type(lin))
            hooks.append(norm.register_forward_pre_hook(pre_hook(f"pre_{g}_{li}")))
            hooks.append(lin.register_forward_pre_hook(lin_hook(f"lin_{g}_{li}")))
            hooks.append(lin.register_forward_hook(out_hook(f"y_{g}_{li}")))
        assert abs(L.input_layernorm.variance_epsilon - cfg.rms_eps) < 1e-12
        assert abs(att.o_proj[0].eps - cfg.subln_eps) < 1e-12 and abs(mlp.down_proj[0].eps - cfg.subln_eps) < 1e-12
    with torch.no_grad():
        model(prompt, use_cache=False)
    for h in hooks:
        h.remove()
    arrays = {}
    for k, v in rec.items():
        arrays[k] = v.numpy().astype(np.int8 if k.startswith("codes") else np.float32)
    np.savez_compressed(
        OUT, seed=np.array([e2e.SEED]), prompt=prompt.numpy()[0].astype(np.int64), layers=np.array(LAYERS, np.int64),
        positions=np.arange(32)[KEEP].astype(np.int64), **arrays,
        versions=np.array([f"torch {torch.__version__}", f"transformers {transformers.__version__}",
                           f"numpy {np.__version__}", f"python {platform.python_version()}"]),
    )
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {sorted(arrays)[:6]} ...")


if __name__ == "__main__":
    main()
