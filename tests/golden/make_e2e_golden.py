"""Write tests/golden/ref_e2e_smollm2.npz: greedy decoding of the reference's OWN stage-1 BitNet model.

configs[0]'s model as the reference builds it: transformers' LlamaForCausalLM at the SmolLM2-135M shape
(30 layers, hidden 576, 9/3 heads, head_dim 64, FFN 1536 SiLU, vocab 49152, tied embeddings, rope theta
100000, rms eps 1e-5; packages/training/configs/model/smollm2_135m.yaml), converted by the reference's
``convert_model_to_bitnet`` (packages/training/src/wrinklefree/training/stage1.py:169-214: BitLinear for
q/k/v/gate/up, SubLN + BitLinear for o/down), run in float32 with the reference BitLinear's own forward
(packages/training/src/wrinklefree/models/bitlinear.py:86-113, lambda = 1).  Those HF-model numerics are
not pinned by any reference test or closed form, so this script imports the reference in the build
container and stores inputs and outputs only (no reference code).

Weights: ``random_float_state(SMOLLM2_135M, SEED)`` of this package (normal(0, 0.02), ones for the
norms, a seeded CPU generator), so the GPU test rebuilds the same floats without the fixture holding
135M of them.  Prompt: 32 seeded random ids.  Greedy: 128 new tokens, each from a full forward of the
sequence so far (no KV cache), eager attention.  Recorded: the prompt, the 128 token ids, the top-5
logits (ids and values) of every step, the full last-position logits of the prompt forward, and the
library versions.

The model's own sensitivity to rounding-level noise, recorded beside it: the same model with its input
embeddings multiplied by (1 + 1e-7 * N(0, 1)) (a fixed seeded draw per position) -- its prompt logits,
its logits at the unperturbed run's top-5 ids when fed the unperturbed tokens (teacher forcing), and
its own free-running greedy tokens.  An int8 activation code sits next to a rounding boundary often
enough that such noise flips a few codes per layer and the flips compound over 30 layers; the GPU test
reads its tolerances from this spread.  Also the residual stream entering and leaving layers
0, 1, 10, 15, 20 and 29 in the prompt forward, so single layers can be compared without compounding.

Run from the repository root:  python tests/golden/make_e2e_golden.py
"""

from __future__ import annotations

import importlib.util
import platform
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
REF_SRC = Path("/root/reference/packages/training/src")
OUT = Path(__file__).resolve().parent / "ref_e2e_smollm2.npz"
SEED, PROMPT_SEED, PROMPT_LEN, NEW = 2026, 7, 32, 128


def load_stage1():
    sys.path.insert(0, str(REF_SRC))
    path = REF_SRC / "wrinklefree" / "training" / "stage1.py"
    spec = importlib.util.spec_from_file_location("wrinklefree_training_stage1", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def build_reference_model():
    """The reference's stage-1 BitNet model at the SmolLM2-135M shape from random_float_state(cfg, SEED):
    returns (model, cfg, model.py module)."""
    import transformers

    sys.path.insert(0, str(ROOT))
    import __graft_entry__

    M = __graft_entry__.load_package().model  # model.py's CPU-only helpers (no GPU work here)
    cfg = M.SMOLLM2_135M
    stage1 = load_stage1()
    hf_cfg = transformers.LlamaConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_layers, num_attention_heads=cfg.num_heads, num_key_value_heads=cfg.num_kv_heads,
        head_dim=cfg.head_dim, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_eps, tie_word_embeddings=True,
        hidden_act="silu", max_position_embeddings=2048, attention_bias=False, mlp_bias=False)
    hf_cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = transformers.LlamaForCausalLM(hf_cfg).to(torch.float32).eval()
    state = M.random_float_state(cfg, SEED)
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}, (missing, unexpected)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()  # tied
    model = stage1.convert_model_to_bitnet(model, cfg.hidden_size, cfg.intermediate_size)
    n_bitlinear = sum(type(m).__name__ == "BitLinear" for m in model.modules())
    assert n_bitlinear == 7 * cfg.num_layers, n_bitlinear
    return model, cfg, M


def main() -> None:
    import transformers

    model, cfg, M = build_reference_model()

    prompt = torch.randint(0, cfg.vocab_size, (1, PROMPT_LEN), generator=torch.Generator().manual_seed(PROMPT_SEED))
    noise = 1e-7 * torch.randn((1, PROMPT_LEN + NEW, cfg.hidden_size), generator=torch.Generator().manual_seed(11))
    embed = model.model.embed_tokens

    def last_logits(ids, perturbed=False):
        if not perturbed:
            return model(ids, use_cache=False).logits[0, -1].float()
        e = embed(ids)
        return model(inputs_embeds=e * (1 + noise[:, :ids.shape[1]]), use_cache=False).logits[0, -1].float()

    layers = (0, 1, 10, 15, 20, 29)
    io = {}

    def keep(name, t):  # hooks must return None (a value would replace the layer's inputs or output)
        io.setdefault(name, t[0].detach().numpy().copy())

    hooks = []
    for li in layers:
        layer = model.model.layers[li]
        hooks.append(layer.register_forward_pre_hook(lambda mod, args, li=li: keep(f"layer{li}_in", args[0])))
        hooks.append(layer.register_forward_hook(
            lambda mod, args, out, li=li: keep(f"layer{li}_out", out[0] if isinstance(out, tuple) else out)))

    ids = prompt.clone()
    tokens, top_ids, top_vals = [], [], []
    with torch.no_grad():
        for step in range(NEW):
            logits = last_logits(ids)
            if step == 0:
                prefill_logits = logits.numpy().copy()
                for h in hooks:
                    h.remove()
            v, i = torch.topk(logits, 5)
            top_ids.append(i.numpy())
            top_vals.append(v.numpy())
            nxt = int(torch.argmax(logits))
            tokens.append(nxt)
            ids = torch.cat([ids, torch.tensor([[nxt]])], dim=1)
            if step % 16 == 0:
                print(f"step {step}: token {nxt}, top-2 gap {float(v[0] - v[1]):.3e}", flush=True)
        # the perturbed model, teacher-forced on the tokens above, then free-running
        ids = prompt.clone()
        pert_top = []
        for step in range(NEW):
            logits = last_logits(ids, perturbed=True)
            if step == 0:
                pert_prefill = logits.numpy().copy()
            pert_top.append(logits.numpy()[top_ids[step]])
            ids = torch.cat([ids, torch.tensor([[tokens[step]]])], dim=1)
        ids = prompt.clone()
        pert_tokens = []
        for step in range(NEW):
            nxt = int(torch.argmax(last_logits(ids, perturbed=True)))
            pert_tokens.append(nxt)
            ids = torch.cat([ids, torch.tensor([[nxt]])], dim=1)
    pert_top = np.stack(pert_top)
    same = np.array(pert_tokens) == np.array(tokens)
    print(f"perturbed: prompt logits moved {np.abs(pert_prefill - prefill_logits).max():.3e}, teacher-forced top-5 "
          f"{np.abs(pert_top - np.stack(top_vals)).max():.3e}; free-running tokens equal for the first "
          f"{int(np.argmin(same)) if not same.all() else NEW} steps", flush=True)

    np.savez_compressed(
        OUT,
        seed=np.array([SEED]), prompt=prompt.numpy()[0].astype(np.int64), tokens=np.array(tokens, np.int64),
        top5_ids=np.stack(top_ids).astype(np.int64), top5_logits=np.stack(top_vals).astype(np.float32),
        prefill_logits=prefill_logits.astype(np.float32),
        perturbed_prefill_logits=pert_prefill.astype(np.float32), perturbed_top5_logits=pert_top.astype(np.float32),
        perturbed_tokens=np.array(pert_tokens, np.int64), layers=np.array(layers, np.int64),
        **{k: v.astype(np.float32) for k, v in io.items()},
        versions=np.array([f"torch {torch.__version__}", f"transformers {transformers.__version__}",
                           f"numpy {np.__version__}", f"python {platform.python_version()}"]),
    )
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes); {len(set(tokens))} distinct tokens")


if __name__ == "__main__":
    main()
