"""Write tests/golden/ref_bitlinear.npz from the reference's OWN float BitLinear module.

The module is packages/training/src/wrinklefree/models/bitlinear.py (BitLinear.weight_quant :46-64,
.activation_quant :66-84, .forward :86-113).  Its numerics (bf16 arithmetic for bf16 inputs, the
eps clamps, torch.round) are not pinned by any reference test or closed-form check, so this script
imports it in the build container, runs it on small seeded inputs and stores inputs + outputs only.
The fixture is data (no reference code); the tests read it on machines without the reference.

The module file is loaded by path, with the reference's ``wrinklefree`` package (torch-only imports)
on sys.path for its ``get_current_lambda`` import; no global lambda warmup is set, so lambda = 1
(full quantisation, the inference forward).

Run from the repository root:  python tests/golden/make_bitlinear_golden.py
"""

from __future__ import annotations

import importlib.util
import platform
import sys
from pathlib import Path

import numpy as np
import torch

REF_SRC = Path("/root/reference/packages/training/src")
OUT = Path(__file__).resolve().parent / "ref_bitlinear.npz"


def load_reference_bitlinear():
    sys.path.insert(0, str(REF_SRC))
    path = REF_SRC / "wrinklefree" / "models" / "bitlinear.py"
    spec = importlib.util.spec_from_file_location("wrinklefree_models_bitlinear", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.BitLinear


def hidden(g: torch.Generator, m: int, k: int) -> torch.Tensor:
    """N(0, 1) with 1% of entries at +-20 (the fused-quant input distribution of the benchmark)."""
    x = torch.randn(m, k, generator=g)
    sel = torch.rand(m, k, generator=g) < 0.01
    sign = torch.where(torch.rand(m, k, generator=g) < 0.5, -20.0, 20.0)
    return torch.where(sel, sign, x)


def main() -> None:
    BitLinear = load_reference_bitlinear()
    g = torch.Generator().manual_seed(20261202)
    data: dict[str, np.ndarray] = {}
    cases = []

    def record(name, x, weight, bias=None):
        k, n = weight.shape[1], weight.shape[0]
        mod = BitLinear(k, n, bias=bias is not None).to(x.dtype)
        with torch.no_grad():
            mod.weight.copy_(weight.to(x.dtype))
            if bias is not None:
                mod.bias.copy_(bias.to(x.dtype))
            w = mod.weight.to(x.dtype)
            wq = mod.weight_quant(w)
            xq = mod.activation_quant(x)
            y = mod(x)
        data[f"{name}_x"] = x.float().numpy()
        data[f"{name}_w"] = mod.weight.detach().float().numpy()
        data[f"{name}_bias"] = (mod.bias.detach().float().numpy() if bias is not None else np.zeros(0, np.float32))
        data[f"{name}_wq"] = wq.float().numpy()
        data[f"{name}_xq"] = xq.float().numpy()
        data[f"{name}_y"] = y.float().numpy()
        data[f"{name}_bf16"] = np.array(x.dtype == torch.bfloat16)
        cases.append(name)

    # fp32, K = 256, one all-zero token (eps clamp path)
    x = torch.randn(4, 256, generator=g)
    x[3] = 0.0
    record("f32", x, torch.randn(96, 256, generator=g) * 0.02)
    # fp32 with bias, K = 384
    record("f32_bias", torch.randn(3, 384, generator=g) * 3.0, torch.randn(64, 384, generator=g) * 0.05,
           bias=torch.randn(64, generator=g) * 0.1)
    # bf16 end to end (the module computes in the input dtype), outlier activations, K = 640
    record("bf16", hidden(g, 5, 640).to(torch.bfloat16), (torch.randn(80, 640, generator=g) * 0.02).to(torch.bfloat16))
    # exact ties: |w| in {0.5, 1.5} half each per tensor -> mean |w| = 1 exactly, so w * scale hits .5;
    # activations with absmax 127 -> scale 1, entries at k + 0.5
    mag = torch.where(torch.arange(32 * 128).reshape(32, 128) % 2 == 0, 0.5, 1.5)
    mag = mag[:, torch.randperm(128, generator=g)]
    sgn = torch.where(torch.rand(32, 128, generator=g) < 0.5, -1.0, 1.0)
    xt = torch.randint(-120, 121, (2, 128), generator=g).float() + 0.5
    xt[:, 0] = 127.0
    record("ties", xt, mag * sgn)

    data["cases"] = np.array(cases)
    data["versions"] = np.array([f"torch {torch.__version__}", f"python {platform.python_version()}",
                                 f"numpy {np.__version__}"])
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {', '.join(cases)}")


if __name__ == "__main__":
    main()
