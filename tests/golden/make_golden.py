"""Write tests/golden/ref_kernels.npz from the reference's OWN compiled CPU kernels.

The reference source packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp
is compiled in place by oracle/Makefile (target ``ref``) into oracle/_ref/libref_bitnet_avx2.so;
this script calls it on small seeded inputs and stores inputs + outputs.  The fixture is data only
(no reference code), so the oracle can be checked against it on machines without the reference.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import bitnet_oracle as orc  # noqa: E402
from oracle import refbind  # noqa: E402

OUT = Path(__file__).resolve().parent / "ref_kernels.npz"


def main() -> None:
    refbind.build(with_ref=True)
    ref = refbind.RefLib(refbind.REF_AVX2)
    rng = np.random.default_rng(20261201)
    data: dict[str, np.ndarray] = {}

    # bitnet_vec_dot_i2_i8 on single rows (bias-corrected int result returned as float)
    for k in (128, 256, 640, 2560, 6912):
        packed = orc.pack_i2s(orc.random_ternary(rng, 3, k))
        a = orc.random_int8(rng, 1, k)[0]
        # include the extreme activation -128 in a few places
        a[rng.integers(0, k, 4)] = -128
        res = np.array([ref.vec_dot(packed[r], a) for r in range(3)], np.float32)
        data[f"dot_k{k}_packed"] = packed
        data[f"dot_k{k}_act"] = a
        data[f"dot_k{k}_out"] = res

    # bitnet_gemm_i2_i8: [out, batch] layout, scale applied
    packed = orc.pack_i2s(orc.random_ternary(rng, 37, 384))
    a = orc.random_int8(rng, 5, 384)
    data["gemm_packed"] = packed
    data["gemm_act"] = a
    data["gemm_scale"] = np.array([0.0371], np.float32)
    data["gemm_out"] = ref.gemm(packed, a, 0.0371)

    # quantize_activations_i8 (one scale per call): random, ties, zeros, tiny
    cases = {
        "rand": rng.standard_normal(512).astype(np.float32) * 3,
        "ties": np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5] * 4, np.float32),
        "zero": np.zeros(64, np.float32),
        "tiny": np.full(32, 5e-7, np.float32),
        "outl": orc.outlier_hidden(rng, 1, 640)[0],
    }
    for name, x in cases.items():
        q, s = ref.quantize(x)
        data[f"quant_{name}_in"] = x
        data[f"quant_{name}_q"] = q
        data[f"quant_{name}_scale"] = np.array([s], np.float32)

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
