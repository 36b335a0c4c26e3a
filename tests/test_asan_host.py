"""Host-side AddressSanitizer run of the C ABI (a sanitizer pass over the host code; the reference builds
-O3 -DNDEBUG with none, SGB/sgl-kernel/csrc/bitnet/CMakeLists.txt:45).

tests/asan/abi_driver.cpp, linked against the library whose host-only sources (entry-point validation
and dispatch, the native engine) are compiled with ASan (wrinklefree-monorepo_amd/_build.py build_asan,
run by __graft_entry__.build()), drives every argument check of the op entry points, the rotary tables,
the NULL-engine contract, the sampler, and the engine's SGLBITNT loader on the model files written here:
the files themselves, every truncation inside their headers, samples inside their data, every 4- and
8-byte header field set to extreme values, seeded bit flips and hostile config texts.  No GPU is used
(without one a well-formed file fails at the first HIP call).  The run must finish with every
expectation met and no sanitizer report."""

import os
import subprocess
from pathlib import Path

import pytest
import torch

import test_engine_abi as eng

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "wrinklefree-monorepo_amd" / "_build" / "asan" / "abi_driver"


@pytest.mark.skipif(not DRIVER.exists(), reason="ASan driver not built (run __graft_entry__.build())")
def test_c_abi_and_engine_loader_under_asan(pkg, tmp_path):
    files = []
    cfg = eng._cfg(eos_token_id=[3, 5], hidden_act="relu2")
    p = tmp_path / "tied.bin"
    pkg.write_sglbitnt(p, cfg, eng._tensors(cfg))
    files.append(p)
    t = eng._tensors(eng._cfg())
    t["lm_head.weight"] = (torch.full((64, 32), 0x55, dtype=torch.uint8), 0.25)  # ternary head
    t["model.layers.0.self_attn.attn_sub_norm.weight"] = (torch.ones(128, dtype=torch.bfloat16), None)
    t["model.layers.0.mlp.ffn_sub_norm.weight"] = (torch.ones(256, dtype=torch.float16), None)
    p = tmp_path / "ternary_head.bin"
    pkg.write_sglbitnt(p, eng._cfg(), t)
    files.append(p)
    t = eng._tensors(eng._cfg())
    t["lm_head.weight"] = (torch.zeros(64, 128), None)  # dense head
    p = tmp_path / "dense_head.bin"
    pkg.write_sglbitnt(p, eng._cfg(), t)
    files.append(p)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1")
    res = subprocess.run([str(DRIVER), *map(str, files)], capture_output=True, text=True, env=env, timeout=600)
    out = res.stdout + res.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert res.returncode == 0, out[-4000:]
    assert ", 0 failures" in res.stdout and "engine creates" in res.stdout
