"""The MFMA-rate diagnostic runs and writes its sink (its timing is reported by bench.py)."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("random_operands", [0, 1])
def test_diag_mfma_runs(pkg, dev, random_operands):
    sink = torch.full((4 * 256,), -12345, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pkg._lib.call("wfb_diag_mfma_i8", random_operands, 4, 3, ctypes.c_void_p(sink.data_ptr()), stream)
    torch.cuda.synchronize()
    s = sink.cpu()
    if random_operands == 0:
        # constant operands: every lane of every wave ends with the same sum
        assert bool((s == s[0]).all()) and int(s[0]) != -12345
    else:
        assert int((s != -12345).sum()) == s.numel()
