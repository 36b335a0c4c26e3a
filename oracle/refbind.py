"""ctypes access to the compiled CPU checkers -- TEST INFRASTRUCTURE ONLY.

* ``oracle/c/liboracle_c.so``: our C restatements -- the scalar checker (oracle/c/i2s_oracle.c) and
  the AVX2 port of the reference CPU GEMV op (oracle/c/i2s_cpu_avx2.c), which bench.py times as
  its CPU baseline.
* ``oracle/_ref/libref_bitnet_avx2.so``: the reference's own bitnet_gemv.cpp compiled by
  oracle/Makefile (AVX2 path); ``libref_bitnet_avx512.so`` adds the reference CMake's AVX-512
  flags.  Both exist only where the reference tree was present at build time; callers skip
  when they are missing.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_C = HERE / "c" / "liboracle_c.so"
REF_AVX2 = HERE / "_ref" / "libref_bitnet_avx2.so"
REF_AVX512 = HERE / "_ref" / "libref_bitnet_avx512.so"

_vp = ctypes.c_void_p
_int = ctypes.c_int


def build(with_ref: bool = True) -> None:
    """make -C oracle (and the reference build when its source tree is present)."""
    targets = ["all"]
    ref_src = Path("/root/reference/packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/bitnet/bitnet_gemv.cpp")
    if with_ref and ref_src.exists():
        targets.append("ref")
    res = subprocess.run(["make", "-s", "-C", str(HERE), *targets], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


class OracleC:
    def __init__(self, path: Path = ORACLE_C):
        self.lib = ctypes.CDLL(str(path))
        self.lib.orc_vec_dot_i2_i8.restype = ctypes.c_int32
        self.lib.orc_vec_dot_i2_i8.argtypes = [_int, _vp, _vp]
        self.lib.orc_gemm_i2_i8.restype = _int
        self.lib.orc_gemm_i2_i8.argtypes = [_int, _int, _int, _vp, _vp, _vp, ctypes.c_float]
        self.lib.orc_acc_i2_i8.restype = _int
        self.lib.orc_acc_i2_i8.argtypes = [_int, _int, _int, _vp, _vp, _vp]
        self.lib.orc_quantize_i8.restype = None
        self.lib.orc_quantize_i8.argtypes = [_int, _vp, _vp, _vp]
        self.lib.cpu_gemv_i2s_avx2.restype = _int
        self.lib.cpu_gemv_i2s_avx2.argtypes = [_int, _int, _vp, _vp, _vp, ctypes.c_float]
        self.lib.cpu_gemm_i2s_avx2.restype = _int
        self.lib.cpu_gemm_i2s_avx2.argtypes = [_int, _int, _int, _vp, _vp, _vp, ctypes.c_float]

    def gemv_avx2(self, packed: np.ndarray, a: np.ndarray, scale: float, out: np.ndarray | None = None) -> np.ndarray:
        """AVX2 port of the reference bitnet_gemv_cpu op: fp32 [N] = acc * scale."""
        packed = np.ascontiguousarray(packed, np.uint8)
        a = np.ascontiguousarray(a, np.int8).ravel()
        n, k = packed.shape[0], packed.shape[1] * 4
        if a.size != k:
            raise ValueError("activations must hold packed_weights.shape[1] * 4 values")
        if out is None:
            out = np.empty(n, np.float32)
        if self.lib.cpu_gemv_i2s_avx2(n, k, _ptr(out), _ptr(packed), _ptr(a), float(scale)) != 0:
            raise ValueError("K must be a multiple of 128")
        return out

    def gemm_avx2(self, packed: np.ndarray, a: np.ndarray, scale: float) -> np.ndarray:
        """AVX2 port of the reference bitnet_gemm_cpu op: fp32 in its [out, batch] layout (batch <= 64)."""
        packed = np.ascontiguousarray(packed, np.uint8)
        a2 = np.ascontiguousarray(np.atleast_2d(a), np.int8)
        n, k = packed.shape[0], packed.shape[1] * 4
        if a2.shape[1] != k:
            raise ValueError("activations must hold packed_weights.shape[1] * 4 columns")
        out = np.empty((n, a2.shape[0]), np.float32)
        if self.lib.cpu_gemm_i2s_avx2(n, a2.shape[0], k, _ptr(out), _ptr(packed), _ptr(a2), float(scale)) != 0:
            raise ValueError("K must be a multiple of 128 and the batch at most 64")
        return out

    def acc(self, packed: np.ndarray, a: np.ndarray) -> np.ndarray:
        packed = np.ascontiguousarray(packed, np.uint8)
        a2 = np.ascontiguousarray(np.atleast_2d(a), np.int8)
        n, k = packed.shape[0], packed.shape[1] * 4
        out = np.empty((a2.shape[0], n), np.int32)
        if self.lib.orc_acc_i2_i8(n, a2.shape[0], k, _ptr(out), _ptr(packed), _ptr(a2)) != 0:
            raise ValueError("K must be a multiple of 128")
        return out

    def gemm(self, packed: np.ndarray, a: np.ndarray, scale: float) -> np.ndarray:
        """[out, batch] fp32, the reference layout."""
        packed = np.ascontiguousarray(packed, np.uint8)
        a2 = np.ascontiguousarray(np.atleast_2d(a), np.int8)
        n, k = packed.shape[0], packed.shape[1] * 4
        out = np.empty((n, a2.shape[0]), np.float32)
        if self.lib.orc_gemm_i2_i8(n, a2.shape[0], k, _ptr(out), _ptr(packed), _ptr(a2), float(scale)) != 0:
            raise ValueError("K must be a multiple of 128")
        return out

    def quantize(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.empty(x.size, np.int8)
        s = np.empty(1, np.float32)
        self.lib.orc_quantize_i8(x.size, _ptr(q), _ptr(x), _ptr(s))
        return q, s[0]


class CpuModel(ctypes.Structure):
    """oracle/c/cpu_decode.c's cpu_model."""
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "hidden", "inter", "heads", "kv_heads", "head_dim", "vocab",
                                               "max_len", "kpad_h", "kpad_qd", "kpad_f", "act")] + \
               [("rms_eps", ctypes.c_float), ("subln_eps", ctypes.c_float)] + \
               [(n, _vp) for n in ("embed", "head", "final_norm", "in_norm", "post_norm", "attn_sub", "ffn_sub",
                                   "scales", "wq", "wk", "wv", "wo", "wg", "wu", "wd", "rope_cos", "rope_sin")]


class CpuDecoder:
    """Greedy decoding of a BitNet Llama model on the host (oracle/c/cpu_decode.c): the end-to-end CPU
    baseline.  ``arrays``: numpy arrays named as cpu_model's pointer fields (contiguous, fp32 / uint8);
    ``dims``: its integer and float fields."""

    def __init__(self, dims: dict, arrays: dict, path: Path = ORACLE_C):
        self.lib = ctypes.CDLL(str(path))
        self.lib.cpu_decode_greedy.restype = _int
        self.lib.cpu_decode_greedy.argtypes = [ctypes.POINTER(CpuModel), _vp, _int, _int, _vp, _vp]
        self._keep = {}
        m = CpuModel()
        for k, v in dims.items():
            setattr(m, k, v)
        for k, v in arrays.items():
            want = np.uint8 if k.startswith("w") else np.float32
            a = np.ascontiguousarray(v, want)
            self._keep[k] = a
            setattr(m, k, a.ctypes.data)
        self.m = m

    def greedy(self, prompt, n_new: int):
        """(n_new generated token ids, logits [vocab] after the prompt)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        logits = np.zeros(self.m.vocab, np.float32)
        if self.lib.cpu_decode_greedy(ctypes.byref(self.m), _ptr(p), p.size, n_new, _ptr(out), _ptr(logits)) != 0:
            raise ValueError("cpu_decode_greedy: bad sizes or out of memory")
        return out[:n_new], logits


class RefLib:
    """The reference's compiled kernels (bitnet_gemv.cpp) behind oracle/c/ref_shim.cpp."""

    def __init__(self, path: Path = REF_AVX2):
        self.path = path
        self.lib = ctypes.CDLL(str(path))
        L = self.lib
        L.ref_vec_dot_i2_i8.restype = _int
        L.ref_vec_dot_i2_i8.argtypes = [_int, _vp, _vp, _vp]
        L.ref_gemm_i2_i8.restype = _int
        L.ref_gemm_i2_i8.argtypes = [_int, _int, _int, _vp, _vp, _vp, ctypes.c_float]
        L.ref_gemv_op.restype = _int
        L.ref_gemv_op.argtypes = [_int, _int, _vp, _vp, _vp, ctypes.c_float]
        L.ref_quantize_activations_i8.restype = None
        L.ref_quantize_activations_i8.argtypes = [_int, _vp, _vp, _vp]

    @staticmethod
    def exists(path: Path = REF_AVX2) -> bool:
        return path.exists()

    def vec_dot(self, packed_row: np.ndarray, a: np.ndarray) -> float:
        packed_row = np.ascontiguousarray(packed_row, np.uint8)
        a = np.ascontiguousarray(a, np.int8)
        r = np.zeros(1, np.float32)
        if self.lib.ref_vec_dot_i2_i8(a.size, _ptr(r), _ptr(packed_row), _ptr(a)) != 0:
            raise ValueError("reference bitnet_vec_dot_i2_i8 rejected the input")
        return float(r[0])

    def gemm(self, packed: np.ndarray, a: np.ndarray, scale: float) -> np.ndarray:
        """Reference bitnet_gemm_i2_i8 output in its own [out, batch] layout."""
        packed = np.ascontiguousarray(packed, np.uint8)
        a2 = np.ascontiguousarray(np.atleast_2d(a), np.int8)
        n, k = packed.shape[0], packed.shape[1] * 4
        out = np.zeros((n, a2.shape[0]), np.float32)
        if self.lib.ref_gemm_i2_i8(n, a2.shape[0], k, _ptr(out), _ptr(packed), _ptr(a2), float(scale)) != 0:
            raise ValueError("reference bitnet_gemm_i2_i8 rejected the input")
        return out

    def gemv(self, packed: np.ndarray, a: np.ndarray, scale: float, out: np.ndarray | None = None) -> np.ndarray:
        packed = np.ascontiguousarray(packed, np.uint8)
        a = np.ascontiguousarray(a, np.int8).ravel()
        n, k = packed.shape[0], packed.shape[1] * 4
        if out is None:
            out = np.zeros(n, np.float32)
        if self.lib.ref_gemv_op(n, k, _ptr(out), _ptr(packed), _ptr(a), float(scale)) != 0:
            raise ValueError("reference bitnet_gemv rejected the input")
        return out

    def quantize(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        s = np.zeros(1, np.float32)
        self.lib.ref_quantize_activations_i8(x.size, _ptr(q), _ptr(x), _ptr(s))
        return q, s[0]
