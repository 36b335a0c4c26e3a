"""ctypes binding of the native engine ABI (include/wfbitnet_engine.h) in libwfbitnet.so.

The same entry points, structs and error behaviour as the reference's native engine
(packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/inference/bitnet_engine.h:14-161), which its Rust
gateway binds (sgl-model-gateway/src/inference/bitnet_ffi.rs:55-100); :class:`NativeEngine` is the
Python counterpart of that gateway's NativeEngine wrapper.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

from . import _lib


class BitNetConfig(ctypes.Structure):
    _fields_ = [("max_seq_len", ctypes.c_int32), ("num_threads", ctypes.c_int32), ("kv_cache_size", ctypes.c_int32)]


class SamplingParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("repetition_penalty", ctypes.c_float), ("max_tokens", ctypes.c_int32)]


class GenerationResult(ctypes.Structure):
    _fields_ = [("output_ids", ctypes.POINTER(ctypes.c_int32)), ("num_tokens", ctypes.c_int32),
                ("logits", ctypes.POINTER(ctypes.c_float)), ("logits_size", ctypes.c_int32)]


_vp = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
# name -> (restype, argtypes)
SIGNATURES = {
    "bitnet_engine_create": (_vp, [ctypes.c_char_p, ctypes.POINTER(BitNetConfig)]),
    "bitnet_engine_destroy": (None, [_vp]),
    "bitnet_get_error": (ctypes.c_char_p, []),
    "bitnet_generate": (ctypes.c_int, [_vp, _i32p, ctypes.c_int32, ctypes.POINTER(SamplingParams),
                                       ctypes.POINTER(GenerationResult)]),
    "bitnet_prefill": (ctypes.c_int, [_vp, _i32p, ctypes.c_int32]),
    "bitnet_decode_step": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.POINTER(SamplingParams), _i32p]),
    "bitnet_reset_cache": (None, [_vp]),
    "bitnet_vocab_size": (ctypes.c_int32, [_vp]),
    "bitnet_hidden_size": (ctypes.c_int32, [_vp]),
    "bitnet_num_layers": (ctypes.c_int32, [_vp]),
    "bitnet_max_seq_len": (ctypes.c_int32, [_vp]),
    "bitnet_get_num_kv_heads": (ctypes.c_int, [_vp]),
    "bitnet_free_result": (None, [ctypes.POINTER(GenerationResult)]),
    "wfb_engine_sample_top_p": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_float, ctypes.c_float, ctypes.c_uint32,
                                               ctypes.c_int32, _i32p]),
    "wfb_engine_fail_alloc_after": (ctypes.c_int, [ctypes.c_int64]),
}

_bound = None


def lib() -> ctypes.CDLL:
    """libwfbitnet with the engine signatures set (raises if the library is not built)."""
    global _bound
    if _bound is None:
        L = _lib.load()
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _bound = L
    return _bound


def last_error() -> str:
    msg = lib().bitnet_get_error()
    return msg.decode() if msg else ""


def sampling(temperature: float = 0.0, top_p: float = 1.0, max_tokens: int = 256, top_k: int = 0,
             repetition_penalty: float = 1.0) -> SamplingParams:
    return SamplingParams(temperature, top_p, top_k, repetition_penalty, max_tokens)


def _ids(ids: Sequence[int]):
    arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
    return arr, len(ids)


class NativeEngine:
    """One engine over an SGLBITNT model file on the current HIP device.  Errors raise RuntimeError with
    bitnet_get_error()'s message."""

    def __init__(self, path: str, max_seq_len: int = 0):
        cfg = BitNetConfig(max_seq_len, 0, 0)
        h = lib().bitnet_engine_create(str(path).encode(), ctypes.byref(cfg))
        if not h:
            raise RuntimeError(f"bitnet_engine_create failed: {last_error()}")
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().bitnet_engine_destroy(self._h)
            self._h = None

    def __enter__(self) -> "NativeEngine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int, what: str) -> None:
        if st != 0:
            raise RuntimeError(f"{what} failed: {last_error()}")

    def generate(self, ids: Sequence[int], params: Optional[SamplingParams] = None, **kw) -> List[int]:
        p = params if params is not None else sampling(**kw)
        arr, n = _ids(ids)
        res = GenerationResult()
        self._check(lib().bitnet_generate(self._h, arr, n, ctypes.byref(p), ctypes.byref(res)), "bitnet_generate")
        try:
            return [res.output_ids[i] for i in range(res.num_tokens)]
        finally:
            lib().bitnet_free_result(ctypes.byref(res))

    def prefill(self, ids: Sequence[int]) -> None:
        arr, n = _ids(ids)
        self._check(lib().bitnet_prefill(self._h, arr, n), "bitnet_prefill")

    def decode_step(self, position: int, params: Optional[SamplingParams] = None, **kw) -> int:
        p = params if params is not None else sampling(**kw)
        out = ctypes.c_int32(-1)
        self._check(lib().bitnet_decode_step(self._h, position, ctypes.byref(p), ctypes.byref(out)),
                    "bitnet_decode_step")
        return out.value

    def reset(self) -> None:
        lib().bitnet_reset_cache(self._h)

    @property
    def vocab_size(self) -> int:
        return lib().bitnet_vocab_size(self._h)

    @property
    def hidden_size(self) -> int:
        return lib().bitnet_hidden_size(self._h)

    @property
    def num_layers(self) -> int:
        return lib().bitnet_num_layers(self._h)

    @property
    def max_seq_len(self) -> int:
        return lib().bitnet_max_seq_len(self._h)

    @property
    def num_kv_heads(self) -> int:
        return lib().bitnet_get_num_kv_heads(self._h)


def sample_top_p(logits: Sequence[float], temperature: float, top_p: float, seed: int, draws: int) -> List[int]:
    """`draws` picks of the engine's sampler from the same float32 logits with a fresh mt19937(seed)."""
    n = len(logits)
    arr = (ctypes.c_float * max(n, 1))(*logits)
    out = (ctypes.c_int32 * max(draws, 1))()
    st = lib().wfb_engine_sample_top_p(ctypes.cast(arr, _vp), n, temperature, top_p, seed, draws, out)
    if st != 0:
        raise RuntimeError(f"wfb_engine_sample_top_p failed: {last_error()}")
    return list(out[:draws])


def fail_alloc_after(n: int) -> None:
    """Test hook: after `n` more successful engine allocations the next one fails (n < 0: never)."""
    lib().wfb_engine_fail_alloc_after(int(n))
