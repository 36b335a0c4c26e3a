"""ctypes binding of libwfbitnet.so (the C ABI declared in include/wfbitnet.h).

The library is loaded from this package directory.  There is no fallback: if it is missing or
does not load, every op raises, the way the reference serving method fails loudly without its
native kernels (SGB/python/sglang/srt/layers/quantization/bitnet.py:243-250).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_NAME = "libwfbitnet.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

# dtype codes of the C ABI
WFB_F32 = 0
WFB_BF16 = 1
WFB_F16 = 2
WFB_OK = 0
WFB_QK_I2S = 128
WFB_ABSMEAN_WS_DOUBLES = 1024
WFB_NORM_MAX_H = 16384
WFB_MAX_SEGMENTS = 8
WFB_SCALE_REFERENCE = 0
WFB_SCALE_CHECKPOINT = 1
WFB_ACT_SILU = 1
WFB_ACT_RELU2 = 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (restype is int for all but the two queries)
SIGNATURES = {
    "wfb_weight_absmean": [_vp, _int, _i64, _vp, _vp, _vp],
    "wfb_pack_i2s": [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp],
    "wfb_unpack_i2s": [_vp, _i64, _i64, _vp, _vp],
    "wfb_quantize_act_i8": [_vp, _int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp],
    "wfb_quantize_act_i8_tensor": [_vp, _int, _i64, _vp, _vp, _vp],
    "wfb_rmsnorm_quant_i8": [_vp, _int, _i64, _vp, _int, _f32, _i64, _i64, _vp, _i64, _i64, _vp, _vp],
    "wfb_linear_i2s": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _int, _vp, _int, _i64, _vp, _vp],
    "wfb_gemv_i2s": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _int, _vp, _int, _i64, _vp, _vp],
    "wfb_gemm_i2s": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _int, _vp, _int, _i64, _vp, _vp],
    "wfb_linear_i2s_segmented": [_vp, _i64, _i64, _int, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _int, _vp, _int, _i64,
                                 _vp, _vp],
    "wfb_glu_rmsnorm_quant_i8": [_vp, _vp, _int, _i64, _int, _vp, _int, _f32, _i64, _i64, _vp, _i64, _i64, _vp, _vp],
    "wfb_convert_hf_offline_i2s": [_vp, _i64, _i64, _i64, _i64, _vp, _int, _f32, _int, _vp, _vp, _vp, _vp],
    "wfb_linear_i2s_residual": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _int, _i64, _vp, _int, _i64,
                                _vp],
    "wfb_linear_i2s_argmax": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _f32, _vp, _int, _i64, _vp, _vp, _vp],
    "wfb_lm_head_argmax": [_vp, _int, _i64, _vp, _int, _f32, _vp, _int, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp,
                           _vp],
    "wfb_gqa_decode_attention": [_vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64,
                                 _i64, _i64, _f32, _vp, _i64, _vp, _vp],
    "wfb_gqa_decode_attention_noalloc": [_vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64,
                                         _i64, _i64, _i64, _f32, _vp, _i64, _vp],
    "wfb_gqa_prefill_attention": [_vp, _i64, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i64, _f32, _vp, _i64, _vp],
    "wfb_linear_i2s_glu": [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _int, _int, _vp, _i64, _vp],
    "wfb_rmsnorm_linear_i2s": [_vp, _int, _i64, _vp, _int, _f32, _i64, _i64, _vp, _i64, _i64, _int, _vp, _vp, _vp,
                               _int, _i64, _vp, _int, _i64, _vp],
    "wfb_rope_tables": [ctypes.c_double, _i64, _i64, _vp, _vp],
    "wfb_rmsnorm_linear_i2s_glu": [_vp, _int, _i64, _vp, _int, _f32, _i64, _i64, _vp, _i64, _i64, _vp, _int, _int, _vp,
                                   _i64, _vp],
}

_lib = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if it is not built or does not load."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        _load_error = f"{LIB_PATH} is not built (run __graft_entry__.build() or wrinklefree-monorepo_amd/_build.py)"
        raise RuntimeError(_load_error)
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as e:  # pragma: no cover - depends on the ROCm runtime
        _load_error = f"failed to load {LIB_PATH}: {e}"
        raise RuntimeError(_load_error) from e
    lib.wfb_last_error.restype = ctypes.c_char_p
    lib.wfb_last_error.argtypes = []
    lib.wfb_version.restype = ctypes.c_int
    lib.wfb_version.argtypes = []
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def last_error() -> str:
    return load().wfb_last_error().decode()


def call(name: str, *args) -> None:
    """Call an entry point; a non-zero status raises RuntimeError carrying wfb_last_error()."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != WFB_OK:
        raise RuntimeError(f"{name} failed ({st}): {lib.wfb_last_error().decode()}")


def status(name: str, *args) -> int:
    """Call an entry point and return its raw status (for tests of the error contract)."""
    return getattr(load(), name)(*args)
