"""SGLBITNT model files: the reader (and the writer used to produce them) of the packed-model format
of the reference's native engine.

Format (little endian), as read by SGLKernelModelLoader::load
(packages/inference/extern/sglang-bitnet/sgl-kernel/csrc/inference/sglkernel_loader.h:75-161) and written by
convert_checkpoint / write_tensor (packages/inference/scripts/convert_to_sglkernel.py:135-160, 288-322):

    8 bytes  magic "SGLBITNT"
    u32      version (1)
    u32      config JSON length, then the JSON (HF config.json keys)
    u32      number of tensors; per tensor:
        u32 name length, name (UTF-8)
        u32 dtype (0 uint8, 1 float32, 2 float16, 3 bfloat16)
        u32 ndims, ndims x u32 shape
        u32 scale flag (1 = present), then f32 scale if present
        u64 data size in bytes, then the raw data (row-major)

Packed linears are uint8 [out, in/4] in I2_S with their per-tensor scale in the header; the rest
(embedding, norms) are float32.  Tensor data is memory-mapped, not read whole, and goes to the GPU one
tensor at a time.  Errors raise ``ValueError`` with the loader's messages ("Invalid magic number",
"Unsupported version: N", "Invalid config: vocab_size or hidden_size is 0").
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Mapping, Optional, Tuple, Union

import numpy as np
import torch

MAGIC = b"SGLBITNT"
VERSION = 1
DTYPE_IDS = {0: torch.uint8, 1: torch.float32, 2: torch.float16, 3: torch.bfloat16}
_IDS = {v: k for k, v in DTYPE_IDS.items()}
_NP = {0: np.uint8, 1: np.float32, 2: np.float16, 3: np.uint16}  # bf16 is read as its bits


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype_id: int
    shape: Tuple[int, ...]
    scale: Optional[float]  # present for packed linears
    offset: int             # byte offset of the data in the file
    nbytes: int


class SGLBitNetFile:
    """Header of an SGLBITNT file plus memory-mapped access to its tensors."""

    def __init__(self, path: Union[str, Path]):
        self.path = Path(path)
        self.tensors: Dict[str, TensorInfo] = {}
        with open(self.path, "rb") as f:
            if f.read(8) != MAGIC:
                raise ValueError("Invalid magic number")
            (version,) = struct.unpack("<I", _read(f, 4))
            if version != VERSION:
                raise ValueError(f"Unsupported version: {version}")
            (clen,) = struct.unpack("<I", _read(f, 4))
            self.config = json.loads(_read(f, clen).decode("utf-8"))
            if not self.config.get("vocab_size") or not self.config.get("hidden_size"):
                raise ValueError("Invalid config: vocab_size or hidden_size is 0")
            (count,) = struct.unpack("<I", _read(f, 4))
            for _ in range(count):
                (nlen,) = struct.unpack("<I", _read(f, 4))
                name = _read(f, nlen).decode("utf-8")
                dtype_id, ndims = struct.unpack("<II", _read(f, 8))
                if dtype_id not in DTYPE_IDS:
                    raise ValueError(f"{name}: unknown dtype id {dtype_id}")
                shape = struct.unpack(f"<{ndims}I", _read(f, 4 * ndims))
                (has_scale,) = struct.unpack("<I", _read(f, 4))
                scale = struct.unpack("<f", _read(f, 4))[0] if has_scale == 1 else None
                (nbytes,) = struct.unpack("<Q", _read(f, 8))
                offset = f.tell()
                expect = int(np.prod(shape, dtype=np.int64)) * np.dtype(_NP[dtype_id]).itemsize
                if nbytes != expect:
                    raise ValueError(f"{name}: {nbytes} data bytes for shape {tuple(shape)}, expected {expect}")
                f.seek(nbytes, 1)
                if f.tell() > self.path.stat().st_size:
                    raise ValueError(f"{name}: data runs past the end of the file")
                self.tensors[name] = TensorInfo(name, dtype_id, tuple(shape), scale, offset, nbytes)

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def numpy(self, name: str) -> np.ndarray:
        """Read-only memory map of a tensor (bfloat16 as uint16 bits)."""
        t = self.tensors[name]
        return np.memmap(self.path, dtype=_NP[t.dtype_id], mode="r", offset=t.offset, shape=t.shape)

    def tensor(self, name: str, device: Union[str, torch.device] = "cpu") -> torch.Tensor:
        t = self.tensors[name]
        a = torch.from_numpy(np.array(self.numpy(name)))  # one copy out of the map
        if t.dtype_id == 3:
            a = a.view(torch.bfloat16)
        return a.to(device)


def _read(f, n: int) -> bytes:
    b = f.read(n)
    if len(b) != n:
        raise ValueError("truncated SGLBITNT file")
    return b


def write_sglbitnt(path: Union[str, Path], config: Mapping,
                   tensors: Mapping[str, Tuple[torch.Tensor, Optional[float]]]) -> None:
    """Write ``tensors`` (name -> (tensor, scale or None)) in the order given."""
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<I", VERSION))
        cj = json.dumps(dict(config)).encode("utf-8")
        f.write(struct.pack("<I", len(cj)))
        f.write(cj)
        f.write(struct.pack("<I", len(tensors)))
        for name, (t, scale) in tensors.items():
            t = t.detach().contiguous().cpu()
            if t.dtype not in _IDS:
                t = t.float()
            dtype_id = _IDS[t.dtype]
            nb = name.encode("utf-8")
            f.write(struct.pack("<I", len(nb)))
            f.write(nb)
            f.write(struct.pack("<II", dtype_id, t.dim()))
            f.write(struct.pack(f"<{t.dim()}I", *t.shape))
            if scale is None:
                f.write(struct.pack("<I", 0))
            else:
                f.write(struct.pack("<If", 1, float(scale)))
            data = (t.view(torch.uint16) if t.dtype == torch.bfloat16 else t).numpy().tobytes()
            f.write(struct.pack("<Q", len(data)))
            f.write(data)
