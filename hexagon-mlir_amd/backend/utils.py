"""dtype ids and the raw tensor file format of the reference's launcher.

Output files (test/utils/dsp/include/tensor.h:232-257, read back by
qcom_hexagon_backend/backend/hexagon_executor.py:142-158):
    int32  dtype id
    int64  rank
    int64  shape[rank]
    data   (row-major, native little-endian)
Input files are the bare data (hexagon_launcher_base.py:426-449).
"""
from __future__ import annotations

import pathlib
import struct
from typing import Union

import numpy as np
import torch

# test/utils/dsp/include/tensor.h:26-37; backend/utils.py:36-53
DTYPE_IDS = {
    torch.float16: 1,
    torch.float32: 2,
    torch.float64: 3,
    torch.int8: 4,
    torch.int16: 5,
    torch.int32: 6,
    torch.int64: 7,
    torch.uint8: 8,
    torch.uint16: 9,
    torch.uint32: 10,
}
_FROM_ID = {v: k for k, v in DTYPE_IDS.items()}


def to_torch_type(type_id: int) -> torch.dtype:
    """dtype id -> torch dtype (backend/utils.py:36-53); KeyError if unknown."""
    return _FROM_ID[type_id]


def dtype_id(dtype: torch.dtype) -> int:
    if dtype not in DTYPE_IDS:
        raise ValueError(f"no raw-file dtype id for {dtype}")
    return DTYPE_IDS[dtype]


PathLike = Union[str, pathlib.Path]


def _bytes(t: torch.Tensor) -> bytes:
    """Raw little-endian bytes of a contiguous CPU tensor (any rank)."""
    if t.numel() == 0:
        return b""
    return t.reshape(-1).view(torch.uint8).numpy().tobytes()


def write_output_tensor(path: PathLike, t: torch.Tensor) -> None:
    """Write t in the output-file format (header + data)."""
    t = t.detach().contiguous().cpu()
    with open(path, "wb") as f:
        f.write(struct.pack("<i", dtype_id(t.dtype)))
        f.write(struct.pack("<q", t.dim()))
        if t.dim():
            f.write(struct.pack(f"<{t.dim()}q", *t.shape))
        f.write(_bytes(t))


def read_output_tensor(path: PathLike) -> torch.Tensor:
    """Read an output-format file back into a CPU tensor."""
    data = pathlib.Path(path).read_bytes()
    if len(data) < 12:
        raise ValueError(f"{path}: truncated header")
    dtype = to_torch_type(struct.unpack_from("<I", data, 0)[0])
    rank = struct.unpack_from("<q", data, 4)[0]
    if rank < 0 or 12 + 8 * rank > len(data):
        raise ValueError(f"{path}: bad rank {rank}")
    shape = list(struct.unpack_from(f"<{rank}q", data, 12)) if rank else []
    payload = data[12 + 8 * rank:]
    esize = torch.empty((), dtype=dtype).element_size()
    n = int(np.prod(shape)) if shape else 1
    if len(payload) != n * esize:
        raise ValueError(f"{path}: {len(payload)} data bytes for shape {shape} of {dtype}")
    flat = torch.frombuffer(bytearray(payload), dtype=torch.uint8).view(dtype)
    return flat.reshape(shape)


def write_input_tensor(path: PathLike, t: torch.Tensor) -> None:
    """Write t as a bare input file (data only)."""
    t = t.detach().contiguous().cpu()
    pathlib.Path(path).write_bytes(_bytes(t))
