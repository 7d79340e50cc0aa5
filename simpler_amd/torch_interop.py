"""torch dtype ↔ DataType mapping (``simpler_setup/torch_interop.py:39-81``)."""

from __future__ import annotations

from .task_interface import DataType

_MAP = None


def _ensure():
    global _MAP
    if _MAP is None:
        import torch

        _MAP = {
            torch.float32: DataType.FLOAT32,
            torch.float16: DataType.FLOAT16,
            torch.int32: DataType.INT32,
            torch.int16: DataType.INT16,
            torch.int8: DataType.INT8,
            torch.uint8: DataType.UINT8,
            torch.bfloat16: DataType.BFLOAT16,
            torch.int64: DataType.INT64,
            torch.uint16: DataType.UINT16,
            torch.uint32: DataType.UINT32,
        }
        fp8 = getattr(torch, "float8_e4m3fn", None)
        if fp8 is not None:
            _MAP[fp8] = DataType.FP8E4M3FN
    return _MAP


def torch_dtype_to_datatype(dt) -> DataType:
    """``torch.dtype`` → ``DataType``; raises ``KeyError`` for unsupported dtypes."""
    return _ensure()[dt]
