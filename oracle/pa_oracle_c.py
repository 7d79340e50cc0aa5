"""ctypes binding of ``oracle/_build/libpa_oracle.so`` (the C restatement).

Test infrastructure only: tests use it as a second, independent restatement and
bench.py times it as the CPU baseline.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import LIB

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} missing: run `python -m oracle.build`")
        _lib = ctypes.CDLL(str(LIB))
        _lib.pa_oracle_decode.restype = ctypes.c_int
        _lib.pa_oracle_decode.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 8 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return _lib


def decode(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray | None, block_table: np.ndarray,
           context_lens: np.ndarray, scale: float, *, causal: bool = False, v_dim: int | None = None,
           n_threads: int | None = None, n_items: int = 0, out: np.ndarray | None = None) -> np.ndarray:
    """Run the C restatement on bf16 bit arrays (uint16).

    q_bits [B, q_len, Hq, Dk] (or [B, Hq, Dk]); k_bits [nblk, BS, Hkv, Dk];
    v_bits [nblk, BS, Hkv, Dv] or None for MLA (V = K[..., :v_dim]).
    Returns fp32 out shaped like the query with Dv columns.
    """
    squeeze = q_bits.ndim == 3
    q4 = q_bits[:, None] if squeeze else q_bits
    q4 = np.ascontiguousarray(q4, dtype=np.uint16)
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    mla = v_bits is None
    v = k if mla else np.ascontiguousarray(v_bits, dtype=np.uint16)
    bsz, q_len, hq, dk = q4.shape
    _, bs, hkv, _ = k.shape
    dv = v_dim if mla else v.shape[-1]
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    if out is None:
        out = np.zeros((bsz, q_len, hq, dv), dtype=np.float32)
    nt = n_threads if n_threads is not None else (os.cpu_count() or 1)
    rc = lib().pa_oracle_decode(
        q4.ctypes.data, k.ctypes.data, v.ctypes.data, bt.ctypes.data, cl.ctypes.data, out.ctypes.data,
        bsz, q_len, hq, hkv, dk, dv, bs, bt.shape[1], ctypes.c_float(scale), int(causal), int(mla), nt,
        int(n_items))
    if rc != 0:
        raise ValueError(f"pa_oracle_decode rejected the arguments ({rc})")
    return out[:, 0] if squeeze else out
