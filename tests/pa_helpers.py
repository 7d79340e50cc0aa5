"""Shared helpers for the paged-attention tests (oracle calls, tolerances)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import pa_oracle
from oracle import pa_oracle_c

# Tolerances of the benchmark contract (bf16 inputs, fp32 accumulation).
MAX_ABS = 2e-2
REL_L2 = 1e-3
# The reference's own paged-attention scene test uses allclose(rtol=1e-3, atol=1e-3)
# (examples/a2a3/tensormap_and_ringbuffer/paged_attention/test_paged_attention.py:22-23).
REF_RTOL = 1e-3
REF_ATOL = 1e-3


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor → uint16 bit pattern array."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def oracle_numpy(case) -> np.ndarray:
    c = case.config
    return pa_oracle.paged_attention_decode(
        f32(case.query), f32(case.key_cache), None if c.mla else f32(case.value_cache),
        case.block_table.numpy(), case.context_lens.numpy(), case.scale, causal=c.causal,
        v_dim=c.head_dim_v if c.mla else None,
        p_dtype="fp16" if case.query.dtype == torch.float16 else "bf16")


def oracle_c(case, n_threads: int | None = None) -> np.ndarray:
    c = case.config
    return pa_oracle_c.decode(
        bits(case.query), bits(case.key_cache), None if c.mla else bits(case.value_cache),
        case.block_table.numpy(), case.context_lens.numpy(), case.scale, causal=c.causal,
        v_dim=c.head_dim_v if c.mla else None, n_threads=n_threads)


def errors(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    max_abs = float(np.max(np.abs(got - ref))) if got.size else 0.0
    denom = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(got - ref) / denom) if denom > 0 else float(np.linalg.norm(got - ref))
    return max_abs, rel


def assert_close(got, ref, max_abs: float = MAX_ABS, rel_l2: float = REL_L2, what: str = "") -> tuple[float, float]:
    a, r = errors(got, ref)
    assert np.all(np.isfinite(np.asarray(got, dtype=np.float64))), f"{what}: non-finite output"
    assert a <= max_abs and r <= rel_l2, f"{what}: max_abs={a:.3e} (tol {max_abs}) rel_l2={r:.3e} (tol {rel_l2})"
    return a, r
