"""CPU oracle for the KV-cache append and the Qwen3 decode prelude — TEST INFRASTRUCTURE ONLY.

Nothing in the product path (``simpler_amd``) may import this module. Only
``tests/`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only as the
checker. The product path has no CPU fallback.

A numpy restatement of the decode-layer prelude and cache write of simpler's
Qwen3-14B decode golden (``simpler_setup/goldens/qwen3_14b_decode.py``):

* slot mapping (``:106-115``): the current token of sequence ``b`` sits at
  position ``p = seq_len − 1``; its slot is ``phys_page · BLOCK_SIZE + p % BLOCK_SIZE``
  with ``phys_page = block_table[b, p // BLOCK_SIZE]``.
* cache write (``:261-269``): in the flat BSND view ``[pages · BLOCK_SIZE ·
  kv_heads, head_dim]`` the row ``slot · kv_heads + kv_head`` receives the
  current token's K (and V), rounded to bf16 — in 4-D terms
  ``cache[slot // BS, slot % BS, kv_head, :]``.
* prelude (``:207-226``): ``q = (q_proj · inv_rms)`` per head, then
  ``q · rsqrt(mean(q²) + eps) · q_norm_weight`` (``_rmsnorm_inv``, ``:95-96``),
  the same for K with ``k_norm_weight``, ``v = v_proj · inv_rms``; RoPE of the
  half-split form (``_rope_half``, ``:99-103``) at position ``p`` on q and k; q,
  k and v rounded to bf16 (``:222-224``).

Pinning: ``tests/test_kv_oracle.py`` checks these against closed forms (the
reference's identity paging puts each token at ``cache[b·maxblk + p//BS,
p%BS]``; only ``B·Hkv·D`` cache elements change; RoPE with cos = 1, sin = 0 is
the identity and with cos = 0, sin = 1 maps ``[lo, hi]`` to ``[−hi, lo]``; RoPE with
the reference's tables preserves each ``(lo_i, hi_i)`` pair's norm; the RMS
norm of a constant vector ``c`` is ``c / sqrt(c² + eps)``; the RMS norm matches
an fp64 evaluation).
"""

from __future__ import annotations

import numpy as np

from oracle.pa_oracle import bf16_bits_to_f32, f32_to_bf16_bits

EPS = 1e-6  # goldens/qwen3_14b_decode.py:46


def slot_of(block_table: np.ndarray, seq_lens: np.ndarray, block_size: int) -> np.ndarray:
    """Slot of each sequence's current token (goldens/qwen3_14b_decode.py:106-115)."""
    pos = seq_lens.astype(np.int64) - 1
    phys = block_table[np.arange(len(pos)), pos // block_size].astype(np.int64)
    return (phys * block_size + pos % block_size).astype(np.int32)


def new_token_slots(block_table: np.ndarray, seq_lens: np.ndarray, block_size: int, n_new: int) -> np.ndarray:
    """Slots ``[B, n_new]`` of each sequence's last ``n_new`` positions
    ``seq_len - n_new .. seq_len - 1``, derived as the reference derives the
    current token's (goldens/qwen3_14b_decode.py:106-115; ``n_new = 1`` is
    ``slot_of``); positions below 0, or past what the table row holds
    (``block_table.shape[1] * block_size`` and up), get slot -1 (skipped by
    ``kv_append``)."""
    pos = seq_lens.astype(np.int64)[:, None] - n_new + np.arange(n_new, dtype=np.int64)[None, :]
    cap = block_table.shape[1] * block_size
    rows = np.arange(len(seq_lens))[:, None]
    phys = block_table[rows, np.clip(pos, 0, max(cap - 1, 0)) // block_size].astype(np.int64)
    ok = (pos >= 0) & (pos < cap)
    return np.where(ok, phys * block_size + pos % block_size, -1).astype(np.int32)


def kv_append(key_cache: np.ndarray, value_cache: np.ndarray | None, key: np.ndarray, value: np.ndarray | None,
              slot_mapping: np.ndarray) -> tuple[np.ndarray, np.ndarray | None]:
    """Write token ``t``'s ``[kv_heads, D]`` rows at ``slot_mapping[t]`` (goldens/qwen3_14b_decode.py:261-269).

    Caches are ``[num_blocks, block_size, kv_heads, D]`` bit patterns (uint16);
    negative slots are skipped (padding tokens). Returns updated copies.
    """
    kc = key_cache.copy()
    vc = None if value_cache is None else value_cache.copy()
    bs = kc.shape[1]
    for t, slot in enumerate(np.asarray(slot_mapping, dtype=np.int64)):
        if slot < 0:
            continue
        kc[slot // bs, slot % bs] = key[t]
        if vc is not None:
            vc[slot // bs, slot % bs] = value[t]
    return kc, vc


def rms_inv(x: np.ndarray, eps: float = EPS) -> np.ndarray:
    """``rsqrt(mean(x², -1) + eps)`` in fp32 (goldens/qwen3_14b_decode.py:95-96)."""
    x = np.asarray(x, dtype=np.float32)
    return (np.float32(1.0) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32) + np.float32(eps))
            ).astype(np.float32)


def rope_half(vec: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Half-split RoPE (goldens/qwen3_14b_decode.py:99-103)."""
    h = vec.shape[-1] // 2
    lo, hi = vec[..., :h], vec[..., h:]
    out = np.concatenate([lo * cos[..., :h] - hi * sin[..., :h], hi * cos[..., h:] + lo * sin[..., h:]], axis=-1)
    return out.astype(np.float32)


def qk_norm_rope(q_proj: np.ndarray, k_proj: np.ndarray, v_proj: np.ndarray, inv_rms: np.ndarray,
                 q_norm_weight: np.ndarray, k_norm_weight: np.ndarray, rope_cos: np.ndarray, rope_sin: np.ndarray,
                 seq_lens: np.ndarray, num_heads: int, num_kv_heads: int, eps: float = EPS
                 ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Prelude of one decode layer (goldens/qwen3_14b_decode.py:207-226).

    ``q_proj [B, Hq·D]``, ``k_proj``/``v_proj [B, Hkv·D]``, ``inv_rms [B]`` fp32;
    returns bf16 bit patterns ``q [B, Hq, D]``, ``k [B, Hkv, D]``, ``v [B, Hkv, D]``.
    """
    b = q_proj.shape[0]
    d = q_proj.shape[1] // num_heads
    ir = np.asarray(inv_rms, dtype=np.float32).reshape(b, 1, 1)
    qh = np.asarray(q_proj, dtype=np.float32).reshape(b, num_heads, d) * ir
    qh = (qh * rms_inv(qh, eps) * np.asarray(q_norm_weight, dtype=np.float32)).astype(np.float32)
    kh = np.asarray(k_proj, dtype=np.float32).reshape(b, num_kv_heads, d) * ir
    kh = (kh * rms_inv(kh, eps) * np.asarray(k_norm_weight, dtype=np.float32)).astype(np.float32)
    vh = (np.asarray(v_proj, dtype=np.float32).reshape(b, num_kv_heads, d) * ir).astype(np.float32)
    pos = np.asarray(seq_lens, dtype=np.int64) - 1
    cos = np.asarray(rope_cos, dtype=np.float32)[pos][:, None, :]
    sin = np.asarray(rope_sin, dtype=np.float32)[pos][:, None, :]
    q = f32_to_bf16_bits(rope_half(qh, cos, sin))
    k = f32_to_bf16_bits(rope_half(kh, cos, sin))
    v = f32_to_bf16_bits(vh)
    return q, k, v


def rope_tables(max_pos: int, head_dim: int, theta: float = 1.0e4) -> tuple[np.ndarray, np.ndarray]:
    """The reference's RoPE tables (goldens/qwen3_14b_decode.py:149-153): both halves share the angles."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (np.arange(half, dtype=np.float32) / half))
    ang = np.arange(max_pos, dtype=np.float32)[:, None] * inv_freq[None, :].astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return np.concatenate([cos, cos], axis=1), np.concatenate([sin, sin], axis=1)


__all__ = ["EPS", "slot_of", "kv_append", "rms_inv", "rope_half", "qk_norm_rope", "rope_tables",
           "bf16_bits_to_f32", "f32_to_bf16_bits"]
