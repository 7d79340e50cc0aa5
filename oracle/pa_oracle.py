"""CPU oracle for paged-attention decode — TEST INFRASTRUCTURE ONLY.

Nothing in the product path (``simpler_amd``) may import this module. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use
it, and only as the checker. The product path has no CPU fallback.

This is a numpy restatement of simpler's paged-attention golden and of the
four per-block kernels it models:

* ``simpler_setup/goldens/paged_attention.py:91-189`` — online softmax over KV
  blocks: scores ``s = q·kᵀ·scale`` in fp32 (``:149``), columns past the valid
  length masked to −inf (``:151-157``), block max clamped at −1e30 (``:159-160``),
  ``p = exp(s − m_blk)`` with masked entries forced to 0 (``:161-163``), **p rounded
  to the input dtype (bf16) before the row sum and the PV product** (``:164-165``),
  ``o_blk = p·V`` (``:167``), then the online merge ``m' = max(m, m_blk)``,
  ``α = e^{m−m'}``, ``β = e^{m_blk−m'}``, ``l' = αl + βl_blk``, ``o' = αo + βo_blk``
  (``:174-183``) and ``out = o / l`` (``:187``).
* The same arithmetic per kernel: ``aic_qk_matmul.cpp:38-100`` (QK),
  ``aiv_softmax_prepare.cpp:96-131`` (mask, scale, rowmax, exp, bf16 round,
  rowsum), ``aic_pv_matmul.cpp:38-99`` (PV), ``aiv_online_update.cpp:125-224``
  (merge, final divide) — all under
  ``examples/a2a3/tensormap_and_ringbuffer/paged_attention/kernels/``.
* GQA head mapping ``kv_head = h // (Hq/Hkv)`` from
  ``tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention_highperf/
  test_spmd_paged_attention_highperf.py:69-85``.
* KV cache layout BSND ``[num_blocks, block_size, kv_heads, head_dim]``
  (``goldens/paged_attention.py:76-77``); 4-D query ``[B, q_len, Hq, D]`` as in
  ``tests/st/.../paged_attention_unroll_4dims/test_paged_attention_unroll_4dims.py:120-125``.

Extensions with no reference counterpart (documented as such in the tests):
multi-token causal verify (row ``i`` of ``q_len`` sees ``ctx − (q_len−1−i)``
tokens) and MLA (``V = K[..., :Dv]``, one latent KV head).

Pinning: ``tests/test_oracle.py`` checks every function here against the
fp64 textbook softmax (``attention_fp64``), closed forms (single token, constant
keys, one-hot scores, per-head constant values), a hand-computed bf16-rounding
case, masking invariance and the C restatement ``pa_oracle.c``.
"""

from __future__ import annotations

import numpy as np

NEG_CLAMP = np.float32(-1e30)


# ---------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, as torch's ``.to(torch.bfloat16)``)
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 → bf16 bit pattern (uint16), round-to-nearest-even; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 and return them as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# The oracle proper
# ---------------------------------------------------------------------------


def fp16_round(x: np.ndarray) -> np.ndarray:
    """fp32 → nearest fp16 (IEEE round-to-nearest-even, subnormals kept) → fp32,
    as torch's ``.to(torch.float16)``."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def _row_lengths(ctx: int, q_len: int, g: int, causal: bool) -> np.ndarray:
    """Valid context length for each (query token i, group head) row of one KV head."""
    i = np.repeat(np.arange(q_len), g)
    if causal:
        return (ctx - (q_len - 1 - i)).astype(np.int64)
    return np.full(q_len * g, ctx, dtype=np.int64)


def paged_attention_decode(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray | None,
    block_table: np.ndarray,
    context_lens: np.ndarray,
    scale: float,
    *,
    causal: bool = False,
    v_dim: int | None = None,
    p_dtype: str = "bf16",
) -> np.ndarray:
    """Blockwise online-softmax paged attention (the reference golden's algorithm).

    query:       fp32 ``[B, q_len, Hq, Dk]`` (or ``[B, Hq, Dk]`` for q_len 1), values
                 already representable in the input dtype.
    p_dtype:     the input dtype p is rounded to before the row sum and PV
                 (``goldens/paged_attention.py:168``: ``p.to(query dtype)``):
                 ``"bf16"`` or ``"fp16"``.
    key_cache:   fp32 ``[num_blocks, BS, Hkv, Dk]``.
    value_cache: fp32 ``[num_blocks, BS, Hkv, Dv]``; ``None`` selects MLA, where V is
                 ``key_cache[..., :v_dim]``.
    Returns fp32 ``[B, q_len, Hq, Dv]`` (3-D if the query was 3-D).
    """
    squeeze = query.ndim == 3
    q4 = query[:, None] if squeeze else query
    q4 = np.asarray(q4, dtype=np.float32)
    kc = np.asarray(key_cache, dtype=np.float32)
    if value_cache is None:
        if v_dim is None:
            raise ValueError("MLA (value_cache=None) needs v_dim")
        vc = kc[..., :v_dim]
    else:
        vc = np.asarray(value_cache, dtype=np.float32)
    bsz, q_len, hq, dk = q4.shape
    _, bs, hkv, _ = kc.shape
    dv = vc.shape[-1]
    if hq % hkv:
        raise ValueError("num_heads must be a multiple of kv_heads")
    g = hq // hkv
    sc = np.float32(scale)
    out = np.zeros((bsz, q_len, hq, dv), dtype=np.float32)
    for b in range(bsz):
        ctx = int(context_lens[b])
        nblk = (ctx + bs - 1) // bs
        rlen = _row_lengths(ctx, q_len, g, causal)
        for kvh in range(hkv):
            # rows ordered (query token i, head-in-group hh)
            qr = q4[b, :, kvh * g : (kvh + 1) * g, :].reshape(q_len * g, dk)
            m = l = o = None
            for bn in range(nblk):
                blk = int(block_table[b, bn])
                k = kc[blk, :, kvh, :]
                v = vc[blk, :, kvh, :]
                s = (qr @ k.T).astype(np.float32) * sc
                pos = bn * bs + np.arange(bs)
                valid = pos[None, :] < rlen[:, None]
                s = np.where(valid, s, np.float32(-np.inf))
                mb = np.maximum(s.max(axis=1), NEG_CLAMP)
                with np.errstate(invalid="ignore", over="ignore"):
                    p = np.exp(s - mb[:, None]).astype(np.float32)
                p = np.where(valid, p, np.float32(0.0))
                p = bf16_round(p) if p_dtype == "bf16" else fp16_round(p)
                lb = p.sum(axis=1, dtype=np.float32)
                ob = (p @ v).astype(np.float32)
                if m is None:
                    m, l, o = mb, lb, ob
                else:
                    mn = np.maximum(m, mb)
                    alpha = np.exp(m - mn).astype(np.float32)
                    beta = np.exp(mb - mn).astype(np.float32)
                    l = alpha * l + beta * lb
                    o = alpha[:, None] * o + beta[:, None] * ob
                    m = mn
            if m is None:  # empty context: defined as zero output
                continue
            with np.errstate(invalid="ignore", divide="ignore"):
                res = np.where(l[:, None] > 0, o / l[:, None], np.float32(0.0))
            out[b, :, kvh * g : (kvh + 1) * g, :] = res.reshape(q_len, g, dv)
    return out[:, 0] if squeeze else out


def attention_fp64(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray | None,
    block_table: np.ndarray,
    context_lens: np.ndarray,
    scale: float,
    *,
    causal: bool = False,
    v_dim: int | None = None,
) -> np.ndarray:
    """Textbook ``softmax(q·Kᵀ·scale)·V`` per head in float64 with no rounding.

    Follows the GQA golden of ``test_spmd_paged_attention_highperf.py:56-86``
    (gather the valid tokens through the block table, full softmax per head).
    Used only to pin :func:`paged_attention_decode`.
    """
    squeeze = query.ndim == 3
    q4 = np.asarray(query[:, None] if squeeze else query, dtype=np.float64)
    kc = np.asarray(key_cache, dtype=np.float64)
    vc = kc[..., :v_dim] if value_cache is None else np.asarray(value_cache, dtype=np.float64)
    bsz, q_len, hq, _ = q4.shape
    _, bs, hkv, _ = kc.shape
    g = hq // hkv
    out = np.zeros((bsz, q_len, hq, vc.shape[-1]), dtype=np.float64)
    for b in range(bsz):
        ctx = int(context_lens[b])
        nblk = (ctx + bs - 1) // bs
        blocks = [int(x) for x in block_table[b, :nblk]]
        for h in range(hq):
            kvh = h // g
            keys = np.concatenate([kc[blk, :, kvh, :] for blk in blocks], axis=0)[:ctx]
            vals = np.concatenate([vc[blk, :, kvh, :] for blk in blocks], axis=0)[:ctx]
            for i in range(q_len):
                n = ctx - (q_len - 1 - i) if causal else ctx
                s = keys[:n] @ q4[b, i, h] * scale
                w = np.exp(s - s.max())
                out[b, i, h] = (w / w.sum()) @ vals[:n]
    return out[:, 0] if squeeze else out


# ---------------------------------------------------------------------------
# The four per-block kernels one at a time (the task-graph backend runs them
# as separate tasks). Composing them block by block reproduces
# paged_attention_decode exactly; tests/test_task_graph_oracle.py checks that
# and the closed forms of each step.
# ---------------------------------------------------------------------------


def qk_matmul(qi: np.ndarray, kj: np.ndarray) -> np.ndarray:
    """``sij = qi · kjᵀ`` in fp32 (``aic_qk_matmul.cpp:38-100``); qi ``[M, D]``, kj ``[N, D]``."""
    return (np.asarray(qi, np.float32) @ np.asarray(kj, np.float32).T).astype(np.float32)


def softmax_prepare(sij: np.ndarray, valid_len: int, scale: float) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``aiv_softmax_prepare.cpp:96-131``: columns ``>= valid_len`` → −inf, ``s·scale``,
    ``m = rowmax``, ``p = exp(s − m)`` rounded to bf16, ``l = rowsum(p)``.

    Returns ``(p, m, l)`` with p as fp32 values on the bf16 grid. A block with no
    valid column gives m = −1e30, l = 0, p = 0 (``batch_paged_attention/kernels/aiv/
    aiv_softmax_prepare.cpp:105-121``).
    """
    s = np.asarray(sij, np.float32)
    n = s.shape[1]
    valid = np.arange(n)[None, :] < valid_len
    x = np.where(valid, s * np.float32(scale), np.float32(-np.inf)).astype(np.float32)
    if valid_len <= 0:
        m = np.full(s.shape[0], NEG_CLAMP, np.float32)
        return np.zeros_like(s), m, np.zeros(s.shape[0], np.float32)
    m = x.max(axis=1).astype(np.float32)
    p = bf16_round(np.exp(x - m[:, None]).astype(np.float32))
    return p, m, p.sum(axis=1, dtype=np.float32)


def pv_matmul(pij: np.ndarray, vj: np.ndarray) -> np.ndarray:
    """``oi_new = pij · vj`` in fp32 (``aic_pv_matmul.cpp:38-99``)."""
    return (np.asarray(pij, np.float32) @ np.asarray(vj, np.float32)).astype(np.float32)


def online_update(mij, lij, oi_new, mi, li, oi, is_first: bool, is_last: bool):
    """``aiv_online_update.cpp:125-224``. Returns ``(mi, li, oi, dst)``; dst is None unless is_last.

    First block: the block's (m, l, o) are taken as they are (dst = o / l if also
    last). Otherwise ``m' = max(mi, mij)``, ``α = e^{mi−m'}``, ``β = e^{mij−m'}``,
    ``li = α·li + β·lij``, ``oi = α·oi + β·oi_new``; dst = oi / li when last.
    """
    mij, lij, oi_new = (np.asarray(x, np.float32) for x in (mij, lij, oi_new))
    if is_first:
        dst = (oi_new / lij[:, None]).astype(np.float32) if is_last else None
        return mij.copy(), lij.copy(), oi_new.copy(), dst
    mi, li, oi = (np.asarray(x, np.float32) for x in (mi, li, oi))
    mn = np.maximum(mi, mij)
    alpha = np.exp(mi - mn).astype(np.float32)
    beta = np.exp(mij - mn).astype(np.float32)
    l2 = (alpha * li + beta * lij).astype(np.float32)
    o2 = (oi * alpha[:, None] + oi_new * beta[:, None]).astype(np.float32)
    dst = (o2 / l2[:, None]).astype(np.float32) if is_last else None
    return mn, l2, o2, dst


# ---------------------------------------------------------------------------
# fp8 KV caches (E4M3FN bytes + one fp32 scale per (block, kv head)). There is
# no reference kernel for this format (the reference defines the dtype code,
# src/common/task_interface/data_type.h:63); the oracle dequantises and runs
# the golden above on the fp32 values.
# ---------------------------------------------------------------------------


def fp8_e4m3fn_to_f32(b: np.ndarray) -> np.ndarray:
    """OCP E4M3FN decode: sign, 4 exponent bits (bias 7), 3 mantissa bits;
    exponent 0 is subnormal (m · 2^-9); S.1111.111 is NaN; no infinities."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e, m = (b >> 3) & 0xF, b & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (sign * val).astype(np.float32)


def dequantize_kv(cache8: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``[nblk, BS, Hkv, D]`` E4M3FN bytes and ``[nblk, Hkv]`` scales -> fp32 values."""
    return (fp8_e4m3fn_to_f32(cache8) * np.asarray(scale, np.float32)[:, None, :, None]).astype(np.float32)
