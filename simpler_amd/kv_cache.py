"""KV-cache append and the fused Qwen3 decode prelude on the HIP backend.

The step before paged-attention decode in simpler's Qwen3 decode layer
(``simpler_setup/goldens/qwen3_14b_decode.py``): the current token's K/V are
written into the paged BSND pool at ``slot_mapping`` (``:106-115,261-269``), and
the prelude that produces them and the query — per-head RMS norm with a
weight, half-split RoPE at position ``seq_len − 1``, bf16 rounding
(``:207-226``) — runs fused with that write. Both are kernels in
``libsimpler_hip.so`` (``include/simpler_hip/kv_cache.h``); torch supplies device
memory and the stream only, and there is no fallback.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .paged_attention import PagedAttentionError

EPS = 1e-6  # the golden's eps (qwen3_14b_decode.py:46)

V_SKEW_BYTES = 256  # V pool's distance from K's end, past a multiple of 512 bytes


def alloc_kv_pools(num_blocks: int, block_size: int, kv_heads: int, head_dim: int,
                   dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda",
                   head_dim_v: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """K and V pools, ``[num_blocks, block_size, kv_heads, head_dim(_v)]`` each, in one device allocation.

    V starts ``V_SKEW_BYTES`` past K's end rounded up to 512 bytes, so the two
    pools sit an odd multiple of 256 bytes apart. Pools a multiple of 512
    bytes apart (two separate allocations, or one ``[2, ...]`` tensor) put each
    kv head's K row and V row on the same address bits 8-9; a decode worker
    streams both of its head's rows at once, and those pairs then contend for
    the same HBM channels. Measured on one MI355X, main decode kernel, the
    same inputs in both layouts (bit-identical outputs):

    ========================  ==========  ==========
    config                    apart 0     apart 256
    ========================  ==========  ==========
    Qwen3-8B GQA, B=32        105.8 µs    101.5 µs
    GQA, B=8, L=32768         162.2 µs    158.5 µs
    verify, B=16, q_len=8     129.8 µs    128.0 µs
    ========================  ==========  ==========

    The kernels take any pool addresses; this only places them. Returns the
    two views; the allocation lives as long as either does.
    """
    dv = head_dim if head_dim_v is None else head_dim_v
    esz = torch.empty((), dtype=dtype).element_size()
    k_elems = num_blocks * block_size * kv_heads * head_dim
    v_elems = num_blocks * block_size * kv_heads * dv
    v_start = ((k_elems * esz + 511) // 512 * 512 + V_SKEW_BYTES) // esz
    buf = torch.empty(v_start + v_elems, dtype=dtype, device=device)
    k = buf[:k_elems].view(num_blocks, block_size, kv_heads, head_dim)
    v = buf[v_start:v_start + v_elems].view(num_blocks, block_size, kv_heads, dv)
    return k, v


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a device (cuda/HIP) tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


def _cache_strides(cache: torch.Tensor, name: str) -> tuple[int, int, int]:
    if cache.dim() != 4 or cache.stride(-1) != 1:
        raise ValueError(f"{name} must be [num_blocks, block_size, kv_heads, head_dim] with unit head-dim stride")
    return cache.stride()[:3]


def kv_append(key: torch.Tensor, value: torch.Tensor | None, slot_mapping: torch.Tensor, key_cache: torch.Tensor,
              value_cache: torch.Tensor | None, error_count: torch.Tensor | None = None,
              stream: int | None = None) -> None:
    """Write ``key[t]`` (and ``value[t]``), ``[kv_heads, D]`` bf16, at ``slot_mapping[t]`` of the caches.

    ``slot = physical_block · block_size + offset``; negative slots are skipped;
    slots past the pool are skipped and counted in ``error_count`` (an int32
    device tensor of one element) when given. ``value``/``value_cache`` may be
    ``None`` for a K-only (MLA latent) cache.
    """
    a = append_args(key, value, slot_mapping, key_cache, value_cache, error_count)
    launch_append(a, key.device if stream is None else None, stream)


def launch_append(a: _lib.KvAppendArgs, device: torch.device | None = None, stream: int | None = None) -> None:
    """Enqueue a prepared append (``append_args``) on ``stream`` (default: torch's current stream)."""
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    rc = _lib.lib().simpler_hip_kv_append(ctypes.byref(a), stream)
    if rc != 0:
        raise PagedAttentionError(rc, "simpler_hip_kv_append")


def append_args(key: torch.Tensor, value: torch.Tensor | None, slot_mapping: torch.Tensor, key_cache: torch.Tensor,
                value_cache: torch.Tensor | None, error_count: torch.Tensor | None = None) -> _lib.KvAppendArgs:
    """Validate the tensors of an append and fill the C ``SimplerHipKvAppendArgs``."""
    _dev(key, "key", torch.bfloat16)
    _dev(slot_mapping, "slot_mapping", torch.int32)
    _dev(key_cache, "key_cache", torch.bfloat16)
    if (value is None) != (value_cache is None):
        raise ValueError("value and value_cache go together")
    if key.dim() != 3 or key.stride(-1) != 1:
        raise ValueError("key must be [num_tokens, kv_heads, head_dim] with unit head-dim stride")
    if not slot_mapping.is_contiguous() or slot_mapping.shape != (key.shape[0],):
        raise ValueError("slot_mapping must be a contiguous [num_tokens] tensor")
    a = _lib.KvAppendArgs()
    a.key, a.slot_mapping, a.key_cache = key.data_ptr(), slot_mapping.data_ptr(), key_cache.data_ptr()
    a.key_token_stride, a.key_head_stride = key.stride()[:2]
    a.k_block_stride, a.k_token_stride, a.k_head_stride = _cache_strides(key_cache, "key_cache")
    nblk, bs, hkv, dk = key_cache.shape
    if key.shape[1:] != (hkv, dk):
        raise ValueError(f"key rows {tuple(key.shape[1:])} do not match the cache ({hkv}, {dk})")
    a.num_tokens, a.num_kv_heads, a.head_dim_k, a.block_size, a.num_blocks = key.shape[0], hkv, dk, bs, nblk
    if value is not None:
        _dev(value, "value", torch.bfloat16)
        _dev(value_cache, "value_cache", torch.bfloat16)
        if value.dim() != 3 or value.stride(-1) != 1 or value.shape[:2] != key.shape[:2]:
            raise ValueError("value must be [num_tokens, kv_heads, head_dim_v] with unit head-dim stride")
        a.value, a.value_cache = value.data_ptr(), value_cache.data_ptr()
        a.value_token_stride, a.value_head_stride = value.stride()[:2]
        a.v_block_stride, a.v_token_stride, a.v_head_stride = _cache_strides(value_cache, "value_cache")
        if value_cache.shape[:3] != key_cache.shape[:3] or value_cache.shape[3] != value.shape[2]:
            raise ValueError("value_cache shape does not match key_cache/value")
        a.head_dim_v = value.shape[2]
    if error_count is not None:
        _dev(error_count, "error_count", torch.int32)
        a.error_count = error_count.data_ptr()
    return a


def qk_norm_rope_append(q_proj: torch.Tensor, k_proj: torch.Tensor, v_proj: torch.Tensor, inv_rms: torch.Tensor,
                        q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, rope_cos: torch.Tensor,
                        rope_sin: torch.Tensor, seq_lens: torch.Tensor, slot_mapping: torch.Tensor,
                        key_cache: torch.Tensor, value_cache: torch.Tensor, num_heads: int,
                        q_out: torch.Tensor | None = None, eps: float = EPS,
                        error_count: torch.Tensor | None = None, stream: int | None = None) -> torch.Tensor:
    """The decode prelude fused with the cache write; returns ``q_out`` ``[B, Hq, D]`` bf16.

    ``q_proj [B, Hq·D]``, ``k_proj``/``v_proj [B, Hkv·D]``, ``inv_rms [B]``,
    ``*_norm_weight [D]``, ``rope_cos``/``rope_sin [max_position, D]`` — all fp32
    and contiguous; ``seq_lens``, ``slot_mapping [B]`` int32.
    """
    if q_out is None:
        q_out = torch.empty((q_proj.shape[0], num_heads, key_cache.shape[3]), dtype=torch.bfloat16,
                            device=q_proj.device)
    a = prelude_args(q_proj, k_proj, v_proj, inv_rms, q_norm_weight, k_norm_weight, rope_cos, rope_sin, seq_lens,
                     slot_mapping, key_cache, value_cache, num_heads, q_out, eps, error_count)
    launch_prelude(a, q_proj.device if stream is None else None, stream)
    return q_out


def launch_prelude(a: _lib.QkNormRopeAppendArgs, device: torch.device | None = None,
                   stream: int | None = None) -> None:
    """Enqueue a prepared prelude (``prelude_args``) on ``stream`` (default: torch's current stream)."""
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    rc = _lib.lib().simpler_hip_qk_norm_rope_append(ctypes.byref(a), stream)
    if rc != 0:
        raise PagedAttentionError(rc, "simpler_hip_qk_norm_rope_append")


def prelude_args(q_proj: torch.Tensor, k_proj: torch.Tensor, v_proj: torch.Tensor, inv_rms: torch.Tensor,
                 q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, rope_cos: torch.Tensor,
                 rope_sin: torch.Tensor, seq_lens: torch.Tensor, slot_mapping: torch.Tensor,
                 key_cache: torch.Tensor, value_cache: torch.Tensor, num_heads: int, q_out: torch.Tensor,
                 eps: float = EPS, error_count: torch.Tensor | None = None) -> _lib.QkNormRopeAppendArgs:
    """Validate the tensors of a prelude call and fill the C ``SimplerHipQkNormRopeAppendArgs``."""
    for t, n in ((q_proj, "q_proj"), (k_proj, "k_proj"), (v_proj, "v_proj"), (inv_rms, "inv_rms"),
                 (q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight"), (rope_cos, "rope_cos"),
                 (rope_sin, "rope_sin")):
        _dev(t, n, torch.float32)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n in ((seq_lens, "seq_lens"), (slot_mapping, "slot_mapping")):
        _dev(t, n, torch.int32)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    _dev(key_cache, "key_cache", torch.bfloat16)
    _dev(value_cache, "value_cache", torch.bfloat16)
    nblk, bs, hkv, d = key_cache.shape
    b = q_proj.shape[0]
    if q_proj.shape != (b, num_heads * d) or k_proj.shape != (b, hkv * d) or v_proj.shape != (b, hkv * d):
        raise ValueError("projection shapes do not match num_heads/kv_heads/head_dim of the cache")
    if inv_rms.numel() != b or seq_lens.shape != (b,) or slot_mapping.shape != (b,):
        raise ValueError("inv_rms/seq_lens/slot_mapping must have one entry per sequence")
    if q_norm_weight.numel() != d or k_norm_weight.numel() != d:
        raise ValueError("norm weights must have head_dim entries")
    if rope_cos.dim() != 2 or rope_cos.shape[1] != d or rope_sin.shape != rope_cos.shape:
        raise ValueError("rope tables must be [max_position, head_dim]")
    if value_cache.shape != key_cache.shape:
        raise ValueError("value_cache must match key_cache")
    _dev(q_out, "q_out", torch.bfloat16)
    if not q_out.is_contiguous() or q_out.shape != (b, num_heads, d):
        raise ValueError("q_out must be a contiguous [B, Hq, D] tensor")
    a = _lib.QkNormRopeAppendArgs()
    a.q_proj, a.k_proj, a.v_proj, a.inv_rms = (t.data_ptr() for t in (q_proj, k_proj, v_proj, inv_rms))
    a.q_norm_weight, a.k_norm_weight = q_norm_weight.data_ptr(), k_norm_weight.data_ptr()
    a.rope_cos, a.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
    a.seq_lens, a.slot_mapping, a.q_out = seq_lens.data_ptr(), slot_mapping.data_ptr(), q_out.data_ptr()
    a.key_cache, a.value_cache = key_cache.data_ptr(), value_cache.data_ptr()
    a.k_block_stride, a.k_token_stride, a.k_head_stride = _cache_strides(key_cache, "key_cache")
    a.v_block_stride, a.v_token_stride, a.v_head_stride = _cache_strides(value_cache, "value_cache")
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = b, num_heads, hkv, d
    a.block_size, a.num_blocks, a.max_position = bs, nblk, rope_cos.shape[0]
    a.eps = float(eps)
    if error_count is not None:
        _dev(error_count, "error_count", torch.int32)
        a.error_count = error_count.data_ptr()
    return a
