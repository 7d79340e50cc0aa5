"""Synthetic paged-attention decode workloads (seeded), plus their roofline figures.

Plays the role of the reference's input generator
(``simpler_setup/goldens/paged_attention.py:30-88``): query/K/V in the same
layouts — query ``[B, Hq, D]`` (``[B, q_len, Hq, D]`` for multi-token decode),
caches ``[num_blocks, block_size, kv_heads, D]``, ``block_table [B, max_blocks]``
int32, ``context_lens [B]`` int32 — but seeded and drawn the way the benchmark
configs specify: context lengths, then the block table, then Q, K, V, each
value N(0, 1) in fp32 rounded to bf16.

Config names map to the five benchmark configurations (index = position):
``cfg1_small``, ``cfg2_qwen3_8b``, ``cfg3_long``, ``cfg4_mla``, ``cfg5_verify``;
``cfg2_fp8`` is cfg2's draws with fp8 caches and ``ref_unroll_case1`` the
reference's own paged_attention_unroll Case1 shape.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

SEED_BASE = 20261201


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    index: int
    batch: int
    num_heads: int
    kv_heads: int
    head_dim_k: int
    head_dim_v: int
    block_size: int
    ctx_min: int
    ctx_max: int
    q_len: int = 1
    causal: bool = False
    mla: bool = False
    pool: str = "exact"  # "exact": pool = sum of blocks needed; "fixed:<n>": pool of n blocks
    max_blocks: int | None = None  # block_table width (defaults to ceil(ctx_max/BS))
    out_dtype: torch.dtype = torch.bfloat16
    description: str = ""
    kv_format: str = "bf16"  # "fp8": E4M3FN caches with a power-of-two scale per (block, kv head)

    @property
    def group(self) -> int:
        return self.num_heads // self.kv_heads


CONFIGS: dict[str, DecodeConfig] = {
    c.name: c
    for c in [
        DecodeConfig("cfg1_small", 0, 2, 16, 1, 128, 128, 128, 512, 512, pool="fixed:16", max_blocks=8,
                     description="small decode: B=2, Hq=16, Hkv=1, D=128, BS=128, L=512, pool of 16 blocks"),
        DecodeConfig("cfg2_qwen3_8b", 1, 32, 32, 8, 128, 128, 128, 1024, 8192,
                     description="Qwen3-8B GQA decode: B=32, Hq=32, Hkv=8, D=128, BS=128, L~U[1024,8192]"),
        DecodeConfig("cfg3_long", 2, 8, 64, 8, 128, 128, 128, 32768, 32768,
                     description="long-context GQA: B=8, Hq=64, Hkv=8, D=128, BS=128, L=32768"),
        DecodeConfig("cfg4_mla", 3, 128, 128, 1, 576, 512, 64, 512, 8192, mla=True,
                     description="MLA absorbed MQA: B=128, Hq=128, 1 latent head, Dk=576, Dv=512, BS=64, "
                                 "L~U[512,8192]"),
        DecodeConfig("cfg5_verify", 4, 16, 32, 8, 128, 128, 128, 2048 + 8, 16384 + 8, q_len=8, causal=True,
                     description="speculative verify: B=16, q_len=8 causal, Hq=32, Hkv=8, D=128, BS=128, "
                                 "prefix~U[2048,16384]"),
        # cfg2's draws (same seed index), K/V quantised to fp8 E4M3FN per (block, kv head)
        DecodeConfig("cfg2_fp8", 1, 32, 32, 8, 128, 128, 128, 1024, 8192, kv_format="fp8",
                     description="Qwen3-8B GQA decode, fp8 E4M3FN KV with per-(block, kv head) scales: B=32, Hq=32, "
                                 "Hkv=8, D=128, BS=128, L~U[1024,8192]"),
        # the reference's paged_attention_unroll Case1 (test_paged_attention_unroll.py:63-76); block ids drawn
        # without sharing (every sequence reads its own blocks), table width max_model_len / BS = 256
        DecodeConfig("ref_unroll_case1", 5, 256, 16, 1, 128, 128, 128, 8192, 8192, max_blocks=256,
                     description="reference unroll Case1: B=256, Hq=16, Hkv=1, D=128, BS=128, L=8192, "
                                 "max_model_len 32768"),
    ]
}


@dataclass
class DecodeCase:
    config: DecodeConfig
    seed: int
    query: torch.Tensor  # bf16
    key_cache: torch.Tensor  # bf16 [nblk, BS, Hkv, Dk]
    value_cache: torch.Tensor  # bf16 [nblk, BS, Hkv, Dv] (a view of key_cache for MLA)
    block_table: torch.Tensor  # int32 [B, max_blocks]
    context_lens: torch.Tensor  # int32 [B]
    scale: float
    extra: dict = field(default_factory=dict)
    k_scale: torch.Tensor | None = None  # fp8 caches: fp32 [num_blocks, kv_heads]
    v_scale: torch.Tensor | None = None

    def to(self, device, kv_pool: bool = False) -> "DecodeCase":
        """The case on ``device``. ``kv_pool``: separate K and V caches share one
        allocation laid out by ``kv_cache.alloc_kv_pools`` (V an odd multiple of
        256 bytes from K) instead of two allocations."""
        if kv_pool and not self.config.mla:
            from .kv_cache import alloc_kv_pools

            nblk, bs, hkv, dk = self.key_cache.shape
            k, v = alloc_kv_pools(nblk, bs, hkv, dk, self.key_cache.dtype, device, self.value_cache.shape[3])
            k.copy_(self.key_cache)
            v.copy_(self.value_cache)
        else:
            k = self.key_cache.to(device)
            v = k[..., : self.config.head_dim_v] if self.config.mla else self.value_cache.to(device)
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return DecodeCase(self.config, self.seed, self.query.to(device), k, v, self.block_table.to(device),
                          self.context_lens.to(device), self.scale, dict(self.extra), mv(self.k_scale),
                          mv(self.v_scale))

    @property
    def fp8(self) -> bool:
        return self.k_scale is not None

    def out_shape(self) -> tuple[int, ...]:
        return (*self.query.shape[:-1], self.config.head_dim_v)


def _randn_bf16(shape, gen: torch.Generator, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """N(0, 1) drawn in fp32, rounded to ``dtype`` (bf16 unless stated)."""
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(dtype)


FP8_MAX = 448.0  # largest finite E4M3FN value


def quantize_kv_fp8(cache: torch.Tensor, pow2: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """``[nblk, BS, Hkv, D]`` -> (E4M3FN cache, fp32 scale ``[nblk, Hkv]``).

    One scale per (block, kv head): the block's largest magnitude maps to at
    most 448 (rounded up to a power of two with ``pow2``, so that the
    dequantised values ``fp8 * scale`` are exactly bf16 values). An all-zero
    block gets scale 0."""
    x = cache.float()
    amax = x.abs().amax(dim=(1, 3))
    scale = amax / FP8_MAX
    if pow2:
        scale = torch.where(amax > 0, torch.exp2(torch.ceil(torch.log2(scale.clamp_min(1e-30)))), scale)
    q = torch.where(scale[:, None, :, None] > 0, x / scale[:, None, :, None].clamp_min(1e-30), torch.zeros_like(x))
    return q.to(torch.float8_e4m3fn), scale.contiguous()


def dequantize_kv_fp8(cache8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 values the fp8 cache stands for: ``float(byte) * scale[blk, h]``."""
    return cache8.float() * scale[:, None, :, None].float()


def make_case(cfg: DecodeConfig | str, seed: int | None = None, *, ctx_override: list[int] | None = None,
              batch_override: int | None = None) -> DecodeCase:
    """Generate one seeded case on the CPU (deterministic across machines)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    if batch_override is not None:
        cfg = DecodeConfig(**{**cfg.__dict__, "batch": batch_override})
    seed = SEED_BASE + cfg.index if seed is None else seed
    gen = torch.Generator("cpu").manual_seed(seed)
    bsz, bs = cfg.batch, cfg.block_size
    # 1. context lengths
    if ctx_override is not None:
        lens = torch.tensor(ctx_override, dtype=torch.int32)
        if lens.numel() != bsz:
            raise ValueError("ctx_override must have one length per sequence")
    elif cfg.ctx_min == cfg.ctx_max:
        lens = torch.full((bsz,), cfg.ctx_max, dtype=torch.int32)
    else:
        lens = torch.randint(cfg.ctx_min, cfg.ctx_max + 1, (bsz,), generator=gen, dtype=torch.int32)
    nblk_seq = [(int(n) + bs - 1) // bs for n in lens]
    max_blocks = cfg.max_blocks or max(math.ceil(cfg.ctx_max / bs), max(nblk_seq))
    # 2. block table: random non-overlapping assignment from the pool
    if cfg.pool.startswith("fixed:"):
        pool = int(cfg.pool.split(":")[1])
    else:
        pool = sum(nblk_seq)
    if sum(nblk_seq) > pool:
        raise ValueError("pool too small for the context lengths")
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    table = torch.zeros((bsz, max_blocks), dtype=torch.int32)
    off = 0
    for b, n in enumerate(nblk_seq):
        table[b, :n] = perm[off : off + n]
        off += n
    # 3-5. Q, K, V
    qshape = (bsz, cfg.q_len, cfg.num_heads, cfg.head_dim_k) if cfg.q_len > 1 else (bsz, cfg.num_heads,
                                                                                     cfg.head_dim_k)
    query = _randn_bf16(qshape, gen)
    key = _randn_bf16((pool, bs, cfg.kv_heads, cfg.head_dim_k), gen)
    if cfg.mla:
        value = key[..., : cfg.head_dim_v]
    else:
        value = _randn_bf16((pool, bs, cfg.kv_heads, cfg.head_dim_v), gen)
    case = DecodeCase(cfg, seed, query, key, value, table, lens, 1.0 / math.sqrt(cfg.head_dim_k))
    if cfg.kv_format == "fp8":
        case.key_cache, case.k_scale = quantize_kv_fp8(key)
        case.value_cache, case.v_scale = quantize_kv_fp8(value)
    return case


def make_custom_case(*, batch: int, num_heads: int, kv_heads: int, head_dim: int, block_size: int,
                     context_lens: list[int], seed: int, q_len: int = 1, causal: bool = False,
                     head_dim_v: int | None = None, mla: bool = False, max_blocks: int | None = None,
                     pool_extra: int = 0, scale: float | None = None, value_range: float | None = None,
                     dtype: torch.dtype = torch.bfloat16) -> DecodeCase:
    """Arbitrary-shape case (tests): same draw order, pool = blocks needed + ``pool_extra``;
    query and caches in ``dtype`` (bf16, or fp16 for the reference's GQA dtype)."""
    dv = head_dim_v or head_dim
    cfg = DecodeConfig("custom", -1, batch, num_heads, kv_heads, head_dim, dv, block_size,
                       min(context_lens), max(context_lens), q_len=q_len, causal=causal, mla=mla,
                       max_blocks=max_blocks or max(1, math.ceil(max(context_lens) / block_size)))
    gen = torch.Generator("cpu").manual_seed(seed)
    lens = torch.tensor(context_lens, dtype=torch.int32)
    nblk_seq = [(int(n) + block_size - 1) // block_size for n in context_lens]
    pool = max(1, sum(nblk_seq) + pool_extra)
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    table = torch.zeros((batch, cfg.max_blocks), dtype=torch.int32)
    off = 0
    for b, n in enumerate(nblk_seq):
        table[b, :n] = perm[off : off + n]
        off += n
    qshape = (batch, q_len, num_heads, head_dim) if q_len > 1 else (batch, num_heads, head_dim)
    query = _randn_bf16(qshape, gen, dtype)
    key = _randn_bf16((pool, block_size, kv_heads, head_dim), gen, dtype)
    value = key[..., :dv] if mla else _randn_bf16((pool, block_size, kv_heads, dv), gen, dtype)
    if value_range is not None:
        query, key = (query.float() * value_range).to(dtype), (key.float() * value_range).to(dtype)
        if mla:
            value = key[..., :dv]
    return DecodeCase(cfg, seed, query, key, value, table, lens,
                      scale if scale is not None else 1.0 / math.sqrt(head_dim))


def make_reference_case(params: dict, seed: int) -> DecodeCase:
    """Inputs drawn the way the reference's scene tests draw them
    (``simpler_setup/goldens/paged_attention.py:30-88``), seeded:

    * ``context_lens``: ``context_len`` for every sequence, or
      ``context_lens_list`` cycled to the batch;
    * ``block_table [B, max_model_len // block_size]``: uniform block ids in
      ``[0, B * ceil(max_len / block_size))``, drawn with replacement (sequences
      may share blocks; entries past a sequence's length are never read);
    * query, key ~ U(-0.5, 0.5), value ~ U(-1, 1), rounded to ``dtype``
      (bfloat16 here); scale 1.0, as the reference's inputs and golden use.

    ``params`` takes the reference's case keys (``batch``, ``num_heads``,
    ``kv_head_num``, ``head_dim``, ``block_size``, ``context_len``,
    ``max_model_len``, optional ``context_lens_list`` and ``dtype``: "bfloat16"
    or "float16")."""
    batch, hq, hkv = params["batch"], params["num_heads"], params["kv_head_num"]
    dtype = getattr(torch, params.get("dtype", "bfloat16"))
    d, bs = params["head_dim"], params["block_size"]
    gen = torch.Generator("cpu").manual_seed(seed)
    lst = params.get("context_lens_list")
    if lst is not None:
        vals = (list(lst) * ((batch + len(lst) - 1) // len(lst)))[:batch]
        lens = torch.tensor(vals, dtype=torch.int32)
    else:
        lens = torch.full((batch,), params["context_len"], dtype=torch.int32)
    max_blocks = params["max_model_len"] // bs
    total = batch * ((int(lens.max()) + bs - 1) // bs)
    table = torch.randint(0, max(total, 1), (batch, max_blocks), generator=gen, dtype=torch.int32)

    def uni(shape, lo, hi):
        return (torch.rand(shape, generator=gen, dtype=torch.float32) * (hi - lo) + lo).to(dtype)

    query = uni((batch, hq, d), -0.5, 0.5)
    key = uni((total, bs, hkv, d), -0.5, 0.5)
    value = uni((total, bs, hkv, d), -1.0, 1.0)
    cfg = DecodeConfig("reference", -1, batch, hq, hkv, d, d, bs, int(lens.min()), int(lens.max()),
                       max_blocks=max_blocks, out_dtype=torch.float32)
    return DecodeCase(cfg, seed, query, key, value, table, lens, 1.0)


# Tiling-tensor layout of the reference's high-performance SPMD paged attention
# (tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention_highperf/kernels/
# pa_tiling.py:18-62,360-430): int32 header words, then per sequence
# TILING_PARA_SIZE words, word 1 of which is its KV length.
TILING_HEAD_SIZE, TILING_PARA_SIZE = 44, 17


def highperf_tiling(*, batch: int, num_heads: int, kv_heads: int, head_dim: int, num_blocks: int, block_size: int,
                    max_blocks: int, scale: float, kv_seq_lens: list[int]) -> torch.Tensor:
    """The header and per-sequence words of the reference's tiling tensor that
    describe the problem (batch, heads, head dim, blocks, scale, KV lengths);
    the reference's core-split fields (which its own kernel reads to divide
    work among AICores) are left 0."""
    import struct

    t = [0] * (TILING_HEAD_SIZE + batch * TILING_PARA_SIZE)
    t[0], t[1], t[2], t[3], t[4], t[5] = batch, num_heads, head_dim, num_blocks, block_size, max_blocks
    t[6] = struct.unpack("<i", struct.pack("<f", float(scale)))[0]  # TOR: the scale's fp32 bits
    t[7] = kv_heads
    t[17], t[18] = TILING_HEAD_SIZE, TILING_PARA_SIZE
    t[22] = max(kv_seq_lens) if kv_seq_lens else 0  # max KV length
    t[28] = batch  # decoder batch
    t[29] = head_dim  # head dim of V
    for b, n in enumerate(kv_seq_lens):
        base = TILING_HEAD_SIZE + b * TILING_PARA_SIZE
        t[base + 0] = 1  # query tokens
        t[base + 1] = int(n)  # KV length
        t[base + 3] = block_size
        t[base + 8] = b
    return torch.tensor(t, dtype=torch.int32)


def make_highperf_case(params: dict, seed: int) -> tuple[DecodeCase, torch.Tensor]:
    """Inputs drawn the way the reference's high-performance SPMD scene test
    draws them (``test_spmd_paged_attention_highperf.py:28-54,289-347``),
    seeded: query and dense K/V ~ N(0, 1) in ``dtype`` (float16), K/V packed
    into a paged pool ``[B * L/BS, BS, Hkv, D]`` whose block table is the
    identity assignment, every length ``kv_seq``, scale 1/sqrt(D). Returns the
    case and its tiling tensor."""
    batch, hq, hkv, d = params["batch"], params["num_heads"], params["num_kv_heads"], params["head_dim"]
    seq, bs = params["kv_seq"], params["block_size"]
    dtype = getattr(torch, params.get("dtype", "float16"))
    gen = torch.Generator("cpu").manual_seed(seed)
    query = torch.randn(batch, hq, d, generator=gen).to(dtype)
    k_dense = torch.randn(batch, seq, hkv * d, generator=gen).to(dtype)
    v_dense = torch.randn(batch, seq, hkv * d, generator=gen).to(dtype)
    nblk = seq // bs
    key = k_dense.reshape(batch * nblk, bs, hkv, d).contiguous()
    value = v_dense.reshape(batch * nblk, bs, hkv, d).contiguous()
    table = (torch.arange(nblk, dtype=torch.int32)[None, :] + torch.arange(batch, dtype=torch.int32)[:, None] * nblk)
    lens = torch.full((batch,), seq, dtype=torch.int32)
    scale = 1.0 / math.sqrt(d)
    cfg = DecodeConfig("highperf", -1, batch, hq, hkv, d, d, bs, seq, seq, max_blocks=nblk, out_dtype=dtype)
    case = DecodeCase(cfg, seed, query, key, value, table.contiguous(), lens, scale)
    tiling = highperf_tiling(batch=batch, num_heads=hq, kv_heads=hkv, head_dim=d, num_blocks=batch * nblk,
                             block_size=bs, max_blocks=nblk, scale=scale, kv_seq_lens=[seq] * batch)
    return case, tiling


# ---------------------------------------------------------------------------
# Roofline accounting
# ---------------------------------------------------------------------------


def algorithmic_bytes(case: DecodeCase, out_bytes: int = 2) -> int:
    """HBM bytes the op must move at minimum.

    K and V of the valid tokens (MLA: K only, V is a prefix of K), the query,
    the output, the used block-table entries and the lengths. Split-K workspace
    traffic is not counted.
    """
    c = case.config
    lens = [int(x) for x in case.context_lens.tolist()]
    tok = sum(lens)
    kv_cols = c.head_dim_k if c.mla else c.head_dim_k + c.head_dim_v
    kv = tok * c.kv_heads * kv_cols * (1 if case.fp8 else 2)
    if case.fp8:  # one K and one V scale per (visited block, kv head)
        kv += 8 * c.kv_heads * sum((n + c.block_size - 1) // c.block_size for n in lens)
    q = c.batch * c.q_len * c.num_heads * c.head_dim_k * 2
    o = c.batch * c.q_len * c.num_heads * c.head_dim_v * out_bytes
    tables = 4 * sum((n + c.block_size - 1) // c.block_size for n in lens) + 4 * c.batch
    return kv + q + o + tables


def kv_bytes(case: DecodeCase) -> int:
    c = case.config
    tok = sum(int(x) for x in case.context_lens.tolist())
    kv_cols = c.head_dim_k if c.mla else c.head_dim_k + c.head_dim_v
    return tok * c.kv_heads * kv_cols * (1 if case.fp8 else 2)


def algorithmic_flops(case: DecodeCase) -> int:
    """QKᵀ + PV multiply-adds ×2 over unmasked (row, token) pairs."""
    c = case.config
    total = 0
    for n in (int(x) for x in case.context_lens.tolist()):
        if c.causal:
            pairs = sum(n - (c.q_len - 1 - i) for i in range(c.q_len))
        else:
            pairs = c.q_len * n
        total += pairs * c.num_heads * 2 * (c.head_dim_k + c.head_dim_v)
    return total


# ---------------------------------------------------------------------------
# Decode-layer prelude inputs (the KV-append step before attention)
# ---------------------------------------------------------------------------


def rope_tables(max_position: int, head_dim: int, theta: float = 1.0e4) -> tuple[torch.Tensor, torch.Tensor]:
    """RoPE tables ``[max_position, head_dim]`` fp32 with both halves sharing the angles,
    as simpler's Qwen3 decode inputs build them (``goldens/qwen3_14b_decode.py:149-153``)."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half).float() / half))
    ang = torch.arange(max_position).float().unsqueeze(1) * inv_freq.unsqueeze(0)
    return torch.cat([ang.cos(), ang.cos()], dim=1).float(), torch.cat([ang.sin(), ang.sin()], dim=1).float()


def current_token_slots(block_table: torch.Tensor, seq_lens: torch.Tensor, block_size: int) -> torch.Tensor:
    """Slot of each sequence's current token (position ``seq_len - 1``):
    ``block_table[b, p // block_size] * block_size + p % block_size``
    (``goldens/qwen3_14b_decode.py:106-115``)."""
    pos = seq_lens.long() - 1
    phys = block_table[torch.arange(len(pos)), pos // block_size].long()
    return (phys * block_size + pos % block_size).to(torch.int32)
