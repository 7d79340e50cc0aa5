"""Seeded random shapes through the decode entry against the oracle.

Each case draws a valid configuration: GQA (head dim 16–256, block size
16–128, 1–8 kv heads, group 1–16, q_len 1–8 with or without the causal mask,
bf16 or fp16, fp32 or input-dtype output), MLA (Dk 576 / Dv 512, block size 32
or 64, 16–192 heads) or fp8 E4M3FN caches; 1–12 sequences with lengths up to
4,000 tokens, some empty; 0 (the default), 1, 3, 17, 200 or 2,000 workers;
every other case with K and V in one allocation (kv_cache.alloc_kv_pools).
Tolerance: the decode tolerance (max-abs 2e-2, rel-L2 1e-3) against the numpy
oracle, or against the oracle on the dequantised caches for fp8. The fused
append entry gets its own seeded sweep.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import pa_oracle as po
from simpler_amd import paged_attention as pa
from simpler_amd.workloads import make_custom_case, quantize_kv_fp8
from tests.pa_helpers import assert_close, oracle_numpy

pytestmark = pytest.mark.gpu


def _draw(rng: random.Random, i: int, seed: int):
    kind = rng.choice(["gqa"] * 6 + ["mla", "fp8"])
    d, bs = rng.choice([16, 32, 64, 128, 256]), rng.choice([16, 32, 64, 128])
    hkv, g = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 3, 4, 5, 8, 16])
    q_len = rng.choice([1, 1, 1, 2, 4, 8])
    causal = q_len > 1 and rng.random() < 0.8
    batch = rng.randint(1, 12)
    maxl = rng.choice([64, 300, 1500, 4000])
    lens = [rng.randint(q_len if causal else 0, maxl) for _ in range(batch)]
    if rng.random() < 0.2:
        lens[rng.randrange(batch)] = q_len if causal else 0
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    out_dtype = rng.choice([torch.float32, dtype])
    workers = rng.choice([0, 0, 0, 1, 3, 17, 200, 2000])
    if kind == "mla":
        d, bs, hkv, g, dtype = 576, rng.choice([32, 64]), 1, rng.choice([16, 64, 100, 128, 192]), torch.bfloat16
        q_len = rng.choice([1, 1, 2, 4])
        causal = q_len > 1 and rng.random() < 0.8
        lens = [rng.randint(q_len if causal else 0, rng.choice([64, 700, 2000])) for _ in range(batch)]
        out_dtype = rng.choice([torch.float32, torch.bfloat16])
    elif kind == "fp8":
        d, dtype = 128, torch.bfloat16
        out_dtype = rng.choice([torch.float32, torch.bfloat16])
    case = make_custom_case(batch=batch, num_heads=hkv * g, kv_heads=hkv, head_dim=d, block_size=bs, q_len=q_len,
                            causal=causal, context_lens=lens, seed=seed * 1000 + i, dtype=dtype,
                            head_dim_v=512 if kind == "mla" else None, mla=kind == "mla")
    desc = (f"#{i} {kind} d={d} bs={bs} hkv={hkv} g={g} q={q_len} causal={causal} B={batch} lens={lens} "
            f"{dtype} out={out_dtype} w={workers}")
    return kind, case, causal, out_dtype, workers, desc


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_random_shapes_match_the_oracle(seed, device):
    rng = random.Random(seed)
    for i in range(60):
        kind, case, causal, out_dtype, workers, desc = _draw(rng, i, seed)
        print(f"[case] seed {seed} {desc}", flush=True)
        kw = {}
        if kind == "fp8":
            case.key_cache, case.k_scale = quantize_kv_fp8(case.key_cache, pow2=False)
            case.value_cache, case.v_scale = quantize_kv_fp8(case.value_cache, pow2=False)
            k = po.dequantize_kv(case.key_cache.view(torch.uint8).numpy(), case.k_scale.numpy())
            v = po.dequantize_kv(case.value_cache.view(torch.uint8).numpy(), case.v_scale.numpy())
            ref = po.paged_attention_decode(case.query.float().numpy(), k, v, case.block_table.numpy(),
                                            case.context_lens.numpy(), case.scale, causal=causal)
        else:
            ref = oracle_numpy(case)
        dc = case.to(device, kv_pool=i % 2 == 1)  # every other case: K and V in one allocation
        if kind == "fp8":
            kw = dict(k_scale=dc.k_scale, v_scale=dc.v_scale)
        out = torch.empty(case.out_shape(), dtype=out_dtype, device=device)
        pa.paged_attention_decode(dc.query, dc.key_cache, dc.value_cache, dc.block_table, dc.context_lens, out,
                                  case.scale, causal=causal, num_workers=workers, **kw)
        torch.cuda.synchronize(device)
        pa.check_errors(device)
        if out_dtype != torch.float32:
            ref = torch.tensor(ref).to(out_dtype).float().numpy()
        assert_close(out.float().cpu().numpy(), np.asarray(ref), what=desc)


@pytest.mark.parametrize("seed", [21])
def test_random_shapes_fused_append(seed, device):
    """Seeded random shapes through the fused append entry: the caches equal
    the oracle's append bit for bit, the output equals the plain decode on
    those caches bit for bit and is within the decode tolerance of the
    oracle (GQA head dims 16–256 in bf16/fp16, MLA, q_len up to 16)."""
    from tests.test_append_gpu import new_tokens, oracle_appended, poison_new_rows, run_decode, u16

    rng = random.Random(seed)
    for i in range(60):
        mla = rng.random() < 0.15
        q_len = rng.choice([1, 1, 2, 4, 8, 16])
        causal = q_len > 1 and rng.random() < 0.8
        batch = rng.randint(1, 8)
        if mla:
            d, bs, hkv, g, dtype = 576, rng.choice([32, 64]), 1, rng.choice([16, 128]), torch.bfloat16
            q_len = min(q_len, 4)
        else:
            d, bs = rng.choice([16, 64, 128, 256]), rng.choice([16, 32, 64, 128])
            hkv, g = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4, 8])
            dtype = rng.choice([torch.bfloat16, torch.float16])
        lens = [rng.randint(q_len, rng.choice([q_len + 3, 200, 1500])) for _ in range(batch)]
        workers = rng.choice([0, 0, 1, 5, 300])
        desc = (f"#{i} {'mla' if mla else 'gqa'} d={d} bs={bs} hkv={hkv} g={g} q={q_len} causal={causal} "
                f"lens={lens} {dtype} w={workers}")
        print(f"[case] append seed {seed} {desc}", flush=True)
        case = make_custom_case(batch=batch, num_heads=hkv * g, kv_heads=hkv, head_dim=d, block_size=bs,
                                q_len=q_len, causal=causal, context_lens=lens, seed=seed * 1000 + i, dtype=dtype,
                                head_dim_v=512 if mla else None, mla=mla)
        k_new, v_new = new_tokens(case, seed * 1000 + i)
        appended = oracle_appended(case, k_new, v_new)
        poison_new_rows(case)
        got, kc, vc = run_decode(case, device, workers, k_new, v_new)
        np.testing.assert_array_equal(u16(kc), u16(appended.key_cache))
        if not mla:
            np.testing.assert_array_equal(u16(vc), u16(appended.value_cache))
        plain, _, _ = run_decode(appended, device, workers)
        np.testing.assert_array_equal(got, plain)
        assert_close(got, oracle_numpy(appended), what=desc)
