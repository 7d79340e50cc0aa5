"""Pins the CPU oracle (oracle/pa_oracle.py and oracle/pa_oracle.c).

The reference ships no golden vectors for paged attention (its goldens are
recomputed from unseeded random inputs, simpler_setup/goldens/paged_attention.py
:68-78), so the oracle is pinned by what the mathematics fixes:

* the fp64 textbook softmax attention (a separate, unrounded formulation)
* closed forms: one token, constant keys, one-hot scores, per-head constant V
* a hand-computed case that only passes if p is rounded to bf16 before the row
  sum and the PV product (goldens/paged_attention.py:164-165)
* masking: values past the context length and unused table entries are ignored
* the fully-masked-block rule m = -1e30 (golden :160) under a causal query
* agreement of the two independent restatements (numpy and C)
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import pa_oracle
from simpler_amd.workloads import make_custom_case
from tests.pa_helpers import assert_close, oracle_c, oracle_numpy

SMALL_CASES = {
    # reference-style cases (test_paged_attention.py CaseSmall1 / CaseVarSeq2 / CaseVarSeq4)
    "case_small1": dict(batch=1, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[33]),
    "case_varseq2": dict(batch=2, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[33, 17]),
    "case_varseq4": dict(batch=4, num_heads=16, kv_heads=1, head_dim=16, block_size=16,
                         context_lens=[33, 64, 128, 15]),
    "gqa": dict(batch=2, num_heads=8, kv_heads=2, head_dim=32, block_size=16, context_lens=[40, 7]),
    "gqa_bs128": dict(batch=2, num_heads=8, kv_heads=2, head_dim=64, block_size=128, context_lens=[300, 129]),
    "causal": dict(batch=2, num_heads=4, kv_heads=2, head_dim=32, block_size=16, context_lens=[20, 35], q_len=3,
                   causal=True),
    "causal_masked_block": dict(batch=1, num_heads=2, kv_heads=1, head_dim=16, block_size=16, context_lens=[33],
                                q_len=4, causal=True),
    "mla": dict(batch=2, num_heads=8, kv_heads=1, head_dim=64, head_dim_v=48, block_size=16,
                context_lens=[30, 50], mla=True),
}


@pytest.mark.parametrize("name", sorted(SMALL_CASES))
def test_oracle_matches_fp64_textbook(name):
    case = make_custom_case(seed=7, **SMALL_CASES[name])
    c = case.config
    got = oracle_numpy(case)
    ref = pa_oracle.attention_fp64(
        case.query.float().numpy(), case.key_cache.float().numpy(),
        None if c.mla else case.value_cache.float().numpy(), case.block_table.numpy(),
        case.context_lens.numpy(), case.scale, causal=c.causal, v_dim=c.head_dim_v if c.mla else None)
    # bf16 rounding of p (relative 2^-9) is the only deviation from the textbook
    assert_close(got, ref, max_abs=2e-2, rel_l2=5e-3, what=name)
    # ...and it is there: the oracle is not the unrounded softmax
    assert np.max(np.abs(got - ref)) > 1e-7


@pytest.mark.parametrize("name", sorted(SMALL_CASES))
def test_c_restatement_matches_numpy(name):
    case = make_custom_case(seed=11, **SMALL_CASES[name])
    assert_close(oracle_c(case, n_threads=2), oracle_numpy(case), max_abs=2e-3, rel_l2=1e-4, what=name)


def test_single_token_returns_first_value_row():
    case = make_custom_case(batch=3, num_heads=4, kv_heads=2, head_dim=32, block_size=16, context_lens=[1, 1, 1],
                            seed=3)
    out = oracle_numpy(case)
    v = case.value_cache.float().numpy()
    for b in range(3):
        blk = int(case.block_table[b, 0])
        for h in range(4):
            np.testing.assert_array_equal(out[b, h], v[blk, 0, h // 2])


def test_constant_keys_give_mean_of_values():
    case = make_custom_case(batch=2, num_heads=4, kv_heads=1, head_dim=32, block_size=16, context_lens=[37, 50],
                            seed=5)
    case.key_cache[:] = case.key_cache[0, 0]  # every token has the same key
    out = oracle_numpy(case)
    v = case.value_cache.float().numpy().astype(np.float64)
    for b, n in enumerate([37, 50]):
        rows = np.concatenate([v[int(case.block_table[b, j]), :, 0, :] for j in range((n + 15) // 16)])[:n]
        np.testing.assert_allclose(out[b], np.broadcast_to(rows.mean(axis=0), out[b].shape), atol=1e-6)


@pytest.mark.parametrize("shape", ["gqa", "gqa_causal_q4", "mla"])
def test_scale_zero_gives_mean_of_visible_values(shape):
    # scale 0: every visible score is 0, p = bf16(e^0) = 1 exactly, so row r of
    # query token i is the plain mean of the V rows it sees. With a causal
    # multi-token query, token i sees ctx - (q_len - 1 - i) tokens: an
    # off-by-one in that window, or a wrong kv head (h // g), fails here.
    lens = [5, 37, 50]
    if shape == "gqa":
        case = make_custom_case(batch=3, num_heads=8, kv_heads=2, head_dim=32, block_size=16, context_lens=lens,
                                seed=31, scale=0.0)
    elif shape == "gqa_causal_q4":
        case = make_custom_case(batch=3, num_heads=8, kv_heads=2, head_dim=32, block_size=16, context_lens=lens,
                                seed=32, scale=0.0, q_len=4, causal=True)
    else:
        case = make_custom_case(batch=3, num_heads=4, kv_heads=1, head_dim=64, head_dim_v=48, block_size=16,
                                context_lens=lens, seed=33, scale=0.0, mla=True)
    c = case.config
    out = oracle_numpy(case)
    v_all = (case.key_cache.float().numpy()[..., : c.head_dim_v] if c.mla else case.value_cache.float().numpy())
    g = c.num_heads // c.kv_heads
    for b, n in enumerate(lens):
        rows = np.concatenate([v_all[int(case.block_table[b, j])] for j in range((n + 15) // 16)])[:n]
        for i in range(c.q_len):
            seen = n - (c.q_len - 1 - i) if c.causal else n
            for h in range(c.num_heads):
                want = rows[:seen, h // g].astype(np.float64).mean(axis=0)
                got = out[b, i, h] if c.q_len > 1 else out[b, h]
                np.testing.assert_allclose(got, want, atol=1e-6, err_msg=f"{shape} b{b} token{i} head{h}")


def test_one_hot_scores_select_one_value():
    case = make_custom_case(batch=1, num_heads=2, kv_heads=1, head_dim=16, block_size=16, context_lens=[40], seed=9,
                            scale=1.0)
    case.query.zero_()
    case.query[..., 0] = 1.0
    case.key_cache.zero_()
    target = 23  # token 23 lives in logical block 1, row 7
    blk = int(case.block_table[0, 1])
    case.key_cache[blk, 7, 0, 0] = 100.0
    out = oracle_numpy(case)
    np.testing.assert_array_equal(out[0, 0], case.value_cache[blk, 7, 0].float().numpy())
    assert target == 16 + 7


def test_p_is_rounded_to_bf16_before_sum_and_pv():
    # s0 = 0 (block max), s1 = -0.2138671875: exp(s1) = 0.807455... rounds to 207/256 in bf16.
    case = make_custom_case(batch=1, num_heads=1, kv_heads=1, head_dim=16, block_size=16, context_lens=[2], seed=1,
                            scale=1.0)
    case.query.zero_()
    case.query[0, 0, 0] = 1.0
    blk = int(case.block_table[0, 0])
    case.key_cache.zero_()
    case.key_cache[blk, 1, 0, 0] = -0.2138671875
    case.value_cache.zero_()
    case.value_cache[blk, 1, 0, 0] = 1.0
    out = oracle_numpy(case)
    assert out[0, 0, 0] == pytest.approx(207.0 / 463.0, abs=2e-7)  # (207/256) / (1 + 207/256)
    unrounded = math.exp(-0.2138671875) / (1 + math.exp(-0.2138671875))
    assert abs(out[0, 0, 0] - unrounded) > 3e-4


def test_gqa_head_mapping_uses_h_div_group():
    case = make_custom_case(batch=2, num_heads=12, kv_heads=3, head_dim=16, block_size=16, context_lens=[21, 40],
                            seed=13)
    for j in range(3):
        case.value_cache[:, :, j, :] = float(2 ** j)
    out = oracle_numpy(case)
    for h in range(12):
        np.testing.assert_array_equal(out[:, h], np.full((2, 16), float(2 ** (h // 4)), dtype=np.float32))


def test_tokens_past_context_and_unused_blocks_are_ignored():
    case = make_custom_case(batch=2, num_heads=4, kv_heads=2, head_dim=32, block_size=16, context_lens=[21, 9],
                            seed=17, pool_extra=3, max_blocks=4)
    base = oracle_numpy(case)
    for b, n in enumerate([21, 9]):
        last = int(case.block_table[b, (n - 1) // 16])
        case.key_cache[last, n % 16 or 16 :] = 1e4
        case.value_cache[last, n % 16 or 16 :] = 1e4
    used = set(int(x) for b, n in enumerate([21, 9]) for x in case.block_table[b, : (n + 15) // 16])
    for blk in range(case.key_cache.shape[0]):
        if blk not in used:
            case.key_cache[blk] = 1e4
            case.value_cache[blk] = -1e4
    case.block_table[0, 2:] = 1
    case.block_table[1, 1:] = 2
    np.testing.assert_array_equal(oracle_numpy(case), base)


def test_oracle_rejects_nothing_silently_on_empty_context():
    case = make_custom_case(batch=2, num_heads=2, kv_heads=1, head_dim=16, block_size=16, context_lens=[0, 5],
                            seed=19, max_blocks=1)
    out = oracle_numpy(case)
    assert np.all(out[0] == 0) and np.all(np.isfinite(out))
    np.testing.assert_array_equal(oracle_c(case), out)


def test_bf16_helpers_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, 3.0e38], dtype=np.float32)
    # ties: 1+2^-8 is halfway between 1 and 1+2^-7 -> even (1.0); 1+3*2^-8 -> 1+2^-6
    expect = np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0, -2.5], dtype=np.float32)
    np.testing.assert_array_equal(pa_oracle.bf16_round(x)[:5], expect)
    t = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(pa_oracle.bf16_round(x), t)


# ---- fp16 inputs (the reference's GQA scene cases are fp16; the golden rounds p
# to the input dtype, goldens/paged_attention.py:168) ----------------------------

def test_p_is_rounded_to_fp16_for_fp16_inputs():
    # s0 = 0 (block max), s1 = -0.2138671875 (exact in fp16): exp(s1) = 0.807455...
    # rounds to 1654/2048 in fp16 (spacing 2^-11 on [0.5, 1)), so the output is
    # (1654/2048) / (1 + 1654/2048) = 1654/3702, not the bf16 value 207/463.
    q = np.zeros((1, 1, 16), np.float32)
    q[0, 0, 0] = 1.0
    k = np.zeros((1, 16, 1, 16), np.float32)
    k[0, 1, 0, 0] = -0.2138671875
    v = np.zeros((1, 16, 1, 16), np.float32)
    v[0, 1, 0, 0] = 1.0
    args = (q, k, v, np.zeros((1, 1), np.int32), np.array([2], np.int32), 1.0)
    out16 = pa_oracle.paged_attention_decode(*args, p_dtype="fp16")
    assert out16[0, 0, 0] == pytest.approx(1654.0 / 3702.0, abs=2e-7)
    out_bf = pa_oracle.paged_attention_decode(*args)
    assert out_bf[0, 0, 0] == pytest.approx(207.0 / 463.0, abs=2e-7)
    unrounded = math.exp(-0.2138671875) / (1 + math.exp(-0.2138671875))
    assert abs(out16[0, 0, 0] - unrounded) > 3e-5


def test_fp16_round_matches_torch():
    g = torch.Generator().manual_seed(5)
    x = torch.cat([torch.randn(4096, generator=g), torch.randn(512, generator=g) * 1e-6,  # fp16 subnormals
                   torch.tensor([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2 ** -24 * 0.5, 2 ** -24 * 1.5, 65504.0])])
    got = pa_oracle.fp16_round(x.numpy())
    want = x.to(torch.float16).float().numpy()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("name", ["gqa", "gqa_bs128", "causal", "case_varseq4"])
def test_fp16_oracle_matches_fp64_textbook(name):
    case = make_custom_case(seed=8, dtype=torch.float16, **SMALL_CASES[name])
    c = case.config
    got = oracle_numpy(case)
    ref = pa_oracle.attention_fp64(
        case.query.float().numpy(), case.key_cache.float().numpy(), case.value_cache.float().numpy(),
        case.block_table.numpy(), case.context_lens.numpy(), case.scale, causal=c.causal)
    # fp16 rounding of p (relative 2^-11) is the only deviation from the textbook
    assert_close(got, ref, max_abs=5e-3, rel_l2=1.5e-3, what=name)
    assert np.max(np.abs(got - ref)) > 1e-8
    # and it differs from the bf16-rounded recipe on the same values
    bf = pa_oracle.paged_attention_decode(
        case.query.float().numpy(), case.key_cache.float().numpy(), case.value_cache.float().numpy(),
        case.block_table.numpy(), case.context_lens.numpy(), case.scale, causal=c.causal, p_dtype="bf16")
    assert np.max(np.abs(got - bf)) > 1e-6
