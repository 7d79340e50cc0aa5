"""Pins for the KV-append / decode-prelude oracle (CPU only).

Each check is a closed form or an independent evaluation, chosen so that a
plausible slip in ``oracle/kv_oracle.py`` (wrong slot arithmetic, swapped RoPE
halves or sign, a missing eps or weight, a wrong reduction axis) fails one of them.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kv_oracle as ko


def _identity_paging(batch: int, max_blocks: int, seq_lens: np.ndarray, bs: int):
    # goldens/qwen3_14b_decode.py:106-115: page b*max_blocks + logical block
    table = np.arange(batch * max_blocks, dtype=np.int32).reshape(batch, max_blocks)
    pos = seq_lens - 1
    expect = ((np.arange(batch) * max_blocks + pos // bs) * bs + pos % bs).astype(np.int32)
    return table, expect


def test_slot_of_matches_reference_identity_paging():
    seq_lens = np.array([1, 128, 129, 3500, 5500], dtype=np.int32)
    table, expect = _identity_paging(5, 43, seq_lens, 128)
    np.testing.assert_array_equal(ko.slot_of(table, seq_lens, 128), expect)


def test_new_token_slots_extend_the_reference_slot():
    seq_lens = np.array([1, 3, 128, 129, 3500], dtype=np.int32)
    table, expect = _identity_paging(5, 43, seq_lens, 128)
    # one new token: the reference's current-token slot
    np.testing.assert_array_equal(ko.new_token_slots(table, seq_lens, 128, 1)[:, 0], expect)
    # four: positions len-4 .. len-1 under identity paging (page b*43 + pos//128), -1 below position 0
    got = ko.new_token_slots(table, seq_lens, 128, 4)
    for b, n in enumerate(seq_lens.tolist()):
        for j in range(4):
            p = n - 4 + j
            assert got[b, j] == ((b * 43 + p // 128) * 128 + p % 128 if p >= 0 else -1)
    # a shuffled table: each slot's block is the table entry of the position's logical block
    rng = np.random.default_rng(3)
    shuffled = rng.permutation(5 * 43).astype(np.int32).reshape(5, 43)
    got = ko.new_token_slots(shuffled, seq_lens, 128, 2)
    assert got[3, 0] == shuffled[3, 0] * 128 + 127 and got[3, 1] == shuffled[3, 1] * 128


def test_new_token_slots_past_the_table_row_are_dropped():
    # a row of 3 blocks of 16 holds positions 0..47: a length of 50 with 4 new
    # tokens puts them at 46..49, of which 46 and 47 fit
    table = np.array([[5, 2, 9], [1, 0, 4]], dtype=np.int32)
    got = ko.new_token_slots(table, np.array([50, 48], dtype=np.int32), 16, 4)
    np.testing.assert_array_equal(got[0], [9 * 16 + 14, 9 * 16 + 15, -1, -1])
    np.testing.assert_array_equal(got[1], [4 * 16 + 12, 4 * 16 + 13, 4 * 16 + 14, 4 * 16 + 15])
    # far past the row: nothing fits
    np.testing.assert_array_equal(ko.new_token_slots(table, np.array([10_000, 1], dtype=np.int32), 16, 2)[0],
                                  [-1, -1])


def test_append_writes_exactly_the_slots():
    rng = np.random.default_rng(1)
    nblk, bs, hkv, d = 12, 16, 3, 8
    kc = rng.integers(0, 1 << 16, size=(nblk, bs, hkv, d), dtype=np.uint16)
    vc = rng.integers(0, 1 << 16, size=(nblk, bs, hkv, d), dtype=np.uint16)
    key = rng.integers(0, 1 << 16, size=(4, hkv, d), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, size=(4, hkv, d), dtype=np.uint16)
    slots = np.array([0, 17, -1, nblk * bs - 1], dtype=np.int32)
    k2, v2 = ko.kv_append(kc, vc, key, val, slots)
    # flat row view of the reference: row = slot * kv_heads + kv_head
    kflat = k2.reshape(-1, d)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        for h in range(hkv):
            np.testing.assert_array_equal(kflat[s * hkv + h], key[t, h])
            np.testing.assert_array_equal(v2.reshape(-1, d)[s * hkv + h], val[t, h])
    # nothing else changed (3 written tokens x kv_heads x d), padding token skipped
    assert int(np.count_nonzero(k2 != kc)) <= 3 * hkv * d
    assert np.array_equal(np.delete(k2.reshape(-1, d), [s * hkv + h for s in (0, 17, nblk * bs - 1)
                                                       for h in range(hkv)], axis=0),
                          np.delete(kc.reshape(-1, d), [s * hkv + h for s in (0, 17, nblk * bs - 1)
                                                       for h in range(hkv)], axis=0))


def test_rope_identity_and_quarter_turn():
    rng = np.random.default_rng(2)
    v = rng.standard_normal((3, 8)).astype(np.float32)
    one, zero = np.ones((3, 8), np.float32), np.zeros((3, 8), np.float32)
    np.testing.assert_array_equal(ko.rope_half(v, one, zero), v)
    np.testing.assert_array_equal(ko.rope_half(v, zero, one), np.concatenate([-v[:, 4:], v[:, :4]], axis=1))


def test_rope_with_reference_tables_rotates_pairs():
    cos, sin = ko.rope_tables(64, 16)
    assert cos.shape == (64, 16) and np.array_equal(cos[:, :8], cos[:, 8:])
    np.testing.assert_allclose(cos[0], 1.0) and np.testing.assert_allclose(sin[0], 0.0)
    rng = np.random.default_rng(3)
    v = rng.standard_normal((64, 16)).astype(np.float32)
    r = ko.rope_half(v, cos, sin)
    np.testing.assert_allclose(r[:, :8] ** 2 + r[:, 8:] ** 2, v[:, :8] ** 2 + v[:, 8:] ** 2, rtol=1e-5, atol=1e-6)
    # position 1, pair 0 rotates by exactly 1 radian
    np.testing.assert_allclose(r[1, 0], v[1, 0] * np.cos(1.0) - v[1, 8] * np.sin(1.0), rtol=1e-6)


@pytest.mark.parametrize("c", [0.5, -3.0, 1e-4])
def test_rms_norm_of_a_constant(c):
    x = np.full((2, 16), c, dtype=np.float32)
    np.testing.assert_allclose(x * ko.rms_inv(x), c / np.sqrt(c * c + ko.EPS), rtol=1e-6)


def test_rms_norm_against_fp64():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 7, 128)).astype(np.float32) * 3
    ref = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True) + ko.EPS)
    np.testing.assert_allclose(ko.rms_inv(x), ref, rtol=2e-6)


def test_prelude_shapes_weights_and_positions():
    rng = np.random.default_rng(5)
    b, hq, hkv, d = 3, 4, 2, 16
    qp = rng.standard_normal((b, hq * d)).astype(np.float32)
    kp = rng.standard_normal((b, hkv * d)).astype(np.float32)
    vp = rng.standard_normal((b, hkv * d)).astype(np.float32)
    ir = np.array([0.5, 1.0, 2.0], np.float32)
    qw = np.full(d, 2.0, np.float32)
    kw = np.ones(d, np.float32)
    cos, sin = ko.rope_tables(32, d)
    seq = np.array([1, 5, 32], np.int32)
    q, k, v = ko.qk_norm_rope(qp, kp, vp, ir, qw, kw, cos, sin, seq, hq, hkv)
    qf, kf, vf = (ko.bf16_bits_to_f32(x) for x in (q, k, v))
    # v is only scaled by inv_rms (then rounded)
    np.testing.assert_array_equal(v, ko.f32_to_bf16_bits(vp.reshape(b, hkv, d) * ir[:, None, None]))
    # sequence 0 is at position 0: no rotation, so q = 2 * rms-normalised q_proj (inv_rms cancels)
    qn = qp[0].reshape(hq, d) / np.sqrt(np.mean(qp[0].reshape(hq, d).astype(np.float64) ** 2, -1,
                                                 keepdims=True) + ko.EPS / 0.25)
    np.testing.assert_allclose(qf[0], 2.0 * qn, rtol=8e-3, atol=1e-6)
    # rotation keeps every pair's norm: |k| per head equals the unrotated normalised |k| (bf16 rounding aside)
    kn = kp.reshape(b, hkv, d) * ir[:, None, None]
    kn = kn / np.sqrt(np.mean(kn.astype(np.float64) ** 2, -1, keepdims=True) + ko.EPS)
    np.testing.assert_allclose(np.linalg.norm(kf, axis=-1), np.linalg.norm(kn, axis=-1), rtol=8e-3)


def test_input_helpers_agree_with_the_oracle():
    # the product-side input builders (simpler_amd.workloads) and the oracle's own
    import torch

    from simpler_amd.workloads import current_token_slots, rope_tables
    cos, sin = rope_tables(300, 64)
    ocos, osin = ko.rope_tables(300, 64)
    # angles up to ~300 rad are fp32 (ulp 3e-5); torch and numpy evaluate cos/sin with different libraries
    np.testing.assert_allclose(cos.numpy(), ocos, rtol=0, atol=1e-4)
    np.testing.assert_allclose(sin.numpy(), osin, rtol=0, atol=1e-4)
    seq = np.array([1, 128, 129, 300], np.int32)
    table = np.random.default_rng(6).permutation(40).astype(np.int32).reshape(4, 10)
    np.testing.assert_array_equal(current_token_slots(torch.from_numpy(table), torch.from_numpy(seq), 32).numpy(),
                                  ko.slot_of(table, seq, 32))
