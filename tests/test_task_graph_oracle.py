"""Pins for the oracle's per-kernel step functions (CPU only).

``oracle.pa_oracle.{qk_matmul, softmax_prepare, pv_matmul, online_update}`` are
what the task-graph backend's incore kernels are checked against. Each is
pinned here by something other than its own formula: composing the steps block
by block must reproduce the whole-op oracle (itself pinned against the fp64
textbook softmax in test_oracle.py) bit for bit; the softmax step has the
closed forms max(p) = 1 and 1 <= l <= valid_len, and masks; the matmuls agree
with fp64 products; the online update of two blocks equals one softmax over
their union (associativity) in fp64.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pa_oracle as po


def _bf16(rng, *shape, scale=1.0):
    return po.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def test_steps_compose_to_the_whole_op_oracle():
    rng = np.random.default_rng(11)
    b, hq, d, bs, nblk = 2, 16, 64, 32, 10
    q = _bf16(rng, b, hq, d)
    kc = _bf16(rng, nblk, bs, 1, d)
    vc = _bf16(rng, nblk, bs, 1, d)
    table = rng.permutation(nblk).astype(np.int32).reshape(b, nblk // b)
    lens = np.array([bs * 5, bs * 2 + 7], np.int32)
    scale = 1 / np.sqrt(d)
    want = po.paged_attention_decode(q, kc, vc, table, lens, scale)
    for bi in range(b):
        nb = (lens[bi] + bs - 1) // bs
        mi = li = oi = None
        for bn in range(nb):
            blk = table[bi, bn]
            s = po.qk_matmul(q[bi], kc[blk, :, 0])
            p, m, l = po.softmax_prepare(s, min(bs, lens[bi] - bn * bs), scale)
            o = po.pv_matmul(p, vc[blk, :, 0])
            mi, li, oi, dst = po.online_update(m, l, o, mi, li, oi, bn == 0, bn == nb - 1)
        np.testing.assert_array_equal(dst, want[bi])


@pytest.mark.parametrize("valid", [1, 5, 32])
def test_softmax_prepare_closed_forms(valid):
    rng = np.random.default_rng(12 + valid)
    s = (rng.standard_normal((16, 32)) * 4).astype(np.float32)
    p, m, l = po.softmax_prepare(s, valid, 0.5)
    assert np.all(p[:, valid:] == 0)
    np.testing.assert_array_equal(p[:, :valid].max(axis=1), 1.0)  # the max entry is exp(0) = 1
    assert np.all(l >= 1.0) and np.all(l <= valid)
    np.testing.assert_array_equal(m, (s[:, :valid] * np.float32(0.5)).max(axis=1))
    assert np.array_equal(p, po.bf16_round(p))  # on the bf16 grid
    # a constant row spreads evenly: every valid p is exactly 1, l = valid
    p1, _, l1 = po.softmax_prepare(np.full((2, 32), 3.0, np.float32), valid, 1.0)
    assert np.all(p1[:, :valid] == 1.0) and np.all(l1 == valid)


def test_softmax_prepare_empty_block():
    p, m, l = po.softmax_prepare(np.ones((4, 8), np.float32), 0, 1.0)
    assert np.all(p == 0) and np.all(l == 0) and np.all(m == np.float32(-1e30))


def test_matmuls_against_fp64():
    rng = np.random.default_rng(13)
    q, k, v = _bf16(rng, 16, 128), _bf16(rng, 128, 128), _bf16(rng, 128, 128)
    np.testing.assert_allclose(po.qk_matmul(q, k), q.astype(np.float64) @ k.T.astype(np.float64), rtol=1e-5, atol=1e-4)
    p = po.bf16_round(np.abs(rng.standard_normal((16, 128))).astype(np.float32))
    np.testing.assert_allclose(po.pv_matmul(p, v), p.astype(np.float64) @ v.astype(np.float64), rtol=1e-5, atol=1e-4)


def test_online_update_equals_softmax_over_the_union():
    # two blocks merged = softmax over both (p unrounded: fp64, so the only
    # difference is fp32 rounding)
    rng = np.random.default_rng(14)
    s1, s2 = rng.standard_normal((8, 16)) * 3, rng.standard_normal((8, 16)) * 3 + 1
    v1, v2 = rng.standard_normal((16, 24)), rng.standard_normal((16, 24))

    def block(s, v):
        m = s.max(axis=1)
        p = np.exp(s - m[:, None])
        return m.astype(np.float32), p.sum(1).astype(np.float32), (p @ v).astype(np.float32)

    m1, l1, o1 = block(s1, v1)
    m2, l2, o2 = block(s2, v2)
    mi, li, oi, dst = po.online_update(m1, l1, o1, None, None, None, True, False)
    assert dst is None
    _, _, _, dst = po.online_update(m2, l2, o2, mi, li, oi, False, True)
    s = np.concatenate([s1, s2], axis=1)
    w = np.exp(s - s.max(axis=1, keepdims=True))
    want = (w / w.sum(axis=1, keepdims=True)) @ np.concatenate([v1, v2])
    np.testing.assert_allclose(dst, want, rtol=1e-5, atol=1e-6)
    # first-and-last block: o / l
    _, _, _, d1 = po.online_update(m1, l1, o1, None, None, None, True, True)
    np.testing.assert_allclose(d1, o1 / l1[:, None], rtol=0, atol=0)
