"""GPU parity of the KV-cache append and the fused decode prelude (through the C ABI).

* ``simpler_hip_kv_append`` is byte movement: bit-exact against the oracle, for
  the written rows and for every untouched cache element (random bit patterns,
  NaN patterns included), with padding (-1) and out-of-pool slots.
* ``simpler_hip_qk_norm_rope_append`` is fp32 arithmetic rounded to bf16: the
  sum of squares is reduced in another order than the golden's mean, so an
  element may land one bf16 step away from the oracle. Tolerance: at most one
  bf16 ulp per element, and such elements are rare (< 2%); untouched cache
  elements are bit-exact.
* The prelude -> append -> decode chain matches the oracle chain within the
  decode tolerance (max-abs 2e-2, rel-L2 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as ko
from simpler_amd import kv_cache as kvc
from simpler_amd import paged_attention as pa
from tests.pa_helpers import assert_close

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _from_bits(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(device)


@pytest.mark.parametrize("hkv,dk,dv,bs,ntok", [(8, 128, 128, 128, 32), (1, 576, None, 64, 20), (2, 16, 24, 16, 7)])
def test_kv_append_bit_exact(hkv, dk, dv, bs, ntok, device):
    print(f"[case] append hkv={hkv} dk={dk} dv={dv} bs={bs} ntok={ntok}", flush=True)
    rng = np.random.default_rng(900 + dk)
    nblk = 3 * ntok // bs + 4
    kc = rng.integers(0, 1 << 16, size=(nblk, bs, hkv, dk), dtype=np.uint16)
    key = rng.integers(0, 1 << 16, size=(ntok, hkv, dk), dtype=np.uint16)
    vc = val = None
    if dv:
        vc = rng.integers(0, 1 << 16, size=(nblk, bs, hkv, dv), dtype=np.uint16)
        val = rng.integers(0, 1 << 16, size=(ntok, hkv, dv), dtype=np.uint16)
    slots = rng.permutation(nblk * bs)[:ntok].astype(np.int32)
    slots[1] = -1                 # padding token
    slots[2] = nblk * bs + 5      # past the pool: skipped and counted
    want_k, want_v = ko.kv_append(kc, vc, key, val, np.where(slots >= nblk * bs, -1, slots))
    kc_d = _from_bits(kc, device)
    vc_d = None if vc is None else _from_bits(vc, device)
    err = torch.zeros(1, dtype=torch.int32, device=device)
    kvc.kv_append(_from_bits(key, device), None if val is None else _from_bits(val, device),
                  torch.from_numpy(slots).to(device), kc_d, vc_d, error_count=err)
    torch.cuda.synchronize(device)
    np.testing.assert_array_equal(_bits(kc_d), want_k)
    if vc is not None:
        np.testing.assert_array_equal(_bits(vc_d), want_v)
    assert int(err.item()) == 1


def test_kv_append_into_strided_cache_views(device):
    # K and V caches as views into one [nblk, bs, 2, hkv, d] allocation (non-contiguous blocks)
    rng = np.random.default_rng(901)
    nblk, bs, hkv, d, ntok = 6, 32, 4, 64, 9
    both = rng.integers(0, 1 << 16, size=(nblk, bs, 2, hkv, d), dtype=np.uint16)
    key = rng.integers(0, 1 << 16, size=(ntok, hkv, d), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, size=(ntok, hkv, d), dtype=np.uint16)
    slots = rng.permutation(nblk * bs)[:ntok].astype(np.int32)
    want_k, want_v = ko.kv_append(both[:, :, 0], both[:, :, 1], key, val, slots)
    both_d = _from_bits(both, device)
    kvc.kv_append(_from_bits(key, device), _from_bits(val, device), torch.from_numpy(slots).to(device),
                  both_d[:, :, 0], both_d[:, :, 1])
    torch.cuda.synchronize(device)
    got = _bits(both_d)
    np.testing.assert_array_equal(got[:, :, 0], want_k)
    np.testing.assert_array_equal(got[:, :, 1], want_v)


def _prelude_inputs(b, hq, hkv, d, bs, max_blocks, seq_lens, seed, rope_len=None):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s, std=1.0, bias=0.0: torch.empty(s).normal_(0.0, std, generator=g) + bias
    table = torch.arange(b * max_blocks, dtype=torch.int32).reshape(b, max_blocks)  # reference identity paging
    seq = torch.tensor(seq_lens, dtype=torch.int32)
    slots = torch.from_numpy(ko.slot_of(table.numpy(), seq.numpy(), bs))
    cos, sin = ko.rope_tables(rope_len or max_blocks * bs, d)
    return dict(q_proj=rn(b, hq * d, std=0.5), k_proj=rn(b, hkv * d, std=0.5), v_proj=rn(b, hkv * d, std=0.5),
                inv_rms=rn(b, std=0.2, bias=1.0).abs(), q_norm_weight=rn(d, std=0.1, bias=1.0),
                k_norm_weight=rn(d, std=0.1, bias=1.0), rope_cos=torch.from_numpy(cos), rope_sin=torch.from_numpy(sin),
                seq_lens=seq, slot_mapping=slots, block_table=table,
                key_cache=rn(b * max_blocks, bs, hkv, d, std=0.5).to(torch.bfloat16),
                value_cache=rn(b * max_blocks, bs, hkv, d, std=0.5).to(torch.bfloat16))


def _ulp_check(got: np.ndarray, want: np.ndarray, what: str, max_frac: float = 0.02) -> None:
    g = ko.bf16_bits_to_f32(got).astype(np.float64)
    w = ko.bf16_bits_to_f32(want).astype(np.float64)
    assert np.all(np.isfinite(g)), what
    diff = g != w
    # one bf16 step at the larger magnitude: 2^(exponent - 7)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(w), 1e-30))) - 7)
    assert np.all(np.abs(g - w) <= step * 1.0001), f"{what}: difference above one bf16 step"
    assert diff.mean() <= max_frac, f"{what}: {diff.mean():.3%} elements differ by one step"


@pytest.mark.parametrize("b,hq,hkv,d,seq", [(16, 40, 8, 128, [3500] * 16), (5, 8, 2, 64, [1, 2, 100, 255, 256])])
def test_qk_norm_rope_append_matches_oracle(b, hq, hkv, d, seq, device):
    print(f"[case] prelude b={b} hq={hq} hkv={hkv} d={d}", flush=True)
    bs, max_blocks = 128, 43 if d == 128 else 2
    x = _prelude_inputs(b, hq, hkv, d, bs, max_blocks, seq, seed=910 + d)
    q, k, v = ko.qk_norm_rope(x["q_proj"].numpy(), x["k_proj"].numpy(), x["v_proj"].numpy(), x["inv_rms"].numpy(),
                              x["q_norm_weight"].numpy(), x["k_norm_weight"].numpy(), x["rope_cos"].numpy(),
                              x["rope_sin"].numpy(), x["seq_lens"].numpy(), hq, hkv)
    kc0, vc0 = _bits(x["key_cache"]), _bits(x["value_cache"])
    want_k, want_v = ko.kv_append(kc0, vc0, k, v, x["slot_mapping"].numpy())
    d_ = {n: t.to(device) for n, t in x.items()}
    q_out = kvc.qk_norm_rope_append(d_["q_proj"], d_["k_proj"], d_["v_proj"], d_["inv_rms"], d_["q_norm_weight"],
                                    d_["k_norm_weight"], d_["rope_cos"], d_["rope_sin"], d_["seq_lens"],
                                    d_["slot_mapping"], d_["key_cache"], d_["value_cache"], num_heads=hq)
    torch.cuda.synchronize(device)
    _ulp_check(_bits(q_out), q, "q")
    got_k, got_v = _bits(d_["key_cache"]), _bits(d_["value_cache"])
    written = np.zeros(kc0.shape[:2], dtype=bool)
    s = x["slot_mapping"].numpy()
    written[s // bs, s % bs] = True
    np.testing.assert_array_equal(got_k[~written], kc0[~written])  # untouched rows bit-exact
    np.testing.assert_array_equal(got_v[~written], vc0[~written])
    _ulp_check(got_k[written], want_k[written], "k")
    np.testing.assert_array_equal(got_v[written], want_v[written])  # v: one product, then bf16 — exact


def test_prelude_position_outside_rope_table(device):
    x = _prelude_inputs(3, 4, 2, 32, 16, 3, [5, 33, 7], seed=920, rope_len=32)  # position 32: past the table
    kc0 = _bits(x["key_cache"])
    d_ = {n: t.to(device) for n, t in x.items()}
    err = torch.zeros(1, dtype=torch.int32, device=device)
    q_out = kvc.qk_norm_rope_append(d_["q_proj"], d_["k_proj"], d_["v_proj"], d_["inv_rms"], d_["q_norm_weight"],
                                    d_["k_norm_weight"], d_["rope_cos"], d_["rope_sin"], d_["seq_lens"],
                                    d_["slot_mapping"], d_["key_cache"], d_["value_cache"], num_heads=4,
                                    error_count=err)
    torch.cuda.synchronize(device)
    assert int(err.item()) == 1
    assert torch.all(q_out[1] == 0)
    s = int(x["slot_mapping"][1])
    np.testing.assert_array_equal(_bits(d_["key_cache"])[s // 16, s % 16], kc0[s // 16, s % 16])


def test_prelude_then_decode_chain(device):
    # the decode layer's attention: prelude + cache write, then paged attention over the updated cache
    b, hq, hkv, d, bs, max_blocks = 8, 32, 8, 128, 128, 12
    seq = [1, 129, 400, 777, 1024, 1500, 1536, 64]
    x = _prelude_inputs(b, hq, hkv, d, bs, max_blocks, seq, seed=930)
    q, k, v = ko.qk_norm_rope(x["q_proj"].numpy(), x["k_proj"].numpy(), x["v_proj"].numpy(), x["inv_rms"].numpy(),
                              x["q_norm_weight"].numpy(), x["k_norm_weight"].numpy(), x["rope_cos"].numpy(),
                              x["rope_sin"].numpy(), x["seq_lens"].numpy(), hq, hkv)
    kc, vc = ko.kv_append(_bits(x["key_cache"]), _bits(x["value_cache"]), k, v, x["slot_mapping"].numpy())
    from oracle import pa_oracle
    scale = 1.0 / np.sqrt(d)
    ref = pa_oracle.paged_attention_decode(ko.bf16_bits_to_f32(q), ko.bf16_bits_to_f32(kc), ko.bf16_bits_to_f32(vc),
                                           x["block_table"].numpy(), x["seq_lens"].numpy(), scale)
    d_ = {n: t.to(device) for n, t in x.items()}
    q_out = kvc.qk_norm_rope_append(d_["q_proj"], d_["k_proj"], d_["v_proj"], d_["inv_rms"], d_["q_norm_weight"],
                                    d_["k_norm_weight"], d_["rope_cos"], d_["rope_sin"], d_["seq_lens"],
                                    d_["slot_mapping"], d_["key_cache"], d_["value_cache"], num_heads=hq)
    out = pa.paged_attention_decode(q_out, d_["key_cache"], d_["value_cache"], d_["block_table"], d_["seq_lens"],
                                    scale=scale)
    torch.cuda.synchronize(device)
    assert_close(out.cpu().numpy(), ref, what="prelude+decode")
