"""Pins for the oracle's fp8 (E4M3FN) decode and the fp8 workload generator (CPU only).

The decode is a bit-level formula; it is checked against torch's own
float8_e4m3fn conversion on all 256 codes (an independent implementation) and
against hand-computed points of the format (1.0, 448, the smallest subnormal
and normal, signed zero, NaN). The generator's quantisation is checked to
round-trip through the oracle's decode and to stay within fp8's relative step.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import pa_oracle as po
from simpler_amd.workloads import dequantize_kv_fp8, make_custom_case, quantize_kv_fp8


def test_decode_matches_torch_on_every_code():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = po.fp8_e4m3fn_to_f32(codes)
    nan = np.isnan(want)
    assert list(np.nonzero(nan)[0]) == [127, 255]
    assert np.all(np.isnan(got[nan]))
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_decode_closed_form_points():
    f = po.fp8_e4m3fn_to_f32
    assert f(np.uint8(0x38)) == 1.0 and f(np.uint8(0x7E)) == 448.0 and f(np.uint8(0xFE)) == -448.0
    assert f(np.uint8(0x01)) == 2.0 ** -9 and f(np.uint8(0x08)) == 2.0 ** -6 and f(np.uint8(0x07)) == 7 * 2.0 ** -9
    z = f(np.uint8(0x80))
    assert z == 0.0 and np.signbit(z)


def test_quantize_round_trip_and_error_bound():
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=32,
                            context_lens=[40, 64], seed=3)
    k = case.key_cache
    k8, ks = quantize_kv_fp8(k, pow2=False)
    deq_t = dequantize_kv_fp8(k8, ks).numpy()
    deq_o = po.dequantize_kv(k8.view(torch.uint8).numpy(), ks.numpy())
    np.testing.assert_array_equal(deq_t, deq_o)  # generator and oracle agree on the meaning
    x = k.float().numpy()
    amax = np.abs(x).max(axis=(1, 3))
    # E4M3 keeps 4 significant bits: |err| <= 2^-4 |x| for normals, and subnormal
    # steps are 2^-9 * scale
    err = np.abs(deq_o - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, (amax / 448.0)[:, None, :, None] * 2.0 ** -9 / 2)
    assert np.all(err <= bound * 1.0001)
    # power-of-two scales make the dequantised values bf16 values
    k8p, ksp = quantize_kv_fp8(k, pow2=True)
    d = dequantize_kv_fp8(k8p, ksp)
    assert torch.equal(d, d.to(torch.bfloat16).float())
    assert torch.all(torch.log2(ksp[ksp > 0]) == torch.round(torch.log2(ksp[ksp > 0])))


def test_zero_block_scale():
    c = torch.zeros(3, 16, 2, 128, dtype=torch.bfloat16)
    c[1] = 1.0
    q8, s = quantize_kv_fp8(c)
    assert s[0].eq(0).all() and s[2].eq(0).all() and s[1].gt(0).all()
    assert torch.all(dequantize_kv_fp8(q8, s)[0] == 0)
