"""GPU parity of the fp8 (E4M3FN + per-(block, kv head) scale) KV decode.

No reference kernel uses this format (the reference defines the dtype code,
``data_type.h:63``), so the contract is the golden on the dequantised caches:
``K = fp8(byte) * k_scale[blk, h]``, ``V`` likewise (``oracle.pa_oracle.dequantize_kv``,
pinned in test_fp8_oracle.py), then ``paged_attention_decode``. Tolerance: the
decode tolerance (max-abs 2e-2, rel-L2 1e-3).

At full cfg2 size the fp8 kernel is compared with the bf16 kernel (itself
pinned against the oracle) on bf16 caches holding the dequantised values:
power-of-two scales make those exactly bf16, so the two kernels compute the
same products. They differ only in the order the QK sum visits the dims, and
in p values that sit on a bf16 rounding boundary. Bound: max-abs 2e-3,
rel-L2 1e-4 (f32 output). Both kernels are also deterministic.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import pa_oracle as po
from simpler_amd import TaskArgs, Worker
from simpler_amd import paged_attention as pa
from simpler_amd.task_interface import TensorArgType
from simpler_amd.workloads import dequantize_kv_fp8, make_case, make_custom_case, quantize_kv_fp8
from tests.pa_helpers import assert_close, errors

pytestmark = pytest.mark.gpu


def fp8_case(pow2: bool, **kw):
    case = make_custom_case(**kw)
    case.key_cache, case.k_scale = quantize_kv_fp8(case.key_cache, pow2=pow2)
    case.value_cache, case.v_scale = quantize_kv_fp8(case.value_cache, pow2=pow2)
    return case


def oracle_fp8(case) -> np.ndarray:
    k = po.dequantize_kv(case.key_cache.view(torch.uint8).numpy(), case.k_scale.numpy())
    v = po.dequantize_kv(case.value_cache.view(torch.uint8).numpy(), case.v_scale.numpy())
    return po.paged_attention_decode(case.query.float().numpy(), k, v, case.block_table.numpy(),
                                     case.context_lens.numpy(), case.scale, causal=case.config.causal)


def run_fp8(case, device, out_dtype=torch.float32, num_workers=0):
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=out_dtype, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              causal=case.config.causal, num_workers=num_workers, k_scale=d.k_scale,
                              v_scale=d.v_scale)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    return out.float().cpu().numpy()


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
@pytest.mark.parametrize("pow2", [True, False])
def test_fp8_matches_oracle(device, bs, pow2):
    print(f"[case] fp8 bs={bs} pow2={pow2}", flush=True)
    case = fp8_case(pow2, batch=5, num_heads=32, kv_heads=8, head_dim=128, block_size=bs,
                    context_lens=[1, bs - 1, bs + 1, 3 * bs, 517], seed=200 + bs)
    got = run_fp8(case, device)
    assert_close(got, oracle_fp8(case), what=f"fp8 bs={bs}")


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_fp8_workers_and_output_dtype(device, out_dtype):
    print(f"[case] fp8 workers out={out_dtype}", flush=True)
    case = fp8_case(False, batch=3, num_heads=16, kv_heads=2, head_dim=128, block_size=64,
                    context_lens=[700, 0, 129], seed=211)
    ref = oracle_fp8(case)
    if out_dtype == torch.bfloat16:
        ref = torch.tensor(ref).to(torch.bfloat16).float().numpy()
    for w in (0, 1, 7, 64):  # splits at arbitrary block boundaries exercise the merge
        assert_close(run_fp8(case, device, out_dtype, num_workers=w), ref, what=f"fp8 workers={w}")


def test_fp8_causal_verify(device):
    print("[case] fp8 causal q_len=8", flush=True)
    case = fp8_case(False, batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8, causal=True,
                    context_lens=[9, 300, 1030], seed=212)
    assert_close(run_fp8(case, device), oracle_fp8(case), what="fp8 causal")


def test_fp8_zero_scales(device):
    # blocks whose K or V scale is 0 (all-zero blocks in the cache): V adds nothing,
    # K gives zero scores; the frame logic must not divide by the zero scale
    print("[case] fp8 zero scales", flush=True)
    case = fp8_case(False, batch=2, num_heads=16, kv_heads=2, head_dim=128, block_size=32,
                    context_lens=[200, 96], seed=213)
    blocks = case.block_table[0, :3].long()
    case.v_scale[blocks[1]] = 0.0
    case.k_scale[blocks[2]] = 0.0
    case.v_scale[case.block_table[1, 0].long(), 0] = 0.0
    assert_close(run_fp8(case, device), oracle_fp8(case), what="fp8 zero scales")


def test_fp8_full_size_matches_bf16_kernel(device):
    print("[case] fp8 cfg2 full size vs bf16 kernel", flush=True)
    case = make_case("cfg2_fp8")
    got = run_fp8(case, device)
    got2 = run_fp8(case, device)
    np.testing.assert_array_equal(got, got2)  # deterministic
    d = case.to(device)
    kb = dequantize_kv_fp8(d.key_cache, d.k_scale).to(torch.bfloat16)
    vb = dequantize_kv_fp8(d.value_cache, d.v_scale).to(torch.bfloat16)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, kb, vb, d.block_table, d.context_lens, out, case.scale)
    torch.cuda.synchronize(device)
    ref = out.cpu().numpy()
    max_abs, rel = errors(got, ref)
    print(f"fp8 vs bf16 kernel on identical values: max-abs {max_abs:.2e}, rel-L2 {rel:.2e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-4
    assert np.all(np.isfinite(got))


def test_fp8_bad_block_reported(device):
    case = fp8_case(True, batch=2, num_heads=16, kv_heads=2, head_dim=128, block_size=32,
                    context_lens=[64, 40], seed=214)
    d = case.to(device)
    d.block_table[1, 1] = case.key_cache.shape[0] + 5
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              k_scale=d.k_scale, v_scale=d.v_scale)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)


def test_fp8_through_simpler_run(device):
    # FP8E4M3FN caches through the ChipWorker path: tensors 6 and 7 carry the scales
    print("[case] fp8 via Worker", flush=True)
    case = fp8_case(False, batch=3, num_heads=16, kv_heads=4, head_dim=128, block_size=64,
                    context_lens=[65, 200, 1], seed=215)
    w = Worker(level=2, platform="mi355x", device_id=device.index or 0)
    w.init()
    try:
        h = w.register(pa.reference_chain_callable())
        out = torch.zeros(case.out_shape(), dtype=torch.float32)
        args = TaskArgs()
        for t in (case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens):
            args.add_tensor(t, TensorArgType.INPUT)
        args.add_tensor(out, TensorArgType.OUTPUT_EXISTING)
        args.add_tensor(case.k_scale, TensorArgType.INPUT)
        args.add_tensor(case.v_scale, TensorArgType.INPUT)
        args.add_scalar(ctypes.c_float(case.scale))
        w.run(h, args)
        assert_close(out.numpy(), oracle_fp8(case), what="fp8 worker")
    finally:
        w.close()


def test_fp8_blocks_shared_between_sequences(device):
    """fp8 caches with block tables that share physical blocks (and their
    per-(block, kv head) scales) between sequences match the dequantised
    oracle on the same table."""
    case = fp8_case(pow2=False, batch=4, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                    context_lens=[1000, 1000, 300, 2049], seed=962)
    bt = case.block_table
    for b in range(1, 4):
        bt[b, :4] = bt[0, :4]
    assert_close(run_fp8(case, device), oracle_fp8(case), what="fp8 shared blocks")


def test_fp8_fused_kv_buffer(device):
    """fp8 K and V as the two halves of one [num_blocks, 2, bs, h, d] byte
    buffer (strided views) match the dequantised oracle."""
    case = fp8_case(pow2=False, batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=64,
                    context_lens=[700, 65, 1500], seed=965)
    k8, v8 = case.key_cache.view(torch.uint8), case.value_cache.view(torch.uint8)
    buf = torch.full((k8.shape[0], 2, *k8.shape[1:]), 0x7F, dtype=torch.uint8)  # 0x7F: E4M3FN NaN
    buf[:, 0], buf[:, 1] = k8, v8
    buf = buf.to(device)
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, buf[:, 0], buf[:, 1], d.block_table, d.context_lens, out, case.scale,
                              k_scale=d.k_scale, v_scale=d.v_scale)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert_close(out.cpu().numpy(), oracle_fp8(case), what="fp8 fused kv")
