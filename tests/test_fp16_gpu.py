"""fp16 query and caches (kv_format SIMPLER_HIP_KV_FP16) on the GPU, through the C ABI.

The reference's GQA scene cases are fp16 (tests/st/a2a3/tensormap_and_ringbuffer/
spmd_paged_attention_highperf/test_spmd_paged_attention_highperf.py:170-232),
and its generic golden rounds p to the input dtype (goldens/paged_attention.py
:168), so the fp16 kernels round p to fp16 and are checked against the oracle
with p_dtype="fp16". The high-performance SPMD callable itself (tiling tensor
with lengths and scale, fp16 output) runs through Worker.run and is compared
with the oracle and with that test's fp32 softmax golden at its tolerance
(RTOL 5e-3, ATOL 2e-2, :94-95).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import pa_oracle
from simpler_amd import TaskArgs, Worker
from simpler_amd import paged_attention as pa
from simpler_amd.task_interface import ChipStorageTaskArgs, ChipTensor, DataType, TensorArgType
from simpler_amd.workloads import make_custom_case, make_highperf_case
from tests.pa_helpers import REF_ATOL, REF_RTOL, assert_close, oracle_numpy

pytestmark = pytest.mark.gpu

# test_spmd_paged_attention_highperf.py:170-232 (the sim-capable and CI cases)
HIGHPERF_CASES = {
    "b1_h32_kv8_s128_bs128": dict(batch=1, num_heads=32, num_kv_heads=8, head_dim=128, kv_seq=128, block_size=128),
    "b4_h32_kv8_s512_bs128": dict(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, kv_seq=512, block_size=128),
    "b1_h32_kv8_s4096_bs128": dict(batch=1, num_heads=32, num_kv_heads=8, head_dim=128, kv_seq=4096, block_size=128),
    "b1_h32_kv8_s8192_bs128": dict(batch=1, num_heads=32, num_kv_heads=8, head_dim=128, kv_seq=8192, block_size=128),
    "b2_h32_kv8_s8192_bs128": dict(batch=2, num_heads=32, num_kv_heads=8, head_dim=128, kv_seq=8192, block_size=128),
}
HIGHPERF_RTOL, HIGHPERF_ATOL = 5e-3, 2e-2


def run_gpu(case, device, out_dtype=torch.float32, num_workers=0):
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=out_dtype, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              causal=case.config.causal, num_workers=num_workers)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    return out.float().cpu().numpy()


def gqa_golden(case) -> np.ndarray:
    """The highperf test's golden: full softmax per head in fp32 (no p rounding)."""
    return pa_oracle.attention_fp64(case.query.float().numpy(), case.key_cache.float().numpy(),
                                    case.value_cache.float().numpy(), case.block_table.numpy(),
                                    case.context_lens.numpy(), case.scale)


@pytest.mark.parametrize("name", sorted(HIGHPERF_CASES))
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_highperf_shapes_direct_entry(name, out_dtype, device):
    print(f"[case] fp16 {name} out={out_dtype}", flush=True)
    case, _ = make_highperf_case(HIGHPERF_CASES[name], seed=42)
    got = run_gpu(case, device, out_dtype=out_dtype)
    ref = oracle_numpy(case)
    if out_dtype == torch.float16:
        ref = torch.from_numpy(ref).to(torch.float16).float().numpy()
    assert_close(got, ref, what=name)
    np.testing.assert_allclose(got, gqa_golden(case), rtol=HIGHPERF_RTOL, atol=HIGHPERF_ATOL)


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp16_block_sizes_and_head_dims(bs, d, device):
    print(f"[case] fp16 bs={bs} d={d}", flush=True)
    case = make_custom_case(batch=3, num_heads=16, kv_heads=4, head_dim=d, block_size=bs,
                            context_lens=[1, 333, 2 * bs + 5], seed=100 + bs + d, dtype=torch.float16)
    got = run_gpu(case, device)
    ref = oracle_numpy(case)
    assert_close(got, ref, what=f"fp16 bs{bs} d{d}")
    np.testing.assert_allclose(got, ref, rtol=REF_RTOL, atol=REF_ATOL)


@pytest.mark.parametrize("workers", [0, 7, 1000])
def test_fp16_causal_verify_and_worker_counts(workers, device):
    print(f"[case] fp16 causal q_len 8 workers={workers}", flush=True)
    case = make_custom_case(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8, causal=True,
                            context_lens=[8, 900, 2500], seed=77, dtype=torch.float16)
    assert_close(run_gpu(case, device, num_workers=workers), oracle_numpy(case), what=f"fp16 causal w{workers}")


@pytest.fixture(scope="module")
def worker(device):
    w = Worker(level=2, platform="mi355x", runtime="tensormap_and_ringbuffer", device_id=device.index or 0)
    w.init()
    yield w
    w.close()


def _highperf_args(case, tiling, out, device=None):
    """The 15 tensors + 1 scalar of the highperf CALLABLE (test :331-347); the
    eight workspaces are small placeholders (the HIP backend does not use them)."""
    tensors = [case.query, case.key_cache, case.value_cache, case.block_table, out]
    tensors += [torch.zeros(16, dtype=torch.uint8) for _ in range(8)]
    tensors += [tiling, torch.zeros(1, dtype=torch.uint8)]
    if device is None:
        args = TaskArgs()
        for i, t in enumerate(tensors):
            args.add_tensor(t.contiguous(), TensorArgType.OUTPUT_EXISTING if i == 4 else TensorArgType.INPUT)
        args.add_scalar(ctypes.c_int64(24))  # effective_block_dim (unused here)
        return args, None
    dev = [t.to(device) for t in tensors]
    dev[4] = out
    args = ChipStorageTaskArgs()
    dt = {torch.float16: DataType.FLOAT16, torch.int32: DataType.INT32, torch.uint8: DataType.UINT8}
    for t in dev:
        args.add_tensor(ChipTensor.make(t.data_ptr(), tuple(t.shape), dt[t.dtype], child_memory=True))
    args.add_scalar(ctypes.c_int64(24))
    return args, dev


@pytest.mark.parametrize("name", ["b1_h32_kv8_s128_bs128", "b4_h32_kv8_s512_bs128", "b2_h32_kv8_s8192_bs128"])
@pytest.mark.parametrize("where", ["host", "device"])
def test_highperf_callable_through_worker(worker, device, name, where):
    print(f"[case] highperf callable {name} {where} tensors", flush=True)
    case, tiling = make_highperf_case(HIGHPERF_CASES[name], seed=42)
    handle = worker.register(pa.reference_callable("spmd_paged_attention_highperf"))
    assert worker.chip_worker.callable_family(handle) == "highperf"
    if where == "host":
        out = torch.zeros(case.query.shape, dtype=torch.float16)
        args, _ = _highperf_args(case, tiling, out)
        worker.run(handle, args)
        got = out.float().numpy()
    else:
        out = torch.full(case.query.shape, float("nan"), dtype=torch.float16, device=device)
        args, keep = _highperf_args(case, tiling, out, device)
        torch.cuda.synchronize(device)
        worker.chip_worker.run(handle, args)
        got = out.float().cpu().numpy()
    ref = torch.from_numpy(oracle_numpy(case)).to(torch.float16).float().numpy()
    assert_close(got, ref, what=f"highperf {name}")
    np.testing.assert_allclose(got, gqa_golden(case), rtol=HIGHPERF_RTOL, atol=HIGHPERF_ATOL)
    worker.unregister(handle)


def test_highperf_callable_rejects_a_mismatched_tiling(worker):
    case, tiling = make_highperf_case(HIGHPERF_CASES["b1_h32_kv8_s128_bs128"], seed=1)
    tiling[1] = 16  # num_heads in the header disagrees with the query
    handle = worker.register(pa.reference_callable("spmd_paged_attention_highperf"))
    out = torch.zeros(case.query.shape, dtype=torch.float16)
    args, _ = _highperf_args(case, tiling, out)
    with pytest.raises(RuntimeError, match="-1"):
        worker.run(handle, args)
    worker.unregister(handle)
