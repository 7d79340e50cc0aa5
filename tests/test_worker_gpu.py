"""The drop-in path end to end: Worker(level=2) / ChipWorker → simpler_* C API → fused kernel.

Mirrors how the reference's scene test drives paged attention
(simpler_setup/scene_test.py:1623-1694 → Worker.run → simpler_run): the PA
CALLABLE (QK/SF/PV/UP chain) is registered, a ChipStorageTaskArgs with the 7
arguments is submitted, outputs are compared with the golden (here: the oracle).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from simpler_amd import TaskArgs, Worker
from simpler_amd import paged_attention as pa
from simpler_amd.task_interface import ChipStorageTaskArgs, ChipTensor, DataType, TensorArgType
from simpler_amd.workloads import make_case, make_custom_case
from tests.pa_helpers import REF_ATOL, REF_RTOL, assert_close, oracle_numpy

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def worker(device):
    w = Worker(level=2, platform="mi355x", runtime="tensormap_and_ringbuffer", device_id=device.index or 0)
    w.init()
    yield w
    w.close()


def host_args(case, out):
    args = TaskArgs()
    for t in (case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens):
        args.add_tensor(t.contiguous(), TensorArgType.INPUT)
    args.add_tensor(out, TensorArgType.OUTPUT_EXISTING)
    args.add_scalar(ctypes.c_float(case.scale))
    return args


@pytest.mark.parametrize("callable_kind", ["reference_chain", "native"])
def test_worker_run_with_host_tensors(worker, callable_kind):
    print(f"[case] worker host tensors {callable_kind}", flush=True)
    case = make_custom_case(batch=4, num_heads=16, kv_heads=1, head_dim=16, block_size=16,
                            context_lens=[33, 64, 128, 15], seed=42, max_blocks=16)  # CaseVarSeq4
    handle = worker.register(pa.reference_chain_callable() if callable_kind == "reference_chain"
                             else pa.native_callable())
    out = torch.zeros(case.out_shape(), dtype=torch.float32)
    worker.run(handle, host_args(case, out))
    ref = oracle_numpy(case)
    assert_close(out.numpy(), ref, what="worker/host")
    np.testing.assert_allclose(out.numpy(), ref, rtol=REF_RTOL, atol=REF_ATOL)
    worker.unregister(handle)


def test_worker_run_with_device_tensors_and_bf16_out(worker, device):
    print("[case] worker device tensors cfg1", flush=True)
    case = make_case("cfg1_small")
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.bfloat16, device=device)
    handle = worker.register(pa.reference_chain_callable())
    args = ChipStorageTaskArgs()
    for t in (d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out):
        args.add_tensor(ChipTensor.make(t.data_ptr(), tuple(t.shape), {
            torch.bfloat16: DataType.BFLOAT16, torch.int32: DataType.INT32}[t.dtype], child_memory=True))
    args.add_scalar(ctypes.c_float(case.scale))
    torch.cuda.synchronize(device)
    worker.chip_worker.run(handle, args)
    ref = torch.tensor(oracle_numpy(case)).to(torch.bfloat16).float().numpy()
    assert_close(out.float().cpu().numpy(), ref, what="worker/device")


def device_args(d, out):
    args = ChipStorageTaskArgs()
    for t in (d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out):
        args.add_tensor(ChipTensor.make(t.data_ptr(), tuple(t.shape), {
            torch.bfloat16: DataType.BFLOAT16, torch.int32: DataType.INT32,
            torch.float32: DataType.FLOAT32}[t.dtype], child_memory=True))
    args.add_scalar(ctypes.c_float(d.scale))
    return args


def test_worker_reports_device_bad_block_then_recovers(worker, device):
    """A device-resident table with an out-of-pool id is only seen by the kernel:
    the run fails with SIMPLER_HIP_ERR_BAD_BLOCK (-6), the error word is cleared,
    and the runs after it on the same context succeed and match the oracle."""
    print("[case] worker device bad block, then three good runs", flush=True)
    case = make_custom_case(batch=3, num_heads=16, kv_heads=2, head_dim=64, block_size=16,
                            context_lens=[40, 17, 64], seed=11, max_blocks=8)
    d = case.to(device)
    handle = worker.register(pa.reference_chain_callable())
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    bad_table = d.block_table.clone()
    bad_table[1, 1] = case.key_cache.shape[0] + 5
    good_table = d.block_table
    d.block_table = bad_table
    torch.cuda.synchronize(device)
    with pytest.raises(RuntimeError, match="-6"):
        worker.chip_worker.run(handle, device_args(d, out))
    d.block_table = good_table
    ref = oracle_numpy(case)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize(device)
        worker.chip_worker.run(handle, device_args(d, out))
        assert_close(out.cpu().numpy(), ref, what=f"worker/device run {i} after a bad block")
    worker.unregister(handle)


def test_worker_malloc_copy_roundtrip(worker):
    buf = worker.malloc(4096)
    src = torch.arange(1024, dtype=torch.int32)
    dst = torch.zeros(1024, dtype=torch.int32)
    worker.copy_to(buf, src)
    worker.copy_from(dst, buf)
    assert torch.equal(src, dst)
    assert worker.chip_worker.committed_device_memory() >= 4096
    worker.free(buf)


def test_worker_rejects_out_of_pool_block_on_host(worker):
    case = make_custom_case(batch=2, num_heads=16, kv_heads=1, head_dim=16, block_size=16,
                            context_lens=[33, 17], seed=1)
    case.block_table[1, 0] = 999
    handle = worker.register(pa.reference_chain_callable())
    out = torch.zeros(case.out_shape(), dtype=torch.float32)
    with pytest.raises(RuntimeError, match="-1"):
        worker.run(handle, host_args(case, out))


def test_worker_rejects_wrong_dtypes(worker):
    case = make_custom_case(batch=1, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[33], seed=2)
    handle = worker.register(pa.reference_chain_callable())
    args = TaskArgs()
    args.add_tensor(case.query.float())  # FLOAT32 query is not accepted
    for t in (case.key_cache, case.value_cache, case.block_table, case.context_lens):
        args.add_tensor(t)
    args.add_tensor(torch.zeros(case.out_shape()))
    args.add_scalar(1.0)
    with pytest.raises(RuntimeError):
        worker.run(handle, args)


def test_worker_reports_bad_device_length_then_recovers(worker, device):
    """A device-resident context_lens entry longer than its block-table row is
    only seen by the kernel: the run fails with SIMPLER_HIP_ERR_BAD_LENGTH (-7)
    and the next good run on the same context matches the oracle."""
    print("[case] worker device bad length, then a good run", flush=True)
    case = make_custom_case(batch=3, num_heads=16, kv_heads=2, head_dim=64, block_size=16,
                            context_lens=[40, 17, 64], seed=12, max_blocks=8)
    d = case.to(device)
    handle = worker.register(pa.reference_chain_callable())
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    good_lens = d.context_lens
    d.context_lens = good_lens.clone()
    d.context_lens[2] = 8 * 16 + 1
    torch.cuda.synchronize(device)
    with pytest.raises(RuntimeError, match="-7"):
        worker.chip_worker.run(handle, device_args(d, out))
    d.context_lens = good_lens
    out.zero_()
    torch.cuda.synchronize(device)
    worker.chip_worker.run(handle, device_args(d, out))
    assert_close(out.cpu().numpy(), oracle_numpy(case), what="worker run after a bad length")
    worker.unregister(handle)
