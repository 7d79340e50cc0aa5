"""Every paged-attention CALLABLE the reference defines, through the drop-in.

Each reference scene test registers its CALLABLE and runs it through
``Worker.run`` with the inputs of ``simpler_setup/goldens/paged_attention.py
:30-88`` (U(-0.5, 0.5) query/key, U(-1, 1) value, scale 1.0, block ids drawn
with replacement), then compares ``out`` with the golden at its RTOL/ATOL.
Here: the same callables (per-block chain, grouped "unroll" chain including the
4-D ``[B, 1, H, D]`` query/out variant, SPMD mix), the same input recipe
seeded, against the oracle, on a CaseVarSeq4-style shape with host tensors and
on the unroll Case1 shape (B=256, Hq=16, Hkv=1, D=128, BS=128, L=8192; the only
paged-attention case the reference reports timings for) with device tensors.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from simpler_amd import TaskArgs, Worker
from simpler_amd import paged_attention as pa
from simpler_amd.task_interface import ChipStorageTaskArgs, ChipTensor, DataType, TensorArgType
from simpler_amd.workloads import make_reference_case
from tests.pa_helpers import REF_ATOL, REF_RTOL, assert_close, oracle_c, oracle_numpy

pytestmark = pytest.mark.gpu

# test_batch_paged_attention.py CaseVarSeq4 (:168-181)
SMALL = {"batch": 4, "num_heads": 16, "kv_head_num": 1, "head_dim": 16, "block_size": 16, "context_len": 128,
         "context_lens_list": [33, 64, 128, 15], "max_model_len": 256}
# test_paged_attention_unroll.py Case1 (:61-74)
CASE1 = {"batch": 256, "num_heads": 16, "kv_head_num": 1, "head_dim": 128, "block_size": 128, "context_len": 8192,
         "max_model_len": 32768}


@pytest.fixture(scope="module")
def worker(device):
    w = Worker(level=2, platform="mi355x", runtime="tensormap_and_ringbuffer", device_id=device.index or 0)
    w.init()
    yield w
    w.close()


def four_dims(name: str) -> bool:
    return name == "paged_attention_unroll_4dims"


@pytest.fixture(scope="module")
def small_case():
    case = make_reference_case(SMALL, seed=7)
    return case, oracle_numpy(case)


@pytest.fixture(scope="module")
def case1(device):
    case = make_reference_case(CASE1, seed=8)
    ref = oracle_c(case)
    d = case.to(device)
    torch.cuda.synchronize(device)
    return case, d, ref


@pytest.mark.parametrize("name", pa.SEVEN_ARGUMENT_CALLABLES)
def test_reference_callable_small_host_tensors(worker, small_case, name):
    print(f"[case] {name} CaseVarSeq4 host tensors", flush=True)
    case, ref = small_case
    handle = worker.register(pa.reference_callable(name))
    assert worker.chip_worker.callable_family(handle) == pa.REFERENCE_FAMILIES[name]
    b, h, d = case.query.shape
    q = case.query.reshape(b, 1, h, d) if four_dims(name) else case.query
    out = torch.zeros((b, 1, h, d) if four_dims(name) else (b, h, d), dtype=torch.float32)
    args = TaskArgs()
    for t in (q, case.key_cache, case.value_cache, case.block_table, case.context_lens):
        args.add_tensor(t.contiguous(), TensorArgType.INPUT)
    args.add_tensor(out, TensorArgType.OUTPUT_EXISTING)
    args.add_scalar(ctypes.c_float(case.scale))
    worker.run(handle, args)
    got = out.reshape(b, h, d).numpy()
    assert_close(got, ref, what=name)
    np.testing.assert_allclose(got, ref, rtol=REF_RTOL, atol=REF_ATOL)
    worker.unregister(handle)


@pytest.mark.parametrize("name", pa.SEVEN_ARGUMENT_CALLABLES)
def test_reference_callable_case1_device_tensors(worker, case1, device, name):
    print(f"[case] {name} unroll Case1 (B=256, L=8192) device tensors", flush=True)
    case, d, ref = case1
    handle = worker.register(pa.reference_callable(name))
    b, h, dim = case.query.shape
    q = d.query.reshape(b, 1, h, dim) if four_dims(name) else d.query
    out = torch.full((b, 1, h, dim) if four_dims(name) else (b, h, dim), float("nan"), dtype=torch.float32,
                     device=device)
    dt = {torch.bfloat16: DataType.BFLOAT16, torch.int32: DataType.INT32, torch.float32: DataType.FLOAT32}
    args = ChipStorageTaskArgs()
    for t in (q, d.key_cache, d.value_cache, d.block_table, d.context_lens, out):
        args.add_tensor(ChipTensor.make(t.data_ptr(), tuple(t.shape), dt[t.dtype], child_memory=True))
    args.add_scalar(ctypes.c_float(case.scale))
    torch.cuda.synchronize(device)
    worker.chip_worker.run(handle, args)
    got = out.reshape(b, h, dim).cpu().numpy()
    assert_close(got, ref, what=f"{name} Case1")
    np.testing.assert_allclose(got, ref, rtol=REF_RTOL, atol=REF_ATOL)
    worker.unregister(handle)
