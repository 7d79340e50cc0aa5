"""simpler_hip_pa_decode_noalloc: the decode with the library's fixed per-GPU
scratch array in place of a caller workspace (it allocates nothing).

Through the C ABI: its output must equal simpler_hip_pa_decode's on the same
args bit for bit (same kernels, same plan), and match the oracle, on two calls
in a row where the second is smaller (the scratch keeps the first call's
contents). A plan larger than the scratch is refused before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from simpler_amd import _lib
from simpler_amd import paged_attention as pa
from simpler_amd.workloads import make_case, make_custom_case
from tests.pa_helpers import assert_close, oracle_c

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 136 << 20  # SIMPLER_HIP_PA_NOALLOC_SCRATCH_BYTES


def _args(d, out, case, num_workers=0):
    return pa.make_args(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                        causal=case.config.causal, num_workers=num_workers)


def _both(case, device):
    """(no-alloc output, workspace-entry output) on the same device inputs."""
    d = case.to(device)
    stream = torch.cuda.current_stream(device).cuda_stream
    out_na = torch.full(case.out_shape(), float("nan"), dtype=torch.float32, device=device)
    out_ws = torch.full(case.out_shape(), float("nan"), dtype=torch.float32, device=device)
    rc = _lib.lib().simpler_hip_pa_decode_noalloc(ctypes.byref(_args(d, out_na, case)), stream)
    assert rc == 0, rc
    pa.launch(_args(d, out_ws, case), device, stream)
    torch.cuda.synchronize(device)
    return out_na.cpu().numpy(), out_ws.cpu().numpy()


@pytest.mark.parametrize("first,second", [("cfg2_qwen3_8b", "gqa_small"), ("cfg4_mla", "mla_small")])
def test_noalloc_matches_workspace_entry_on_two_calls(first, second, device):
    print(f"[case] noalloc {first} then {second}", flush=True)
    big = make_case(first)
    if second == "gqa_small":
        small = make_custom_case(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                 context_lens=[1, 700, 2049], seed=961)
    else:
        small = make_custom_case(batch=2, num_heads=128, kv_heads=1, head_dim=576, head_dim_v=512, mla=True,
                                 block_size=64, context_lens=[65, 1000], seed=962)
    for case in (big, small):
        got, want = _both(case, device)
        np.testing.assert_array_equal(got, want)
        assert_close(got, oracle_c(case, n_threads=16), what=f"noalloc {case.config.name}")


def test_noalloc_refuses_a_plan_beyond_its_scratch(device):
    case = make_case("cfg2_qwen3_8b", batch_override=2)
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    # 16 rows x 128 dims x 4 B x 2 slots = 16 KiB per worker: 9000 workers need ~141 MiB
    a = _args(d, out, case, num_workers=9000)
    assert _lib.lib().simpler_hip_pa_decode_workspace_size(ctypes.byref(a)) > SCRATCH_BYTES
    stream = torch.cuda.current_stream(device).cuda_stream
    assert _lib.lib().simpler_hip_pa_decode_noalloc(ctypes.byref(a), stream) == -4
    torch.cuda.synchronize(device)
    assert torch.count_nonzero(out).item() == 0  # nothing was launched
