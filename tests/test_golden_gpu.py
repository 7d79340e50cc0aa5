"""The fused kernel against the committed cfg1 fixture (inputs and expected
output read from tests/golden/cfg1_small.npz, not regenerated), through the C ABI."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from simpler_amd import paged_attention as pa
from tests.pa_helpers import REF_ATOL, REF_RTOL, assert_close

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "cfg1_small.npz"


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_kernel_matches_committed_cfg1_output(device, out_dtype):
    print(f"[case] committed cfg1 fixture out={out_dtype}", flush=True)
    with np.load(GOLDEN, allow_pickle=False) as z:
        f = {k: z[k] for k in z.files}

    def bf16(bits):
        return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)

    q, k, v = bf16(f["query_bits"]), bf16(f["key_cache_bits"]), bf16(f["value_cache_bits"])
    bt = torch.from_numpy(f["block_table"]).to(device)
    cl = torch.from_numpy(f["context_lens"]).to(device)
    out = torch.empty(f["out"].shape, dtype=out_dtype, device=device)
    pa.paged_attention_decode(q, k, v, bt, cl, out, float(f["scale"][0]))
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    got = out.float().cpu().numpy()
    want = f["out"]
    if out_dtype == torch.bfloat16:
        want = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
    assert_close(got, want, what="committed cfg1")
    np.testing.assert_allclose(got, want, rtol=REF_RTOL, atol=REF_ATOL)
