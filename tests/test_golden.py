"""The committed golden fixtures (tests/golden/, written by make_fixtures.py)
still hold: the seeded generator reproduces every config's inputs bit for bit
(SHA-256), and the oracle reproduces the committed outputs. A change of torch's
RNG stream, of the generator's draw order or of the oracle's arithmetic fails
here instead of moving the inputs and the expected outputs together."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import pa_oracle
from simpler_amd.workloads import CONFIGS, make_case
from tests.golden import make_fixtures as mf
from tests.pa_helpers import f32, oracle_numpy

GOLDEN = Path(__file__).resolve().parent / "golden"
CONFIGS_JSON = json.loads((GOLDEN / "configs.json").read_text())


def load_cfg1():
    with np.load(GOLDEN / "cfg1_small.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def stats_match(got: dict, want: dict) -> bool:
    if got["shape"] != want["shape"] or got["sample_index"] != want["sample_index"]:
        return False
    for k in ("sum", "l2", "abs_sum"):
        if not np.isclose(got[k], want[k], rtol=1e-6, atol=1e-6):
            return False
    return bool(np.allclose(got["sample"], want["sample"], rtol=1e-6, atol=1e-6))


def test_cfg1_inputs_and_output_reproduce():
    z = load_cfg1()
    case = make_case("cfg1_small")
    arrays = mf.cfg1_arrays()
    for k in ("query_bits", "key_cache_bits", "value_cache_bits", "block_table", "context_lens", "scale", "seed"):
        np.testing.assert_array_equal(arrays[k], z[k], err_msg=k)
    np.testing.assert_array_equal(oracle_numpy(case), z["out"])


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_config_inputs_and_oracle_output_reproduce(name):
    want = CONFIGS_JSON[name]
    case = make_case(name)
    assert case.seed == want["seed"]
    assert mf.input_hashes(case) == want["inputs_sha256"]
    got = mf.output_stats(mf.oracle_output(case))
    assert stats_match(got, want["oracle_out"]), (got["sum"], want["oracle_out"]["sum"])


def test_a_perturbed_seed_fails_the_hashes():
    case = make_case("cfg1_small", seed=CONFIGS_JSON["cfg1_small"]["seed"] + 1)
    hashes = mf.input_hashes(case)
    want = CONFIGS_JSON["cfg1_small"]["inputs_sha256"]
    assert all(hashes[k] != want[k] for k in ("query", "key_cache", "value_cache"))


def test_a_perturbed_oracle_fails_the_outputs():
    """A planted mistake in the oracle (its scale off by 1%, or p left
    unrounded before the row sum) no longer reproduces the committed cfg1
    output."""
    z = load_cfg1()
    case = make_case("cfg1_small")
    args = (f32(case.query), f32(case.key_cache), f32(case.value_cache), case.block_table.numpy(),
            case.context_lens.numpy())
    off_scale = pa_oracle.paged_attention_decode(*args, case.scale * 1.01)
    assert np.max(np.abs(off_scale - z["out"])) > 1e-4
    orig = pa_oracle.bf16_round
    try:
        pa_oracle.bf16_round = lambda x: np.asarray(x, np.float32)  # p not rounded to bf16
        unrounded = pa_oracle.paged_attention_decode(*args, case.scale)
    finally:
        pa_oracle.bf16_round = orig
    assert np.max(np.abs(unrounded - z["out"])) > 1e-6
