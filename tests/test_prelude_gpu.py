"""The decode prelude, append and decode in one call (``simpler_hip_pa_decode_prelude``) on the GPU.

Checked bit for bit against the chain it replaces, on the same inputs: the
standalone prelude ``simpler_hip_qk_norm_rope_append`` (one call over every new
token, at position ``len - q_len + i`` and the slot its block-table entry gives)
followed by ``simpler_hip_pa_decode`` on the query it wrote. That prelude is
itself pinned against the oracle (tests/test_kv_cache_gpu.py), the decode
likewise (tests/test_pa_gpu.py). The output and both caches must be equal.
Shapes: one row tile (q_len 1, the Qwen3-8B head layout), causal q_len 4 with
16-token blocks and a forced worker count, two row tiles in one wave (q_len 8),
four tiles as sibling waves (q_len 16), lengths past the RoPE table
(reported as BAD_LENGTH, those tokens' query rows zero and their cache rows
untouched, as the standalone prelude leaves them), lengths below q_len, and
replays of the call captured in a HIP graph.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as ko
from simpler_amd import kv_cache as kvc
from simpler_amd import paged_attention as pa

pytestmark = pytest.mark.gpu

D = 128


def _inputs(batch, hq, hkv, bs, lens, q_len, seed, rope_len=None):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s, std=1.0, bias=0.0: torch.empty(s).normal_(0.0, std, generator=g) + bias  # noqa: E731
    max_blocks = max(1, math.ceil(max(lens) / bs)) + 1
    pool = batch * max_blocks
    table = torch.randperm(pool, generator=g).to(torch.int32).reshape(batch, max_blocks)
    cos, sin = ko.rope_tables(rope_len or max_blocks * bs, D)
    return dict(
        q_proj=rn(batch, q_len, hq, D, std=0.5), k_proj=rn(batch, q_len, hkv, D, std=0.5),
        v_proj=rn(batch, q_len, hkv, D, std=0.5), inv_rms=rn(batch, q_len, std=0.2, bias=1.0).abs(),
        q_norm_weight=rn(D, std=0.1, bias=1.0), k_norm_weight=rn(D, std=0.1, bias=1.0),
        rope_cos=torch.from_numpy(cos), rope_sin=torch.from_numpy(sin), block_table=table,
        context_lens=torch.tensor(lens, dtype=torch.int32),
        key_cache=rn(pool, bs, hkv, D, std=0.5).to(torch.bfloat16),
        value_cache=rn(pool, bs, hkv, D, std=0.5).to(torch.bfloat16))


def _standalone_prelude(x, hq, q_len, bs):
    """The standalone prelude over every new token (positions and slots built here); returns the query."""
    batch = x["q_proj"].shape[0]
    hkv = x["k_proj"].shape[2]
    lens = x["context_lens"].cpu().long()
    pos = lens[:, None] - q_len + torch.arange(q_len)[None, :]  # [batch, q_len]
    table = x["block_table"].cpu().long()
    slot = table.gather(1, (pos // bs).clamp(min=0)) * bs + pos % bs
    slot = torch.where(pos >= 0, slot, torch.full_like(slot, -1))
    dev = x["q_proj"].device
    tok = batch * q_len
    q_out = kvc.qk_norm_rope_append(
        x["q_proj"].reshape(tok, hq * D), x["k_proj"].reshape(tok, hkv * D), x["v_proj"].reshape(tok, hkv * D),
        x["inv_rms"].reshape(tok), x["q_norm_weight"], x["k_norm_weight"], x["rope_cos"], x["rope_sin"],
        (pos + 1).reshape(tok).to(torch.int32).to(dev), slot.reshape(tok).to(torch.int32).to(dev), x["key_cache"],
        x["value_cache"], num_heads=hq, error_count=torch.zeros(1, dtype=torch.int32, device=dev))
    return q_out.reshape(batch, q_len, hq, D) if q_len > 1 else q_out


def _chain(x, hq, q_len, bs, scale, workers):
    """Standalone prelude over every new token, then the plain decode."""
    query = _standalone_prelude(x, hq, q_len, bs)
    return pa.paged_attention_decode(query, x["key_cache"], x["value_cache"], x["block_table"], x["context_lens"],
                                     scale=scale, causal=q_len > 1, num_workers=workers)


def _one_call(x, q_len, scale, workers):
    q_proj = x["q_proj"] if q_len > 1 else x["q_proj"][:, 0]
    k_proj = x["k_proj"] if q_len > 1 else x["k_proj"][:, 0]
    v_proj = x["v_proj"] if q_len > 1 else x["v_proj"][:, 0]
    return pa.paged_attention_decode_prelude(
        q_proj.contiguous(), k_proj.contiguous(), v_proj.contiguous(), x["inv_rms"], x["q_norm_weight"],
        x["k_norm_weight"], x["rope_cos"], x["rope_sin"], x["key_cache"], x["value_cache"], x["block_table"],
        x["context_lens"], scale=scale, eps=kvc.EPS, causal=q_len > 1, num_workers=workers)


CASES = {
    # name: (batch, hq, hkv, block_size, lens, q_len, workers)
    "q1_qwen3_heads": (4, 32, 8, 128, [1, 129, 700, 2000], 1, 0),
    "q4_bs16_w7": (3, 16, 4, 16, [4, 40, 300], 4, 7),
    "q8_two_tiles": (3, 32, 8, 128, [8, 130, 2000], 8, 0),
    "q8_two_tiles_w333": (2, 32, 8, 128, [700, 1500], 8, 333),
    "q16_siblings": (2, 32, 8, 64, [16, 500], 16, 0),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_prelude_in_one_call_equals_prelude_then_decode(name, device):
    batch, hq, hkv, bs, lens, q_len, workers = CASES[name]
    print(f"[case] prelude in one call {name}", flush=True)
    x = _inputs(batch, hq, hkv, bs, lens, q_len, seed=960 + len(name))
    a = {n: t.to(device) for n, t in x.items()}
    b = {n: (t.clone() if n in ("key_cache", "value_cache") else t) for n, t in a.items()}
    scale = 1.0 / math.sqrt(D)
    want = _chain(a, hq, q_len, bs, scale, workers)
    got = _one_call(b, q_len, scale, workers)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert torch.equal(got, want), f"{name}: output differs from prelude then decode"
    assert torch.equal(b["key_cache"], a["key_cache"]), f"{name}: key cache differs"
    assert torch.equal(b["value_cache"], a["value_cache"]), f"{name}: value cache differs"
    assert torch.isfinite(got).all()


def test_prelude_in_one_call_positions_past_the_rope_table(device):
    # sequence 1's new tokens sit at positions 36..39 of a 32-row RoPE table
    print("[case] prelude in one call past the RoPE table", flush=True)
    q_len = 4
    x = _inputs(2, 16, 4, 16, [5, 40], q_len, seed=990, rope_len=32)
    a = {n: t.to(device) for n, t in x.items()}
    b = {n: (t.clone() if n in ("key_cache", "value_cache") else t) for n, t in a.items()}
    scale = 1.0 / math.sqrt(D)
    want = _chain(a, 16, q_len, 16, scale, 0)
    torch.cuda.synchronize(device)
    pa.check_errors(device)  # the plain decode sees valid lengths
    got = _one_call(b, q_len, scale, 0)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    assert torch.equal(got, want)
    assert torch.equal(b["key_cache"], a["key_cache"]) and torch.equal(b["value_cache"], a["value_cache"])
    np.testing.assert_array_equal(got[1].float().cpu().numpy(), want[1].float().cpu().numpy())


def test_prelude_in_one_call_length_shorter_than_the_new_tokens_is_reported(device):
    # non-causal q_len 8 (two row tiles per kv head): sequence 1 holds 5 tokens
    print("[case] prelude in one call with a length below q_len", flush=True)
    q_len = 8
    x = _inputs(2, 32, 8, 128, [300, 5], q_len, seed=995)
    a = {n: t.to(device) for n, t in x.items()}
    b = {n: (t.clone() if n in ("key_cache", "value_cache") else t) for n, t in a.items()}
    scale = 1.0 / math.sqrt(D)
    got = pa.paged_attention_decode_prelude(
        b["q_proj"], b["k_proj"], b["v_proj"], b["inv_rms"], b["q_norm_weight"], b["k_norm_weight"], b["rope_cos"],
        b["rope_sin"], b["key_cache"], b["value_cache"], b["block_table"], b["context_lens"], scale=scale,
        eps=kvc.EPS, causal=False)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    # the rows at positions 0..4 were written as the standalone prelude writes them
    _standalone_prelude(a, 32, q_len, 128)
    torch.cuda.synchronize(device)
    assert torch.equal(b["key_cache"], a["key_cache"]) and torch.equal(b["value_cache"], a["value_cache"])
    assert torch.isfinite(got[0]).all()



@pytest.mark.parametrize("name", ["q1_qwen3_heads", "q8_two_tiles"])
def test_prelude_in_one_call_replays_from_a_hip_graph(name, device):
    # The one call allocates nothing once its workspace is sized, so a caller
    # can capture its three launches. Between replays, eager work changes the
    # projections and restores the caches; every replay must equal the
    # standalone prelude then decode on the same inputs.
    batch, hq, hkv, bs, lens, q_len, workers = CASES[name]
    print(f"[case] prelude in one call, hip graph replays {name}", flush=True)
    xs = [_inputs(batch, hq, hkv, bs, lens, q_len, seed=1200 + s) for s in range(2)]
    scale = 1.0 / math.sqrt(D)
    wants = []
    for x in xs:  # the projections of x, everything else (tables, weights, caches) of xs[0]
        a = {n: (x[n] if n in ("q_proj", "k_proj", "v_proj", "inv_rms") else t).to(device) for n, t in xs[0].items()}
        wants.append(_chain(a, hq, q_len, bs, scale, workers))
    torch.cuda.synchronize(device)
    b = {n: t.to(device) for n, t in xs[0].items()}
    caches0 = (xs[0]["key_cache"].to(device), xs[0]["value_cache"].to(device))
    out = torch.empty(wants[0].shape, dtype=torch.float32, device=device)

    def step():
        proj = [b[n] if q_len > 1 else b[n][:, 0] for n in ("q_proj", "k_proj", "v_proj")]
        pa.paged_attention_decode_prelude(
            *proj, b["inv_rms"], b["q_norm_weight"], b["k_norm_weight"], b["rope_cos"], b["rope_sin"],
            b["key_cache"], b["value_cache"], b["block_table"], b["context_lens"], out, scale, eps=kvc.EPS,
            causal=q_len > 1, num_workers=workers)

    side = torch.cuda.Stream(device)
    with torch.cuda.stream(side):
        step()  # sizes and zeroes the capture stream's workspace outside the capture
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    torch.cuda.synchronize(device)
    for i in range(4):
        x = xs[i % 2]
        for n in ("q_proj", "k_proj", "v_proj", "inv_rms"):
            b[n].copy_(x[n].to(device))
        b["key_cache"].copy_(caches0[0])
        b["value_cache"].copy_(caches0[1])
        out.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out, wants[i % 2]), f"{name}: replay {i} differs"
    with torch.cuda.stream(side):  # the replays ran on the capture stream, whose workspace holds their flags
        pa.check_errors(device)
