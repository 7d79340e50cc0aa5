"""KV-cache append fused into the decode (simpler_hip_pa_decode_append), on the GPU.

The reference appends the current token's K/V into the paged pool at a slot
derived from the block table and the sequence length
(simpler_setup/goldens/qwen3_14b_decode.py:106-115,261-269) and then runs the
decode over the context that includes it. Each case here runs the fused entry
on caches whose new-token rows hold NaN, and checks:

* the caches afterwards equal the oracle's append (``oracle/kv_oracle.py``,
  slots from ``new_token_slots``) bit for bit;
* the output equals, bit for bit, the plain decode run on those appended
  caches (the same kernels reading the rows from the cache), and is within
  the decode tolerance of the oracle.

Shapes cover each kernel path: K staged through LDS (D = 128, one row tile),
K in registers (D = 64), blocks larger than the registers (BS = 128,
D = 256); with the append as a launch of its own ahead of the decode: two row
tiles in one wave (D = 128, causal q_len 8), sibling row-tile waves (D = 64,
two row tiles), MLA (576/512, one 128-row workgroup); fp16, several worker
counts, new tokens across a block boundary, lengths past the table row.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle
from simpler_amd import paged_attention as pa
from simpler_amd.workloads import DecodeCase, make_custom_case
from tests.pa_helpers import assert_close, oracle_numpy

pytestmark = pytest.mark.gpu


def new_tokens(case: DecodeCase, seed: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    c = case.config
    gen = torch.Generator("cpu").manual_seed(seed)
    dt = case.key_cache.dtype
    shape = (c.batch, c.q_len, c.kv_heads)
    k = torch.randn((*shape, c.head_dim_k), generator=gen).to(dt)
    v = None if c.mla else torch.randn((*shape, c.head_dim_v), generator=gen).to(dt)
    return k, v


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_appended(case: DecodeCase, k_new: torch.Tensor, v_new: torch.Tensor | None) -> DecodeCase:
    """The case with the new tokens written by the oracle's append."""
    c = case.config
    slots = kv_oracle.new_token_slots(case.block_table.numpy(), case.context_lens.numpy(), c.block_size, c.q_len)
    kb, vb = kv_oracle.kv_append(u16(case.key_cache), None if c.mla else u16(case.value_cache),
                                 u16(k_new).reshape(-1, c.kv_heads, c.head_dim_k),
                                 None if c.mla else u16(v_new).reshape(-1, c.kv_heads, c.head_dim_v),
                                 slots.reshape(-1))
    to_t = lambda a: torch.from_numpy(a.view(np.int16)).view(case.key_cache.dtype)  # noqa: E731
    key = to_t(kb)
    value = key[..., : c.head_dim_v] if c.mla else to_t(vb)
    return DecodeCase(c, case.seed, case.query, key, value, case.block_table, case.context_lens, case.scale)


def poison_new_rows(case: DecodeCase) -> None:
    """NaN in the cache rows the new tokens go to: the fused path must not read them."""
    c = case.config
    for b, n in enumerate(case.context_lens.tolist()):
        for p in range(max(n - c.q_len, 0), n):
            blk = int(case.block_table[b, p // c.block_size])
            case.key_cache[blk, p % c.block_size] = float("nan")
            if not c.mla:
                case.value_cache[blk, p % c.block_size] = float("nan")


def run_decode(case: DecodeCase, device, num_workers: int = 0, k_new=None, v_new=None):
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    if k_new is None:
        pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out,
                                  case.scale, causal=case.config.causal, num_workers=num_workers)
    else:
        pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens,
                                         k_new.to(device), None if v_new is None else v_new.to(device), out,
                                         case.scale, causal=case.config.causal, num_workers=num_workers)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    return out.cpu().numpy(), d.key_cache.cpu(), d.value_cache.cpu()


CASES = {
    # K through LDS (D = 128, one row tile), the headline kernel
    "gqa_d128": dict(batch=4, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                     context_lens=[1, 128, 129, 3000]),
    # K in registers
    "gqa_d64_bs16": dict(batch=4, num_heads=16, kv_heads=4, head_dim=64, block_size=16, context_lens=[1, 16, 17, 300]),
    "gqa_d16_bs64": dict(batch=2, num_heads=16, kv_heads=1, head_dim=16, block_size=64, context_lens=[33, 640]),
    # blocks larger than the registers
    "gqa_bs128_d256": dict(batch=3, num_heads=16, kv_heads=2, head_dim=256, block_size=128,
                           context_lens=[1, 1000, 2049]),
    # two row tiles in one wave (the append as its own launch); new tokens 122..129 straddle blocks 0 and 1
    "verify_q8": dict(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8, causal=True,
                      context_lens=[8, 130, 2000]),
    # 16 new tokens, one row tile per kv head, straddling 16-token blocks
    "verify_q16": dict(batch=2, num_heads=2, kv_heads=2, head_dim=64, block_size=16, q_len=16, causal=True,
                       context_lens=[16, 40]),
    # sibling row-tile waves (D = 64: two row tiles of 4 heads x 8 tokens), the append as its own launch
    "multi_d64_q8": dict(batch=3, num_heads=32, kv_heads=8, head_dim=64, block_size=16, q_len=8, causal=True,
                         context_lens=[8, 20, 700]),
    "fp16_d128": dict(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128, context_lens=[5, 129, 900],
                      dtype=torch.float16),
    # fp16, two row tiles per kv head: the append's own launch ahead of the decode
    "fp16_verify_q8": dict(batch=2, num_heads=32, kv_heads=8, head_dim=128, block_size=64, q_len=8, causal=True,
                           context_lens=[70, 1000], dtype=torch.float16),
    "mla_q1": dict(batch=3, num_heads=128, kv_heads=1, head_dim=576, head_dim_v=512, block_size=64, mla=True,
                   context_lens=[1, 64, 700]),
    "mla_q4": dict(batch=2, num_heads=16, kv_heads=1, head_dim=576, head_dim_v=512, block_size=32, mla=True,
                   q_len=4, causal=True, context_lens=[4, 34]),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("workers", [0, 7])
def test_fused_append_equals_append_then_decode(name, workers, device):
    print(f"[case] append {name} workers={workers}", flush=True)
    seed = 900 + sorted(CASES).index(name)
    case = make_custom_case(seed=seed, **CASES[name])
    k_new, v_new = new_tokens(case, seed + 1)
    want = oracle_appended(case, k_new, v_new)
    poison_new_rows(case)
    got, key_after, value_after = run_decode(case, device, workers, k_new, v_new)
    # caches: exactly the oracle's append
    np.testing.assert_array_equal(u16(key_after), u16(want.key_cache))
    if not case.config.mla:
        np.testing.assert_array_equal(u16(value_after), u16(want.value_cache))
    # output: the plain decode on the appended caches, bit for bit, and the oracle
    plain, _, _ = run_decode(want, device, workers)
    np.testing.assert_array_equal(got, plain)
    assert_close(got, oracle_numpy(want), what=f"append {name}")


@pytest.mark.parametrize("workers", [1, 1000])
def test_fused_append_worker_counts_at_qwen3_shape(workers, device):
    # 1 worker walks every block of every sequence; 1000 cut the new-token
    # blocks into one-block pieces
    print(f"[case] append qwen3 shape workers={workers}", flush=True)
    case = make_custom_case(batch=8, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                            context_lens=[1, 127, 128, 129, 1000, 2047, 4096, 8191], seed=950)
    k_new, v_new = new_tokens(case, 951)
    want = oracle_appended(case, k_new, v_new)
    poison_new_rows(case)
    got, key_after, value_after = run_decode(case, device, workers, k_new, v_new)
    np.testing.assert_array_equal(u16(key_after), u16(want.key_cache))
    np.testing.assert_array_equal(u16(value_after), u16(want.value_cache))
    plain, _, _ = run_decode(want, device, workers)
    np.testing.assert_array_equal(got, plain)


@pytest.mark.parametrize("name", ["gqa_d128", "verify_q8", "multi_d64_q8", "fp16_d128"])
def test_fused_append_into_pooled_caches_stays_in_its_pools(name, device):
    """K and V pools in one allocation (kv_cache.alloc_kv_pools, the
    benchmark's layout): the fused append writes exactly the oracle's rows
    into each pool and nothing into the bytes between them, and the output is
    the plain decode's on the appended caches, bit for bit."""
    from simpler_amd.kv_cache import alloc_kv_pools

    print(f"[case] append into pooled caches {name}", flush=True)
    seed = 900 + sorted(CASES).index(name)
    case = make_custom_case(seed=seed, **CASES[name])
    c = case.config
    k_new, v_new = new_tokens(case, seed + 1)
    want = oracle_appended(case, k_new, v_new)
    poison_new_rows(case)
    nblk, bs, hkv, dk = case.key_cache.shape
    kc, vc = alloc_kv_pools(nblk, bs, hkv, dk, case.key_cache.dtype, device, case.value_cache.shape[3])
    buf = torch.empty(0, dtype=kc.dtype, device=device).set_(kc.untyped_storage())
    buf.fill_(-7.0)  # exact in bf16 and fp16; stays in the gap
    kc.copy_(case.key_cache)
    vc.copy_(case.value_cache)
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode_append(d.query, kc, vc, d.block_table, d.context_lens, k_new.to(device),
                                     v_new.to(device), out, case.scale, causal=c.causal)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    np.testing.assert_array_equal(u16(kc.cpu()), u16(want.key_cache))
    np.testing.assert_array_equal(u16(vc.cpu()), u16(want.value_cache))
    gap = buf[kc.numel(): vc.storage_offset()]
    assert gap.numel() > 0 and bool((gap == -7.0).all())
    plain, _, _ = run_decode(want, device)
    np.testing.assert_array_equal(out.cpu().numpy(), plain)


def test_fused_append_out_of_pool_block_is_reported_and_not_written(device):
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[300, 50], seed=960)
    k_new, v_new = new_tokens(case, 961)
    case.block_table[0, 2] = 10_000  # the block of sequence 0's new token (position 299)
    d = case.to(device)
    before = d.key_cache.clone(), d.value_cache.clone()
    pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens,
                                     k_new.to(device), v_new.to(device), scale=case.scale)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)
    # only sequence 1's new token was written
    changed = (d.key_cache != before[0]).any(dim=(2, 3)).nonzero().tolist()
    blk1 = int(case.block_table[1, 0])
    assert changed == [[blk1, 49]]
    assert (d.value_cache != before[1]).any(dim=(2, 3)).nonzero().tolist() == [[blk1, 49]]
    pa.check_errors(device)


def test_fused_append_length_shorter_than_the_new_tokens_is_reported(device):
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=128, q_len=4,
                            causal=True, context_lens=[300, 50], seed=970)
    k_new, v_new = new_tokens(case, 971)
    d = case.to(device)
    lens = d.context_lens.clone()
    lens[1] = 2  # below q_len
    pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, lens, k_new.to(device),
                                     v_new.to(device), scale=case.scale, causal=True)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)
    pa.check_errors(device)


def test_append_of_two_row_tiles_length_shorter_than_the_new_tokens_is_reported(device):
    # 32 query rows per kv head (two row tiles per worker): the append runs as
    # its own launch ahead of the decode, non-causal, so only it sees the length
    case = make_custom_case(batch=2, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8,
                            context_lens=[300, 50], seed=975)
    k_new, v_new = new_tokens(case, 976)
    d = case.to(device)
    lens = d.context_lens.clone()
    lens[1] = 5  # below q_len: tokens 3..7 of sequence 1 land at positions 0..4
    before = d.key_cache.clone()
    pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, lens, k_new.to(device),
                                     v_new.to(device), scale=case.scale)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    blk = int(case.block_table[1, 0])
    changed = sorted(set(tuple(x) for x in (d.key_cache != before).any(dim=(2, 3)).nonzero().tolist()))
    assert [t for t in changed if t[0] == blk] == [(blk, p) for p in range(5)]
    pa.check_errors(device)


OVERLONG = {
    # one row tile per worker: the append fused into the decode's launches
    "fused_one_tile": dict(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=128, q_len=4, causal=True,
                           context_lens=[300, 50]),
    # two row tiles per worker: the append's own launch ahead of the decode
    "routed_two_tiles": dict(batch=2, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8,
                             causal=True, context_lens=[300, 50]),
    "mla": dict(batch=2, num_heads=16, kv_heads=1, head_dim=576, head_dim_v=512, block_size=32, mla=True, q_len=4,
                causal=True, context_lens=[40, 10]),
}


@pytest.mark.parametrize("name", sorted(OVERLONG))
def test_append_length_past_the_table_row_writes_only_in_table_positions(name, device):
    # The first sequence's length is one past what its table row holds (cap =
    # max_blocks * block_size). Its new tokens keep the positions the raw length
    # gives (len - q_len + j); those at cap and up are dropped, no other row
    # changes, BAD_LENGTH is reported, and the decode attends over cap tokens.
    print(f"[case] append length cap+1 {name}", flush=True)
    seed = 990 + sorted(OVERLONG).index(name)
    case = make_custom_case(seed=seed, **OVERLONG[name])
    c = case.config
    cap = c.max_blocks * c.block_size
    k_new, v_new = new_tokens(case, seed + 1)
    raw = case.context_lens.clone()
    raw[0] = cap + 1
    over = DecodeCase(c, case.seed, case.query, case.key_cache, case.value_cache, case.block_table, raw, case.scale)
    want = oracle_appended(over, k_new, v_new)  # slots at cap and up are -1: skipped
    assert (u16(want.key_cache) != u16(case.key_cache)).any(axis=(2, 3)).sum() == (c.q_len - 1) + c.q_len
    d = over.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens,
                                     k_new.to(device), None if v_new is None else v_new.to(device), out,
                                     case.scale, causal=c.causal)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    np.testing.assert_array_equal(u16(d.key_cache.cpu()), u16(want.key_cache))
    if not c.mla:
        np.testing.assert_array_equal(u16(d.value_cache.cpu()), u16(want.value_cache))
    # the output: the plain decode of the appended caches at the clamped length
    clamped = raw.clone()
    clamped[0] = cap
    plain, _, _ = run_decode(DecodeCase(c, case.seed, case.query, want.key_cache, want.value_cache,
                                        case.block_table, clamped, case.scale), device)
    np.testing.assert_array_equal(out.cpu().numpy(), plain)


@pytest.mark.parametrize("name", ["gqa_d128", "verify_q8", "mla_q1"])
def test_fused_append_replays_from_a_hip_graph(name, device):
    # The fused append allocates nothing once its workspace is sized, so a
    # caller can capture it. Between replays, eager work changes the new
    # tokens and poisons their cache rows again; every replay must write the
    # new rows and match the plain decode on the appended caches.
    print(f"[case] append hip graph replays {name}", flush=True)
    seed = 980 + sorted(CASES).index(name)
    case = make_custom_case(seed=seed, **CASES[name])
    news = [new_tokens(case, seed + 1), new_tokens(case, seed + 2)]
    wants = [oracle_appended(case, k, v) for k, v in news]
    plains = [run_decode(w, device)[0] for w in wants]
    poison_new_rows(case)
    d = case.to(device)
    k_dev = news[0][0].to(device)
    v_dev = None if case.config.mla else news[0][1].to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)

    def step():
        pa.paged_attention_decode_append(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens,
                                         k_dev, v_dev, out, case.scale, causal=case.config.causal)

    side = torch.cuda.Stream(device)
    with torch.cuda.stream(side):
        step()  # sizes and zeroes the capture stream's workspace outside the capture
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    torch.cuda.synchronize(device)
    poisoned_k, poisoned_v = case.key_cache.to(device), case.value_cache.to(device)
    for i in range(4):
        k = i % 2
        k_dev.copy_(news[k][0].to(device))
        if v_dev is not None:
            v_dev.copy_(news[k][1].to(device))
        d.key_cache.copy_(poisoned_k)
        if not case.config.mla:
            d.value_cache.copy_(poisoned_v)
        out.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        np.testing.assert_array_equal(u16(d.key_cache.cpu()), u16(wants[k].key_cache))
        if not case.config.mla:
            np.testing.assert_array_equal(u16(d.value_cache.cpu()), u16(wants[k].value_cache))
        np.testing.assert_array_equal(out.cpu().numpy(), plains[k])
    with torch.cuda.stream(side):  # the replays ran on the capture stream, whose workspace holds their flags
        pa.check_errors(device)
