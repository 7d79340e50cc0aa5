"""GPU parity of the fused decode kernel against the CPU oracle (through the C ABI).

Every call goes through ``simpler_hip_pa_decode`` in libsimpler_hip.so. Cases:
the reference's own scene-test shapes (CaseSmall1/CaseVarSeq2/CaseVarSeq4 of
examples/a2a3/tensormap_and_ringbuffer/paged_attention/test_paged_attention.py
:108-168 and the GQA cases of spmd_paged_attention_highperf/
test_spmd_paged_attention_highperf.py:170-232), the five benchmark configs,
ragged and edge lengths, every supported block size and head dim, and
size-independent properties at full size (worker-count invariance, determinism).
Tolerance: max-abs 2e-2 and rel-L2 1e-3 (bf16 inputs, fp32 accumulation); the
reference scene tests' allclose(1e-3, 1e-3) is checked where it applies.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from simpler_amd import paged_attention as pa
from simpler_amd.workloads import CONFIGS, make_case, make_custom_case
from tests.pa_helpers import REF_ATOL, REF_RTOL, assert_close, oracle_c, oracle_numpy

pytestmark = pytest.mark.gpu


def run_gpu(case, device, out_dtype=torch.float32, num_workers=0):
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=out_dtype, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              causal=case.config.causal, num_workers=num_workers)
    torch.cuda.synchronize(device)
    return out.float().cpu().numpy()


REFERENCE_CASES = {
    "CaseSmall1": dict(batch=1, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[33]),
    "CaseSmall2": dict(batch=1, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[128]),
    "CaseVarSeq2": dict(batch=2, num_heads=16, kv_heads=1, head_dim=16, block_size=16, context_lens=[33, 17]),
    "CaseVarSeq4": dict(batch=4, num_heads=16, kv_heads=1, head_dim=16, block_size=16,
                        context_lens=[33, 64, 128, 15]),
    "highperf_b1_h32_kv8_s128": dict(batch=1, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                     context_lens=[128]),
    "highperf_b4_h32_kv8_s512": dict(batch=4, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                     context_lens=[512] * 4),
    "highperf_b1_h32_kv8_s4096": dict(batch=1, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                      context_lens=[4096]),
    "Case2_h64_bs64_short": dict(batch=2, num_heads=64, kv_heads=1, head_dim=128, block_size=64,
                                 context_lens=[700, 1000]),
    "Case3_d256_bs64_short": dict(batch=2, num_heads=64, kv_heads=1, head_dim=256, block_size=64,
                                  context_lens=[640, 333]),
}


@pytest.mark.parametrize("name", sorted(REFERENCE_CASES))
def test_reference_scene_cases(name, device):
    print(f"[case] {name}", flush=True)
    case = make_custom_case(seed=42, **REFERENCE_CASES[name])
    ref = oracle_numpy(case)
    got = run_gpu(case, device)
    assert_close(got, ref, what=name)
    np.testing.assert_allclose(got, ref, rtol=REF_RTOL, atol=REF_ATOL)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_cfg1_small(out_dtype, device):
    print(f"[case] cfg1_small out={out_dtype}", flush=True)
    case = make_case("cfg1_small")
    ref = oracle_numpy(case)
    got = run_gpu(case, device, out_dtype=out_dtype)
    if out_dtype == torch.bfloat16:
        ref = torch.tensor(ref).to(torch.bfloat16).float().numpy()
    assert_close(got, ref, what="cfg1")


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_block_sizes_and_head_dims(bs, d, device):
    print(f"[case] bs={bs} d={d}", flush=True)
    case = make_custom_case(batch=3, num_heads=8, kv_heads=2, head_dim=d, block_size=bs,
                            context_lens=[1, bs + 3, 5 * bs - 1], seed=100 + bs + d)
    assert_close(run_gpu(case, device), oracle_numpy(case), what=f"bs{bs}_d{d}")


@pytest.mark.parametrize("workers,q_len,value_range", [(0, 1, None), (7, 4, None), (1000, 4, None),
                                                       (37, 1, 8.0)])
def test_blocks_larger_than_the_registers(workers, q_len, value_range, device):
    # 128 tokens x 256 dims: K and V of a block are loaded in tile groups;
    # causal rows across two row tiles, split segments, large score ranges
    print(f"[case] bs=128 d=256 workers={workers} q_len={q_len} range={value_range}", flush=True)
    case = make_custom_case(batch=3, num_heads=16, kv_heads=2, head_dim=256, block_size=128, q_len=q_len,
                            causal=q_len > 1, context_lens=[q_len, 1000, 2049], seed=150 + workers + q_len,
                            value_range=value_range)
    assert_close(run_gpu(case, device, num_workers=workers), oracle_numpy(case), what=f"big w{workers}")


def test_blocks_larger_than_the_registers_ignore_garbage_and_report_bad_blocks(device):
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=256, block_size=128,
                            context_lens=[300, 50], seed=710, pool_extra=2)
    base = run_gpu(case, device)
    for b, n in enumerate([300, 50]):
        last = int(case.block_table[b, (n - 1) // 128])
        case.value_cache[last, n % 128 :] = float("nan")
        case.key_cache[last, n % 128 :] = float("inf")
    np.testing.assert_array_equal(run_gpu(case, device), base)
    case.block_table[0, 1] = 10_000
    run_gpu(case, device)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)
    pa.check_errors(device)


@pytest.mark.parametrize("group", [1, 2, 4, 5, 8, 16, 32])
def test_gqa_groups(group, device):
    print(f"[case] group={group}", flush=True)
    case = make_custom_case(batch=2, num_heads=2 * group, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[777, 1500], seed=200 + group)
    assert_close(run_gpu(case, device), oracle_numpy(case), what=f"g{group}")


@pytest.mark.parametrize("q_len", [2, 4, 8])
def test_causal_multi_token(q_len, device):
    print(f"[case] causal q_len={q_len}", flush=True)
    case = make_custom_case(batch=3, num_heads=8, kv_heads=2, head_dim=128, block_size=128, q_len=q_len,
                            causal=True, context_lens=[q_len, 129 + q_len, 1000], seed=300 + q_len)
    assert_close(run_gpu(case, device), oracle_numpy(case), what=f"causal{q_len}")


@pytest.mark.parametrize("heads,q_len,workers", [(8, 8, 0), (12, 4, 0), (12, 4, 7), (80, 5, 0), (80, 5, 1),
                                                 (80, 5, 333)])
def test_row_tiles_share_a_worker(heads, q_len, workers, device):
    # one kv head, 16 rows per tile: 64 rows -> 4 tiles (one workgroup of 4
    # waves), 48 -> 3, 400 -> 25 tiles (7 row groups of 4 waves, the last one
    # with a single live wave)
    print(f"[case] heads={heads} q_len={q_len} workers={workers}", flush=True)
    case = make_custom_case(batch=3, num_heads=heads, kv_heads=1, head_dim=128,
                            block_size=64, q_len=q_len, causal=True,
                            context_lens=[q_len, 700, 2100], seed=310 + heads + q_len)
    assert_close(run_gpu(case, device, num_workers=workers), oracle_numpy(case), what=f"rowtiles{heads}x{q_len}")


@pytest.mark.parametrize("bs,heads,q_len,dtype,workers", [(128, 64, 1, torch.bfloat16, 0),
                                                          (128, 16, 3, torch.bfloat16, 0),
                                                          (16, 64, 1, torch.bfloat16, 7),
                                                          (128, 40, 2, torch.float16, 0),
                                                          (32, 32, 1, torch.float16, 333),
                                                          (128, 6, 4, torch.bfloat16, 0),
                                                          (64, 6, 4, torch.float16, 5)])
def test_sibling_waves_stage_k_through_lds(bs, heads, q_len, dtype, workers, device):
    # 128-dim heads with several row tiles per kv head: every sibling wave of a
    # workgroup stages K in its own BS x 256 bytes of the launch's dynamic LDS
    # (four waves x 32 KB at BS = 128). 64 rows -> 4 tiles, 48 -> 3, 80 -> 5
    # (a second row group with one live wave); 32 rows -> 2 tiles and 24 -> 2
    # (the second one partial) run in one wave (the two-tile kernel).
    print(f"[case] sibling K through LDS bs={bs} rows={heads * q_len} {dtype} workers={workers}", flush=True)
    case = make_custom_case(batch=3, num_heads=heads, kv_heads=1, head_dim=128, block_size=bs, q_len=q_len,
                            causal=q_len > 1, context_lens=[q_len, 3 * bs + 5, 2000], seed=330 + heads + bs,
                            dtype=dtype)
    got = run_gpu(case, device, num_workers=workers)
    pa.check_errors(device)
    assert_close(got, oracle_numpy(case), what=f"sibling-klds bs{bs} rows{heads * q_len}")


def test_causal_fully_masked_last_block(device):
    # prefix ends on a block boundary: rows 0..q_len-2 see nothing of the last block
    case = make_custom_case(batch=1, num_heads=4, kv_heads=1, head_dim=64, block_size=16, q_len=4, causal=True,
                            context_lens=[33], seed=301)
    assert_close(run_gpu(case, device), oracle_numpy(case), what="causal_masked_block")


@pytest.mark.parametrize("workers", [1, 2, 3, 7, 64, 511, 5000])
def test_worker_counts_agree(workers, device):
    # 1 worker walks every tile serially (segments longer than the 64-entry
    # block-table window); many workers cut tiles into 1-block pieces
    print(f"[case] workers={workers}", flush=True)
    case = make_custom_case(batch=4, num_heads=16, kv_heads=4, head_dim=128, block_size=128,
                            context_lens=[1, 128, 4000, 8191], seed=400)
    assert_close(run_gpu(case, device, num_workers=workers), oracle_numpy(case), what=f"workers{workers}")


def test_empty_and_single_token_contexts(device):
    case = make_custom_case(batch=3, num_heads=8, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[0, 1, 2], seed=500)
    got = run_gpu(case, device)
    assert np.all(got[0] == 0)
    assert_close(got, oracle_numpy(case), what="empty/single")


def test_large_score_magnitudes_stay_finite(device):
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[3000, 2500], seed=600, value_range=8.0)
    assert_close(run_gpu(case, device, num_workers=37), oracle_numpy(case), what="large scores")


def test_garbage_past_context_is_ignored(device):
    case = make_custom_case(batch=2, num_heads=8, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[300, 50], seed=700, pool_extra=2)
    base = run_gpu(case, device)
    for b, n in enumerate([300, 50]):
        last = int(case.block_table[b, (n - 1) // 128])
        case.value_cache[last, n % 128 :] = float("nan")
        case.key_cache[last, n % 128 :] = float("inf")
    np.testing.assert_array_equal(run_gpu(case, device), base)


def test_out_of_pool_block_is_reported_not_read(device):
    case = make_custom_case(batch=1, num_heads=8, kv_heads=2, head_dim=128, block_size=128,
                            context_lens=[300], seed=800)
    case.block_table[0, 1] = 10_000
    run_gpu(case, device)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)
    pa.check_errors(device)  # cleared


@pytest.mark.parametrize("name", ["cfg1_small", "cfg2_qwen3_8b", "cfg5_verify", "ref_unroll_case1"])
def test_benchmark_configs_full_size(name, device):
    print(f"[case] {name} full size", flush=True)
    case = make_case(name)
    ref = oracle_c(case, n_threads=16)
    got = run_gpu(case, device, out_dtype=torch.float32)
    assert_close(got, ref, what=name)


def test_cfg3_long_context_reduced_batch(device):
    # same shape per sequence as cfg3 (L=32768, 64 q heads, 8 kv heads); two sequences keep the CPU oracle short
    case = make_case("cfg3_long", batch_override=2)
    assert_close(run_gpu(case, device), oracle_c(case, n_threads=16), what="cfg3 x2")


def test_full_size_split_invariance_and_determinism(device):
    case = make_case("cfg3_long").to(device)
    outs = []
    for workers in (4096, 1024, 100, 1024):
        out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
        pa.paged_attention_decode(case.query, case.key_cache, case.value_cache, case.block_table,
                                  case.context_lens, out, case.scale, num_workers=workers)
        outs.append(out)
    torch.cuda.synchronize(device)
    ref = outs[1].cpu().numpy()
    for o in outs:
        assert_close(o.cpu().numpy(), ref, max_abs=1e-4, rel_l2=1e-5, what="worker-count invariance")
    np.testing.assert_array_equal(outs[3].cpu().numpy(), ref)  # same plan, same bits


# ---- MLA (one latent KV head, Dk=576, V = K[..., :512]) -------------------------------------------

def _mla_case(*, heads, lens, seed, block_size=64, **kw):
    return make_custom_case(batch=len(lens), num_heads=heads, kv_heads=1, head_dim=576, head_dim_v=512,
                            block_size=block_size, context_lens=lens, seed=seed, mla=True, **kw)


@pytest.mark.parametrize("heads,block_size,workers", [(128, 64, 0), (128, 64, 1), (128, 64, 7), (128, 32, 0),
                                                       (16, 64, 0), (100, 64, 5), (192, 32, 3)])
def test_mla_rows_blocks_and_workers(heads, block_size, workers, device):
    # 128 rows = two 64-row groups; 16 rows leave three waves idle; 100 and 192
    # rows leave part of the last group idle; 1..7 workers cut tiles into pieces
    print(f"[case] mla heads={heads} bs={block_size} workers={workers}", flush=True)
    case = _mla_case(heads=heads, lens=[1, block_size + 5, 700, 2100], seed=700 + heads + block_size)
    assert_close(run_gpu(case, device, num_workers=workers), oracle_numpy(case), what=f"mla h{heads}")


def test_mla_empty_context_and_bf16_out(device):
    case = _mla_case(heads=128, lens=[0, 33, 64, 1000], seed=710)
    got = run_gpu(case, device, out_dtype=torch.bfloat16)
    assert np.all(got[0] == 0)
    ref = torch.tensor(oracle_numpy(case)).to(torch.bfloat16).float().numpy()
    assert_close(got, ref, what="mla empty/bf16")


def test_mla_garbage_past_context_is_ignored(device):
    case = _mla_case(heads=128, lens=[100, 70], seed=720)
    ref = oracle_numpy(case)
    kc = case.key_cache.clone()
    for b, n in enumerate(case.context_lens.tolist()):
        blk = int(case.block_table[b, n // 64])
        kc[blk, n % 64:] = float("nan")  # tokens past the context in the last block
    case.key_cache, case.value_cache = kc, kc[..., :512]
    assert_close(run_gpu(case, device), ref, what="mla garbage tail")


def test_mla_out_of_pool_block_is_reported(device):
    case = _mla_case(heads=128, lens=[200], seed=730)
    case.block_table[0, 1] = 10_000
    got = run_gpu(case, device)
    with pytest.raises(pa.PagedAttentionError):
        pa.check_errors(device)
    pa.check_errors(device)  # cleared
    assert np.all(np.isfinite(got))


def test_mla_cfg4_reduced_batch(device):
    # cfg4 per-sequence shape (128 heads, Dk 576, BS 64, L~U[512,8192]) on 16 sequences against the C oracle
    case = make_case("cfg4_mla", batch_override=16)
    assert_close(run_gpu(case, device), oracle_c(case, n_threads=16), what="cfg4 x16")


def test_mla_cfg4_full_size_invariance(device):
    case = make_case("cfg4_mla").to(device)
    outs = []
    for workers in (0, 61, 0):
        out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
        pa.paged_attention_decode(case.query, case.key_cache, case.value_cache, case.block_table,
                                  case.context_lens, out, case.scale, num_workers=workers)
        outs.append(out)
    torch.cuda.synchronize(device)
    ref = outs[0].cpu().numpy()
    assert np.all(np.isfinite(ref))
    assert_close(outs[1].cpu().numpy(), ref, max_abs=1e-4, rel_l2=1e-5, what="mla worker-count invariance")
    np.testing.assert_array_equal(outs[2].cpu().numpy(), ref)  # same plan, same bits


def test_workspace_reused_across_plans(device):
    # Regression: a workspace reused by a call with a different shape and worker
    # count must not leak state from the previous call into the next.
    small = make_case("cfg3_long", batch_override=2)
    run_gpu(small, device, num_workers=300)
    big = make_case("cfg3_long")
    got = run_gpu(big, device, num_workers=1024)
    assert_close(got, oracle_c(big, n_threads=16), what="workspace reuse")


def test_workspace_shared_by_every_kernel(device):
    # Calls of different kernels, shapes and worker counts (GQA, MLA, few or many
    # tiles, cut at different places) share the one per-device workspace: no call
    # may pick up another's partial results.
    gqa = make_custom_case(batch=5, num_heads=32, kv_heads=8, head_dim=128, block_size=64,
                           context_lens=[1, 700, 2100, 333, 64], seed=901)
    ref = oracle_numpy(gqa)
    mla = _mla_case(heads=128, lens=[1, 69, 700, 2100], seed=902)
    mla_ref = oracle_numpy(mla)
    few = make_custom_case(batch=2, num_heads=16, kv_heads=1, head_dim=64, block_size=16,
                           context_lens=[300, 45], seed=903)
    few_ref = oracle_numpy(few)
    for workers in (64, 7, 0, 333):
        print(f"[case] shared workspace workers={workers}", flush=True)
        assert_close(run_gpu(mla, device, num_workers=workers), mla_ref, what=f"mla w{workers}")
        assert_close(run_gpu(gqa, device, num_workers=workers), ref, what=f"gqa after mla w{workers}")
        assert_close(run_gpu(few, device, num_workers=workers), few_ref, what=f"few tiles w{workers}")
        assert_close(run_gpu(gqa, device, num_workers=workers), ref, what=f"gqa after few w{workers}")


def _visible_v_mean(case) -> np.ndarray:
    """Closed form for scale 0: every visible token weighs exactly 1 (p =
    bf16(e^0)), so each output row is the mean of its visible V rows."""
    c = case.config
    bs = case.key_cache.shape[1]
    v_all = case.value_cache.float().numpy() if not c.mla else case.key_cache.float().numpy()[..., : c.head_dim_v]
    out = np.zeros(case.out_shape(), dtype=np.float64)
    for b in range(case.query.shape[0]):
        L = int(case.context_lens[b])
        rows = v_all[case.block_table[b, : (L + bs - 1) // bs].long().numpy()].reshape(-1, *v_all.shape[2:])[:L]
        g = c.num_heads // c.kv_heads
        for h in range(c.num_heads):
            out[b, h] = rows[:, h // g].mean(axis=0)
    return out


@pytest.mark.parametrize("shape", ["gqa_d128_bs128", "gqa_d64_bs16", "mla"])
def test_scale_zero_and_negative(shape, device):
    # The kernels fold a positive scale into the exponent and scale the scores
    # first otherwise. Scale 0 must give the plain mean of the visible V rows;
    # a negative scale must match the oracle.
    print(f"[case] scale 0 / negative {shape}", flush=True)
    lens = [1, 130, 333, 700]
    if shape == "gqa_d128_bs128":
        case = make_custom_case(batch=4, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                context_lens=lens, seed=921)
    elif shape == "gqa_d64_bs16":
        case = make_custom_case(batch=4, num_heads=16, kv_heads=2, head_dim=64, block_size=16,
                                context_lens=lens, seed=922)
    else:
        case = _mla_case(heads=128, lens=lens, seed=923)
    case.scale = 0.0
    got = run_gpu(case, device)
    assert_close(got, _visible_v_mean(case), what=f"{shape} scale 0 vs the mean of V")
    assert_close(got, oracle_numpy(case), what=f"{shape} scale 0 vs oracle")
    case.scale = -0.088
    assert_close(run_gpu(case, device), oracle_numpy(case), what=f"{shape} scale -0.088")


@pytest.mark.parametrize("shape", ["gqa_d128", "verify_q8", "mla"])
def test_decode_replays_from_a_hip_graph(shape, device):
    # The decode launches no memset and allocates nothing once its workspace is
    # sized, so a caller can capture it. Replays after eager work that changes
    # the query must each match the oracle for the query of that moment.
    print(f"[case] hip graph replays {shape}", flush=True)
    if shape == "gqa_d128":
        case = make_custom_case(batch=6, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                context_lens=[1, 700, 2048, 129, 3000, 64], seed=931)
    elif shape == "verify_q8":
        case = make_custom_case(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128, q_len=8,
                                causal=True, context_lens=[8, 900, 2500], seed=932)
    else:
        case = _mla_case(heads=128, lens=[1, 69, 700, 2100], seed=933)
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    queries = [d.query.clone(), (d.query.float() * -0.5).to(d.query.dtype)]

    def decode():
        pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out,
                                  case.scale, causal=case.config.causal)

    side = torch.cuda.Stream(device)
    with torch.cuda.stream(side):
        decode()  # sizes and zeroes the capture stream's workspace outside the capture
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        decode()
    torch.cuda.synchronize(device)
    expected = []
    for q in queries:
        case.query = q.cpu()
        expected.append(oracle_numpy(case))
    for i in range(3):
        k = i % 2
        d.query.copy_(queries[k])  # eager work between replays
        out.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert_close(out.cpu().numpy(), expected[k], what=f"{shape} graph replay {i}")
    pa.check_errors(device)


def _poison_workspace(device):
    """Fill the workspace's partial slots and zero page with 0xFF bytes (NaN as
    fp32), keeping the first 256 bytes (error word, zeros): a piece the merge
    reads but no segment wrote turns the output into NaN."""
    torch.cuda.synchronize(device)
    buf = pa._WORKSPACE._buf[(device.index or 0, torch.cuda.current_stream(device).cuda_stream)]
    buf[256:].fill_(255)
    torch.cuda.synchronize(device)


@pytest.mark.parametrize("shape", ["d128_bs128", "d64_bs16"])
@pytest.mark.parametrize("workers", [0, 7, 333])
def test_every_piece_the_merge_reads_is_written(shape, workers, device):
    # The merge kernel reads the partial pieces of every cut tile. On a workspace
    # whose partial slots hold NaN, three launches must match the oracle and each
    # other bit for bit: no piece is read that this launch did not write.
    print(f"[case] poisoned workspace {shape} workers={workers}", flush=True)
    if shape == "d128_bs128":
        case = make_custom_case(batch=12, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                                context_lens=[1, 5000, 129, 2048, 7000, 300, 0, 4097, 128, 6500, 50, 3333], seed=911)
    else:
        case = make_custom_case(batch=9, num_heads=16, kv_heads=4, head_dim=64, block_size=16,
                                context_lens=[17, 900, 1, 1600, 333, 16, 1200, 0, 777], seed=912)
    ref = oracle_numpy(case)
    run_gpu(case, device, num_workers=workers)  # sizes the workspace for this plan
    _poison_workspace(device)
    runs = [run_gpu(case, device, num_workers=workers) for _ in range(3)]
    for i, got in enumerate(runs):
        assert np.isfinite(got).all(), f"launch {i}: a piece was read that no segment wrote"
        assert_close(got, ref, what=f"poisoned workspace {shape} w{workers} launch {i}")
    assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2])


@pytest.mark.parametrize("workers", [0, 5000])
def test_many_short_tiles(workers, device):
    # 520 sequences x 32 kv heads = 16640 tiles of 0..3 blocks each, with 1024
    # (per-kv-head work lists) or 5000 workers: many tiles cut into pieces, and
    # empty contexts zero-filled by the merge kernel
    print(f"[case] 16640 tiles workers={workers}", flush=True)
    lens = torch.randint(0, 49, (520,), generator=torch.Generator().manual_seed(904)).tolist()
    lens[3] = 0
    case = make_custom_case(batch=520, num_heads=64, kv_heads=32, head_dim=32, block_size=16,
                            context_lens=lens, seed=905)
    got = run_gpu(case, device, num_workers=workers)
    assert np.all(got[3] == 0)
    assert_close(got, oracle_numpy(case), what=f"16640 tiles w{workers}")


def test_graph_keeps_its_workspace_when_the_stream_grows_one(device):
    """A graph captured on a stream keeps using the workspace it captured after
    an eager call on that stream needs a larger one (the old buffer is retired,
    not freed). The first capture also creates the stream's workspace inside the
    capture (its zeroing is a kernel, recorded in the graph). Replays alternate
    with eager work and each must match the oracle."""
    print("[case] graph replay after workspace growth", flush=True)
    small = make_custom_case(batch=2, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                             context_lens=[300, 1000], seed=941)
    big = make_case("cfg3_long", batch_override=2)
    ds, db = small.to(device), big.to(device)
    ref_small, ref_big = oracle_numpy(small), oracle_c(big, n_threads=16)
    out_s = torch.empty(small.out_shape(), dtype=torch.float32, device=device)
    out_b = torch.empty(big.out_shape(), dtype=torch.float32, device=device)
    side = torch.cuda.Stream(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        pa.paged_attention_decode(ds.query, ds.key_cache, ds.value_cache, ds.block_table, ds.context_lens, out_s,
                                  small.scale, num_workers=64)
    torch.cuda.synchronize(device)
    for i in range(3):
        with torch.cuda.stream(side):  # eager, same stream: grows the workspace on the first pass
            pa.paged_attention_decode(db.query, db.key_cache, db.value_cache, db.block_table, db.context_lens,
                                      out_b, big.scale, num_workers=4096 + 512 * i)
        torch.cuda.synchronize(device)
        assert_close(out_b.cpu().numpy(), ref_big, what=f"eager big {i}")
        out_s.fill_(float("nan"))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert_close(out_s.cpu().numpy(), ref_small, what=f"graph replay {i} after growth")
    with torch.cuda.stream(side):
        pa.check_errors(device)


@pytest.mark.parametrize("bad", ["negative", "past_table", "causal_short"])
def test_bad_device_lengths_are_reported_then_next_run_is_good(bad, device):
    """Device-resident context_lens are only seen by the kernels: a length below
    0, beyond what the block-table row holds, or (causal) shorter than q_len is
    reported as SIMPLER_HIP_ERR_BAD_LENGTH (-7) by the check, and the next call
    with good lengths on the same workspace matches the oracle."""
    print(f"[case] bad device length: {bad}", flush=True)
    causal = bad == "causal_short"
    case = make_custom_case(batch=3, num_heads=16, kv_heads=2, head_dim=128, block_size=64,
                            context_lens=[200, 64, 130], seed=950, q_len=4 if causal else 1, causal=causal)
    d = case.to(device)
    bad_lens = d.context_lens.clone()
    bad_lens[1] = {"negative": -5, "past_table": case.block_table.shape[1] * 64 + 1, "causal_short": 2}[bad]
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, bad_lens, out, case.scale,
                              causal=causal)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    pa.check_errors(device)  # cleared
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              causal=causal)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert_close(out.cpu().numpy(), oracle_numpy(case), what=f"good run after {bad}")


@pytest.mark.parametrize("batch, bad_at, workers", [(100, 97, 0), (300, 5, 0), (600, 590, 0), (600, 70, 333)])
def test_bad_device_length_found_in_a_large_batch(batch, bad_at, workers, device):
    """Batches above 64 sequences check and scan their lengths in groups of
    512 (one load round trip per group): a bad length anywhere in the batch is
    reported, and the next call with good lengths matches the oracle."""
    print(f"[case] bad length at {bad_at} of {batch}, workers={workers}", flush=True)
    lens = [(7 * i) % 50 + 1 for i in range(batch)]
    case = make_custom_case(batch=batch, num_heads=8, kv_heads=4, head_dim=32, block_size=16, context_lens=lens,
                            seed=952)
    d = case.to(device)
    bad_lens = d.context_lens.clone()
    bad_lens[bad_at] = -3
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, bad_lens, out, case.scale,
                              num_workers=workers)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out, case.scale,
                              num_workers=workers)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert_close(out.cpu().numpy(), oracle_numpy(case), what=f"batch {batch} workers {workers}")


def test_mla_bad_device_length_is_reported(device):
    case = _mla_case(heads=128, lens=[200, 70], seed=951)
    d = case.to(device)
    bad_lens = d.context_lens.clone()
    bad_lens[0] = -1
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, bad_lens, out, case.scale)
    torch.cuda.synchronize(device)
    with pytest.raises(pa.PagedAttentionError) as ei:
        pa.check_errors(device)
    assert ei.value.rc == -7
    pa.check_errors(device)


def _share_prefix_blocks(case, shared: int, repeat_in_row: bool = False):
    """Prefix caching / beam search: sequences 1.. point their first `shared`
    block-table entries at sequence 0's physical blocks (and, with
    repeat_in_row, sequence 0 reads its own first block a second time in place
    of its last full block). The cache contents are those of the blocks the
    table names, so the oracle reads the same bytes."""
    bt = case.block_table
    for b in range(1, bt.shape[0]):
        n = min(shared, (int(case.context_lens[b]) + case.config.block_size - 1) // case.config.block_size)
        bt[b, :n] = bt[0, :n]
    if repeat_in_row:
        nb0 = (int(case.context_lens[0]) + case.config.block_size - 1) // case.config.block_size
        if nb0 > 2:
            bt[0, nb0 - 2] = bt[0, 0]
    return case


@pytest.mark.parametrize("kind,workers", [("gqa", 0), ("gqa", 77), ("gqa_verify", 0), ("mla", 0), ("mla", 9)])
def test_blocks_shared_between_sequences(kind, workers, device):
    """Sequences whose block tables name the same physical blocks (a shared
    prompt prefix, beam-search siblings, one block twice in a row) read those
    blocks like any other: the result matches the oracle on the same table."""
    print(f"[case] shared blocks {kind} workers={workers}", flush=True)
    if kind == "mla":
        case = _mla_case(heads=128, lens=[700, 700, 450, 1000], seed=960)
        shared = 6
    else:
        q_len = 4 if kind == "gqa_verify" else 1
        case = make_custom_case(batch=5, num_heads=32, kv_heads=8, head_dim=128, block_size=64, q_len=q_len,
                                causal=q_len > 1, context_lens=[900, 900, 700, 1500, 65], seed=961)
        shared = 8
    _share_prefix_blocks(case, shared, repeat_in_row=True)
    got = run_gpu(case, device, num_workers=workers)
    pa.check_errors(device)
    assert_close(got, oracle_numpy(case), what=f"shared blocks {kind} w{workers}")


def _strided_caches(k, v, layout: str, device):
    """Device views of the dense caches k, v [nb, bs, h, d] in another memory
    layout, with everything the views do not cover set to NaN:
    fused_kv: one buffer [nb, 2, bs, h, d] holding K then V of each block;
    hnd: head-major blocks [nb, h, bs, d] seen through a permute;
    padded: rows of d + 16 elements, the caches the first d."""
    nb, bs, h, d = k.shape
    if layout == "fused_kv":
        buf = torch.full((nb, 2, bs, h, d), float("nan"), dtype=k.dtype)
        buf[:, 0], buf[:, 1] = k, v
        buf = buf.to(device)
        return buf[:, 0], buf[:, 1], buf
    if layout == "hnd":
        kb, vb = k.permute(0, 2, 1, 3).contiguous().to(device), v.permute(0, 2, 1, 3).contiguous().to(device)
        return kb.permute(0, 2, 1, 3), vb.permute(0, 2, 1, 3), (kb, vb)
    assert layout == "padded"
    kb = torch.full((nb, bs, h, d + 16), float("nan"), dtype=k.dtype)
    vb = torch.full((nb, bs, h, v.shape[-1] + 16), float("nan"), dtype=v.dtype)
    kb[..., :d], vb[..., : v.shape[-1]] = k, v
    kb, vb = kb.to(device), vb.to(device)
    return kb[..., :d], vb[..., : v.shape[-1]], (kb, vb)


@pytest.mark.parametrize("layout", ["fused_kv", "hnd", "padded"])
@pytest.mark.parametrize("q_len,dtype", [(1, torch.bfloat16), (8, torch.bfloat16), (1, torch.float16)])
def test_cache_layouts_through_strides(layout, q_len, dtype, device):
    """The entry takes the caches' block, token and head strides: K and V in
    one fused buffer, head-major blocks and padded rows give the oracle's
    result on the dense caches, and never read the NaN padding (bf16 and fp16
    caches)."""
    print(f"[case] cache layout {layout} q_len={q_len} {dtype}", flush=True)
    case = make_custom_case(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=64, q_len=q_len,
                            causal=q_len > 1, context_lens=[700, 64 + q_len, 1500], seed=963, dtype=dtype)
    kc, vc, _keep = _strided_caches(case.key_cache, case.value_cache, layout, device)
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, kc, vc, d.block_table, d.context_lens, out, case.scale,
                              causal=case.config.causal)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert_close(out.cpu().numpy(), oracle_numpy(case), what=f"layout {layout} q{q_len}")


@pytest.mark.parametrize("name", ["cfg2_qwen3_8b", "cfg5_verify", "cfg2_fp8", "cfg1_small"])
def test_pooled_kv_layout_is_bit_identical(name, device):
    """The benchmark's cache layout (K and V in one allocation from
    kv_cache.alloc_kv_pools, V an odd multiple of 256 bytes from K) gives the
    same bits as two separate allocations, at the configs' full sizes; on the
    small config both also match the oracle."""
    print(f"[case] pooled kv layout {name}", flush=True)
    case = make_case(name)
    outs = []
    for pool in (False, True):
        d = case.to(device, kv_pool=pool)
        gap = d.value_cache.data_ptr() - d.key_cache.data_ptr()
        assert (gap % 512 == 256) == pool
        out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
        pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens, out,
                                  case.scale, causal=case.config.causal, k_scale=d.k_scale, v_scale=d.v_scale)
        torch.cuda.synchronize(device)
        pa.check_errors(device)
        outs.append(out.cpu())
        del d
    assert torch.equal(outs[0], outs[1])
    if name == "cfg1_small":
        assert_close(outs[1].numpy(), oracle_numpy(case), what="pooled layout")


def test_mla_padded_token_rows(device):
    """MLA with the latent cache's token rows padded past 576 elements (NaN in
    the padding): V stays the first 512 dims of the same rows."""
    case = _mla_case(heads=128, lens=[700, 70, 1300], seed=964)
    nb, bs, h, dk = case.key_cache.shape
    buf = torch.full((nb, bs, h, dk + 32), float("nan"), dtype=case.key_cache.dtype)
    buf[..., :dk] = case.key_cache
    buf = buf.to(device)
    kc = buf[..., :dk]
    d = case.to(device)
    out = torch.empty(case.out_shape(), dtype=torch.float32, device=device)
    pa.paged_attention_decode(d.query, kc, kc[..., :512], d.block_table, d.context_lens, out, case.scale)
    torch.cuda.synchronize(device)
    pa.check_errors(device)
    assert_close(out.cpu().numpy(), oracle_numpy(case), what="mla padded rows")


def test_threads_on_their_own_streams(device):
    """Host threads calling the decode at the same time, each on a stream of
    its own (default priority), get their own workspaces and correct results:
    GQA and MLA shapes interleaved, several calls per thread."""
    import threading

    cases = [make_custom_case(batch=3, num_heads=32, kv_heads=8, head_dim=128, block_size=128,
                              context_lens=[900, 129, 2500], seed=966),
             _mla_case(heads=128, lens=[300, 1100], seed=967)]
    refs = [oracle_numpy(c) for c in cases]
    dev_cases = [c.to(device) for c in cases]
    results, errors_seen = {}, []

    def worker(tid):
        try:
            s = torch.cuda.Stream(device=device)
            outs = []
            with torch.cuda.stream(s):
                for i in range(6):
                    ci = (tid + i) % 2
                    d, c = dev_cases[ci], cases[ci]
                    out = torch.empty(c.out_shape(), dtype=torch.float32, device=device)
                    pa.paged_attention_decode(d.query, d.key_cache, d.value_cache, d.block_table, d.context_lens,
                                              out, c.scale)
                    outs.append((ci, out))
                s.synchronize()
                pa.check_errors(device)
            results[tid] = [(ci, o.cpu().numpy()) for ci, o in outs]
        except Exception as e:  # reported below, with the thread that raised it
            errors_seen.append((tid, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(3)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a decode thread did not finish"
    assert not errors_seen, errors_seen
    for tid, outs in results.items():
        for i, (ci, got) in enumerate(outs):
            assert_close(got, refs[ci], what=f"thread {tid} call {i}")
